// Defines.hpp -- device identifiers of the host layer.
// Same names and meaning as the reference's Device / DeviceType
// (reference include/Defines.hpp:57-67): DeviceType::CUDA names the GPU, as in
// the reference, and DeviceType::GPU is an alias of it.
#pragma once

#include <cstddef>
#include <cstdint>

constexpr size_t MAX_DIMS = 8;

enum class DeviceType { CPU, CUDA, GPU = CUDA };

struct Device {
    DeviceType type;
    uint8_t index;

    Device(DeviceType t = DeviceType::CPU, uint8_t i = 0) : type(t), index(i) {}

    bool operator==(const Device& o) const { return type == o.type && index == o.index; }
    bool operator!=(const Device& o) const { return !(*this == o); }
    bool is_gpu() const { return type == DeviceType::CUDA; }
};
