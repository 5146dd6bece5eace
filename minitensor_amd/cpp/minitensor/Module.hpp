// Module.hpp -- the modules that own GEMMs: Linear and Conv2D.
//
// Linear keeps the reference's parameter layout (include/Module.hpp:83-124):
// weight_ [in,out], bias_ [1,out], He init N(0, √(2/in)) from std::mt19937
// seeded 1000000, 1000001, ... per instance; forward(x) = x·weight_ + bias_,
// here one GEMM with the bias fused (the reference: matmul then a broadcast add).
// Conv2D as the reference (include/Module.hpp:199-251): weight_ [out,in,k,k],
// bias_ [out] zero, He init N(0, √(2/(in·k·k))) seeded 42, 43, ...
#pragma once

#include <cmath>
#include <random>
#include <vector>

#include "Functional.hpp"

template <typename T>
class Module {
public:
    virtual ~Module() = default;
    virtual Tensor<T> forward(const Tensor<T>& x) = 0;
    virtual std::vector<Tensor<T>> parameters() const { return {}; }
    virtual void to(Device) {}
    virtual const char* name() const { return "Module"; }
    Tensor<T> operator()(const Tensor<T>& x) { return forward(x); }
    void zero_grad() {
        for (auto& p : parameters()) {
            Tensor<T> q = p;
            q.zero_grad();
        }
    }
};

template <typename T>
class Linear : public Module<T> {
public:
    Tensor<T> weight_;
    Tensor<T> bias_;

    Linear(size_t in_features, size_t out_features, Device device = {}) {
        Tensor<T> w({in_features, out_features});
        static std::mt19937::result_type seed = 1000000;
        std::mt19937 gen(seed++);
        std::normal_distribution<T> dist(0.0, std::sqrt(2.0 / in_features));
        for (size_t i = 0; i < w.total_elements(); ++i) w.data()[i] = dist(gen);
        weight_ = w.to(device);
        bias_ = Tensor<T>({1, out_features}, device);
        bias_.fill(T(0));
        weight_.set_requires_grad(true);
        bias_.set_requires_grad(true);
    }

    const char* name() const override { return "Linear"; }
    Tensor<T> forward(const Tensor<T>& x) override { return linear_impl(x, weight_, bias_, true); }
    std::vector<Tensor<T>> parameters() const override { return {weight_, bias_}; }
    void to(Device d) override {
        weight_ = weight_.to(d);
        bias_ = bias_.to(d);
    }
};

template <typename T>
class Conv2D : public Module<T> {
public:
    Tensor<T> weight_;
    Tensor<T> bias_;
    size_t stride_, padding_;

    Conv2D(size_t in_channels, size_t out_channels, size_t kernel_size, size_t stride = 1,
           size_t padding = 0, bool bias = true, Device device = {})
        : stride_(stride), padding_(padding) {
        Tensor<T> w({out_channels, in_channels, kernel_size, kernel_size});
        const T fan_in = static_cast<T>(in_channels * kernel_size * kernel_size);
        static std::mt19937::result_type seed = 42;
        std::mt19937 gen(seed++);
        std::normal_distribution<T> dist(0.0, std::sqrt(T(2.0) / fan_in));
        for (size_t i = 0; i < w.total_elements(); ++i) w.data()[i] = dist(gen);
        weight_ = w.to(device);
        weight_.set_requires_grad(true);
        if (bias) {
            bias_ = Tensor<T>({out_channels}, device);
            bias_.fill(T(0));
            bias_.set_requires_grad(true);
        }
    }

    const char* name() const override { return "Conv2D"; }
    Tensor<T> forward(const Tensor<T>& x) override {
        return conv2d(x, weight_, bias_, stride_, padding_);
    }
    std::vector<Tensor<T>> parameters() const override {
        if (!bias_.defined() || bias_.empty()) return {weight_};
        return {weight_, bias_};
    }
    void to(Device d) override {
        weight_ = weight_.to(d);
        if (bias_.defined() && !bias_.empty()) bias_ = bias_.to(d);
    }
};
