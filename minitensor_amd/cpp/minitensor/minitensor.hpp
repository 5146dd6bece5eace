// minitensor.hpp -- umbrella header of the host layer (link with libmtgemm.so).
#pragma once

#include "Defines.hpp"
#include "GpuUtils.hpp"
#include "MemoryPool.hpp"
#include "Tensor.hpp"
#include "Autograd.hpp"
#include "TensorOps.hpp"
#include "Functional.hpp"
#include "Dispatch.hpp"
#include "Module.hpp"
