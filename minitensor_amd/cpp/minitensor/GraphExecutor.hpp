// GraphExecutor.hpp -- HIP-graph capture and replay of a training step on the
// GEMM path.  Mirrors the reference's GraphExecutor
// (include/GraphExecutor.hpp:22-220): the first step runs eagerly (so the
// pool holds every block the step needs), the second copies the batch into
// static inputs and captures the step on a capture stream with
// active_stream() redirected to it, then launches the graph; later steps copy
// the batch in and replay.  A batch of another shape runs eagerly.
//
// Differences, on purpose:
//   * the step is a user function (forward, loss gradient, backward, update):
//     losses and optimizers are not part of this backend;
//   * every block the pool hands out during capture stays reserved for the
//     executor's lifetime (MemoryPool::Reservation), so a replay never writes
//     into memory that was given to another tensor after the capture;
//   * capture_allocations() reports how many of those blocks needed a fresh
//     hipMalloc (0 once the warm-up step has filled the pool).
// Everything the library launches in a step is a kernel on the active stream
// (no hipMemsetAsync, no host sync), so the graph holds kernels only.
#pragma once

#include <hip/hip_runtime.h>

#include <functional>
#include <utility>
#include <vector>

#include "GpuUtils.hpp"
#include "MemoryPool.hpp"
#include "Tensor.hpp"
#include "TensorOps.hpp"

template <typename T>
class GraphExecutor {
public:
    using StepFn = std::function<Tensor<T>(const Tensor<T>& x, const Tensor<T>& y)>;

    explicit GraphExecutor(StepFn step) : step_(std::move(step)) {
        GPU_CHECK(hipStreamCreate(&stream_));
    }

    ~GraphExecutor() {
        if (stream_) (void)hipStreamSynchronize(stream_);
        if (exec_) (void)hipGraphExecDestroy(exec_);
        if (graph_) (void)hipGraphDestroy(graph_);
        if (stream_) (void)hipStreamDestroy(stream_);
    }

    GraphExecutor(const GraphExecutor&) = delete;
    GraphExecutor& operator=(const GraphExecutor&) = delete;

    // One training step on batch (x, y); returns the step's result tensor
    // (for replays, the static tensor the graph writes).
    Tensor<T> step(const Tensor<T>& x, const Tensor<T>& y) {
        if (!x.device().is_gpu() || !y.device().is_gpu())
            throw std::invalid_argument("GraphExecutor: GPU tensors expected");
        if (state_ == State::GraphReady && (x.shape() != x_.shape() || y.shape() != y_.shape()))
            return step_(x, y);
        if (state_ == State::NeedsWarmup) {
            Tensor<T> out = step_(x, y);
            x_ = Tensor<T>(x.shape(), x.device());
            y_ = Tensor<T>(y.shape(), y.device());
            state_ = State::NeedsCapture;
            return out;
        }
        if (state_ == State::NeedsCapture) {
            load(x, y);
            GPU_CHECK(hipStreamSynchronize(stream_));
            capture();   // on an exception: state_ is NeedsWarmup again
            state_ = State::GraphReady;
        }
        return replay(x, y);
    }

    bool captured() const { return state_ == State::GraphReady; }
    hipStream_t stream() const { return stream_; }
    size_t capture_allocations() const { return reservation_.fresh_allocations(); }

private:
    enum class State { NeedsWarmup, NeedsCapture, GraphReady };

    void load(const Tensor<T>& x, const Tensor<T>& y) {
        ActiveStreamGuard g(stream_);
        copy_gpu_strided(x, x_);
        copy_gpu_strided(y, y_);
    }

    // If the step throws while it is being captured, the capture is ended and
    // its partial graph destroyed, the reservation stops pinning this
    // thread's allocations, and the executor starts over with an eager
    // warm-up step on the next call; the exception propagates.
    void capture() {
        GPU_CHECK(hipStreamBeginCapture(stream_, hipStreamCaptureModeRelaxed));
        reservation_.start();
        try {
            ActiveStreamGuard g(stream_);
            out_ = step_(x_, y_);
        } catch (...) {
            hipGraph_t partial = nullptr;
            (void)hipStreamEndCapture(stream_, &partial);
            if (partial) (void)hipGraphDestroy(partial);
            (void)hipGetLastError();
            reservation_.stop();
            state_ = State::NeedsWarmup;
            throw;
        }
        const hipError_t e = hipStreamEndCapture(stream_, &graph_);
        reservation_.stop();
        GPU_CHECK(e);
        GPU_CHECK(hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0));
    }

    Tensor<T> replay(const Tensor<T>& x, const Tensor<T>& y) {
        load(x, y);
        GPU_CHECK(hipGraphLaunch(exec_, stream_));
        GPU_CHECK(hipStreamSynchronize(stream_));
        return out_;
    }

    StepFn step_;
    State state_ = State::NeedsWarmup;
    Tensor<T> x_, y_, out_;
    MemoryPool::Reservation reservation_;
    hipStream_t stream_ = nullptr;
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t exec_ = nullptr;
};
