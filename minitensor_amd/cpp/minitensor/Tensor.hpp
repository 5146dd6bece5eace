// Tensor.hpp -- the Tensor<T> the GEMM backend consumes.
//
// Keeps the reference's Tensor API and view semantics (reference
// include/Tensor.hpp:1-160, include/TensorImpl.hpp:23-292):
//   * shape / strides in elements, an element offset, storage shared by views;
//   * data() is the storage base and data() + offset() the first element;
//   * transpose swaps strides, slice advances the offset, expand gives stride 0;
//   * is_contiguous() checks strides only (an offset view can be contiguous);
//   * autograd fields (grad, grad_fn, requires_grad, version counter) and
//     backward() seeding ones and walking the graph in reverse topological order.
// Differences, on purpose: storage is freed back to the MemoryPool by a
// destructor; reshape() of a non-contiguous view throws instead of
// reinterpreting strides; as_strided() builds arbitrary views (bmm needs it).
#pragma once

#include <algorithm>
#include <cstring>
#include <functional>
#include <memory>
#include <numeric>
#include <stdexcept>
#include <string>
#include <unordered_set>
#include <vector>

#include "Defines.hpp"
#include "GpuUtils.hpp"
#include "MemoryPool.hpp"
#include "mtgemm.h"

template <typename T> class Tensor;
template <typename T> struct AutogradNode;
template <typename T> void add_(Tensor<T>& A, const Tensor<T>& B);
template <typename T> void copy_strided(const Tensor<T>& src, Tensor<T>& dst);

template <typename T>
class TensorStorage {
public:
    TensorStorage(size_t size, Device device) : size_(size), device_(device) {
        data_ = static_cast<T*>(MemoryPool::get().allocate(size * sizeof(T), device));
        if (!device.is_gpu() && size) std::memset(data_, 0, size * sizeof(T));
    }
    ~TensorStorage() { MemoryPool::get().free(data_, size_ * sizeof(T), device_); }
    TensorStorage(const TensorStorage&) = delete;
    TensorStorage& operator=(const TensorStorage&) = delete;

    T* data() const noexcept { return data_; }
    Device device() const noexcept { return device_; }
    size_t size() const noexcept { return size_; }

    void fill(const T& v) {
        if (!device_.is_gpu()) {
            std::fill(data_, data_ + size_, v);
            return;
        }
        static_assert(std::is_same_v<T, float>, "GPU tensors are float32");
        // A fill kernel (not a memset) so it stays correct inside graph capture.
        mt_check_status(mt_fill_f32(data_, (int64_t)size_, v, active_stream()), "fill");
    }

    uint32_t version() const noexcept { return version_; }
    void bump_version() noexcept { ++version_; }

private:
    T* data_ = nullptr;
    size_t size_;
    Device device_;
    uint32_t version_ = 0;
};

inline std::vector<size_t> contiguous_strides(const std::vector<size_t>& shape) {
    std::vector<size_t> st(shape.size());
    size_t s = 1;
    for (size_t i = shape.size(); i-- > 0;) {
        st[i] = s;
        s *= shape[i];
    }
    return st;
}

inline size_t numel_of(const std::vector<size_t>& shape) {
    return std::accumulate(shape.begin(), shape.end(), (size_t)1, std::multiplies<size_t>{});
}

template <typename T>
struct TensorImpl {
    std::shared_ptr<TensorStorage<T>> storage_;
    std::vector<size_t> shape_;
    std::vector<size_t> strides_;
    size_t offset_;
    Tensor<T> grad_;
    std::shared_ptr<AutogradNode<T>> grad_fn_;
    bool requires_grad_;

    TensorImpl(std::shared_ptr<TensorStorage<T>> storage, std::vector<size_t> shape,
               std::vector<size_t> strides, size_t offset, bool requires_grad = false)
        : storage_(std::move(storage)), shape_(std::move(shape)), strides_(std::move(strides)),
          offset_(offset), requires_grad_(requires_grad) {
        if (shape_.size() != strides_.size())
            throw std::invalid_argument("TensorImpl: shape and strides differ in rank");
        if (shape_.size() > MAX_DIMS) throw std::runtime_error("Exceeded MAX_DIMS");
    }

    bool is_contiguous() const noexcept {
        size_t expect = 1;
        for (size_t i = shape_.size(); i-- > 0;) {
            if (shape_[i] != 1 && strides_[i] != expect) return false;
            expect *= shape_[i];
        }
        return true;
    }
};

template <typename T>
class Tensor {
public:
    using Self = Tensor<T>;

    Tensor() = default;

    Tensor(std::vector<size_t> shape, Device device = {}) {
        auto storage = std::make_shared<TensorStorage<T>>(numel_of(shape), device);
        auto strides = contiguous_strides(shape);
        impl_ = std::make_shared<TensorImpl<T>>(std::move(storage), std::move(shape),
                                                std::move(strides), 0);
    }

    explicit Tensor(std::shared_ptr<TensorImpl<T>> impl) : impl_(std::move(impl)) {}

    static Self ones_like(const std::vector<size_t>& shape, const Device& device = {}) {
        Self t(shape, device);
        t.fill(T(1));
        return t;
    }

    // A view on this tensor's storage with explicit geometry (elements).
    Self as_strided(std::vector<size_t> shape, std::vector<size_t> strides, size_t offset) const {
        return Self(std::make_shared<TensorImpl<T>>(impl_->storage_, std::move(shape),
                                                    std::move(strides), offset, requires_grad()));
    }

    T& at(const std::vector<size_t>& idx) {
        if (device().is_gpu()) throw std::runtime_error("at(): CPU tensors only");
        if (idx.size() != shape().size()) throw std::out_of_range("at(): wrong number of indices");
        size_t e = offset();
        for (size_t i = 0; i < idx.size(); ++i) {
            if (idx[i] >= shape()[i]) throw std::out_of_range("Index out of range");
            e += idx[i] * strides()[i];
        }
        return data()[e];
    }

    Self transpose(size_t d0, size_t d1) const {
        if (d0 >= shape().size() || d1 >= shape().size())
            throw std::out_of_range("transpose: dimension out of range");
        auto sh = shape();
        auto st = strides();
        std::swap(sh[d0], sh[d1]);
        std::swap(st[d0], st[d1]);
        return as_strided(std::move(sh), std::move(st), offset());
    }

    // Broadcast to `target` (leading dims added, size-1 dims stretched with stride 0).
    Self expand(const std::vector<size_t>& target) const {
        const auto& sh = shape();
        if (target.size() < sh.size())
            throw std::invalid_argument("Cannot expand to a smaller number of dimensions.");
        const size_t lead = target.size() - sh.size();
        std::vector<size_t> st(target.size(), 0);
        for (size_t i = 0; i < target.size(); ++i) {
            if (i < lead) continue;
            const size_t d = sh[i - lead];
            if (d != target[i] && d != 1)
                throw std::invalid_argument("Incompatible shapes for broadcasting.");
            st[i] = (d == target[i]) ? strides()[i - lead] : 0;
        }
        return as_strided(target, std::move(st), offset());
    }

    Self reshape(const std::vector<size_t>& new_shape) const {
        if (numel_of(new_shape) != total_elements())
            throw std::invalid_argument("reshape: total element count mismatch");
        if (!is_contiguous())
            throw std::invalid_argument("reshape: view is not contiguous; call contiguous() first");
        return as_strided(new_shape, contiguous_strides(new_shape), offset());
    }

    Self slice(size_t dim, size_t start, size_t end) const {
        if (dim >= shape().size()) throw std::out_of_range("slice: dimension out of range");
        if (start >= end || end > shape()[dim]) throw std::out_of_range("slice: invalid range");
        if (start == 0 && end == shape()[dim]) return *this;
        auto sh = shape();
        sh[dim] = end - start;
        return as_strided(std::move(sh), strides(), offset() + start * strides()[dim]);
    }

    // Copies the whole storage to `target` and keeps the view geometry
    // (the reference's TensorImpl::to, include/TensorImpl.hpp:246-278).
    Self to(Device target) const {
        if (device() == target) return as_strided(shape(), strides(), offset());
        const size_t n = impl_->storage_->size();
        auto st = std::make_shared<TensorStorage<T>>(n, target);
        const size_t bytes = n * sizeof(T);
        if (bytes) {
            if (device().is_gpu()) GPU_CHECK(hipStreamSynchronize(active_stream()));
            if (!device().is_gpu() && target.is_gpu())
                GPU_CHECK(hipMemcpy(st->data(), data(), bytes, hipMemcpyHostToDevice));
            else if (device().is_gpu() && !target.is_gpu())
                GPU_CHECK(hipMemcpy(st->data(), data(), bytes, hipMemcpyDeviceToHost));
            else
                GPU_CHECK(hipMemcpy(st->data(), data(), bytes, hipMemcpyDeviceToDevice));
        }
        return Self(std::make_shared<TensorImpl<T>>(st, shape(), strides(), offset(),
                                                    requires_grad()));
    }

    Self contiguous() const {
        if (is_contiguous() && offset() == 0) return *this;
        Self out(shape(), device());
        copy_strided(*this, out);
        return out;
    }

    bool defined() const noexcept { return impl_ != nullptr; }
    bool empty() const noexcept { return impl_ == nullptr || total_elements() == 0; }
    const std::vector<size_t>& shape() const noexcept { return impl_->shape_; }
    const std::vector<size_t>& strides() const noexcept { return impl_->strides_; }
    Device device() const noexcept { return impl_->storage_->device(); }
    T* data() noexcept { return impl_->storage_->data(); }
    const T* data() const noexcept { return impl_->storage_->data(); }
    size_t total_elements() const noexcept { return numel_of(impl_->shape_); }
    size_t offset() const noexcept { return impl_->offset_; }
    size_t storage_size() const noexcept { return impl_->storage_->size(); }
    bool is_contiguous() const noexcept { return impl_->is_contiguous(); }
    bool same_storage(const Self& o) const noexcept {
        return impl_ && o.impl_ && impl_->storage_ == o.impl_->storage_;
    }
    void fill(const T& v) { impl_->storage_->fill(v); }
    void zero_grad() {
        if (impl_->grad_.defined() && !impl_->grad_.empty()) impl_->grad_.fill(T(0));
    }

    bool requires_grad() const noexcept { return impl_ && impl_->requires_grad_; }
    void set_requires_grad(bool r) noexcept { impl_->requires_grad_ = r; }
    Self& grad() { return impl_->grad_; }
    const Self& grad() const { return impl_->grad_; }
    void accumulate_grad(const Self& g) {
        if (!impl_->grad_.defined() || impl_->grad_.empty()) impl_->grad_ = g;
        else add_(impl_->grad_, g);
    }
    std::shared_ptr<AutogradNode<T>> grad_fn() const noexcept { return impl_->grad_fn_; }
    void set_grad_fn(std::shared_ptr<AutogradNode<T>> fn) { impl_->grad_fn_ = std::move(fn); }

    void backward() {
        if (!requires_grad())
            throw std::runtime_error("Called backward on a tensor that does not require gradients.");
        if (!grad().defined() || grad().empty()) impl_->grad_ = ones_like(shape(), device());
        std::vector<Self> order;
        std::unordered_set<const TensorImpl<T>*> seen;
        std::function<void(const Self&)> visit = [&](const Self& t) {
            if (!t.defined() || t.empty()) return;
            if (!seen.insert(t.impl_.get()).second) return;
            if (t.grad_fn())
                for (const auto& in : t.grad_fn()->get_inputs()) visit(in);
            order.push_back(t);
        };
        visit(*this);
        for (auto it = order.rbegin(); it != order.rend(); ++it)
            if (it->grad_fn() && it->grad().defined() && !it->grad().empty())
                it->grad_fn()->apply(it->grad());
    }

    uint32_t version() const { return impl_ ? impl_->storage_->version() : 0; }
    void bump_version() {
        if (impl_) impl_->storage_->bump_version();
    }
    bool is_leaf() const { return !impl_ || impl_->grad_fn_ == nullptr; }
    const std::shared_ptr<TensorImpl<T>>& impl() const noexcept { return impl_; }

private:
    std::shared_ptr<TensorImpl<T>> impl_;
};
