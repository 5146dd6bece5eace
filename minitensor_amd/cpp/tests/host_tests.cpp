// host_tests.cpp -- tests of the C++ host layer (Tensor / matmul / bmm / conv2d /
// F::linear / Linear / Conv2D / Dispatch) on the CPU device and on the GPU.
//
//   mt_host_tests --cpu [--golden FILE]   CPU-device tests (no GPU needed)
//   mt_host_tests --gpu [--golden FILE]   GPU tests: known answers and CPU-vs-GPU equivalence
//
// FILE is tests/golden/reference_vectors.bin: inputs and outputs of the
// reference's own CPU code (tests/golden/make_golden.py).  The CPU device is
// checked against it bit for bit, so the GPU comparisons against the CPU
// device are anchored to the reference.
//
// Known answers are the reference's own tests: test/tensor_test.cpp:258-510,
// test/engien_test.cpp:80-96, test/spatial_test.cpp:155-230, test/view_test.cpp.
// Equivalence uses the GEMM parity bound 1e-5·√K·max|A|·max|B|.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <map>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "minitensor/minitensor.hpp"
#include "minitensor/GraphExecutor.hpp"

namespace {

struct Case {
    const char* name;
    bool gpu;
    void (*fn)();
};
std::vector<Case>& cases() {
    static std::vector<Case> c;
    return c;
}
struct Reg {
    Reg(const char* n, bool g, void (*f)()) { cases().push_back({n, g, f}); }
};
int g_fail = 0;
const char* g_cur = "";

#define TEST_CPU(name) static void name(); static Reg reg_##name(#name, false, name); static void name()
#define TEST_GPU(name) static void name(); static Reg reg_##name(#name, true, name); static void name()
#define CHECK(cond)                                                                   \
    do {                                                                              \
        if (!(cond)) {                                                                \
            std::printf("  FAIL %s: %s (line %d)\n", g_cur, #cond, __LINE__);         \
            ++g_fail;                                                                 \
        }                                                                             \
    } while (0)
#define CHECK_EQ_F(a, b) CHECK(std::fabs((double)(a) - (double)(b)) <= 1e-6 * (1 + std::fabs((double)(b))))
#define CHECK_THROWS(expr, Exc)                     \
    do {                                            \
        bool thrown_ = false;                       \
        try { expr; } catch (const Exc&) { thrown_ = true; } \
        CHECK(thrown_ && #Exc);                     \
    } while (0)

const Device CPU{DeviceType::CPU};
const Device GPU{DeviceType::CUDA, 0};

Tensor<float> host(const Tensor<float>& t) { return t.to(CPU).contiguous(); }

float val(const Tensor<float>& t, size_t i) {
    Tensor<float> h = t.to(CPU);
    return h.data()[h.offset() + i];
}

// Seeded U(lo,hi) from std::mt19937 with an explicit transform.
Tensor<float> uniform(std::vector<size_t> shape, unsigned seed, float lo = -1.f, float hi = 1.f) {
    Tensor<float> t(shape);
    std::mt19937 g(seed);
    for (size_t i = 0; i < t.total_elements(); ++i)
        t.data()[i] = lo + (hi - lo) * (float)((g() >> 8) * (1.0 / 16777216.0));
    return t;
}

float amax(const Tensor<float>& t) {
    Tensor<float> h = host(t);
    float m = 0;
    for (size_t i = 0; i < h.total_elements(); ++i) m = std::max(m, std::fabs(h.data()[i]));
    return m;
}

// max |a - b| over two same-shape tensors (any device / strides).
double max_err(const Tensor<float>& a, const Tensor<float>& b) {
    Tensor<float> x = host(a), y = host(b);
    CHECK(x.shape() == y.shape());
    double e = 0;
    for (size_t i = 0; i < x.total_elements(); ++i)
        e = std::max(e, (double)std::fabs(x.data()[i] - y.data()[i]));
    return e;
}

void check_close(const Tensor<float>& got, const Tensor<float>& want, size_t K, float am, float bm,
                 double extra = 0.0) {
    const double bound = 1e-5 * std::sqrt((double)std::max<size_t>(K, 1)) * am * bm + extra;
    const double e = max_err(got, want);
    if (!(e <= bound)) std::printf("  %s: max|err| %.3e > bound %.3e\n", g_cur, e, bound);
    CHECK(e <= bound);
}

// ---- golden vectors (tests/golden/reference_vectors.bin) ---------------------
std::string g_golden_path;

std::map<std::string, Tensor<float>>& golden_arrays() {
    static std::map<std::string, Tensor<float>> arrays;
    static bool loaded = false;
    if (loaded) return arrays;
    loaded = true;
    if (g_golden_path.empty()) throw std::runtime_error("no --golden file given");
    std::ifstream f(g_golden_path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + g_golden_path);
    char magic[8];
    f.read(magic, 8);
    if (!f || std::memcmp(magic, "MTGOLD01", 8) != 0) throw std::runtime_error("bad golden file");
    uint32_t count = 0;
    f.read(reinterpret_cast<char*>(&count), 4);
    for (uint32_t i = 0; i < count && f; ++i) {
        uint32_t len = 0, nd = 0;
        f.read(reinterpret_cast<char*>(&len), 4);
        std::string name(len, '\0');
        f.read(name.data(), len);
        f.read(reinterpret_cast<char*>(&nd), 4);
        std::vector<size_t> shape(nd);
        for (auto& d : shape) {
            uint64_t v = 0;
            f.read(reinterpret_cast<char*>(&v), 8);
            d = (size_t)v;
        }
        Tensor<float> t(shape);
        f.read(reinterpret_cast<char*>(t.data()), (std::streamsize)(t.total_elements() * 4));
        arrays[name] = t;
    }
    if (!f) throw std::runtime_error("truncated golden file");
    return arrays;
}

Tensor<float> gold(const std::string& name) {
    auto& a = golden_arrays();
    auto it = a.find(name);
    if (it == a.end()) throw std::runtime_error("golden array missing: " + name);
    return it->second;
}

Tensor<float> mat23() {
    Tensor<float> A({2, 3});
    for (int i = 0; i < 6; ++i) A.data()[i] = (float)(i + 1);
    return A;
}
Tensor<float> mat32() {
    Tensor<float> B({3, 2});
    for (int i = 0; i < 6; ++i) B.data()[i] = (float)(i + 7);
    return B;
}

// =====================================================================
// CPU device
// =====================================================================
TEST_CPU(cpu_matmul_known_answer) {  // tensor_test.cpp:258-283
    Tensor<float> C = matmul(mat23(), mat32());
    CHECK(C.shape() == (std::vector<size_t>{2, 2}));
    CHECK_EQ_F(C.data()[0], 58); CHECK_EQ_F(C.data()[1], 64);
    CHECK_EQ_F(C.data()[2], 139); CHECK_EQ_F(C.data()[3], 154);
}

TEST_CPU(cpu_autograd_matmul) {  // tensor_test.cpp:368-419
    Tensor<float> A = mat23(), B = mat32();
    A.set_requires_grad(true);
    B.set_requires_grad(true);
    Tensor<float> C = matmul(A, B);
    C.backward();
    const float dA[] = {15, 19, 23, 15, 19, 23}, dB[] = {5, 5, 7, 7, 9, 9};
    for (int i = 0; i < 6; ++i) {
        CHECK_EQ_F(A.grad().data()[i], dA[i]);
        CHECK_EQ_F(B.grad().data()[i], dB[i]);
    }
}

TEST_CPU(cpu_chained_matmul_plus_bias) {  // tensor_test.cpp:448-488
    Tensor<float> A = mat23(), B = mat32(), C({2});
    C.data()[0] = 10; C.data()[1] = 20;
    A.set_requires_grad(true); B.set_requires_grad(true); C.set_requires_grad(true);
    Tensor<float> D = matmul(A, B) + C;
    CHECK_EQ_F(D.data()[0], 68); CHECK_EQ_F(D.data()[3], 174);
    D.backward();
    CHECK_EQ_F(A.grad().data()[0], 15); CHECK_EQ_F(A.grad().data()[2], 23);
    CHECK_EQ_F(B.grad().data()[0], 5); CHECK_EQ_F(B.grad().data()[4], 9);
    CHECK_EQ_F(C.grad().data()[0], 2); CHECK_EQ_F(C.grad().data()[1], 2);
}

TEST_CPU(cpu_broadcast_add_grads) {  // tensor_test.cpp AutogradTest.BroadcastingAddition
    Tensor<float> A({2, 3}), B({3});
    A.fill(1); B.fill(2);
    A.set_requires_grad(true); B.set_requires_grad(true);
    Tensor<float> C = A + B;
    C.backward();
    CHECK_EQ_F(A.grad().data()[5], 1);
    CHECK(B.grad().shape() == (std::vector<size_t>{3}));
    for (int i = 0; i < 3; ++i) CHECK_EQ_F(B.grad().data()[i], 2);
}

TEST_CPU(cpu_matmul_backward_fills) {  // engien_test.cpp:80-96
    Tensor<float> a({2, 3}), b({3, 2});
    a.fill(2); b.fill(3);
    a.set_requires_grad(true); b.set_requires_grad(true);
    Tensor<float> c = matmul(a, b);
    CHECK_EQ_F(val(c, 0), 18);
    c.backward();
    CHECK_EQ_F(val(a.grad(), 0), 6);
    CHECK_EQ_F(val(b.grad(), 0), 4);
}

TEST_CPU(cpu_views_slice_transpose_expand) {
    Tensor<float> big = uniform({10, 6}, 1);
    Tensor<float> s = big.slice(0, 3, 8);  // offset view, strides unchanged
    CHECK(s.offset() == 18 && s.is_contiguous());
    Tensor<float> B = uniform({6, 4}, 2);
    check_close(matmul(s, B), matmul(s.contiguous(), B), 6, 1, 1);
    Tensor<float> bt = uniform({4, 6}, 3).transpose(0, 1);  // [6,4] strides (1,6)
    CHECK(!bt.is_contiguous());
    check_close(matmul(s, bt), matmul(s, bt.contiguous()), 6, 1, 1);
    Tensor<float> row = uniform({1, 6}, 4).expand({5, 6});  // stride 0
    CHECK(row.strides()[0] == 0);
    check_close(matmul(row, B), matmul(row.contiguous(), B), 6, 1, 1);
    CHECK_THROWS(big.slice(0, 5, 3), std::out_of_range);
    CHECK_THROWS(big.slice(2, 0, 1), std::out_of_range);
}

TEST_CPU(cpu_matmul_errors) {  // include/TensorOps.hpp:995-1005 error behaviour
    CHECK_THROWS(matmul(Tensor<float>({2, 3}), Tensor<float>({2, 3})), std::invalid_argument);
    CHECK_THROWS(matmul(Tensor<float>({2, 3, 1}), Tensor<float>({3, 2})), std::invalid_argument);
    CHECK_THROWS(bmm(Tensor<float>({2, 3, 4}), Tensor<float>({3, 4, 2})), std::invalid_argument);
    CHECK_THROWS(bmm(Tensor<float>({2, 3, 4}), Tensor<float>({2, 5, 2})), std::invalid_argument);
    CHECK_THROWS(F::linear(Tensor<float>({2, 3}), Tensor<float>({4, 5})), std::invalid_argument);
}

TEST_CPU(cpu_saved_tensor_version_check) {
    Tensor<float> A = mat23(), B = mat32();
    A.set_requires_grad(true);
    Tensor<float> C = matmul(A, B);
    add_(B, mat32());  // in-place change of a saved input
    CHECK_THROWS(C.backward(), std::runtime_error);
}

TEST_CPU(cpu_bmm_and_backward) {
    Tensor<float> A = uniform({3, 4, 5}, 1), B = uniform({3, 5, 2}, 2);
    A.set_requires_grad(true); B.set_requires_grad(true);
    Tensor<float> C = bmm(A, B);
    for (size_t z = 0; z < 3; ++z) {
        auto a = A.as_strided({4, 5}, {5, 1}, z * 20);
        auto b = B.as_strided({5, 2}, {2, 1}, z * 10);
        auto c = C.as_strided({4, 2}, {2, 1}, z * 8);
        NoGradGuard g;
        check_close(c, matmul(a, b), 5, 1, 1);
    }
    C.backward();  // dA = ones·Bᵀ, dB = Aᵀ·ones per batch
    for (size_t z = 0; z < 3; ++z)
        for (size_t i = 0; i < 4; ++i)
            for (size_t k = 0; k < 5; ++k) {
                float want = B.data()[z * 10 + k * 2] + B.data()[z * 10 + k * 2 + 1];
                CHECK(std::fabs(A.grad().data()[z * 20 + i * 5 + k] - want) < 1e-6);
            }
}

TEST_CPU(cpu_conv_known_answer) {  // spatial_test.cpp:155-185
    Tensor<float> x({1, 1, 3, 3}), w({1, 1, 2, 2}), b({1});
    for (int i = 0; i < 9; ++i) x.data()[i] = (float)(i + 1);
    w.fill(1);
    Tensor<float> y = conv2d(x, w, b, 1, 0);
    CHECK(y.shape() == (std::vector<size_t>{1, 1, 2, 2}));
    const float want[] = {12, 16, 24, 28};
    for (int i = 0; i < 4; ++i) CHECK_EQ_F(y.data()[i], want[i]);
}

// L = Σ dY ⊙ f(params); analytic gradients vs central differences.
void gradcheck(Tensor<float>& p, const std::function<Tensor<float>()>& f, const Tensor<float>& dy,
               double tol) {
    auto loss = [&]() {
        NoGradGuard g;
        Tensor<float> y = host(f());
        double s = 0;
        for (size_t i = 0; i < y.total_elements(); ++i) s += (double)y.data()[i] * dy.data()[i];
        return s;
    };
    Tensor<float> g = host(p.grad());
    const float eps = 1e-2f;
    for (size_t i = 0; i < p.total_elements(); i += std::max<size_t>(1, p.total_elements() / 13)) {
        const float old = p.data()[i];
        p.data()[i] = old + eps; const double hi = loss();
        p.data()[i] = old - eps; const double lo = loss();
        p.data()[i] = old;
        const double fd = (hi - lo) / (2 * eps);
        if (std::fabs(fd - g.data()[i]) > tol * (1 + std::fabs(fd)))
            std::printf("  %s: grad[%zu] %.6f vs fd %.6f\n", g_cur, i, g.data()[i], fd);
        CHECK(std::fabs(fd - g.data()[i]) <= tol * (1 + std::fabs(fd)));
    }
}

TEST_CPU(cpu_linear_module_and_F_linear) {
    Linear<float> lin(7, 5);
    CHECK(lin.weight_.shape() == (std::vector<size_t>{7, 5}));
    CHECK(lin.bias_.shape() == (std::vector<size_t>{1, 5}));
    Tensor<float> x = uniform({4, 7}, 9);
    Tensor<float> y = lin.forward(x);
    Tensor<float> ref = matmul(x, lin.weight_) + lin.bias_;
    check_close(y, ref, 7, amax(x), amax(lin.weight_), 1e-6);
    // F::linear with the PyTorch layout gives the same result from wᵀ
    Tensor<float> w = lin.weight_.transpose(0, 1).contiguous();
    check_close(F::linear(x, w, lin.bias_.reshape({5})), y, 7, amax(x), amax(w), 1e-6);
    // backward vs finite differences (the reference's gradcheck recipe)
    Tensor<float> dy = uniform({4, 5}, 10);
    Tensor<float> xs = uniform({4, 7}, 11);
    xs.set_requires_grad(true);
    Tensor<float> out = lin.forward(xs);
    out.grad() = dy;
    out.backward();
    gradcheck(lin.weight_, [&]() { return lin.forward(xs); }, dy, 2e-3);
    gradcheck(lin.bias_, [&]() { return lin.forward(xs); }, dy, 2e-3);
    gradcheck(xs, [&]() { return lin.forward(xs); }, dy, 2e-3);
}

TEST_CPU(cpu_conv_module_backward_gradcheck) {
    Conv2D<float> conv(3, 4, 3, 2, 1);
    Tensor<float> x = uniform({2, 3, 7, 6}, 5);
    x.set_requires_grad(true);
    conv.bias_.fill(0.1f);
    Tensor<float> y = conv.forward(x);
    Tensor<float> dy = uniform(y.shape(), 6);
    y.grad() = dy;
    y.backward();
    gradcheck(conv.weight_, [&]() { return conv.forward(x); }, dy, 2e-3);
    gradcheck(conv.bias_, [&]() { return conv.forward(x); }, dy, 2e-3);
    gradcheck(x, [&]() { return conv.forward(x); }, dy, 2e-3);
}

TEST_CPU(cpu_dispatch_registry) {
    auto* fn = OpRegistry<float>::instance().lookup_binary(OpType::Matmul);
    CHECK(fn != nullptr);
    Tensor<float> out({2, 2});
    dispatch_binary_op(OpType::Matmul, mat23(), mat32(), out);
    CHECK_EQ_F(out.data()[0], 58); CHECK_EQ_F(out.data()[3], 154);
    CHECK(OpRegistry<float>::instance().lookup_binary(OpType::Conv2D) != nullptr);
    // 5x5 input, 2x2 kernel of ones, 4x4 output: only stride 1 without
    // padding gives it (padding 1 gives 6, 3 or 2 columns)
    Tensor<float> x({1, 1, 5, 5}), w({1, 1, 2, 2}), y({1, 1, 4, 4});
    for (int i = 0; i < 25; ++i) x.data()[i] = (float)(i + 1);
    w.fill(1);
    dispatch_binary_op(OpType::Conv2D, x, w, y);
    CHECK_EQ_F(y.data()[0], 16); CHECK_EQ_F(y.data()[15], 88);
}


// ---- the CPU device against the reference's own outputs -----------------------
// tests/golden/make_golden.py ran the reference's CPU code (built from its
// headers) on these inputs; the CPU device computes in the same order, so
// every result must match bit for bit.
TEST_CPU(cpu_golden_matmul_and_views) {
    CHECK(max_err(matmul(gold("dense_a"), gold("dense_b")), gold("dense_c")) == 0);
    // A: rows 2..4 of a [5,5] storage (offset 10); B: [5,4] at offset 3
    Tensor<float> A = gold("offset_a_store").as_strided({3, 5}, {5, 1}, 10);
    Tensor<float> B = gold("offset_b_store").as_strided({5, 4}, {4, 1}, 3);
    CHECK(max_err(matmul(A, B), gold("offset_c")) == 0);
    CHECK(max_err(matmul(gold("bT_a"), gold("bT_bt").transpose(0, 1)), gold("bT_c")) == 0);
    Tensor<float> row = gold("expand_row").reshape({1, 40}).expand({17, 40});
    CHECK(max_err(matmul(row, gold("expand_b")), gold("expand_c")) == 0);
}

TEST_CPU(cpu_golden_conv_forward) {
    CHECK(max_err(conv2d(gold("conv_x"), gold("conv_w"), gold("conv_b"), 2, 1),
                  gold("conv_out")) == 0);
}

TEST_CPU(cpu_golden_linear_forward_backward) {
    // the reference's Linear: Y = matmul(X, W_ref) + b with W_ref [in,out], b [1,out]
    Tensor<float> x = gold("lin_x"), w = gold("lin_w_ref");
    Tensor<float> b = gold("lin_b").reshape({1, w.shape()[1]});
    for (auto* t : {&x, &w, &b}) t->set_requires_grad(true);
    Tensor<float> y = matmul(x, w) + b;
    CHECK(max_err(y, gold("lin_y")) == 0);
    y.grad() = gold("lin_dy");
    y.backward();
    CHECK(max_err(x.grad(), gold("lin_dx")) == 0);
    CHECK(max_err(w.grad(), gold("lin_dw_ref")) == 0);
    CHECK(max_err(b.grad().reshape({b.shape()[1]}), gold("lin_db")) == 0);
}

TEST_CPU(cpu_golden_conv_backward) {
    // three images: dW and db summed per image, then added, as the reference does
    for (const char* tag : {"s1", "s2"}) {
        const std::string k = std::string("cbwd_") + tag + "_";
        Tensor<float> geom = gold(k + "geom");
        const size_t st = (size_t)geom.data()[0], pad = (size_t)geom.data()[1];
        Tensor<float> x = gold(k + "x"), w = gold(k + "w");
        Tensor<float> b({w.shape()[0]});
        b.fill(0.f);
        for (auto* t : {&x, &w, &b}) t->set_requires_grad(true);
        Tensor<float> y = conv2d(x, w, b, st, pad);
        y.grad() = gold(k + "dy");
        y.backward();
        CHECK(max_err(x.grad(), gold(k + "dx")) == 0);
        CHECK(max_err(w.grad(), gold(k + "dw")) == 0);
        CHECK(max_err(b.grad(), gold(k + "db")) == 0);
    }
}

TEST_CPU(cpu_dispatch_conv2d_infers_stride) {
    // OpType::Conv2D gets (input, weight, out) only: stride 1 with the padding
    // that gives out's size, else the "same" padding (kh-1)/2 with the stride
    // that does; both against conv2d
    Tensor<float> x = uniform({2, 3, 11, 10}, 71), w = uniform({4, 3, 3, 3}, 72);
    for (size_t stride : {1u, 2u, 3u}) {
        const size_t pad = 1;
        Tensor<float> want = conv2d(x, w, Tensor<float>(), stride, pad);
        Tensor<float> out(want.shape());
        dispatch_binary_op(OpType::Conv2D, x, w, out);
        CHECK(max_err(out, want) == 0);
    }
    Tensor<float> bad({2, 4, 50, 50});
    CHECK_THROWS(dispatch_binary_op(OpType::Conv2D, x, w, bad), std::invalid_argument);
    // a "full" convolution (stride 1, padding kh - 1) is the only fit of its shape
    Tensor<float> full_want = conv2d(x, w, Tensor<float>(), 1, 2);
    Tensor<float> full(full_want.shape());
    dispatch_binary_op(OpType::Conv2D, x, w, full);
    CHECK(max_err(full, full_want) == 0);
}

TEST_CPU(cpu_dispatch_conv2d_refuses_ambiguous_shapes) {
    // 9x9 input, 3x3 kernel, 3x3 output: stride 3 with padding 0, and stride 3
    // or 4 with padding 1, all give it; 4x4 -> 2x2: stride 1 unpadded or the
    // stride-2 "same" downsample.  The registry cannot tell them apart: it
    // throws, and the caller states stride and padding to conv2d.
    Tensor<float> x = uniform({1, 2, 9, 9}, 81), w = uniform({3, 2, 3, 3}, 82);
    Tensor<float> out({1, 3, 3, 3});
    CHECK_THROWS(dispatch_binary_op(OpType::Conv2D, x, w, out), std::invalid_argument);
    Tensor<float> x4 = uniform({1, 2, 4, 4}, 83), out4({1, 3, 2, 2});
    CHECK_THROWS(dispatch_binary_op(OpType::Conv2D, x4, w, out4), std::invalid_argument);
    // the explicit call computes the intended stride-3, unpadded layer: each
    // output is one whole 3x3 window of the input
    Tensor<float> y = conv2d(x, w, Tensor<float>(), 3, 0);
    CHECK(y.shape() == out.shape());
    for (size_t co = 0; co < 3; ++co)
        for (size_t oh = 0; oh < 3; ++oh)
            for (size_t ow = 0; ow < 3; ++ow) {
                double acc = 0;
                for (size_t ci = 0; ci < 2; ++ci)
                    for (size_t r = 0; r < 3; ++r)
                        for (size_t t = 0; t < 3; ++t)
                            acc += (double)x.data()[(ci * 9 + oh * 3 + r) * 9 + ow * 3 + t] *
                                   w.data()[((co * 2 + ci) * 3 + r) * 3 + t];
                CHECK(std::abs(y.data()[(co * 3 + oh) * 3 + ow] - acc) < 1e-5);
            }
    // a 1x1 output is computed the same way at every stride, so it is one
    // candidate per padding; a 3x3 input and kernel give 1x1 with padding 0
    // (any stride), 1 (stride >= 3) and 2 (stride >= 5): three
    Tensor<float> x3 = uniform({1, 2, 3, 3}, 84), out1({1, 3, 1, 1});
    CHECK_THROWS(dispatch_binary_op(OpType::Conv2D, x3, w, out1), std::invalid_argument);
}

// =====================================================================
// GPU device
// =====================================================================
TEST_GPU(gpu_matmul_known_answer) {  // tensor_test.cpp:285-316
    Tensor<float> C = host(matmul(mat23().to(GPU), mat32().to(GPU)));
    CHECK_EQ_F(C.data()[0], 58); CHECK_EQ_F(C.data()[1], 64);
    CHECK_EQ_F(C.data()[2], 139); CHECK_EQ_F(C.data()[3], 154);
}

TEST_GPU(gpu_gradients_fills) {  // tensor_test.cpp:490-510
    Tensor<float> A({2, 3}, GPU), B({3, 2}, GPU);
    A.fill(2); B.fill(3);
    A.set_requires_grad(true); B.set_requires_grad(true);
    Tensor<float> C = matmul(A, B);
    C.backward();
    CHECK_EQ_F(val(A.grad(), 0), 6);
    CHECK_EQ_F(val(B.grad(), 0), 4);
}

TEST_GPU(gpu_chained_matmul_plus_bias) {
    Tensor<float> A = mat23().to(GPU), B = mat32().to(GPU), C({2});
    C.data()[0] = 10; C.data()[1] = 20;
    Tensor<float> Cg = C.to(GPU);
    A.set_requires_grad(true); B.set_requires_grad(true); Cg.set_requires_grad(true);
    Tensor<float> D = matmul(A, B) + Cg;
    CHECK_EQ_F(val(D, 0), 68); CHECK_EQ_F(val(D, 3), 174);
    D.backward();
    CHECK_EQ_F(val(A.grad(), 2), 23);
    CHECK_EQ_F(val(B.grad(), 4), 9);
    CHECK_EQ_F(val(Cg.grad(), 0), 2); CHECK_EQ_F(val(Cg.grad(), 1), 2);
}

TEST_GPU(gpu_cpu_equivalence_views) {
    // a row/column slice with an offset (the reference's GPU path drops it), a
    // transpose view and an expand view, each against the CPU device
    Tensor<float> big = uniform({400, 300}, 1), b = uniform({250, 200}, 2);
    Tensor<float> a = big.slice(0, 37, 337).slice(1, 100, 300);            // [300,200]
    Tensor<float> Ag = big.to(GPU).slice(0, 37, 337).slice(1, 100, 300);
    Tensor<float> B = b.transpose(0, 1), Bg = b.to(GPU).transpose(0, 1);   // [200,250]
    check_close(matmul(Ag, Bg), matmul(a, B), 200, 1, 1);
    check_close(matmul(Ag.transpose(0, 1), Ag), matmul(a.transpose(0, 1), a), 300, 1, 1);
    Tensor<float> row = uniform({1, 300}, 3);
    check_close(matmul(row.to(GPU).expand({50, 300}), Ag), matmul(row.expand({50, 300}), a), 300,
                1, 1);
}

TEST_GPU(gpu_bmm_forward_backward) {
    Tensor<float> A = uniform({8, 33, 40}, 1), B = uniform({8, 40, 21}, 2);
    Tensor<float> Ag = A.to(GPU), Bg = B.to(GPU);
    A.set_requires_grad(true); B.set_requires_grad(true);
    Ag.set_requires_grad(true); Bg.set_requires_grad(true);
    Tensor<float> C = bmm(A, B), Cg = bmm(Ag, Bg);
    check_close(Cg, C, 40, 1, 1);
    Tensor<float> dy = uniform({8, 33, 21}, 3);
    C.grad() = dy;
    Cg.grad() = dy.to(GPU);
    C.backward();
    Cg.backward();
    check_close(Ag.grad(), A.grad(), 21, 1, 1);
    check_close(Bg.grad(), B.grad(), 33, 1, 1);
}

TEST_GPU(gpu_linear_config4_equivalence) {
    // benchmark config 4 shape through the Linear module (W_ref [2048,1000]) and F::linear.
    Linear<float> lin(2048, 1000);
    Tensor<float> x = uniform({256, 2048}, 42), dy = uniform({256, 1000}, 44, -0.01f, 0.01f);
    Linear<float> lg = lin;  // same parameters, moved to the GPU below
    lg.weight_ = lin.weight_.to(GPU);
    lg.bias_ = lin.bias_.to(GPU);
    lg.weight_.set_requires_grad(true);
    lg.bias_.set_requires_grad(true);
    Tensor<float> xg = x.to(GPU);
    x.set_requires_grad(true);
    xg.set_requires_grad(true);
    Tensor<float> y = lin.forward(x), yg = lg.forward(xg);
    check_close(yg, y, 2048, amax(x), amax(lin.weight_), 1e-6);
    y.grad() = dy;
    yg.grad() = dy.to(GPU);
    y.backward();
    yg.backward();
    check_close(xg.grad(), x.grad(), 1000, amax(dy), amax(lin.weight_));
    check_close(lg.weight_.grad(), lin.weight_.grad(), 256, amax(dy), amax(x));
    check_close(lg.bias_.grad(), lin.bias_.grad(), 256, amax(dy), 1);
    // F::linear (PyTorch layout) on the GPU equals the module
    Tensor<float> w = lg.weight_.transpose(0, 1);
    check_close(F::linear(xg, w, lg.bias_.reshape({1000})), yg, 2048, amax(x), amax(lin.weight_), 1e-6);
}

TEST_GPU(gpu_grad_accumulation_in_epilogue) {
    // A weight used twice: the second gradient is accumulated by the GEMM epilogue.
    Tensor<float> W = uniform({64, 48}, 1).to(GPU), x1 = uniform({32, 64}, 2).to(GPU),
                  x2 = uniform({32, 64}, 3).to(GPU);
    W.set_requires_grad(true);
    Tensor<float> y = matmul(x1, W) + matmul(x2, W);
    y.backward();
    Tensor<float> Wc = host(W);
    Wc.set_requires_grad(true);
    Tensor<float> yc = matmul(host(x1), Wc) + matmul(host(x2), Wc);
    yc.backward();
    check_close(W.grad(), Wc.grad(), 64, 2, 1, 1e-5);
}

TEST_GPU(gpu_conv_equivalence_and_backward) {
    // reference spatial_test.cpp:209-230 shape, plus a full backward
    Tensor<float> x = uniform({4, 3, 32, 32}, 1), w = uniform({16, 3, 3, 3}, 2), b({16});
    b.fill(0.1f);
    Tensor<float> xg = x.to(GPU), wg = w.to(GPU), bg = b.to(GPU);
    for (auto* t : {&x, &w, &b, &xg, &wg, &bg}) t->set_requires_grad(true);
    Tensor<float> y = conv2d(x, w, b, 2, 1), yg = conv2d(xg, wg, bg, 2, 1);
    check_close(yg, y, 27, 1, 1, 1e-5);
    Tensor<float> dy = uniform(y.shape(), 3);
    y.grad() = dy;
    yg.grad() = dy.to(GPU);
    y.backward();
    yg.backward();
    check_close(xg.grad(), x.grad(), 16 * 9, 1, 1);
    check_close(wg.grad(), w.grad(), 4 * 16 * 16, 1, 1);
    check_close(bg.grad(), b.grad(), 4 * 16 * 16, 1, 1);
}

TEST_GPU(gpu_conv_strided_input_views) {
    // conv2d reads non-contiguous NCHW inputs in place (reference conv2d_gpu_strided,
    // src/gpu_ops.cpp:2367-2399): channel slice (implicit GEMM, c_in = 16) and a
    // transposed view (explicit im2col, c_in = 3), against the CPU device on copies.
    Tensor<float> big = uniform({2, 20, 9, 10}, 4);
    Tensor<float> w16 = uniform({6, 16, 3, 3}, 5), b6 = uniform({6}, 6);
    Tensor<float> xs = big.to(GPU).slice(1, 2, 18);
    CHECK(!xs.is_contiguous());
    Tensor<float> want = conv2d(big.slice(1, 2, 18).contiguous(), w16, b6, 1, 1);
    check_close(conv2d(xs, w16.to(GPU), b6.to(GPU), 1, 1), want, 16 * 9, 1, 1, 1e-5);
    Tensor<float> t = uniform({2, 10, 3, 9}, 7);          // transpose(1, 2) -> [2, 3, 10, 9]
    Tensor<float> w3 = uniform({4, 3, 3, 3}, 8), b4 = uniform({4}, 9);
    Tensor<float> xt = t.to(GPU).transpose(1, 2);
    CHECK(!xt.is_contiguous());
    Tensor<float> want3 = conv2d(t.transpose(1, 2).contiguous(), w3, b4, 2, 1);
    check_close(conv2d(xt, w3.to(GPU), b4.to(GPU), 2, 1), want3, 27, 1, 1, 1e-5);
}

TEST_GPU(gpu_conv_backward_views) {
    // conv2d_backward_{input,weight,bias}_gpu on strided views: dY a transposed
    // view, dX and dW slices of wider tensors (their neighbours must survive),
    // dW and db accumulated with beta = 1 into a view; against the CPU device on
    // dense copies.  Both dX geometries: implicit (c_out = 16) and column buffer.
    for (size_t co : {16, 6}) {
        const size_t n = 2, c = 4, h = 7, w = 8, k = 3;
        Tensor<float> x = uniform({n, c, h, w}, 21), wt = uniform({co, c, k, k}, 22);
        Tensor<float> dyt = uniform({n, co, w, h}, 23);            // stored W-major
        Tensor<float> dy = dyt.transpose(2, 3).contiguous();       // [n, co, h, w]
        Tensor<float> dx_want({n, c, h, w}), dw_want({co, c, k, k}), db_want({co});
        conv2d_backward_input(dy, wt, dx_want, 1, 1);
        conv2d_backward_weight(dy, x, dw_want, 1, 1);
        conv2d_backward_bias(dy, db_want);

        Tensor<float> dyg = dyt.to(GPU).transpose(2, 3);
        CHECK(!dyg.is_contiguous());
        Tensor<float> dx_big({n, c + 3, h, w}, GPU);
        dx_big.fill(7.f);
        Tensor<float> dx = dx_big.slice(1, 1, 1 + c);
        CHECK(!dx.is_contiguous());
        conv2d_backward_input(dyg, wt.to(GPU), dx, 1, 1);
        check_close(dx, dx_want, co * k * k, 1, 1);
        CHECK_EQ_F(val(dx_big.slice(1, 0, 1).contiguous(), 5), 7.f);
        CHECK_EQ_F(val(dx_big.slice(1, c + 1, c + 2).contiguous(), 3), 7.f);

        Tensor<float> dw_big({co, c + 2, k, k}, GPU);
        dw_big.fill(1.f);
        Tensor<float> dw = dw_big.slice(1, 2, 2 + c);
        conv2d_backward_weight_gpu(dyg, x.to(GPU), dw, 1, 1, 1.f);   // dW = 1 + ∂L/∂W
        Tensor<float> ones({co, c, k, k});
        ones.fill(1.f);
        check_close(dw, dw_want + ones, n * h * w, 1, 1, 1e-6);
        CHECK_EQ_F(val(dw_big.slice(1, 0, 1).contiguous(), 0), 1.f);

        Tensor<float> db_big({2 * co}, GPU);
        db_big.fill(2.f);
        Tensor<float> db = db_big.as_strided({co}, {2}, 0);          // every other element
        conv2d_backward_bias_gpu(dyg, db, 1.f);                       // db = 2 + Σ dY
        Tensor<float> twos({co});
        twos.fill(2.f);
        check_close(db, db_want + twos, n * h * w, 1, 1, 1e-6);
        CHECK_EQ_F(val(db_big, 1), 2.f);
    }
}

void check_equal(const Tensor<float>& a, const Tensor<float>& b, const char* what) {
    Tensor<float> ha = host(a), hb = host(b);
    CHECK(ha.shape() == hb.shape());
    if (std::memcmp(ha.data(), hb.data(), ha.total_elements() * sizeof(float)) != 0) {
        std::printf("    %s differs\n", what);
        CHECK(false);
    }
}

TEST_GPU(gpu_graph_executor_training_loop) {
    // A Linear layer trained with SGD on L = ½‖x·W + b - y‖² through GraphExecutor
    // (eager warm-up, capture, replays; reference include/GraphExecutor.hpp:22-220),
    // next to a copy trained by the same steps run eagerly: every weight, bias and
    // loss gradient must be bit-identical, and the capture must allocate nothing.
    const float lr = 0.05f;
    Linear<float> a(64, 32, GPU), b(64, 32, GPU);
    copy_gpu_strided(a.weight_, b.weight_);
    copy_gpu_strided(a.bias_, b.bias_);
    for (Linear<float>* m : {&a, &b}) {
        m->weight_.grad() = Tensor<float>(m->weight_.shape(), GPU);
        m->bias_.grad() = Tensor<float>(m->bias_.shape(), GPU);
    }
    auto make_step = [lr](Linear<float>& m) {
        return [&m, lr](const Tensor<float>& x, const Tensor<float>& y) {
            m.weight_.grad().fill(0.f);
            m.bias_.grad().fill(0.f);
            Tensor<float> yh = m.forward(x);                 // one GEMM, bias fused
            Tensor<float> d(yh.shape(), yh.device());
            copy_gpu_strided(yh, d);
            mt_detail::axpby(y, -1.f, d, 1.f);               // dL/dyh = yh - y
            yh.grad() = d;
            yh.backward();                                    // dX-free: dW GEMM (+ db)
            mt_detail::axpby(m.weight_.grad(), -lr, m.weight_, 1.f);
            mt_detail::axpby(m.bias_.grad(), -lr, m.bias_, 1.f);
            return d;
        };
    };
    GraphExecutor<float> ex(make_step(a));
    auto eager = make_step(b);
    for (int it = 0; it < 5; ++it) {
        Tensor<float> x = uniform({128, 64}, 100 + it).to(GPU);
        Tensor<float> y = uniform({128, 32}, 200 + it).to(GPU);
        Tensor<float> d1 = ex.step(x, y);
        Tensor<float> d2 = eager(x, y);
        GPU_CHECK(hipDeviceSynchronize());
        check_equal(d1, d2, "loss gradient");
        check_equal(a.weight_, b.weight_, "weight");
        check_equal(a.bias_, b.bias_, "bias");
    }
    CHECK(ex.captured());
    CHECK(ex.capture_allocations() == 0);
    // a batch of another shape runs eagerly and still trains the same way
    Tensor<float> x = uniform({96, 64}, 300).to(GPU), y = uniform({96, 32}, 301).to(GPU);
    ex.step(x, y);
    eager(x, y);
    GPU_CHECK(hipDeviceSynchronize());
    check_equal(a.weight_, b.weight_, "weight after an eager step");
}

TEST_CPU(cpu_pool_reservation) {
    // Blocks handed out under a Reservation are not recycled until it ends.
    MemoryPool& pool = MemoryPool::get();
    void* p0 = pool.allocate(1000, CPU);
    pool.free(p0, 1000, CPU);                     // cached
    void* held = nullptr;
    {
        MemoryPool::Reservation r;
        r.start();
        held = pool.allocate(1000, CPU);          // reuses the cached block
        r.stop();
        CHECK(held == p0);
        CHECK(r.fresh_allocations() == 0);
        pool.free(held, 1000, CPU);               // held back for the reservation
        void* other = pool.allocate(1000, CPU);   // must not get the held block
        CHECK(other != held);
        pool.free(other, 1000, CPU);
    }
    void* again = pool.allocate(1000, CPU);       // the held block is back in the cache
    void* again2 = pool.allocate(1000, CPU);
    CHECK(again == held || again2 == held);
    pool.free(again, 1000, CPU);
    pool.free(again2, 1000, CPU);
}

TEST_GPU(gpu_contiguous_and_dispatch) {
    Tensor<float> a = uniform({37, 53}, 1);
    Tensor<float> t = a.to(GPU).transpose(0, 1);
    Tensor<float> c = t.contiguous();
    CHECK(c.is_contiguous() && c.offset() == 0);
    check_close(c, a.transpose(0, 1).contiguous(), 1, 0, 0);
    Tensor<float> out({2, 2}, GPU);
    dispatch_binary_op(OpType::Matmul, mat23().to(GPU), mat32().to(GPU), out);
    CHECK_EQ_F(val(out, 0), 58); CHECK_EQ_F(val(out, 3), 154);
    CHECK_THROWS(matmul(mat23().to(GPU), mat32()), std::invalid_argument);
}


// The reference's modules and launchers by name on the GPU device, each
// against the CPU device (itself pinned to the reference by the golden tests).
// Conv2D<float> is the reference's main GPU consumer (test/resnet.cpp,
// test/mnist.cpp): a ResNet-like 3x3 (implicit GEMM), a strided 3x3 and a
// c_in = 3 stem layer (explicit im2col), forward and backward.
TEST_GPU(gpu_conv2d_module_forward_backward) {
    struct Layer { size_t n, c, h, w, co, k, st, pad; };
    for (const Layer& L : {Layer{4, 64, 14, 14, 64, 3, 1, 1}, Layer{2, 32, 15, 15, 64, 3, 2, 1},
                           Layer{2, 3, 32, 32, 16, 7, 2, 3}}) {
        Conv2D<float> m(L.c, L.co, L.k, L.st, L.pad);        // CPU parameters
        m.bias_.fill(0.05f);
        Conv2D<float> mg = m;                                // the same values on the GPU
        mg.to(GPU);
        mg.weight_.set_requires_grad(true);
        mg.bias_.set_requires_grad(true);
        Tensor<float> x = uniform({L.n, L.c, L.h, L.w}, 80 + (unsigned)L.c);
        Tensor<float> xg = x.to(GPU);
        x.set_requires_grad(true);
        xg.set_requires_grad(true);
        Tensor<float> y = m.forward(x), yg = mg.forward(xg);
        CHECK(yg.device().is_gpu());
        const size_t kg = L.c * L.k * L.k;
        check_close(yg, y, kg, 1, amax(m.weight_), 1e-6);
        Tensor<float> dy = uniform(y.shape(), 90 + (unsigned)L.c);
        y.grad() = dy;
        yg.grad() = dy.to(GPU);
        y.backward();
        yg.backward();
        const size_t np = L.n * y.shape()[2] * y.shape()[3];
        check_close(xg.grad(), x.grad(), L.co * L.k * L.k, 1, amax(m.weight_));
        check_close(mg.weight_.grad(), m.weight_.grad(), np, 1, 1);
        check_close(mg.bias_.grad(), m.bias_.grad(), np, 1, 1);
    }
}

TEST_GPU(gpu_F_conv2d_golden) {
    Tensor<float> y = F::conv2d(gold("conv_x").to(GPU), gold("conv_w").to(GPU),
                                gold("conv_b").to(GPU), 2, 1);
    CHECK(y.device().is_gpu());
    check_close(y, gold("conv_out"), 27, amax(gold("conv_x")), amax(gold("conv_w")), 1e-6);
}

TEST_GPU(gpu_matmul_launchers_by_name) {
    // the reference's benchmark calls these by name (test/benchmark.cpp:225-251)
    const Tensor<float> a = gold("dense_a").to(GPU), b = gold("dense_b").to(GPU);
    const Tensor<float> want = gold("dense_c");
    const float am = amax(gold("dense_a")), bm = amax(gold("dense_b"));
    Tensor<float> c1({64, 80}, GPU), c2({64, 80}, GPU), c3({64, 80}, GPU), c4({33, 29}, GPU);
    matmul_gpu<float>(a, b, c1);
    matmul_gpu_v2<float>(a, b, c2);
    matmul_gpu_bk16<float>(a, b, c3);
    matmul_gpu_strided<float>(gold("bT_a").to(GPU), gold("bT_bt").to(GPU).transpose(0, 1), c4);
    for (Tensor<float>* c : {&c1, &c2, &c3}) check_close(*c, want, 96, am, bm);
    check_close(c4, gold("bT_c"), 47, 1, 1);
}

TEST_GPU(gpu_dispatch_conv2d) {
    // OpType::Conv2D on the GPU: stride 1 and the inferred strides 2 and 3
    Tensor<float> x = uniform({2, 16, 13, 12}, 73), w = uniform({8, 16, 3, 3}, 74);
    for (size_t stride : {1u, 2u, 3u}) {
        Tensor<float> want = conv2d(x, w, Tensor<float>(), stride, 1);
        Tensor<float> out(want.shape(), GPU);
        dispatch_binary_op(OpType::Conv2D, x.to(GPU), w.to(GPU), out);
        check_close(out, want, 144, 1, 1);
    }
    // shapes that several stride/padding pairs give are refused on the GPU too
    Tensor<float> x9 = uniform({1, 16, 9, 9}, 85);
    Tensor<float> out9({1, 8, 3, 3}, GPU);
    CHECK_THROWS(dispatch_binary_op(OpType::Conv2D, x9.to(GPU), w.to(GPU), out9),
                 std::invalid_argument);
    Tensor<float> want9 = conv2d(x9, w, Tensor<float>(), 3, 0);
    check_close(conv2d(x9.to(GPU), w.to(GPU), Tensor<float>(), 3, 0), want9, 144, 1, 1);
}

TEST_GPU(gpu_sum_and_copy_launchers_by_name) {
    // sum_gpu(input, axis, keepdims) and copy_gpu_strided(src, T* dst) with the
    // reference's signatures (include/TensorOps.hpp:707, 717)
    Tensor<float> a = uniform({5, 7, 9}, 75);
    Tensor<float> ag = a.to(GPU).transpose(0, 2);            // a strided view [9,7,5]
    Tensor<float> ac = a.transpose(0, 2);
    for (size_t axis = 0; axis < 3; ++axis)
        for (bool keep : {false, true}) {
            Tensor<float> got = sum_gpu(ag, axis, keep);
            Tensor<float> want = sum_cpu(ac, axis, keep);
            CHECK(got.shape() == want.shape());
            check_close(got, want, ac.shape()[axis], 1, 1);
        }
    Tensor<float> dense({9, 7, 5}, GPU);
    copy_gpu_strided<float>(ag, dense.data());
    CHECK(max_err(dense, ac.contiguous()) == 0);
}

TEST_GPU(gpu_graph_executor_step_throws_during_capture) {
    // a step that fails while it is being captured: the exception propagates,
    // the stream leaves capture mode, this thread's allocations are no longer
    // pinned, and the next step runs eagerly and correctly
    int calls = 0;
    Tensor<float> w = uniform({16, 8}, 76).to(GPU);
    GraphExecutor<float> ex([&](const Tensor<float>& x, const Tensor<float>&) {
        if (++calls == 2) throw std::runtime_error("step failed");
        return matmul(x, w);
    });
    Tensor<float> x = uniform({4, 16}, 77).to(GPU), y = uniform({4, 8}, 78).to(GPU);
    ex.step(x, y);                                           // eager warm-up
    CHECK_THROWS(ex.step(x, y), std::runtime_error);         // the capture throws
    hipStreamCaptureStatus st = hipStreamCaptureStatusActive;
    GPU_CHECK(hipStreamIsCapturing(ex.stream(), &st));
    CHECK(st == hipStreamCaptureStatusNone);
    CHECK(!MemoryPool::Reservation::active_on_this_thread());
    CHECK(!ex.captured());
    Tensor<float> out = ex.step(x, y);                       // eager again
    GPU_CHECK(hipDeviceSynchronize());
    check_close(out, matmul(host(x), host(w)), 16, 1, 1);
    ex.step(x, y);                                           // captures now
    CHECK(ex.captured());
}

}  // namespace

int main(int argc, char** argv) {
    const bool want_gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
    const bool want_cpu = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
    if (argc > 3 && std::strcmp(argv[2], "--golden") == 0) g_golden_path = argv[3];
    if (!want_gpu && !want_cpu) {
        std::printf("usage: %s --cpu | --gpu [--golden FILE]\n", argv[0]);
        return 2;
    }
    int ran = 0;
    for (auto& c : cases()) {
        if (c.gpu != want_gpu) continue;
        g_cur = c.name;
        const int before = g_fail;
        std::printf("[ RUN  ] %s\n", c.name);
        std::fflush(stdout);
        try {
            c.fn();
        } catch (const std::exception& e) {
            std::printf("  FAIL %s: exception %s\n", c.name, e.what());
            ++g_fail;
        }
        std::printf("[ %s ] %s\n", g_fail == before ? " OK " : "FAIL", c.name);
        std::fflush(stdout);
        ++ran;
    }
    std::printf("%d tests, %d failures\n", ran, g_fail);
    return g_fail ? 1 : 0;
}
