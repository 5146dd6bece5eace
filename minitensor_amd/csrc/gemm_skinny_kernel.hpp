// gemm_skinny_kernel.hpp -- the HBM-bound GEMM shapes, on the vector ALUs.
//
// Two shapes of the reference's matmul benchmark (test/benchmark.cpp:732,
// 737-738) carry almost no arithmetic per byte:
//   * vector x matrix, C[1,4096] = A[1,4096]·B[4096,4096]: every element of B
//     is used once (0.5 flop per byte), so the work is streaming 64 MiB of B;
//   * the outer product, C[4096,4096] = A[4096,1]·B[1,4096]: K = 1, so the
//     work is writing 64 MiB of C.
// A 32x32 MFMA tile pads the first to 32 rows (31 of them zero) and the second
// to a 16-deep K chunk, and stages both through LDS; these kernels instead
// stream the large operand (or the output) with 16-byte accesses and do the
// few multiply-adds on the vector ALUs.
//
// gemv_mv_f32<MR>: M <= MR <= 8 rows, B mn-contiguous (row-major B).  A
//   workgroup of 4 waves owns 256 consecutive columns (a lane 4 of them, one
//   16-byte load per row of B: a wave reads a 1 KB row segment) and a K range;
//   wave w takes the rows k = w, w+4, w+8, ... of the range, 16 loads in
//   flight, with the range's slice of A in LDS ([k][MR], one broadcast read
//   per k).  The four waves' sums meet in LDS in wave order.
// gemv_kv_f32<MR>: M <= MR <= 8 rows, B k-contiguous (Bᵀ views: the Linear
//   layer's x·Wᵀ with a few samples).  A workgroup owns 16 columns n, one per
//   16-lane group; a group reads 256 contiguous bytes of its column's k run
//   per load (8 loads in flight), multiplies them with A's slice in LDS
//   ([MR][k]), and folds its 16 lanes with a fixed butterfly.
// rankk_f32<KMAX>: K <= KMAX <= 16.  A workgroup writes 16 rows of 1024
//   consecutive columns, a thread four of them: B's K x 4 block in registers,
//   A's 16 x K block in LDS, one 16-byte store per row.
// GEMV workgroups may split K: each writes the raw partial of its split to the
// workspace ([split][batch][M][N], as the MFMA kernels' split-K) and
// skinny_reduce_f32 sums the splits in a fixed order.  Every sum here has a
// fixed order: results are deterministic.
// Host contract (checked in the dispatcher, mtgemm_api.hip): p.tiles_n is the
// number of column groups (256, 16 or 1024 columns), p.tiles_m the number of
// 16-row groups (rank-k), every split's K range non-empty; GEMV: M <= MR,
// N % 4 == 0, B 16-byte aligned with B's k stride (MV) or n stride (KV) a
// multiple of 4 and K % 4 == 0 (KV); rank-k: 1 <= K <= KMAX.
#pragma once

#include "gemm_configs.hpp"
#include "gemm_kernel.hpp"

namespace mtk {

constexpr int kGemvMvSlice = 512;  // k rows of A staged at a time (MV)
constexpr int kGemvMvWavesFew = 8;   // waves per MV workgroup for 1-2 rows of A
constexpr int kGemvMvWavesMany = 4;  // ... for 4-8 rows (the LDS sums: W x MR x 1 KB)
constexpr int kGemvMvRowsInFlight = 32;  // per workgroup and buffer: U = 32 / W per lane
constexpr int kGemvKvLds = 8192;   // floats of A staged at a time (KV): MR x slice

// Waves per GEMV (MV) workgroup, by rows of A: they split the workgroup's K
// range (row k to wave k % W); their partial sums meet in LDS, W x MR x 1 KB.
template <int MR>
constexpr int gemv_mv_waves() { return MR <= 2 ? kGemvMvWavesFew : kGemvMvWavesMany; }

template <int MR>
__global__ void __launch_bounds__(64 * gemv_mv_waves<MR>()) gemv_mv_f32(GemmParams p) {
    static_assert(MR == 1 || MR == 2 || MR == 4 || MR == 8, "MR: 1, 2, 4 or 8 rows");
    constexpr int W = gemv_mv_waves<MR>();
    constexpr int NT = 64 * W;
    constexpr int U = kGemvMvRowsInFlight / W;   // loads in flight per lane and buffer
    constexpr int LDS = W * MR * 256 > kGemvMvSlice * MR ? W * MR * 256 : kGemvMvSlice * MR;
    static_assert(kGemvMvSlice % W == 0, "a slice holds whole rounds of rows");
    __shared__ __attribute__((aligned(16))) float lds[LDS];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int cb = blockIdx.x % p.tiles_n;
    const int rest = blockIdx.x / p.tiles_n;
    const int split = rest % p.splits, bz = rest / p.splits;
    const int kb = split * p.k_per_split;
    const int ke = min(p.K, kb + p.k_per_split);
    const float* const Ab = p.A + (int64_t)bz * p.a_b;
    const int n = cb * kGemvMvCols + 4 * lane;
    // lanes past N read the last valid column group and store nothing
    const float* const Bc = p.B + (int64_t)bz * p.b_b + min(n, p.N - 4);

    f32x4 acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int s0 = kb; s0 < ke; s0 += kGemvMvSlice) {
        const int slen = min(kGemvMvSlice, ke - s0);
        // rows wave + W*i of the slice
        const int nrow = (slen - wave + W - 1) / W;
        // U rows from i0 on; past the last row it re-reads that row, and a wave
        // without rows reads the slice's first (all unused)
        auto load = [&](f32x4 (&b)[U], int i0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int r = nrow > 0 ? wave + W * min(i0 + u, nrow - 1) : 0;
                b[u] = *reinterpret_cast<const f32x4*>(Bc + (int64_t)(s0 + r) * p.b_k);
            }
        };
        auto fma_rows = [&](const f32x4 (&b)[U], int i0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (i0 + u >= nrow) break;   // wave-uniform
                const float* const a = lds + (wave + W * (i0 + u)) * MR;
#pragma unroll
                for (int m = 0; m < MR; ++m) acc[m] += a[m] * b[u];
            }
        };
        f32x4 b0[U], b1[U];
        load(b0, 0);   // in flight while A's slice is staged
        __syncthreads();   // the previous slice's reads of A are done
        for (int e = t; e < slen * MR; e += NT) {
            const int kk = e / MR, m = e % MR;
            lds[e] = m < p.M ? Ab[(int64_t)m * p.a_mn + (int64_t)(s0 + kk) * p.a_k] : 0.f;
        }
        __syncthreads();
        // two buffers of U rows: the next U load while the current U multiply
        int i0 = 0;
        for (; i0 + U < nrow; i0 += 2 * U) {
            load(b1, i0 + U);
            fma_rows(b0, i0);
            if (i0 + 2 * U < nrow) load(b0, i0 + 2 * U);
            fma_rows(b1, i0 + U);
        }
        if (i0 < nrow) fma_rows(b0, i0);
    }
    __syncthreads();
    f32x4* const red = reinterpret_cast<f32x4*>(lds);
#pragma unroll
    for (int m = 0; m < MR; ++m) red[(wave * MR + m) * 64 + lane] = acc[m];
    __syncthreads();
    const bool part = p.splits > 1 || p.part;
    float* const base = part ? p.ws + ((int64_t)split * p.batch + bz) * (int64_t)p.M * p.N
                             : p.C + (int64_t)bz * p.c_b;
    const int64_t rs = part ? (int64_t)p.N : p.c_m;
    for (int e = t; e < MR * 64; e += NT) {
        const int m = e >> 6, l = e & 63;
        const int nn = cb * kGemvMvCols + 4 * l;
        if (m >= p.M || nn >= p.N) continue;
        f32x4 v = red[m * 64 + l];
#pragma unroll
        for (int w = 1; w < W; ++w) v += red[(w * MR + m) * 64 + l];
        store_group4(p, base, rs, part, part ? p.ws_vec : p.c_vec, part ? 0 : p.bias_axis,
                     part ? 0.f : p.beta, m, nn, v);
    }
}

template <int MR>
__global__ void __launch_bounds__(256) gemv_kv_f32(GemmParams p) {
    static_assert(MR == 1 || MR == 2 || MR == 4 || MR == 8, "MR: 1, 2, 4 or 8 rows");
    constexpr int U = 8;                 // loads in flight per lane
    constexpr int SL = kGemvKvLds / MR;  // k per staged slice (a multiple of 64)
    __shared__ __attribute__((aligned(16))) float lds[kGemvKvLds];
    const int t = threadIdx.x;
    const int g = t >> 4, gl = t & 15;   // 16-lane group g owns column n0 + g
    const int cb = blockIdx.x % p.tiles_n;
    const int rest = blockIdx.x / p.tiles_n;
    const int split = rest % p.splits, bz = rest / p.splits;
    const int kb = split * p.k_per_split;
    const int ke = min(p.K, kb + p.k_per_split);
    const float* const Ab = p.A + (int64_t)bz * p.a_b;
    const int n = cb * kGemvKvCols + g;
    // groups past N read the last column and store nothing
    const float* const Bn = p.B + (int64_t)bz * p.b_b + (int64_t)min(n, p.N - 1) * p.b_mn;

    f32x4 acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int s0 = kb; s0 < ke; s0 += SL) {
        const int slen = min(SL, ke - s0);   // a multiple of 4 (K % 4 == 0, kps % 64 == 0)
        const int nj = (slen + 63) >> 6;     // 64-deep steps of a group
        __syncthreads();
        // A(m, s0 + kk) -> lds[m*SL + kk], zero up to the last step's end
#pragma unroll
        for (int m = 0; m < MR; ++m)
            for (int kk = t; kk < nj * 64; kk += 256)
                lds[m * SL + kk] = (m < p.M && kk < slen)
                                       ? Ab[(int64_t)m * p.a_mn + (int64_t)(s0 + kk) * p.a_k]
                                       : 0.f;
        __syncthreads();
        const float* const bs = Bn + s0 + 4 * gl;
        for (int j0 = 0; j0 < nj; j0 += U) {
            f32x4 b[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = min(j0 + u, nj - 1);
                const int kk = 4 * gl + 64 * j;
                // lanes past the slice's end re-read its last 16 bytes and use zeros
                const int kc = min(kk, slen - 4) - 4 * gl;
                b[u] = *reinterpret_cast<const f32x4*>(bs + kc);
                if (kk >= slen) b[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (j0 + u >= nj) break;   // uniform
                const int kk = 4 * gl + 64 * (j0 + u);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const f32x4 a = *reinterpret_cast<const f32x4*>(lds + m * SL + kk);
                    acc[m] += a * b[u];
                }
            }
        }
    }
    // fold each lane's four columns, then the group's 16 lanes (fixed butterfly)
    float s[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        s[m] = (acc[m][0] + acc[m][1]) + (acc[m][2] + acc[m][3]);
#pragma unroll
        for (int x = 8; x >= 1; x >>= 1) s[m] += __shfl_xor(s[m], x, 16);
    }
    if (gl != 0 || n >= p.N) return;
    const bool part = p.splits > 1 || p.part;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        if (m >= p.M) break;
        if (part) {
            p.ws[(((int64_t)split * p.batch + bz) * p.M + m) * p.N + n] = s[m];
            continue;
        }
        float o = s[m];
        if (p.bias_axis == 1) o += p.bias[(int64_t)m * p.bias_stride];
        if (p.bias_axis == 2) o += p.bias[(int64_t)n * p.bias_stride];
        float* const dst = p.C + (int64_t)bz * p.c_b + (int64_t)m * p.c_m + col_offset(p, n);
        if (p.beta != 0.f) o += p.beta * *dst;
        *dst = o;
    }
}

template <int KMAX>
__global__ void __launch_bounds__(256) rankk_f32(GemmParams p) {
    static_assert(KMAX % 4 == 0, "A's rows are read from LDS 16 bytes at a time");
    __shared__ __attribute__((aligned(16))) float la[kRankKRows * KMAX];
    const int t = threadIdx.x;
    const int cb = blockIdx.x % p.tiles_n;
    const int rest = blockIdx.x / p.tiles_n;
    const int rb = rest % p.tiles_m, bz = rest / p.tiles_m;
    const int m0 = rb * kRankKRows;
    const float* const Ab = p.A + (int64_t)bz * p.a_b;
    const float* const Bb = p.B + (int64_t)bz * p.b_b;
    const int n = cb * kRankKCols + 4 * t;
    // B's K x 4 block first, so that its loads are in flight with A's (one
    // memory round trip before the first store instead of two); one 16-byte
    // load per k where the four columns are contiguous and aligned.
    // (Every index into b is a compile-time constant -- whole unrolled loops,
    // a uniform k < K test instead of a break -- so that b stays in registers:
    // with a runtime-bounded loop the 16-deep instance kept it in scratch and
    // took 128 us at K = 16, against 22 us for the MFMA kernel at K = 17.)
    f32x4 b[KMAX];
    const bool bvec = p.b_mn == 1 && n + 3 < p.N && ((uintptr_t)(Bb + n) & 15u) == 0 &&
                      (p.b_k & 3) == 0;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
        if (k < p.K) {
            if (bvec) {
                x = *reinterpret_cast<const f32x4*>(Bb + n + (int64_t)k * p.b_k);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (n + c < p.N) x[c] = Bb[(int64_t)(n + c) * p.b_mn + (int64_t)k * p.b_k];
            }
        }
        b[k] = x;
    }
    for (int e = t; e < kRankKRows * KMAX; e += 256) {
        const int r = e / KMAX, k = e % KMAX, m = m0 + r;
        la[e] = (m < p.M && k < p.K) ? Ab[(int64_t)m * p.a_mn + (int64_t)k * p.a_k] : 0.f;
    }
    __syncthreads();
    if (n >= p.N) return;
    float* const Cb = p.C + (int64_t)bz * p.c_b;
    const int rows = min(kRankKRows, p.M - m0);
    // Row r's sum over k in order, A's row read from LDS 16 bytes at a time
    // (one ds_read_b32 per k per row had made K the kernel's cost: 0.9 us
    // per unit of K at 2048 x 2048).
    auto row_sum = [&](int r) {
        const f32x4* const a4 = reinterpret_cast<const f32x4*>(la + r * KMAX);
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < KMAX / 4; ++q) {
            if (4 * q >= p.K) continue;   // uniform
            const f32x4 a = a4[q];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (4 * q + e < p.K) v += a[e] * b[4 * q + e];
        }
        return v;
    };
    // 16-byte stores without a row bias or beta: the only epilogue loads are
    // the column biases, the same for every row, landed before the first
    // store.  (A load between two stores waits for the first, since vmcnt
    // counts both: with the general epilogue each row waited for the
    // previous row's store, 9.6 us for a 1024 x 4096 output.)
    if (p.c_vec && p.c_n_inner >= p.N && p.bias_axis != 1 && p.beta == 0.f) {
        f32x4 bc = {0.f, 0.f, 0.f, 0.f};
        if (p.bias_axis == 2)
#pragma unroll
            for (int x = 0; x < 4; ++x) bc[x] = p.bias[(int64_t)(n + x) * p.bias_stride];
        float* const c0 = Cb + (int64_t)m0 * p.c_m + n;
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));   // no store is in flight yet
#pragma unroll
        for (int r = 0; r < kRankKRows; ++r)
            if (r < rows) {   // uniform
                f32x4 o = row_sum(r);
                if (p.bias_axis == 2) o += bc;
                *reinterpret_cast<f32x4*>(c0 + (int64_t)r * p.c_m) = o;
            }
    } else {
        for (int r = 0; r < rows; ++r)
            store_group4(p, Cb, p.c_m, false, p.c_vec, p.bias_axis, p.beta, m0 + r, n, row_sum(r));
    }
}

// Sums the GEMV kernels' split-K partials (ws_vec: N % 4 == 0, aligned): a
// workgroup takes kSkRedCols column groups of one output row, and its
// kSkRedSlices thread slices the splits q, q + kSkRedSlices, ... (all their
// loads in flight at once for up to 64 splits); the slices' sums are then
// added in slice order and stored with bias and beta.  Many small workgroups,
// one round trip: the partials of a GEMV are a few hundred KB.
constexpr int kSkRedCols = 16, kSkRedSlices = 16;
__global__ void __launch_bounds__(256) skinny_reduce_f32(GemmParams p) {
    static_assert(kSkRedCols * kSkRedSlices == 256, "one thread per (column group, slice)");
    __shared__ f32x4 part[kSkRedSlices][kSkRedCols];
    const int t = threadIdx.x, l = t % kSkRedCols, q = t / kSkRedCols;
    const int row = blockIdx.y;
    const int bz = row / p.M, m = row - bz * p.M;
    const int n = (blockIdx.x * kSkRedCols + l) * 4;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (n < p.N) {
        const int64_t MN = (int64_t)p.M * p.N;
        const float* const src = p.ws + (int64_t)bz * MN + (int64_t)m * p.N + n;
        const int64_t sstride = (int64_t)p.batch * MN;
        constexpr int kB = 4;
        for (int s0 = q; s0 < p.splits; s0 += kB * kSkRedSlices) {
            f32x4 x[kB];
#pragma unroll
            for (int j = 0; j < kB; ++j)
                if (s0 + kSkRedSlices * j < p.splits)
                    x[j] = *reinterpret_cast<const f32x4*>(
                        src + (int64_t)(s0 + kSkRedSlices * j) * sstride);
#pragma unroll
            for (int j = 0; j < kB; ++j)
                if (s0 + kSkRedSlices * j < p.splits) v += x[j];
        }
    }
    part[q][l] = v;
    __syncthreads();
    if (q != 0 || n >= p.N) return;
    v = part[0][l];
#pragma unroll
    for (int w = 1; w < kSkRedSlices; ++w) v += part[w][l];
    store_group4(p, p.C + (int64_t)bz * p.c_b, p.c_m, false, p.c_vec, p.bias_axis, p.beta, m, n,
                 v);
}

}  // namespace mtk
