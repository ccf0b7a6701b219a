// Kernel (b): per-token symmetric int8 activation quantisation, and the
// Q8_K activation quantisation of the decode path.
//
// A8 (crates/rocknpu-capi/src/lib.rs:614-654, driven per row at :1776-1791):
// scale = max|row| / 127 (1.0 for an all-zero row), q = clamp(round_half_away(
// x / scale), -127, 127), int8 rows zero-padded to k_pad. A row holding a
// non-finite value is rejected by the reference; here its scale is written as
// NaN and its int8 row as zeros, and the host turns that into
// ROCKNPU_STATUS_INVALID_ARGUMENT.
//
// Q8_K (ggml quantize_row_q8_K_ref, llama.cpp ggml-quants.c): per 256-value
// block, the first value of largest magnitude `max` gives iscale = -127/max,
// q = min(127, round_half_even(iscale * x)), bsums[16] = sums of 16 quants,
// d = 1/iscale. An all-zero block stores d = 0, zero quants and zero bsums.
#include "common.h"

#include <algorithm>

namespace rk {
namespace {

constexpr int kA8Threads = 256;

__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < kA8Threads / 64; ++w) r = fmaxf(r, red[w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (a & 0xFF) | (b & 0xFF) << 8 | (c & 0xFF) << 16 | static_cast<uint32_t>(d & 0xFF) << 24;
}

// Workgroup 0 (of nt threads) clears `nzero` words (the split-K counters of
// the GEMM that follows on the stream), so the prompt route needs no separate
// fill launch.
__device__ __forceinline__ void zero_counters(uint32_t* words, int nzero, int nt) {
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < nzero; i += nt) words[i] = 0;
}

// One workgroup per activation row. VEC: k, lda and k_pad are multiples of 4
// and both base pointers are 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(kA8Threads) void quantize_a8_kernel(const float* __restrict__ a,
                                                                 int64_t k, int64_t lda,
                                                                 int64_t k_pad,
                                                                 int8_t* __restrict__ a8,
                                                                 uint32_t* __restrict__ zero_words, int nzero,
                                                                 float* __restrict__ scales) {
    __shared__ float red[kA8Threads / 64];
    zero_counters(zero_words, nzero, kA8Threads);
    const int64_t row = blockIdx.x;
    const float* x = a + row * lda;
    int8_t* q = a8 + row * k_pad;
    const int t = threadIdx.x;

    // Pass 1: max |x| over the row; a non-finite value poisons it to +inf
    // (|x| > FLT_MAX, or NaN mapped to +inf) so one reduction serves both.
    float vmax = 0.0f;
    if constexpr (VEC) {
        for (int64_t i = t; i < k / 4; i += kA8Threads) {
            const float4 v = reinterpret_cast<const float4*>(x)[i];
            const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float m = fabsf(e[j]);
                vmax = fmaxf(vmax, (m <= 3.402823466e38f) ? m : __builtin_inff());
            }
        }
    } else {
        for (int64_t i = t; i < k; i += kA8Threads) {
            const float m = fabsf(x[i]);
            vmax = fmaxf(vmax, (m <= 3.402823466e38f) ? m : __builtin_inff());
        }
    }
    vmax = block_max(vmax, red);
    const bool bad = !(vmax <= 3.402823466e38f);
    const float scale = vmax == 0.0f ? 1.0f : vmax / 127.0f;
    [[maybe_unused]] const float inv = 1.0f / scale;

    // Pass 2: quantise (the row is cache-resident now) and zero the padding.
    if constexpr (VEC) {
        for (int64_t i = t; i < k / 4; i += kA8Threads) {
            const float4 v = reinterpret_cast<const float4*>(x)[i];
            uint32_t w = 0;
            if (!bad) {
                const float e[4] = {v.x, v.y, v.z, v.w};
                int qq[4];
                quant_sym_rcp(e, scale, inv, qq);
                w = pack4(qq[0], qq[1], qq[2], qq[3]);
            }
            reinterpret_cast<uint32_t*>(q)[i] = w;
        }
        for (int64_t i = k / 4 + t; i < k_pad / 4; i += kA8Threads) reinterpret_cast<uint32_t*>(q)[i] = 0;
    } else {
        for (int64_t i = t; i < k_pad; i += kA8Threads)
            q[i] = (i < k && !bad) ? static_cast<int8_t>(quant_sym(x[i], scale)) : 0;
    }
    if (t == 0) scales[row] = bad ? __builtin_nanf("") : scale;
}

// The same for rows of up to 16 * 1024 values with k, lda and k_pad multiples
// of 4 and 16-byte aligned bases, one row per workgroup of blockDim.x threads
// (whole waves, at most 1024): each thread keeps its R float4 of the row
// (float4 t + blockDim.x * j) in registers, so the row is read once. The max
// of |x| is an unsigned max of the bit patterns with the sign cleared (NaN
// patterns order above +inf, so the one reduction also finds non-finite
// rows), and the values are quantised four to a word by quant_sym_rcp_packed.
// The max is order-independent and every value takes quant_sym's result, so
// the output is bit-identical to quantize_a8_kernel's.
template <int R>
__global__ __launch_bounds__(1024) void quantize_a8_regs_kernel(const float* __restrict__ a, int64_t k,
                                                                int64_t lda, int64_t k_pad,
                                                                int8_t* __restrict__ a8,
                                                                uint32_t* __restrict__ zero_words, int nzero,
                                                                int nthreads, float* __restrict__ scales) {
    __shared__ uint32_t red[16];
    // nthreads = blockDim.x, passed as a preloaded argument: blockDim is a
    // hidden argument, read from memory before the row's loads could go out
    const int64_t row = blockIdx.x;
    const float4* x = reinterpret_cast<const float4*>(a + row * lda);
    uint32_t* q = reinterpret_cast<uint32_t*>(a8 + row * k_pad);
    const int t = threadIdx.x, nt = nthreads;
    const int k4 = static_cast<int>(k / 4);
    float vals[4 * R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int i = t + j * nt;
        const float4 v = i < k4 ? x[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        vals[4 * j] = v.x;
        vals[4 * j + 1] = v.y;
        vals[4 * j + 2] = v.z;
        vals[4 * j + 3] = v.w;
    }
    zero_counters(zero_words, nzero, nthreads);  // behind the row's loads
    uint32_t um = 0;
#pragma unroll
    for (int i = 0; i < 4 * R; ++i) um = max(um, __float_as_uint(vals[i]) & 0x7fffffffu);
    um = __float_as_uint(wave_max_nonneg(__uint_as_float(um)));
    if ((t & 63) == 0) red[t >> 6] = um;
    __syncthreads();
    um = red[0];
    for (int w = 1; w < nt / 64; ++w) um = max(um, red[w]);
    const bool bad = um > 0x7f7fffffu;  // an Inf or NaN in the row
    const float vmax = __uint_as_float(um);
    const float scale = bad || vmax == 0.0f ? 1.0f : vmax / 127.0f;
    const float inv = 1.0f / scale;
    uint32_t w[R];
    quant_sym_rcp_packed(vals, scale, inv, scale >= 1.175494351e-38f, w);
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int i = t + j * nt;
        if (i < k4) q[i] = bad ? 0u : w[j];
    }
    for (int64_t i = k4 + t; i < k_pad / 4; i += nt) q[i] = 0;
    if (t == 0) scales[row] = bad ? __builtin_nanf("") : scale;
}

// One wave per 256-value block, 4 blocks per workgroup. VEC: ldx % 4 == 0 and
// x is 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(256) void quantize_q8_k_kernel(const float* __restrict__ x, int64_t m,
                                                            int64_t nb, int64_t ldx,
                                                            uint8_t* __restrict__ y) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t gb = static_cast<int64_t>(blockIdx.x) * 4 + wave;
    if (gb >= m * nb) return;
    const int64_t r = gb / nb, b = gb % nb;
    const float* xb = x + r * ldx + b * kQK;
    float v[4];
    if constexpr (VEC) {
        const float4 f = reinterpret_cast<const float4*>(xb)[lane];
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = xb[4 * lane + j];
    }
    // First index of the largest magnitude (strict '>' in index order, NaN
    // never selected), reduced across the wave with ties to the lower index.
    float best_abs = 0.0f, best_val = 0.0f;
    int best_idx = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float ax = fabsf(v[j]);
        if (ax > best_abs) { best_abs = ax; best_val = v[j]; best_idx = 4 * lane + j; }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float oa = __shfl_xor(best_abs, o, 64);
        const float ov = __shfl_xor(best_val, o, 64);
        const int oi = __shfl_xor(best_idx, o, 64);
        if (oa > best_abs || (oa == best_abs && oi < best_idx)) {
            best_abs = oa; best_val = ov; best_idx = oi;
        }
    }
    uint8_t* yb = y + gb * kQ8KBytes;
    int q[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (best_abs != 0.0f) {
        const float iscale = -127.0f / best_val;
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = min(127, static_cast<int>(__builtin_rintf(iscale * v[j])));
        d = 1.0f / iscale;
    }
    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    *reinterpret_cast<uint32_t*>(yb + 4 + 4 * lane) = pack4(q[0], q[1], q[2], q[3]);
    if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(yb + 260 + 2 * (lane >> 2)) = static_cast<int16_t>(s);
    if (lane == 0) *reinterpret_cast<float*>(yb) = d;
}

}  // namespace

int launch_quantize_a8(const float* a, int64_t m, int64_t k, int64_t lda, int64_t k_pad, int8_t* a8,
                       float* scales, uint32_t* zero_words, int nzero, hipStream_t stream) {
    const bool vec = k % 4 == 0 && lda % 4 == 0 && k_pad % 4 == 0 &&
                     reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(a8) % 16 == 0;
    const dim3 grid(static_cast<unsigned>(m)), block(kA8Threads);
    // Threads per row: two float4 each (one for at most 512 rows of at most
    // 4096 values), in whole waves, at most 1024. Sweeps over 256-1024
    // threads: 512 x 5632 takes 5.85 us (6.87 with 256 threads and six float4
    // each), 128 x 2048 2.55 (2.97), 2048 x 2048 6.83 (7.36), 4096 x 4096 17.2
    // (17.7), 4096 x 14336 54.0 (58.0).
    const int64_t k4 = k / 4;
    const int64_t per = m <= 512 && k4 <= 1024 ? 1 : 2;
    const int64_t nt = std::min<int64_t>(1024, std::max<int64_t>(64, (k4 + per - 1) / per + 63) / 64 * 64);
    const int64_t r = (k4 + nt - 1) / nt;
    if (vec && r <= 4) {
        const dim3 rb(static_cast<unsigned>(nt));
        const int tn = static_cast<int>(nt);
        if (r <= 1) quantize_a8_regs_kernel<1><<<grid, rb, 0, stream>>>(a, k, lda, k_pad, a8, zero_words, nzero, tn, scales);
        else if (r <= 2) quantize_a8_regs_kernel<2><<<grid, rb, 0, stream>>>(a, k, lda, k_pad, a8, zero_words, nzero, tn, scales);
        else if (r <= 3) quantize_a8_regs_kernel<3><<<grid, rb, 0, stream>>>(a, k, lda, k_pad, a8, zero_words, nzero, tn, scales);
        else quantize_a8_regs_kernel<4><<<grid, rb, 0, stream>>>(a, k, lda, k_pad, a8, zero_words, nzero, tn, scales);
    } else if (vec) quantize_a8_kernel<true><<<grid, block, 0, stream>>>(a, k, lda, k_pad, a8, zero_words, nzero, scales);
    else quantize_a8_kernel<false><<<grid, block, 0, stream>>>(a, k, lda, k_pad, a8, zero_words, nzero, scales);
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

int launch_quantize_q8_k(const float* x, int64_t m, int64_t k, int64_t ldx, uint8_t* y,
                         hipStream_t stream) {
    const int64_t nb = k / kQK;
    const bool vec = ldx % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    const dim3 grid(static_cast<unsigned>((m * nb + 3) / 4)), block(256);
    if (vec) quantize_q8_k_kernel<true><<<grid, block, 0, stream>>>(x, m, nb, ldx, y);
    else quantize_q8_k_kernel<false><<<grid, block, 0, stream>>>(x, m, nb, ldx, y);
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace rk
