// Kernel (d): decode GEMV, Q4_K / Q6_K weights x Q8_K activations.
//
// Replaces llama.cpp's CPU decode route that the reference plugin keeps for
// M=1 (adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:674-679 rejects M=1 under
// ROCKNPU_DECODE=cpu): ggml_vec_dot_q4_K_q8_K / ggml_vec_dot_q6_K_q8_K. For
// every (row, super-block) the integer sums are exact:
//   isum = sum_j sc_j * sum_{l in sub-block j} q8[l] * q[l]
//   msum = sum_j mn_j * (bsum pair of sub-block j)         (Q4_K only)
// and the row result is sum_b (d_w*d_a) * isum - (dmin_w*d_a) * msum in f32.
//
// Mapping: the Q8_K activation rows are staged in LDS, split into aligned
// quants / bsums / d arrays. A "unit" is 64 weight values of a Q4_K block
// (4 per block: 32 qs bytes + the 16-byte header) or 32 values of a Q6_K block
// (8 per block). Each wave works on 64/G rows at once, G lanes per row; lanes
// of one block are adjacent, so a block's integer sums are reduced with lane
// shuffles and converted to f32 once per block. Quant dot products use
// v_dot4_i32_i8 (sdot4).
#include "common.h"

namespace rk {
namespace {

constexpr int kGemvWaves = 4;

struct Q8Lds {
    int8_t* qs;     // [m][nb][256]
    int32_t* bs;    // [m][nb][8]  pairs of int16 bsums packed as words
    float* d;       // [m][nb]
};

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

template <int KIND, int MT>
__global__ __launch_bounds__(kGemvWaves * 64) void gemv_q8_k_kernel(
    const uint8_t* __restrict__ w, int64_t n, int nb, const uint8_t* __restrict__ q8k, int64_t ldq,
    int m, int log2g, float* __restrict__ out, int64_t ldo, int32_t* __restrict__ isum_out,
    int32_t* __restrict__ msum_out) {
    constexpr int BB = block_bytes(KIND);
    constexpr int UPB = KIND == 4 ? 4 : 8;  // units per block
    extern __shared__ __align__(16) uint8_t smem[];
    Q8Lds a;
    a.qs = reinterpret_cast<int8_t*>(smem);
    a.bs = reinterpret_cast<int32_t*>(smem + MT * nb * kQK);
    a.d = reinterpret_cast<float*>(smem + MT * nb * (kQK + 32));

    // Stage the activation rows: word-granular copy, split by field.
    const int words = m * nb * (kQ8KBytes / 4);
    for (int i = threadIdx.x; i < words; i += blockDim.x) {
        const int blk = i / (kQ8KBytes / 4), wi = i % (kQ8KBytes / 4);
        const int mi = blk / nb, bi = blk % nb;
        const uint32_t v = *reinterpret_cast<const uint32_t*>(q8k + mi * ldq + bi * kQ8KBytes + 4 * wi);
        const int flat = mi * nb + bi;
        if (wi == 0) a.d[flat] = __uint_as_float(v);
        else if (wi <= 64) reinterpret_cast<uint32_t*>(a.qs + flat * kQK)[wi - 1] = v;
        else a.bs[flat * 8 + (wi - 65)] = static_cast<int32_t>(v);
    }
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int G = 1 << log2g;
    const int gl = lane & (G - 1);
    const int64_t row = (static_cast<int64_t>(blockIdx.x) * kGemvWaves + wave) * (64 >> log2g) + (lane >> log2g);
    const bool row_ok = row < n;
    const uint8_t* wrow = w + (row_ok ? row : 0) * static_cast<int64_t>(nb) * BB;
    const int units = nb * UPB;
    const int iters = (units + G - 1) / G;

    float acc[MT];
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[mi] = 0.0f;

    for (int it = 0; it < iters; ++it) {
        const int u = gl + it * G;
        const bool ok = row_ok && u < units;
        const int b = ok ? u / UPB : 0, v = u % UPB;
        const uint8_t* blk = wrow + b * BB;
        int isum[MT], msum[MT];
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) { isum[mi] = 0; msum[mi] = 0; }
        float dw = 0.0f, dminw = 0.0f;
        if (ok) {
            if constexpr (KIND == 4) {
                const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
                const uint4 qa = *reinterpret_cast<const uint4*>(blk + 16 + 32 * v);
                const uint4 qb = *reinterpret_cast<const uint4*>(blk + 16 + 32 * v + 16);
                dw = f16_bits_to_f32(static_cast<uint16_t>(hdr.x & 0xFFFF));
                dminw = f16_bits_to_f32(static_cast<uint16_t>(hdr.x >> 16));
                int sc_lo, mn_lo, sc_hi, mn_hi;
                scale_min_k4(2 * v, hdr.y, hdr.z, hdr.w, sc_lo, mn_lo);
                scale_min_k4(2 * v + 1, hdr.y, hdr.z, hdr.w, sc_hi, mn_hi);
                const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                for (int mi = 0; mi < MT; ++mi) {
                    if (mi >= m) break;
                    const int flat = mi * nb + b;
                    const uint4* q8 = reinterpret_cast<const uint4*>(a.qs + flat * kQK + 64 * v);
                    const uint4 x0 = q8[0], x1 = q8[1], x2 = q8[2], x3 = q8[3];
                    const uint32_t lo8[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                    const uint32_t hi8[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
                    int dlo = 0, dhi = 0;
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        dlo = dot4(qw[t] & 0x0F0F0F0Fu, lo8[t], dlo);
                        dhi = dot4((qw[t] >> 4) & 0x0F0F0F0Fu, hi8[t], dhi);
                    }
                    isum[mi] = sc_lo * dlo + sc_hi * dhi;
                    const int32_t p0 = a.bs[flat * 8 + 2 * v], p1 = a.bs[flat * 8 + 2 * v + 1];
                    const int bs_lo = static_cast<int16_t>(p0 & 0xFFFF) + static_cast<int16_t>(p0 >> 16);
                    const int bs_hi = static_cast<int16_t>(p1 & 0xFFFF) + static_cast<int16_t>(p1 >> 16);
                    msum[mi] = mn_lo * bs_lo + mn_hi * bs_hi;
                }
            } else {
                const int half = v >> 2, g = v & 3;
                uint32_t l0[2], l1[2], h[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint8_t* p0 = blk + 64 * half + 8 * g + 4 * t;
                    const uint8_t* p1 = p0 + 32;
                    const uint8_t* ph = blk + 128 + 32 * half + 8 * g + 4 * t;
                    l0[t] = ld_u16(p0) | static_cast<uint32_t>(ld_u16(p0 + 2)) << 16;
                    l1[t] = ld_u16(p1) | static_cast<uint32_t>(ld_u16(p1 + 2)) << 16;
                    h[t] = ld_u16(ph) | static_cast<uint32_t>(ld_u16(ph + 2)) << 16;
                }
                const uint32_t sw0 = ld_u16(blk + 192 + 8 * half) | static_cast<uint32_t>(ld_u16(blk + 194 + 8 * half)) << 16;
                const uint32_t sw1 = ld_u16(blk + 196 + 8 * half) | static_cast<uint32_t>(ld_u16(blk + 198 + 8 * half)) << 16;
                dw = f16_bits_to_f32(ld_u16(blk + 208));
                // scale of quarter qd is byte (g/2 + 2*qd) of the 8 half-block scales
                const uint64_t sw = sw0 | static_cast<uint64_t>(sw1) << 32;
                int sc[4];
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) sc[qd] = static_cast<int8_t>((sw >> (8 * ((g >> 1) + 2 * qd))) & 0xFF);
                uint32_t qv[4][2];
#pragma unroll
                for (int qd = 0; qd < 4; ++qd)
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const uint32_t lb = (qd & 1) ? l1[t] : l0[t];
                        const uint32_t lo = (qd < 2) ? (lb & 0x0F0F0F0Fu) : ((lb >> 4) & 0x0F0F0F0Fu);
                        const uint32_t hi = (h[t] >> (2 * qd)) & 0x03030303u;
                        const uint32_t u6 = lo | (hi << 4);  // bytes in [0, 63]
                        qv[qd][t] = ((u6 | 0x80808080u) - 0x20202020u) ^ 0x80808080u;  // bytes - 32
                    }
#pragma unroll
                for (int mi = 0; mi < MT; ++mi) {
                    if (mi >= m) break;
                    const int8_t* q8 = a.qs + (mi * nb + b) * kQK + 128 * half + 8 * g;
                    int s = 0;
#pragma unroll
                    for (int qd = 0; qd < 4; ++qd) {
                        const uint2 x = *reinterpret_cast<const uint2*>(q8 + 32 * qd);
                        const int dq = dot4(qv[qd][1], x.y, dot4(qv[qd][0], x.x, 0));
                        s += sc[qd] * dq;
                    }
                    isum[mi] = s;
                }
            }
        }
        // Reduce the UPB lanes of each block (adjacent lanes), exactly in int.
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
#pragma unroll
            for (int o = 1; o < UPB; o <<= 1) {
                isum[mi] += __shfl_xor(isum[mi], o, 64);
                if constexpr (KIND == 4) msum[mi] += __shfl_xor(msum[mi], o, 64);
            }
        }
        if (ok && v == 0) {
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) {
                if (mi >= m) break;
                const float da = a.d[mi * nb + b];
                float term = (dw * da) * static_cast<float>(isum[mi]);
                if constexpr (KIND == 4) term = term - (dminw * da) * static_cast<float>(msum[mi]);
                acc[mi] += term;
                if (isum_out) {
                    const int64_t idx = (static_cast<int64_t>(mi) * n + row) * nb + b;
                    isum_out[idx] = isum[mi];
                    msum_out[idx] = msum[mi];
                }
            }
        }
    }
    // Sum the row's per-lane partials across its G lanes.
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
        for (int o = 1; o < G; o <<= 1) acc[mi] += __shfl_xor(acc[mi], o, 64);
    }
    if (row_ok && gl == 0) {
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
            if (mi >= m) break;
            out[mi * ldo + row] = acc[mi];
        }
    }
}

template <int KIND>
int launch_kind(const uint8_t* w, int64_t n, int nb, const uint8_t* q8k, int64_t ldq, int m,
                float* out, int64_t ldo, int32_t* isum, int32_t* msum, hipStream_t stream) {
    constexpr int UPB = KIND == 4 ? 4 : 8;
    const int units = nb * UPB;
    int log2g = 0;
    while ((1 << log2g) < units && log2g < 6) ++log2g;
    const int64_t rows_per_wg = static_cast<int64_t>(kGemvWaves) * (64 >> log2g);
    const dim3 grid(static_cast<unsigned>((n + rows_per_wg - 1) / rows_per_wg)), block(kGemvWaves * 64);
    int mt = m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
    const size_t lds = static_cast<size_t>(mt) * nb * (kQK + 32 + 4);
#define RK_GEMV_CASE(MTV)                                                                     \
    case MTV:                                                                                 \
        gemv_q8_k_kernel<KIND, MTV><<<grid, block, lds, stream>>>(w, n, nb, q8k, ldq, m, log2g, \
                                                                  out, ldo, isum, msum);      \
        break;
    switch (mt) {
        RK_GEMV_CASE(1)
        RK_GEMV_CASE(2)
        RK_GEMV_CASE(4)
        RK_GEMV_CASE(8)
    }
#undef RK_GEMV_CASE
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace

// m <= 8 rows per launch; LDS holds m * nb * 292 bytes (callers keep it <= 64 KiB).
int launch_gemv_q8_k(int kind, const uint8_t* w, int64_t n, int nb, const uint8_t* q8k, int64_t ldq,
                     int m, float* out, int64_t ldo, int32_t* isum, int32_t* msum, hipStream_t stream) {
    if (kind == 4) return launch_kind<4>(w, n, nb, q8k, ldq, m, out, ldo, isum, msum, stream);
    if (kind == 6) return launch_kind<6>(w, n, nb, q8k, ldq, m, out, ldo, isum, msum, stream);
    return kStatusInvalid;
}

}  // namespace rk
