// Kernel (d): decode GEMV, Q4_K / Q6_K weights x Q8_K activations.
//
// Replaces llama.cpp's CPU decode route that the reference plugin keeps for
// M=1 (adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:674-679 rejects M=1 under
// ROCKNPU_DECODE=cpu): ggml_vec_dot_q4_K_q8_K / ggml_vec_dot_q6_K_q8_K after
// quantize_row_q8_K. For every (row, super-block) the integer sums are exact:
//   isum = sum_j sc_j * sum_{l in sub-block j} q8[l] * q[l]
//   msum = sum_j mn_j * (bsum pair of sub-block j)         (Q4_K only)
// and the row result is sum_b (d_w*d_a) * isum - (dmin_w*d_a) * msum in f32.
//
// One launch serves up to four projections that share the activation rows
// (q/k/v, gate/up); each workgroup serves one of them, so every per-projection
// value is wave-uniform. The activations are either f32 (quantised to Q8_K by
// every workgroup into LDS: 16 lanes per 256-value block, DPP reductions) or
// Q8_K rows copied to LDS.
//
// Work split: one lane owns one whole super-block (144 bytes of Q4_K, 210 of
// Q6_K), so scales are unpacked once per block and the block's integer sums
// never leave the lane. G lanes (G <= 16) share a weight row, a wave covers
// 64/G rows at once, and a row group takes `iters` blocks per lane. Waves walk
// their row groups grid-stride with D blocks of loads in flight per lane; the
// row's G partial sums are combined with DPP lane moves.
#include "common.h"

namespace rk {
namespace {

constexpr int kGemvWaves = 4;

template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
// DPP controls: quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror.
// Applied in this order they combine aligned groups of 2, 4, 8 and 16 lanes.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppMirror8 = 0x141, kDppMirror16 = 0x140;

__device__ __forceinline__ float max16(float v) {
    v = fmaxf(v, __int_as_float(dpp<kDppXor1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp<kDppXor2>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp<kDppMirror8>(__float_as_int(v))));
    return fmaxf(v, __int_as_float(dpp<kDppMirror16>(__float_as_int(v))));
}
__device__ __forceinline__ int min16(int v) {
    v = min(v, dpp<kDppXor1>(v));
    v = min(v, dpp<kDppXor2>(v));
    v = min(v, dpp<kDppMirror8>(v));
    return min(v, dpp<kDppMirror16>(v));
}
// Sum over aligned groups of G lanes (G a power of two, at most 16).
__device__ __forceinline__ float group_sum(float v, int G) {
    if (G >= 2) v += __int_as_float(dpp<kDppXor1>(__float_as_int(v)));
    if (G >= 4) v += __int_as_float(dpp<kDppXor2>(__float_as_int(v)));
    if (G >= 8) v += __int_as_float(dpp<kDppMirror8>(__float_as_int(v)));
    if (G >= 16) v += __int_as_float(dpp<kDppMirror16>(__float_as_int(v)));
    return v;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// Global-memory (address space 1) views keep global loads and stores even for
// addresses the compiler cannot trace back to a kernel argument.
typedef const __attribute__((address_space(1))) uint8_t* gbytes;
typedef __attribute__((address_space(1))) float* gfloats;
typedef unsigned v4u __attribute__((ext_vector_type(4)));

// Activation rows in LDS (regions sized for MT rows):
//   quants of block b of row mi: 256 bytes at qs + (mi*nb + b) * 272
//   its bsums:                   16 x int16 at bs + (mi*nb + b) * 48
//   its scale:                   d[mi*nb + b]
// The 272- and 48-byte strides put consecutive blocks in different LDS banks,
// and the 16 chunk reads of a block use immediate offsets.
struct Q8Lds {
    uint8_t* qs;
    uint8_t* bs;
    float* d;
    int nb;
    __device__ __forceinline__ const uint8_t* quants(int mi, int b) const {
        return qs + (mi * nb + b) * kGemvLdsQsStride;
    }
    __device__ __forceinline__ const int16_t* bsums(int mi, int b) const {
        return reinterpret_cast<const int16_t*>(bs + (mi * nb + b) * kGemvLdsBsStride);
    }
};

__device__ __forceinline__ Q8Lds q8_lds(uint8_t* smem, int mt, int nb) {
    Q8Lds a;
    a.qs = smem;
    a.bs = smem + mt * nb * kGemvLdsQsStride;
    a.d = reinterpret_cast<float*>(a.bs + mt * nb * kGemvLdsBsStride);
    a.nb = nb;
    return a;
}

// The 16 values of this lane for quantisation block qb.
__device__ __forceinline__ void load_x16(const float* __restrict__ x, int64_t ldx, int nb, int qb, float4 (&f)[4]) {
    const int sub = threadIdx.x & 15;
    const int r = qb / nb, b = qb % nb;
    const float4* src = reinterpret_cast<const float4*>(x + r * ldx + b * kQK + 16 * sub);
#pragma unroll
    for (int t = 0; t < 4; ++t) f[t] = src[t];
}

// Q8_K quantisation of rows [0, m) of x into LDS (ggml quantize_row_q8_K_ref
// semantics, see quant.hip): 16 lanes per block, 16 values per lane. `first`
// holds this lane's values of its first block, loaded by the caller ahead of
// the weight loads so they return first.
__device__ __forceinline__ void quantize_to_lds(const float* __restrict__ x, int64_t ldx, int m, int nb,
                                                const float4 (&first)[4], const Q8Lds& a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane & 15;
    const int slot = wave * 4 + (lane >> 4);
    for (int qb = slot; qb < m * nb; qb += kGemvWaves * 4) {
        const int r = qb / nb, b = qb % nb;
        float4 f[4];
        if (qb == slot) {
#pragma unroll
            for (int t = 0; t < 4; ++t) f[t] = first[t];
        } else {
            load_x16(x, ldx, nb, qb, f);
        }
        float v[16];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            v[4 * t] = f[t].x; v[4 * t + 1] = f[t].y; v[4 * t + 2] = f[t].z; v[4 * t + 3] = f[t].w;
        }
        float amax = 0.0f;
        int first_i = 0;
        bool neg = false;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float ax = fabsf(v[i]);
            if (ax > amax) { amax = ax; first_i = i; neg = v[i] < 0.0f; }
        }
        const float gmax = max16(amax);
        int key = (amax == gmax && gmax > 0.0f) ? ((16 * sub + first_i) * 2 + (neg ? 1 : 0)) : 0x7fffffff;
        key = min16(key);
        int q[16];
        float d = 0.0f;
        if (gmax > 0.0f) {
            const float mx = (key & 1) ? -gmax : gmax;  // the first value of largest magnitude
            const float iscale = -127.0f / mx;
#pragma unroll
            for (int i = 0; i < 16; ++i) q[i] = min(127, static_cast<int>(__builtin_rintf(iscale * v[i])));
            d = 1.0f / iscale;
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) q[i] = 0;
        }
        int s = 0;
        uint32_t wq[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            s += q[4 * t] + q[4 * t + 1] + q[4 * t + 2] + q[4 * t + 3];
            wq[t] = (q[4 * t] & 0xFF) | (q[4 * t + 1] & 0xFF) << 8 | (q[4 * t + 2] & 0xFF) << 16 |
                    static_cast<uint32_t>(q[4 * t + 3] & 0xFF) << 24;
        }
        uint8_t* qdst = a.qs + (r * nb + b) * kGemvLdsQsStride + 16 * sub;
        *reinterpret_cast<uint4*>(qdst) = make_uint4(wq[0], wq[1], wq[2], wq[3]);
        reinterpret_cast<int16_t*>(a.bs + (r * nb + b) * kGemvLdsBsStride)[sub] = static_cast<int16_t>(s);
        if (sub == 0) a.d[r * nb + b] = d;
    }
}

// Copy Q8_K rows (292-byte blocks) into the LDS layout.
__device__ __forceinline__ void stage_q8k(const uint8_t* __restrict__ q8k, int64_t ldq, int m, int nb,
                                          const Q8Lds& a) {
    const int words = m * nb * (kQ8KBytes / 4);
    for (int i = threadIdx.x; i < words; i += blockDim.x) {
        const int blk = i / (kQ8KBytes / 4), wi = i % (kQ8KBytes / 4);
        const int mi = blk / nb, bi = blk % nb;
        const uint32_t v = *reinterpret_cast<const uint32_t*>(q8k + mi * ldq + bi * kQ8KBytes + 4 * wi);
        if (wi == 0) a.d[mi * nb + bi] = __uint_as_float(v);
        else if (wi <= 64) reinterpret_cast<uint32_t*>(a.qs + (mi * nb + bi) * kGemvLdsQsStride)[wi - 1] = v;
        else reinterpret_cast<uint32_t*>(a.bs + (mi * nb + bi) * kGemvLdsBsStride)[wi - 65] = v;
    }
}

// One super-block's raw bytes as 32-bit words.
template <int KIND>
struct Block;

template <>
struct Block<4> {
    uint32_t w[36];  // [0] d|dmin, [1..3] packed scales, [4..35] qs
    __device__ __forceinline__ void load(gbytes blk) {
        typedef const __attribute__((address_space(1))) v4u* gu4;
#pragma unroll
        for (int t = 0; t < 9; ++t) {
            const v4u x = reinterpret_cast<gu4>(blk)[t];
            w[4 * t] = x.x; w[4 * t + 1] = x.y; w[4 * t + 2] = x.z; w[4 * t + 3] = x.w;
        }
    }
};

template <>
struct Block<6> {
    uint32_t w[53];  // [0..31] ql, [32..47] qh, [48..51] scales, [52] d (low 16 bits)
    // Q6_K blocks are only 2-byte aligned; the hardware takes unaligned vector
    // loads, so the first 208 bytes come in as 13 16-byte loads.
    __device__ __forceinline__ void load(gbytes blk) {
        typedef v4u v4u_a2 __attribute__((aligned(2)));
        typedef const __attribute__((address_space(1))) v4u_a2* gu4;
#pragma unroll
        for (int t = 0; t < 13; ++t) {
            const v4u x = reinterpret_cast<gu4>(blk)[t];
            w[4 * t] = x.x; w[4 * t + 1] = x.y; w[4 * t + 2] = x.z; w[4 * t + 3] = x.w;
        }
        w[52] = *reinterpret_cast<const __attribute__((address_space(1))) uint16_t*>(blk + 208);
    }
};

// Per-block decode shared by all activation rows.
template <int KIND>
struct Decoded;

template <>
struct Decoded<4> {
    int sc[8], mn[8];
    __device__ __forceinline__ void decode(const Block<4>& k) {
#pragma unroll
        for (int j = 0; j < 8; ++j) scale_min_k4(j, k.w[1], k.w[2], k.w[3], sc[j], mn[j]);
    }
};

template <>
struct Decoded<6> {
    uint32_t u[64];  // u[p/4]: values p..p+3 as unsigned 6-bit quants (0..63)
    int sc[16];
    __device__ __forceinline__ void decode(const Block<6>& k) {
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
            for (int qd = 0; qd < 4; ++qd)
#pragma unroll
                for (int l = 0; l < 32; l += 4) {
                    const uint32_t lb = k.w[(64 * half + 32 * (qd & 1) + l) / 4];
                    const uint32_t lo = (qd < 2) ? (lb & 0x0F0F0F0Fu) : ((lb >> 4) & 0x0F0F0F0Fu);
                    const uint32_t hi = (k.w[32 + (32 * half + l) / 4] >> (2 * qd)) & 0x03030303u;
                    u[(128 * half + 32 * qd + l) / 4] = lo | (hi << 4);
                }
#pragma unroll
        for (int si = 0; si < 16; ++si) sc[si] = static_cast<int8_t>((k.w[48 + si / 4] >> (8 * (si % 4))) & 0xFF);
    }
};

// Exact integer sums of block b against activation row mi.
__device__ __forceinline__ void block_sums(const Block<4>& k, const Decoded<4>& dc, int mi, int b, const Q8Lds& a,
                                           int& isum, int& msum) {
    const v4u* q8 = reinterpret_cast<const v4u*>(a.quants(mi, b));
    const int16_t* bs = a.bsums(mi, b);
    int is = 0, ms = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // 64-value group j: sub-blocks 2j (low nibbles), 2j+1 (high)
        const v4u x0 = q8[4 * j], x1 = q8[4 * j + 1], x2 = q8[4 * j + 2], x3 = q8[4 * j + 3];
        const uint32_t lo8[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const uint32_t hi8[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
        int dlo = 0, dhi = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t q = k.w[4 + 8 * j + t];
            dlo = dot4(q & 0x0F0F0F0Fu, lo8[t], dlo);
            dhi = dot4((q >> 4) & 0x0F0F0F0Fu, hi8[t], dhi);
        }
        is += dc.sc[2 * j] * dlo + dc.sc[2 * j + 1] * dhi;
        const uint2 pair = *reinterpret_cast<const uint2*>(bs + 4 * j);
        const int b_lo = static_cast<int16_t>(pair.x & 0xFFFF) + static_cast<int16_t>(pair.x >> 16);
        const int b_hi = static_cast<int16_t>(pair.y & 0xFFFF) + static_cast<int16_t>(pair.y >> 16);
        ms += dc.mn[2 * j] * b_lo + dc.mn[2 * j + 1] * b_hi;
    }
    isum = is;
    msum = ms;
}

// Q6_K: the quants are q - 32 with q = 0..63, and bsums hold the sums of the
// 16 activation quants of each sub-block, so sum (q-32)*x = sum q*x - 32*bsum.
__device__ __forceinline__ void block_sums(const Block<6>&, const Decoded<6>& dc, int mi, int b, const Q8Lds& a,
                                           int& isum, int& msum) {
    const v4u* q8 = reinterpret_cast<const v4u*>(a.quants(mi, b));
    const v4u* bsv = reinterpret_cast<const v4u*>(a.bsums(mi, b));
    const v4u b0 = bsv[0], b1 = bsv[1];
    const uint32_t bw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    int is = 0;
#pragma unroll
    for (int si = 0; si < 16; ++si) {  // 16-value sub-block si = chunk si
        const v4u x = q8[si];
        int dq = dot4(dc.u[4 * si], x.x, 0);
        dq = dot4(dc.u[4 * si + 1], x.y, dq);
        dq = dot4(dc.u[4 * si + 2], x.z, dq);
        dq = dot4(dc.u[4 * si + 3], x.w, dq);
        const int bsum = static_cast<int16_t>((bw[si / 2] >> (16 * (si % 2))) & 0xFFFF);
        is += dc.sc[si] * (dq - 32 * bsum);
    }
    isum = is;
    msum = 0;
}

// Position of a lane's block: row group `gi`, iteration `it` inside the group.
struct Pos {
    int64_t gi;
    int it;
};

template <int KIND, int MT, bool FUSED, int D>
__global__ __launch_bounds__(kGemvWaves * 64) void gemv_kernel(const GemvParams p) {
    constexpr int BB = block_bytes(KIND);
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = p.nb, m = p.m, iters = p.iters, log2g = p.log2g;
    const Q8Lds a = q8_lds(smem, MT, nb);

    // the projection this workgroup serves (wave-uniform)
    const int64_t wg = blockIdx.x;
    const uint8_t* w = p.w[0];
    float* out = p.out[0];
    int64_t ldo = p.ldo[0], rows = p.rows[0], wg0 = 0, wg1 = p.wg_end[0];
    if (p.count > 1 && wg >= p.wg_end[0]) { w = p.w[1]; out = p.out[1]; ldo = p.ldo[1]; rows = p.rows[1]; wg0 = p.wg_end[0]; wg1 = p.wg_end[1]; }
    if (p.count > 2 && wg >= p.wg_end[1]) { w = p.w[2]; out = p.out[2]; ldo = p.ldo[2]; rows = p.rows[2]; wg0 = p.wg_end[1]; wg1 = p.wg_end[2]; }
    if (p.count > 3 && wg >= p.wg_end[2]) { w = p.w[3]; out = p.out[3]; ldo = p.ldo[3]; rows = p.rows[3]; wg0 = p.wg_end[2]; wg1 = p.wg_end[3]; }
    const gbytes wg_w = reinterpret_cast<gbytes>(reinterpret_cast<uint64_t>(w));
    const gfloats wg_out = reinterpret_cast<gfloats>(reinterpret_cast<uint64_t>(out));
    int32_t* const isum_out = p.isum;
    int32_t* const msum_out = p.msum;

    const int G = 1 << log2g;
    const int gl = lane & (G - 1);
    const int slot = lane >> log2g;  // row inside the row group
    const int rows_per_group = 64 >> log2g;
    const int64_t row_bytes = static_cast<int64_t>(nb) * BB;
    const int64_t groups = (rows + rows_per_group - 1) / rows_per_group;
    const int64_t wave_gid = (wg - wg0) * kGemvWaves + wave;
    const int64_t wave_stride = (wg1 - wg0) * kGemvWaves;
    // this wave's blocks: row groups wave_gid + i*wave_stride, `iters` per lane each
    const int64_t my_groups = wave_gid < groups ? (groups - 1 - wave_gid) / wave_stride + 1 : 0;
    const int64_t S = my_groups * iters;

    auto advance = [=](Pos& q) {
        if (++q.it == iters) { q.it = 0; q.gi += wave_stride; }
    };
    // Loads are issued unconditionally: a lane without a block re-reads a block
    // of its wave's first row group (in bounds, cache-resident, private to the
    // wave) and ignores it. Branch-free load sequences let the wait-count pass
    // wait for exactly the loads a value depends on.
    const int64_t home_row = min(wave_gid * rows_per_group + slot, rows - 1);
    const int home_b = min(gl, nb - 1);
    auto load_block = [=](const Pos& q, bool in_range, Block<KIND>& k) {
        int64_t row = q.gi * rows_per_group + slot;
        int b = gl + q.it * G;
        if (!(in_range && row < rows && b < nb)) {
            row = home_row;
            b = home_b;
        }
        k.load(wg_w + row * row_bytes + static_cast<int64_t>(b) * BB);
    };

    // First activation values go out first (they return first), then D blocks.
    float4 xfirst[4];
    const int qslot = wave * 4 + (lane >> 4);
    if constexpr (FUSED) load_x16(p.x, p.ldx, nb, qslot < m * nb ? qslot : 0, xfirst);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight loads
    Block<KIND> buf[D];
    Pos lq{wave_gid, 0};  // next block to load
#pragma unroll
    for (int j = 0; j < D; ++j) {
        load_block(lq, j < S, buf[j]);
        advance(lq);
    }
    if constexpr (FUSED) quantize_to_lds(p.x, p.ldx, m, nb, xfirst, a);
    else stage_q8k(p.q8k, p.ldx, m, nb, a);
    __syncthreads();

    float acc[MT];
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[mi] = 0.0f;

    Pos cq{wave_gid, 0};  // block being multiplied
    for (int64_t base = 0; base < S; base += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const int64_t s = base + j;
            if (s >= S) break;  // uniform across the wave
            const int64_t row = cq.gi * rows_per_group + slot;
            const int b = gl + cq.it * G;
            const bool ok = row < rows && b < nb;
            // Every lane computes (a lane without a block holds its home block)
            // and discards the result: straight-line code for all rows mi.
            const int bk = ok ? b : home_b;
            float dw, dminw = 0.0f;
            if constexpr (KIND == 4) {
                dw = f16_bits_to_f32(static_cast<uint16_t>(buf[j].w[0] & 0xFFFF));
                dminw = f16_bits_to_f32(static_cast<uint16_t>(buf[j].w[0] >> 16));
            } else {
                dw = f16_bits_to_f32(static_cast<uint16_t>(buf[j].w[52]));
            }
            Decoded<KIND> dc;
            dc.decode(buf[j]);
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) {
                if (mi >= m) break;
                int isum, msum;
                block_sums(buf[j], dc, mi, bk, a, isum, msum);
                const float da = a.d[mi * nb + bk];
                float term = (dw * da) * static_cast<float>(isum);
                if constexpr (KIND == 4) term = term - (dminw * da) * static_cast<float>(msum);
                acc[mi] += ok ? term : 0.0f;
                if (isum_out && ok) {
                    const int64_t idx = (static_cast<int64_t>(mi) * rows + row) * nb + b;
                    isum_out[idx] = isum;
                    msum_out[idx] = msum;
                }
            }
            // refill this slot with the block D ahead
            load_block(lq, s + D < S, buf[j]);
            advance(lq);
            if (cq.it == iters - 1) {
                // row group done: combine the row's G lanes and store
#pragma unroll
                for (int mi = 0; mi < MT; ++mi) {
                    const float r = group_sum(acc[mi], G);
                    if (gl == 0 && row < rows && mi < m) wg_out[mi * ldo + row] = r;
                    acc[mi] = 0.0f;
                }
            }
            advance(cq);
        }
    }
}

template <int KIND, bool FUSED, int D>
void launch_d(const GemvParams& p, int mt, dim3 grid, size_t lds, hipStream_t stream) {
    const dim3 block(kGemvWaves * 64);
    switch (mt) {
    case 1: gemv_kernel<KIND, 1, FUSED, D><<<grid, block, lds, stream>>>(p); break;
    case 2: gemv_kernel<KIND, 2, FUSED, D><<<grid, block, lds, stream>>>(p); break;
    case 4: gemv_kernel<KIND, 4, FUSED, D><<<grid, block, lds, stream>>>(p); break;
    default: gemv_kernel<KIND, 8, FUSED, D><<<grid, block, lds, stream>>>(p); break;
    }
}

// Lanes per row: the largest power of two <= min(16, nb) whose last pass over
// the row's blocks keeps at least 85% of the lanes busy.
int lanes_per_row_log2(int nb) {
    int lg = 0;
    while ((2 << lg) <= 16 && (2 << lg) <= nb) ++lg;
    while (lg > 0) {
        const int g = 1 << lg, it = (nb + g - 1) / g;
        if (nb * 100 >= 85 * g * it) break;
        --lg;
    }
    return lg;
}

template <int KIND, bool FUSED>
int launch_kind(GemvParams& p, hipStream_t stream) {
    p.log2g = lanes_per_row_log2(p.nb);
    const int G = 1 << p.log2g;
    p.iters = (p.nb + G - 1) / G;
    const int64_t rows_per_group = 64 / G;
    // D blocks per lane in flight; each projection gets about D blocks per
    // lane (one round) worth of workgroups.
    int64_t total_wave_blocks = 0;
    for (int i = 0; i < p.count; ++i) total_wave_blocks += (p.rows[i] + rows_per_group - 1) / rows_per_group * p.iters;
    const int d = total_wave_blocks >= 2 * kGemvWaves * 256 ? 2 : 1;
    int64_t wgs = 0;
    for (int i = 0; i < p.count; ++i) {
        const int64_t wave_blocks = (p.rows[i] + rows_per_group - 1) / rows_per_group * p.iters;
        int64_t n = (wave_blocks + static_cast<int64_t>(d) * kGemvWaves - 1) / (static_cast<int64_t>(d) * kGemvWaves);
        if (n > 2048) n = 2048;
        if (n < 1) n = 1;
        wgs += n;
        p.wg_end[i] = wgs;
    }
    const int mt = p.m <= 1 ? 1 : p.m <= 2 ? 2 : p.m <= 4 ? 4 : 8;
    const size_t lds = static_cast<size_t>(mt) * p.nb * kGemvLdsPerBlock;
    const dim3 grid(static_cast<unsigned>(wgs));
    if (d == 2) launch_d<KIND, FUSED, 2>(p, mt, grid, lds, stream);
    else launch_d<KIND, FUSED, 1>(p, mt, grid, lds, stream);
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace

// p.m <= 8 activation rows; LDS holds m * nb * kGemvLdsPerBlock bytes (callers
// keep it <= 64 KiB).
int launch_gemv(int kind, bool fused, GemvParams& p, hipStream_t stream) {
    if (kind == 4) return fused ? launch_kind<4, true>(p, stream) : launch_kind<4, false>(p, stream);
    if (kind == 6) return fused ? launch_kind<6, true>(p, stream) : launch_kind<6, false>(p, stream);
    return kStatusInvalid;
}

}  // namespace rk
