// Kernel (a): one-time GGUF K-quant -> W8 weight repack.
//
// Replaces the host repack of crates/rocknpu-capi/src/lib.rs:711-757
// (prepare_q4_k_w8a8), :759-806 (prepare_q5_k_w8a8) and :974-994
// (prepare_q6_k_w8a8): each output row is dequantised to f32, then quantised
// symmetrically with scale = max|row| / 127 (1.0 for an all-zero row), value
// = clamp(round_half_away(v / scale), -127, 127) (lib.rs:614-654).
//
// Dequantised values are the correctly rounded f32 of an exact expression
// (Q4_K/Q5_K: d*sc*q has <= 22 significant bits, so only the final "- dmin*m"
// rounds; Q6_K: d*sc*q has <= 24 bits and is exact), so they match every f32
// implementation of the ggml formulas bit for bit.
//
// Mapping: one wave per output row, 4 independent waves per workgroup. A row
// is walked in chunks of 8 super-blocks (2048 values): per chunk the wave
// stages the per-sub-block factors (d*sc, dmin*m) into its own LDS area, one
// sub-block per lane, then every lane decodes one 32-value unit. Rows of up to
// HOLD chunks keep their decoded values in registers between finding
// max|row| and quantising; longer rows decode twice (the second time from
// L2). Quantisation multiplies by the reciprocal scale and divides only where
// the product is within 2^-15 of a rounding boundary (quant_sym_rcp).
#include "common.h"

#include <algorithm>

namespace rk {
namespace {

constexpr int kChunkBlocks = 8;
constexpr int kWaves = 4;

// Stage the per-sub-block factors of `cnt` blocks starting at `chunk` into
// st[16 * block + i]: Q4_K/Q5_K i<8 -> d*sc_i, i>=8 -> dmin*m_(i-8);
// Q6_K i<16 -> d*sc_i.
// Returns whether a staged factor is not finite. A dequantised value is then
// not finite exactly when its factors are not: |d*sc| <= 65504 * 127 and the
// quants are at most 6 bits, so finite factors give finite values.
template <int KIND>
__device__ __forceinline__ bool stage_factors(const uint8_t* chunk, int cnt, int lane, float* st) {
    constexpr int BB = block_bytes(KIND);
    bool bad = false;
    if constexpr (KIND == 4 || KIND == 5) {
        const int bi = lane >> 3, j = lane & 7;
        if (bi < cnt) {
            const uint8_t* blk = chunk + bi * BB;
            const uint32_t w0 = ld_u32(blk);
            const float d = f16_bits_to_f32(static_cast<uint16_t>(w0 & 0xFFFF));
            const float dmin = f16_bits_to_f32(static_cast<uint16_t>(w0 >> 16));
            int sc, mn;
            scale_min_k4(j, ld_u32(blk + 4), ld_u32(blk + 8), ld_u32(blk + 12), sc, mn);
            const float f0 = d * static_cast<float>(sc), f1 = dmin * static_cast<float>(mn);
            st[bi * 16 + j] = f0;
            st[bi * 16 + 8 + j] = f1;
            bad = !(fabsf(f0) <= 3.402823466e38f) || !(fabsf(f1) <= 3.402823466e38f);
        }
    } else {
#pragma unroll
        for (int e = lane; e < kChunkBlocks * 16; e += 64) {
            const int bi = e >> 4, idx = e & 15;
            if (bi < cnt) {
                const uint8_t* blk = chunk + bi * BB;
                const float d = f16_bits_to_f32(ld_u16(blk + 208));
                const int sc = static_cast<int8_t>(blk[192 + idx]);
                const float f = d * static_cast<float>(sc);
                st[bi * 16 + idx] = f;
                bad |= !(fabsf(f) <= 3.402823466e38f);
            }
        }
    }
    return bad;
}

// 32-bit word of the two 16-bit halves at p (2-byte aligned).
__device__ __forceinline__ uint32_t ld_u16x2(const uint8_t* p) {
    return static_cast<uint32_t>(ld_u16(p)) | static_cast<uint32_t>(ld_u16(p + 2)) << 16;
}

// Byte e of w as f32 (v_cvt_f32_ubyte<e>).
template <int E>
__device__ __forceinline__ float ubyte(uint32_t w) {
    return static_cast<float>((w >> (8 * E)) & 0xFF);
}

// Decode unit v (0..7) of a block into vals[32], four quants per 32-bit word.
// Q4_K/Q5_K: j = v/2, h = v%2; vals[0..16) are positions 64j+16h+i (sub-block
//   2j), vals[16..32) are positions 64j+32+16h+i (sub-block 2j+1);
//   value = d_sub * q - m_sub. d_sub * q is exact (a half times a 6-bit scale
//   times a 5-bit quant: at most 22 bits), so the fused multiply-add rounds
//   once, as the product-then-difference does.
// Q6_K: half = v/4, g = v%4; vals[8q+i] is position 128*half + 32q + 8g + i;
//   value = d_sub * (u - 32) = fma(d_sub, u, -32 d_sub), exact either way
//   (at most 24 bits).
template <int KIND>
__device__ __forceinline__ void decode_unit(const uint8_t* blk, int v, const float* st,
                                            float (&vals)[32]) {
    auto put4 = [&](int at, uint32_t w, float d, float neg_m) {
        vals[at] = __builtin_fmaf(d, ubyte<0>(w), neg_m);
        vals[at + 1] = __builtin_fmaf(d, ubyte<1>(w), neg_m);
        vals[at + 2] = __builtin_fmaf(d, ubyte<2>(w), neg_m);
        vals[at + 3] = __builtin_fmaf(d, ubyte<3>(w), neg_m);
    };
    if constexpr (KIND == 4 || KIND == 5) {
        const int j = v >> 1, h = v & 1;
        const uint4 qv = *reinterpret_cast<const uint4*>(blk + (KIND == 4 ? 16 : 48) + 32 * j + 16 * h);
        const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
        const float d1 = st[2 * j], d2 = st[2 * j + 1];
        const float m1 = -st[8 + 2 * j], m2 = -st[8 + 2 * j + 1];
        uint32_t hb[4] = {0, 0, 0, 0};
        if constexpr (KIND == 5) {
            const uint4 hv = *reinterpret_cast<const uint4*>(blk + 16 + 16 * h);
            hb[0] = hv.x; hb[1] = hv.y; hb[2] = hv.z; hb[3] = hv.w;
        }
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t lo = q[w] & 0x0F0F0F0Fu, hi = (q[w] >> 4) & 0x0F0F0F0Fu;
            if constexpr (KIND == 5) {
                lo |= ((hb[w] >> (2 * j)) & 0x01010101u) << 4;
                hi |= ((hb[w] >> (2 * j + 1)) & 0x01010101u) << 4;
            }
            put4(4 * w, lo, d1, m1);
            put4(16 + 4 * w, hi, d2, m2);
        }
    } else {
        const int half = v >> 2, g = v & 3;
        const uint8_t* lp = blk + 64 * half + 8 * g;
        const uint8_t* hp = blk + 128 + 32 * half + 8 * g;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t l0 = ld_u16x2(lp + 4 * t), l1 = ld_u16x2(lp + 32 + 4 * t), hq = ld_u16x2(hp + 4 * t);
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const float ds = st[8 * half + (g >> 1) + 2 * qd];
                const uint32_t lb = (qd & 1) ? l1 : l0;
                const uint32_t lo = qd < 2 ? (lb & 0x0F0F0F0Fu) : ((lb >> 4) & 0x0F0F0F0Fu);
                const uint32_t u = lo | (((hq >> (2 * qd)) & 0x03030303u) << 4);
                put4(8 * qd + 4 * t, u, ds, -32.0f * ds);
            }
        }
    }
}

// Store unit v's 32 int8 values, packed four to a word in decode_unit's
// order (w[i] holds vals[4 i .. 4 i + 3]), at their row positions.
template <int KIND>
__device__ __forceinline__ void store_unit(int8_t* out_blk, int v, const uint32_t (&w)[8]) {
    if constexpr (KIND == 4 || KIND == 5) {
        const int j = v >> 1, h = v & 1;
        *reinterpret_cast<uint4*>(out_blk + 64 * j + 16 * h) = make_uint4(w[0], w[1], w[2], w[3]);
        *reinterpret_cast<uint4*>(out_blk + 64 * j + 32 + 16 * h) = make_uint4(w[4], w[5], w[6], w[7]);
    } else {
        const int half = v >> 2, g = v & 3;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd)
            *reinterpret_cast<uint2*>(out_blk + 128 * half + 32 * qd + 8 * g) = make_uint2(w[2 * qd], w[2 * qd + 1]);
    }
}

// Copy `bytes` (even) from global src to the wave's LDS dst with the widest
// loads the alignment allows: 16-byte pieces read whole cache lines per
// instruction, where per-lane 1- and 2-byte reads of the block fields would
// touch many lines each.
__device__ __forceinline__ void copy_to_lds(const uint8_t* src, int bytes, uint8_t* dst, int lane) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(src);
    if ((a & 15) == 0 && (bytes & 15) == 0) {
        for (int i = lane; i < bytes / 16; i += 64)
            reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
    } else if ((a & 3) == 0 && (bytes & 3) == 0) {
        for (int i = lane; i < bytes / 4; i += 64)
            reinterpret_cast<uint32_t*>(dst)[i] = reinterpret_cast<const uint32_t*>(src)[i];
    } else {
        for (int i = lane; i < bytes / 2; i += 64)
            reinterpret_cast<uint16_t*>(dst)[i] = reinterpret_cast<const uint16_t*>(src)[i];
    }
}

template <int KIND, int HOLD>
__global__ __launch_bounds__(kWaves * 64) void repack_w8_kernel(const uint8_t* __restrict__ blocks,
                                                                int64_t n, int nb, int64_t k_pad,
                                                                int8_t* __restrict__ w8,
                                                                float* __restrict__ scales) {
    constexpr int BB = block_bytes(KIND);
    __shared__ float lds[kWaves][kChunkBlocks * 16];
    __shared__ __align__(16) uint8_t raw[kWaves][kChunkBlocks * BB];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
    if (row >= n) return;  // waves share nothing
    const uint8_t* rowp = blocks + row * static_cast<int64_t>(nb) * BB;
    int8_t* outp = w8 + row * k_pad;
    float* st = lds[wave];
    const int nchunks = (nb + kChunkBlocks - 1) / kChunkBlocks;
    const int bi = lane >> 3, v = lane & 7;

    uint8_t* chunk = raw[wave];
    // decode chunk c into vals (lanes past the row's blocks decode nothing):
    // its blocks are copied to the wave's LDS, the factors staged from there.
    // The wave's LDS operations run in order, so what it wrote is read back
    // without a barrier.
    int bad = 0;
    auto decode = [&](int c, float (&vals)[32]) -> bool {
        const int b0 = c * kChunkBlocks;
        const int cnt = min(kChunkBlocks, nb - b0);
        __builtin_amdgcn_wave_barrier();
        copy_to_lds(rowp + b0 * BB, cnt * BB, chunk, lane);
        __builtin_amdgcn_wave_barrier();
        bad |= stage_factors<KIND>(chunk, cnt, lane, st) ? 1 : 0;
        __builtin_amdgcn_wave_barrier();
        if (bi >= cnt) return false;
        decode_unit<KIND>(chunk + bi * BB, v, st + bi * 16, vals);
        return true;
    };
    float vmax = 0.0f;
    auto track = [&](const float (&vals)[32]) {
#pragma unroll
        for (int i = 0; i < 32; i += 2) vmax = fmaxf(vmax, fmaxf(fabsf(vals[i]), fabsf(vals[i + 1])));
    };
    float scale = 1.0f, inv = 1.0f;
    bool fast = true;
    auto finish_max = [&]() {
        vmax = wave_max_nonneg(vmax);
        bad = __any(bad) ? 1 : 0;
        scale = vmax == 0.0f ? 1.0f : vmax / 127.0f;
        inv = 1.0f / scale;
        fast = scale >= 1.175494351e-38f;  // a normal scale (not one of a subnormal max)
    };
    auto quantise_store = [&](int c, const float (&vals)[32]) {
        uint32_t w[8];
        quant_sym_rcp_packed(vals, scale, inv, fast, w);
        if (bad) {
#pragma unroll
            for (int i = 0; i < 8; ++i) w[i] = 0;
        }
        store_unit<KIND>(outp + (c * kChunkBlocks + bi) * kQK, v, w);
    };
    if constexpr (HOLD > 0) {
        float vals[HOLD][32];
        bool have[HOLD];
#pragma unroll
        for (int c = 0; c < HOLD; ++c) {
            have[c] = c < nchunks && decode(c, vals[c]);
            if (have[c]) track(vals[c]);
        }
        finish_max();
#pragma unroll
        for (int c = 0; c < HOLD; ++c)
            if (have[c]) quantise_store(c, vals[c]);
    } else {
        float vals[32];
        for (int c = 0; c < nchunks; ++c)
            if (decode(c, vals)) track(vals);
        finish_max();
        for (int c = 0; c < nchunks; ++c)
            if (decode(c, vals)) quantise_store(c, vals);
    }
    for (int64_t i = static_cast<int64_t>(nb) * kQK + 16 * lane; i < k_pad; i += 64 * 16)
        *reinterpret_cast<uint4*>(outp + i) = make_uint4(0, 0, 0, 0);
    if (lane == 0) scales[row] = bad ? __builtin_nanf("") : scale;
}

// Rows of one chunk (nb <= 8) whose blocks start 16-byte aligned: each wave
// walks rows r, r + (all waves), ... and holds the next row's blocks in
// registers (at most 105 16-byte pieces, two per lane) while it repacks the
// current one, so a row's loads are in flight during the previous row's
// arithmetic instead of after it. The arithmetic per row is repack_w8_kernel's.
template <int KIND>
__global__ __launch_bounds__(kWaves * 64) void repack_w8_stream_kernel(const uint8_t* __restrict__ blocks,
                                                                       int64_t n, int nb, int64_t k_pad,
                                                                       int8_t* __restrict__ w8,
                                                                       float* __restrict__ scales, int grid) {
    constexpr int BB = block_bytes(KIND);
    static_assert(kChunkBlocks * BB <= 128 * 16, "a row's pieces fit two per lane");
    __shared__ float lds[kWaves][kChunkBlocks * 16];
    __shared__ __align__(16) uint8_t raw[kWaves][kChunkBlocks * BB];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t stride = static_cast<int64_t>(grid) * kWaves;  // grid = gridDim.x, preloaded
    int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
    const int pieces = nb * BB / 16;
    const int64_t row_bytes = static_cast<int64_t>(nb) * BB;
    float* st = lds[wave];
    uint8_t* chunk = raw[wave];
    const int bi = lane >> 3, v = lane & 7;
    uint4 p0 = make_uint4(0, 0, 0, 0), p1 = make_uint4(0, 0, 0, 0);
    auto fetch = [&](int64_t r) {
        const uint4* src = reinterpret_cast<const uint4*>(blocks + r * row_bytes);
        if (lane < pieces) p0 = src[lane];
        if (lane + 64 < pieces) p1 = src[lane + 64];
    };
    if (row < n) fetch(row);
    for (; row < n; row += stride) {
        __builtin_amdgcn_wave_barrier();
        if (lane < pieces) reinterpret_cast<uint4*>(chunk)[lane] = p0;
        if (lane + 64 < pieces) reinterpret_cast<uint4*>(chunk)[lane + 64] = p1;
        __builtin_amdgcn_wave_barrier();
        if (row + stride < n) fetch(row + stride);
        int bad = stage_factors<KIND>(chunk, nb, lane, st) ? 1 : 0;
        __builtin_amdgcn_wave_barrier();
        float vals[32];
        float vmax = 0.0f;
        const bool have = bi < nb;
        if (have) {
            decode_unit<KIND>(chunk + bi * BB, v, st + bi * 16, vals);
#pragma unroll
            for (int i = 0; i < 32; i += 2) vmax = fmaxf(vmax, fmaxf(fabsf(vals[i]), fabsf(vals[i + 1])));
        }
        vmax = wave_max_nonneg(vmax);
        bad = __any(bad) ? 1 : 0;
        const float scale = vmax == 0.0f ? 1.0f : vmax / 127.0f;
        const float inv = 1.0f / scale;
        int8_t* outp = w8 + row * k_pad;
        if (have) {
            uint32_t w[8];
            quant_sym_rcp_packed(vals, scale, inv, scale >= 1.175494351e-38f, w);
            if (bad) {
#pragma unroll
                for (int i = 0; i < 8; ++i) w[i] = 0;
            }
            store_unit<KIND>(outp + bi * kQK, v, w);
        }
        for (int64_t i = static_cast<int64_t>(nb) * kQK + 16 * lane; i < k_pad; i += 64 * 16)
            *reinterpret_cast<uint4*>(outp + i) = make_uint4(0, 0, 0, 0);
        if (lane == 0) scales[row] = bad ? __builtin_nanf("") : scale;
    }
}

template <int KIND>
void launch_kind(int64_t n, int nb, int64_t k_pad, const uint8_t* blocks, int8_t* w8, float* scales,
                 hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((n + kWaves - 1) / kWaves)), block(kWaves * 64);
    const int nchunks = (nb + kChunkBlocks - 1) / kChunkBlocks;
    if (nchunks == 1 && (reinterpret_cast<uintptr_t>(blocks) & 15) == 0 &&
        (static_cast<int64_t>(nb) * block_bytes(KIND)) % 16 == 0) {
        // twelve workgroups per CU at most; each wave walks rows from there
        const int64_t wgs = std::min<int64_t>((n + kWaves - 1) / kWaves, static_cast<int64_t>(device_cu_count()) * 12);
        repack_w8_stream_kernel<KIND><<<dim3(static_cast<unsigned>(wgs)), block, 0, stream>>>(blocks, n, nb, k_pad,
                                                                                            w8, scales,
                                                                                            static_cast<int>(wgs));
    } else if (nchunks == 1) repack_w8_kernel<KIND, 1><<<grid, block, 0, stream>>>(blocks, n, nb, k_pad, w8, scales);
    else if (nchunks == 2) repack_w8_kernel<KIND, 2><<<grid, block, 0, stream>>>(blocks, n, nb, k_pad, w8, scales);
    else repack_w8_kernel<KIND, 0><<<grid, block, 0, stream>>>(blocks, n, nb, k_pad, w8, scales);
}

}  // namespace

int launch_repack_w8(int kind, const uint8_t* blocks, int64_t n, int nb, int64_t k_pad, int8_t* w8,
                     float* scales, hipStream_t stream) {
    switch (kind) {
    case 4: launch_kind<4>(n, nb, k_pad, blocks, w8, scales, stream); break;
    case 5: launch_kind<5>(n, nb, k_pad, blocks, w8, scales, stream); break;
    case 6: launch_kind<6>(n, nb, k_pad, blocks, w8, scales, stream); break;
    default: return kStatusInvalid;
    }
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace rk
