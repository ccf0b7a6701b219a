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
// Mapping: one wave per output row, 4 waves per workgroup. A row is walked in
// chunks of 8 super-blocks (2048 values): per chunk the wave first stages the
// per-sub-block factors (d*sc, dmin*m) into LDS, one sub-block per lane, then
// every lane decodes one 32-value unit. Pass 1 finds max|row|; pass 2 decodes
// again (the row is L2-resident by then), quantises and stores.
#include "common.h"

namespace rk {
namespace {

constexpr int kChunkBlocks = 8;
constexpr int kWaves = 4;

// Stage the per-sub-block factors of `cnt` blocks starting at `chunk` into
// st[16 * block + i]: Q4_K/Q5_K i<8 -> d*sc_i, i>=8 -> dmin*m_(i-8);
// Q6_K i<16 -> d*sc_i.
template <int KIND>
__device__ __forceinline__ void stage_factors(const uint8_t* chunk, int cnt, int lane, float* st) {
    constexpr int BB = block_bytes(KIND);
    if constexpr (KIND == 4 || KIND == 5) {
        const int bi = lane >> 3, j = lane & 7;
        if (bi < cnt) {
            const uint8_t* blk = chunk + bi * BB;
            const uint32_t w0 = ld_u32(blk);
            const float d = f16_bits_to_f32(static_cast<uint16_t>(w0 & 0xFFFF));
            const float dmin = f16_bits_to_f32(static_cast<uint16_t>(w0 >> 16));
            int sc, mn;
            scale_min_k4(j, ld_u32(blk + 4), ld_u32(blk + 8), ld_u32(blk + 12), sc, mn);
            st[bi * 16 + j] = d * static_cast<float>(sc);
            st[bi * 16 + 8 + j] = dmin * static_cast<float>(mn);
        }
    } else {
#pragma unroll
        for (int e = lane; e < kChunkBlocks * 16; e += 64) {
            const int bi = e >> 4, idx = e & 15;
            if (bi < cnt) {
                const uint8_t* blk = chunk + bi * BB;
                const float d = f16_bits_to_f32(ld_u16(blk + 208));
                const int sc = static_cast<int8_t>(blk[192 + idx]);
                st[bi * 16 + idx] = d * static_cast<float>(sc);
            }
        }
    }
}

__device__ __forceinline__ void bytes16(const uint8_t* p, uint8_t (&b)[16]) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    __builtin_memcpy(b, &v, 16);
}

__device__ __forceinline__ void bytes8_u16(const uint8_t* p, uint8_t (&b)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint16_t h = ld_u16(p + 2 * i);
        b[2 * i] = static_cast<uint8_t>(h & 0xFF);
        b[2 * i + 1] = static_cast<uint8_t>(h >> 8);
    }
}

// Decode unit v (0..7) of a block into vals[32].
// Q4_K/Q5_K: j = v/2, h = v%2; vals[0..16) are positions 64j+16h+i (sub-block
//   2j), vals[16..32) are positions 64j+32+16h+i (sub-block 2j+1).
// Q6_K: half = v/4, g = v%4; vals[8q+i] is position 128*half + 32q + 8g + i.
template <int KIND>
__device__ __forceinline__ void decode_unit(const uint8_t* blk, int v, const float* st,
                                            float (&vals)[32]) {
    if constexpr (KIND == 4 || KIND == 5) {
        const int j = v >> 1, h = v & 1;
        uint8_t q[16];
        bytes16(blk + (KIND == 4 ? 16 : 48) + 32 * j + 16 * h, q);
        const float d1 = st[2 * j], d2 = st[2 * j + 1];
        const float m1 = st[8 + 2 * j], m2 = st[8 + 2 * j + 1];
        if constexpr (KIND == 4) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                vals[i] = d1 * static_cast<float>(q[i] & 0xF) - m1;
                vals[16 + i] = d2 * static_cast<float>(q[i] >> 4) - m2;
            }
        } else {
            uint8_t qh[16];
            bytes16(blk + 16 + 16 * h, qh);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int lo = (q[i] & 0xF) + (((qh[i] >> (2 * j)) & 1) << 4);
                const int hi = (q[i] >> 4) + (((qh[i] >> (2 * j + 1)) & 1) << 4);
                vals[i] = d1 * static_cast<float>(lo) - m1;
                vals[16 + i] = d2 * static_cast<float>(hi) - m2;
            }
        }
    } else {
        const int half = v >> 2, g = v & 3;
        uint8_t ql0[8], ql1[8], qh[8];
        bytes8_u16(blk + 64 * half + 8 * g, ql0);
        bytes8_u16(blk + 64 * half + 32 + 8 * g, ql1);
        bytes8_u16(blk + 128 + 32 * half + 8 * g, qh);
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            const float ds = st[8 * half + (g >> 1) + 2 * qd];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint8_t lb = (qd & 1) ? ql1[i] : ql0[i];
                const int lo = (qd < 2) ? (lb & 0xF) : (lb >> 4);
                const int hi = (qh[i] >> (2 * qd)) & 3;
                vals[8 * qd + i] = ds * static_cast<float>((lo | (hi << 4)) - 32);
            }
        }
    }
}

template <int KIND>
__device__ __forceinline__ void store_unit(int8_t* out_blk, int v, const int (&q)[32]) {
    if constexpr (KIND == 4 || KIND == 5) {
        const int j = v >> 1, h = v & 1;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            lo[w] = (q[4 * w] & 0xFF) | (q[4 * w + 1] & 0xFF) << 8 | (q[4 * w + 2] & 0xFF) << 16 |
                    static_cast<uint32_t>(q[4 * w + 3] & 0xFF) << 24;
            hi[w] = (q[16 + 4 * w] & 0xFF) | (q[16 + 4 * w + 1] & 0xFF) << 8 |
                    (q[16 + 4 * w + 2] & 0xFF) << 16 |
                    static_cast<uint32_t>(q[16 + 4 * w + 3] & 0xFF) << 24;
        }
        *reinterpret_cast<uint4*>(out_blk + 64 * j + 16 * h) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *reinterpret_cast<uint4*>(out_blk + 64 * j + 32 + 16 * h) =
            make_uint4(hi[0], hi[1], hi[2], hi[3]);
    } else {
        const int half = v >> 2, g = v & 3;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            uint32_t w[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int* s = &q[8 * qd + 4 * t];
                w[t] = (s[0] & 0xFF) | (s[1] & 0xFF) << 8 | (s[2] & 0xFF) << 16 |
                       static_cast<uint32_t>(s[3] & 0xFF) << 24;
            }
            *reinterpret_cast<uint2*>(out_blk + 128 * half + 32 * qd + 8 * g) = make_uint2(w[0], w[1]);
        }
    }
}

template <int KIND>
__global__ __launch_bounds__(kWaves * 64) void repack_w8_kernel(const uint8_t* __restrict__ blocks,
                                                                int64_t n, int nb, int64_t k_pad,
                                                                int8_t* __restrict__ w8,
                                                                float* __restrict__ scales) {
    constexpr int BB = block_bytes(KIND);
    __shared__ float lds[kWaves][kChunkBlocks * 16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
    const bool active = row < n;
    const uint8_t* rowp = blocks + (active ? row : 0) * static_cast<int64_t>(nb) * BB;
    int8_t* outp = w8 + (active ? row : 0) * k_pad;
    float* st = lds[wave];
    const int nchunks = (nb + kChunkBlocks - 1) / kChunkBlocks;
    const int bi = lane >> 3, v = lane & 7;

    float vmax = 0.0f;
    int bad = 0;
    float scale = 1.0f;
    for (int pass = 0; pass < 2; ++pass) {
        for (int c = 0; c < nchunks; ++c) {
            const int b0 = c * kChunkBlocks;
            const int cnt = min(kChunkBlocks, nb - b0);
            __syncthreads();
            if (active) stage_factors<KIND>(rowp + b0 * BB, cnt, lane, st);
            __syncthreads();
            if (!active || bi >= cnt) continue;
            float vals[32];
            decode_unit<KIND>(rowp + (b0 + bi) * BB, v, st + bi * 16, vals);
            if (pass == 0) {
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const float a = fabsf(vals[i]);
                    bad |= !(a <= 3.402823466e38f);
                    vmax = fmaxf(vmax, a);
                }
            } else {
                int q[32];
#pragma unroll
                for (int i = 0; i < 32; ++i) q[i] = bad ? 0 : quant_sym(vals[i], scale);
                store_unit<KIND>(outp + (b0 + bi) * kQK, v, q);
            }
        }
        if (pass == 0) {
            vmax = wave_max(vmax);
            bad = wave_or(bad);
            scale = vmax == 0.0f ? 1.0f : vmax / 127.0f;
        }
    }
    if (!active) return;
    for (int64_t i = static_cast<int64_t>(nb) * kQK + 16 * lane; i < k_pad; i += 64 * 16)
        *reinterpret_cast<uint4*>(outp + i) = make_uint4(0, 0, 0, 0);
    if (lane == 0) scales[row] = bad ? __builtin_nanf("") : scale;
}

}  // namespace

int launch_repack_w8(int kind, const uint8_t* blocks, int64_t n, int nb, int64_t k_pad, int8_t* w8,
                     float* scales, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((n + kWaves - 1) / kWaves)), block(kWaves * 64);
    switch (kind) {
    case 4: repack_w8_kernel<4><<<grid, block, 0, stream>>>(blocks, n, nb, k_pad, w8, scales); break;
    case 5: repack_w8_kernel<5><<<grid, block, 0, stream>>>(blocks, n, nb, k_pad, w8, scales); break;
    case 6: repack_w8_kernel<6><<<grid, block, 0, stream>>>(blocks, n, nb, k_pad, w8, scales); break;
    default: return kStatusInvalid;
    }
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace rk
