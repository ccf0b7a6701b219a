// Shared definitions for the gfx950 kernels of the MUL_MAT offload path.
//
// GGUF K-quant super-blocks hold 256 values. Byte layouts (public ggml ABI;
// block sizes 144 and 210 are pinned by crates/rocknpu-capi/src/lib.rs:5729-5736):
//   Q4_K 144 B: f16 d | f16 dmin | u8 scales[12] | u8 qs[128]
//   Q5_K 176 B: f16 d | f16 dmin | u8 scales[12] | u8 qh[32] | u8 qs[128]
//   Q6_K 210 B: u8 ql[128] | u8 qh[64] | i8 scales[16] | f16 d
//   Q8_K 292 B: f32 d | i8 qs[256] | i16 bsums[16]
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rk {

constexpr int kQK = 256;
constexpr int kQ4KBytes = 144;
constexpr int kQ5KBytes = 176;
constexpr int kQ6KBytes = 210;
constexpr int kQ8KBytes = 292;

constexpr int kStatusOk = 0;
constexpr int kStatusInvalid = -1;
constexpr int kStatusDevice = -2;
constexpr int kStatusExec = -3;

// Compute units of the current device (queried once per device; 256 when the
// query fails). Defined in launch.hip.
int device_cu_count();

// Largest K (a multiple of 64) whose int32 accumulation stays exact:
// |sum| <= 127 * 127 * K < 2^31 for K <= 133143.
constexpr int kMaxExactK = 133120;
// Rows of A8 (m * k_pad bytes) the weight-streaming GEMM stages in LDS at most.
constexpr int kSkinnyMaxA8 = 112 * 1024;
// A W8A8 GEMM launch: tile bm x bn with `stages` K stages of 128 bytes (bm = 0:
// the weight-streaming kernel for up to 16 rows), K split over `splits`
// workgroups per tile (their i32 partials meet in a workspace).
struct GemmTile {
    int bm, bn, stages;
    int splits = 1;
};
GemmTile gemm_route(int m, int n, int k, int cus);  // gemm.hip
// Columns of the first of two launches that launch_gemm_w8a8 splits an
// M x N x K product into (0: one launch). gemm.hip.
int gemm_column_split(int m, int n, int k, int cus);
// A K-split workspace starts with a fixed 16 KiB block: kSplitCounters tile
// counters (whatever the shape, so a workspace reused for other shapes never
// finds another shape's partials in its counters) and, in its last word, a
// sticky error flag that a launch sets when it finds its counters dirty. Then
// the i32 partial tiles, then one arrival stamp per (tile, split).
constexpr int kSplitCounterWords = 4096;
constexpr int kSplitCounters = kSplitCounterWords - 1;
constexpr int kSplitErrorWord = kSplitCounters;
constexpr size_t kSplitCounterBytes = kSplitCounterWords * 4;
// Workspace bytes a split-K launch of `tile` needs for an m x n product.
size_t gemm_workspace_bytes(const GemmTile& tile, int m, int n);  // gemm.hip
// Whether the K split's exchange (relaxed agent-scope atomics, see gemm.hip)
// has been checked on the current device's architecture: gfx950 only. Other
// devices run every GEMM unsplit. gemm.hip.
bool gemm_split_supported();
// Counter words at the start of that workspace (what must be zero at entry).
int gemm_workspace_counters(const GemmTile& tile, int m, int n);  // gemm.hip
// Per-token A8 quantisation; workgroup 0 also clears `nzero` words at
// zero_words (nullptr, 0: none). quant.hip.
int launch_quantize_a8(const float* a, int64_t m, int64_t k, int64_t lda, int64_t k_pad, int8_t* a8,
                       float* scales, uint32_t* zero_words, int nzero, hipStream_t stream);
// The W8A8 GEMM on the routed tile; the routed K split runs when `workspace`
// holds gemm_workspace_bytes of it with zero counters, else unsplit. gemm.hip.
int launch_gemm_w8a8(const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw, const float* as,
                     const float* ws, int m, int n, int k, float* out, int64_t ldo, int32_t* oi,
                     int64_t ldoi, uint8_t* workspace, size_t workspace_bytes, hipStream_t stream);
// The same on a given tile, stage count and split. gemm.hip.
int launch_gemm_w8a8_tile(const GemmTile& r, const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw,
                          const float* as, const float* ws, int m, int n, int k, float* out, int64_t ldo,
                          int32_t* oi, int64_t ldoi, uint8_t* workspace, hipStream_t stream);
// Decode GEMV launch shape: lanes per super-block and waves per workgroup of
// the lane-per-block kernel, and whether the matrix-core kernel runs instead.
struct GemvLanes {
    int lanes, waves;
};
GemvLanes gemv_lanes(bool fused, bool sums, int m, int nb, const int64_t* rows, int count, int cus);  // gemv.hip
bool gemv_uses_mfma(int kind, int m, int nb, int64_t rows, int cus);                                  // gemv.hip
// Stream waves per workgroup of the Q6_K LDS-stream kernel for such a launch,
// or 0 when another kernel runs it. Defined in gemv.hip.
int gemv_stream_waves(int kind, int m, int nb, int64_t rows, bool sums, int cus);
// Block slots per row of the lane-per-block GEMV (log2): the largest power of
// two <= min(slots, nb) whose last pass over a row keeps >= 85% of them busy.
int slots_per_row_log2(int nb, int slots);
// Activation rows per launch the matrix-core GEMV holds for rows of nb blocks
// (0: none). Defined in gemv_mfma.hip.
int gemv_mfma_rows(int kind, int nb);

__host__ __device__ constexpr int block_bytes(int kind) {
    return kind == 4 ? kQ4KBytes : kind == 5 ? kQ5KBytes : kind == 6 ? kQ6KBytes : 0;
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t bits) {
    _Float16 h;
    __builtin_memcpy(&h, &bits, 2);
    return static_cast<float>(h);  // exact widening
}

__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
    return *reinterpret_cast<const uint32_t*>(p);
}

// 6-bit scale and min of sub-block j (0..7) of a Q4_K/Q5_K block from its
// packed 12-byte field, given as three little-endian words s0 s1 s2.
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             int& sc, int& mn) {
    const int b = (j & 3) * 8;
    if (j < 4) {
        sc = (s0 >> b) & 63;
        mn = (s1 >> b) & 63;
    } else {
        sc = ((s2 >> b) & 0xF) | (((s0 >> b) >> 6 & 3) << 4);
        mn = ((s2 >> b) >> 4 & 0xF) | (((s1 >> b) >> 6 & 3) << 4);
    }
}

// Rust's `(v / s).round().clamp(-127.0, 127.0) as i8` with IEEE division:
// round half away from zero, NaN -> 0.
__device__ __forceinline__ int quant_sym(float v, float s) {
    float r = roundf(v / s);
    if (r != r) return 0;
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return static_cast<int>(r);
}

// quant_sym over N values with the reciprocal inv = f32(1 / s), dividing
// only where it can matter. r = f32(v * inv) is within 1.5 * 2^-23 * |v / s|
// (<= 2.3e-5 for |v / s| <= 128) of the correctly rounded quotient
// f32(v / s), so both round to the same integer, half away from zero, unless
// r lies within 2^-15 of a half-integer; away from half-integers rint (ties
// to even) rounds the same way. r - rint(r) is exact. When any of this lane's
// values is that close (about one in 16000), or |r| > 127.5 or NaN, the
// lane's values all take quant_sym itself.
template <int N>
__device__ __forceinline__ void quant_sym_rcp(const float (&v)[N], float s, float inv, int (&q)[N]) {
    bool exact = false;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float r = v[i] * inv;
        const float rr = rintf(r);
        exact |= !(fabsf(r - rr) < 0.5f - 0x1p-15f) || !(fabsf(r) <= 127.5f);
        q[i] = static_cast<int>(rr);
    }
    if (exact) {
#pragma unroll
        for (int i = 0; i < N; ++i) q[i] = quant_sym(v[i], s);
    }
}

// quant_sym_rcp with the int8 results packed four to a word (value 4 i + b in
// byte b of word i), for callers whose scale s is a normal float (`fast`).
// Then |v| <= 127 s gives |r| <= 127 (1 + 3 * 2^-24) < 127.5 for
// r = f32(v * inv), and u = f32(r + 1.5 * 2^23) is rint(r) (ties to even)
// offset into the low mantissa bits, two's complement, so u's low byte is the
// int8 value; u - 1.5 * 2^23 and r - rint(r) are exact. The same rule as
// quant_sym_rcp picks the lane's fallback to quant_sym: the largest
// |r - rint(r)| over its values reaching 0.5 - 2^-15, or !fast.
template <int N>
__device__ __forceinline__ void quant_sym_rcp_packed(const float (&v)[N], float s, float inv, bool fast,
                                                     uint32_t (&w)[N / 4]) {
    constexpr float kRound = 12582912.0f;
    float err = 0.0f;
    // four values at a time, packed as soon as they are rounded, so only four
    // rounded values are live at once
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
        uint32_t u[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float r = v[4 * i + e] * inv;
            const float ur = r + kRound;
            u[e] = __float_as_uint(ur);
            err = fmaxf(err, fabsf(r - (ur - kRound)));
        }
        const uint32_t lo = __builtin_amdgcn_perm(u[1], u[0], 0x0C0C0400u);
        const uint32_t hi = __builtin_amdgcn_perm(u[3], u[2], 0x0C0C0400u);
        w[i] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
    // a wave-uniform branch (a lane's fallback costs the wave the same either
    // way): the compiler then keeps the divisions out of the common path
    if (__builtin_expect(__any(!(fast && err < 0.5f - 0x1p-15f)), 0)) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            w[i] = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) w[i] |= static_cast<uint32_t>(quant_sym(v[4 * i + b], s) & 0xFF) << (8 * b);
        }
    }
}

// Max over the wave of non-negative floats (their bit patterns order as the
// values): DPP steps across lane bits 0-3 (0 is the identity of an unsigned
// max, so each move folds into v_max_u32_dpp), then the four 16-lane rows by
// lane reads. Every lane gets the result.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    unsigned u = __float_as_uint(v);
    u = max(u, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u), 0xB1, 0xF, 0xF, true)));
    u = max(u, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u), 0x4E, 0xF, 0xF, true)));
    u = max(u, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u), 0x141, 0xF, 0xF, true)));
    u = max(u, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u), 0x140, 0xF, 0xF, true)));
    const unsigned r0 = __builtin_amdgcn_readlane(u, 0), r1 = __builtin_amdgcn_readlane(u, 16);
    const unsigned r2 = __builtin_amdgcn_readlane(u, 32), r3 = __builtin_amdgcn_readlane(u, 48);
    return __uint_as_float(max(max(r0, r1), max(r2, r3)));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}


// Decode GEMV launch description (kernel (d)): up to four projections that
// share K and the activation rows; the launch gives each its own workgroups.
constexpr int kGemvMaxMembers = 4;
// LDS bytes per activation row and super-block: quants with a 272-byte block
// stride, bsums with a 48-byte stride, one f32 scale.
constexpr int kGemvLdsQsStride = 272;
constexpr int kGemvLdsBsStride = 48;
constexpr int kGemvLdsPerBlock = kGemvLdsQsStride + kGemvLdsBsStride + 4;
struct GemvParams {
    const uint8_t* w[kGemvMaxMembers];
    float* out[kGemvMaxMembers];
    int64_t ldo[kGemvMaxMembers];
    int64_t rows[kGemvMaxMembers];     // rows (output columns) of each member
    int count;
    const float* x;      // f32 activations [m, ldx] (quantised in-kernel), or
    const uint8_t* q8k;  // Q8_K rows, ldx bytes apart
    int64_t ldx;
    int m;
    int nb;              // super-blocks per row
    int log2g;           // block slots per row = 1 << log2g
    int iters;           // blocks per slot per row group
    int32_t* isum;       // optional exact per-(mi, row, block) sums (count == 1)
    int32_t* msum;
    // the tiled GEMV's K-split exchange (gemv_tiled_split): zeroed slots and
    // error word, gemv_tiled_split_bytes long; null where no split applies
    void* split_ws;
    size_t split_ws_bytes;
};

// The decode cache's tile-interleaved weight layout (gemv_mfma.hip): bytes of
// the tiled copy of n rows of nb blocks, the conversion from raw GGUF blocks,
// and the matrix-core GEMV on such copies (1 <= p.m <= gemv_mfma_rows).
size_t gemv_tiled_bytes(int kind, int64_t n, int nb);
int launch_gemv_tile_weights(int kind, const uint8_t* src, int64_t n, int nb, uint8_t* dst, hipStream_t stream);
int launch_gemv_tiled(int kind, bool fused, GemvParams& p, hipStream_t stream);
// Whether a tiled launch of m activation rows over rows of nb blocks splits
// each tile's blocks over two workgroups (a function of these alone, so a
// row's f32 order does not depend on the projections sharing the launch), and
// the workspace such a launch over `tiles` 16-row tiles needs (0 without a
// split): one 8-byte slot per tile, lane and register row, then the error word.
bool gemv_tiled_split(int kind, int m, int nb);
size_t gemv_tiled_split_bytes(int kind, int m, int nb, int64_t tiles);
// The generation a split launch (GEMM or GEMV) tags its arrivals with.
uint32_t next_split_generation();

}  // namespace rk
