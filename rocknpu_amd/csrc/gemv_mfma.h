// The decode GEMV on the matrix cores, shared by the kernels on raw GGUF rows
// (gemv_mfma.hip) and on the decode cache's tiled copies (gemv_tiled.hip).
//
// Kernel (d) for up to 16 activation rows (Q4_K) or 8 (Q6_K): the decode
// GEMV with the per-sub-block integer dot products on the matrix cores.
//
// Same arithmetic as gemv.hip (ggml_vec_dot_q{4,6}_K_q8_K, per block and row):
//   isum = sum_s sc_s * sum_{k in sub-block s} q8[k] * q[k]
//          (Q4_K: s = 0..7 of 32 values; Q6_K: s = 0..15 of 16, q = stored - 32)
//   msum = sum_s mn_s * (sum of the activation quants of sub-block s)   (Q4_K)
//   row += (d * d_a) * isum - (dmin * d_a) * msum                 (f32)
// with exact integers up to the f32 scaling.
//
// v_mfma_i32_16x16x32_i8 on gfx950: lane l supplies row l%16 of A and column
// l%16 of B, with K bytes 8*(l/16) .. +7, and holds D column l%16, rows
// 4*(l/16) + e (e = 0..3). B's 16 columns are 16 weight rows of a tile. A's 16
// rows are MT activation rows times SPLIT = 16/MT sub-block slots, placed so
// that A row r holds activation row r / SPLIT and slot r % SPLIT: the four D
// values of lane l then belong to activation rows NR*(l/16) .. +NR-1 (NR =
// MT/4) and slots e % SPLIT, so a lane adds its sub-blocks' scaled sums on its
// own, with the sub-block of every D value known at compile time. Instruction
// t of a group of SPLIT slots carries sub-block (group * SPLIT + t) in the A
// rows of slot t and zeros in the others, so the group's instructions fill
// disjoint rows of one accumulator. Q6_K's 16-value sub-blocks take half an
// instruction's 32 K slots each: slot s sits in K half s & 1 of instruction
// s >> 1 of its group.
//
// Work split: a tile is 16 weight rows. A workgroup holds W waves; wave g owns
// super-blocks g, g + W, .. of every tile its workgroup walks (tiles
// blockIdx.x, + gridDim.x, ..). Each wave quantises the activation blocks it
// owns (f32 -> Q8_K, ggml quantize_row_q8_K_ref) into its own part of LDS, or
// copies them from Q8_K rows, so no wave waits for another before computing.
// When a tile's blocks are done, the waves leave their f32 partial sums in LDS
// and one wave adds them in wave order and stores the rows: a row's f32 order
// depends only on nb and W, the same in fused, grouped and Q8_K-input launches.
//
// Tiled weights (TILED): the same blocks in the decode cache's tile-interleaved
// order (gemv_tiled.hip), loaded by whole-line instructions into the same
// registers, so the arithmetic and its results are unchanged.
#pragma once

#include "gemv_lds.h"

#include <algorithm>
#include <utility>

namespace rk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int kTileRows = 16;
// blocks per stage row of the staged kernel = its waves per workgroup
constexpr int kStageBlocks = 8;
// LDS of one (block, activation row): 256 quants (272-byte stride: consecutive
// rows in different banks), 16 int16 bsums, one f32 scale.
constexpr int kQsStride = 272;
constexpr int kBsStride = 32;
constexpr int kPerRowBlock = kQsStride + kBsStride + 4;
// LDS a workgroup may use: gfx950's 160 KiB per CU.
constexpr int kLdsMax = 160 * 1024;

struct MfmaMember {
    const uint8_t* w;
    float* out;
    int ldo;
    int rows;
    int tile_end;  // cumulative tile count
    int pad;
};
struct MfmaArgs {
    MfmaMember mb[kGemvMaxMembers];
    const float* x;      // fused: f32 activations, ldx floats apart
    const uint8_t* q8k;  // else: Q8_K rows, ldx bytes apart
    int ldx;
    int m;
    int nb;
    int tiles;
    int iters;  // blocks per wave and tile: ceil(nb / W)
    // gemv_tiled_kernel with a K split (S = 2): blocks per range, the
    // exchange slots, the error word and the launch's generation
    int nbs;
    unsigned long long* split_slot;
    uint32_t* split_err;
    uint32_t gen;
};

// The wave-owned activation blocks in LDS: block b, activation row mi.
template <int MT>
struct ActLds {
    uint8_t* base;
    int nb;
    __device__ __forceinline__ uint8_t* quants(int b, int mi) const { return base + (b * MT + mi) * kQsStride; }
    __device__ __forceinline__ uint32_t* bsums(int b, int mi) const {
        return reinterpret_cast<uint32_t*>(base + nb * MT * kQsStride + (b * MT + mi) * kBsStride);
    }
    __device__ __forceinline__ float* d(int b, int mi) const {
        return reinterpret_cast<float*>(base + nb * MT * (kQsStride + kBsStride)) + b * MT + mi;
    }
};

typedef const __attribute__((address_space(1))) uint32_t* gu32;
typedef const __attribute__((address_space(1))) uint64_t* gu64;

// The bytes of one weight block that lane (n, q) loads: its weight row n of
// the tile, K slot group q.
template <int KIND>
struct MPiece;

// Q4_K: the 16-byte header (d, dmin, 12 scale bytes) and, for each sub-block
// pair j, the 8 quant bytes 32j + 8q .. that hold this lane's K slots of
// sub-blocks 2j (low nibbles) and 2j + 1 (high nibbles).
template <>
struct MPiece<4> {
    v4u h;
    uint64_t qp[4];
    __device__ __forceinline__ void load(gbytes blk, int q) {
        h = reinterpret_cast<gv4u>(blk)[0];
#pragma unroll
        for (int j = 0; j < 4; ++j) qp[j] = reinterpret_cast<gu64>(blk + 16 + 32 * j + 8 * q)[0];
    }
    // the same bytes from a tile block of the tiled layout: row n's header at
    // 16 n, lane l's four 8-byte runs at 256 + 32 l
    __device__ __forceinline__ void load_tiled(gbytes tb, int lane) {
        h = reinterpret_cast<gv4u>(tb)[lane & 15];
        const v4u a = reinterpret_cast<gv4u>(tb + 256 + 32 * lane)[0], b = reinterpret_cast<gv4u>(tb + 256 + 32 * lane)[1];
        qp[0] = static_cast<uint64_t>(a.y) << 32 | a.x;
        qp[1] = static_cast<uint64_t>(a.w) << 32 | a.z;
        qp[2] = static_cast<uint64_t>(b.y) << 32 | b.x;
        qp[3] = static_cast<uint64_t>(b.w) << 32 | b.z;
    }
    // this lane's 8 values of sub-block s (0..7), one per byte
    __device__ __forceinline__ uint64_t values(int s) const {
        return (qp[s >> 1] >> (4 * (s & 1))) & 0x0F0F0F0F0F0F0F0Full;
    }
    // 6-bit scales and mins of sub-blocks 0..3 and 4..7 as packed bytes
    // (ggml get_scale_min_k4 on bytes 4..15 of the block, four at a time)
    __device__ __forceinline__ void packed(uint32_t& sc_lo, uint32_t& sc_hi, uint32_t& mn_lo, uint32_t& mn_hi) const {
        sc_lo = h.y & 0x3F3F3F3Fu;
        mn_lo = h.z & 0x3F3F3F3Fu;
        sc_hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        mn_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    }
    __device__ __forceinline__ void scales(float& d, float& dmin) const {
        d = f16_bits_to_f32(static_cast<uint16_t>(h.x & 0xFFFF));
        dmin = f16_bits_to_f32(static_cast<uint16_t>(h.x >> 16));
    }
};

// Q6_K (210 bytes, 2-byte aligned; ggml dequantize_row_q6_K): value
// 128 h + 32 g + l (half h, quarter g, l < 32) is
//   ((ql[64 h + 32 (g & 1) + l] >> 4 (g >> 1)) & 15) | ((qh[32 h + l] >> 2 g) & 3) << 4
// minus 32, in 16-value sub-block 8 h + 2 g + l / 16 with int8 scale sc[that].
// Lane group q takes l in [8q, 8q + 8) of every quarter: the ql runs 64 h +
// 32 i + 8q (i = 0, 1) and the qh runs 128 + 32 h + 8q, 8 bytes each, loaded
// as three 4-byte aligned words from the word boundary at or below them and
// shifted into place (sh = 0 or 2); the scales as four words and the word of
// bytes 206..209 (scales 14-15 and d). Every load stays inside the block.
template <>
struct MPiece<6> {
    uint32_t ql[4][3];  // [2 h + i][word]
    uint32_t qh[2][3];
    v4u sc;
    uint32_t tail;
    uint32_t sh;
    __device__ __forceinline__ void load(gbytes blk, int q) {
        sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(blk)) & 2u;
        const gbytes b4 = blk - sh;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const gu32 w = reinterpret_cast<gu32>(b4 + 64 * (r >> 1) + 32 * (r & 1) + 8 * q);
            ql[r][0] = w[0]; ql[r][1] = w[1]; ql[r][2] = w[2];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const gu32 w = reinterpret_cast<gu32>(b4 + 128 + 32 * h + 8 * q);
            qh[h][0] = w[0]; qh[h][1] = w[1]; qh[h][2] = w[2];
        }
        typedef v4u v4u_a4 __attribute__((aligned(4)));
        sc = *reinterpret_cast<const __attribute__((address_space(1))) v4u_a4*>(b4 + 192);
        typedef uint32_t u32_a2 __attribute__((aligned(2)));
        tail = *reinterpret_cast<const __attribute__((address_space(1))) u32_a2*>(blk + 206);
    }
    // 8 bytes starting sh bytes into words w[0..2]
    __device__ __forceinline__ uint64_t run8(const uint32_t (&w)[3]) const {
        const uint32_t lo = __builtin_amdgcn_alignbyte(w[1], w[0], sh), hi = __builtin_amdgcn_alignbyte(w[2], w[1], sh);
        return static_cast<uint64_t>(hi) << 32 | lo;
    }
    // The 8 signed values of quarter t % 4 of half t / 4 in this lane's K slots
    // (sub-block 2t for lane groups 0-1, 2t + 1 for 2-3).
    __device__ __forceinline__ uint64_t values(int t) const {
        const int h = t >> 2, g = t & 3;
        const uint64_t lo4 = (run8(ql[2 * h + (g & 1)]) >> (4 * (g >> 1))) & 0x0F0F0F0F0F0F0F0Full;
        const uint64_t hi2 = (run8(qh[h]) >> (2 * g)) & 0x0303030303030303ull;
        const uint64_t v = lo4 | hi2 << 4;  // 0..63 per byte
        // v - 32 per byte without borrows between bytes
        return ((v | 0x8080808080808080ull) - 0x2020202020202020ull) ^ 0x8080808080808080ull;
    }
    // the 16 int8 scales as four words
    __device__ __forceinline__ v4u scale_words() const {
        return v4u{__builtin_amdgcn_alignbyte(sc.y, sc.x, sh), __builtin_amdgcn_alignbyte(sc.z, sc.y, sh),
                   __builtin_amdgcn_alignbyte(sc.w, sc.z, sh), __builtin_amdgcn_alignbyte(tail, sc.w, sh)};
    }
    __device__ __forceinline__ void scales(float& d, float& dmin) const {
        d = f16_bits_to_f32(static_cast<uint16_t>(tail >> 16));
        dmin = 0.0f;
    }
};

// Q6_K from a tile block of the tiled layout: row n's 16 scales at 16 n, its
// fp16 d at 256 + 2 n, and lane l's runs at 288 + 48 l: the four ql runs
// 64 h + 32 i + 8q (in the order 2 h + i) and the two qh runs 128 + 32 h + 8q,
// 8 bytes each. The values, scales and d are MPiece<6>'s.
struct MPiece6T {
    uint64_t ql[4], qh[2];
    v4u sc;
    uint32_t dbits;
    __device__ __forceinline__ void load_tiled(gbytes tb, int lane) {
        sc = reinterpret_cast<gv4u>(tb)[lane & 15];
        dbits = reinterpret_cast<const __attribute__((address_space(1))) uint16_t*>(tb + 256)[lane & 15];
        const gv4u r = reinterpret_cast<gv4u>(tb + 288 + 48 * lane);
        const v4u a = r[0], b = r[1], c = r[2];
        ql[0] = static_cast<uint64_t>(a.y) << 32 | a.x;
        ql[1] = static_cast<uint64_t>(a.w) << 32 | a.z;
        ql[2] = static_cast<uint64_t>(b.y) << 32 | b.x;
        ql[3] = static_cast<uint64_t>(b.w) << 32 | b.z;
        qh[0] = static_cast<uint64_t>(c.y) << 32 | c.x;
        qh[1] = static_cast<uint64_t>(c.w) << 32 | c.z;
    }
    __device__ __forceinline__ uint64_t values(int t) const {
        const int h = t >> 2, g = t & 3;
        const uint64_t lo4 = (ql[2 * h + (g & 1)] >> (4 * (g >> 1))) & 0x0F0F0F0F0F0F0F0Full;
        const uint64_t hi2 = (qh[h] >> (2 * g)) & 0x0303030303030303ull;
        const uint64_t v = lo4 | hi2 << 4;
        return ((v | 0x8080808080808080ull) - 0x2020202020202020ull) ^ 0x8080808080808080ull;
    }
    __device__ __forceinline__ v4u scale_words() const { return sc; }
    __device__ __forceinline__ void scales(float& d, float& dmin) const {
        d = f16_bits_to_f32(static_cast<uint16_t>(dbits));
        dmin = 0.0f;
    }
};

// The operand piece of a kind and layout.
template <int KIND, bool TILED>
struct PieceOf {
    using type = MPiece<KIND>;
};
template <>
struct PieceOf<6, true> {
    using type = MPiece6T;
};

// Operand shapes of a launch of MT activation rows.
template <int KIND, int MT>
struct Shape {
    static constexpr int SPLIT = 16 / MT;  // sub-block slots per accumulator
    static constexpr int NR = MT / 4;      // activation rows per lane
    static constexpr int NSUB = KIND == 4 ? 8 : 16;
    static constexpr int GROUPS = NSUB / SPLIT;
    static constexpr int PER_GROUP = KIND == 4 ? SPLIT : SPLIT / 2;  // instructions per group
    static_assert(GROUPS * PER_GROUP == 8, "eight instructions per block");
};

// A operands of block b: instruction i of 8 (group i / PER_GROUP) gets this
// lane's 8 bytes of its activation row's sub-block for the lane's slot, or
// zeros when the lane's slot is not the one instruction i carries.
template <int KIND, int MT>
__device__ __forceinline__ void a_operands(const ActLds<MT>& act, int b, int lane, uint64_t (&a)[8]) {
    using S = Shape<KIND, MT>;
    const int q = lane >> 4, ra = lane & 15, ma = ra / S::SPLIT, sa = ra % S::SPLIT;
    const uint8_t* qs = act.quants(b, ma);
#pragma unroll
    for (int gi = 0; gi < S::GROUPS; ++gi) {
        if constexpr (KIND == 4) {
            const uint64_t v = *reinterpret_cast<const uint64_t*>(qs + 32 * (gi * S::SPLIT + sa) + 8 * q);
#pragma unroll
            for (int t = 0; t < S::SPLIT; ++t) a[gi * S::SPLIT + t] = sa == t ? v : 0;
        } else {
            const uint64_t v = *reinterpret_cast<const uint64_t*>(qs + 16 * (gi * S::SPLIT + sa) + 8 * (q & 1));
            const bool half = (q >> 1) == (sa & 1);
#pragma unroll
            for (int u = 0; u < S::PER_GROUP; ++u) a[gi * S::PER_GROUP + u] = half && (sa >> 1) == u ? v : 0;
        }
    }
}

// bsums (as int16 pairs) and scales of the lane's activation rows in block b
template <int KIND, int MT>
__device__ __forceinline__ void row_data(const ActLds<MT>& act, int b, int lane, uint32_t (&bs)[MT / 4][8],
                                         float (&da)[MT / 4]) {
    constexpr int NR = MT / 4;
    const int q = lane >> 4;
#pragma unroll
    for (int lr = 0; lr < NR; ++lr) {
        const int mo = NR * q + lr;
        if constexpr (KIND == 4) {
            const uint4* src = reinterpret_cast<const uint4*>(act.bsums(b, mo));
            const uint4 v0 = src[0], v1 = src[1];
            bs[lr][0] = v0.x; bs[lr][1] = v0.y; bs[lr][2] = v0.z; bs[lr][3] = v0.w;
            bs[lr][4] = v1.x; bs[lr][5] = v1.y; bs[lr][6] = v1.z; bs[lr][7] = v1.w;
        }
        da[lr] = *act.d(b, mo);
    }
}

// The f32 terms of one weight block for this lane's activation rows:
// (d * d_a) * isum - (dmin * d_a) * msum (Q4_K), (d * d_a) * isum (Q6_K).
template <int KIND, int MT, class P>
__device__ __forceinline__ void block_terms(const P& k, const uint64_t (&a)[8],
                                            const uint32_t (&bs)[MT / 4][8], const float (&da)[MT / 4],
                                            float (&term)[MT / 4]) {
    using S = Shape<KIND, MT>;
    constexpr int NR = S::NR, SPLIT = S::SPLIT;
    int is[NR];
#pragma unroll
    for (int lr = 0; lr < NR; ++lr) is[lr] = 0;
    if constexpr (KIND == 4) {
        uint32_t sc_lo, sc_hi, mn_lo, mn_hi;
        k.packed(sc_lo, sc_hi, mn_lo, mn_hi);
#pragma unroll
        for (int gi = 0; gi < S::GROUPS; ++gi) {
            v4i dacc = {0, 0, 0, 0};
#pragma unroll
            for (int t = 0; t < SPLIT; ++t)
                dacc = __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(a[gi * SPLIT + t]),
                                                             static_cast<long>(k.values(gi * SPLIT + t)), dacc, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int s = gi * SPLIT + e % SPLIT;  // sub-block of D value e
                const int sc = static_cast<int>(((s < 4 ? sc_lo : sc_hi) >> (8 * (s & 3))) & 0xFF);
                is[e / SPLIT] += __mul24(sc, dacc[e]);
            }
        }
        float dw, dmw;
        k.scales(dw, dmw);
#pragma unroll
        for (int lr = 0; lr < NR; ++lr) {
            // mins: sum_s mn_s * (bsums 2s + 2s+1) by int16 dot products
            int ms = 0;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const uint32_t w = s < 4 ? mn_lo : mn_hi;
                const uint32_t sel = 0x0C000C00u | (0x00010001u * static_cast<uint32_t>(s & 3));
                const uint32_t mn2 = __builtin_amdgcn_perm(0u, w, sel);  // (mn_s, mn_s) as int16
                ms = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, bs[lr][s]), __builtin_bit_cast(v2s, mn2), ms, false);
            }
            term[lr] = (dw * da[lr]) * static_cast<float>(is[lr]) - (dmw * da[lr]) * static_cast<float>(ms);
        }
    } else {
        const v4u scw = k.scale_words();
#pragma unroll
        for (int gi = 0; gi < S::GROUPS; ++gi) {
            v4i dacc = {0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < S::PER_GROUP; ++u)
                dacc = __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(a[gi * S::PER_GROUP + u]),
                                                             static_cast<long>(k.values(gi * S::PER_GROUP + u)), dacc, 0,
                                                             0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int s = gi * SPLIT + e % SPLIT;
                const uint32_t w = s < 4 ? scw.x : s < 8 ? scw.y : s < 12 ? scw.z : scw.w;
                const int sc = static_cast<int8_t>((w >> (8 * (s & 3))) & 0xFF);
                is[e / SPLIT] += __mul24(sc, dacc[e]);
            }
        }
        float dw, dmw;
        k.scales(dw, dmw);
#pragma unroll
        for (int lr = 0; lr < NR; ++lr) term[lr] = (dw * da[lr]) * static_cast<float>(is[lr]);
    }
}

// The activation blocks wave `wave` owns, quantised (f32 x, ggml
// quantize_row_q8_K_ref) or copied (Q8_K rows) into its part of LDS: block
// wave + W * it (it < iters) of rows mi < m, four (block, row) items per pass of
// 16 lanes each, so QP = MT / 4 passes per block index; lane group qslot
// takes row 4 i + qslot in pass i. The first block index's activations are
// loaded (`first`) before the caller issues its weight loads, so their waits
// never include those; later ones load during the passes before.
template <int MT, int W, bool FUSED>
struct OwnedActs {
    static constexpr int QP = MT / 4;
    float4 xf[FUSED ? QP : 1][4];
    __device__ __forceinline__ void first(const MfmaArgs& p, int wave) {
        if constexpr (FUSED) {
            const int qslot = (threadIdx.x & 63) >> 4;
#pragma unroll
            for (int i = 0; i < QP; ++i)
                load_x16(p.x, p.ldx, p.nb, min(4 * i + qslot, p.m - 1) * p.nb + min(wave, p.nb - 1), xf[i]);
        }
    }
    // ONE: one block index per wave (iters == 1), quantised from the loaded
    // registers as they are
    template <bool ONE = false>
    __device__ __forceinline__ void stage(const MfmaArgs& p, int wave, const ActLds<MT>& act) {
        const int lane = threadIdx.x & 63, nb = p.nb, m = p.m, iters = p.iters;
        if constexpr (FUSED && ONE) {
            const int qslot = lane >> 4;
#pragma unroll
            for (int i = 0; i < QP; ++i) {
                const int mi = 4 * i + qslot;
                if (mi < m && wave < nb)
                    quantize_block(xf[i], act.quants(wave, mi), reinterpret_cast<int16_t*>(act.bsums(wave, mi)),
                                   act.d(wave, mi));
            }
        } else if constexpr (FUSED) {
            const int qslot = lane >> 4;
            for (int it = 0; it < iters; ++it) {
                const int b = wave + W * it;
#pragma unroll
                for (int i = 0; i < QP; ++i) {
                    float4 cur[4] = {xf[i][0], xf[i][1], xf[i][2], xf[i][3]};
                    if (it + 1 < iters)  // the next block index's activations
                        load_x16(p.x, p.ldx, nb, min(4 * i + qslot, m - 1) * nb + min(b + W, nb - 1), xf[i]);
                    const int mi = 4 * i + qslot;
                    if (mi < m && b < nb)
                        quantize_block(cur, act.quants(b, mi), reinterpret_cast<int16_t*>(act.bsums(b, mi)),
                                       act.d(b, mi));
                }
            }
        } else {
            // Q8_K blocks of 292 bytes: f32 d, 256 quants, 16 int16 bsums
            for (int w = lane; w < iters * MT * (kQ8KBytes / 4); w += 64) {
                const int j = w / (kQ8KBytes / 4), wi = w - j * (kQ8KBytes / 4);
                const int mi = j % MT, b = wave + W * (j / MT);
                if (b >= nb || mi >= m) continue;
                const uint32_t v = *reinterpret_cast<const uint32_t*>(p.q8k + mi * p.ldx + b * kQ8KBytes + 4 * wi);
                if (wi == 0) *act.d(b, mi) = __uint_as_float(v);
                else if (wi <= 64) reinterpret_cast<uint32_t*>(act.quants(b, mi))[wi - 1] = v;
                else act.bsums(b, mi)[wi - 65] = v;
            }
        }
    }
};

// The fields of MfmaArgs that a tiled launch's first loads need, passed ahead
// of it as scalar kernel arguments (14 dwords, preloaded in SGPRs; the struct
// itself is read from the argument segment, a memory round trip at the start
// of every wave): the activations (f32 or Q8_K), the first three members'
// weights and tile ends, the grid size and the counts, two 16-bit halves a
// dword. A launch with a fourth member, or more than 0xffff tiles, is split
// on the host, so member 3 repeats member 2.
struct TiledHead {
    const void* x;
    const uint8_t* w0;
    const uint8_t* w1;
    const uint8_t* w2;
    int te01;     // tile ends of members 0 and 1: te0 | te1 << 16
    int tiles;    // at most 0xffff
    int grid;     // workgroups (gridDim.x, a hidden argument after the struct)
    int ldx;
    int nb_nbs;   // nb | nbs << 16
    int m_iters;  // m | iters << 16
};
// The tile lookups of tile_out / tile_weights on the preloaded fields (t below
// the launch's tile count, so at most member 2). The selects are of values:
// a conditional of two members (lvalues) selects their addresses, and the
// struct would then live in scratch memory.
struct TileMap {
    const uint8_t* w0;
    const uint8_t* w1;
    const uint8_t* w2;
    int te0, te1;
    __device__ __forceinline__ const uint8_t* weights(int t) const {
        const uint8_t *a = w0, *b = w1, *c = w2;
        const int e0 = te0, e1 = te1;
        return t >= e1 ? c : t >= e0 ? b : a;
    }
    __device__ __forceinline__ int row0(int t) const {
        const int e0 = te0, e1 = te1;
        return (t - (t >= e1 ? e1 : t >= e0 ? e0 : 0)) * kTileRows;
    }
};

// The scalar arguments ahead of MfmaArgs (TiledHead); p has at most three
// members (launch_gemv splits a fourth off, and launch_gemv_tiled /
// launch_gemv_mfma larger launches) and 16-bit counts.
TiledHead tiled_head(const MfmaArgs& p, bool fused, unsigned grid) {
    return TiledHead{fused ? static_cast<const void*>(p.x) : static_cast<const void*>(p.q8k), p.mb[0].w, p.mb[1].w,
                     p.mb[2].w,
                     static_cast<int>(static_cast<uint32_t>(p.mb[0].tile_end) |
                                      static_cast<uint32_t>(p.mb[1].tile_end) << 16),
                     p.tiles, static_cast<int>(grid), p.ldx,
                     static_cast<int>(static_cast<uint32_t>(p.nb) | static_cast<uint32_t>(p.nbs) << 16),
                     static_cast<int>(static_cast<uint32_t>(p.m) | static_cast<uint32_t>(p.iters) << 16)};
}
bool head_fits(const MfmaArgs& p) {
    return p.mb[2].tile_end == p.tiles && p.tiles <= 0xffff && p.nb >= 0 && p.nb <= 0xffff && p.nbs >= 0 && p.nbs <= 0xffff && p.m >= 0 &&
           p.m <= 0xffff && p.iters >= 0 && p.iters <= 0xffff;
}
#define RK_HEAD(h) h.x, h.w0, h.w1, h.w2, h.te01, h.tiles, h.grid, h.ldx, h.nb_nbs, h.m_iters

// The member (projection) of tile t and the tile's first row in it.
struct TileOut {
    float* out;
    int ldo, rows, row0;
};
__device__ __forceinline__ TileOut tile_out(const MfmaArgs& p, int t) {
    const bool c1 = t >= p.mb[0].tile_end, c2 = t >= p.mb[1].tile_end, c3 = t >= p.mb[2].tile_end;
    const int t0 = c3 ? p.mb[2].tile_end : c2 ? p.mb[1].tile_end : c1 ? p.mb[0].tile_end : 0;
    return TileOut{c3 ? p.mb[3].out : c2 ? p.mb[2].out : c1 ? p.mb[1].out : p.mb[0].out,
                   c3 ? p.mb[3].ldo : c2 ? p.mb[2].ldo : c1 ? p.mb[1].ldo : p.mb[0].ldo,
                   c3 ? p.mb[3].rows : c2 ? p.mb[2].rows : c1 ? p.mb[1].rows : p.mb[0].rows, (t - t0) * kTileRows};
}
// tile_out on the preloaded tile ends and the fetched output fields (values
// selected, so nothing lives in scratch memory).
__device__ __forceinline__ TileOut tile_out(const TileMap& tm, const MemberOuts& mo, int t) {
    const int e0 = tm.te0, e1 = tm.te1;
    const bool c1 = t >= e0, c2 = t >= e1;
    const float *a = mo.o0, *b = mo.o1, *c = mo.o2;
    const int la = mo.l0, lb = mo.l1, lc = mo.l2, ra = mo.r0, rb = mo.r1, rc = mo.r2;
    return TileOut{const_cast<float*>(c2 ? c : c1 ? b : a), c2 ? lc : c1 ? lb : la, c2 ? rc : c1 ? rb : ra,
                   (t - (c2 ? e1 : c1 ? e0 : 0)) * kTileRows};
}
// A row's f32 sum from the W waves' partial sums pb[wave][lane][NR] of a tile,
// in the order of the 8-wave kernel: the partials in wave order. With 16 waves
// and one block per wave (rows of at most 16 blocks), wave s + 8 holds the
// block that the 8-wave kernel's wave s adds second, so the partials of waves
// s and s + 8 are added first: (0 + t_s) + (0 + t_{s+8}) equals that wave's
// (0 + t_s) + t_{s+8} (adding 0 changes only a -0, and 0 + x is never -0), and
// the row's bits are those of 8 waves whatever the launch's wave count.
template <int W, int NR>
__device__ __forceinline__ float tile_row_sum(const float* pb, int lane, int lr, int iters) {
    if (W == 16 && iters == 1) {
        float r = pb[lane * NR + lr] + pb[(8 * 64 + lane) * NR + lr];
#pragma unroll
        for (int s = 1; s < 8; ++s) r += pb[(s * 64 + lane) * NR + lr] + pb[((s + 8) * 64 + lane) * NR + lr];
        return r;
    }
    float r = pb[lane * NR + lr];
#pragma unroll
    for (int g = 1; g < W; ++g) r += pb[(g * 64 + lane) * NR + lr];
    return r;
}

__device__ __forceinline__ const uint8_t* tile_weights(const MfmaArgs& p, int t) {
    const bool c1 = t >= p.mb[0].tile_end, c2 = t >= p.mb[1].tile_end, c3 = t >= p.mb[2].tile_end;
    return c3 ? p.mb[3].w : c2 ? p.mb[2].w : c1 ? p.mb[1].w : p.mb[0].w;
}

template <int KIND, int MT, bool FUSED, int W, bool AREG, int D, bool TILED>
__global__ __launch_bounds__(W * 64) void gemv_mfma_kernel(const void* x, const uint8_t* w0, const uint8_t* w1,
                                                             const uint8_t* w2, int te01, int tiles, int grid,
                                                             int ldx, int nb_nbs, int m_iters, const MfmaArgs pa) {
    constexpr int BB = block_bytes(KIND);
    using Piece = typename PieceOf<KIND, TILED>::type;
    constexpr int NR = MT / 4;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // p: the arguments, with the preloaded fields (TiledHead) in place of the
    // struct's copies; only its scalar fields are read
    MfmaArgs p = pa;
    p.x = static_cast<const float*>(x);
    p.q8k = static_cast<const uint8_t*>(x);
    p.ldx = ldx;
    p.nb = nb_nbs & 0xffff;
    p.m = m_iters & 0xffff;
    p.iters = static_cast<int>(static_cast<uint32_t>(m_iters) >> 16);
    p.tiles = tiles;
    const TileMap tmap{w0, w1, w2, te01 & 0xffff, static_cast<int>(static_cast<uint32_t>(te01) >> 16)};
    const int nb = p.nb, m = p.m, iters = p.iters;
    const ActLds<MT> act{smem, nb};
    // f32 partial sums of a tile: [buffer][wave][lane][NR], after the activations
    float* part = reinterpret_cast<float*>(smem + ((nb * MT * kPerRowBlock + 15) & ~15));
    const int n = lane & 15, q = lane >> 4;  // B column (weight row in the tile), K slot group

    // Items: (tile t = blockIdx.x + k * gridDim.x, iteration it < iters), walked
    // with counters. With more than one block in flight, loads past the last
    // item re-read the last tile's first block (in bounds) and are never used.
    struct Pos {
        int t;
        int it;
    };
    auto advance = [&](Pos& c) {
        if (++c.it == iters) { c.it = 0; c.t += grid; }
    };
    const int last_t = tiles - 1 - (tiles - 1 - static_cast<int>(blockIdx.x)) % grid;
    // the members' output fields (MemberOuts): on raw rows first thing (the
    // first load needs the member's row count), on tiled copies behind the
    // first weight load (as gemv_tiled_kernel)
    MemberOuts mo{};
    if constexpr (!TILED) mo.fetch(pa);
    auto load = [&](const Pos& c, Piece& k) {
        const bool live = c.t < tiles;
        const int t = live ? c.t : last_t;
        const int b = min(live ? wave + W * c.it : 0, nb - 1);
        const gbytes w = reinterpret_cast<gbytes>(reinterpret_cast<uint64_t>(tmap.weights(t)));
        if constexpr (TILED) {
            // tile block (tile of the member, b): the member's rows are padded to
            // whole tiles, so every lane's bytes exist
            k.load_tiled(w + (static_cast<int64_t>(tmap.row0(t) / kTileRows) * nb + b) * (kTileRows * BB), lane);
        } else {
            // the member's row count (raw rows are not padded to whole tiles)
            const int row = min(tmap.row0(t) + n, tile_out(tmap, mo, t).rows - 1);
            k.load(w + static_cast<int64_t>(row) * (nb * BB) + b * BB, q);
        }
    };

    OwnedActs<MT, W, FUSED> owned;
    owned.first(p, wave);
    // Every wave's activation loads are issued before any weight load: the
    // weight loads miss in the vector L1 and fill its queue, and an activation
    // load issued behind them waits for them.
    __builtin_amdgcn_s_barrier();
    // the first weight block before the quantisation, the rest of the ring after
    // it: each load instruction issued ahead of the quantisation delays it
    Piece buf[D];
    Pos lq{static_cast<int>(blockIdx.x), 0};  // next item to load
    load(lq, buf[0]);
    advance(lq);
    if constexpr (TILED) mo.fetch(pa);
    owned.template stage<AREG>(p, wave, act);
#pragma unroll
    for (int j = 1; j < D; ++j) {
        load(lq, buf[j]);
        advance(lq);
    }
    // The wave's own LDS writes complete before its lanes read each other's
    // bytes; a compiler barrier too, and no wait for the weight loads.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    uint64_t areg[8];
    uint32_t bsreg[NR][8];
    float dareg[NR];
    if constexpr (AREG) {  // one block per wave: its operands stay in registers
        const int b = min(wave, nb - 1);
        a_operands<KIND, MT>(act, b, lane, areg);
        row_data<KIND, MT>(act, b, lane, bsreg, dareg);
    }

    float acc[NR];
#pragma unroll
    for (int lr = 0; lr < NR; ++lr) acc[lr] = 0.0f;
    int tile_iter = 0;
    Pos cq{static_cast<int>(blockIdx.x), 0};  // item being computed
    while (cq.t < tiles) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            if (cq.t < tiles) {  // uniform
                const int it = cq.it;
                const int b = wave + W * it;
                const bool have = b < nb;  // uniform; a missing block is computed on block nb-1 and dropped
                if constexpr (!AREG) {
                    a_operands<KIND, MT>(act, min(b, nb - 1), lane, areg);
                    row_data<KIND, MT>(act, min(b, nb - 1), lane, bsreg, dareg);
                }
                float term[NR];
                block_terms<KIND, MT>(buf[j], areg, bsreg, dareg, term);
#pragma unroll
                for (int lr = 0; lr < NR; ++lr) acc[lr] += have ? term[lr] : 0.0f;
                // With one block in flight a load past the last item is skipped:
                // issued, it queues ahead of the tile's barrier and the wave's
                // end (TinyLlama o and qkv at 4 rows, one tile per workgroup:
                // 4.45 -> 3.9 us). With more in flight the loads stay
                // unconditional, so the wait counts cover exactly the block each
                // value needs.
                if (D > 1 || lq.t < tiles) load(lq, buf[j]);
                advance(lq);
                if (it == iters - 1) {
                    // tile done: partial sums to LDS, then one wave adds them in wave order
                    float* pb = part + (tile_iter & 1) * (W * 64 * NR);
#pragma unroll
                    for (int lr = 0; lr < NR; ++lr) {
                        pb[(wave * 64 + lane) * NR + lr] = acc[lr];
                        acc[lr] = 0.0f;
                    }
                    // the LDS writes complete, then the barrier; a compiler memory
                    // barrier too, and no wait for the weight loads in flight
                    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                    if (wave == (tile_iter & (W - 1))) {
                        const TileOut to = tile_out(tmap, mo, cq.t);
                        const int row = to.row0 + n;
#pragma unroll
                        for (int lr = 0; lr < NR; ++lr) {
                            const float r = tile_row_sum<W, NR>(pb, lane, lr, iters);
                            const int mo = NR * q + lr;
                            if (mo < m && row < to.rows)
                                reinterpret_cast<gfloats>(reinterpret_cast<uint64_t>(to.out))[mo * to.ldo + row] = r;
                        }
                    }
                    ++tile_iter;
                }
                advance(cq);
            }
        }
    }
}

// The kernel arguments of a matrix-core launch with w waves: the members'
// tiles in order, every field checked to fit its 32-bit slot.
int mfma_args(const GemvParams& p, int w, MfmaArgs& ka) {
    ka = MfmaArgs{};
    int tiles = 0;
    for (int i = 0; i < p.count; ++i) {
        if (p.rows[i] > INT32_MAX / 2 || p.ldo[i] > INT32_MAX || p.ldo[i] * (p.m - 1) + p.rows[i] > INT32_MAX)
            return kStatusInvalid;
        tiles += static_cast<int>((p.rows[i] + kTileRows - 1) / kTileRows);
        ka.mb[i] = MfmaMember{p.w[i], p.out[i], static_cast<int>(p.ldo[i]), static_cast<int>(p.rows[i]), tiles, 0};
    }
    if (p.ldx > INT32_MAX / 8) return kStatusInvalid;
    for (int i = p.count; i < kGemvMaxMembers; ++i) ka.mb[i] = ka.mb[p.count - 1];
    ka.x = p.x;
    ka.q8k = p.q8k;
    ka.ldx = static_cast<int>(p.ldx);
    ka.m = p.m;
    ka.nb = p.nb;
    ka.tiles = tiles;
    ka.iters = (p.nb + w - 1) / w;
    return kStatusOk;
}

}  // namespace

// LDS bytes of a launch: the activation blocks of mt rows and the
// double-buffered partial sums of w waves. gemv_mfma.hip.
size_t gemv_mfma_lds(int mt, int nb, int w);

}  // namespace rk
