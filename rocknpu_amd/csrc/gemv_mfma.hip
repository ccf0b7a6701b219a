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
template <int KIND, int MT>
__device__ __forceinline__ void block_terms(const MPiece<KIND>& k, const uint64_t (&a)[8],
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
__device__ __forceinline__ const uint8_t* tile_weights(const MfmaArgs& p, int t) {
    const bool c1 = t >= p.mb[0].tile_end, c2 = t >= p.mb[1].tile_end, c3 = t >= p.mb[2].tile_end;
    return c3 ? p.mb[3].w : c2 ? p.mb[2].w : c1 ? p.mb[1].w : p.mb[0].w;
}

template <int KIND, int MT, bool FUSED, int W, bool AREG, int D>
__global__ __launch_bounds__(W * 64) void gemv_mfma_kernel(const MfmaArgs p) {
    constexpr int BB = block_bytes(KIND);
    constexpr int NR = MT / 4;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
        if (++c.it == iters) { c.it = 0; c.t += gridDim.x; }
    };
    const int last_t = p.tiles - 1 - (p.tiles - 1 - static_cast<int>(blockIdx.x)) % static_cast<int>(gridDim.x);
    auto load = [&](const Pos& c, MPiece<KIND>& k) {
        const bool live = c.t < p.tiles;
        const int t = live ? c.t : last_t;
        const TileOut to = tile_out(p, t);
        const int row = min(to.row0 + n, to.rows - 1);
        const int b = min(live ? wave + W * c.it : 0, nb - 1);
        k.load(reinterpret_cast<gbytes>(reinterpret_cast<uint64_t>(tile_weights(p, t))) +
                   static_cast<int64_t>(row) * (nb * BB) + b * BB,
               q);
    };

    OwnedActs<MT, W, FUSED> owned;
    owned.first(p, wave);
    // Every wave's activation loads are issued before any weight load: the
    // weight loads miss in the vector L1 and fill its queue, and an activation
    // load issued behind them waits for them.
    __builtin_amdgcn_s_barrier();
    // the first weight block before the quantisation, the rest of the ring after
    // it: each load instruction issued ahead of the quantisation delays it
    MPiece<KIND> buf[D];
    Pos lq{static_cast<int>(blockIdx.x), 0};  // next item to load
    load(lq, buf[0]);
    advance(lq);
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
    while (cq.t < p.tiles) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            if (cq.t < p.tiles) {  // uniform
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
                if (D > 1 || lq.t < p.tiles) load(lq, buf[j]);
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
                        const TileOut to = tile_out(p, cq.t);
                        const int row = to.row0 + n;
#pragma unroll
                        for (int lr = 0; lr < NR; ++lr) {
                            float r = pb[lane * NR + lr];
#pragma unroll
                            for (int g = 1; g < W; ++g) r += pb[(g * 64 + lane) * NR + lr];
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

// ------------------------------------------------------------ staged weights
// The same product with the Q4_K weights staged through LDS by direct
// global->LDS loads. Loading 8-byte operand pieces of 16 rows per instruction
// (as gemv_mfma_kernel does) touches 16 partly used cache lines per
// instruction; the texture path then spends the launch waiting on the vector
// L1. Here a stage is 16 rows x 8 blocks (1152 contiguous bytes per row),
// copied in 16-byte chunks: wave g copies rows 2g and 2g + 1 (144 chunks, three
// loads of up to 64 lanes), and wave g then multiplies block g of the stage.
// Row r's chunk c sits at chunk (c + 2r) mod 72 of its 1152-byte LDS row, so
// the operand reads of 16 rows spread over the banks. A ring of R stages keeps
// R - 1 in flight; one barrier per stage both publishes stage s (after each
// wave's own wait for its loads) and frees stage s - 1's buffer for stage
// s + R - 1. Tile sums are reduced into an LDS result buffer and stored when
// the workgroup is done, so the loop issues no other memory operations and
// each wait counts exactly the stage loads behind it.
constexpr int kStageRowChunks = kStageBlocks * kQ4KBytes / 16;  // 72
constexpr int kStageBytes = kTileRows * kStageRowChunks * 16;    // 18432
constexpr int kDmaLoads = 3;                                     // loads per wave and stage

__device__ __forceinline__ int stage_chunk(int r, int c) {
    const int p = c + 2 * r;
    return p >= kStageRowChunks ? p - kStageRowChunks : p;
}

// LDS of a staged launch, all of it in arrays of fixed size (a direct load's
// destination is then known to differ from every other buffer, and no read of
// the activations, partial sums or results waits for the stage loads in
// flight): R stage buffers, the activations of MT rows for at most NB blocks
// per row, the double-buffered partial sums of the eight waves, and the sums
// of at most TILES tiles per workgroup.
template <int MT>
struct StagedCfg {
    static constexpr int R = MT == 16 ? 2 : 3;
    static constexpr int TILES = MT == 4 ? 64 : MT == 8 ? 64 : 24;
    static constexpr int NR = MT / 4;
    // partial sums: two buffers and one that non-final stages write to;
    // results: TILES tiles and one slot that non-final stages write to
    static constexpr int PART = 3 * kStageBlocks * 64 * NR * 4, RES = (TILES + 1) * 64 * NR * 4;
    static constexpr int NB = (kLdsMax - 256 - R * kStageBytes - PART - RES) / (MT * kPerRowBlock);
};

template <int MT, bool FUSED>
__global__ __launch_bounds__(kStageBlocks * 64) void gemv_q4_staged_kernel(const MfmaArgs p) {
    using Cfg = StagedCfg<MT>;
    constexpr int W = kStageBlocks;
    constexpr int NR = MT / 4;
    constexpr int R = Cfg::R;
    static_assert(R >= 2 && R <= 3, "two or three stage buffers");
    // one array per stage, indexed only at compile time (the wait-count pass then
    // sees which buffer a direct load writes)
    __shared__ __align__(16) uint8_t st0[kStageBytes], st1[kStageBytes], st2[R > 2 ? kStageBytes : 16];
    __shared__ __align__(16) uint8_t act_lds[Cfg::NB * MT * kPerRowBlock];
    __shared__ __align__(16) float part[Cfg::PART / 4];
    __shared__ __align__(16) float res[Cfg::RES / 4];  // per tile of this workgroup: [lane][NR], wave-order sums
    auto stage_buf = [&](auto u) -> uint8_t* {
        constexpr int U = decltype(u)::value;
        if constexpr (U == 0) return st0; else if constexpr (U == 1) return st1;
        else return st2;
    };
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = p.nb, m = p.m, iters = p.iters;
    const ActLds<MT> act{act_lds, nb};
    const int n = lane & 15, q = lane >> 4;

    const int grid = gridDim.x, bid = blockIdx.x;
    const int ntile = (p.tiles - bid + grid - 1) / grid;  // tiles bid, bid + grid, ..
    const int ns = ntile * iters;                          // stages: (tile k, K chunk c) = (s / iters, s % iters)

    // A stage is 1152 chunks of 16 bytes, LDS chunk P = 72 r + ((c + 2 r) mod 72)
    // holding chunk c of row r: 18 loads of 64 chunks, load j by wave j % 8.
    // Every wave issues three (waves 2..7 repeat load 16 or 17: the same bytes to
    // the same place), all lanes active, so the wait counts are uniform.
    auto issue = [&](int s, auto u) {
        // a stage past the end issues nothing (the waits below count one stage
        // fewer in flight then): issued, its loads queue ahead of the last
        // stages' barriers and the wave's end (TinyLlama gate+up at 4 rows
        // 8.17 -> 7.75 us)
        if (s >= ns) return;
        const int k = s / iters, c = s - k * iters;
        const int t = bid + k * grid;
        const TileOut to = tile_out(p, t);
        const gbytes w = reinterpret_cast<gbytes>(reinterpret_cast<uint64_t>(tile_weights(p, t)));
        const int valid = min(kStageBlocks, nb - c * kStageBlocks) * (kQ4KBytes / 16);  // chunks per row
        uint8_t* base = stage_buf(u);
#pragma unroll
        for (int i = 0; i < kDmaLoads; ++i) {
            const int j = i < 2 ? wave + W * i : 2 * W + (wave & 1);
            const int pos = 64 * j + lane;
            const int r = pos / kStageRowChunks, cpos = pos - r * kStageRowChunks;
            int cg = cpos - 2 * r;
            cg = cg < 0 ? cg + kStageRowChunks : cg;
            cg = cg < valid ? cg : 0;
            const int row = min(to.row0 + r, to.rows - 1);
            const gbytes src = w + static_cast<int64_t>(row) * (nb * kQ4KBytes) + c * (kStageBlocks * kQ4KBytes) + 16 * cg;
            dma16_untracked(reinterpret_cast<const void*>(reinterpret_cast<uint64_t>(src)), base + 1024 * j);
        }
    };

    // The stage loads are inline asm the wait-count pass does not see (seen, a
    // read of a stage buffer after the loop's back edge waits for all of
    // them); their waits are the explicit wait_vm calls. With one block index
    // per wave the activations are quantised from the registers they were
    // loaded into: they are waited for before any stage load is issued, one
    // stage goes out before the quantisation and the rest after. Otherwise the
    // quantisation loads as it goes, and the stage loads follow it.
    OwnedActs<MT, W, FUSED> owned;
    owned.first(p, wave);
    if (iters == 1) {
        wait_vm<0>();
        issue(0, std::integral_constant<int, 0>{});
        owned.stage(p, wave, act);
        if constexpr (R > 2) issue(1, std::integral_constant<int, 1>{});
    } else {
        owned.stage(p, wave, act);
        unroll_seq([&](auto u) { issue(decltype(u)::value, u); }, std::make_integer_sequence<int, R - 1>{});
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    float acc[NR];
#pragma unroll
    for (int lr = 0; lr < NR; ++lr) acc[lr] = 0.0f;

    // The tile ended by stage s - 1: its waves' partial sums added in wave
    // order. Every wave adds them and writes the same values.
    auto reduce = [&](int k, int slot) {
        const float* pb = part + (k & 1) * (W * 64 * NR);
#pragma unroll
        for (int lr = 0; lr < NR; ++lr) {
            float r = pb[lane * NR + lr];
#pragma unroll
            for (int g = 1; g < W; ++g) r += pb[(g * 64 + lane) * NR + lr];
            res[(slot * 64 + lane) * NR + lr] = r;
        }
    };

    // The stage loop is straight-line code up to its exits: a branch that joins
    // inside it would make the wait-count pass wait for every stage load in
    // flight after the join. So the partial-sum writes and the reduction always
    // run (into spare buffers when no tile ends), and the loop leaves before a
    // stage past the end.
    auto step = [&](auto uu, int s) {
        constexpr int U = decltype(uu)::value;
        // this wave's loads of stage s: the stage after it (R = 3) is in flight
        // unless s is the last
        static_assert(R <= 3, "one stage younger at most");
        if (R > 2 && s + 1 < ns) wait_vm<(R - 2) * kDmaLoads>();
        else wait_vm<0>();
        // everyone's, and every wave's LDS writes (partial sums); stage s - 1 is
        // then free. A compiler memory barrier too.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        issue(s + R - 1, std::integral_constant<int, (U + R - 1) % R>{});
        const int sp = s - 1;  // a tile ended there?
        const int kp = sp < 0 ? 0 : sp / iters;
        const bool ended = sp >= 0 && sp - kp * iters == iters - 1;
        reduce(kp, ended ? kp : Cfg::TILES);
        const int k = s / iters, c = s - k * iters;
        const int b = c * kStageBlocks + wave;
        const bool have = b < nb;
        uint64_t areg[8];
        uint32_t bsreg[NR][8];
        float dareg[NR];
        a_operands<4, MT>(act, min(b, nb - 1), lane, areg);
        row_data<4, MT>(act, min(b, nb - 1), lane, bsreg, dareg);
        // this lane's operand bytes of block `wave` of the stage, row n
        const uint8_t* row = stage_buf(uu) + n * (kStageRowChunks * 16);
        const int c0 = wave * (kQ4KBytes / 16);
        MPiece<4> kp4;
        kp4.h = *reinterpret_cast<const v4u*>(row + 16 * stage_chunk(n, c0));
#pragma unroll
        for (int j = 0; j < 4; ++j)
            kp4.qp[j] =
                *reinterpret_cast<const uint64_t*>(row + 16 * stage_chunk(n, c0 + 1 + 2 * j + (q >> 1)) + 8 * (q & 1));
        float term[NR];
        block_terms<4, MT>(kp4, areg, bsreg, dareg, term);
        const bool last = c == iters - 1;  // tile done: partial sums to LDS
        float* pb = part + (last ? (k & 1) : 2) * (W * 64 * NR);
#pragma unroll
        for (int lr = 0; lr < NR; ++lr) {
            acc[lr] += have ? term[lr] : 0.0f;
            pb[(wave * 64 + lane) * NR + lr] = acc[lr];
            acc[lr] = last ? 0.0f : acc[lr];
        }
    };
    for (int s0 = 0;; s0 += R) {
        if (s0 >= ns) break;
        step(std::integral_constant<int, 0>{}, s0);
        if (s0 + 1 >= ns) break;
        step(std::integral_constant<int, 1>{}, s0 + 1);
        if constexpr (R > 2) {
            if (s0 + 2 >= ns) break;
            step(std::integral_constant<int, 2>{}, s0 + 2);
        }
    }
    wait_vm<0>();
    __syncthreads();
    reduce(ntile - 1, ntile - 1);
    __syncthreads();
    // store every tile's rows: wave g the tiles k = g, g + W, ..
    for (int k = wave; k < ntile; k += W) {
        const TileOut to = tile_out(p, bid + k * grid);
        const int row = to.row0 + n;
#pragma unroll
        for (int lr = 0; lr < NR; ++lr) {
            const int mo = NR * q + lr;
            if (mo < m && row < to.rows)
                reinterpret_cast<gfloats>(reinterpret_cast<uint64_t>(to.out))[mo * to.ldo + row] = res[(k * 64 + lane) * NR + lr];
        }
    }
}

template <int KIND, int MT, bool FUSED, int W, bool AREG>
void launch_d(const MfmaArgs& p, int depth, dim3 grid, size_t lds, hipStream_t stream) {
    if (depth >= 4) gemv_mfma_kernel<KIND, MT, FUSED, W, AREG, 4><<<grid, dim3(W * 64), lds, stream>>>(p);
    else if (depth >= 2) gemv_mfma_kernel<KIND, MT, FUSED, W, AREG, 2><<<grid, dim3(W * 64), lds, stream>>>(p);
    else gemv_mfma_kernel<KIND, MT, FUSED, W, AREG, 1><<<grid, dim3(W * 64), lds, stream>>>(p);
}

template <int KIND, int MT, bool FUSED, int W>
void launch_w(const MfmaArgs& p, int depth, dim3 grid, size_t lds, hipStream_t stream) {
    if (p.iters == 1) launch_d<KIND, MT, FUSED, W, true>(p, depth, grid, lds, stream);
    else launch_d<KIND, MT, FUSED, W, false>(p, depth, grid, lds, stream);
}

template <int KIND, int MT, bool FUSED>
void launch_mt(const MfmaArgs& p, int w, int depth, dim3 grid, size_t lds, hipStream_t stream) {
    if (w == 4) launch_w<KIND, MT, FUSED, 4>(p, depth, grid, lds, stream);
    else launch_w<KIND, MT, FUSED, 8>(p, depth, grid, lds, stream);
}

template <int KIND, bool FUSED>
void launch_kind(int mt, const MfmaArgs& p, int w, int depth, dim3 grid, size_t lds, hipStream_t stream) {
    if (mt == 4) launch_mt<KIND, 4, FUSED>(p, w, depth, grid, lds, stream);
    else if (mt == 8) launch_mt<KIND, 8, FUSED>(p, w, depth, grid, lds, stream);
    else if constexpr (KIND == 4) launch_mt<KIND, 16, FUSED>(p, w, depth, grid, lds, stream);
}

template <bool FUSED>
void launch_staged(int mt, const MfmaArgs& p, dim3 grid, hipStream_t stream) {
    const dim3 block(kStageBlocks * 64);
    if (mt == 4) gemv_q4_staged_kernel<4, FUSED><<<grid, block, 0, stream>>>(p);
    else if (mt == 8) gemv_q4_staged_kernel<8, FUSED><<<grid, block, 0, stream>>>(p);
    else gemv_q4_staged_kernel<16, FUSED><<<grid, block, 0, stream>>>(p);
}

}  // namespace

// LDS bytes of a launch: the activation blocks of mt rows and the double-buffered
// partial sums of w waves.
size_t gemv_mfma_lds(int mt, int nb, int w) {
    return ((static_cast<size_t>(nb) * mt * kPerRowBlock + 15) & ~size_t{15}) + 2 * static_cast<size_t>(w) * 64 * (mt / 4) * 4;
}

// Whether the staged kernel takes a Q4_K launch of mt-row tiles, `tiles` tiles
// per workgroup, whose LDS holds rows of nb blocks: rows of more than one stage
// (nb > 8), and at 4 rows also rows of one stage when a workgroup walks two or
// more tiles. With one stage per tile and one tile per workgroup the unstaged
// kernel is faster (its operand loads start without a barrier): TinyLlama o
// (2048 x 2048) at 4 rows 4.94 against 5.21 us, at 8 rows 5.72 against 6.06 us.
// With several one-stage tiles the staged one is faster at 4 rows (TinyLlama
// gate+up, 2 x 5632 x 2048: 8.46 -> 8.1-8.2 us) and slower at 8 (8.5 against
// 9.8 us). With two or more stages per tile it is faster (Llama-3-8B gate+up,
// 2 x 14336 x 4096, at 4 rows 24.8 -> 22.5 us, at 8 rows 27.1 -> 26.2 us).
bool gemv_staged_fits(int mt, int nb, int tiles) {
    if (nb <= kStageBlocks && (mt != 4 || tiles < 2)) return false;
    if (mt == 4) return nb <= StagedCfg<4>::NB && tiles <= StagedCfg<4>::TILES;
    if (mt == 8) return nb <= StagedCfg<8>::NB && tiles <= StagedCfg<8>::TILES;
    return nb <= StagedCfg<16>::NB && tiles <= StagedCfg<16>::TILES;
}

// Activation rows per launch of the matrix-core kernel for rows of nb blocks:
// the largest register tile (16 for Q4_K, 8 for Q6_K, then 4) whose LDS fits,
// or 0 when none does.
int gemv_mfma_rows(int kind, int nb) {
    for (int mt : {16, 8, 4}) {
        if (kind == 6 && mt == 16) continue;
        if (gemv_mfma_lds(mt, nb, 8) <= static_cast<size_t>(kLdsMax)) return mt;
    }
    return 0;
}

// Q4_K or Q6_K, 2 <= p.m <= gemv_mfma_rows(kind, p.nb).
int launch_gemv_mfma(int kind, bool fused, GemvParams& p, hipStream_t stream) {
    if ((kind != 4 && kind != 6) || p.m < 2 || p.m > gemv_mfma_rows(kind, p.nb)) return kStatusInvalid;
    const int mt = p.m <= 4 ? 4 : p.m <= 8 ? 8 : 16;
    // eight waves (eight block slots per tile) unless the rows are shorter
    const int w = p.nb < 8 ? 4 : 8;
    MfmaArgs ka{};
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
    // one workgroup per CU at most; each walks its tiles
    const int cus = device_cu_count();
    const int wgs = std::min(tiles, cus);
    const int per_wg = (tiles + wgs - 1) / wgs;
    const dim3 grid(static_cast<unsigned>(wgs));
    if (kind == 4) {
        // Q4_K: weights staged through LDS when the activations and the
        // workgroup's tile results fit beside the stage ring
        if (gemv_staged_fits(mt, p.nb, per_wg)) {
            ka.iters = (p.nb + kStageBlocks - 1) / kStageBlocks;
            if (fused) launch_staged<true>(mt, ka, grid, stream);
            else launch_staged<false>(mt, ka, grid, stream);
            return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
        }
    }
    const int depth = per_wg * ka.iters > 1 ? 2 : 1;
    const size_t lds = gemv_mfma_lds(mt, p.nb, w);
    if (kind == 4) {
        if (fused) launch_kind<4, true>(mt, ka, w, depth, grid, lds, stream);
        else launch_kind<4, false>(mt, ka, w, depth, grid, lds, stream);
    } else {
        if (fused) launch_kind<6, true>(mt, ka, w, depth, grid, lds, stream);
        else launch_kind<6, false>(mt, ka, w, depth, grid, lds, stream);
    }
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace rk
