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

namespace rk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int kTileRows = 16;
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

template <int KIND, int MT, bool FUSED, int W, bool AREG, int D>
__global__ __launch_bounds__(W * 64) void gemv_mfma_kernel(const MfmaArgs p) {
    constexpr int BB = block_bytes(KIND);
    constexpr int SPLIT = 16 / MT;  // sub-block slots per accumulator
    constexpr int NR = MT / 4;      // activation rows per lane
    constexpr int NSUB = KIND == 4 ? 8 : 16;
    constexpr int GROUPS = NSUB / SPLIT;
    constexpr int PER_GROUP = KIND == 4 ? SPLIT : SPLIT / 2;  // instructions per group
    static_assert(GROUPS * PER_GROUP == 8, "eight instructions per block");
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = p.nb, m = p.m, iters = p.iters;
    const ActLds<MT> act{smem, nb};
    // f32 partial sums of a tile: [buffer][wave][lane][NR], after the activations
    float* part = reinterpret_cast<float*>(smem + ((nb * MT * kPerRowBlock + 15) & ~15));

    const int n = lane & 15, q = lane >> 4;  // B column (weight row in the tile), K slot group
    const int ra = lane & 15, ma = ra / SPLIT, sa = ra % SPLIT;  // this lane's A row: activation row, slot

    // Items: (tile t = blockIdx.x + k * gridDim.x, iteration it < iters), walked
    // with counters. Loads past the last item re-read the last tile's first
    // block (in bounds) and are never used.
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
        const bool c1 = t >= p.mb[0].tile_end, c2 = t >= p.mb[1].tile_end, c3 = t >= p.mb[2].tile_end;
        const uint8_t* w = c3 ? p.mb[3].w : c2 ? p.mb[2].w : c1 ? p.mb[1].w : p.mb[0].w;
        const int rows = c3 ? p.mb[3].rows : c2 ? p.mb[2].rows : c1 ? p.mb[1].rows : p.mb[0].rows;
        const int t0 = c3 ? p.mb[2].tile_end : c2 ? p.mb[1].tile_end : c1 ? p.mb[0].tile_end : 0;
        const int row = min((t - t0) * kTileRows + n, rows - 1);
        const int b = min(live ? wave + W * c.it : 0, nb - 1);
        k.load(reinterpret_cast<gbytes>(reinterpret_cast<uint64_t>(w)) + static_cast<int64_t>(row) * (nb * BB) + b * BB, q);
    };

    // The activation blocks this wave owns: block wave + W * it (it < iters)
    // of rows mi < m, four (block, row) items per pass of 16 lanes each, so
    // QP = MT / 4 passes per block index; lane group qslot takes row 4 i + qslot
    // in pass i.
    constexpr int QP = MT / 4;
    const int qslot = lane >> 4;
    float4 xf[FUSED ? QP : 1][4];
    auto x_block = [&](int it, int i) { return min(4 * i + qslot, m - 1) * nb + min(wave + W * it, nb - 1); };
    if constexpr (FUSED) {
        // the first block index's activations first, so their waits never include the weight loads
#pragma unroll
        for (int i = 0; i < QP; ++i) load_x16(p.x, p.ldx, nb, x_block(0, i), xf[i]);
    }
    // the first weight block before the quantisation, the rest of the ring after
    // it: each load instruction issued ahead of the quantisation delays it
    MPiece<KIND> buf[D];
    Pos lq{static_cast<int>(blockIdx.x), 0};  // next item to load
    load(lq, buf[0]);
    advance(lq);
    if constexpr (FUSED) {
        for (int it = 0; it < iters; ++it) {
            const int b = wave + W * it;
#pragma unroll
            for (int i = 0; i < QP; ++i) {
                float4 cur[4] = {xf[i][0], xf[i][1], xf[i][2], xf[i][3]};
                if (it + 1 < iters) load_x16(p.x, p.ldx, nb, x_block(it + 1, i), xf[i]);  // next block index
                const int mi = 4 * i + qslot;
                if (mi < m && b < nb)
                    quantize_block(cur, act.quants(b, mi), reinterpret_cast<int16_t*>(act.bsums(b, mi)), act.d(b, mi));
            }
        }
    } else {
        // copy this wave's Q8_K blocks (292 bytes: f32 d, 256 quants, 16 int16 bsums)
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
#pragma unroll
    for (int j = 1; j < D; ++j) {
        load(lq, buf[j]);
        advance(lq);
    }
    // The wave's own LDS writes complete before its lanes read each other's
    // bytes; a compiler barrier too, and no wait for the weight loads.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // A operands of a block: instruction i of 8 (group i / PER_GROUP) gets this
    // lane's 8 bytes of its activation row's sub-block for the lane's slot, or
    // zeros when the lane's slot is not the one instruction i carries.
    auto a_ops = [&](int b, uint64_t (&a)[8]) {
        const uint8_t* qs = act.quants(b, ma);
#pragma unroll
        for (int gi = 0; gi < GROUPS; ++gi) {
            if constexpr (KIND == 4) {
                const uint64_t v = *reinterpret_cast<const uint64_t*>(qs + 32 * (gi * SPLIT + sa) + 8 * q);
#pragma unroll
                for (int t = 0; t < SPLIT; ++t) a[gi * SPLIT + t] = sa == t ? v : 0;
            } else {
                const uint64_t v = *reinterpret_cast<const uint64_t*>(qs + 16 * (gi * SPLIT + sa) + 8 * (q & 1));
                const bool half = (q >> 1) == (sa & 1);
#pragma unroll
                for (int u = 0; u < PER_GROUP; ++u) a[gi * PER_GROUP + u] = half && (sa >> 1) == u ? v : 0;
            }
        }
    };
    // bsums (as int16 pairs) and scales of the lane's activation rows
    auto row_data = [&](int b, uint32_t (&bs)[NR][8], float (&da)[NR]) {
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
    };

    uint64_t areg[AREG ? 8 : 1];
    uint32_t bsreg[AREG ? NR : 1][8];
    float dareg[AREG ? NR : 1];
    if constexpr (AREG) {  // one block per wave: its operands stay in registers
        const int b = min(wave, nb - 1);
        a_ops(b, areg);
        row_data(b, bsreg, dareg);
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
                const int bk = min(b, nb - 1);
                const MPiece<KIND>& k = buf[j];
                uint64_t alocal[AREG ? 1 : 8];
                uint32_t bslocal[AREG ? 1 : NR][8];
                float dalocal[AREG ? 1 : NR];
                if constexpr (!AREG) {
                    a_ops(bk, alocal);
                    row_data(bk, bslocal, dalocal);
                }
                const uint64_t* a = AREG ? areg : alocal;
                int is[NR];
#pragma unroll
                for (int lr = 0; lr < NR; ++lr) is[lr] = 0;
                if constexpr (KIND == 4) {
                    uint32_t sc_lo, sc_hi, mn_lo, mn_hi;
                    k.packed(sc_lo, sc_hi, mn_lo, mn_hi);
#pragma unroll
                    for (int gi = 0; gi < GROUPS; ++gi) {
                        v4i dacc = {0, 0, 0, 0};
#pragma unroll
                        for (int t = 0; t < SPLIT; ++t)
                            dacc = __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(a[gi * SPLIT + t]),
                                                                         static_cast<long>(k.values(gi * SPLIT + t)),
                                                                         dacc, 0, 0, 0);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int s = gi * SPLIT + e % SPLIT;  // sub-block of D value e
                            const int sc = static_cast<int>(((s < 4 ? sc_lo : sc_hi) >> (8 * (s & 3))) & 0xFF);
                            is[e / SPLIT] += __mul24(sc, dacc[e]);
                        }
                    }
                    // mins: sum_s mn_s * (bsums 2s + 2s+1) by int16 dot products
                    int ms[NR];
#pragma unroll
                    for (int lr = 0; lr < NR; ++lr) {
                        const uint32_t(&bsl)[8] = AREG ? bsreg[lr] : bslocal[lr];
                        int acc_ms = 0;
#pragma unroll
                        for (int s = 0; s < 8; ++s) {
                            const uint32_t w = s < 4 ? mn_lo : mn_hi;
                            const uint32_t sel = 0x0C000C00u | (0x00010001u * static_cast<uint32_t>(s & 3));
                            const uint32_t mn2 = __builtin_amdgcn_perm(0u, w, sel);  // (mn_s, mn_s) as int16
                            acc_ms = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, bsl[s]), __builtin_bit_cast(v2s, mn2),
                                                            acc_ms, false);
                        }
                        ms[lr] = acc_ms;
                    }
                    float dw, dmw;
                    k.scales(dw, dmw);
#pragma unroll
                    for (int lr = 0; lr < NR; ++lr) {
                        const float da = AREG ? dareg[lr] : dalocal[lr];
                        const float term = (dw * da) * static_cast<float>(is[lr]) - (dmw * da) * static_cast<float>(ms[lr]);
                        acc[lr] += have ? term : 0.0f;
                    }
                } else {
                    const v4u scw = k.scale_words();
#pragma unroll
                    for (int gi = 0; gi < GROUPS; ++gi) {
                        v4i dacc = {0, 0, 0, 0};
#pragma unroll
                        for (int u = 0; u < PER_GROUP; ++u)
                            dacc = __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(a[gi * PER_GROUP + u]),
                                                                         static_cast<long>(k.values(gi * PER_GROUP + u)),
                                                                         dacc, 0, 0, 0);
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
                    for (int lr = 0; lr < NR; ++lr) {
                        const float da = AREG ? dareg[lr] : dalocal[lr];
                        acc[lr] += have ? (dw * da) * static_cast<float>(is[lr]) : 0.0f;
                    }
                }
                load(lq, buf[j]);
                advance(lq);
                if (it == iters - 1) {
                    // tile done: partial sums to LDS, then one wave adds them in wave order
                    float* pb = part + (tile_iter & 1) * (W * 64 * NR);
                    if constexpr (NR == 1) pb[wave * 64 + lane] = acc[0];
                    else if constexpr (NR == 2) *reinterpret_cast<float2*>(pb + (wave * 64 + lane) * 2) = make_float2(acc[0], acc[1]);
                    else *reinterpret_cast<float4*>(pb + (wave * 64 + lane) * 4) = make_float4(acc[0], acc[1], acc[2], acc[3]);
#pragma unroll
                    for (int lr = 0; lr < NR; ++lr) acc[lr] = 0.0f;
                    // the LDS writes complete, then the barrier; a compiler memory
                    // barrier too, and no wait for the weight loads in flight
                    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                    if (wave == (tile_iter & (W - 1))) {
                        const int t = cq.t;
                        const bool c1 = t >= p.mb[0].tile_end, c2 = t >= p.mb[1].tile_end, c3 = t >= p.mb[2].tile_end;
                        float* out = c3 ? p.mb[3].out : c2 ? p.mb[2].out : c1 ? p.mb[1].out : p.mb[0].out;
                        const int ldo = c3 ? p.mb[3].ldo : c2 ? p.mb[2].ldo : c1 ? p.mb[1].ldo : p.mb[0].ldo;
                        const int rows = c3 ? p.mb[3].rows : c2 ? p.mb[2].rows : c1 ? p.mb[1].rows : p.mb[0].rows;
                        const int t0 = c3 ? p.mb[2].tile_end : c2 ? p.mb[1].tile_end : c1 ? p.mb[0].tile_end : 0;
                        const int row = (t - t0) * kTileRows + n;
#pragma unroll
                        for (int lr = 0; lr < NR; ++lr) {
                            float r = pb[lane * NR + lr];
#pragma unroll
                            for (int g = 1; g < W; ++g) r += pb[(g * 64 + lane) * NR + lr];
                            const int mo = NR * q + lr;
                            if (mo < m && row < rows)
                                reinterpret_cast<gfloats>(reinterpret_cast<uint64_t>(out))[mo * ldo + row] = r;
                        }
                    }
                    ++tile_iter;
                }
                advance(cq);
            }
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
    else if (MT == 4 && w == 16) launch_w<KIND, MT, FUSED, MT == 4 ? 16 : 8>(p, depth, grid, lds, stream);
    else launch_w<KIND, MT, FUSED, 8>(p, depth, grid, lds, stream);
}

template <int KIND, bool FUSED>
void launch_kind(int mt, const MfmaArgs& p, int w, int depth, dim3 grid, size_t lds, hipStream_t stream) {
    if (mt == 4) launch_mt<KIND, 4, FUSED>(p, w, depth, grid, lds, stream);
    else if (mt == 8) launch_mt<KIND, 8, FUSED>(p, w, depth, grid, lds, stream);
    else if constexpr (KIND == 4) launch_mt<KIND, 16, FUSED>(p, w, depth, grid, lds, stream);
}

}  // namespace

// LDS bytes of a launch: the activation blocks of mt rows and the double-buffered
// partial sums of w waves.
size_t gemv_mfma_lds(int mt, int nb, int w) {
    return ((static_cast<size_t>(nb) * mt * kPerRowBlock + 15) & ~size_t{15}) + 2 * static_cast<size_t>(w) * 64 * (mt / 4) * 4;
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
    const int depth = per_wg * ka.iters > 1 ? 2 : 1;
    const size_t lds = gemv_mfma_lds(mt, p.nb, w);
    const dim3 grid(static_cast<unsigned>(wgs));
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
