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
// Q8_K rows copied to LDS. Workgroups hold 16 waves and there is at most one
// per CU, so that quantisation is repeated at most once per CU.
//
// Work split: L lanes (1, 2, 4 or 8) share a super-block; lane p of the L
// takes 8/L of the 16-byte "units" of the block's 128 quant bytes (Q4_K:
// units p, p + L, ..; Q6_K: a contiguous run), plus the scale bytes every
// lane of the block reads. A wave therefore holds 64/L
// block slots; G slots share a weight row, and a row group of 64/(L*G) rows
// takes `iters` = ceil(nb/G) blocks per slot. Waves walk their row groups
// grid-stride with D blocks of loads in flight per lane. A block's integer
// sums are added over its L lanes with DPP moves before the f32 scaling, so
// every block contributes one f32 term; a row's G slot sums are added when the
// row group ends. Small launches use large L (short per-lane work, many lanes
// busy); large launches use L = 1, which spends the fewest instructions per
// block.
#include "gemv_lds.h"
#include "rocknpu_hip.h"

#include <algorithm>
#include <atomic>

namespace rk {
namespace {

// Integer sum over aligned groups of L lanes (L <= 8), in every lane of the group.
template <int L>
__device__ __forceinline__ int sum_lanes(int v) {
    // dpp0: the moves fold into v_add_u32_dpp (every lane reads a lane)
    if constexpr (L >= 2) v += static_cast<int>(dpp0<kDppXor1>(static_cast<unsigned>(v)));
    if constexpr (L >= 4) v += static_cast<int>(dpp0<kDppXor2>(static_cast<unsigned>(v)));
    if constexpr (L >= 8) v += static_cast<int>(dpp0<kDppMirror8>(static_cast<unsigned>(v)));
    return v;
}
// Sum over lane-index bits [lo, hi) of a value uniform over bits below lo.
__device__ __forceinline__ float sum_bits(float v, int lo, int hi) {
    if (lo <= 0 && hi > 0) v += __int_as_float(dpp<kDppXor1>(__float_as_int(v)));
    if (lo <= 1 && hi > 1) v += __int_as_float(dpp<kDppXor2>(__float_as_int(v)));
    if (lo <= 2 && hi > 2) v += __int_as_float(dpp<kDppMirror8>(__float_as_int(v)));
    if (lo <= 3 && hi > 3) v += __int_as_float(dpp<kDppMirror16>(__float_as_int(v)));
    if (lo <= 4 && hi > 4) v += __shfl_xor(v, 16);
    if (lo <= 5 && hi > 5) v += __shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// The bytes lane p of a block's L lanes loads.
template <int KIND, int L>
struct Piece;

// Q4_K (144 bytes): d|dmin, 12 packed scale bytes, 128 quant bytes. Unit u
// (16 quant bytes 32j + 16h ..) holds values 64j + 16h + t (low nibbles,
// sub-block 2j) and 64j + 32 + 16h + t (high nibbles, sub-block 2j + 1).
// Lane p of the L takes units p, p + L, ..., so each load instruction reads
// 16 L contiguous bytes of every block.
template <int L>
struct Piece<4, L> {
    static constexpr int NU = 8 / L;
    v4u h;
    v4u q[NU];
    __device__ __forceinline__ static int unit(int p, int u) { return p + L * u; }
    __device__ __forceinline__ void load(gbytes blk, int p) {
        h = reinterpret_cast<gv4u>(blk)[0];
#pragma unroll
        for (int u = 0; u < NU; ++u) q[u] = reinterpret_cast<gv4u>(blk)[1 + unit(p, u)];
    }
};

// Q6_K (210 bytes): ql[128], qh[64], 16 int8 scales, f16 d. Unit u (16 ql
// bytes at 16u, half h = u/4, quarter a = u/2 % 2, c = u % 2) with qh bytes
// 32h + 16c .. holds values 128h + 32a + 16c + t (low nibbles) and that + 64
// (high nibbles), of sub-blocks 8h + 2a + c and 8h + 2a + c + 4.
// Blocks are only 2-byte aligned. The pieces are loaded as 4-byte aligned
// words from the word boundary at or below the block (sh = 0 or 2 bytes
// lower), each run of 16-byte pieces with the word that follows it, and
// shifted into place when used; the last word (bytes 206..209: scales 14-15
// and d) serves the scales' shift and d. Every load stays inside the block.
typedef v4u v4u_a4 __attribute__((aligned(4)));
typedef const __attribute__((address_space(1))) v4u_a4* gv4u_a4;
typedef uint32_t u32_a2 __attribute__((aligned(2)));

// Bytes sh.. of the 16-byte run v followed by word nx (sh = 0 or 2).
__device__ __forceinline__ v4u shift_run(const v4u& v, uint32_t nx, uint32_t sh) {
    return v4u{__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh),
               __builtin_amdgcn_alignbyte(v.w, v.z, sh), __builtin_amdgcn_alignbyte(nx, v.w, sh)};
}

template <int L>
struct Piece<6, L> {
    static constexpr int NU = 8 / L;
    static constexpr int NH = L == 1 ? 4 : (L == 8 ? 1 : 2);  // qh pieces of the lane's units
    v4u ql[NU];
    uint32_t ql_next;
    v4u qh[NH];
    uint32_t qh_next;
    v4u sc;
    uint32_t tail;  // bytes 206..209
    uint32_t sh;
    // first qh piece (index 2h + c) of lane p
    __device__ __forceinline__ static int qh_first(int p) {
        if constexpr (L == 1) return 0;
        else if constexpr (L == 2) return 2 * p;
        else if constexpr (L == 4) return 2 * (p >> 1);
        else return 2 * (p >> 2) + (p & 1);
    }
    __device__ __forceinline__ void load(gbytes blk, int p) {
        sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(blk)) & 2u;
        const gbytes b4 = blk - sh;
        typedef const __attribute__((address_space(1))) uint32_t* gu32;
#pragma unroll
        for (int u = 0; u < NU; ++u) ql[u] = reinterpret_cast<gv4u_a4>(b4)[NU * p + u];
        ql_next = reinterpret_cast<gu32>(b4 + 16 * (NU * p + NU))[0];
#pragma unroll
        for (int i = 0; i < NH; ++i) qh[i] = reinterpret_cast<gv4u_a4>(b4 + 128)[qh_first(p) + i];
        qh_next = reinterpret_cast<gu32>(b4 + 128 + 16 * (qh_first(p) + NH))[0];
        sc = reinterpret_cast<gv4u_a4>(b4 + 192)[0];
        tail = *reinterpret_cast<const __attribute__((address_space(1))) u32_a2*>(blk + 206);
    }
    __device__ __forceinline__ v4u get_ql(int u) const { return shift_run(ql[u], u + 1 < NU ? ql[u + 1].x : ql_next, sh); }
    __device__ __forceinline__ v4u get_qh(int i) const { return shift_run(qh[i], i + 1 < NH ? qh[i + 1].x : qh_next, sh); }
    __device__ __forceinline__ v4u get_sc() const { return shift_run(sc, tail, sh); }
};

// Sub-block scale/min pairs (2j, 2j+1) of a Q4_K block (ggml get_scale_min_k4).
__device__ __forceinline__ void q4_scales(const v4u& h, int j, int& sc0, int& sc1, int& mn0, int& mn1) {
    const int sh = 16 * (j & 1);
    const uint32_t y = h.y >> sh, z = h.z >> sh, w = h.w >> sh;
    const uint32_t scp = j < 2 ? (y & 0x3F3Fu) : ((w & 0x0F0Fu) | ((y >> 2) & 0x3030u));
    const uint32_t mnp = j < 2 ? (z & 0x3F3Fu) : (((w >> 4) & 0x0F0Fu) | ((z >> 2) & 0x3030u));
    sc0 = scp & 0xFF;
    sc1 = scp >> 8;
    mn0 = mnp & 0xFF;
    mn1 = mnp >> 8;
}

__device__ __forceinline__ int sbyte(const v4u& v, int i) {
    const uint32_t w = i < 8 ? (i < 4 ? v.x : v.y) : (i < 12 ? v.z : v.w);
    return static_cast<int8_t>((w >> (8 * (i & 3))) & 0xFF);
}

// This lane's share of the exact integer sums of block b against the
// activation rows [0, m): is[mi], ms[mi].
template <int L, int MT>
__device__ __forceinline__ void lane_sums(const Piece<4, L>& k, int p, const Q8Lds& a, int nb, int b, int m,
                                          int (&is)[MT], int (&ms)[MT]) {
    constexpr int NU = Piece<4, L>::NU;
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) { is[mi] = 0; ms[mi] = 0; }
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int gu = Piece<4, L>::unit(p, u);
        const int j = gu >> 1, hh = gu & 1;
        int sc0, sc1, mn0, mn1;
        q4_scales(k.h, j, sc0, sc1, mn0, mn1);
        const uint32_t q[4] = {k.q[u].x, k.q[u].y, k.q[u].z, k.q[u].w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            lo[t] = q[t] & 0x0F0F0F0Fu;
            hi[t] = (q[t] >> 4) & 0x0F0F0F0Fu;
        }
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
            if (mi >= m) break;
            // LDS addresses in 32 bits (full-rate 24-bit index products)
            const uint32_t blk = static_cast<uint32_t>(mi * nb + b);
            const uint32_t xq = a.qs_lds() + __umul24(blk, kGemvLdsQsStride) + 64 * j + 16 * hh;
            const v4u x0 = *lds_at<v4u>(xq);
            const v4u x1 = *lds_at<v4u>(xq + 32);
            int d0 = dot4(lo[0], x0.x, 0);
            d0 = dot4(lo[1], x0.y, d0);
            d0 = dot4(lo[2], x0.z, d0);
            d0 = dot4(lo[3], x0.w, d0);
            int d1 = dot4(hi[0], x1.x, 0);
            d1 = dot4(hi[1], x1.y, d1);
            d1 = dot4(hi[2], x1.z, d1);
            d1 = dot4(hi[3], x1.w, d1);
            const auto* bs = lds_at<int16_t>(a.bs_lds() + __umul24(blk, kGemvLdsBsStride));
            // |d| <= 16 * 15 * 128 and sc, mn < 64: the 24-bit products are exact
            is[mi] += __mul24(sc0, d0) + __mul24(sc1, d1);
            ms[mi] += __mul24(mn0, bs[4 * j + hh]) + __mul24(mn1, bs[4 * j + 2 + hh]);
        }
    }
}

// Q6_K quants are q - 32 with q = 0..63; bsums hold the sums of the 16
// activation quants of each sub-block, so sum (q-32)*x = sum q*x - 32*bsum.
// One unit (gu: half h, quarter qa, column c) of block b: 16 ql bytes, the
// matching 16 qh bytes and the scales of its two sub-blocks s0 and s0 + 4.
// qs0, bs0: LDS addresses of the quants and bsums of block b of activation
// row 0 (row mi is mi * nb blocks further).
template <int MT>
__device__ __forceinline__ void q6_unit(const v4u& qlv, const v4u& qhv, int sc0, int sc1, int gu, uint32_t qs0,
                                        uint32_t bs0, int nb, int m, int (&is)[MT]) {
    const int h = gu >> 2, qa = (gu >> 1) & 1, c = gu & 1;
    const int s0 = 8 * h + 2 * qa + c;
    const uint32_t ql[4] = {qlv.x, qlv.y, qlv.z, qlv.w};
    const uint32_t qh[4] = {qhv.x, qhv.y, qhv.z, qhv.w};
    const int sh = 2 * qa;
    // q = low nibble | 2 qh bits << 4. The qh bits of value byte k sit at bits
    // sh, sh + 1 (low nibbles) and sh + 4, sh + 5 (high nibbles) of qh byte k,
    // so one shift and one mask per nibble place them (sh <= 2: no bit
    // crosses a byte).
    uint32_t u0[4], u1[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        u0[t] = (ql[t] & 0x0F0F0F0Fu) | ((qh[t] << (4 - sh)) & 0x30303030u);
        u1[t] = ((ql[t] >> 4) & 0x0F0F0F0Fu) | ((qh[t] >> sh) & 0x30303030u);
    }
    // LDS addressing in 32 bits
    const uint32_t qs = qs0 + 128 * h + 32 * qa + 16 * c;
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
        if (mi >= m) break;
        const uint32_t xq = qs + mi * nb * kGemvLdsQsStride;
        const v4u x0 = *lds_at<v4u>(xq);
        const v4u x1 = *lds_at<v4u>(xq + 64);
        int d0 = dot4(u0[0], x0.x, 0);
        d0 = dot4(u0[1], x0.y, d0);
        d0 = dot4(u0[2], x0.z, d0);
        d0 = dot4(u0[3], x0.w, d0);
        int d1 = dot4(u1[0], x1.x, 0);
        d1 = dot4(u1[1], x1.y, d1);
        d1 = dot4(u1[2], x1.z, d1);
        d1 = dot4(u1[3], x1.w, d1);
        const auto* bs = lds_at<int16_t>(bs0 + mi * nb * kGemvLdsBsStride);
        // |d - 32 bsum| <= 16 * 63 * 128 + 32 * 2048 < 2^23 and |sc| <= 128: the
        // 24-bit products are exact
        is[mi] += __mul24(sc0, d0 - 32 * bs[s0]) + __mul24(sc1, d1 - 32 * bs[s0 + 4]);
    }
}

template <int L, int MT>
__device__ __forceinline__ void lane_sums(const Piece<6, L>& k, int p, const Q8Lds& a, int nb, int b, int m,
                                          int (&is)[MT], int (&ms)[MT]) {
    constexpr int NU = Piece<6, L>::NU;
    const v4u scv = k.get_sc();
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) { is[mi] = 0; ms[mi] = 0; }
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int gu = NU * p + u;
        const int h = gu >> 2, qa = (gu >> 1) & 1, c = gu & 1;
        const int hq = L == 1 ? 2 * h + c : (L == 8 ? 0 : c);
        const int s0 = 8 * h + 2 * qa + c;
        q6_unit<MT>(k.get_ql(u), k.get_qh(hq), sbyte(scv, s0), sbyte(scv, s0 + 4), gu,
                    a.qs_lds() + __umul24(static_cast<uint32_t>(b), kGemvLdsQsStride),
                    a.bs_lds() + __umul24(static_cast<uint32_t>(b), kGemvLdsBsStride), nb, m, is);
    }
}

// A Q6_K block as the stream kernel stages it in LDS, from a 16-byte-aligned
// address: 14 pieces of 16 bytes, pieces 0..12 = block bytes 0..207 in place,
// piece 13 = bytes 194..209 (so d, bytes 208..209, sits at +222). Lane p of
// the block's 8 takes unit p: ql bytes 16p.., the qh piece 2(p/4) + p%2, the
// scales of sub-blocks s0 = 8(p/4) + 2(p/2 % 2) + p%2 and s0 + 4.
constexpr int kQ6Pieces = 14;
constexpr int kQ6LdsBlock = kQ6Pieces * 16;
struct Piece6Lds {
    v4u ql, qh;
    int sc0, sc1;
    uint32_t tail;  // d in the upper half, as Piece<6, L>::tail
    __device__ __forceinline__ void load(const uint8_t* blk, int p) {
        const int s0 = 8 * (p >> 2) + 2 * ((p >> 1) & 1) + (p & 1);
        ql = *reinterpret_cast<const v4u*>(blk + 16 * p);
        qh = *reinterpret_cast<const v4u*>(blk + 128 + 16 * (2 * (p >> 2) + (p & 1)));
        sc0 = static_cast<int8_t>(blk[192 + s0]);
        sc1 = static_cast<int8_t>(blk[196 + s0]);
        tail = static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(blk + 222)) << 16;
    }
};



template <int L>
__device__ __forceinline__ void block_scales(const Piece<4, L>& k, float& d, float& dmin) {
    d = f16_bits_to_f32(static_cast<uint16_t>(k.h.x & 0xFFFF));
    dmin = f16_bits_to_f32(static_cast<uint16_t>(k.h.x >> 16));
}
template <int L>
__device__ __forceinline__ void block_scales(const Piece<6, L>& k, float& d, float& dmin) {
    d = f16_bits_to_f32(static_cast<uint16_t>(k.tail >> 16));
    dmin = 0.0f;
}
__device__ __forceinline__ void block_scales(const Piece6Lds& k, float& d, float& dmin) {
    d = f16_bits_to_f32(static_cast<uint16_t>(k.tail >> 16));
    dmin = 0.0f;
}

// A slot's block: row group `gi`, iteration `it` inside the group.
struct Pos {
    int gi;
    int it;
};

// Kernel arguments, derived on the host from GemvParams: 32-bit counts and
// per-member row-group totals, so the kernel's set-up is one round of scalar
// loads and a few selects, with no 64-bit division.
struct GemvMember {
    const uint8_t* w;
    float* out;
    int ldo;
    int rows;
    int groups;  // row groups of this member
    int wg_end;  // cumulative workgroup count
};
struct GemvArgs {
    GemvMember mb[kGemvMaxMembers];
    const float* x;      // fused: f32 activations, ldx floats apart
    const uint8_t* q8k;  // else: Q8_K rows, ldx bytes apart
    int32_t* isum;
    int32_t* msum;
    int ldx;
    int m;
    int nb;
    int log2g;
    int iters;
    int* stall;       // fused: set to 1 (pinned host memory) by a wave whose wait gives up
    int spin_limit;   // fused: polls of the wait for the quantising waves
    int ready_extra;  // fused: arrivals waited for beyond the quantising waves (0; 1 tests the give-up)
    int wave_major;   // row groups dealt to waves across the workgroups first (else workgroup by workgroup)
};

// The fields of GemvArgs that a launch's first loads need, passed ahead of it
// as scalar kernel arguments (14 dwords, preloaded in SGPRs; the struct itself
// is read from the argument segment, a memory round trip at the start of
// every wave): the activations (f32 or Q8_K), the first three members'
// weights and rows, and the counts packed. A launch with a fourth member is
// split on the host, so a workgroup's member is one of three.
struct LaneHead {
    const void* x;
    const uint8_t* w0;
    const uint8_t* w1;
    const uint8_t* w2;
    int rows0, rows1, rows2;
    int wg_ends;  // the members' workgroup ends, 10 bits each: e0 | e1 << 10 | e2 << 20
    int counts;   // nb | iters << 10 | m << 20 | log2g << 24 | wave_major << 27
    int ldx;
};
#define RK_LANE_HEAD(h) h.x, h.w0, h.w1, h.w2, h.rows0, h.rows1, h.rows2, h.wg_ends, h.counts, h.ldx
// The workgroup's member on the device: its weights, rows and workgroup
// range [wg0, wg1), and (by the same selects) which member it is.
struct LaneMember {
    const uint8_t* w;
    int rows, wg0, wg1;
    bool c1, c2;
};
__device__ __forceinline__ LaneMember lane_member(int wg, const uint8_t* w0, const uint8_t* w1, const uint8_t* w2,
                                                  int rows0, int rows1, int rows2, int wg_ends) {
    const int e0 = wg_ends & 0x3ff, e1 = (wg_ends >> 10) & 0x3ff, e2 = (wg_ends >> 20) & 0x3ff;
    const bool c1 = wg >= e0, c2 = wg >= e1;
    return LaneMember{c2 ? w2 : c1 ? w1 : w0, c2 ? rows2 : c1 ? rows1 : rows0, c2 ? e1 : c1 ? e0 : 0,
                      c2 ? e2 : c1 ? e1 : e0, c1, c2};
}
// The preloaded arguments of a launch (LaneHead), and whether its fields fit
// their packed slots: at most three members (launch_gemv splits a fourth off,
// so member 3 repeats member 2) and 1023 workgroups, rows of at most 1023
// blocks (the LDS holds far fewer), up to 15 activation rows.
LaneHead lane_head(const GemvArgs& p, bool fused) {
    const auto u = [](int v) { return static_cast<uint32_t>(v); };
    return LaneHead{fused ? static_cast<const void*>(p.x) : static_cast<const void*>(p.q8k),
                    p.mb[0].w,
                    p.mb[1].w,
                    p.mb[2].w,
                    p.mb[0].rows,
                    p.mb[1].rows,
                    p.mb[2].rows,
                    static_cast<int>(u(p.mb[0].wg_end) | u(p.mb[1].wg_end) << 10 | u(p.mb[2].wg_end) << 20),
                    static_cast<int>(u(p.nb) | u(p.iters) << 10 | u(p.m) << 20 | u(p.log2g) << 24 |
                                     u(p.wave_major) << 27),
                    p.ldx};
}
bool lane_head_fits(const GemvArgs& p) {
    return p.mb[3].wg_end == p.mb[2].wg_end && p.mb[0].wg_end >= 0 && p.mb[2].wg_end <= 0x3ff && p.nb >= 0 &&
           p.nb <= 0x3ff && p.iters >= 0 && p.iters <= 0x3ff && p.m >= 0 && p.m <= 0xf && p.log2g >= 0 &&
           p.log2g <= 7 && (p.wave_major == 0 || p.wave_major == 1);
}

// The activations into LDS, after the first weight loads are issued. Fused
// launches: the quantising waves (whose activation loads went out first)
// quantise and count themselves in `ready`; every wave (owners too: each
// reads all blocks) waits for the count. Bounded for safety only: the owners
// depend on nothing but their own activation loads, so the count arrives. A
// wave that gives up reports it (host-visible flag) and gets true back, and
// writes NaN for its outputs. Otherwise the Q8_K rows are copied.
template <bool FUSED, int THREADS, int QP>
__device__ __forceinline__ bool stage_activations(const GemvArgs& p, const XPre<THREADS, QP>& xpre, bool quant_wave,
                                                  int quant_waves, const Q8Lds& a, int& ready) {
    // The barriers here publish LDS writes only (lgkmcnt(0), then s_barrier):
    // a fence would also wait for every direct global->LDS load in flight.
    if constexpr (FUSED) {
        if (threadIdx.x == 0) ready = 0;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (quant_wave) {
            xpre.quantize(p.x, p.ldx, p.m, p.nb, a);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(&ready, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        const int need = quant_waves + p.ready_extra;
        for (int spin = 0; spin < p.spin_limit; ++spin) {
            if (__hip_atomic_load(&ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= need) break;
            __builtin_amdgcn_s_sleep(1);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        const bool stalled = __hip_atomic_load(&ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < need;
        if (stalled && (threadIdx.x & 63) == 0) __hip_atomic_store(p.stall, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return stalled;
    } else {
        stage_q8k<THREADS>(p.q8k, p.ldx, p.m, p.nb, a);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        return false;
    }
}

// SUMS: also write every block's exact integer sums (p.isum / p.msum).
// QP: activation quantisation passes whose loads are issued up front.
template <int KIND, int L, int MT, bool FUSED, int D, bool SUMS, int W, int QP>
__global__ __launch_bounds__(W * 64) void gemv_kernel(const void* x, const uint8_t* w0, const uint8_t* w1,
                                                        const uint8_t* w2, int rows0, int rows1, int rows2, int wg_ends,
                                                        int counts, int ldx, const GemvArgs pa) {
    constexpr int BB = block_bytes(KIND);
    constexpr int SW = 64 / L;  // block slots per wave
    constexpr int LOG2L = L == 1 ? 0 : L == 2 ? 1 : L == 4 ? 2 : 3;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int q8_ready;  // waves done quantising the activations (fused launches)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: keeps row math scalar
    // p: the arguments, with the preloaded fields (LaneHead) in place of the
    // struct's copies; only its scalar fields are read
    GemvArgs p = pa;
    p.x = static_cast<const float*>(x);
    p.q8k = static_cast<const uint8_t*>(x);
    p.ldx = ldx;
    p.nb = counts & 0x3ff;
    p.iters = (counts >> 10) & 0x3ff;
    p.m = (counts >> 20) & 0xf;
    p.log2g = (counts >> 24) & 0x7;
    p.wave_major = (counts >> 27) & 1;
    const int nb = p.nb, m = p.m, iters = p.iters, log2g = p.log2g;
    const Q8Lds a = q8_lds(smem, MT, nb);

    // The projection this workgroup serves (wave-uniform), from the preloaded
    // fields; its output from the struct's (read at the first store).
    const int wg = blockIdx.x;
    const LaneMember mem = lane_member(wg, w0, w1, w2, rows0, rows1, rows2, wg_ends);
    const bool c1 = mem.c1, c2 = mem.c2;
    const int rows = mem.rows;
    // row groups: the host's ceil(rows / rows_per_group), a power of two
    const int groups = (rows + (SW >> log2g) - 1) >> (6 - LOG2L - log2g);
    const int wg0 = mem.wg0, wg1 = mem.wg1;
    const gbytes wg_w = reinterpret_cast<gbytes>(reinterpret_cast<uint64_t>(mem.w));

    const int sl = lane >> LOG2L, pc = lane & (L - 1);  // block slot, lane inside the block
    const int G = 1 << log2g;
    const int gl = sl & (G - 1);                         // slot inside the row
    const int rs = sl >> log2g;                          // row inside the row group
    const int rows_per_group = SW >> log2g;
    const int64_t row_bytes = static_cast<int64_t>(nb) * BB;
    // this wave's row groups: wave_gid, wave_gid + wave_stride, ... below `groups`
    // (gemv_wave_major chooses the order of the first ones)
    const int wave_gid = p.wave_major ? wave * (wg1 - wg0) + (wg - wg0) : (wg - wg0) * W + wave;
    const int wave_stride = (wg1 - wg0) * W;

    auto advance = [=](Pos& q) {
        if (++q.it == iters) { q.it = 0; q.gi += wave_stride; }
    };
    // With more than one block in flight, loads are issued unconditionally: a
    // slot without a block re-reads a block of the wave's first row group (in
    // bounds, cache-resident) and ignores it. Branch-free load sequences let
    // the wait-count pass wait for exactly the loads a value depends on.
    const int home_row = min(wave_gid * rows_per_group + rs, rows - 1);
    const int home_b = min(gl, nb - 1);
    auto load_block = [=](const Pos& q, Piece<KIND, L>& k) {
        int row = q.gi * rows_per_group + rs;
        int b = gl + q.it * G;
        if (!(q.gi < groups && row < rows && b < nb)) {
            row = home_row;
            b = home_b;
        }
        // row, b >= 0 and row_bytes < 2^32: one 32 x 32 -> 64-bit product
        k.load(wg_w + static_cast<uint64_t>(static_cast<uint32_t>(row)) * static_cast<uint32_t>(row_bytes) +
                   __umul24(static_cast<uint32_t>(b), static_cast<uint32_t>(BB)),
               pc);
    };

    // Issue order: the owners of quantisation blocks load their activations
    // first, then every wave loads its first D weight blocks, so the weights
    // are in flight during the set-up below, and an owner's wait for its
    // activations (an in-order count) does not include its weight loads.
    // One barrier then publishes the cleared q8_ready; the owners quantise
    // and count themselves in it; every wave waits for that count. Only the
    // owners' progress gates the rest, so no wave waits for another wave's
    // weight loads.
    const int quant_waves = FUSED ? min(W, (m * nb + 3) / 4) : 0;
    const bool quant_wave = wave < quant_waves;
    bool stalled = false;  // the wait below gave up
    XPre<W * 64, QP> xpre;
    if constexpr (FUSED) {
        if (quant_wave) xpre.issue(p.x, p.ldx, m, nb);
    }
    Piece<KIND, L> buf[D];
    Pos lq{wave_gid, 0};  // next block to load
#pragma unroll
    for (int j = 0; j < D; ++j) {
        load_block(lq, buf[j]);
        advance(lq);
    }
    // the member's output, read from the argument segment now, behind the
    // first loads, rather than at the first store
    MemberOuts mo;
    mo.fetch(pa);
    const float* out = c2 ? mo.o2 : c1 ? mo.o1 : mo.o0;
    const int ldo = c2 ? mo.l2 : c1 ? mo.l1 : mo.l0;
    // (held here: the compiler would otherwise sink the loads past the wait
    // below to the first store; here the wait below covers them)
    asm volatile("" ::"s"(out), "s"(ldo));
    const gfloats wg_out = reinterpret_cast<gfloats>(reinterpret_cast<uint64_t>(out));
    stalled = stage_activations<FUSED>(p, xpre, quant_wave, quant_waves, a, q8_ready);

    float acc[MT];
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[mi] = 0.0f;

    Pos cq{wave_gid, 0};  // block being multiplied
    while (cq.gi < groups) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const bool live = cq.gi < groups;  // uniform across the wave
            const int row = cq.gi * rows_per_group + rs;
            const int b = gl + cq.it * G;
            const bool have = row < rows && b < nb;  // uniform inside each block's L lanes
            if (live) {
                const int bk = have ? b : home_b;
                int is[MT], ms[MT];
                lane_sums<L, MT>(buf[j], pc, a, nb, bk, m, is, ms);
                float dw, dminw;
                block_scales<L>(buf[j], dw, dminw);
#pragma unroll
                for (int mi = 0; mi < MT; ++mi) {
                    if (mi >= m) break;
                    const int isum = sum_lanes<L>(is[mi]);
                    const int msum = KIND == 4 ? sum_lanes<L>(ms[mi]) : 0;
                    const float da = *lds_at<float>(a.d_lds() + 4 * __umul24(static_cast<uint32_t>(mi * nb + bk), 1u));
                    float term = (dw * da) * static_cast<float>(isum);
                    if constexpr (KIND == 4) term = term - (dminw * da) * static_cast<float>(msum);
                    acc[mi] += have ? term : 0.0f;
                    if constexpr (SUMS) {
                        if (have && pc == 0) {
                            const int64_t idx = (static_cast<int64_t>(mi) * rows + row) * nb + b;
                            p.isum[idx] = isum;
                            p.msum[idx] = msum;
                        }
                    }
                }
            }
            if (live && cq.it == iters - 1) {
                // row group done: add each row's G slot sums and store
#pragma unroll
                for (int mi = 0; mi < MT; ++mi) {
                    const float r = sum_bits(acc[mi], LOG2L, LOG2L + log2g);
                    if (gl == 0 && pc == 0 && row < rows && mi < m)
                        wg_out[mi * ldo + row] = stalled ? __builtin_nanf("") : r;
                    acc[mi] = 0.0f;
                }
            }
            // Refill this slot with the block D ahead, after the row's store (a
            // load issued first would queue ahead of it). With one block in
            // flight a load past the wave's last block is skipped (issued, the
            // wave's end waits for it); with more the loads stay unconditional.
            // TinyLlama o at one row 3.5 -> 3.4 us, qkv 3.58 -> 3.49, o at two
            // rows 4.1 -> 3.9, Llama-3-8B gate+up 14.5 -> 14.1.
            if (D > 1 || lq.gi < groups) load_block(lq, buf[j]);
            advance(lq);
            advance(cq);
        }
    }
}

// Q6_K stream kernel: the lane-per-block arithmetic at L = 8 lanes per block
// and G = 8 block slots per row (one row per row group), with the weights
// staged in LDS instead of loaded into registers. Q6_K blocks (210 bytes) are
// only 2-byte aligned; loaded per lane they cost several partial-line
// requests per 16 bytes, and the L1 request rate then bounds the launch.
// Here a stream wave moves each step (one row's 8 blocks of one iteration:
// 1680 contiguous bytes) with two direct global->LDS loads of 16-byte pieces,
// each piece read from its 2-byte-aligned place in the block and written to a
// 16-byte-aligned LDS place (Piece6Lds), into a private ring of S step slots
// kept S steps ahead. Per block the arithmetic and the order of the f32 sums
// are those of gemv_kernel, so results are bit-identical to it.
//
// A workgroup has 16 waves; waves [0, WS) stream rows (WS = 8 or 16). Every
// wave first loads its share of the activations (all passes at once), waits
// for them, then issues its first S steps and quantises from registers (or
// copies Q8_K rows, then issues), counts itself in `ready` and waits for all
// 16. Activation loads thus reach the memory system before any weight load,
// and no wave has both in flight (the compiler's wait counts would otherwise
// wait for all of them before quantising).
constexpr int kQ6StepBytes = 8 * kQ6KBytes;      // one step: 8 blocks of a row
constexpr int kQ6SlotBytes = 8 * kQ6LdsBlock;    // a ring slot: 112 pieces of 16 bytes
constexpr int kQ6StreamMaxBlocks = 64;           // blocks per row
constexpr int kQ6Waves = 16;                     // waves per workgroup
constexpr int kQ6MaxLds = 160 * 1024;

// A direct global->LDS load of 16 bytes per lane (to lds + 16 * lane) that the
// wait-count pass does not see (inline asm): seen, every later LDS read of
// the wave would wait for all such loads in flight. The caller waits for it
// explicitly (wait_vm) before reading its bytes and before the wave ends.
// The source is base (wave-uniform) + off (this lane's 32-bit offset).
__device__ __forceinline__ void dma16_untracked(const uint8_t* base, uint32_t off, uint8_t* lds_dst) {
    const uint32_t lds = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)(lds_dst)));
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds) : "memory");
}

// LDS: the activations of m rows (m * nb * kGemvLdsPerBlock bytes, rounded up
// to 16), then S ring slots of WS waves.
template <int MT, int WS, int S, bool FUSED, int QP>
__global__ __launch_bounds__(kQ6Waves * 64) void gemv_q6_stream_kernel(const void* x, const uint8_t* w0,
                                                                       const uint8_t* w1, const uint8_t* w2,
                                                                       int rows0, int rows1, int rows2, int wg_ends,
                                                                       int counts, int ldx, const GemvArgs pa) {
    static_assert(WS == 8 || WS == 16, "8 or 16 stream waves");
    static_assert(S == 2 || S == 4, "2 or 4 ring slots");
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int ready;  // waves done staging their share of the activations
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // p: the arguments, with the preloaded fields (LaneHead) in place of the
    // struct's copies; only its scalar fields are read
    GemvArgs p = pa;
    p.x = static_cast<const float*>(x);
    p.q8k = static_cast<const uint8_t*>(x);
    p.ldx = ldx;
    p.nb = counts & 0x3ff;
    p.iters = (counts >> 10) & 0x3ff;
    p.m = (counts >> 20) & 0xf;
    const int nb = p.nb, m = p.m, iters = p.iters;
    const Q8Lds a = q8_lds(smem, m, nb);
    uint8_t* const ring_base = smem + (m * nb * kGemvLdsPerBlock + 15) / 16 * 16;

    XPre<kQ6Waves * 64, QP> xpre;
    if constexpr (FUSED) xpre.issue(p.x, p.ldx, m, nb);
    if (threadIdx.x == 0) ready = 0;
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    const int wg = blockIdx.x;
    const LaneMember mem = lane_member(wg, w0, w1, w2, rows0, rows1, rows2, wg_ends);
    const bool c1 = mem.c1, c2 = mem.c2;
    float* out = c2 ? pa.mb[2].out : c1 ? pa.mb[1].out : pa.mb[0].out;
    const int ldo = c2 ? pa.mb[2].ldo : c1 ? pa.mb[1].ldo : pa.mb[0].ldo;
    const int rows = mem.rows;
    const int wg0 = mem.wg0, wg1 = mem.wg1;
    const gbytes wg_w = reinterpret_cast<gbytes>(reinterpret_cast<uint64_t>(mem.w));
    const gfloats wg_out = reinterpret_cast<gfloats>(reinterpret_cast<uint64_t>(out));

    const int sl = lane >> 3, pc = lane & 7;  // block slot (block of the step), lane inside the block
    const int64_t row_bytes = static_cast<int64_t>(nb) * kQ6KBytes;
    // this wave's rows: wave_gid, wave_gid + wave_stride, ... below `rows`
    // (none for waves WS and up)
    const bool streams = wave < WS;
    const int wave_gid = streams ? (wg - wg0) * WS + wave : rows;
    const int wave_stride = (wg1 - wg0) * WS;
    auto advance = [=](Pos& q) {
        if (++q.it == iters) { q.it = 0; q.gi += wave_stride; }
    };
    auto slot = [&](int u) { return ring_base + (u * WS + wave) * kQ6SlotBytes; };

    // The pieces this lane loads in every step: pieces lane and 64 + lane
    // (the second for lanes below 48) of the step's 8 x 14: block pb, byte po
    // of the block, byte so = 210 pb + po of the step.
    int pb[2], po[2], so[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = min(64 * i + lane, 8 * kQ6Pieces - 1);
        pb[i] = q / kQ6Pieces;
        const int g = q - kQ6Pieces * pb[i];
        po[i] = (g < kQ6Pieces - 1 ? 16 * g : kQ6KBytes - 16);
        so[i] = pb[i] * kQ6KBytes + po[i];
    }
    // Issue step q (one of the wave's, q.gi < rows) into ring slot u: two
    // loads from the row's start plus 32-bit offsets. In a row's last step,
    // blocks past the row's end load the same piece of the row's block 0 (in
    // bounds, never read).
    auto issue = [&](const Pos& q, int u) {
        const uint8_t* row_start =
            reinterpret_cast<const uint8_t*>(reinterpret_cast<uint64_t>(wg_w + static_cast<int64_t>(q.gi) * row_bytes));
        const int step0 = q.it * kQ6StepBytes;
        uint32_t off[2];
        if (q.it * 8 + 8 <= nb) {
#pragma unroll
            for (int i = 0; i < 2; ++i) off[i] = static_cast<uint32_t>(step0 + so[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 2; ++i) off[i] = static_cast<uint32_t>(q.it * 8 + pb[i] < nb ? step0 + so[i] : po[i]);
        }
        uint8_t* dst = slot(u);
        dma16_untracked(row_start, off[0], dst);
        if (lane < 8 * kQ6Pieces - 64) dma16_untracked(row_start, off[1], dst + 1024);
    };
    // Only the wave's own steps are loaded, so nothing is left in flight at
    // its end. `ahead`: steps loaded after the current one.
    Pos lq{wave_gid, 0};  // next step to load
    int ahead = -1;
    auto fill = [&](int u0, int u1) {
        for (int u = u0; u < u1; ++u)
            if (lq.gi < rows) {
                issue(lq, u);
                advance(lq);
                ++ahead;
            }
    };

    // The first step goes out before the quantisation and the rest after:
    // issuing all S first stalls the waves at a full memory pipeline before
    // they quantise (TinyLlama down, 2048 x 5632: 6.2 -> 5.7 us at one row,
    // 8.65 -> 8.15 at four).
    // A wave counts itself in before issuing the rest of its ring: the issue
    // can wait for room in the memory pipeline.
    if constexpr (FUSED) {
        // the activation loads have landed (an explicit wait: the quantisation
        // below then waits for nothing, and the direct loads are not waited for)
        wait_vm<0>();
        fill(0, 1);
        xpre.quantize(p.x, p.ldx, m, nb, a);
    } else {
        stage_q8k<kQ6Waves * 64>(p.q8k, p.ldx, m, nb, a);
        fill(0, 1);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) __hip_atomic_fetch_add(&ready, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (!streams) return;
    fill(1, S);

    // Wait for every wave's share. Bounded for safety only: each depends on
    // nothing but its own activation loads, so the count arrives. A wave that
    // gives up reports it (host-visible flag) and writes NaN for its outputs.
    const int need = kQ6Waves + p.ready_extra;
    for (int spin = 0; spin < p.spin_limit; ++spin) {
        if (__hip_atomic_load(&ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= need) break;
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const bool stalled = __hip_atomic_load(&ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < need;
    if (stalled && lane == 0) __hip_atomic_store(p.stall, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);

    float acc[MT];
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[mi] = 0.0f;
    // this lane's activation addresses for block slot sl of row 0 (the steps
    // add uniform offsets)
    const uint32_t lane_qs = a.qs_lds() + sl * kGemvLdsQsStride;
    const uint32_t lane_bs = a.bs_lds() + sl * kGemvLdsBsStride;
    const uint32_t lane_d = a.d_lds() + 4 * sl;
    Pos cq{wave_gid, 0};  // step being multiplied
    for (int u = 0; cq.gi < rows; u = u + 1 == S ? 0 : u + 1) {
        // this step's two loads have landed: at most 2 * ahead loads younger
        // than them are in flight (row-end stores only add to the count)
        switch (ahead) {
        case 3: wait_vm<6>(); break;
        case 2: wait_vm<4>(); break;
        case 1: wait_vm<2>(); break;
        default: wait_vm<0>(); break;
        }
        asm volatile("" ::: "memory");
        Piece6Lds k;
        k.load(slot(u) + sl * kQ6LdsBlock, pc);
        const int row = cq.gi;
        // Lanes past the row's end (b < nb + 8) read activation bytes past
        // their row: still inside the workgroup's LDS (the ring follows the
        // activations), and their term is dropped by a select.
        const int b = sl + cq.it * 8;
        const bool have = b < nb;
        int is[MT];
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) is[mi] = 0;
        const int b0 = cq.it * 8;  // uniform part of b
        q6_unit<MT>(k.ql, k.qh, k.sc0, k.sc1, pc, lane_qs + b0 * kGemvLdsQsStride, lane_bs + b0 * kGemvLdsBsStride,
                    nb, m, is);
        float dw, dminw;
        block_scales(k, dw, dminw);
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
            if (mi >= m) break;
            const int isum = sum_lanes<8>(is[mi]);
            const float da = *lds_at<float>(lane_d + 4 * (mi * nb + b0));
            const float term = (dw * da) * static_cast<float>(isum);
            acc[mi] += have ? term : 0.0f;
        }
        if (cq.it == iters - 1) {
            // row done: add its 8 slot sums and store
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) {
                const float r = sum_bits(acc[mi], 3, 6);
                if (lane == 0 && mi < m) wg_out[mi * ldo + row] = stalled ? __builtin_nanf("") : r;
                acc[mi] = 0.0f;
            }
        }
        // the slot's LDS reads are done before its refill is issued
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lq.gi < rows) {
            issue(lq, u);
            advance(lq);
        } else {
            --ahead;
        }
        advance(cq);
    }
    // every load has landed (and been read) before the wave ends
    wait_vm<0>();
}

// Most blocks in flight per lane, by kind and lanes per block: 64-150 bytes
// of weights per lane, within the 128 VGPRs a 1024-thread workgroup allows
// (halved for eight activation rows).
template <int KIND, int L>
constexpr int max_depth() {
    if constexpr (KIND == 4) return L <= 2 ? 2 : 4;
    else return L == 1 ? 1 : L == 8 ? 4 : 2;
}

template <int KIND, int L, int MT, bool FUSED, bool SUMS, int W, int QP>
void launch_d(const GemvArgs& p, int d, dim3 grid, size_t lds, hipStream_t stream) {
    // eight activation rows, and Q6_K at four rows and L = 2 within 128
    // VGPRs, hold half the blocks in flight
    constexpr bool HALF = MT == 8 || (MT == 4 && KIND == 6 && L == 2 && W == 16);
    constexpr int DM = SUMS ? 1 : (HALF ? (max_depth<KIND, L>() > 1 ? max_depth<KIND, L>() / 2 : 1)
                                        : max_depth<KIND, L>());
    const dim3 block(W * 64);
    const LaneHead h = lane_head(p, FUSED);
    if (DM >= 2 && d >= 2)
        gemv_kernel<KIND, L, MT, FUSED, (DM >= 2 ? 2 : 1), SUMS, W, QP><<<grid, block, lds, stream>>>(RK_LANE_HEAD(h), p);
    else gemv_kernel<KIND, L, MT, FUSED, 1, SUMS, W, QP><<<grid, block, lds, stream>>>(RK_LANE_HEAD(h), p);
}

// Activation passes loaded up front: all of them (up to 4) in 8-wave
// workgroups that quantise more than one pass (their VGPR budget holds
// them), else the first.
template <int KIND, int L, int MT, bool FUSED, bool SUMS, int W>
void launch_mt(const GemvArgs& p, int d, int passes, dim3 grid, size_t lds, hipStream_t stream) {
    if constexpr (FUSED && W == 8) {
        if (passes > 1) return launch_d<KIND, L, MT, FUSED, SUMS, W, 4>(p, d, grid, lds, stream);
    }
    launch_d<KIND, L, MT, FUSED, SUMS, W, 1>(p, d, grid, lds, stream);
}

template <int KIND, int L, bool FUSED, bool SUMS, int W>
void launch_w(const GemvArgs& p, int mt, int d, int passes, dim3 grid, size_t lds, hipStream_t stream) {
    switch (mt) {
    case 1: launch_mt<KIND, L, 1, FUSED, SUMS, W>(p, d, passes, grid, lds, stream); break;
    case 2: launch_mt<KIND, L, 2, FUSED, SUMS, W>(p, d, passes, grid, lds, stream); break;
    case 4: launch_mt<KIND, L, 4, FUSED, SUMS, W>(p, d, passes, grid, lds, stream); break;
    default:
        // eight rows run with L <= 2 only (more lanes per block would spill)
        if constexpr (L <= 2) launch_mt<KIND, L, 8, FUSED, SUMS, W>(p, d, passes, grid, lds, stream);
        break;
    }
}

// 8-wave workgroups serve fused launches only.
template <int KIND, int L, bool FUSED, bool SUMS>
void launch_l(const GemvArgs& p, int w, int mt, int d, int passes, dim3 grid, size_t lds, hipStream_t stream) {
    if constexpr (FUSED && !SUMS) {
        if (w == 8) return launch_w<KIND, L, FUSED, SUMS, 8>(p, mt, d, passes, grid, lds, stream);
    }
    launch_w<KIND, L, FUSED, SUMS, 16>(p, mt, d, passes, grid, lds, stream);
}

}  // namespace

// Slots per row: the largest power of two <= min(slots, nb) whose last pass
// over the row's blocks keeps at least 85% of the slots busy.
int slots_per_row_log2(int nb, int slots) {
    int lg = 0;
    while ((2 << lg) <= slots && (2 << lg) <= nb) ++lg;
    while (lg > 0) {
        const int g = 1 << lg, it = (nb + g - 1) / g;
        if (nb * 100 >= 85 * g * it) break;
        --lg;
    }
    return lg;
}

namespace {

// The stall flag of fused launches: one int of pinned host memory, allocated
// by the first fused launch and kept until the process ends.
std::atomic<int*> g_stall_flag{nullptr};
std::atomic<int> g_test_stall_spins{0};

int* stall_flag() {
    static int* const flag = [] {
        void* mem = nullptr;
        if (hipHostMalloc(&mem, 64, hipHostMallocDefault) != hipSuccess) return static_cast<int*>(nullptr);
        int* f = static_cast<int*>(mem);
        __atomic_store_n(f, 0, __ATOMIC_SEQ_CST);
        g_stall_flag.store(f);
        return f;
    }();
    return flag;
}

// The bounded wait for the activations: the stall flag, the polls allowed,
// and the extra arrivals a test of the give-up asks for.
int set_wait(GemvArgs& ka) {
    ka.stall = stall_flag();
    if (ka.stall == nullptr) return kStatusExec;
    const int test_spins = g_test_stall_spins.load(std::memory_order_relaxed);
    ka.spin_limit = test_spins > 0 ? test_spins : 1 << 24;
    ka.ready_extra = test_spins > 0 ? 1 : 0;
    return kStatusOk;
}

// Kernel arguments for W-wave workgroups and row groups of rows_per_group
// rows: at most one workgroup per CU and one per W row groups, split between
// the projections in proportion to their row groups. Sets wgs and per_wave
// (the most row groups a wave gets, times p.iters).
// Whether `groups` row groups dealt to n workgroups of W waves go wave by
// wave across the workgroups (group g to wave g / n of workgroup g % n) rather
// than workgroup by workgroup (to wave g % W of workgroup g / W); later rounds
// repeat the first. Workgroup 0 gets the most groups either way; wave-major
// is chosen when it gets fewer so. TinyLlama gate+up at one row (2 x 2816
// groups of two rows, 128 workgroups of 16 waves each): 32 row groups on 48
// CUs and 16 on the rest workgroup by workgroup, 22 on every CU wave by wave;
// 5.6 -> 5.25 us (at two rows 6.9 -> 6.25 us).
bool gemv_wave_major(int64_t groups, int64_t n, int W) {
    const int64_t stride = n * W;
    int64_t by_wg = 0, by_wave = 0;
    for (int j = 0; j < W; ++j) {
        by_wg += std::max<int64_t>(0, (groups - j + stride - 1) / stride);
        by_wave += std::max<int64_t>(0, (groups - j * n + stride - 1) / stride);
    }
    return by_wave < by_wg;
}

template <bool FUSED>
int plan_args(const GemvParams& p, int W, int64_t rows_per_group, int cus, GemvArgs& ka, int64_t& wgs,
              int64_t& per_wave) {
    int64_t total_groups = 0;
    for (int i = 0; i < p.count; ++i) total_groups += (p.rows[i] + rows_per_group - 1) / rows_per_group;
    const int64_t budget = std::max<int64_t>(p.count, std::min<int64_t>(cus, (total_groups + W - 1) / W));
    ka = GemvArgs{};
    wgs = 0;
    per_wave = 1;
    for (int i = 0; i < p.count; ++i) {
        const int64_t groups = (p.rows[i] + rows_per_group - 1) / rows_per_group;
        int64_t n = (budget * groups + total_groups / 2) / total_groups;
        n = std::max<int64_t>(1, std::min(n, (groups + W - 1) / W));
        wgs += n;
        per_wave = std::max(per_wave, (groups + n * W - 1) / (n * W) * p.iters);
        // the kernel's row, output and group arithmetic is 32-bit
        if (p.rows[i] > INT32_MAX / 2 || p.ldo[i] > INT32_MAX || p.ldo[i] * (p.m - 1) + p.rows[i] > INT32_MAX)
            return kStatusInvalid;
        ka.mb[i] = GemvMember{p.w[i], p.out[i], static_cast<int>(p.ldo[i]), static_cast<int>(p.rows[i]),
                              static_cast<int>(groups), static_cast<int>(wgs)};
        if (gemv_wave_major(groups, n, W)) ka.wave_major = 1;
    }
    if (p.ldx > INT32_MAX / 8 || wgs * W > INT32_MAX / 2) return kStatusInvalid;
    for (int i = p.count; i < kGemvMaxMembers; ++i) ka.mb[i] = ka.mb[p.count - 1];
    ka.x = p.x;
    ka.q8k = p.q8k;
    ka.isum = p.isum;
    ka.msum = p.msum;
    ka.ldx = static_cast<int>(p.ldx);
    ka.m = p.m;
    ka.nb = p.nb;
    ka.log2g = p.log2g;
    ka.iters = p.iters;
    if (!lane_head_fits(ka)) return kStatusInvalid;
    if constexpr (FUSED) return set_wait(ka);
    return kStatusOk;
}

// The Q6_K stream kernel serves up to 4 activation rows, rows of at most
// kQ6StreamMaxBlocks blocks split into 8 slots (slots_per_row_log2 = 3), and
// no exact-sums output.
bool q6_stream_fits(int m, int nb, bool sums) {
    return !sums && m >= 1 && m <= 4 && nb <= kQ6StreamMaxBlocks && slots_per_row_log2(nb, 8) == 3;
}

template <int MT, int WS, bool FUSED>
void launch_q6_stream_ws(const GemvArgs& ka, int passes, int slots, size_t lds, dim3 grid, hipStream_t stream) {
    const dim3 block(kQ6Waves * 64);
    const LaneHead h = lane_head(ka, FUSED);
    auto go = [&](auto s) {
        constexpr int S = decltype(s)::value;
        // activation passes, all loaded up front (q6_stream_fits keeps them <= 4)
        if constexpr (FUSED) {
            if (passes > 2) return gemv_q6_stream_kernel<MT, WS, S, FUSED, 4><<<grid, block, lds, stream>>>(RK_LANE_HEAD(h), ka);
            if (passes > 1) return gemv_q6_stream_kernel<MT, WS, S, FUSED, 2><<<grid, block, lds, stream>>>(RK_LANE_HEAD(h), ka);
        }
        gemv_q6_stream_kernel<MT, WS, S, FUSED, 1><<<grid, block, lds, stream>>>(RK_LANE_HEAD(h), ka);
    };
    if (slots >= 4) go(std::integral_constant<int, 4>{});
    else go(std::integral_constant<int, 2>{});
}

}  // namespace

// Stream waves per workgroup of the Q6_K stream kernel for a launch of m
// activation rows over `rows` weight rows of nb blocks, or 0 when another
// kernel runs it.
int gemv_stream_waves(int kind, int m, int nb, int64_t rows, bool sums, int cus) {
    if (kind != 6 || !q6_stream_fits(m, nb, sums)) return 0;
    return m > 1 && rows >= 16 * static_cast<int64_t>(cus) ? 16 : 8;
}

namespace {

// One row per row group and stream wave: 16 stream waves for 2 or more
// activation rows where the rows give every CU 16, else 8. Ring slots: 4
// where the LDS holds them beside the activations, else 2. Deeper rings
// measured slower: the larger first burst of weight loads delays everything
// behind it (Llama-3-8B down, 4096 x 14336, one row: 13.4 us with 4 slots,
// 15.7 us with 8). Llama-3-8B down at one row takes 12.6 us with 8 stream
// waves (two rows each) against 13.6 with 16; at 2 and 4 rows the arithmetic
// per step doubles and 16 waves win.
template <bool FUSED>
int launch_q6_stream(GemvParams& p, hipStream_t stream) {
    const int cus = device_cu_count();
    const int mt = p.m <= 1 ? 1 : p.m <= 2 ? 2 : 4;
    p.log2g = 3;
    p.iters = (p.nb + 7) / 8;
    int64_t rows = 0;
    for (int i = 0; i < p.count; ++i) rows += p.rows[i];
    const int WS = gemv_stream_waves(6, p.m, p.nb, rows, false, cus);
    if (WS == 0) return kStatusInvalid;
    const size_t act = (static_cast<size_t>(p.m) * p.nb * kGemvLdsPerBlock + 15) / 16 * 16;
    const int fit = static_cast<int>((kQ6MaxLds - 64 - act) / (WS * kQ6SlotBytes));
    const int slots = fit >= 4 ? 4 : 2;
    if (fit < 2) return kStatusInvalid;  // q6_stream_fits keeps m * nb small enough
    const size_t lds = act + static_cast<size_t>(slots) * WS * kQ6SlotBytes;
    GemvArgs ka;
    int64_t wgs = 0, per_wave = 0;
    int st = plan_args<FUSED>(p, WS, 1, cus, ka, wgs, per_wave);
    if (st == kStatusOk && !FUSED) st = set_wait(ka);  // the waves wait for each other's Q8_K copies too
    if (st != kStatusOk) return st;
    const int passes = (p.m * p.nb + kQ6Waves * 4 - 1) / (kQ6Waves * 4);  // 16 lanes per block: at most 4
    const dim3 grid(static_cast<unsigned>(wgs));
    if (WS == 16) {
        if (mt == 1) launch_q6_stream_ws<1, 16, FUSED>(ka, passes, slots, lds, grid, stream);
        else if (mt == 2) launch_q6_stream_ws<2, 16, FUSED>(ka, passes, slots, lds, grid, stream);
        else launch_q6_stream_ws<4, 16, FUSED>(ka, passes, slots, lds, grid, stream);
    } else {
        if (mt == 1) launch_q6_stream_ws<1, 8, FUSED>(ka, passes, slots, lds, grid, stream);
        else if (mt == 2) launch_q6_stream_ws<2, 8, FUSED>(ka, passes, slots, lds, grid, stream);
        else launch_q6_stream_ws<4, 8, FUSED>(ka, passes, slots, lds, grid, stream);
    }
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

template <int KIND, bool FUSED>
int launch_kind(GemvParams& p, hipStream_t stream) {
    const bool sums = !FUSED && p.isum != nullptr;
    const int cus = device_cu_count();
    const int mt = p.m <= 1 ? 1 : p.m <= 2 ? 2 : p.m <= 4 ? 4 : 8;
    // At most 8 slots per row whatever L is: a row's f32 sum then runs in the
    // same order for every L and every grouping of projections.
    p.log2g = slots_per_row_log2(p.nb, 8);
    const int G = 1 << p.log2g;
    p.iters = (p.nb + G - 1) / G;
    const GemvLanes shape = gemv_lanes(FUSED, sums, p.m, p.nb, p.rows, p.count, cus);
    const int L = shape.lanes, W = shape.waves;
    const int64_t rows_per_group = 64 / L / G;
    // blocks in flight per lane = the blocks a wave ends up with, up to the
    // kernel's most
    GemvArgs ka;
    int64_t wgs = 0, per_wave = 1;
    const int st = plan_args<FUSED>(p, W, rows_per_group, cus, ka, wgs, per_wave);
    if (st != kStatusOk) return st;
    // Blocks in flight per lane: one Q6_K block, and Q4_K blocks for 16 per
    // CU and lane position (two with 8 waves, one with 16). More measured
    // slower in every shape (the memory pipeline of a CU is full with fewer):
    // TinyLlama down (Q6_K, 2048 x 5632) 6.9 -> 6.2 us, Llama-3-8B gate+up
    // (Q4_K, 28672 x 4096) 15.9 -> 14.1 us; TinyLlama gate+up at L = 4 and 16
    // waves takes 5.45 us with one Q4_K block in flight, 6.9 us with two.
    const int d = static_cast<int>(std::min<int64_t>(per_wave, KIND == 6 ? 1 : 16 / W));
    const int passes = (p.m * p.nb + W * 4 - 1) / (W * 4);  // 16 lanes per block
    const size_t lds = static_cast<size_t>(mt) * p.nb * kGemvLdsPerBlock;
    const dim3 grid(static_cast<unsigned>(wgs));
    if (sums) {
        if constexpr (!FUSED) launch_l<KIND, 1, FUSED, true>(ka, W, mt, d, passes, grid, lds, stream);
    } else if (L == 1) {
        launch_l<KIND, 1, FUSED, false>(ka, W, mt, d, passes, grid, lds, stream);
    } else if (L == 2) {
        launch_l<KIND, 2, FUSED, false>(ka, W, mt, d, passes, grid, lds, stream);
    } else if (L == 4) {
        launch_l<KIND, 4, FUSED, false>(ka, W, mt, d, passes, grid, lds, stream);
    } else {
        launch_l<KIND, 8, FUSED, false>(ka, W, mt, d, passes, grid, lds, stream);
    }
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace

int launch_gemv_mfma(int kind, bool fused, GemvParams& p, hipStream_t stream);  // gemv_mfma.hip

// The lane-per-block kernel takes p.m <= 8 activation rows; its LDS holds
// m * nb * kGemvLdsPerBlock bytes (callers keep it <= 112 KiB). Q4_K with 3..16
// rows and Q6_K with 5..8 rows run on the matrix cores, where they are faster
// (TinyLlama gate+up Q4_K: 8.96 against 9.23 us at 4 rows, 11.6 against 14.3
// us at 8; down Q6_K: 13.6 against 20.0 us at 6 rows, while at 4 rows the
// lane-per-block kernel's 11.4 us beats 12.4), except where the exact
// per-block sums are asked for.
// Lanes per block L and waves per workgroup W of the lane-per-block kernel for
// m activation rows, rows of nb super-blocks, and `count` projections of the
// given rows, on `cus` CUs.
GemvLanes gemv_lanes(bool fused, bool sums, int m, int nb, const int64_t* rows, int count, int cus) {
    const int mt = m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
    const int G = 1 << slots_per_row_log2(nb, 8);
    const int iters = (nb + G - 1) / G;
    auto row_groups = [&](int lanes_per_block) {
        const int64_t rpg = 64 / lanes_per_block / G;
        int64_t n = 0;
        for (int i = 0; i < count; ++i) n += (rows[i] + rpg - 1) / rpg;
        return n;
    };
    // Lanes per block L and waves per workgroup W. Where some L >= 2 gives
    // every row group a wave of its own (one round trip per wave), take the
    // largest such L (the most contiguous loads), with 8-wave workgroups if
    // they suffice, else 16. Otherwise (several row groups per wave) L = 4
    // and 8 waves. Eight activation rows allow L <= 2 (more would spill);
    // the exact-sums path runs L = 1 and 16 waves; 8-wave workgroups serve
    // fused launches only.
    const int max_l = sums ? 1 : mt == 8 ? 2 : 8;
    const bool w8_ok = fused && !sums;
    const int64_t slots8 = static_cast<int64_t>(cus) * 8, slots16 = static_cast<int64_t>(cus) * 16;
    int L = 0, W = 16;
    // Long rows (4 or more blocks per slot) first try 16 waves with the
    // largest L that still gives every row group a wave: Llama-3-8B down
    // (Q6_K, 4096 x 14336) then takes 14.5 us, against 15.8 us with L = 4 and
    // 8 waves.
    if (iters >= 4)
        for (int l = max_l; l >= 2 && L == 0; l >>= 1)
            if (row_groups(l) <= slots16) { L = l; W = 16; }
    for (int l = max_l; l >= 2 && L == 0; l >>= 1)
        if (w8_ok && row_groups(l) <= slots8) { L = l; W = 8; }
    for (int l = max_l; l >= 2 && L == 0; l >>= 1)
        if (row_groups(l) <= slots16) { L = l; W = 16; }
    if (L == 0) { L = std::min(4, max_l); W = w8_ok ? 8 : 16; }
    // A shape that leaves CUs idle gives way to a wider L with 16 waves when
    // that fills every CU within two row groups per wave: TinyLlama gate+up
    // (2 x 5632 rows, K = 2048) runs L = 4 on 256 CUs in 5.45 us, against L = 2
    // on 176 CUs in 5.95 us.
    auto wgs_for = [&](int l, int w) { return std::min<int64_t>(cus, (row_groups(l) + w - 1) / w); };
    if (wgs_for(L, W) < cus)
        for (int l = max_l; l > L; l >>= 1)
            if (wgs_for(l, 16) >= cus && row_groups(l) <= 2 * slots16) { L = l; W = 16; break; }
    return GemvLanes{L, W};
}

// The matrix-core kernel from 3 rows for Q4_K, from 5 rows for Q6_K, and for
// Q6_K at 3 or 4 rows when its 16-row tiles fill every CU (Llama-3-8B down,
// 4096 x 14336, at 4 rows: 25.8 -> 22.5 us; TinyLlama down, 2048 rows, stays
// on the lane-per-block kernel, 10.6 against 11.1 us), whenever its LDS holds
// the launch's rows (gemv_mfma_rows).
bool gemv_uses_mfma(int kind, int m, int nb, int64_t rows, int cus) {
    if (m > gemv_mfma_rows(kind, nb)) return false;
    return kind == 4 ? m >= 3 : m >= 5 || (m >= 3 && rows >= 16 * int64_t{cus});
}

int launch_gemv(int kind, bool fused, GemvParams& p, hipStream_t stream) {
    if (p.count == 4) {
        // the lane and stream kernels take three members' fields as preloaded
        // arguments (LaneHead): the fourth member is a launch of its own, with
        // the same bits (a row's arithmetic does not depend on its launch)
        GemvParams a = p, b = p;
        a.count = 3;
        b.count = 1;
        b.w[0] = p.w[3];
        b.out[0] = p.out[3];
        b.ldo[0] = p.ldo[3];
        b.rows[0] = p.rows[3];
        const int st = launch_gemv(kind, fused, a, stream);
        return st != kStatusOk ? st : launch_gemv(kind, fused, b, stream);
    }
    int64_t rows = 0;
    for (int i = 0; i < p.count; ++i) rows += p.rows[i];
    if (gemv_stream_waves(kind, p.m, p.nb, rows, p.isum != nullptr, device_cu_count()) != 0)
        return fused ? launch_q6_stream<true>(p, stream) : launch_q6_stream<false>(p, stream);
    if (gemv_uses_mfma(kind, p.m, p.nb, rows, device_cu_count()) && p.isum == nullptr)
        return launch_gemv_mfma(kind, fused, p, stream);
    if (kind == 4) return fused ? launch_kind<4, true>(p, stream) : launch_kind<4, false>(p, stream);
    if (kind == 6) return fused ? launch_kind<6, true>(p, stream) : launch_kind<6, false>(p, stream);
    return kStatusInvalid;
}

}  // namespace rk

extern "C" int rocknpu_hip_gemv_take_stall(void) {
    int* f = rk::g_stall_flag.load();
    return f != nullptr && __atomic_exchange_n(f, 0, __ATOMIC_SEQ_CST) != 0 ? 1 : 0;
}

extern "C" int rocknpu_hip_gemv_test_stall(int spins) {
    if (spins < 0) return rk::kStatusInvalid;
    rk::g_test_stall_spins.store(spins);
    return rk::kStatusOk;
}
