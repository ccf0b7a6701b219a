// Device helpers shared by the decode GEMV kernels (gemv.hip, gemv_mfma.hip):
// DPP reductions over 16-lane rows, the LDS layout of Q8_K activation rows,
// the in-kernel Q8_K quantisation of f32 activations into it, and the copy of
// Q8_K rows into it.
#pragma once

#include "common.h"

#include <utility>

namespace rk {
namespace {

// A direct global->LDS load of 16 bytes per lane (to lds_dst + 16 * lane,
// lds_dst wave-uniform) from src, issued by inline asm the compiler's
// wait-count pass does not see: the caller waits for it explicitly (wait_vm)
// before reading its bytes and before the wave ends.
__device__ __forceinline__ void dma16_untracked(const void* src, uint8_t* lds_dst) {
    const uint32_t lds = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)(lds_dst)));
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory");
}

// Calls f(integral_constant<int, I>) for I in the sequence, in order.
template <typename F, int... I>
__device__ __forceinline__ void unroll_seq(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4]
// | lgkmcnt[11:8] | vmcnt[5:4] at bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
// The same move with 0 for lanes that read nothing (none do with these
// controls): 0 is the identity of an unsigned max and of an add, so the
// compiler can fold the move into the DPP form of that operation.
template <int CTRL>
__device__ __forceinline__ unsigned dpp0(unsigned v) {
    return static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, true));
}
// DPP controls: quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror.
// Applied in this order to a value that is uniform over the lower lane-index
// bits, they exchange across lane-index bits 0, 1, 2 and 3.
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
// Global-memory (address space 1) views keep global loads and stores even for
// addresses the compiler cannot trace back to a kernel argument.
typedef const __attribute__((address_space(1))) uint8_t* gbytes;
typedef __attribute__((address_space(1))) float* gfloats;
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef v4u v4u_a2 __attribute__((aligned(2)));
typedef const __attribute__((address_space(1))) v4u* gv4u;
typedef const __attribute__((address_space(1))) v4u_a2* gv4u_a2;

// Activation rows in LDS (regions sized for MT rows; blk = mi*nb + b):
//   quants of block blk: 256 bytes at qs + blk * 272
//   its bsums:           16 x int16 at bs + blk * 48
//   its scale:           d[blk]
// The 272- and 48-byte strides put consecutive blocks in different LDS banks.
struct Q8Lds {
    uint8_t* qs;
    uint8_t* bs;
    float* d;
    __device__ __forceinline__ const uint8_t* quants(int blk) const { return qs + blk * kGemvLdsQsStride; }
    __device__ __forceinline__ const int16_t* bsums(int blk) const {
        return reinterpret_cast<const int16_t*>(bs + blk * kGemvLdsBsStride);
    }
    // the arrays' LDS byte addresses, for 32-bit address arithmetic (lds_at)
    __device__ __forceinline__ uint32_t qs_lds() const { return lds_addr(qs); }
    __device__ __forceinline__ uint32_t bs_lds() const { return lds_addr(bs); }
    __device__ __forceinline__ uint32_t d_lds() const { return lds_addr(d); }
    __device__ __forceinline__ static uint32_t lds_addr(const void* p) {
        return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)(p)));
    }
};
// An LDS pointer from a 32-bit LDS byte address.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(3))) T* lds_at(uint32_t a) {
    return reinterpret_cast<const __attribute__((address_space(3))) T*>(static_cast<uintptr_t>(a));
}

__device__ __forceinline__ Q8Lds q8_lds(uint8_t* smem, int mt, int nb) {
    Q8Lds a;
    a.qs = smem;
    a.bs = smem + mt * nb * kGemvLdsQsStride;
    a.d = reinterpret_cast<float*>(a.bs + mt * nb * kGemvLdsBsStride);
    return a;
}

// The 16 values of this lane for quantisation block qb: lane sub of the 16
// holds values 64 t + 4 sub + e (t, e = 0..3), so each of the four loads reads
// 256 contiguous bytes per 16 lanes (whole cache lines).
__device__ __forceinline__ void load_x16(const float* __restrict__ x, int64_t ldx, int nb, int qb, float4 (&f)[4]) {
    const int sub = threadIdx.x & 15;
    const int r = qb / nb, b = qb % nb;
    const float4* src = reinterpret_cast<const float4*>(x + r * ldx + b * kQK + 4 * sub);
#pragma unroll
    for (int t = 0; t < 4; ++t) f[t] = src[16 * t];
}

// Q8_K quantisation of one 256-value block (ggml quantize_row_q8_K_ref) by 16
// lanes, lane sub holding values 64 t + 4 sub + e as loaded by load_x16:
//   max = the first value of largest magnitude; iscale = -127/max;
//   q = min(127, nearest_int(iscale * x)); d = 1/iscale; bsums = sums of 16 q.
// nearest_int is ggml's own: add 1.5 * 2^23 and keep the low mantissa bits,
// i.e. round half to even. |iscale * x| <= 127 (1 + 2^-24)^2 < 127.5, so q is
// in [-127, 127] (the min never binds) and its low byte is q as int8.
// The magnitude and sign of max come from one reduction over the 16 lanes of
// key = (bits of |lane extreme| << 1) | (that extreme is negative): for
// non-negative floats the bit patterns order as the values. Where a value and
// its negation both reach the magnitude (found with two ballots), the first
// one in block order is searched for. Writes the 256 quants at qs, the 16 int16
// bsums at bs and d.
__device__ __forceinline__ void quantize_block(const float4 (&f)[4], uint8_t* qs, int16_t* bs, float* d_out) {
    const int lane = threadIdx.x & 63, sub = lane & 15;
    float v[16];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        v[4 * t] = f[t].x; v[4 * t + 1] = f[t].y; v[4 * t + 2] = f[t].z; v[4 * t + 3] = f[t].w;
    }
    float vmax = v[0], vmin = v[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) {
        vmax = fmaxf(vmax, v[i]);
        vmin = fminf(vmin, v[i]);
    }
    const float amag = fmaxf(fabsf(vmax), fabsf(vmin));
    unsigned key = (__float_as_uint(amag) << 1) | (vmax < amag ? 1u : 0u);
    key = max(key, dpp0<kDppXor1>(key));
    key = max(key, dpp0<kDppXor2>(key));
    key = max(key, dpp0<kDppMirror8>(key));
    key = max(key, dpp0<kDppMirror16>(key));
    const float gmax = __uint_as_float(key >> 1);
    float mx = (key & 1u) ? -gmax : gmax;
    // +gmax and -gmax both in a group: its lanes search for the first. Bit
    // 16 j of `both` is set for such a group j (ballots folded per 16 lanes).
    uint64_t pos = __ballot(gmax > 0.0f && vmax == gmax), neg = __ballot(gmax > 0.0f && vmin == -gmax);
    pos |= pos >> 8; pos |= pos >> 4; pos |= pos >> 2; pos |= pos >> 1;
    neg |= neg >> 8; neg |= neg >> 4; neg |= neg >> 2; neg |= neg >> 1;
    const uint64_t both_groups = pos & neg & 0x0001000100010001ull;
    if (both_groups) {
        const bool both = (both_groups >> (lane & 48)) & 1;
        int first = 0x7fffffff;
#pragma unroll
        for (int i = 15; i >= 0; --i)
            if (fabsf(v[i]) == gmax) first = min(first, (64 * (i >> 2) + 4 * sub + (i & 3)) * 2 + (v[i] < 0.0f ? 1 : 0));
        first = min16(first);
        if (both) mx = (first & 1) ? -gmax : gmax;
    }
    uint32_t wq[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (gmax > 0.0f) {
        const float iscale = -127.0f / mx;
        uint32_t r[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) r[i] = __float_as_uint(iscale * v[i] + 12582912.0f);
        // the low bytes of four rounded values per word: bytes 0,1, then 2,3, by v_perm
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t lo = __builtin_amdgcn_perm(r[4 * t + 1], r[4 * t], 0x0C0C0400u);
            const uint32_t hi = __builtin_amdgcn_perm(r[4 * t + 3], r[4 * t + 2], 0x0C0C0400u);
            wq[t] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        }
        d = 1.0f / iscale;
    }
    // bsum of 16-value group 4 t + sub / 4: four lanes' word sums, added over the lane quad
    int gs[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        unsigned g = static_cast<unsigned>(__builtin_amdgcn_sdot4(static_cast<int>(wq[t]), 0x01010101, 0, false));
        g += dpp0<kDppXor1>(g);
        g += dpp0<kDppXor2>(g);
        gs[t] = static_cast<int>(g);
        *reinterpret_cast<uint32_t*>(qs + 64 * t + 4 * sub) = wq[t];
    }
    // lane tq of each quad writes group 4 tq + sub / 4 (selects on the bits of tq)
    const int tq = sub & 3;
    const int g01 = (tq & 1) ? gs[1] : gs[0], g23 = (tq & 1) ? gs[3] : gs[2];
    bs[4 * tq + (sub >> 2)] = static_cast<int16_t>((tq & 2) ? g23 : g01);
    if (sub == 0) *d_out = d;
}

__device__ __forceinline__ void quantize_block_to_lds(const float4 (&f)[4], int qb, const Q8Lds& a) {
    quantize_block(f, a.qs + qb * kGemvLdsQsStride, reinterpret_cast<int16_t*>(a.bs + qb * kGemvLdsBsStride),
                   a.d + qb);
}

// Q8_K quantisation of rows [0, m) of x into LDS by the first waves of the
// workgroup: THREADS/16 blocks per pass. The activations of the first P
// passes are loaded up front (XPre::issue, before the weight loads), so their
// latencies overlap; later passes, if any, load as they go.
template <int THREADS, int P>
struct XPre {
    float4 f[P][4];
    // t: this thread's index among the THREADS that quantise (default: the
    // workgroup's first THREADS)
    __device__ __forceinline__ void issue(const float* __restrict__ x, int64_t ldx, int m, int nb) {
        issue(x, ldx, m, nb, static_cast<int>(threadIdx.x));
    }
    __device__ __forceinline__ void issue(const float* __restrict__ x, int64_t ldx, int m, int nb, int t) {
        const int slot = t >> 4, last = m * nb - 1;
#pragma unroll
        for (int i = 0; i < P; ++i) load_x16(x, ldx, nb, min(slot + i * (THREADS / 16), last), f[i]);
    }
    __device__ __forceinline__ void quantize(const float* __restrict__ x, int64_t ldx, int m, int nb,
                                             const Q8Lds& a) const {
        quantize(x, ldx, m, nb, a, static_cast<int>(threadIdx.x));
    }
    __device__ __forceinline__ void quantize(const float* __restrict__ x, int64_t ldx, int m, int nb,
                                             const Q8Lds& a, int t) const {
        const int slot = t >> 4;
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const int qb = slot + i * (THREADS / 16);
            if (qb < m * nb) quantize_block_to_lds(f[i], qb, a);
        }
        for (int qb = slot + P * (THREADS / 16); qb < m * nb; qb += THREADS / 16) {
            float4 g[4];
            load_x16(x, ldx, nb, qb, g);
            quantize_block_to_lds(g, qb, a);
        }
    }
};

// The first three members' output fields (out, ldo, rows), read from the
// argument segment where fetch() is called (behind a launch's first loads)
// rather than at the first store, where the compiler puts them otherwise.
struct MemberOuts {
    const float* o0;
    const float* o1;
    const float* o2;
    int l0, l1, l2, r0, r1, r2;
    template <class Args>
    __device__ __forceinline__ void fetch(const Args& p) {
        o0 = p.mb[0].out;
        o1 = p.mb[1].out;
        o2 = p.mb[2].out;
        l0 = p.mb[0].ldo;
        l1 = p.mb[1].ldo;
        l2 = p.mb[2].ldo;
        r0 = p.mb[0].rows;
        r1 = p.mb[1].rows;
        r2 = p.mb[2].rows;
    }
};

// Copy Q8_K rows (292-byte blocks: f32 d, 256 quants, 16 int16 bsums) into
// the LDS layout, one 32-bit word per thread and step.
// t: this thread's index among the THREADS that copy.
template <int THREADS>
__device__ __forceinline__ void stage_q8k(const uint8_t* __restrict__ q8k, int64_t ldq, int m, int nb,
                                          const Q8Lds& a, int t) {
    const int words = m * nb * (kQ8KBytes / 4);
    for (int i = t; i < words; i += THREADS) {
        const int blk = i / (kQ8KBytes / 4), wi = i % (kQ8KBytes / 4);
        const int mi = blk / nb, bi = blk % nb;
        const uint32_t v = *reinterpret_cast<const uint32_t*>(q8k + mi * ldq + bi * kQ8KBytes + 4 * wi);
        if (wi == 0) a.d[blk] = __uint_as_float(v);
        else if (wi <= 64) reinterpret_cast<uint32_t*>(a.qs + blk * kGemvLdsQsStride)[wi - 1] = v;
        else reinterpret_cast<uint32_t*>(a.bs + blk * kGemvLdsBsStride)[wi - 65] = v;
    }
}
template <int THREADS>
__device__ __forceinline__ void stage_q8k(const uint8_t* __restrict__ q8k, int64_t ldq, int m, int nb,
                                          const Q8Lds& a) {
    stage_q8k<THREADS>(q8k, ldq, m, nb, a, static_cast<int>(threadIdx.x));
}

}  // namespace
}  // namespace rk
