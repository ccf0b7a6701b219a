// Kernel (d) for 2..8 activation rows, Q4_K and Q6_K weights (the launch
// layer sends Q4_K at 3..8 rows and Q6_K at 5..8 here): the decode GEMV with
// the per-sub-block integer dot products on the matrix cores.
//
// Same arithmetic as gemv.hip (ggml_vec_dot_q{4,6}_K_q8_K, per block and row):
//   isum = sum_s sc_s * sum_{k in sub-block s} q8[k] * q[k]
//          (Q4_K: s = 0..7 of 32 values; Q6_K: s = 0..15 of 16, q = stored - 32)
//   msum = sum_s mn_s * (sum of the activation quants of sub-block s)   (Q4_K)
//   row += (d * d_a) * isum - (dmin * d_a) * msum                 (f32)
// with exact integers up to the f32 scaling, so the results differ from the
// VALU kernel's only in the f32 order of the per-block terms.
//
// v_mfma_i32_16x16x32_i8 on gfx950: lane l supplies row l%16 of A and column
// l%16 of B, with K bytes 8*(l/16) .. +7, and holds D column l%16, rows
// 4*(l/16) + e (e = 0..3). Here B's 16 columns are 16 weight rows and A's 16
// rows are MT activation rows times SPLIT = 16/MT sub-blocks: A row r =
// (sub-block r / MT of the instruction's group, activation row r % MT), and
// instruction t of a group of SPLIT sub-blocks puts the activations of its
// sub-block t in rows t*MT .. t*MT+MT-1 and zeros elsewhere. The SPLIT
// instructions of a group then fill disjoint rows of one accumulator, so D
// holds SPLIT sub-block products for all MT rows and 16 weight rows with no
// padding. Q6_K's 16-value sub-blocks take half an instruction's 32 K slots
// each: slot r / MT then holds its sub-block in K half (r / MT) & 1, so one
// instruction serves two slots and a group of SPLIT slots takes SPLIT / 2.
// Each lane scales its four D values by its weight row's sub-block scales
// (integer multiply-add), and the lanes that hold the same activation row and
// weight row add their sub-blocks' sums with lane exchanges.
//
// Work split: a tile is 16 weight rows. A workgroup holds 8 waves; wave g
// takes blocks g, g + 8, .. of every tile its workgroup walks (tiles
// blockIdx.x, + gridDim.x, ..), with D blocks of loads in flight (the
// launcher runs D = 1). When a
// tile's blocks are done, the waves leave their f32 partial sums in LDS and
// wave 0 adds them in wave order and stores the rows. The f32 order of a
// row's terms therefore depends only on nb: the same in fused launches, in
// grouped launches and in Q8_K-input launches.
#include "gemv_lds.h"

#include <algorithm>

namespace rk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kMfmaWaves = 8;  // waves per workgroup = block slots per tile
constexpr int kTileRows = 16;

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
};

// Scale and min of Q4_K sub-block 4*hi + idx (idx = 0..3; ggml
// get_scale_min_k4) from the three scale words s0 s1 s2 of the header.
__device__ __forceinline__ void q4_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, bool hi, int idx, int& sc,
                                             int& mn) {
    const int sh = 8 * idx;
    const uint32_t a0 = s0 >> sh, a1 = s1 >> sh, a2 = s2 >> sh;
    sc = hi ? static_cast<int>((a2 & 0xF) | ((a0 >> 2) & 0x30)) : static_cast<int>(a0 & 63);
    mn = hi ? static_cast<int>(((a2 >> 4) & 0xF) | ((a1 >> 2) & 0x30)) : static_cast<int>(a1 & 63);
}

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
    // The 8 signed values of quarter t % 4 of half t / 4 in this lane's K slots.
    __device__ __forceinline__ uint64_t values(int t) const {
        const int h = t >> 2, g = t & 3;
        const uint64_t lo4 = (run8(ql[2 * h + (g & 1)]) >> (4 * (g >> 1))) & 0x0F0F0F0F0F0F0F0Full;
        const uint64_t hi2 = (run8(qh[h]) >> (2 * g)) & 0x0303030303030303ull;
        const uint64_t v = lo4 | hi2 << 4;  // 0..63 per byte
        // v - 32 per byte without borrows between bytes
        return ((v | 0x8080808080808080ull) - 0x2020202020202020ull) ^ 0x8080808080808080ull;
    }
    // int8 scale of 16-value sub-block s
    __device__ __forceinline__ int scale(int s) const {
        const v4u v = v4u{__builtin_amdgcn_alignbyte(sc.y, sc.x, sh), __builtin_amdgcn_alignbyte(sc.z, sc.y, sh),
                          __builtin_amdgcn_alignbyte(sc.w, sc.z, sh), __builtin_amdgcn_alignbyte(tail, sc.w, sh)};
        const uint32_t w = s < 4 ? v.x : s < 8 ? v.y : s < 12 ? v.z : v.w;
        return static_cast<int8_t>((w >> (8 * (s & 3))) & 0xFF);
    }
    __device__ __forceinline__ void scales(float& d, float& dmin) const {
        d = f16_bits_to_f32(static_cast<uint16_t>(tail >> 16));
        dmin = 0.0f;
    }
};

// Sums of v over lanes l and l ^ 16, and over l and l ^ 32: gfx950's row swaps
// (v_permlane16_swap / v_permlane32_swap exchange the odd 16-lane rows of one
// operand with the even rows of the other; with both operands v, the two
// results hold v of the lane and of its partner).
__device__ __forceinline__ int sum_xor16(int v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return static_cast<int>(r[0]) + static_cast<int>(r[1]);
}
__device__ __forceinline__ int sum_xor32(int v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return static_cast<int>(r[0]) + static_cast<int>(r[1]);
}

template <int KIND, int MT, bool FUSED, int D, int QP>
__global__ __launch_bounds__(kMfmaWaves * 64) void gemv_mfma_kernel(const MfmaArgs p) {
    constexpr int W = kMfmaWaves;
    constexpr int BB = block_bytes(KIND);
    constexpr int SPLIT = 16 / MT;  // sub-block slots per accumulator
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int q8_ready;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = p.nb, m = p.m;
    const Q8Lds a = q8_lds(smem, MT, nb);
    // f32 partial sums of a tile: [buffer][wave][lane][e], after the activations
    float* part = reinterpret_cast<float*>(smem + ((MT * nb * kGemvLdsPerBlock + 15) & ~15));

    const int n = lane & 15, q = lane >> 4;  // B column (weight row in the tile), K slot group
    const int iters = (nb + W - 1) / W;       // blocks per wave and tile

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

    const int quant_waves = FUSED ? min(W, (m * nb + 3) / 4) : 0;
    const bool quant_wave = wave < quant_waves;
    XPre<W * 64, QP> xpre;
    if constexpr (FUSED) {
        if (quant_wave) xpre.issue(p.x, p.ldx, m, nb);
    }
    MPiece<KIND> buf[D];
    Pos lq{static_cast<int>(blockIdx.x), 0};  // next item to load
#pragma unroll
    for (int j = 0; j < D; ++j) {
        load(lq, buf[j]);
        advance(lq);
    }
    if constexpr (FUSED) {
        if (threadIdx.x == 0) q8_ready = 0;
        __syncthreads();
        if (quant_wave) {
            xpre.quantize(p.x, p.ldx, m, nb, a);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_fetch_add(&q8_ready, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        for (int spin = 0; spin < (1 << 24); ++spin) {
            if (__hip_atomic_load(&q8_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= quant_waves) break;
            __builtin_amdgcn_s_sleep(1);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    } else {
        stage_q8k<W * 64>(p.q8k, p.ldx, m, nb, a);
        __syncthreads();
    }

    // A operand row of this lane: sub-block slot sa of a group, activation row ma
    const int ra = lane & 15, sa = ra / MT, ma = ra % MT;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
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
                int is[4] = {0, 0, 0, 0}, ms[4] = {0, 0, 0, 0};
                if constexpr (KIND == 4) {
                    // 8 sub-blocks of 32: SPLIT per accumulator, one per instruction
#pragma unroll
                    for (int gi = 0; gi < 8 / SPLIT; ++gi) {
                        // this lane's activation bytes for its A row (rows >= m of the LDS area are
                        // not written: read, then replaced by zeros)
                        uint64_t xa = *reinterpret_cast<const uint64_t*>(a.quants(ma * nb + bk) + 32 * (gi * SPLIT + sa) + 8 * q);
                        xa = ma < m ? xa : 0;
                        v4i dacc = {0, 0, 0, 0};
#pragma unroll
                        for (int t = 0; t < SPLIT; ++t) {
                            const int s = gi * SPLIT + t;  // sub-block
                            const uint64_t wq = (k.qp[s >> 1] >> (4 * (s & 1))) & 0x0F0F0F0F0F0F0F0Full;
                            const uint64_t av = sa == t ? xa : 0;
                            dacc = __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(av), static_cast<long>(wq),
                                                                         dacc, 0, 0, 0);
                        }
                        // D row 4q + e = (sub-block slot so, activation row mo)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int r = 4 * q + e, so = r / MT, mo = r % MT;
                            const int s = gi * SPLIT + so;
                            int sc, mn;
                            q4_scale_min(k.h.y, k.h.z, k.h.w, s >= 4, s & 3, sc, mn);
                            is[e] += sc * dacc[e];
                            const uint32_t bp = *reinterpret_cast<const uint32_t*>(a.bsums(mo * nb + bk) + 2 * s);
                            const int bsum = static_cast<int16_t>(bp & 0xFFFF) + static_cast<int16_t>(bp >> 16);
                            ms[e] += mn * (mo < m ? bsum : 0);
                        }
                    }
                } else {
                    // 16 sub-blocks of 16: an instruction covers two (K slots 0-15 and 16-31,
                    // lane groups q >> 1 = 0 and 1), so SPLIT / 2 instructions per accumulator;
                    // slot sa of the A rows holds sub-block gi * SPLIT + sa in K half sa & 1
                    const bool my_half = (q >> 1) == (sa & 1);
#pragma unroll
                    for (int gi = 0; gi < 16 / SPLIT; ++gi) {
                        uint64_t xa = *reinterpret_cast<const uint64_t*>(a.quants(ma * nb + bk) + 16 * (gi * SPLIT + sa) + 8 * (q & 1));
                        xa = ma < m && my_half ? xa : 0;
                        v4i dacc = {0, 0, 0, 0};
#pragma unroll
                        for (int u = 0; u < SPLIT / 2; ++u) {
                            const uint64_t wq = k.values(gi * SPLIT / 2 + u);
                            const uint64_t av = (sa >> 1) == u ? xa : 0;
                            dacc = __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(av), static_cast<long>(wq),
                                                                         dacc, 0, 0, 0);
                        }
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int so = (4 * q + e) / MT;
                            is[e] += k.scale(gi * SPLIT + so) * dacc[e];
                        }
                    }
                }
                // add the sub-block slots holding the same activation row
                if constexpr (MT == 2) {  // rows 4q + e: slot 2q + e/2, row e%2
#pragma unroll
                    for (int e = 0; e < 2; ++e) { is[e] += is[e + 2]; ms[e] += ms[e + 2]; }
                }
                constexpr int NE = MT == 2 ? 2 : 4;
#pragma unroll
                for (int e = 0; e < NE; ++e) {
                    if constexpr (MT <= 4) {
                        is[e] = sum_xor16(is[e]);
                        if constexpr (KIND == 4) ms[e] = sum_xor16(ms[e]);
                    }
                    if constexpr (MT <= 8) {
                        is[e] = sum_xor32(is[e]);
                        if constexpr (KIND == 4) ms[e] = sum_xor32(ms[e]);
                    }
                }
                float dw, dmw;
                k.scales(dw, dmw);
#pragma unroll
                for (int e = 0; e < NE; ++e) {
                    const int mo = (4 * q + e) % MT;
                    const float da = a.d[mo * nb + bk];
                    float term = (dw * da) * static_cast<float>(is[e]);
                    if constexpr (KIND == 4) term = term - (dmw * da) * static_cast<float>(ms[e]);
                    acc[e] += have ? term : 0.0f;
                }
                load(lq, buf[j]);
                advance(lq);
                if (it == iters - 1) {
                    // tile done: partial sums to LDS, then wave 0 adds them in wave order
                    float* pb = part + (tile_iter & 1) * (W * 64 * 4);
                    *reinterpret_cast<float4*>(pb + (wave * 64 + lane) * 4) = make_float4(acc[0], acc[1], acc[2], acc[3]);
                    acc[0] = acc[1] = acc[2] = acc[3] = 0.0f;
                    // the LDS writes complete, then the barrier; a compiler memory
                    // barrier too, and no wait for the weight loads in flight
                    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                    if (wave == 0) {
                        const int t = cq.t;
                        const bool c1 = t >= p.mb[0].tile_end, c2 = t >= p.mb[1].tile_end, c3 = t >= p.mb[2].tile_end;
                        float* out = c3 ? p.mb[3].out : c2 ? p.mb[2].out : c1 ? p.mb[1].out : p.mb[0].out;
                        const int ldo = c3 ? p.mb[3].ldo : c2 ? p.mb[2].ldo : c1 ? p.mb[1].ldo : p.mb[0].ldo;
                        const int rows = c3 ? p.mb[3].rows : c2 ? p.mb[2].rows : c1 ? p.mb[1].rows : p.mb[0].rows;
                        const int t0 = c3 ? p.mb[2].tile_end : c2 ? p.mb[1].tile_end : c1 ? p.mb[0].tile_end : 0;
                        const int row = (t - t0) * kTileRows + n;
                        // activation row mo is held by lane 16 (mo / 4) + n, element mo % 4
#pragma unroll
                        for (int k4 = 0; k4 < (MT + 3) / 4; ++k4) {
                            const int mo = q + 4 * k4;
                            if (mo < m && row < rows) {
                                const int src = 16 * (mo >> 2) + n, e = mo & 3;
                                float r = pb[src * 4 + e];
#pragma unroll
                                for (int g = 1; g < W; ++g) r += pb[(g * 64 + src) * 4 + e];
                                reinterpret_cast<gfloats>(reinterpret_cast<uint64_t>(out))[mo * ldo + row] = r;
                            }
                        }
                    }
                    ++tile_iter;
                }
                advance(cq);
            }
        }
    }
}

// One block of loads in flight per wave: deeper rings measured slower in
// every shape (TinyLlama gate+up at 4 rows 8.95 -> 8.40 us, Llama-3-8B
// gate+up at 4 rows 28.0 -> 26.7 us, with one instead of up to four).
template <int KIND, int MT, bool FUSED, int QP>
void launch_d(const MfmaArgs& p, dim3 grid, size_t lds, hipStream_t stream) {
    gemv_mfma_kernel<KIND, MT, FUSED, 1, QP><<<grid, dim3(kMfmaWaves * 64), lds, stream>>>(p);
}

template <int KIND, int MT, bool FUSED>
void launch_mt(const MfmaArgs& p, int passes, dim3 grid, size_t lds, hipStream_t stream) {
    if constexpr (FUSED) {
        if (passes > 1) return launch_d<KIND, MT, FUSED, 4>(p, grid, lds, stream);
    }
    launch_d<KIND, MT, FUSED, 1>(p, grid, lds, stream);
}

template <int KIND>
void launch_kind(bool fused, int mt, const MfmaArgs& ka, int passes, dim3 grid, size_t lds,
                 hipStream_t stream) {
    if (fused) {
        if (mt == 2) launch_mt<KIND, 2, true>(ka, passes, grid, lds, stream);
        else if (mt == 4) launch_mt<KIND, 4, true>(ka, passes, grid, lds, stream);
        else launch_mt<KIND, 8, true>(ka, passes, grid, lds, stream);
    } else {
        if (mt == 2) launch_mt<KIND, 2, false>(ka, passes, grid, lds, stream);
        else if (mt == 4) launch_mt<KIND, 4, false>(ka, passes, grid, lds, stream);
        else launch_mt<KIND, 8, false>(ka, passes, grid, lds, stream);
    }
}

}  // namespace

// Q4_K or Q6_K, 2 <= p.m <= 8.
int launch_gemv_mfma(int kind, bool fused, GemvParams& p, hipStream_t stream) {
    if (p.m < 2 || p.m > 8 || (kind != 4 && kind != 6)) return kStatusInvalid;
    const int mt = p.m <= 2 ? 2 : p.m <= 4 ? 4 : 8;
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
    // one workgroup per CU at most; each walks its tiles
    const int cus = device_cu_count();
    const int wgs = std::min(tiles, cus);
    const int passes = (p.m * p.nb + kMfmaWaves * 4 - 1) / (kMfmaWaves * 4);
    const size_t lds = ((static_cast<size_t>(mt) * p.nb * kGemvLdsPerBlock + 15) & ~size_t{15}) +
                       2 * kMfmaWaves * 64 * 4 * sizeof(float);
    const dim3 grid(static_cast<unsigned>(wgs));
    if (kind == 4) launch_kind<4>(fused, mt, ka, passes, grid, lds, stream);
    else launch_kind<6>(fused, mt, ka, passes, grid, lds, stream);
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace rk
