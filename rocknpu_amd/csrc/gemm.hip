// Kernel (c): prefill W8A8 GEMM on CDNA4 int8 MFMA with the rescale fused.
//
// C_i32[m,n] = sum_k A8[m,k] * W8[n,k]   (exact; |C| <= 127^2 * K < 2^31)
// out[m,n]   = (f32(C) * a_scale[m]) * w_scale[n]
// which is the reference's M-tile product and rescale_i32_row
// (crates/rocknpu-capi/src/lib.rs:692-709, :1868-1884; NPU program
// crates/rocknpu-regcmd/src/int8.rs:112-205). Both operands are K-contiguous
// int8 rows; K is a multiple of 64 (rows are zero-padded, which is exact).
//
// Tiling: a workgroup computes a BM x BN tile with WM x WN waves; each wave
// owns a (BM/WM) x (BN/WN) sub-tile of 16x16 MFMA fragments
// (v_mfma_i32_16x16x64_i8: lane l supplies row l%16 and the 16 bytes of
// k-slot l/16 for both operands; it receives rows 4*(l/16)+i, column l%16).
// K advances in 64-byte slabs through double-buffered LDS with an XOR swizzle
// on the 16-byte chunk index so fragment reads are bank-conflict free.
#include "common.h"

#include <utility>

#include <type_traits>

namespace rk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;

__device__ __forceinline__ int swz(int r, int kc) { return r * kBK + ((kc ^ ((r >> 1) & 3)) << 4); }

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM* WN * 64) void gemm_w8a8_kernel(
    const int8_t* __restrict__ a8, int64_t lda, const int8_t* __restrict__ w8, int64_t ldw,
    const float* __restrict__ a_scales, const float* __restrict__ w_scales, int m, int n, int k,
    float* __restrict__ out, int64_t ldo, int32_t* __restrict__ out_i32, int64_t ldo_i32) {
    constexpr int T = WM * WN * 64;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 16, FN = TN / 16;
    constexpr int A_CHUNKS = BM * kBK / 16, B_CHUNKS = BN * kBK / 16;
    constexpr int A_PER = (A_CHUNKS + T - 1) / T, B_PER = (B_CHUNKS + T - 1) / T;
    static_assert(FM >= 1 && FN >= 1, "wave tile must hold at least one 16x16 fragment");
    __shared__ __align__(16) int8_t As[2][BM * kBK];
    __shared__ __align__(16) int8_t Bs[2][BN * kBK];

    const int tiles_n = (n + BN - 1) / BN;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    uint4 ra[A_PER], rb[B_PER];
    auto gload = [&](int kt) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + i * T;
            const int r = c >> 2, kc = c & 3;
            const int gr = m0 + r;
            ra[i] = (c < A_CHUNKS && gr < m)
                        ? *reinterpret_cast<const uint4*>(a8 + gr * lda + kt * kBK + kc * 16)
                        : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + i * T;
            const int r = c >> 2, kc = c & 3;
            const int gr = n0 + r;
            rb[i] = (c < B_CHUNKS && gr < n)
                        ? *reinterpret_cast<const uint4*>(w8 + gr * ldw + kt * kBK + kc * 16)
                        : make_uint4(0, 0, 0, 0);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + i * T;
            if (c < A_CHUNKS) *reinterpret_cast<uint4*>(&As[buf][swz(c >> 2, c & 3)]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + i * T;
            if (c < B_CHUNKS) *reinterpret_cast<uint4*>(&Bs[buf][swz(c >> 2, c & 3)]) = rb[i];
        }
    };

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    const int KT = k / kBK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);
        v4i af[FM], bf[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
            af[i] = *reinterpret_cast<const v4i*>(&As[cur][swz(wm * TM + i * 16 + (lane & 15), lane >> 4)]);
#pragma unroll
        for (int j = 0; j < FN; ++j)
            bf[j] = *reinterpret_cast<const v4i*>(&Bs[cur][swz(wn * TN + j * 16 + (lane & 15), lane >> 4)]);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = n0 + wn * TN + j * 16 + (lane & 15);
            if (col >= n) continue;
            const float ws = w_scales[col];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = m0 + wm * TM + i * 16 + 4 * (lane >> 4) + e;
                if (row >= m) continue;
                const int v = acc[i][j][e];
                const float t = static_cast<float>(v) * a_scales[row];
                out[row * ldo + col] = t * ws;
                if (out_i32) out_i32[row * ldo_i32 + col] = v;
            }
        }
}

// Direct-load tiles: the same product with a pipeline of ST (4 or 8) LDS
// stage buffers filled by direct global->LDS loads (global_load_lds_dwordx4,
// no register staging). Each wave issues its share of a stage as 1 KiB
// segments (16 rows x 64 bytes; lane i's 16 bytes land at segment + 16*i, so
// the lane loads the global chunk that the swizzled layout puts there).
// Stage s+ST-1 is issued while stage s is multiplied; one barrier per K step
// both publishes stage s (after each wave's own wait for its loads) and frees
// stage s-1 for reuse. The barrier is a bare s_barrier: a fenced one would
// wait for every load in flight, stages ahead included. Small tiles run 8
// stages: their K steps hold few MFMAs, so more of the load latency must be
// in flight.
template <int BM, int BN, int WM, int WN>
struct DmaTile {
    static constexpr int T = WM * WN * 64;
    static constexpr int W = WM * WN;
    // 1 KiB segments (16 rows) per wave and stage. When a tile has fewer
    // segments than waves, waves load segments twice (the same bytes to the
    // same LDS place), so every wave issues the same number of loads.
    static constexpr int A_ROWSEG = BM / 16, B_ROWSEG = BN / 16;
    static constexpr int A_SEG = A_ROWSEG >= W ? A_ROWSEG / W : 1, B_SEG = B_ROWSEG >= W ? B_ROWSEG / W : 1;
    static_assert(BM % 16 == 0 && BN % 16 == 0, "tile rows must split into 16-row segments");
    static_assert((B_ROWSEG >= W ? B_SEG * W == B_ROWSEG : W % B_ROWSEG == 0) &&
                      (A_ROWSEG >= W ? A_SEG * W == A_ROWSEG : W % A_ROWSEG == 0),
                  "segments split evenly over the waves");
};

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4]
// | lgkmcnt[11:8] | vmcnt[5:4] at bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | ((0x3) << 14)); }

// One 16-byte direct global->LDS load per lane; `lds` must be wave-uniform
// (the 64 lanes fill lds .. lds + 1023).
__device__ __forceinline__ void dma16(const int8_t* src, int8_t* lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds), 16, 0, 0);
}

// Calls f(integral_constant<int, I>) for I in the sequence, in order.
template <typename F, int... I>
__device__ __forceinline__ void unroll_seq(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}

template <int BM, int BN, int WM, int WN, int ST>
__global__ __launch_bounds__(WM* WN * 64) void gemm_w8a8_dma_kernel(
    const int8_t* __restrict__ a8, int64_t lda, const int8_t* __restrict__ w8, int64_t ldw,
    const float* __restrict__ a_scales, const float* __restrict__ w_scales, int m, int n, int k,
    float* __restrict__ out, int64_t ldo, int32_t* __restrict__ out_i32, int64_t ldo_i32) {
    using Cfg = DmaTile<BM, BN, WM, WN>;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 fragments
    // One array per stage, always indexed by a compile-time stage: the
    // wait-count pass then sees which LDS buffer a direct load writes and does
    // not wait for every load in flight before each LDS read.
    // ST = 4..8 stages; arrays of stages >= ST are unused placeholders.
    static_assert(ST >= 4 && ST <= 8, "four to eight stage buffers");
    constexpr int A4 = ST > 4 ? BM * kBK : 16, A5 = ST > 5 ? BM * kBK : 16, A6 = ST > 6 ? BM * kBK : 16,
                  A7 = ST > 7 ? BM * kBK : 16;
    constexpr int B4 = ST > 4 ? BN * kBK : 16, B5 = ST > 5 ? BN * kBK : 16, B6 = ST > 6 ? BN * kBK : 16,
                  B7 = ST > 7 ? BN * kBK : 16;
    __shared__ __align__(16) int8_t la0[BM * kBK], la1[BM * kBK], la2[BM * kBK], la3[BM * kBK];
    __shared__ __align__(16) int8_t lb0[BN * kBK], lb1[BN * kBK], lb2[BN * kBK], lb3[BN * kBK];
    __shared__ __align__(16) int8_t la4[A4], la5[A5], la6[A6], la7[A7];
    __shared__ __align__(16) int8_t lb4[B4], lb5[B5], lb6[B6], lb7[B7];
    auto stage_a = [&](auto st) -> int8_t* {
        constexpr int S = decltype(st)::value;
        if constexpr (S == 0) return la0; else if constexpr (S == 1) return la1;
        else if constexpr (S == 2) return la2; else if constexpr (S == 3) return la3;
        else if constexpr (S == 4) return la4; else if constexpr (S == 5) return la5;
        else if constexpr (S == 6) return la6; else return la7;
    };
    auto stage_b = [&](auto st) -> int8_t* {
        constexpr int S = decltype(st)::value;
        if constexpr (S == 0) return lb0; else if constexpr (S == 1) return lb1;
        else if constexpr (S == 2) return lb2; else if constexpr (S == 3) return lb3;
        else if constexpr (S == 4) return lb4; else if constexpr (S == 5) return lb5;
        else if constexpr (S == 6) return lb6; else return lb7;
    };

    // XCD-aware tile order: workgroup b runs on XCD b % 8, so each XCD takes a
    // contiguous range of tile indices, walked in groups of 4 tile rows; the
    // 32 tiles an XCD runs at once then share A rows and W rows in its L2.
    const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
    const int tiles = tiles_m * tiles_n;
    const int bid = blockIdx.x, xcd = bid & 7, per = tiles >> 3, rem = tiles & 7;
    const int t = xcd * per + min(xcd, rem) + (bid >> 3);
    constexpr int GM = 4;
    const int group = t / (GM * tiles_n), first_m = group * GM;
    const int gsize = min(tiles_m - first_m, GM);
    const int tm = first_m + (t % (GM * tiles_n)) % gsize, tn = (t % (GM * tiles_n)) / gsize;
    const int m0 = tm * BM, n0 = tn * BN;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;

    // This lane's source row and chunk for each of its segments. Rows past the
    // matrix re-read its last row (their products land in rows/columns that
    // are never stored).
    const int8_t* asrc[Cfg::A_SEG];
    const int8_t* bsrc[Cfg::B_SEG];
#pragma unroll
    for (int q = 0; q < Cfg::A_SEG; ++q) {
        const int r = ((wave * Cfg::A_SEG + q) % Cfg::A_ROWSEG) * 16 + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 1) & 3);
        asrc[q] = a8 + static_cast<int64_t>(min(m0 + r, m - 1)) * lda + c * 16;
    }
#pragma unroll
    for (int q = 0; q < Cfg::B_SEG; ++q) {
        const int r = ((wave * Cfg::B_SEG + q) % Cfg::B_ROWSEG) * 16 + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 1) & 3);
        bsrc[q] = w8 + static_cast<int64_t>(min(n0 + r, n - 1)) * ldw + c * 16;
    }
    auto issue = [&](auto st, int kt) {
        int8_t* la = stage_a(st);
        int8_t* lb = stage_b(st);
#pragma unroll
        for (int q = 0; q < Cfg::A_SEG; ++q)
            dma16(asrc[q] + kt * kBK, la + ((wave * Cfg::A_SEG + q) % Cfg::A_ROWSEG) * 1024);
#pragma unroll
        for (int q = 0; q < Cfg::B_SEG; ++q)
            dma16(bsrc[q] + kt * kBK, lb + ((wave * Cfg::B_SEG + q) % Cfg::B_ROWSEG) * 1024);
    };

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16i{};

    const int KT = k / kBK;
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    // Pipeline per K step s (stage s's fragments were read in step s-1):
    //   wait for those reads and for this wave's loads of stage s+1; barrier
    //   (every wave's stage s+1 is in, and every wave holds stage s in
    //   registers, so its buffer is free); issue stage s+4 into that buffer;
    //   read stage s+1's fragments into the other register set; then the
    //   MFMAs of stage s, which run while those reads complete.
    // Past the last K step the issue re-reads the last step into a buffer no
    // step reads, so the count of loads in flight stays fixed.
    constexpr int PER_STAGE = Cfg::A_SEG + Cfg::B_SEG;  // loads per wave and stage
    v4i fa[2][2][FM], fb[2][2][FN];  // [register set][32-deep half][fragment]
    // lane l supplies row l%32 and the 16 bytes of chunk 2*h + l/32
    auto read_half = [&](auto st, auto set, auto half) {
        constexpr int R = decltype(set)::value, H = decltype(half)::value;
        const int8_t* la = stage_a(st);
        const int8_t* lb = stage_b(st);
#pragma unroll
        for (int i = 0; i < FM; ++i)
            fa[R][H][i] = *reinterpret_cast<const v4i*>(la + swz(wm * TM + i * 32 + (lane & 31), 2 * H + (lane >> 5)));
#pragma unroll
        for (int j = 0; j < FN; ++j)
            fb[R][H][j] = *reinterpret_cast<const v4i*>(lb + swz(wn * TN + j * 32 + (lane & 31), 2 * H + (lane >> 5)));
    };
    using H0 = std::integral_constant<int, 0>;
    using H1 = std::integral_constant<int, 1>;
    auto read_frags = [&](auto st, auto set) {
        read_half(st, set, H0{});
        read_half(st, set, H1{});
    };
    auto mfma_half = [&](auto set, auto half) {
        constexpr int R = decltype(set)::value, H = decltype(half)::value;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int i = 0; i < FM; ++i)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[R][H][i], fb[R][H][j], acc[i][j], 0, 0, 0);
    };
    using R0 = std::integral_constant<int, 0>;
    using R1 = std::integral_constant<int, 1>;
    // prologue: stages 0 .. ST-2 in flight, wait for stage 0, then stage ST-1
    unroll_seq([&](auto i) { issue(i, min(static_cast<int>(decltype(i)::value), KT - 1)); },
               std::make_integer_sequence<int, ST - 1>{});
    wait_vm<(ST - 2) * PER_STAGE>();
    __builtin_amdgcn_s_barrier();
    issue(std::integral_constant<int, ST - 1>{}, min(ST - 1, KT - 1));
    read_frags(S0{}, R0{});
    // step s: stage s in register set s%2; S1N = stage of s+1
    // Each step is one basic block: the barrier, the direct loads of stage
    // s+ST and the fragment reads of stage s+1 are spread between the MFMAs of
    // stage s (scheduling groups of one load, its share of the reads and of
    // the MFMAs), so the LDS and memory traffic overlaps the matrix cores
    // instead of stalling them. After the last K step the barrier, loads and reads
    // still run (on buffers no step reads), which keeps the block branch-free.
    auto step = [&](auto set, auto next_st, auto refill_st, int kt) {
        using NSET = std::integral_constant<int, 1 - decltype(set)::value>;
        wait_lgkm0();
        wait_vm<(ST - 2) * PER_STAGE>();  // stage s+1 done (s+2 .. s+ST-1 may be in flight)
        __builtin_amdgcn_s_barrier();
        issue(refill_st, min(kt + ST, KT - 1));
        read_frags(next_st, NSET{});
        mfma_half(set, H0{});
        mfma_half(set, H1{});
        constexpr int READS = 2 * (FM + FN), MFMAS = 2 * FM * FN;
        if constexpr (READS % PER_STAGE == 0 && MFMAS % PER_STAGE == 0) {
#pragma unroll
            for (int q = 0; q < PER_STAGE; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                  // VMEM read (direct load)
                __builtin_amdgcn_sched_group_barrier(0x100, READS / PER_STAGE, 0);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, MFMAS / PER_STAGE, 0);  // MFMA
            }
        }
    };
    // step kt + I: register set I % 2, next stage (I + 1) % ST, refill stage I
    // (U = ST steps per loop pass, 2 ST when ST is odd, so the register sets alternate)
    auto step_i = [&](auto i, int kt) {
        constexpr int I = decltype(i)::value;
        step(std::integral_constant<int, I % 2>{}, std::integral_constant<int, (I + 1) % ST>{},
             std::integral_constant<int, I % ST>{}, kt + I);
    };
    constexpr int U = ST % 2 == 0 ? ST : 2 * ST;
    const int KTA = KT - KT % U;
    for (int kt = 0; kt < KTA; kt += U) unroll_seq([&](auto i) { step_i(i, kt); }, std::make_integer_sequence<int, U>{});
    unroll_seq([&](auto i) { if (KTA + decltype(i)::value < KT) step_i(i, KTA); }, std::make_integer_sequence<int, U - 1>{});
    // Every wave's direct loads and fragment reads are done before any wave
    // reuses the stage buffers below.
    wait_vm<0>();
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();

    // Epilogue. lane l holds column l%32 of each 32x32 fragment, rows
    // (e%4) + 4*(l/32) + 8*(e/4). Each fragment is scaled, written to an
    // HR x 40 f32 tile of the wave's own stage buffer (HR = 32 rows, or 16 in
    // two passes when the buffer is smaller), and read back 8 rows x 32
    // columns at a time, so every lane stores 16 contiguous bytes and eight
    // lanes fill a 128-byte row segment.
    constexpr int TS = 40;  // tile row stride in floats: 16-byte aligned rows, rows 4 apart 32 banks apart
    // waves 0-3 use stage buffers la0..la3, waves 4-7 lb0..lb3
    constexpr int BUF = WM * WN > 4 ? (BM < BN ? BM : BN) * kBK : BM * kBK;
    constexpr int HR = 32 * TS * 4 <= BUF ? 32 : 16;
    static_assert(HR * TS * 4 <= BUF, "epilogue tile fits a stage buffer");
    static_assert(WM * WN <= 8, "one stage buffer per wave");
    float* tile = reinterpret_cast<float*>(wave == 0 ? la0 : wave == 1 ? la1 : wave == 2 ? la2 : wave == 3 ? la3
                                           : wave == 4 ? lb0 : wave == 5 ? lb1 : wave == 6 ? lb2 : lb3);
    typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));  // scales and outputs: 4-byte alignment
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int rbase = m0 + wm * TM + i * 32 + 4 * (lane >> 5);
        float rs[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = rbase + 8 * q;
            if (r + 3 < m) {
                const f4u v = *reinterpret_cast<const f4u*>(a_scales + r);
                rs[4 * q] = v.x; rs[4 * q + 1] = v.y; rs[4 * q + 2] = v.z; rs[4 * q + 3] = v.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) rs[4 * q + e] = r + e < m ? a_scales[r + e] : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int c0 = n0 + wn * TN + j * 32;
            const float ws = w_scales[min(c0 + (lane & 31), n - 1)];
#pragma unroll
            for (int h = 0; h < 32 / HR; ++h) {
                // elements e of rows [h*HR, (h+1)*HR) are e in [h*HR/2, (h+1)*HR/2)
#pragma unroll
                for (int e = h * HR / 2; e < (h + 1) * HR / 2; ++e) {
                    const int lr = (e & 3) + 4 * (lane >> 5) + 8 * (e >> 2) - h * HR;
                    tile[lr * TS + (lane & 31)] = (static_cast<float>(acc[i][j][e]) * rs[e]) * ws;
                }
                // same wave: its LDS writes land before its reads, and its
                // reads before the next pass's writes
#pragma unroll
                for (int t = 0; t < HR / 8; ++t) {
                    const int lr = (lane >> 3) + 8 * t, lc = 4 * (lane & 7);
                    const f4u v = *reinterpret_cast<const f4u*>(tile + lr * TS + lc);
                    const int row = m0 + wm * TM + i * 32 + h * HR + lr, col = c0 + lc;
                    if (row < m) {
                        float* dst = out + static_cast<int64_t>(row) * ldo + col;
                        if (col + 3 < n) {
                            *reinterpret_cast<f4u*>(dst) = v;
                        } else {
                            if (col < n) dst[0] = v.x;
                            if (col + 1 < n) dst[1] = v.y;
                            if (col + 2 < n) dst[2] = v.z;
                        }
                    }
                }
            }
            if (out_i32) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = rbase + (e & 3) + 8 * (e >> 2), col = c0 + (lane & 31);
                    if (row < m && col < n) out_i32[static_cast<int64_t>(row) * ldo_i32 + col] = acc[i][j][e];
                }
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, int ST>
int launch_dma(const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw, const float* as,
               const float* ws, int m, int n, int k, float* out, int64_t ldo, int32_t* oi,
               int64_t ldoi, hipStream_t stream) {
    const int64_t tiles = static_cast<int64_t>((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    gemm_w8a8_dma_kernel<BM, BN, WM, WN, ST><<<dim3(static_cast<unsigned>(tiles)), dim3(WM * WN * 64), 0, stream>>>(
        a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi);
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

template <int BM, int BN, int WM, int WN>
int launch_cfg(const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw, const float* as,
               const float* ws, int m, int n, int k, float* out, int64_t ldo, int32_t* oi,
               int64_t ldoi, hipStream_t stream) {
    const int64_t tiles = static_cast<int64_t>((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    gemm_w8a8_kernel<BM, BN, WM, WN><<<dim3(static_cast<unsigned>(tiles)), dim3(WM * WN * 64), 0, stream>>>(
        a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi);
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace

int launch_gemm_w8a8_skinny(const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw, const float* as,
                            const float* ws, int m, int n, int k, float* out, int64_t ldo, int32_t* oi,
                            int64_t ldoi, hipStream_t stream);  // gemm_skinny.hip

// Tile choice by M. Up to 16 rows the weight-streaming kernel of
// gemm_skinny.hip (when the A8 rows fit its LDS), else the register-staged
// kernel (16/32 x 64 tiles) up to 32 rows; up to 256 rows small direct-load tiles, which for M = 128,
// N = 5632, K = 2048 take 10.3 us against 20.3 us for the register-staged
// 64x64 tile (the K loop's load latency, not the matrix cores, bounds these);
// beyond that 256x256 tiles when they make at least one per CU, else 128x128.
int launch_gemm_w8a8(const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw, const float* as,
                     const float* ws, int m, int n, int k, float* out, int64_t ldo, int32_t* oi,
                     int64_t ldoi, hipStream_t stream) {
    if (m <= 16) {
        const int st = launch_gemm_w8a8_skinny(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
        if (st != kStatusInvalid) return st;
        return launch_cfg<16, 64, 1, 4>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
    }
    if (m <= 32) return launch_cfg<32, 64, 1, 4>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
    if (m <= 64) return launch_dma<64, 32, 2, 1, 8>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
    if (m <= 128) return launch_dma<64, 64, 2, 2, 8>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
    if (m <= 256) return launch_dma<128, 64, 4, 1, 4>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
    const int64_t big_tiles = static_cast<int64_t>((m + 255) / 256) * ((n + 255) / 256);
    if (big_tiles >= 256) return launch_dma<256, 256, 2, 2, 4>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
    return launch_dma<128, 128, 2, 2, 4>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
}

}  // namespace rk
