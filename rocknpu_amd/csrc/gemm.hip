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
// owns a (BM/WM) x (BN/WN) sub-tile of 32x32 fragments of
// v_mfma_i32_32x32x32_i8. Operands reach LDS through a pipeline of stage
// buffers filled by direct global->LDS loads (below). Up to 16 rows the
// weight-streaming kernel of gemm_skinny.hip runs instead.
#include "common.h"

#include <algorithm>
#include <atomic>
#include <cstring>
#include <type_traits>
#include <utility>

namespace rk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Direct-load tiles: the same product with a pipeline of ST (2 to 8) LDS
// stage buffers filled by direct global->LDS loads (global_load_lds_dwordx4,
// no register staging). A stage holds KB (64 or 128) bytes of K per row. Each
// wave issues its share of a stage as 1 KiB segments (1024 / KB rows of KB
// bytes; lane i's 16 bytes land at segment + 16*i, so the lane loads the
// global chunk that the swizzled layout puts there). Stage s+ST-1 is issued
// while stage s is multiplied; one barrier per stage both publishes stage s+1
// (after each wave's own wait for its loads) and frees stage s for reuse. The
// barrier is a bare s_barrier: a fenced one would wait for every load in
// flight, stages ahead included.
template <int BM, int BN, int WM, int WN, int KB>
struct DmaTile {
    static constexpr int T = WM * WN * 64;
    static constexpr int W = WM * WN;
    // 1 KiB segments (RPI rows of KB bytes) per wave and stage. When a tile
    // has fewer segments than waves, waves load segments twice (the same
    // bytes to the same LDS place), so every wave issues the same number of
    // loads.
    static constexpr int RPI = 1024 / KB;
    static constexpr int A_ROWSEG = BM / RPI, B_ROWSEG = BN / RPI;
    static constexpr int A_SEG = A_ROWSEG >= W ? A_ROWSEG / W : 1, B_SEG = B_ROWSEG >= W ? B_ROWSEG / W : 1;
    static_assert(BM % RPI == 0 && BN % RPI == 0, "tile rows must split into whole segments");
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

// Stage layout of the direct-load tiles: rows of KB bytes (64 or 128), the
// 16-byte chunks XOR-swizzled by row / 2, so the fragment reads (32 rows,
// one chunk column per half wave) do not collide in the LDS banks.
template <int KB>
__device__ __forceinline__ int swz_kb(int r, int kc) { return r * KB + ((kc ^ ((r >> 1) & (KB / 16 - 1))) << 4); }

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

// Split-K (SK): the grid holds `splits` workgroups per tile, workgroup s of a
// tile taking K bytes [s * k_split, (s + 1) * k_split). Each writes its i32
// partial tile to `partials` in the accumulator layout (lane-contiguous, so
// every store is a full 256-byte row) and its arrival stamp (the launch's
// generation `gen`, never 0), then counts itself in at the tile's counter; the
// last to arrive adds the other partials to its own (int32 addition: exact and
// order-free), runs the epilogue, and resets the tile's stamps and counter to
// zero, so a workspace that starts zeroed ends every call zeroed.
//
// A counter that was not zero at entry (a workspace never zeroed, a call that
// did not complete, two calls overlapping on one workspace) is detected rather
// than trusted: an arrival that finds the count at or above `splits`, or a
// last arrival that finds another split's stamp different from `gen`, writes
// NaN for the tile's f32 results and sets the workspace's sticky error word
// (rocknpu_hip_gemm_workspace_check reads and clears it).
//
// Memory ordering. A tile's splits can run on different XCDs (at the edges of
// an XCD's range of the bid mapping below), and each XCD has its own L2, so
// the exchange must bypass those L2s. The partials, stamps and counters are
// relaxed agent-scope atomics: gfx950 compiles these stores and loads with
// the sc1 bit, which writes through to and reads from the device-coherent
// level past the XCD's L2. Each wave then waits for its own stores to complete
// (s_waitcnt vmcnt(0): on gfx9 stores count in vmcnt) before the workgroup
// barrier and the relaxed fetch_add that counts it in. That ordering is a
// property of how gfx950 lowers these operations, not of the HIP memory model
// (which would need release/acquire); it is checked on gfx950 only, and
// gemm_split_supported() keeps every other architecture unsplit. A
// device-scope fence instead would write back and invalidate the whole L2 of
// the XCD, which cost 50 us per launch at 352 workgroups.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the K-split exchange of gemm_w8a8_dma_kernel is checked on gfx950 only"
#endif
template <int BM, int BN, int WM, int WN, int ST, int KB, bool SK>
__global__ __launch_bounds__(WM* WN * 64) void gemm_w8a8_dma_kernel(
    const int8_t* __restrict__ a8, int64_t lda, const int8_t* __restrict__ w8, int64_t ldw, int m, int n, int k,
    int splits, int k_split, const float* __restrict__ a_scales, const float* __restrict__ w_scales,
    float* __restrict__ out, int64_t ldo, int32_t* __restrict__ out_i32, int64_t ldo_i32,
    int32_t* __restrict__ partials, uint32_t* __restrict__ counters, uint32_t* __restrict__ stamps, uint32_t gen) {
    using Cfg = DmaTile<BM, BN, WM, WN, KB>;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 fragments
    // A stage holds KB bytes of K (64, or 128: whole 128-byte lines per row,
    // which the L2 serves at twice the rate of half lines) and is consumed
    // in SUB sub-steps of 64.
    static_assert(KB == 64 || KB == 128, "64- or 128-byte stages");
    constexpr int SUB = KB / 64;
    // One array per stage, always indexed by a compile-time stage: the
    // wait-count pass then sees which LDS buffer a direct load writes and does
    // not wait for every load in flight before each LDS read.
    // ST = 2..8 stages; arrays of stages >= ST are unused placeholders.
    static_assert(ST >= 2 && ST <= 8, "two to eight stage buffers");
    constexpr int A2 = ST > 2 ? BM * KB : 16, A3 = ST > 3 ? BM * KB : 16;
    constexpr int B2 = ST > 2 ? BN * KB : 16, B3 = ST > 3 ? BN * KB : 16;
    constexpr int A4 = ST > 4 ? BM * KB : 16, A5 = ST > 5 ? BM * KB : 16, A6 = ST > 6 ? BM * KB : 16,
                  A7 = ST > 7 ? BM * KB : 16;
    constexpr int B4 = ST > 4 ? BN * KB : 16, B5 = ST > 5 ? BN * KB : 16, B6 = ST > 6 ? BN * KB : 16,
                  B7 = ST > 7 ? BN * KB : 16;
    __shared__ __align__(16) int8_t la0[BM * KB], la1[BM * KB], la2[A2], la3[A3];
    __shared__ __align__(16) int8_t lb0[BN * KB], lb1[BN * KB], lb2[B2], lb3[B3];
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
    // With split-K the (tile, split) pairs are ordered tile-major, so most of
    // a tile's splits run on one XCD; a tile whose splits straddle the end of
    // an XCD's range has them on two, which is why the exchange above goes
    // past the L2s.
    const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
    const int tiles = tiles_m * tiles_n;
    const int total = SK ? tiles * splits : tiles;
    const int bid = blockIdx.x, xcd = bid & 7, per = total >> 3, rem = total & 7;
    const int v = xcd * per + min(xcd, rem) + (bid >> 3);
    const int t = SK ? v / splits : v;
    const int split = SK ? v - t * splits : 0;
    if constexpr (SK) {
        // this split's K range: operands start k0 bytes in, k bytes long
        const int k0 = split * k_split;
        a8 += k0;
        w8 += k0;
        k = min(k - k0, k_split);
    }
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
    // lane l fills the 16 bytes at segment + 16 l: row l / CPR of the
    // segment, swizzled chunk position l % CPR, so it loads the chunk whose
    // swizzled place that is
    constexpr int CPR = KB / 16;  // chunks per row
#pragma unroll
    for (int q = 0; q < Cfg::A_SEG; ++q) {
        const int r = ((wave * Cfg::A_SEG + q) % Cfg::A_ROWSEG) * Cfg::RPI + lane / CPR;
        const int c = (lane % CPR) ^ ((r >> 1) & (CPR - 1));
        asrc[q] = a8 + static_cast<int64_t>(min(m0 + r, m - 1)) * lda + c * 16;
    }
#pragma unroll
    for (int q = 0; q < Cfg::B_SEG; ++q) {
        const int r = ((wave * Cfg::B_SEG + q) % Cfg::B_ROWSEG) * Cfg::RPI + lane / CPR;
        const int c = (lane % CPR) ^ ((r >> 1) & (CPR - 1));
        bsrc[q] = w8 + static_cast<int64_t>(min(n0 + r, n - 1)) * ldw + c * 16;
    }
    // stage number ks (K bytes ks*KB ..) into stage buffer st
    auto issue = [&](auto st, int ks) {
        int8_t* la = stage_a(st);
        int8_t* lb = stage_b(st);
#pragma unroll
        for (int q = 0; q < Cfg::A_SEG; ++q)
            dma16(asrc[q] + ks * KB, la + ((wave * Cfg::A_SEG + q) % Cfg::A_ROWSEG) * 1024);
#pragma unroll
        for (int q = 0; q < Cfg::B_SEG; ++q)
            dma16(bsrc[q] + ks * KB, lb + ((wave * Cfg::B_SEG + q) % Cfg::B_ROWSEG) * 1024);
    };

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16i{};

    const int KS = k / KB;  // stages
    const int KT = k / 64;  // 64-deep steps
    using S0 = std::integral_constant<int, 0>;
    // Pipeline per 64-deep K step j (its fragments were read in step j-1):
    //   wait for those reads. When j is the last step of its stage P: wait
    //   for this wave's loads of stage P+1 and pass a barrier (every wave's
    //   stage P+1 is in, and every wave holds all of stage P in registers, so
    //   its buffer is free), then issue stage P+ST into that buffer.
    //   Read step j+1's fragments into the other register set; then the MFMAs
    //   of step j, which run while those reads complete.
    // Past the last stage the issue re-reads the last stage into a buffer no
    // step reads, so the count of loads in flight stays fixed.
    constexpr int PER_STAGE = Cfg::A_SEG + Cfg::B_SEG;  // loads per wave and stage
    v4i fa[2][2][FM], fb[2][2][FN];  // [register set][32-deep half][fragment]
    // step sub-step u of a stage: lane l supplies row l%32 and the 16 bytes of
    // chunk 4u + 2h + l/32
    auto read_half = [&](auto st, auto set, auto u, auto half) {
        constexpr int R = decltype(set)::value, H = decltype(half)::value, SU = decltype(u)::value;
        const int8_t* la = stage_a(st);
        const int8_t* lb = stage_b(st);
#pragma unroll
        for (int i = 0; i < FM; ++i)
            fa[R][H][i] = *reinterpret_cast<const v4i*>(
                la + swz_kb<KB>(wm * TM + i * 32 + (lane & 31), 4 * SU + 2 * H + (lane >> 5)));
#pragma unroll
        for (int j = 0; j < FN; ++j)
            fb[R][H][j] = *reinterpret_cast<const v4i*>(
                lb + swz_kb<KB>(wn * TN + j * 32 + (lane & 31), 4 * SU + 2 * H + (lane >> 5)));
    };
    using H0 = std::integral_constant<int, 0>;
    using H1 = std::integral_constant<int, 1>;
    auto read_frags = [&](auto st, auto set, auto u) {
        read_half(st, set, u, H0{});
        read_half(st, set, u, H1{});
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
    // The epilogue's scales: lane rows' a_scales (16 per 32-row fragment) and
    // its column's w_scale per 32-column fragment. Small tiles (at most one
    // row and two column fragments a wave: 17-18 registers) load them here,
    // before the first stage: older than every stage load, so the stages'
    // in-order wait counts stay exact, and the epilogue does not open with a
    // memory round trip (TinyLlama down at 128 tokens, 128 x 2048 x 5632 in
    // two K splits: 11.2 -> 10.8 us; config 0, 128 x 5632 x 2048: 8.20 ->
    // 8.15 us; 512 x 2048 x 5632: 15.6 -> 15.4 us).
    constexpr bool PRE = FM * 16 + FN <= 24;
    auto load_rs = [&](int i, float (&rs)[16]) {
        const int rbase = m0 + wm * TM + i * 32 + 4 * (lane >> 5);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = rbase + 8 * q;
            if (r + 3 < m) {
                typedef float f4s __attribute__((ext_vector_type(4), aligned(4)));
                const f4s v = *reinterpret_cast<const f4s*>(a_scales + r);
                rs[4 * q] = v.x; rs[4 * q + 1] = v.y; rs[4 * q + 2] = v.z; rs[4 * q + 3] = v.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) rs[4 * q + e] = r + e < m ? a_scales[r + e] : 0.0f;
            }
        }
    };
    auto load_ws = [&](int j) { return w_scales[min(n0 + wn * TN + j * 32 + (lane & 31), n - 1)]; };
    float rs_pre[PRE ? FM : 1][16];
    float ws_pre[PRE ? FN : 1];
    if constexpr (PRE) {
#pragma unroll
        for (int i = 0; i < FM; ++i) load_rs(i, rs_pre[i]);
#pragma unroll
        for (int j = 0; j < FN; ++j) ws_pre[j] = load_ws(j);
    }
    // Larger tiles have no registers to spare: each thread loads one or two
    // of the tile's BM + BN scales here (rows and columns past the matrix
    // re-read its last one; they are never stored), and writes them to LDS
    // once the first stage has landed (the loads are older, so they have
    // too); the K loop's barriers publish them, and the epilogue reads them
    // from LDS.
    constexpr int NSC = BM + BN, THREADS = WM * WN * 64, SCP = PRE ? 1 : (NSC + THREADS - 1) / THREADS;
    __shared__ float lsc[PRE ? 1 : NSC];
    float scv[SCP];
    if constexpr (!PRE) {
#pragma unroll
        for (int u = 0; u < SCP; ++u) {
            const int idx = threadIdx.x + u * THREADS;
            scv[u] = idx < BM ? a_scales[min(m0 + idx, m - 1)] : w_scales[min(n0 + min(idx, NSC - 1) - BM, n - 1)];
        }
    }
    // prologue: stages 0 .. ST-2 in flight, wait for stage 0, then stage ST-1
    unroll_seq([&](auto i) { issue(i, min(static_cast<int>(decltype(i)::value), KS - 1)); },
               std::make_integer_sequence<int, ST - 1>{});
    wait_vm<(ST - 2) * PER_STAGE>();
    if constexpr (!PRE) {
#pragma unroll
        for (int u = 0; u < SCP; ++u) {
            const int idx = threadIdx.x + u * THREADS;
            if (idx < NSC) lsc[idx] = scv[u];
        }
    }
    __builtin_amdgcn_s_barrier();
    issue(std::integral_constant<int, ST - 1>{}, min(ST - 1, KS - 1));
    read_frags(S0{}, R0{}, S0{});
    // Each step is one basic block: the barrier, the direct loads of stage
    // P+ST and the fragment reads of step j+1 are spread between the MFMAs of
    // step j (scheduling groups of one load, its share of the reads and of
    // the MFMAs), so the LDS and memory traffic overlaps the matrix cores
    // instead of stalling them. After the last step the barrier, loads and
    // reads still run (on buffers no step reads), which keeps the block
    // branch-free.
    auto step = [&](auto set, auto next_st, auto next_u, auto refill_st, auto last_of_stage, int p) {
        using NSET = std::integral_constant<int, 1 - decltype(set)::value>;
        constexpr bool LAST = decltype(last_of_stage)::value;
        wait_lgkm0();
        if constexpr (LAST) {
            wait_vm<(ST - 2) * PER_STAGE>();  // stage P+1 done (P+2 .. P+ST-1 may be in flight)
            __builtin_amdgcn_s_barrier();
            issue(refill_st, min(p + ST, KS - 1));
        }
        read_frags(next_st, NSET{}, next_u);
        mfma_half(set, H0{});
        mfma_half(set, H1{});
        constexpr int READS = 2 * (FM + FN), MFMAS = 2 * FM * FN;
        if constexpr (LAST && READS % PER_STAGE == 0 && MFMAS % PER_STAGE == 0) {
#pragma unroll
            for (int q = 0; q < PER_STAGE; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                  // VMEM read (direct load)
                __builtin_amdgcn_sched_group_barrier(0x100, READS / PER_STAGE, 0);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, MFMAS / PER_STAGE, 0);  // MFMA
            }
        } else if constexpr (!LAST && MFMAS % READS == 0) {
#pragma unroll
            for (int q = 0; q < READS; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);             // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, MFMAS / READS, 0);  // MFMA
            }
        }
    };
    // step kt + I: register set I % 2; stage buffer (I / SUB) % ST, sub-step
    // I % SUB; the next step's buffer and sub-step; the last step of a stage
    // refills that stage's buffer. U steps per loop pass: a multiple of
    // ST * SUB and of 2, so buffers and register sets repeat.
    auto step_i = [&](auto i, int kt) {
        constexpr int I = decltype(i)::value;
        step(std::integral_constant<int, I % 2>{}, std::integral_constant<int, ((I + 1) / SUB) % ST>{},
             std::integral_constant<int, (I + 1) % SUB>{}, std::integral_constant<int, (I / SUB) % ST>{},
             std::integral_constant<bool, (I + 1) % SUB == 0>{}, (kt + I) / SUB);
    };
    constexpr int U = (ST * SUB) % 2 == 0 ? ST * SUB : 2 * ST * SUB;
    const int KTA = KT - KT % U;
    for (int kt = 0; kt < KTA; kt += U) unroll_seq([&](auto i) { step_i(i, kt); }, std::make_integer_sequence<int, U>{});
    unroll_seq([&](auto i) { if (KTA + decltype(i)::value < KT) step_i(i, KTA); }, std::make_integer_sequence<int, U - 1>{});
    // Every wave's direct loads and fragment reads are done before any wave
    // reuses the stage buffers below.
    wait_vm<0>();
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();

    bool poison = false;  // this tile's counters were dirty: its f32 results are NaN
    if constexpr (SK) {
        constexpr int PART = FM * FN * 16 * 64;  // ints of one wave's partial
        __shared__ int verdict;                  // 0: not last, 1: last, 2: dirty counters
        int32_t* mine = partials + (static_cast<int64_t>(t) * splits + split) * (WM * WN * PART) + wave * PART;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    __hip_atomic_store(mine + ((i * FN + j) * 16 + e) * 64 + lane, acc[i][j][e], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        // every wave's partial has reached the device-coherent level before the count
        wait_vm<0>();
        __syncthreads();
        uint32_t* tile_stamps = stamps + static_cast<int64_t>(t) * splits;
        if (threadIdx.x == 0) {
            __hip_atomic_store(tile_stamps + split, gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wait_vm<0>();  // the stamp, like the partials, lands before the count
            const uint32_t old = __hip_atomic_fetch_add(counters + t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            int v = old == static_cast<uint32_t>(splits - 1) ? 1 : old >= static_cast<uint32_t>(splits) ? 2 : 0;
            if (v == 1)  // every split of this call has counted in, or the count started dirty
                for (int s2 = 0; s2 < splits; ++s2)
                    if (__hip_atomic_load(tile_stamps + s2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != gen) v = 2;
            if (v == 2)
                __hip_atomic_store(counters + kSplitErrorWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            verdict = v;
        }
        __syncthreads();
        const int v = verdict;
        if (v == 0) return;
        poison = v == 2;
        if (!poison) {
            // the other splits counted in after their partials completed; read
            // them at device scope (past this XCD's L2)
            for (int s2 = 0; s2 < splits; ++s2) {
                if (s2 == split) continue;
                int32_t* other =
                    partials + (static_cast<int64_t>(t) * splits + s2) * (WM * WN * PART) + wave * PART;
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            acc[i][j][e] += __hip_atomic_load(other + ((i * FN + j) * 16 + e) * 64 + lane,
                                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            // a dirty tile keeps its state, so every later call on the
            // workspace reports it until the caller zeroes the workspace
            if (threadIdx.x < splits)
                __hip_atomic_store(tile_stamps + threadIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (threadIdx.x == 0) __hip_atomic_store(counters + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    // Epilogue. lane l holds column l%32 of each 32x32 fragment, rows
    // (e%4) + 4*(l/32) + 8*(e/4). Each fragment is scaled, written to an
    // HR x 40 f32 tile of the wave's own stage buffer (HR = 32 rows, or 16 in
    // two passes when the buffer is smaller), and read back 8 rows x 32
    // columns at a time, so every lane stores 16 contiguous bytes and eight
    // lanes fill a 128-byte row segment.
    constexpr int TS = 40;  // tile row stride in floats: 16-byte aligned rows, rows 4 apart 32 banks apart
    // With four or more stages, waves 0-3 use stage buffers la0..la3 and
    // waves 4-7 lb0..lb3; with fewer, the first half of the waves' tiles sit
    // side by side in la0 and the rest in lb0.
    constexpr int W = WM * WN, WH = (W + 1) / 2;
    constexpr int BUF = ST >= 4 ? (W > 4 ? (BM < BN ? BM : BN) * KB : BM * KB) : (BM < BN ? BM : BN) * KB / WH;
    constexpr int HR = 32 * TS * 4 <= BUF ? 32 : 16;
    static_assert(HR * TS * 4 <= BUF && BUF % 16 == 0, "epilogue tile fits its buffer");
    static_assert(ST < 4 || W <= 8, "one stage buffer per wave");
    float* tile;
    if constexpr (ST >= 4)
        tile = reinterpret_cast<float*>(wave == 0 ? la0 : wave == 1 ? la1 : wave == 2 ? la2 : wave == 3 ? la3
                                        : wave == 4 ? lb0 : wave == 5 ? lb1 : wave == 6 ? lb2 : lb3);
    else
        tile = reinterpret_cast<float*>(wave < WH ? la0 + wave * BUF : lb0 + (wave - WH) * BUF);
    typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));  // scales and outputs: 4-byte alignment
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int rbase = m0 + wm * TM + i * 32 + 4 * (lane >> 5);
        float rs[16];
        if constexpr (PRE) {
#pragma unroll
            for (int e = 0; e < 16; ++e) rs[e] = rs_pre[i][e];
        } else {
            // row rbase + (e & 3) + 8 (e >> 2) of the tile's scales in LDS
#pragma unroll
            for (int e = 0; e < 16; ++e) rs[e] = lsc[rbase - m0 + (e & 3) + 8 * (e >> 2)];
        }
        if constexpr (SK)
            if (poison)
#pragma unroll
                for (int e = 0; e < 16; ++e) rs[e] = __builtin_nanf("");
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int c0 = n0 + wn * TN + j * 32;
            const float ws = PRE ? ws_pre[PRE ? j : 0] : lsc[PRE ? 0 : BM + wn * TN + j * 32 + (lane & 31)];
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
                            // streamed once: non-temporal, so the output does not
                            // evict operand lines from L2 (4096 x 14336 x 4096:
                            // 275 -> 260 us)
                            __builtin_nontemporal_store(v, reinterpret_cast<f4u*>(dst));
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

// Splits that get K stages when `splits` are asked for over `ks` stages, and
// the stages of each (the last may have fewer).
struct SplitK {
    int splits, stages_per;
};
SplitK split_k(int ks, int splits) {
    if (splits <= 1 || ks <= 1) return {1, ks};
    const int per = (ks + splits - 1) / splits;
    return {(ks + per - 1) / per, per};
}

template <int BM, int BN, int WM, int WN, int ST, int KB = 64>
int launch_dma(const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw, const float* as,
               const float* ws, int m, int n, int k, float* out, int64_t ldo, int32_t* oi,
               int64_t ldoi, int splits, uint8_t* workspace, hipStream_t stream) {
    // 128-byte stages need K % 128 == 0 (a stage never reads past a row)
    if constexpr (KB != 64)
        if (k % KB != 0) {
            if constexpr (BM >= 64)
                return launch_dma<BM, BN, WM, WN, (ST < 4 ? 4 : ST), 64>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo,
                                                                         oi, ldoi, splits, workspace, stream);
            else
                return kStatusInvalid;
        }
    const int64_t tiles = static_cast<int64_t>((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    const SplitK sk =
        split_k(k / KB, workspace && tiles <= kSplitCounters && gemm_split_supported() ? splits : 1);
    if (sk.splits > 1) {
        uint32_t* counters = reinterpret_cast<uint32_t*>(workspace);
        int32_t* partials = reinterpret_cast<int32_t*>(workspace + kSplitCounterBytes);
        uint32_t* stamps = reinterpret_cast<uint32_t*>(partials + tiles * sk.splits * BM * BN);
        gemm_w8a8_dma_kernel<BM, BN, WM, WN, ST, KB, true>
            <<<dim3(static_cast<unsigned>(tiles * sk.splits)), dim3(WM * WN * 64), 0, stream>>>(
                a8, lda, w8, ldw, m, n, k, sk.splits, sk.stages_per * KB, as, ws, out, ldo, oi, ldoi, partials,
                counters, stamps, next_split_generation());
    } else {
        gemm_w8a8_dma_kernel<BM, BN, WM, WN, ST, KB, false><<<dim3(static_cast<unsigned>(tiles)), dim3(WM * WN * 64), 0,
                                                              stream>>>(a8, lda, w8, ldw, m, n, k, 1, k, as, ws,
                                                                        out, ldo, oi, ldoi, nullptr, nullptr, nullptr,
                                                                        0);
    }
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace

// The generation a split launch stamps its arrivals with: distinct for every
// launch of the process (until it wraps after 2^32 - 1 of them), never 0,
// which is what a zeroed or reset stamp holds.
uint32_t next_split_generation() {
    static std::atomic<uint32_t> gen{0};
    uint32_t g = gen.fetch_add(1, std::memory_order_relaxed) + 1;
    while (g == 0) g = gen.fetch_add(1, std::memory_order_relaxed) + 1;
    return g;
}

int launch_gemm_w8a8_skinny(const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw, const float* as,
                            const float* ws, int m, int n, int k, float* out, int64_t ldo, int32_t* oi,
                            int64_t ldoi, hipStream_t stream);  // gemm_skinny.hip
GemmTile gemm_tile(int m, int n, int k, int cus);

// Tile and stage count of the GEMM for an M x N x K product on `cus` CUs
// (bm = 0: the weight-streaming kernel of gemm_skinny.hip). "Fits" below
// means the tiles number at most the CUs: one round, one workgroup per CU.
//
// Stages: 2 where tiles outnumber the CUs (two workgroups share a CU, so the
// extra tiles do not wait for a second round), else 4 (a deeper pipeline);
// M = 256, N = 4096, K = 14336 (128 tiles) takes 49 us with four against 86
// with two, M = 256, N = 11264, K = 2048 (352 tiles) 19.7 us with two against
// 21.8 with four. 128-byte stages read whole 128-byte lines of each row, which
// the L2 serves at about twice the rate of half lines (4096 x 14336 x 4096:
// 284 -> 272 us; 512 x 11264 x 2048: 31.5 -> 25.7 us).
//
// By M (times on MI355X):
// - <= 16: the weight-streaming kernel while its A8 rows fit its LDS.
// - <= 64: 64 x 32 tiles with four stages when they fit (for M = 32, N =
//   5632, K = 2048 they take 7.6 us against 18.5 us for register-staged 32 x
//   64 tiles). Else, up to 32 rows (K % 128 == 0), 32 x 64 direct-load tiles
//   with four stages: half the activation rows per tile (32 x 28672 x 4096:
//   31.8 -> 28.4 us; 17 x 32000 x 2048 18.4 -> 15.7; 32 x 11264 x 2048 8.6
//   -> 8.2; 17 x 32000 x 2048 against 64 x 64 tiles 16.1 against 16.9 us);
//   from 33 rows 64 x 64 tiles, four stages while they are at most 1.75 per
//   CU (64 x 28672 x 4096, 448 tiles: 34.5 -> 31.1 us), else two (64 x 32000
//   x 2048, 500 tiles: 17.9 against 19.2 us with four; 64 x 128256 x 2048:
//   77.3 -> 62.0 us).
// - <= 128: 128 x 64 with four stages when 64 x 64 tiles do not fit but those
//   do (128 x 11264 x 2048: 15.5 -> 11.8 us); 128 x 128 with three stages when
//   64 x 64 tiles would be more than three per CU, 128 x 64 tiles do not fit
//   and those do (the TinyLlama head, 128 x 32000 x 2048: 28.4 -> 23.8 us with
//   1000 64 x 64 tiles against 250), two per CU when they do not fit either
//   (the Llama-3.2-1B head, 128 x 128256 x 2048: 95.6 -> 71.3 us against 64 x
//   64 tiles two per CU); else the filling choice without 128-row tiles.
// - <= 256: 128 x 128 with three stages when 128 x 64 tiles do not fit but
//   those do (256 x 11264 x 2048: 19.1 -> 15.5 us); the rules below when
//   128 x 128 tiles do not fit (256 x 28672 x 2048 on 256 x 128 tiles: 40.8 ->
//   22.6 us; 256 x 128256 x 2048 on 256 x 256: 138.7 -> 90.5); else the
//   filling choice.
// - above, with a 256 x 256 tile per CU: 256 x 256 tiles, or 256 x 128 tiles
//   with eight waves and three stages when their rounds cost less (a round of
//   them takes about 0.61 of a round of 256 x 256 tiles; 2048 x 11264 x 2048:
//   76.6 -> 71.8 us).
// - above, when 128 x 128 tiles do not fit: 256 x 128 tiles (eight waves,
//   three stages) if they fit (512 x 11264 x 2048: 27.2 -> 23.6 us); else
//   256 x 256 tiles when their rounds cost less than two-per-CU rounds of
//   128 x 128 tiles (a round takes about 1.38 of one; 1024 x 14336 x 4096:
//   93 -> 80 us); else 128 x 128 tiles, two per CU.
// - else the filling choice: the first of 64 x 32, 64 x 64 and 128 x 64 that
//   fits, then 128 x 128 with three stages, else 128 x 64 two per CU
//   (512 x 2048 x 5632: 21.9 -> 16.5 us; 1024 x 2560 x 4096: 29.9 -> 23.5 us).
// Tiles that need a second round where smaller or larger ones fit in one
// measured slower, which is why each rule asks for one round. Above 256 rows,
// launch_gemm_w8a8 first checks gemm_column_split, which can run a product
// as two launches (whole rounds of 256 x 256 tiles, then the rest routed by
// these rules).
//
// K split (with a workspace): when the chosen tiles are at most 64 x 64 and
// fill at most half the CUs, each tile's K range is split over
// min(cus / tiles, stages / 10, 3) workgroups, so the units fill the CUs with
// at least 10 stages each: K of 4096 and more (128 x 2048 x 4096: 10.9 ->
// 10.2 us; 128 x 2048 x 5632: 13.6 -> 11.7; 128 x 2048 x 8192: 18.0 -> 13.8;
// 32 x 2048 x 5632 in three: 13.2 -> 10.5), but not 2048 (128 x 2048 x 2048:
// 6.6 unsplit against 8.0 in two; 32 x 2560 x 2048: 7.3 against 8.4), and
// at most three (32 x 2560 x 4096: 9.8 against 10.6 in four). Larger tiles,
// and tiles filling more than half the CUs, measured slower split (128 x 5632
// x 2048 on 176 64 x 64 tiles: 8.4 -> 12.0 us at two splits; 1024 x 8192 x
// 4096 on 128 256 x 256 tiles: 58.5 -> 63.9 us).
GemmTile gemm_route(int m, int n, int k, int cus) {
    GemmTile r = gemm_tile(m, n, k, cus);
    if (r.bm == 0 || r.bm * r.bn > 64 * 64) return r;
    const int64_t tiles = static_cast<int64_t>((m + r.bm - 1) / r.bm) * ((n + r.bn - 1) / r.bn);
    const int stages = k % 128 == 0 ? k / 128 : k / 64;
    if (2 * tiles > cus || tiles > kSplitCounters) return r;
    const int s = static_cast<int>(std::min<int64_t>(std::min(cus / tiles, static_cast<int64_t>(stages / 10)), 3));
    if (s >= 2) r.splits = s;
    return r;
}

// The tile and stage count (no split) of gemm_route.
GemmTile gemm_tile(int m, int n, int k, int cus) {
    auto tiles = [&](int bm, int bn) { return static_cast<int64_t>((m + bm - 1) / bm) * ((n + bn - 1) / bn); };
    auto by_tiles = [&](int bm, int bn) { return GemmTile{bm, bn, tiles(bm, bn) > cus ? 2 : 4}; };
    auto rounds = [&](int64_t t, int per_cu) { return (t + per_cu * cus - 1) / (per_cu * cus); };
    auto filling = [&](bool allow_128) {
        if (tiles(64, 32) <= cus) return GemmTile{64, 32, 4};
        if (!allow_128 || tiles(64, 64) <= cus) return by_tiles(64, 64);
        if (tiles(128, 64) > cus && tiles(128, 128) <= cus) return GemmTile{128, 128, 3};
        return by_tiles(128, 64);
    };
    if (m <= 16 && k % 64 == 0 && static_cast<int64_t>(m) * k <= kSkinnyMaxA8) return GemmTile{0, 0, 0};
    if (m <= 64) {
        if (tiles(64, 32) <= cus) return GemmTile{64, 32, 4};
        if (m <= 32 && k % 128 == 0) return GemmTile{32, 64, 4};
        if (4 * tiles(64, 64) <= 7 * static_cast<int64_t>(cus)) return GemmTile{64, 64, 4};
        return GemmTile{64, 64, 2};
    }
    if (m <= 128) {
        if (tiles(64, 64) > cus && tiles(128, 64) <= cus) return GemmTile{128, 64, 4};
        if (tiles(64, 64) > 3 * cus && tiles(128, 64) > cus)
            return GemmTile{128, 128, tiles(128, 128) <= cus ? 3 : 2};
        return filling(false);
    }
    if (m <= 256) {
        if (tiles(128, 64) > cus && tiles(128, 128) <= cus) return GemmTile{128, 128, 3};
        // 128 x 128 tiles that do not fit: the rules of longer products below
        if (tiles(128, 128) <= cus) return filling(true);
    }
    if (tiles(256, 256) >= cus) {
        if (rounds(tiles(256, 128), 1) * 61 < rounds(tiles(256, 256), 1) * 100) return GemmTile{256, 128, 3};
        return GemmTile{256, 256, 2};
    }
    if (tiles(128, 128) > cus) {
        if (tiles(256, 128) <= cus) return GemmTile{256, 128, 3};
        if (rounds(tiles(256, 256), 1) * 138 < rounds(tiles(128, 128), 2) * 100) return GemmTile{256, 256, 2};
        return GemmTile{128, 128, 2};
    }
    return filling(true);
}

int gemm_workspace_counters(const GemmTile& tile, int m, int n) {
    if (tile.bm == 0 || tile.splits <= 1) return 0;
    return ((m + tile.bm - 1) / tile.bm) * ((n + tile.bn - 1) / tile.bn);
}

size_t gemm_workspace_bytes(const GemmTile& tile, int m, int n) {
    const size_t tiles = static_cast<size_t>(gemm_workspace_counters(tile, m, n));
    if (tiles == 0) return 0;
    const size_t units = tiles * tile.splits;
    // counter block, i32 partial tiles, one stamp per unit (256-byte rounded)
    return kSplitCounterBytes + units * tile.bm * tile.bn * 4 + (units * 4 + 255) / 256 * 256;
}

bool gemm_split_supported() {
    static std::atomic<int> cached[64] = {};  // 0 unknown, 1 yes, 2 no (host threads may ask at once)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        hipDeviceProp_t prop{};
        const bool ok = hipGetDeviceProperties(&prop, dev) == hipSuccess &&
                        std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 &&
                        (prop.gcnArchName[6] == '\0' || prop.gcnArchName[6] == ':');
        v = ok ? 1 : 2;
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v == 1;
}

// The GEMM on a given tile, stage count and split (splits > 1 needs a
// workspace of gemm_workspace_bytes(r, m, n) whose counters are zero; else it
// runs unsplit).
int launch_gemm_w8a8_tile(const GemmTile& r, const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw,
                          const float* as, const float* ws, int m, int n, int k, float* out, int64_t ldo,
                          int32_t* oi, int64_t ldoi, uint8_t* workspace, hipStream_t stream) {
    const int sp = r.splits;
#define RK_GEMM(BM, BN, WM, WN, ST) \
    launch_dma<BM, BN, WM, WN, ST, 128>(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, sp, workspace, stream)
    if (r.bm == 0) return launch_gemm_w8a8_skinny(a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, stream);
    if (r.bm == 32 && r.bn == 64) return RK_GEMM(32, 64, 1, 2, 4);
    if (r.bm == 64 && r.bn == 32) return r.stages == 2 ? RK_GEMM(64, 32, 2, 1, 2) : RK_GEMM(64, 32, 2, 1, 4);
    if (r.bm == 64) return r.stages == 2 ? RK_GEMM(64, 64, 2, 2, 2) : RK_GEMM(64, 64, 2, 2, 4);
    if (r.bm == 128 && r.bn == 64) return r.stages == 2 ? RK_GEMM(128, 64, 4, 1, 2) : RK_GEMM(128, 64, 4, 1, 4);
    if (r.bm == 128) return r.stages == 2 ? RK_GEMM(128, 128, 2, 2, 2) : RK_GEMM(128, 128, 2, 2, 3);
    if (r.bn == 128) return RK_GEMM(256, 128, 4, 2, 3);
    return RK_GEMM(256, 256, 2, 2, 2);
#undef RK_GEMM
}

// Column split: when the 256 x 256 tiles of an M > 256 product make one or
// more whole rounds on the CUs plus a last round at most half full, the
// columns of those whole rounds run as one launch of 256 x 256 tiles and the
// rest as a second, routed launch of its own (smaller tiles that fill the
// GPU), instead of a last round of a few large tiles, each of which takes as
// long as a full round. Returns the first launch's columns (a multiple of
// 256), or 0 for one launch. The bits are the same: each output is still one
// tile's exact int32 sum and rescale. Measured (MI355X, 256 CUs; all 14
// shapes of M >= 768, K = 2048 and 4096, of the prefill set it applies to
// ran 3-15 % faster): 1536 x 11264 x 4096 101 -> 85.8 us, 4096 x 14336 x 4096 249 ->
// 241 us, 4096 x 5632 x 4096 108.5 -> 100.8 us, 768 x 28672 x 2048 76 -> 71
// us; last rounds more than half full measured level or slower (1024 x 28672
// x 4096, 2048 x 14336, 4096 x 11264: 0-2 % slower).
int gemm_column_split(int m, int n, int k, int cus) {
    (void)k;
    if (m <= 256 || n <= 256 || cus <= 0) return 0;
    const int64_t tm = (m + 255) / 256, tn = (n + 255) / 256, t = tm * tn;
    const int64_t rounds = t / cus, rem = t - rounds * cus;
    if (rounds < 1 || rem == 0 || 2 * rem > cus) return 0;
    const int64_t cols = rounds * cus / tm;
    return cols > 0 && cols < tn ? static_cast<int>(cols * 256) : 0;
}

int launch_gemm_w8a8(const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw, const float* as,
                     const float* ws, int m, int n, int k, float* out, int64_t ldo, int32_t* oi,
                     int64_t ldoi, uint8_t* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (const int n0 = gemm_column_split(m, n, k, device_cu_count()); n0 > 0) {
        const int st = launch_gemm_w8a8_tile(GemmTile{256, 256, 2}, a8, lda, w8, ldw, as, ws, m, n0, k, out, ldo, oi,
                                             ldoi, nullptr, stream);
        if (st != kStatusOk) return st;
        return launch_gemm_w8a8(a8, lda, w8 + static_cast<int64_t>(n0) * ldw, ldw, as, ws + n0, m, n - n0, k,
                                out + n0, ldo, oi ? oi + n0 : nullptr, ldoi, workspace, workspace_bytes, stream);
    }
    GemmTile r = gemm_route(m, n, k, device_cu_count());
    if (!workspace || workspace_bytes < gemm_workspace_bytes(r, m, n)) r.splits = 1;
    return launch_gemm_w8a8_tile(r, a8, lda, w8, ldw, as, ws, m, n, k, out, ldo, oi, ldoi, workspace, stream);
}

}  // namespace rk
