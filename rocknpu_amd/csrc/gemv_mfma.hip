// Kernel (d) for up to 16 activation rows (Q4_K) or 8 (Q6_K) on raw GGUF
// rows: the matrix-core GEMV of gemv_mfma.h, and for Q4_K rows longer than one
// stage the same product with the weights staged through LDS.
#include "gemv_mfma.h"

namespace rk {
namespace {

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
    const TiledHead h = tiled_head(p, FUSED, grid.x);
    if (depth >= 4) gemv_mfma_kernel<KIND, MT, FUSED, W, AREG, 4, false><<<grid, dim3(W * 64), lds, stream>>>(RK_HEAD(h), p);
    else if (depth >= 2) gemv_mfma_kernel<KIND, MT, FUSED, W, AREG, 2, false><<<grid, dim3(W * 64), lds, stream>>>(RK_HEAD(h), p);
    else gemv_mfma_kernel<KIND, MT, FUSED, W, AREG, 1, false><<<grid, dim3(W * 64), lds, stream>>>(RK_HEAD(h), p);
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
    int64_t all_tiles = 0;
    for (int i = 0; i < p.count; ++i) all_tiles += (p.rows[i] + kTileRows - 1) / kTileRows;
    if (all_tiles > 0xffff) {
        // the preloaded arguments (TiledHead) hold at most 0xffff tiles: larger
        // launches go member by member, and a larger member in runs of rows
        // (the same bits: a row's arithmetic does not depend on its launch)
        for (int i = 0; i < p.count; ++i) {
            constexpr int64_t kRun = int64_t{0xffff} * kTileRows;
            for (int64_t r0 = 0; r0 < p.rows[i]; r0 += kRun) {
                GemvParams a = p;
                a.count = 1;
                a.w[0] = p.w[i] + r0 * p.nb * block_bytes(kind);
                a.out[0] = p.out[i] + r0;
                a.ldo[0] = p.ldo[i];
                a.rows[0] = std::min(kRun, p.rows[i] - r0);
                const int st = launch_gemv_mfma(kind, fused, a, stream);
                if (st != kStatusOk) return st;
            }
        }
        return kStatusOk;
    }
    MfmaArgs ka;
    if (mfma_args(p, w, ka) != kStatusOk || !head_fits(ka)) return kStatusInvalid;
    const int tiles = ka.tiles;
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
