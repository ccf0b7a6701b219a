// Kernel (d) on the decode cache's tiled copies of Q4_K/Q6_K weights: the
// layout and its conversion from raw GGUF rows, and the matrix-core GEMV of
// gemv_mfma.h reading them with whole-line loads.
//
// In the tiled copy the 16 rows of a tile have block b in one contiguous run
// whose bytes sit in the order the lanes take them: the 16 rows' headers, then
// each lane's operand bytes together. A wave then loads a tile's block with
// three (Q4_K) or five (Q6_K) whole-line instructions instead of 16 partly
// used lines per instruction, into the same registers, so the arithmetic and
// its results are those of the kernel on raw rows.
#include "gemv_mfma.h"

namespace rk {
namespace {

// ------------------------------------------------------------ tiled, pipelined
// The matrix-core GEMV on tiled weights with NI items per wave (an item is a
// tile of the workgroup and one of the wave's block indices) known at compile
// time and D of them in flight. The item loop is unrolled into straight-line
// code: in gemv_mfma_kernel's loop the compiler waits for every load in flight
// at the loop's head, so a second block in flight was waited for together with
// the first. The tile sums go to LDS and are stored after the loop, so no store
// sits among the loads either. A row's arithmetic and f32 order are those of
// gemv_mfma_kernel (wave g adds blocks g, g + W, .. in order; the W partial
// sums are added in wave order), so the results are the same bits.
// The activation blocks a wave owns (block indices wave + W * it, it < IT,
// of rows < m) with every f32 load issued up front: later block indices no
// longer wait, one after another, for loads issued while the one before is
// quantised. Past `iters` (or nb, or m) the loads re-read a valid block and
// nothing is quantised from them; Q8_K rows are copied as OwnedActs does.
template <int MT, int W, bool FUSED, int IT>
struct AllActs {
    static constexpr int QP = MT / 4;
    float4 xf[FUSED ? IT : 1][FUSED ? QP : 1][4];
    __device__ __forceinline__ void first(const MfmaArgs& p, int wave) {
        if constexpr (FUSED) {
            const int qslot = (threadIdx.x & 63) >> 4;
#pragma unroll
            for (int it = 0; it < IT; ++it)
#pragma unroll
                for (int i = 0; i < QP; ++i)
                    load_x16(p.x, p.ldx, p.nb, min(4 * i + qslot, p.m - 1) * p.nb + min(wave + W * it, p.nb - 1),
                             xf[it][i]);
        }
    }
    // the wave's block index `it` (< IT, a constant once unrolled) into LDS
    __device__ __forceinline__ void quantise_one(const MfmaArgs& p, int wave, const ActLds<MT>& act, int it) {
        const int qslot = (threadIdx.x & 63) >> 4;
        const int b = wave + W * it;
#pragma unroll
        for (int i = 0; i < QP; ++i) {
            const int mi = 4 * i + qslot;
            if (it < p.iters && mi < p.m && b < p.nb)
                quantize_block(xf[it][i], act.quants(b, mi), reinterpret_cast<int16_t*>(act.bsums(b, mi)),
                               act.d(b, mi));
        }
    }
    __device__ __forceinline__ void stage(const MfmaArgs& p, int wave, const ActLds<MT>& act) {
        if constexpr (FUSED) {
#pragma unroll
            for (int it = 0; it < IT; ++it) quantise_one(p, wave, act, it);
        } else {
            OwnedActs<MT, W, false> o;
            o.stage(p, wave, act);
        }
    }
};

//
// K split (S = 2, 4 or 8 ranges): unit u = (tile u / S, block range u % S),
// range r being blocks [r nb / S, (r + 1) nb / S); the grid is a multiple of
// S, so the units bid, bid + grid, .. of a workgroup share its range, whose
// activations it quantises once and whose weights alone it reads. A launch of
// few tiles so fills S times the workgroups. The ranges' partial sums meet in
// exchange slots (below, and gemv_tiled_ranges).
template <int KIND, int MT, bool FUSED, int W, bool AREG, int NI, int D, int IT, bool LAZY = false, int S = 1>
__global__ __launch_bounds__(W * 64) void gemv_tiled_kernel(const void* x, const uint8_t* w0, const uint8_t* w1,
                                                              const uint8_t* w2, int te01, int tiles, int grid,
                                                              int ldx, int nb_nbs, int m_iters, const MfmaArgs pa) {
    constexpr int BB = block_bytes(KIND);
    constexpr int NR = MT / 4;
    static_assert(D >= 1 && D <= NI, "one to NI items in flight");
    static_assert(S == 1 || S == 2 || S == 4 || S == 8, "unsplit, or 2, 4 or 8 block ranges");
    using Piece = typename PieceOf<KIND, true>::type;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int bid = blockIdx.x;
    // The launch's arguments: pa, with the fields the first loads need
    // preloaded ahead of it (TiledHead) and taken from there; the rest of pa
    // is read behind the first weight load (MemberOuts, below). Only
    // scalar fields of the local copy p are read (an array member indexed at
    // run time would put the copy in scratch memory).
    const int nb0 = nb_nbs & 0xffff, nbs0 = static_cast<int>(static_cast<uint32_t>(nb_nbs) >> 16);
    const TileMap tmap{w0, w1, w2, te01 & 0xffff, static_cast<int>(static_cast<uint32_t>(te01) >> 16)};
    // p: the range's view of the activations (its blocks from b0)
    // range sp: blocks [sp nb / S, (sp + 1) nb / S), at most nbs = ceil(nb / S)
    const int sp = S > 1 ? bid % S : 0, b0 = sp * nb0 / S;
    MfmaArgs p = pa;
    p.x = static_cast<const float*>(x);
    p.q8k = static_cast<const uint8_t*>(x);
    p.ldx = ldx;
    p.nb = nb0;
    p.m = m_iters & 0xffff;
    p.iters = static_cast<int>(static_cast<uint32_t>(m_iters) >> 16);
    p.tiles = tiles;
    if constexpr (S > 1) {
        p.nb = (sp + 1) * nb0 / S - b0;
        if constexpr (FUSED) p.x = static_cast<const float*>(x) + static_cast<int64_t>(b0) * kQK;
        else p.q8k = static_cast<const uint8_t*>(x) + static_cast<int64_t>(b0) * kQ8KBytes;
    }
    const int nb = p.nb, m = p.m, iters = p.iters;
    const int lnb = S > 1 ? nbs0 : nb;  // blocks the LDS layout holds
    const ActLds<MT> act{smem, lnb};
    // partial sums [2][W][64][NR], then the tile sums [NI][64][NR]
    float* part = reinterpret_cast<float*>(smem + ((lnb * MT * kPerRowBlock + 15) & ~15));
    float* res = part + 2 * W * 64 * NR;
    const int n = lane & 15, q = lane >> 4;
    const int ntile = (tiles * S - bid + grid - 1) / grid;  // units bid, bid + grid, ..
    const int items = ntile * iters;                           // <= NI (the host's choice)
    // item i: unit i / iters of the workgroup, block index i % iters; items
    // past the workgroup's last re-read its last one (in bounds) and are dropped
    auto load_item = [&](int i, Piece& k) {
        const int ic = min(i, items - 1);
        const int kt = ic / iters, it = ic - kt * iters;
        const int t = (bid + kt * grid) / S;
        const int b = b0 + min(wave + W * it, nb - 1);
        const gbytes w = reinterpret_cast<gbytes>(reinterpret_cast<uint64_t>(tmap.weights(t)));
        k.load_tiled(w + (static_cast<int64_t>(tmap.row0(t) / kTileRows) * nb0 + b) * (kTileRows * BB), lane);
    };

    // The activations of the wave's IT = iters block indices: with one, as
    // gemv_mfma_kernel loads them; with two to four, all loaded up front
    // (TinyLlama down, 2048 x 5632, three per wave: 6.93 -> 6.72 us at one row;
    // Llama-3-8B down, 4096 x 14336, four per wave: 14.4 -> 13.4 us).
    static_assert(AREG == (IT == 1), "one block index per wave keeps its operands in registers");
    OwnedActs<MT, W, FUSED> owned;
    AllActs<MT, W, FUSED, IT> all;
    if constexpr (IT == 1) owned.first(p, wave);
    else all.first(p, wave);
    // every wave's activation loads ahead of any weight load (gemv_mfma_kernel;
    // without this barrier TinyLlama o takes 4.1 instead of 3.6 us; with the
    // arguments preloaded, 3.50 instead of 3.00 at one row, and every decode
    // shape 0.4-0.7 us slower)
    __builtin_amdgcn_s_barrier();
    Piece buf[D];
    load_item(0, buf[0]);
    // Unsplit launches read the members' outputs here, behind the first
    // weight load: read where the stores use them, they are scalar loads that
    // the compiler issues at the stores, and their round trips (the member's
    // selection first, then its fields) sit at the end of every launch
    // (TinyLlama o at one row 3.32 -> 3.05 us; the decode set's 66 Q4_K
    // launches at one row 3.90 -> 3.67 us on average, at four rows 3.91 ->
    // 3.68). Holding them in registers right here (an empty asm) waits for
    // them at once: 0.4 us slower than that. Split launches keep them at
    // the stores: read here, the compiler places the exchange's loads just
    // before the quantisation's LDS wait, which then waits for them
    // (TinyLlama down at four rows 5.22 -> 5.38 us).
    MemberOuts mo{};
    if constexpr (S == 1) mo.fetch(pa);
    // LAZY: only block index 0 quantised here, block index i (< IT) just
    // before item i, the first that reads it, so item 0's terms wait for one
    // quantisation instead of IT (each wave quantises and reads only its own
    // block indices, so no barrier is needed between)
    constexpr bool lazy = LAZY && FUSED && IT > 1;
    if constexpr (IT == 1) owned.template stage<true>(p, wave, act);
    else if constexpr (lazy) all.quantise_one(p, wave, act, 0);
    else all.stage(p, wave, act);
#pragma unroll
    for (int j = 1; j < D; ++j) load_item(j, buf[j]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    uint64_t areg[8];
    uint32_t bsreg[NR][8];
    float dareg[NR];
    if constexpr (AREG) {
        const int b = min(wave, nb - 1);
        a_operands<KIND, MT>(act, b, lane, areg);
        row_data<KIND, MT>(act, b, lane, bsreg, dareg);
    }
    float acc[NR];
#pragma unroll
    for (int lr = 0; lr < NR; ++lr) acc[lr] = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        if constexpr (lazy) {
            if (i >= 1 && i < IT) {  // block index i, first used by item i
                all.quantise_one(p, wave, act, i);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
        }
        const int kt = i / iters, it = i - kt * iters;
        const int b = wave + W * it;
        if constexpr (!AREG) {
            a_operands<KIND, MT>(act, min(b, nb - 1), lane, areg);
            row_data<KIND, MT>(act, min(b, nb - 1), lane, bsreg, dareg);
        }
        float term[NR];
        block_terms<KIND, MT>(buf[i % D], areg, bsreg, dareg, term);
        if (i + D < NI) load_item(i + D, buf[i % D]);
        const bool have = b < nb && i < items;  // uniform
#pragma unroll
        for (int lr = 0; lr < NR; ++lr) acc[lr] += have ? term[lr] : 0.0f;
        if (it == iters - 1) {  // uniform: tile kt done
            float* pb = part + (kt & 1) * (W * 64 * NR);
#pragma unroll
            for (int lr = 0; lr < NR; ++lr) {
                pb[(wave * 64 + lane) * NR + lr] = acc[lr];
                acc[lr] = 0.0f;
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (wave == (kt & (W - 1))) {
#pragma unroll
                for (int lr = 0; lr < NR; ++lr) {
                    res[(kt * 64 + lane) * NR + lr] = tile_row_sum<W, NR>(pb, lane, lr, iters);
                }
            }
        }
    }
    __syncthreads();
    for (int kt = wave; kt < ntile; kt += W) {
        const int t = (bid + kt * grid) / S;
        const TileOut to = S == 1 ? tile_out(tmap, mo, t) : tile_out(pa, t);
        const int row = to.row0 + n;
#pragma unroll
        for (int lr = 0; lr < NR; ++lr) {
            float r = res[(kt * 64 + lane) * NR + lr];
            if constexpr (S > 1) {
                // The S ranges' values of each (tile, lane, register row) are
                // added as a binary tree: at level L, node j = range >> (L + 1)
                // has one slot where its two children's sums meet, by one
                // atomic swap that leaves the child's tag (2 g + side, for
                // the launch's generation g) and value there. Finding the slot
                // empty (0), the child is first and stops. Finding the other
                // side's tag of this launch, it is second: it adds the two
                // values (two addends: the same sum in either order, so the
                // tree's result is fixed), empties the slot and climbs; the
                // root's second child writes the output. Every launch so
                // leaves the slots as it found them. Anything else in a slot (one
                // not emptied by an earlier launch, or a launch sharing the
                // workspace) sets the error word, and its finder writes NaN;
                // the other side, if it swaps before the finder empties the
                // slot, adds and writes the exact sum instead. Never other
                // bits. Relaxed agent-scope atomics on one address are ordered
                // for all workgroups of the device.
                const uint32_t g = pa.gen % 0x7fffffffu + 1u;  // tags 2 .. 2^32 - 1, never 0
                bool first = false;
                int64_t base = 0;
#pragma unroll
                for (int lv = 0; (1 << lv) < S; ++lv) {
                    const int per = S >> (lv + 1), j = sp >> (lv + 1), side = (sp >> lv) & 1;
                    unsigned long long* slot =
                        pa.split_slot + base + ((static_cast<int64_t>(t) * per + j) * 64 + lane) * NR + lr;
                    base += static_cast<int64_t>(tiles) * per * 64 * NR;
                    const unsigned long long old = __hip_atomic_exchange(
                        slot, static_cast<unsigned long long>(2 * g + side) << 32 | __float_as_uint(r),
                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (old == 0) {
                        first = true;
                        break;
                    }
                    __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (static_cast<uint32_t>(old >> 32) != 2 * g + (1 - side)) {
                        r = __builtin_nanf("");
                        __hip_atomic_store(pa.split_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;  // written now, as NaN
                    }
                    r += __uint_as_float(static_cast<uint32_t>(old));
                }
                if (first) continue;
            }
            const int mo = NR * q + lr;
            if (mo < m && row < to.rows)
                reinterpret_cast<gfloats>(reinterpret_cast<uint64_t>(to.out))[mo * to.ldo + row] = r;
        }
    }
}

}  // namespace

// ------------------------------------------------------------ tiled layout
// The decode cache's copy of a weight: tiles of 16 rows (the last padded with
// zero rows), each tile's nb blocks one after another, and each block of the
// tile one run of 16 * B_blk bytes in the order the lanes of a wave take them
// (tile block, byte u):
//   Q4_K (2304 bytes): u < 256 row u / 16's 16-byte header (d, dmin, 12 scale
//     bytes); else lane l = (u - 256) / 32, with row n = l % 16 and K group
//     q = l / 16: the quant bytes 32 j + 8 q .. + 7 of row n, j = 0..3.
//   Q6_K (3360 bytes): u < 256 row u / 16's 16 scales; u < 288 row (u - 256)
//     / 2's fp16 d; else lane l = (u - 288) / 48: the ql runs 64 h + 32 i + 8 q
//     (in the order 2 h + i) and the qh runs 128 + 32 h + 8 q, 8 bytes each.
// A bijection of the raw bytes (plus the zero rows), so the GEMV's results on
// it are those on the raw blocks.
size_t gemv_tiled_bytes(int kind, int64_t n, int nb) {
    return static_cast<size_t>((n + kTileRows - 1) / kTileRows) * kTileRows * nb * block_bytes(kind);
}

namespace {
// One 2-byte unit of the tiled copy per thread: every run above starts at an
// even byte and has an even length, so a unit's bytes are one aligned 2-byte
// piece of one raw block (blocks are 2-byte aligned).
template <int KIND>
__global__ __launch_bounds__(256) void gemv_tile_weights_kernel(const uint8_t* __restrict__ src, int64_t n, int nb,
                                                                uint16_t* __restrict__ dst, int64_t units) {
    constexpr int BB = block_bytes(KIND), TB = kTileRows * BB;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < units;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t o = 2 * i, tbi = o / TB;
        const int u = static_cast<int>(o - tbi * TB);
        const int64_t t = tbi / nb;
        const int b = static_cast<int>(tbi - t * nb);
        int r, off;
        if constexpr (KIND == 4) {
            if (u < 256) {
                r = u >> 4;
                off = u & 15;
            } else {
                const int v = u - 256, l = v >> 5, w = v & 31;
                r = l & 15;
                off = 16 + 32 * (w >> 3) + 8 * (l >> 4) + (w & 7);
            }
        } else {
            if (u < 256) {
                r = u >> 4;
                off = 192 + (u & 15);
            } else if (u < 288) {
                r = (u - 256) >> 1;
                off = 208;
            } else {
                const int v = u - 288, l = v / 48, w = v - 48 * l, q = l >> 4;
                r = l & 15;
                off = w < 32 ? 64 * (w >> 4) + 32 * ((w >> 3) & 1) + 8 * q + (w & 7)
                             : 128 + 32 * ((w - 32) >> 3) + 8 * q + (w & 7);
            }
        }
        const int64_t row = t * kTileRows + r;
        dst[i] = row < n ? *reinterpret_cast<const uint16_t*>(src + (row * nb + b) * BB + off) : uint16_t{0};
    }
}
}  // namespace

int launch_gemv_tile_weights(int kind, const uint8_t* src, int64_t n, int nb, uint8_t* dst, hipStream_t stream) {
    const int64_t units = static_cast<int64_t>(gemv_tiled_bytes(kind, n, nb) / 2);
    const int64_t want = (units + 255) / 256;
    const dim3 grid(static_cast<unsigned>(std::min<int64_t>(want, 65536)));
    if (kind == 4)
        gemv_tile_weights_kernel<4><<<grid, dim3(256), 0, stream>>>(src, n, nb, reinterpret_cast<uint16_t*>(dst), units);
    else if (kind == 6)
        gemv_tile_weights_kernel<6><<<grid, dim3(256), 0, stream>>>(src, n, nb, reinterpret_cast<uint16_t*>(dst), units);
    else
        return kStatusInvalid;
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

namespace {
// Pipelined kernel, NI items per wave (ni tiles of iters block indices): two
// in flight for two or three items (TinyLlama gate+up, 2 x 5632 x 2048, three
// tiles per workgroup at 4 rows: 5.32 us against 5.51 with one and 5.42 with
// three, and with the arguments preloaded 4.77 against 4.93 with three;
// TinyLlama down, 2048 x 5632 on 8 waves, three blocks per wave: 6.95 against
// 7.46 with one), one for four (Llama-3-8B down, 4096 x 14336 on 16 waves:
// 14.8 against 14.8-15.1 us with two or four; the 32000 x 2048 Q6_K head, two
// eight-wave workgroups on most CUs: 11.4 against 11.9 / 12.5 us),
// but two for four on eight waves with one workgroup per CU (Llama-3.2-1B
// gate+up, 2 x 8192 x 2048, four tiles per workgroup: 6.0 against 6.3 us at
// one row, 6.9 against 7.3 at eight).
template <int KIND, int MT, bool FUSED, int W>
void launch_pipe(int ni, int iters, const MfmaArgs& p, dim3 grid, size_t lds, hipStream_t stream) {
    const dim3 block(W * 64);
    const TiledHead h = tiled_head(p, FUSED, grid.x);
    if (iters == 1) {
        if (ni == 1) gemv_tiled_kernel<KIND, MT, FUSED, W, true, 1, 1, 1><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
        else if (ni == 2) gemv_tiled_kernel<KIND, MT, FUSED, W, true, 2, 2, 1><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
        else if (ni == 3) gemv_tiled_kernel<KIND, MT, FUSED, W, true, 3, 2, 1><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
        else if (W == 8 && static_cast<int>(grid.x) <= device_cu_count())
            gemv_tiled_kernel<KIND, MT, FUSED, W, true, 4, 2, 1><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
        else gemv_tiled_kernel<KIND, MT, FUSED, W, true, 4, 1, 1><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
    } else if (iters == 2) {
        // block index 1 quantised after item 0's terms (Llama-3-8B q/o, 4096 x
        // 4096: 5.37 -> 5.19 us; q/k/v, 6144 x 4096: 7.17 -> 6.76 us)
        if (ni == 2) gemv_tiled_kernel<KIND, MT, FUSED, W, false, 2, 2, 2, true><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
        else gemv_tiled_kernel<KIND, MT, FUSED, W, false, 4, 1, 2, true><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
    } else if (iters == 3) {
        gemv_tiled_kernel<KIND, MT, FUSED, W, false, 3, 2, 3><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
    } else {
        gemv_tiled_kernel<KIND, MT, FUSED, W, false, 4, 1, 4><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
    }
}

template <int KIND, int MT, bool FUSED, int W>
void launch_tiled_w(int ni, const MfmaArgs& p, dim3 grid, size_t lds_loop, size_t lds_pipe, hipStream_t stream) {
    // Eight rows on 16 waves with three or four block indices a wave: the
    // activations loaded up front do not fit the 128 registers of a 1024-lane
    // workgroup and spill (Llama-3-8B down, 4096 x 14336, eight rows: 33.1 us
    // against 20.0 in the item loop)
    if constexpr (MT <= 8) {
        const bool spills = MT == 8 && W == 16 && p.iters >= 3;
        if (ni <= 4 && !spills) {
            launch_pipe<KIND, MT, FUSED, W>(ni, p.iters, p, grid, lds_pipe, stream);
            return;
        }
    }
    {
        // more items per wave than the pipelined kernel unrolls: the item loop
        // with one block in flight (two or four measured slower there)
        const TiledHead h = tiled_head(p, FUSED, grid.x);
        if (p.iters == 1)
            gemv_mfma_kernel<KIND, MT, FUSED, W, true, 1, true><<<grid, dim3(W * 64), lds_loop, stream>>>(RK_HEAD(h), p);
        else gemv_mfma_kernel<KIND, MT, FUSED, W, false, 1, true><<<grid, dim3(W * 64), lds_loop, stream>>>(RK_HEAD(h), p);
    }
}

template <int KIND, bool FUSED>
void launch_tiled_kind(int mt, int w, int ni, const MfmaArgs& p, dim3 grid, size_t lds_loop, size_t lds_pipe,
                       hipStream_t stream) {
#define RK_TW(MT)                                                                                   \
    (w == 16 ? launch_tiled_w<KIND, MT, FUSED, 16>(ni, p, grid, lds_loop, lds_pipe, stream)         \
             : launch_tiled_w<KIND, MT, FUSED, 8>(ni, p, grid, lds_loop, lds_pipe, stream))
    if (mt == 4) RK_TW(4);
    else if (mt == 8) RK_TW(8);
    else if constexpr (KIND == 4) RK_TW(16);
#undef RK_TW
}
}  // namespace

// Waves per workgroup of a tiled launch, from the row length alone (a row's f32
// order must not depend on how many projections share the launch, so grouped
// and separate calls agree bit for bit): 8 up to 8 blocks a row, 16 from 9.
// Rows of at most 16 blocks give the same bits with 8 or 16 waves (with 16,
// tile_row_sum adds waves s and s + 8 first, which is the 8-wave order), and 16
// measured faster for every such row (Llama-3-8B q/o, 4096 x 4096, at one row
// 5.11 -> 4.67 us, q/k/v 6.75 -> 5.90, gate+up 18.3 -> 13.3; 3072-wide rows: q/o
// at 4 rows 4.67 -> 4.31, gate+up 2 x 8192 11.1 -> 8.1). Longer rows take 16
// from 32 blocks (Llama-3-8B down unsplit 16.4 -> 14.3 us) and 8 for 17-31
// (TinyLlama down 6.9 against 7.4 us with 16), where the split launches take
// over from two rows. Rows shorter than 8 blocks leave waves without a block;
// they compute block nb - 1 and drop it, adding +0.0 to the row's sum.
int tiled_waves(int nb) {
    if (nb > 16) return nb >= 32 ? 16 : 8;
    return nb >= 9 ? 16 : 8;
}

// The matrix-core GEMV on tiled weights (p.w[i] each a tiled copy of its
// member's rows): Q4_K or Q6_K, 1 <= p.m <= gemv_mfma_rows(kind, p.nb). One
// workgroup per CU at most, each walking its tiles; one block in flight per
// wave in the item loop, or the pipelined kernel where a wave has at most four
// items and the launch at most 8 rows.
// The K split of a tiled launch, by kind, rows and row length alone (so a
// row's f32 order does not depend on the projections sharing the launch):
// - 2 to 8 activation rows over rows of 17 to 31 blocks (8 waves with three or
//   four block indices each unsplit): at up to 4 rows two ranges of 9-16
//   blocks, two block indices a wave (TinyLlama down, Q6_K 2048 x 5632, 128
//   tiles, at 4 rows: 6.58 -> 5.42-5.65 us; four ranges measure the same
//   there), at 5-8 rows four ranges of 5-8 (at 8 rows 8.1 -> 7.7 us against
//   two ranges).
// - 1 to 8 rows over rows of 32 to 64 blocks: 4 ranges, one block index a
//   wave: of 8 blocks on 8 waves at 32 blocks, of 9-16 on 16 waves above.
//   Llama-3-8B down (Q6_K 4096 x 14336) at 1 / 4 / 8 rows 12.9 (raw rows) /
//   14.4 / 22.0 -> 11.8 / 11.9 / 14.7 us (8 ranges of 7 blocks on 8 waves:
//   12.3 / 12.5 / 16.3, one tree level more); its Q4_K form at 1 / 4 rows 11.3
//   (raw) / 12.7 -> 9.6 / 9.7; Llama-3.2-1B down (Q6_K 2048 x 8192) 7.05 (raw)
//   / 7.8 -> 6.2 / 6.2 (two ranges of 16 on 16 waves: the same).
// Not split: rows of at most 16 blocks (one or two block indices a wave), which
// measured slower in two ranges on 4 or 8 waves (TinyLlama o at 4 rows 3.50 ->
// 3.92 us, gate+up 5.33 -> 6.73): there the exchange costs more than the
// ranges' workgroups save; one row over 17-31 blocks, where Q6_K's raw LDS
// stream stays faster; and rows of more than 64 blocks.
// Workspace: the error word, padding to 256 bytes, then the tree's slots, level
// by level: [level][tile][node][64 lanes][MT / 4 rows] x 8 bytes, S - 1 per
// tile, lane and row.
constexpr size_t kSplitSlotBase = 256;
int gemv_tiled_ranges(int kind, int m, int nb) {
    if ((kind != 4 && kind != 6) || m < 1 || m > 8) return 1;
    if (m >= 2 && nb >= 17 && nb <= 31) return m <= 4 ? 2 : 4;
    if (nb >= 32 && nb <= 64) return 4;
    return 1;
}
bool gemv_tiled_split(int kind, int m, int nb) { return gemv_tiled_ranges(kind, m, nb) > 1; }
size_t gemv_tiled_split_bytes(int kind, int m, int nb, int64_t tiles) {
    const int s = gemv_tiled_ranges(kind, m, nb);
    if (s == 1) return 0;
    return kSplitSlotBase + static_cast<size_t>(tiles) * 64 * (m <= 4 ? 1 : 2) * (s - 1) * 8;
}

namespace {
// Split launches: ranges of 9-16 blocks (two ranges) take two block indices a
// wave, the second quantised after the first item; ranges of at most 8 one.
template <int KIND, int MT, bool FUSED, int S>
void launch_split_s(int ni, const MfmaArgs& p, dim3 grid, size_t lds, hipStream_t stream) {
    const dim3 block(8 * 64);
    const TiledHead h = tiled_head(p, FUSED, grid.x);
    if (p.iters == 2) {
        if constexpr (S == 2) {
            if (ni == 2) gemv_tiled_kernel<KIND, MT, FUSED, 8, false, 2, 2, 2, true, 2><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
            else gemv_tiled_kernel<KIND, MT, FUSED, 8, false, 4, 1, 2, true, 2><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
        }
    } else if (ni == 1) {
        gemv_tiled_kernel<KIND, MT, FUSED, 8, true, 1, 1, 1, false, S><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
    } else if (ni == 2) {
        gemv_tiled_kernel<KIND, MT, FUSED, 8, true, 2, 2, 1, false, S><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
    } else if (ni == 3) {
        gemv_tiled_kernel<KIND, MT, FUSED, 8, true, 3, 2, 1, false, S><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
    } else {
        gemv_tiled_kernel<KIND, MT, FUSED, 8, true, 4, 1, 1, false, S><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
    }
}
// Four items a wave keep one in flight (Llama-3-8B down in four ranges at one
// row, arguments preloaded: 11.6 against 12.8 us with two).
template <int KIND, int MT, bool FUSED, int S>
void launch_split_w16(int ni, const MfmaArgs& p, dim3 grid, size_t lds, hipStream_t stream) {
    const dim3 block(16 * 64);
    const TiledHead h = tiled_head(p, FUSED, grid.x);
    if (ni == 1) gemv_tiled_kernel<KIND, MT, FUSED, 16, true, 1, 1, 1, false, S><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
    else if (ni == 2) gemv_tiled_kernel<KIND, MT, FUSED, 16, true, 2, 2, 1, false, S><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
    else if (ni == 3) gemv_tiled_kernel<KIND, MT, FUSED, 16, true, 3, 2, 1, false, S><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
    else gemv_tiled_kernel<KIND, MT, FUSED, 16, true, 4, 1, 1, false, S><<<grid, block, lds, stream>>>(RK_HEAD(h), p);
}
template <int KIND, int MT, bool FUSED>
void launch_split(int s, int w, int ni, const MfmaArgs& p, dim3 grid, size_t lds, hipStream_t stream) {
    if (w == 16) launch_split_w16<KIND, MT, FUSED, 4>(ni, p, grid, lds, stream);
    else if (s == 2) launch_split_s<KIND, MT, FUSED, 2>(ni, p, grid, lds, stream);
    else launch_split_s<KIND, MT, FUSED, 4>(ni, p, grid, lds, stream);
}
template <int KIND, bool FUSED>
void launch_split_k(int mt, int s, int w, int ni, const MfmaArgs& p, dim3 grid, size_t lds, hipStream_t stream) {
    if (mt == 4) launch_split<KIND, 4, FUSED>(s, w, ni, p, grid, lds, stream);
    else launch_split<KIND, 8, FUSED>(s, w, ni, p, grid, lds, stream);
}
}  // namespace

int launch_gemv_tiled(int kind, bool fused, GemvParams& p, hipStream_t stream) {
    if ((kind != 4 && kind != 6) || p.m < 1 || p.m > gemv_mfma_rows(kind, p.nb)) return kStatusInvalid;
    if (p.count == 4) {
        // the kernels take three members' fields as preloaded arguments
        // (TiledHead): the fourth member is a launch of its own, with the
        // same bits (a row's arithmetic does not depend on its launch)
        GemvParams a = p, b = p;
        a.count = 3;
        b.count = 1;
        b.w[0] = p.w[3];
        b.out[0] = p.out[3];
        b.ldo[0] = p.ldo[3];
        b.rows[0] = p.rows[3];
        const int st = launch_gemv_tiled(kind, fused, a, stream);
        return st != kStatusOk ? st : launch_gemv_tiled(kind, fused, b, stream);
    }
    // and at most 0xffff tiles (1,048,560 rows): larger launches go member by
    // member, and a larger member in runs of 0xffff tiles
    int64_t all_tiles = 0;
    for (int i = 0; i < p.count; ++i) all_tiles += (p.rows[i] + kTileRows - 1) / kTileRows;
    if (all_tiles > 0xffff) {
        for (int i = 0; i < p.count; ++i) {
            constexpr int64_t kRun = int64_t{0xffff} * kTileRows;
            for (int64_t r0 = 0; r0 < p.rows[i]; r0 += kRun) {
                GemvParams a = p;
                a.count = 1;
                a.w[0] = p.w[i] + (r0 / kTileRows) * p.nb * kTileRows * block_bytes(kind);
                a.out[0] = p.out[i] + r0;
                a.ldo[0] = p.ldo[i];
                a.rows[0] = std::min(kRun, p.rows[i] - r0);
                const int st = launch_gemv_tiled(kind, fused, a, stream);
                if (st != kStatusOk) return st;
            }
        }
        return kStatusOk;
    }
    const int mt = p.m <= 4 ? 4 : p.m <= 8 ? 8 : 16;
    const int cus = device_cu_count();
    int64_t tiles = 0;
    for (int i = 0; i < p.count; ++i) tiles += (p.rows[i] + kTileRows - 1) / kTileRows;
    if (const int sr = gemv_tiled_ranges(kind, p.m, p.nb); sr > 1) {
        if (!p.split_ws || p.split_ws_bytes < gemv_tiled_split_bytes(kind, p.m, p.nb, tiles) ||
            reinterpret_cast<uintptr_t>(p.split_ws) % 256 != 0)
            return kStatusInvalid;
        // waves: 8, with one block index each for ranges of at most 8 blocks
        // and two for the 9-16 of two ranges; 16 with one each for the 9-16 of
        // four ranges
        MfmaArgs ka;
        const int nbs = (p.nb + sr - 1) / sr, sw = sr == 4 && nbs > 8 ? 16 : 8;
        if (mfma_args(p, sw, ka) != kStatusOk) return kStatusInvalid;
        ka.nbs = nbs;
        ka.iters = (nbs + sw - 1) / sw;
        if (ka.iters > 2 || (ka.iters == 2 && sr != 2) || !head_fits(ka)) return kStatusInvalid;
        ka.split_err = static_cast<uint32_t*>(p.split_ws);
        ka.split_slot = reinterpret_cast<unsigned long long*>(static_cast<uint8_t*>(p.split_ws) + kSplitSlotBase);
        ka.gen = next_split_generation();
        // (tile, range) units on a grid of a multiple of sr workgroups (so a
        // workgroup's units share its range): one round on the CUs, or as
        // many workgroups as keep a workgroup's items within 4
        const int64_t units = static_cast<int64_t>(ka.tiles) * sr, upw = 4 / ka.iters;
        int64_t wgs = std::min<int64_t>(units, cus) / sr * sr;
        if ((units + wgs - 1) / wgs > upw) wgs = ((units + upw - 1) / upw + sr - 1) / sr * sr;
        const int ni = static_cast<int>((units + wgs - 1) / wgs) * ka.iters;
        const dim3 grid(static_cast<unsigned>(wgs));
        const size_t lds = gemv_mfma_lds(mt, ka.nbs, sw) + static_cast<size_t>(std::min(ni, 4)) * 64 * (mt / 4) * 4;
        if (lds > static_cast<size_t>(kLdsMax) || ni > 4) return kStatusInvalid;
        if (kind == 4) {
            if (fused) launch_split_k<4, true>(mt, sr, sw, ni, ka, grid, lds, stream);
            else launch_split_k<4, false>(mt, sr, sw, ni, ka, grid, lds, stream);
        } else {
            if (fused) launch_split_k<6, true>(mt, sr, sw, ni, ka, grid, lds, stream);
            else launch_split_k<6, false>(mt, sr, sw, ni, ka, grid, lds, stream);
        }
        return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
    }
    const int w = tiled_waves(p.nb);
    MfmaArgs ka;
    if (mfma_args(p, w, ka) != kStatusOk || !head_fits(ka)) return kStatusInvalid;
    // one round of workgroups on the CUs; but eight-wave launches of one block
    // index a wave and more than four tiles a CU get a workgroup per four
    // tiles (two on some CUs), so the pipelined kernel takes them instead of
    // the item loop: the 32000 x 2048 Q6_K head at 1/4/8 rows 12.1/12.5/13.8
    // -> 11.4/11.6/12.3 us, the 128256 x 2048 one 41.0/44.2/48.3 ->
    // 38.8/41.6/46.4 us. Fewer tiles a workgroup than four measured slower
    // there, and so did this for 16-wave launches (Llama-3-8B gate+up,
    // 2 x 14336 x 4096, one row: 13.4 -> 15.5 us).
    int wgs = std::min(ka.tiles, cus);
    if (w == 8 && mt <= 8 && ka.iters == 1 && ka.tiles > 4 * wgs) wgs = (ka.tiles + 3) / 4;
    const dim3 grid(static_cast<unsigned>(wgs));
    const int ni = (ka.tiles + wgs - 1) / wgs * ka.iters;
    const size_t lds_loop = gemv_mfma_lds(mt, p.nb, w);
    // the pipelined kernel keeps each tile's sums in LDS until its stores
    const size_t lds_pipe = lds_loop + static_cast<size_t>(std::min(ni, 4)) * 64 * (mt / 4) * 4;
    if (lds_pipe > static_cast<size_t>(kLdsMax)) return kStatusInvalid;
    if (kind == 4) {
        if (fused) launch_tiled_kind<4, true>(mt, w, ni, ka, grid, lds_loop, lds_pipe, stream);
        else launch_tiled_kind<4, false>(mt, w, ni, ka, grid, lds_loop, lds_pipe, stream);
    } else {
        if (fused) launch_tiled_kind<6, true>(mt, w, ni, ka, grid, lds_loop, lds_pipe, stream);
        else launch_tiled_kind<6, false>(mt, w, ni, ka, grid, lds_loop, lds_pipe, stream);
    }
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace rk
