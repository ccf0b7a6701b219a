// Kernel (c) for up to 16 activation rows: the W8A8 GEMM as a weight stream.
//
// out[m, n] = (f32(sum_k A8[m, k] * W8[n, k]) * a_scale[m]) * w_scale[n], the
// same exact i32 products and the same rescale order as gemm.hip
// (crates/rocknpu-capi/src/lib.rs:692-709), for the decode-sized M where the
// GEMM is bound by reading W8 once (the reference's M=1 route,
// execute_cached_w8a8_m1, lib.rs:1567-1701).
//
// v_mfma_i32_16x16x32_i8: lane l supplies row l%16 of A and column l%16 of B
// with 8 K bytes, and holds D column l%16, rows 4*(l/16) + e. B's 16 columns
// are 16 weight rows, A's 16 rows the activation rows (zeros past m). A dot
// product does not depend on which K index sits in which slot, so lane group
// q = l/16 loads the 16 bytes 64c + 16q .. of K chunk c for both operands and
// feeds their two halves to two instructions that accumulate into one D.
//
// Work split: a tile is 16 weight rows. A workgroup of 8 waves holds the A8
// rows in LDS and walks its tiles (blockIdx.x, + gridDim.x, ..); wave g takes
// K chunks g, g + 8, .. of a tile with D chunks of weight loads in flight.
// The waves' i32 accumulators are added in LDS (exact) and wave 0 rescales and
// stores the tile.
#include "common.h"

#include <algorithm>

namespace rk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kSkinnyWaves = 8;

template <int D>
__global__ __launch_bounds__(kSkinnyWaves * 64) void gemm_w8a8_skinny_kernel(
    const int8_t* __restrict__ a8, int64_t lda, const int8_t* __restrict__ w8, int64_t ldw, int m, int n, int k,
    int grid, const float* __restrict__ a_scales, const float* __restrict__ w_scales, float* __restrict__ out,
    int64_t ldo, int32_t* __restrict__ out_i32, int64_t ldo_i32) {
    constexpr int W = kSkinnyWaves;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, q = lane >> 4;  // weight row in the tile, K slot group
    const int chunks = k / 64;
    const int iters = (chunks + W - 1) / W;  // chunks per wave and tile
    const int tiles = (n + 15) / 16;
    int8_t* la = reinterpret_cast<int8_t*>(smem);
    int* part = reinterpret_cast<int*>(smem + ((static_cast<size_t>(m) * k + 15) & ~size_t{15}));

    struct Pos {
        int t;
        int it;
    };
    auto advance = [&](Pos& c) {
        if (++c.it == iters) { c.it = 0; c.t += grid; }  // grid = gridDim.x, preloaded
    };
    // Weight loads: 16 bytes of row col of tile t, K chunk wave + 8 it, and the
    // row's scale (rows and chunks past the ends re-read row n-1 / chunk 0;
    // their products are dropped). Every load is unconditional and consumed in
    // order, so each wait covers exactly the loads a value depends on.
    struct Item {
        uint4 v;
        float ws;
    };
    auto load = [&](const Pos& c, Item& it) {
        const bool live = c.t < tiles;
        const int row = min((live ? c.t : 0) * 16 + col, n - 1);
        const int ch = live && wave + W * c.it < chunks ? wave + W * c.it : 0;
        it.v = *reinterpret_cast<const uint4*>(w8 + static_cast<int64_t>(row) * ldw + ch * 64 + q * 16);
        it.ws = w_scales[row];
    };
    // this lane's activation-row scales (rows 4q + e of D), loaded before the ring
    float as_e[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) as_e[e] = a_scales[min(4 * q + e, m - 1)];
    Item buf[D];
    Pos lq{static_cast<int>(blockIdx.x), 0};
#pragma unroll
    for (int j = 0; j < D; ++j) {
        load(lq, buf[j]);
        advance(lq);
    }
    // A8 rows into LDS, 16 bytes per thread and step
    const int a_vecs = m * (k / 16);
    for (int i = threadIdx.x; i < a_vecs; i += W * 64) {
        const int r = i / (k / 16), c16 = i % (k / 16);
        reinterpret_cast<uint4*>(la)[i] = *reinterpret_cast<const uint4*>(a8 + r * lda + c16 * 16);
    }
    __syncthreads();

    v4i acc = {0, 0, 0, 0};
    int tile_iter = 0;
    Pos cq{static_cast<int>(blockIdx.x), 0};
    while (cq.t < tiles) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            if (cq.t < tiles) {  // uniform
                const int ch = wave + W * cq.it;
                // activation bytes (zero past m and past the last chunk); the LDS
                // read stays inside the A8 rows
                uint4 av = *reinterpret_cast<const uint4*>(la + min(col, m - 1) * k + min(ch, chunks - 1) * 64 + q * 16);
                if (col >= m || ch >= chunks) av = uint4{0, 0, 0, 0};
                const uint4 wv = buf[j].v;
                const float ws = buf[j].ws;
                acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(static_cast<uint64_t>(av.y) << 32 | av.x),
                                                            static_cast<long>(static_cast<uint64_t>(wv.y) << 32 | wv.x),
                                                            acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(static_cast<uint64_t>(av.w) << 32 | av.z),
                                                            static_cast<long>(static_cast<uint64_t>(wv.w) << 32 | wv.z),
                                                            acc, 0, 0, 0);
                load(lq, buf[j]);
                advance(lq);
                if (cq.it == iters - 1) {
                    // tile done: the waves' sums to LDS, wave 0 adds them (exact) and stores
                    int* pb = part + (tile_iter & 1) * (W * 64 * 4);
                    *reinterpret_cast<v4i*>(pb + (wave * 64 + lane) * 4) = acc;
                    acc = v4i{0, 0, 0, 0};
                    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                    if (wave == 0) {
                        // D column col = weight row t*16 + col; lane holds activation rows 4q + e
                        const int nn = cq.t * 16 + col;
                        v4i s = *reinterpret_cast<const v4i*>(pb + lane * 4);
#pragma unroll
                        for (int g = 1; g < W; ++g) s += *reinterpret_cast<const v4i*>(pb + (g * 64 + lane) * 4);
                        if (nn < n) {
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int mm = 4 * q + e;
                                if (mm < m) {
                                    out[mm * ldo + nn] = (static_cast<float>(s[e]) * as_e[e]) * ws;
                                    if (out_i32) out_i32[mm * ldo_i32 + nn] = s[e];
                                }
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

}  // namespace

// m <= 16, k % 64 == 0, m * k <= 112 KiB; else kStatusInvalid (callers route
// other shapes to the tiled kernels).
int launch_gemm_w8a8_skinny(const int8_t* a8, int64_t lda, const int8_t* w8, int64_t ldw, const float* as,
                            const float* ws, int m, int n, int k, float* out, int64_t ldo, int32_t* oi,
                            int64_t ldoi, hipStream_t stream) {
    if (m < 1 || m > 16 || k % 64 != 0 || static_cast<int64_t>(m) * k > kSkinnyMaxA8) return kStatusInvalid;
    const int tiles = (n + 15) / 16;
    const size_t lds = ((static_cast<size_t>(m) * k + 15) & ~size_t{15}) + 2 * kSkinnyWaves * 64 * 4 * sizeof(int);
    // two workgroups per CU where both fit its 160 KiB of LDS: more weight
    // loads in flight (1 x 28672 x 4096: 28.5 -> 26.6 us)
    const int per_cu = 2 * lds <= 160 * 1024 ? 2 : 1;
    const int wgs = std::min(tiles, per_cu * device_cu_count());
    const int iters = (k / 64 + kSkinnyWaves - 1) / kSkinnyWaves;
    const int per_wave = (tiles + wgs - 1) / wgs * iters;
    const dim3 grid(static_cast<unsigned>(wgs)), block(kSkinnyWaves * 64);
    if (per_wave >= 8)
        gemm_w8a8_skinny_kernel<8><<<grid, block, lds, stream>>>(a8, lda, w8, ldw, m, n, k, static_cast<int>(grid.x), as, ws, out, ldo, oi, ldoi);
    else if (per_wave >= 4)
        gemm_w8a8_skinny_kernel<4><<<grid, block, lds, stream>>>(a8, lda, w8, ldw, m, n, k, static_cast<int>(grid.x), as, ws, out, ldo, oi, ldoi);
    else
        gemm_w8a8_skinny_kernel<2><<<grid, block, lds, stream>>>(a8, lda, w8, ldw, m, n, k, static_cast<int>(grid.x), as, ws, out, ldo, oi, ldoi);
    return hipGetLastError() == hipSuccess ? kStatusOk : kStatusExec;
}

}  // namespace rk
