// Device-pointer launch layer (include/rocknpu_hip.h): host-side argument
// checks, then one enqueue per kernel. Every shape and alignment the kernels
// assume is checked here, before anything reaches the GPU.
#include <algorithm>
#include <atomic>
#include <climits>

#include "common.h"
#include "rocknpu_hip.h"

namespace rk {
int launch_repack_w8(int kind, const uint8_t* blocks, int64_t n, int nb, int64_t k_pad, int8_t* w8,
                     float* scales, hipStream_t stream);
int launch_quantize_q8_k(const float* x, int64_t m, int64_t k, int64_t ldx, uint8_t* y,
                         hipStream_t stream);
int launch_gemv(int kind, bool fused, GemvParams& p, hipStream_t stream);

int device_cu_count() {
    // per device, filled on first use; atomic, as host threads may ask at once
    static std::atomic<int> cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}
}  // namespace rk

namespace {

bool aligned(const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

constexpr size_t kMaxGrid = 0x7fffffff;
// LDS a decode GEMV workgroup may give the Q8_K activation rows: of the 160
// KiB of a gfx950 CU, 112 KiB, leaving room for the matrix-core kernel's
// 16 KiB of partial sums; one workgroup runs per CU either way.
constexpr size_t kGemvLdsBytes = 112 * 1024;

// Rows of the next launch when `rem` activation rows are left: as many as the
// matrix-core kernel holds when it takes them, else a power of two (the
// lane-per-block kernel's register tile, at most 8) whose Q8_K blocks fit the
// LDS that kernel stages them in.
size_t gemv_rows_per_launch(uint32_t kind, size_t nb, size_t rem, int64_t rows, bool sums, int cus) {
    const size_t mf = static_cast<size_t>(rk::gemv_mfma_rows(static_cast<int>(kind), static_cast<int>(nb)));
    const size_t c = std::min(rem, mf);
    if (!sums && c >= 3 &&
        rk::gemv_uses_mfma(static_cast<int>(kind), static_cast<int>(c), static_cast<int>(nb), rows, cus))
        return c;
    size_t chunk = 8;
    while (chunk > 1 && chunk * nb * rk::kGemvLdsPerBlock > kGemvLdsBytes) chunk >>= 1;
    return std::min(rem, chunk);
}

}  // namespace

extern "C" int rocknpu_hip_repack_w8(uint32_t kind, const uint8_t* blocks, size_t blocks_bytes, size_t k,
                                     size_t n, size_t k_pad, int8_t* w8, float* scales, void* stream) {
    const size_t bb = rk::block_bytes(static_cast<int>(kind));
    if (bb == 0 || !blocks || !w8 || !scales || k == 0 || n == 0 || k % rk::kQK != 0) return rk::kStatusInvalid;
    if (k_pad < k || k_pad % 64 != 0 || blocks_bytes / bb / (k / rk::kQK) != n || blocks_bytes % bb != 0 ||
        blocks_bytes != n * (k / rk::kQK) * bb)
        return rk::kStatusInvalid;
    if (!aligned(blocks, kind == 6 ? 2 : 16) || !aligned(w8, 16) || k / rk::kQK > INT_MAX ||
        (n + 3) / 4 > kMaxGrid)
        return rk::kStatusInvalid;
    return rk::launch_repack_w8(static_cast<int>(kind), blocks, static_cast<int64_t>(n),
                                static_cast<int>(k / rk::kQK), static_cast<int64_t>(k_pad), w8, scales,
                                static_cast<hipStream_t>(stream));
}

extern "C" int rocknpu_hip_quantize_a8(const float* a, size_t m, size_t k, size_t lda, size_t k_pad,
                                       int8_t* a8, float* scales, void* stream) {
    if (!a || !a8 || !scales || m == 0 || k == 0 || lda < k || k_pad < k || m > kMaxGrid)
        return rk::kStatusInvalid;
    return rk::launch_quantize_a8(a, static_cast<int64_t>(m), static_cast<int64_t>(k),
                                  static_cast<int64_t>(lda), static_cast<int64_t>(k_pad), a8, scales, nullptr, 0,
                                  static_cast<hipStream_t>(stream));
}

namespace {
bool gemm_args_ok(const int8_t* a8, const float* a_scales, const int8_t* w8, const float* w_scales, size_t m,
                  size_t n, size_t k_pad, const float* out, size_t ldo) {
    if (!a8 || !a_scales || !w8 || !w_scales || !out || m == 0 || n == 0 || k_pad == 0 || k_pad % 64 != 0 ||
        ldo < n || m > INT_MAX || n > INT_MAX || k_pad > rk::kMaxExactK)
        return false;
    if (!aligned(a8, 16) || !aligned(w8, 16)) return false;
    // worst-case tile count (16-row tiles, 64-column tiles) must fit one grid;
    // routed K splits only run on tiles filling at most half the CUs
    return ((m + 15) / 16) * ((n + 63) / 64) <= kMaxGrid;
}
}  // namespace

extern "C" int rocknpu_hip_gemm_w8a8_ws(const int8_t* a8, const float* a_scales, const int8_t* w8,
                                        const float* w_scales, size_t m, size_t n, size_t k_pad, float* out,
                                        size_t ldo, int32_t* out_i32, void* workspace, size_t workspace_bytes,
                                        void* stream) {
    if (!gemm_args_ok(a8, a_scales, w8, w_scales, m, n, k_pad, out, ldo)) return rk::kStatusInvalid;
    if (workspace_bytes > 0 && (!workspace || !aligned(workspace, 256))) return rk::kStatusInvalid;
    return rk::launch_gemm_w8a8(a8, static_cast<int64_t>(k_pad), w8, static_cast<int64_t>(k_pad), a_scales,
                                w_scales, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k_pad), out,
                                static_cast<int64_t>(ldo), out_i32, static_cast<int64_t>(n),
                                static_cast<uint8_t*>(workspace), workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int rocknpu_hip_gemm_w8a8(const int8_t* a8, const float* a_scales, const int8_t* w8,
                                     const float* w_scales, size_t m, size_t n, size_t k_pad, float* out,
                                     size_t ldo, int32_t* out_i32, void* stream) {
    return rocknpu_hip_gemm_w8a8_ws(a8, a_scales, w8, w_scales, m, n, k_pad, out, ldo, out_i32, nullptr, 0, stream);
}

extern "C" int rocknpu_hip_gemm_w8a8_tile(int bm, int bn, int stages, int splits, const int8_t* a8,
                                          const float* a_scales, const int8_t* w8, const float* w_scales, size_t m,
                                          size_t n, size_t k_pad, float* out, size_t ldo, int32_t* out_i32,
                                          void* workspace, size_t workspace_bytes, void* stream) {
    if (!gemm_args_ok(a8, a_scales, w8, w_scales, m, n, k_pad, out, ldo)) return rk::kStatusInvalid;
    // the tiles and stage counts the launcher instantiates
    const bool known = (bm == 0 && m <= 16 && m * k_pad <= static_cast<size_t>(rk::kSkinnyMaxA8)) ||
                       (bm == 64 && bn == 32 && (stages == 2 || stages == 4)) ||
                       (bm == 64 && bn == 64 && (stages == 2 || stages == 4)) ||
                       (bm == 128 && bn == 64 && (stages == 2 || stages == 4)) ||
                       (bm == 128 && bn == 128 && (stages == 2 || stages == 3)) ||
                       (bm == 256 && bn == 128 && stages == 3) || (bm == 256 && bn == 256 && stages == 2) ||
                       (bm == 32 && bn == 64 && stages == 4 && k_pad % 128 == 0);
    if (!known || splits < 1 || splits > 16) return rk::kStatusInvalid;
    rk::GemmTile r{bm, bn, stages};
    r.splits = bm == 0 ? 1 : splits;
    if (r.splits > 1 &&
        (!workspace || !aligned(workspace, 256) ||
         workspace_bytes < rk::gemm_workspace_bytes(r, static_cast<int>(m), static_cast<int>(n)) ||
         rk::gemm_workspace_counters(r, static_cast<int>(m), static_cast<int>(n)) > rk::kSplitCounters))
        return rk::kStatusInvalid;
    return rk::launch_gemm_w8a8_tile(r, a8, static_cast<int64_t>(k_pad), w8, static_cast<int64_t>(k_pad), a_scales,
                                     w_scales, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k_pad), out,
                                     static_cast<int64_t>(ldo), out_i32, static_cast<int64_t>(n),
                                     static_cast<uint8_t*>(workspace), static_cast<hipStream_t>(stream));
}

extern "C" int rocknpu_hip_gemm_workspace(size_t m, size_t n, size_t k_pad, int cus, size_t* bytes, int* splits) {
    if (!bytes || !splits || m == 0 || n == 0 || k_pad == 0 || k_pad % 64 != 0 || m > INT_MAX || n > INT_MAX ||
        k_pad > INT_MAX)
        return rk::kStatusInvalid;
    if (cus <= 0) cus = rk::device_cu_count();
    const rk::GemmTile r = rk::gemm_route(static_cast<int>(m), static_cast<int>(n), static_cast<int>(k_pad), cus);
    *bytes = rk::gemm_workspace_bytes(r, static_cast<int>(m), static_cast<int>(n));
    *splits = r.splits;
    return rk::kStatusOk;
}

extern "C" int rocknpu_hip_gemm_workspace_check(void* workspace, void* stream) {
    if (!workspace) return rk::kStatusInvalid;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t* word = static_cast<uint32_t*>(workspace) + rk::kSplitErrorWord;
    uint32_t flag = 0;
    if (hipMemcpyAsync(&flag, word, sizeof flag, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return rk::kStatusExec;
    if (flag == 0) return rk::kStatusOk;
    static const uint32_t zero = 0;
    if (hipMemcpyAsync(word, &zero, sizeof zero, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return rk::kStatusExec;
    return rk::kStatusExec;
}

extern "C" int rocknpu_hip_gemm_column_split(size_t m, size_t n, size_t k_pad, int cus, size_t* n0) {
    if (!n0 || m == 0 || n == 0 || k_pad == 0 || k_pad % 64 != 0 || m > INT_MAX || n > INT_MAX || k_pad > INT_MAX)
        return rk::kStatusInvalid;
    if (cus <= 0) cus = rk::device_cu_count();
    *n0 = static_cast<size_t>(
        rk::gemm_column_split(static_cast<int>(m), static_cast<int>(n), static_cast<int>(k_pad), cus));
    return rk::kStatusOk;
}

extern "C" int rocknpu_hip_gemm_route(size_t m, size_t n, size_t k_pad, int cus, int* bm, int* bn, int* stages) {
    if (!bm || !bn || !stages || m == 0 || n == 0 || k_pad == 0 || k_pad % 64 != 0 || m > INT_MAX || n > INT_MAX ||
        k_pad > INT_MAX)
        return rk::kStatusInvalid;
    if (cus <= 0) cus = rk::device_cu_count();
    const rk::GemmTile r = rk::gemm_route(static_cast<int>(m), static_cast<int>(n), static_cast<int>(k_pad), cus);
    *bm = r.bm;
    *bn = r.bn;
    *stages = r.stages;
    return rk::kStatusOk;
}

extern "C" int rocknpu_hip_gemv_shape(uint32_t kind, size_t m, size_t k, const size_t* n, size_t count, int fused,
                                      int cus, int* mfma, int* lanes, int* waves) {
    if ((kind != 4 && kind != 6) || !n || !mfma || !lanes || !waves || m == 0 || m > INT_MAX || k == 0 ||
        k % rk::kQK != 0 || count == 0 || count > rk::kGemvMaxMembers || k / rk::kQK > INT_MAX)
        return rk::kStatusInvalid;
    if (cus <= 0) cus = rk::device_cu_count();
    const size_t nb = k / rk::kQK;
    if (nb * rk::kGemvLdsPerBlock > kGemvLdsBytes) return rk::kStatusInvalid;
    int64_t rows[rk::kGemvMaxMembers] = {};
    int64_t total = 0;
    for (size_t i = 0; i < count; ++i) {
        if (n[i] == 0 || n[i] > INT32_MAX / 2) return rk::kStatusInvalid;
        rows[i] = static_cast<int64_t>(n[i]);
        total += rows[i];
    }
    // the first launch's rows
    const int rows0 = static_cast<int>(gemv_rows_per_launch(kind, nb, m, total, false, cus));
    const int stream_waves = rk::gemv_stream_waves(static_cast<int>(kind), rows0, static_cast<int>(nb), total, false, cus);
    if (stream_waves != 0) {
        *mfma = 2;
        *lanes = 8;
        *waves = stream_waves;
        return rk::kStatusOk;
    }
    *mfma = rk::gemv_uses_mfma(static_cast<int>(kind), rows0, static_cast<int>(nb), total, cus) ? 1 : 0;
    const rk::GemvLanes l = rk::gemv_lanes(fused != 0, false, rows0, static_cast<int>(nb), rows,
                                           static_cast<int>(count), cus);
    *lanes = *mfma ? 0 : l.lanes;
    *waves = *mfma ? 0 : l.waves;
    return rk::kStatusOk;
}

extern "C" int rocknpu_hip_quantize_q8_k(const float* x, size_t m, size_t k, size_t ldx, uint8_t* q8k,
                                         void* stream) {
    if (!x || !q8k || m == 0 || k == 0 || k % rk::kQK != 0 || ldx < k || !aligned(q8k, 4))
        return rk::kStatusInvalid;
    if ((m * (k / rk::kQK) + 3) / 4 > kMaxGrid) return rk::kStatusInvalid;
    return rk::launch_quantize_q8_k(x, static_cast<int64_t>(m), static_cast<int64_t>(k),
                                    static_cast<int64_t>(ldx), q8k, static_cast<hipStream_t>(stream));
}


extern "C" int rocknpu_hip_gemv_q8_k(uint32_t kind, const uint8_t* w, size_t w_bytes, size_t k, size_t n,
                                     const uint8_t* q8k, size_t m, float* out, size_t ldo, int32_t* isum,
                                     int32_t* msum, void* stream) {
    if ((kind != 4 && kind != 6) || !w || !q8k || !out || k == 0 || k % rk::kQK != 0 || n == 0 || m == 0 ||
        ldo < n || n > INT_MAX)
        return rk::kStatusInvalid;
    const size_t bb = rk::block_bytes(static_cast<int>(kind)), nb = k / rk::kQK;
    if (w_bytes != n * nb * bb || !aligned(w, kind == 4 ? 16 : 2) || !aligned(q8k, 4)) return rk::kStatusInvalid;
    if ((isum == nullptr) != (msum == nullptr)) return rk::kStatusInvalid;
    const size_t per_row = nb * rk::kQ8KBytes;
    if (nb * rk::kGemvLdsPerBlock > kGemvLdsBytes) return rk::kStatusInvalid;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (size_t m0 = 0, chunk = 0; m0 < m; m0 += chunk) {
        chunk = gemv_rows_per_launch(kind, nb, m - m0, static_cast<int64_t>(n), isum != nullptr, rk::device_cu_count());
        rk::GemvParams p{};
        p.count = 1;
        p.w[0] = w;
        p.out[0] = out + m0 * ldo;
        p.ldo[0] = static_cast<int64_t>(ldo);
        p.rows[0] = static_cast<int64_t>(n);
        p.q8k = q8k + m0 * per_row;
        p.ldx = static_cast<int64_t>(per_row);
        p.m = static_cast<int>(std::min(chunk, m - m0));
        p.nb = static_cast<int>(nb);
        p.isum = isum ? isum + m0 * n * nb : nullptr;
        p.msum = msum ? msum + m0 * n * nb : nullptr;
        const int st = rk::launch_gemv(static_cast<int>(kind), false, p, s);
        if (st != rk::kStatusOk) return st;
    }
    return rk::kStatusOk;
}

extern "C" size_t rocknpu_hip_gemv_tiled_bytes(uint32_t kind, size_t k, size_t n) {
    if ((kind != 4 && kind != 6) || k == 0 || k % rk::kQK != 0 || n == 0 || n > INT32_MAX / 2 ||
        k / rk::kQK > INT_MAX)
        return 0;
    return rk::gemv_tiled_bytes(static_cast<int>(kind), static_cast<int64_t>(n), static_cast<int>(k / rk::kQK));
}

extern "C" int rocknpu_hip_gemv_tile_weights(uint32_t kind, const uint8_t* w, size_t w_bytes, size_t k, size_t n,
                                             uint8_t* tiled, size_t tiled_bytes, void* stream) {
    const size_t need = rocknpu_hip_gemv_tiled_bytes(kind, k, n);
    if (need == 0 || !w || !tiled || tiled_bytes < need) return rk::kStatusInvalid;
    const size_t bb = rk::block_bytes(static_cast<int>(kind)), nb = k / rk::kQK;
    if (w_bytes != n * nb * bb || !aligned(w, 2) || !aligned(tiled, 16)) return rk::kStatusInvalid;
    return rk::launch_gemv_tile_weights(static_cast<int>(kind), w, static_cast<int64_t>(n), static_cast<int>(nb),
                                        tiled, static_cast<hipStream_t>(stream));
}

// Measured on the decode shapes of TinyLlama, Llama-3.2-1B and Llama-3-8B and
// on rows of 2-31 blocks, 2048 and 4096 rows (HIP graph, weights rotating
// through > 1 GB): from two rows the tiled copy wins on every shape (TinyLlama
// o at 4 rows 3.41 against 4.21 us, gate+up 4.85 against 7.43, down 5.41
// against 7.24). At one row the lane-per-block kernel on raw rows runs well
// where a row's blocks fill its 8 block slots in whole passes, and the Q6_K
// LDS stream likewise; elsewhere it takes one to four slots a row and runs
// 1.3-2.6x longer. So at one row:
// - rows of at most 4 blocks keep the raw rows (level: 3.12-3.45 us either
//   way, and no tiled copy is needed);
// - rows of 5-16 blocks and of 32-64 run tiled (Q4_K 2048 wide: 5 blocks 3.35
//   against 6.85 us, 7 blocks 3.37 against 3.77, TinyLlama qkv 3.38 against
//   3.48 and gate+up 4.87 against 5.17, o 3.32 against 3.30; 10 blocks 4.13
//   against 6.95; Q6_K 6 blocks 3.47 against 5.32; Llama-3-8B down 11.5
//   against 11.8), and Q4_K rows of more than 64;
// - rows of 17-31 blocks keep the raw rows where those fill 8 slots (21-24
//   and 28-31 blocks: TinyLlama down, Q6_K 2048 x 5632, 4.85 against 6.22 on
//   the LDS stream; Q4_K 2048 x 5632 4.73 against 5.80) and run tiled where
//   not (17-20 and 25-27: Q4_K 17 blocks 5.43 against 7.22, Q6_K 26 blocks
//   7.41 against 11.5).
extern "C" int rocknpu_hip_gemv_tiled_preferred(uint32_t kind, size_t m, size_t k) {
    if ((kind != 4 && kind != 6) || m == 0 || k == 0 || k % rk::kQK != 0) return 0;
    if (m >= 2) return 1;
    const size_t nb = k / rk::kQK;
    if (nb <= 4) return 0;
    if (nb >= 17 && nb <= 31) return rk::slots_per_row_log2(static_cast<int>(nb), 8) < 3 ? 1 : 0;
    if (kind == 4) return 1;
    return nb <= 64 ? 1 : 0;
}

namespace {
// Activation rows per launch of the tiled GEMV: the matrix-core kernel's most.
size_t tiled_rows_per_launch(uint32_t kind, size_t nb) {
    return static_cast<size_t>(rk::gemv_mfma_rows(static_cast<int>(kind), static_cast<int>(nb)));
}
}  // namespace

extern "C" size_t rocknpu_hip_gemv_tiled_workspace_bytes(uint32_t kind, size_t m, size_t k, size_t rows) {
    if ((kind != 4 && kind != 6) || m == 0 || k == 0 || k % rk::kQK != 0 || rows == 0 || rows > INT32_MAX / 2)
        return 0;
    const size_t nb = k / rk::kQK, chunk = tiled_rows_per_launch(kind, nb);
    if (chunk == 0) return 0;
    const int64_t tiles = static_cast<int64_t>((rows + 15) / 16);  // 16-row tiles
    // the launches of m rows: full chunks, then the rest
    const size_t full = std::min(chunk, m), rest = m % chunk;
    return std::max(rk::gemv_tiled_split_bytes(static_cast<int>(kind), static_cast<int>(full), static_cast<int>(nb), tiles),
                    rest ? rk::gemv_tiled_split_bytes(static_cast<int>(kind), static_cast<int>(rest),
                                                      static_cast<int>(nb), tiles)
                         : size_t{0});
}

extern "C" int rocknpu_hip_gemv_tiled_workspace_check(void* workspace, void* stream) {
    // the error word is the workspace's first
    if (!workspace) return rk::kStatusInvalid;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t* word = static_cast<uint32_t*>(workspace);
    uint32_t flag = 0;
    if (hipMemcpyAsync(&flag, word, sizeof flag, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return rk::kStatusExec;
    if (flag == 0) return rk::kStatusOk;
    static const uint32_t zero = 0;
    if (hipMemcpyAsync(word, &zero, sizeof zero, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return rk::kStatusExec;
    return rk::kStatusExec;
}

extern "C" int rocknpu_hip_gemv_q8_k_tiled(uint32_t kind, const uint8_t* w, size_t w_bytes, size_t k, size_t n,
                                           const uint8_t* q8k, size_t m, float* out, size_t ldo, void* workspace,
                                           size_t workspace_bytes, void* stream) {
    if ((kind != 4 && kind != 6) || !w || !q8k || !out || k == 0 || k % rk::kQK != 0 || n == 0 || m == 0 ||
        ldo < n || n > INT32_MAX / 2)
        return rk::kStatusInvalid;
    const size_t nb = k / rk::kQK;
    if (w_bytes != rocknpu_hip_gemv_tiled_bytes(kind, k, n) || !aligned(w, 16) || !aligned(q8k, 4))
        return rk::kStatusInvalid;
    const size_t per_row = nb * rk::kQ8KBytes, chunk = tiled_rows_per_launch(kind, nb);
    if (chunk == 0) return rk::kStatusInvalid;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (size_t m0 = 0; m0 < m; m0 += chunk) {
        rk::GemvParams p{};
        p.count = 1;
        p.w[0] = w;
        p.out[0] = out + m0 * ldo;
        p.ldo[0] = static_cast<int64_t>(ldo);
        p.rows[0] = static_cast<int64_t>(n);
        p.q8k = q8k + m0 * per_row;
        p.ldx = static_cast<int64_t>(per_row);
        p.m = static_cast<int>(std::min(chunk, m - m0));
        p.nb = static_cast<int>(nb);
        p.split_ws = workspace;
        p.split_ws_bytes = workspace ? workspace_bytes : 0;
        const int st = rk::launch_gemv_tiled(static_cast<int>(kind), false, p, s);
        if (st != rk::kStatusOk) return st;
    }
    return rk::kStatusOk;
}

extern "C" int rocknpu_hip_gemv_q_f32_tiled(uint32_t kind, size_t count, const uint8_t* const* w,
                                            const size_t* w_bytes, const size_t* n, size_t k, const float* x,
                                            size_t ldx, size_t m, float* const* out, const size_t* ldo,
                                            void* workspace, size_t workspace_bytes, void* stream) {
    if ((kind != 4 && kind != 6) || count < 1 || count > static_cast<size_t>(rk::kGemvMaxMembers) || !w ||
        !w_bytes || !n || !x || !out || !ldo || k == 0 || k % rk::kQK != 0 || m == 0 || ldx < k)
        return rk::kStatusInvalid;
    if (ldx % 4 != 0 || !aligned(x, 16)) return rk::kStatusInvalid;
    const size_t nb = k / rk::kQK, chunk = tiled_rows_per_launch(kind, nb);
    if (chunk == 0) return rk::kStatusInvalid;
    size_t total = 0;
    for (size_t i = 0; i < count; ++i) {
        if (!w[i] || !out[i] || n[i] == 0 || ldo[i] < n[i] || n[i] > INT32_MAX / 2 ||
            w_bytes[i] != rocknpu_hip_gemv_tiled_bytes(kind, k, n[i]) || !aligned(w[i], 16))
            return rk::kStatusInvalid;
        total += n[i];
    }
    if (total > INT_MAX) return rk::kStatusInvalid;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (size_t m0 = 0; m0 < m; m0 += chunk) {
        rk::GemvParams p{};
        p.count = static_cast<int>(count);
        for (size_t i = 0; i < count; ++i) {
            p.w[i] = w[i];
            p.out[i] = out[i] + m0 * ldo[i];
            p.ldo[i] = static_cast<int64_t>(ldo[i]);
            p.rows[i] = static_cast<int64_t>(n[i]);
        }
        p.x = x + m0 * ldx;
        p.ldx = static_cast<int64_t>(ldx);
        p.m = static_cast<int>(std::min(chunk, m - m0));
        p.nb = static_cast<int>(nb);
        p.split_ws = workspace;
        p.split_ws_bytes = workspace ? workspace_bytes : 0;
        const int st = rk::launch_gemv_tiled(static_cast<int>(kind), true, p, s);
        if (st != rk::kStatusOk) return st;
    }
    return rk::kStatusOk;
}

extern "C" int rocknpu_hip_gemv_q_f32(uint32_t kind, size_t count, const uint8_t* const* w, const size_t* w_bytes,
                                      const size_t* n, size_t k, const float* x, size_t ldx, size_t m,
                                      float* const* out, const size_t* ldo, void* stream) {
    if ((kind != 4 && kind != 6) || count < 1 || count > static_cast<size_t>(rk::kGemvMaxMembers) || !w ||
        !w_bytes || !n || !x || !out || !ldo || k == 0 || k % rk::kQK != 0 || m == 0 || ldx < k)
        return rk::kStatusInvalid;
    if (ldx % 4 != 0 || !aligned(x, 16)) return rk::kStatusInvalid;
    const size_t bb = rk::block_bytes(static_cast<int>(kind)), nb = k / rk::kQK;
    if (nb * rk::kGemvLdsPerBlock > kGemvLdsBytes) return rk::kStatusInvalid;
    size_t total = 0;
    for (size_t i = 0; i < count; ++i) {
        if (!w[i] || !out[i] || n[i] == 0 || ldo[i] < n[i] || w_bytes[i] != n[i] * nb * bb ||
            !aligned(w[i], kind == 4 ? 16 : 2))
            return rk::kStatusInvalid;
        total += n[i];
    }
    if (total > INT_MAX) return rk::kStatusInvalid;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (size_t m0 = 0, chunk = 0; m0 < m; m0 += chunk) {
        chunk = gemv_rows_per_launch(kind, nb, m - m0, static_cast<int64_t>(total), false, rk::device_cu_count());
        rk::GemvParams p{};
        p.count = static_cast<int>(count);
        for (size_t i = 0; i < count; ++i) {
            p.w[i] = w[i];
            p.out[i] = out[i] + m0 * ldo[i];
            p.ldo[i] = static_cast<int64_t>(ldo[i]);
            p.rows[i] = static_cast<int64_t>(n[i]);
        }
        p.x = x + m0 * ldx;
        p.ldx = static_cast<int64_t>(ldx);
        p.m = static_cast<int>(std::min(chunk, m - m0));
        p.nb = static_cast<int>(nb);
        const int st = rk::launch_gemv(static_cast<int>(kind), true, p, s);
        if (st != rk::kStatusOk) return st;
    }
    return rk::kStatusOk;
}
