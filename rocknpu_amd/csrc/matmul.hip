// The W8A8 prompt route on device buffers: per-token int8 quantisation of f32
// activations into an A8 workspace, then the int8 matrix-core GEMM against a
// resident W8 with the f32 rescale. The sequence of
// execute_cached_w8a8_mtile_pool_padded (crates/rocknpu-capi/src/lib.rs:
// 1776-1791 quantise, :1868-1884 GEMM + rescale) without its weight cache.
#include <climits>
#include <cstdio>
#include <mutex>

#include "common.h"
#include "rocknpu_hip.h"

namespace {

bool aligned(const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

// Workspace layout: the m f32 activation scales, then A8 [m, k_pad] from the
// next 256-byte boundary, then the GEMM's K-split workspace (tile counters,
// i32 partial tiles) from the 256-byte boundary after that.
size_t scales_bytes(size_t m) { return (m * sizeof(float) + 255) / 256 * 256; }
size_t a8_end(size_t m, size_t k_pad) { return scales_bytes(m) + (m * k_pad + 255) / 256 * 256; }
size_t split_bytes(size_t m, size_t n, size_t k_pad) {
    const rk::GemmTile r =
        rk::gemm_route(static_cast<int>(m), static_cast<int>(n), static_cast<int>(k_pad), rk::device_cu_count());
    return rk::gemm_workspace_bytes(r, static_cast<int>(m), static_cast<int>(n));
}

bool matmul_args_ok(const float* a, size_t m, size_t k, size_t lda, const int8_t* w8, const float* w_scales,
                    size_t n, size_t k_pad, const float* out, size_t ldo) {
    return a && w8 && w_scales && out && m > 0 && k > 0 && n > 0 && lda >= k && k_pad >= k && k_pad % 64 == 0 &&
           k_pad <= rk::kMaxExactK && ldo >= n && m <= INT_MAX && n <= INT_MAX && aligned(w8, 16);
}

// Quantise, then multiply. `split_avail` bytes follow the A8 for the GEMM's
// K split: when the routed split fits, the quantiser clears its counters (the
// GEMM leaves them zero too), else the GEMM runs unsplit; results are the same
// either way.
int run(const float* a, size_t m, size_t k, size_t lda, const int8_t* w8, const float* w_scales, size_t n,
        size_t k_pad, float* out, size_t ldo, uint8_t* workspace, size_t split_avail, void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    float* as = reinterpret_cast<float*>(workspace);
    int8_t* a8 = reinterpret_cast<int8_t*>(workspace + scales_bytes(m));
    uint8_t* split = workspace + a8_end(m, k_pad);
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k_pad);
    const rk::GemmTile r = rk::gemm_route(mi, ni, ki, rk::device_cu_count());
    const size_t need = rk::gemm_workspace_bytes(r, mi, ni);
    const bool use = need > 0 && need <= split_avail;
    const int st = rk::launch_quantize_a8(a, static_cast<int64_t>(m), static_cast<int64_t>(k), static_cast<int64_t>(lda),
                                          static_cast<int64_t>(k_pad), a8, as,
                                          use ? reinterpret_cast<uint32_t*>(split) : nullptr,
                                          use ? rk::gemm_workspace_counters(r, mi, ni) : 0, s);
    if (st != rk::kStatusOk) return st;
    return rk::launch_gemm_w8a8(a8, static_cast<int64_t>(k_pad), w8, static_cast<int64_t>(k_pad), as, w_scales, mi, ni,
                                ki, out, static_cast<int64_t>(ldo), nullptr, 0, use ? split : nullptr, use ? need : 0, s);
}

// The no-allocation variant's workspace: a fixed array in device memory, one
// copy per GPU, held until the process ends. Scales of at most kNoAllocRows
// rows, then A8 of at most kNoAllocA8Bytes (the layout above: A8 starts at
// scales_bytes(m) <= kNoAllocRows * 4).
// Then the GEMM's K-split workspace: 4 MiB + 17 KiB holds every split the
// route takes on up to 256 CUs (the counter block, then at most 256 units of a
// 64 x 64 i32 tile and their 256 stamps); a larger split runs unsplit instead.
constexpr size_t kNoAllocRows = 16384;
constexpr size_t kNoAllocA8Bytes = size_t{32} << 20;
constexpr size_t kNoAllocSplitBytes = (size_t{4} << 20) + rk::kSplitCounterBytes + 1024;
constexpr size_t kScratchBytes = kNoAllocRows * sizeof(float) + kNoAllocA8Bytes + kNoAllocSplitBytes;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// scratch's address on each device, looked up (with that device current) by
// the first call on the device. Host code uses these, never the array's name.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices] = {};

uint8_t* scratch_on(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        int cur = 0;
        if (hipGetDevice(&cur) != hipSuccess) return nullptr;
        if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess || p == nullptr) return nullptr;
        g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int rocknpu_hip_matmul_w8a8_f32(const float* a, size_t m, size_t k, size_t lda, const int8_t* w8,
                                           const float* w_scales, size_t n, size_t k_pad, float* out, size_t ldo,
                                           void* stream) {
    if (!matmul_args_ok(a, m, k, lda, w8, w_scales, n, k_pad, out, ldo)) return rk::kStatusInvalid;
    if (m > (SIZE_MAX - 256) / (k_pad + sizeof(float))) return rk::kStatusInvalid;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t split = split_bytes(m, n, k_pad);
    void* ws = nullptr;
    if (hipMallocAsync(&ws, a8_end(m, k_pad) + split, s) != hipSuccess) return rk::kStatusExec;
    const int st = run(a, m, k, lda, w8, w_scales, n, k_pad, out, ldo, static_cast<uint8_t*>(ws), split, stream);
    const hipError_t fe = hipFreeAsync(ws, s);
    if (st != rk::kStatusOk) return st;
    return fe == hipSuccess ? rk::kStatusOk : rk::kStatusExec;
}

extern "C" int rocknpu_hip_matmul_w8a8_f32_noalloc(const float* a, size_t m, size_t k, size_t lda, const int8_t* w8,
                                                   const float* w_scales, size_t n, size_t k_pad, float* out,
                                                   size_t ldo, void* stream) {
    if (!matmul_args_ok(a, m, k, lda, w8, w_scales, n, k_pad, out, ldo)) return rk::kStatusInvalid;
    if (m > kNoAllocRows || m * k_pad > kNoAllocA8Bytes) {
        std::fprintf(stderr,
                     "rocknpu_hip_matmul_w8a8_f32_noalloc: m = %zu, m * k_pad = %zu beyond the fixed workspace "
                     "(at most %zu rows and %zu bytes)\n",
                     m, m * k_pad, kNoAllocRows, kNoAllocA8Bytes);
        return rk::kStatusInvalid;
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int dev = 0;
    if ((s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev)) != hipSuccess) return rk::kStatusDevice;
    uint8_t* ws = scratch_on(dev);
    if (ws == nullptr) return rk::kStatusDevice;
    return run(a, m, k, lda, w8, w_scales, n, k_pad, out, ldo, ws, kScratchBytes - a8_end(m, k_pad), stream);
}
