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
// next 256-byte boundary.
size_t scales_bytes(size_t m) { return (m * sizeof(float) + 255) / 256 * 256; }

bool matmul_args_ok(const float* a, size_t m, size_t k, size_t lda, const int8_t* w8, const float* w_scales,
                    size_t n, size_t k_pad, const float* out, size_t ldo) {
    return a && w8 && w_scales && out && m > 0 && k > 0 && n > 0 && lda >= k && k_pad >= k && k_pad % 64 == 0 &&
           k_pad <= rk::kMaxExactK && ldo >= n && m <= INT_MAX && n <= INT_MAX && aligned(w8, 16);
}

int run(const float* a, size_t m, size_t k, size_t lda, const int8_t* w8, const float* w_scales, size_t n,
        size_t k_pad, float* out, size_t ldo, uint8_t* workspace, void* stream) {
    float* as = reinterpret_cast<float*>(workspace);
    int8_t* a8 = reinterpret_cast<int8_t*>(workspace + scales_bytes(m));
    const int st = rocknpu_hip_quantize_a8(a, m, k, lda, k_pad, a8, as, stream);
    if (st != rk::kStatusOk) return st;
    return rocknpu_hip_gemm_w8a8(a8, as, w8, w_scales, m, n, k_pad, out, ldo, nullptr, stream);
}

// The no-allocation variant's workspace: a fixed array in device memory, one
// copy per GPU, held until the process ends. Scales of at most kNoAllocRows
// rows, then A8 of at most kNoAllocA8Bytes (the layout above: A8 starts at
// scales_bytes(m) <= kNoAllocRows * 4).
constexpr size_t kNoAllocRows = 16384;
constexpr size_t kNoAllocA8Bytes = size_t{32} << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocRows * sizeof(float) + kNoAllocA8Bytes];

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
    void* ws = nullptr;
    if (hipMallocAsync(&ws, scales_bytes(m) + m * k_pad, s) != hipSuccess) return rk::kStatusExec;
    const int st = run(a, m, k, lda, w8, w_scales, n, k_pad, out, ldo, static_cast<uint8_t*>(ws), stream);
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
    return run(a, m, k, lda, w8, w_scales, n, k_pad, out, ldo, ws, stream);
}
