// Host side of the C ABI in include/rocknpu.h (and the decode extension in
// include/rocknpu_ggml.h): argument validation with the reference's status
// codes, a device-resident W8 cache keyed like the reference's
// DecodeWeightKey, and the W8A8 pipeline (upload -> A8 quant -> int8-MFMA GEMM
// with fused rescale -> download) on one HIP stream per context.
//
// Reference: crates/rocknpu-capi/src/lib.rs. Routing differences, by design:
// the NPU tile constraints (M in {4..128}, K % 512, N <= 8192, K-split,
// 128-row chunking, N chunking, K zero-padding) are numerically invisible in
// the reference and have no GPU counterpart, so every M > 1 shape runs as one
// GEMM; M = 1 runs the same W8A8 formula (lib.rs:1567-1701).
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "context.h"
#include "rocknpu.h"
#include "rocknpu_ggml.h"
#include "rocknpu_hip.h"

namespace {

constexpr int kOk = ROCKNPU_STATUS_OK;
constexpr int kInvalid = ROCKNPU_STATUS_INVALID_ARGUMENT;
constexpr int kExec = ROCKNPU_STATUS_EXECUTION_ERROR;
constexpr size_t kQK = 256;

size_t block_bytes(uint32_t kind) { return kind == 4 ? 144 : kind == 5 ? 176 : kind == 6 ? 210 : 0; }
using rk::round_up;

bool env_enabled(const char* name) {
    const char* v = std::getenv(name);
    return v && v[0] != '\0' && std::strcmp(v, "0") != 0;
}

bool mul_ok(size_t a, size_t b, size_t* out) { return !__builtin_mul_overflow(a, b, out); }

uint64_t now_ns() {
    return static_cast<uint64_t>(std::chrono::duration_cast<std::chrono::nanoseconds>(
                                     std::chrono::steady_clock::now().time_since_epoch())
                                     .count());
}

using rk::DecodeWeight;
using rk::DevBuf;
using rk::DeviceW8;
using rk::KeyHash;
using rk::PinnedBuf;
using rk::Profile;
using rk::W8Ptr;
using rk::WeightKey;

}  // namespace

namespace {

bool hip_ok(hipError_t e, RockNpuContext* ctx, const char* what) {
    if (e == hipSuccess) return true;
    if (ctx && ctx->trace) std::fprintf(stderr, "ROCKNPU MTILE ERROR %s: %s\n", what, hipGetErrorString(e));
    return false;
}

void run_overlap(RockNpuContext* ctx) {
    rocknpu_overlap_fn fn = ctx->overlap;
    void* user = ctx->overlap_user;
    ctx->overlap = nullptr;
    ctx->overlap_user = nullptr;
    if (fn) fn(user);
}

// Look a cached W8 up in `primary`, else reuse the same weight's entry from
// the other cache (both hold identical W8 for a key).
W8Ptr find_w8(std::unordered_map<WeightKey, W8Ptr, KeyHash>& primary,
              std::unordered_map<WeightKey, W8Ptr, KeyHash>& other, const WeightKey& key) {
    auto it = primary.find(key);
    if (it != primary.end()) return it->second;
    auto jt = other.find(key);
    if (jt != other.end()) {
        primary.emplace(key, jt->second);
        return jt->second;
    }
    return nullptr;
}

W8Ptr alloc_w8(size_t n, size_t k) {
    auto w = std::make_shared<DeviceW8>();
    w->n = n;
    w->k = k;
    w->k_pad = round_up(k, 64);
    if (hipMalloc(reinterpret_cast<void**>(&w->w8), w->n * w->k_pad) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&w->scales), w->n * sizeof(float)) != hipSuccess)
        return nullptr;
    return w;
}

// Repack raw K-quant rows into rows [row0, row0 + n) of `dst`; returns
// kInvalid when a dequantised row is non-finite (prepare_* returns None).
int repack_into(RockNpuContext* ctx, uint32_t kind, const uint8_t* host, size_t bytes, size_t k, size_t n,
                DeviceW8& dst, size_t row0) {
    if (!ctx->d_raw.ensure(bytes) || !ctx->h_as.ensure(n * sizeof(float))) return kExec;
    if (!hip_ok(hipMemcpyAsync(ctx->d_raw.p, host, bytes, hipMemcpyHostToDevice, ctx->stream), ctx, "upload"))
        return kExec;
    int st = rocknpu_hip_repack_w8(kind, ctx->d_raw.as<uint8_t>(), bytes, k, n, dst.k_pad,
                                   dst.w8 + row0 * dst.k_pad, dst.scales + row0, ctx->stream);
    if (st != kOk) return st;
    if (!hip_ok(hipMemcpyAsync(ctx->h_as.p, dst.scales + row0, n * sizeof(float), hipMemcpyDeviceToHost,
                               ctx->stream),
                ctx, "scales") ||
        !hip_ok(hipStreamSynchronize(ctx->stream), ctx, "repack"))
        return kExec;
    const float* s = ctx->h_as.as<float>();
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(s[i])) return kInvalid;
    return kOk;
}

// Copy caller int8 [n, k] + scales into rows [row0, row0 + n) of `dst`.
int upload_w8_into(RockNpuContext* ctx, const int8_t* w, const float* scales, size_t k, size_t n, DeviceW8& dst,
                   size_t row0) {
    int8_t* d = dst.w8 + row0 * dst.k_pad;
    if (dst.k_pad != k) {
        if (!hip_ok(hipMemsetAsync(d, 0, n * dst.k_pad, ctx->stream), ctx, "pad")) return kExec;
        if (!hip_ok(hipMemcpy2DAsync(d, dst.k_pad, w, k, k, n, hipMemcpyHostToDevice, ctx->stream), ctx, "w8"))
            return kExec;
    } else if (!hip_ok(hipMemcpyAsync(d, w, n * k, hipMemcpyHostToDevice, ctx->stream), ctx, "w8")) {
        return kExec;
    }
    if (!hip_ok(hipMemcpyAsync(dst.scales + row0, scales, n * sizeof(float), hipMemcpyHostToDevice, ctx->stream),
                ctx, "scales") ||
        !hip_ok(hipStreamSynchronize(ctx->stream), ctx, "upload"))
        return kExec;
    return kOk;
}

// One projection source for a (possibly concatenated) W8 matrix.
struct Source {
    WeightKey key;
    const uint8_t* blocks;   // raw K-quant rows (kind 4/5/6), or
    const int8_t* w8;        // caller int8 rows (kind 8)
    const float* scales;
};

int build_w8(RockNpuContext* ctx, const std::vector<Source>& srcs, size_t k, W8Ptr* out) {
    size_t total_n = 0;
    for (const auto& s : srcs) total_n += s.key.n;
    W8Ptr w = alloc_w8(total_n, k);
    if (!w) return kExec;
    size_t row = 0;
    for (const auto& s : srcs) {
        const int st = s.key.kind == 8 ? upload_w8_into(ctx, s.w8, s.scales, k, s.key.n, *w, row)
                                       : repack_into(ctx, s.key.kind, s.blocks, s.key.bytes, k, s.key.n, *w, row);
        if (st != kOk) return st;
        row += s.key.n;
    }
    *out = w;
    return kOk;
}

// Two-part activation encoding of prompt projections (lib.rs:2005-2083):
// each activation row x is quantised as usual, its residual
// r = x - f32(q) * scale (f32, no contraction) is stacked as an extra row,
// both run through the same W8A8 GEMM, and the two output halves are added.
// ROCKNPU_PREFILL_HILO "1"/"all": every prompt projection (M >= 2); "down":
// only wide-K ones (K > 4096 or K not a multiple of 512).
int hilo_mode_from_env() {
    const char* v = std::getenv("ROCKNPU_PREFILL_HILO");
    if (!v) return 0;
    if (std::strcmp(v, "1") == 0 || std::strcmp(v, "all") == 0) return 2;
    if (std::strcmp(v, "down") == 0) return 1;
    return 0;
}

bool hilo_applies(const RockNpuContext* ctx, size_t m, size_t k) {
    if (ctx->hilo == 0 || m < 2 || k == 0) return false;
    return !(ctx->hilo == 1 && k <= 4096 && k % 512 == 0);
}

// Rows m..2m-1 of act = x - f32(a8) * scale of rows 0..m-1.
__global__ void hilo_residual_kernel(float* __restrict__ act, const int8_t* __restrict__ a8,
                                     const float* __restrict__ scales, int64_t m, int64_t k, int64_t k_pad) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= m * k) return;
    const int64_t r = idx / k, c = idx % k;
    const float deq = static_cast<float>(a8[r * k_pad + c]) * scales[r];
    act[(m + r) * k + c] = act[idx] - deq;
}

// out[r, :] += out[m + r, :] for rows r < m of an [2m, n] output.
__global__ void hilo_sum_kernel(float* __restrict__ out, int64_t m, int64_t n) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= m * n) return;
    out[idx] = out[idx] + out[m * n + idx];
}

// h[i] = (g * (1 / (1 + exp(-g)))) * u with g = gu[i], u = gu[n + i]: the
// reference's SwiGLU between the gate/up and down projections
// (crates/rocknpu-capi/src/lib.rs:4378-4383), on the device. expf is the
// device library's (within an ulp or two of the host's std::exp).
__global__ void swiglu_kernel(const float* __restrict__ gu, float* __restrict__ h, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float g = gu[i], u = gu[n + i];
    const float sig = 1.0f / (1.0f + expf(-g));
    h[i] = g * sig * u;
}

// Quantise host activations [m, k], run the GEMM against `w`, download and
// scatter the columns into outs[i] ([m, ns[i]] each, ns summing to w->n).
// `hilo_ok`: the entry point is one the two-part encoding serves.
int run_w8a8(RockNpuContext* ctx, const DeviceW8& w, const float* act, size_t m, size_t k,
             const std::vector<float*>& outs, const std::vector<size_t>& ns, bool decode, bool hilo_ok = false) {
    const bool hilo = hilo_ok && hilo_applies(ctx, m, k);
    const size_t rows = hilo ? 2 * m : m;  // GEMM rows
    size_t a_bytes, o_elems, a_rows_bytes, o_rows;
    if (!mul_ok(m, k, &a_bytes) || !mul_ok(a_bytes, sizeof(float), &a_bytes) || !mul_ok(m, w.n, &o_elems) ||
        !mul_ok(rows, k * sizeof(float), &a_rows_bytes) || !mul_ok(rows, w.n, &o_rows))
        return kInvalid;
    if (!ctx->d_act.ensure(a_rows_bytes) || !ctx->d_a8.ensure(rows * w.k_pad) ||
        !ctx->d_as.ensure(rows * sizeof(float)) || !ctx->d_out.ensure(o_rows * sizeof(float)) ||
        !ctx->h_out.ensure(o_elems * sizeof(float)) || !ctx->h_as.ensure(rows * sizeof(float)))
        return kExec;
    // the GEMM's K-split workspace; the (first) quantisation clears its
    // counters and error word
    const rk::GemmTile route = rk::gemm_route(static_cast<int>(rows), static_cast<int>(w.n),
                                              static_cast<int>(w.k_pad), rk::device_cu_count());
    const size_t split = rk::gemm_workspace_bytes(route, static_cast<int>(rows), static_cast<int>(w.n));
    if (split > 0 && (!ctx->d_split.ensure(split) || !ctx->h_err.ensure(sizeof(uint32_t)))) return kExec;
    if (!hip_ok(hipMemcpyAsync(ctx->d_act.p, act, a_bytes, hipMemcpyHostToDevice, ctx->stream), ctx, "act"))
        return kExec;
    int st = rk::launch_quantize_a8(ctx->d_act.as<float>(), static_cast<int64_t>(m), static_cast<int64_t>(k),
                                    static_cast<int64_t>(k), static_cast<int64_t>(w.k_pad), ctx->d_a8.as<int8_t>(),
                                    ctx->d_as.as<float>(), split > 0 ? ctx->d_split.as<uint32_t>() : nullptr,
                                    split > 0 ? rk::kSplitCounterWords : 0, ctx->stream);
    if (st != kOk) return st;
    if (hilo) {
        const int64_t total = static_cast<int64_t>(m * k);
        hilo_residual_kernel<<<static_cast<unsigned>((total + 255) / 256), 256, 0, ctx->stream>>>(
            ctx->d_act.as<float>(), ctx->d_a8.as<int8_t>(), ctx->d_as.as<float>(), static_cast<int64_t>(m),
            static_cast<int64_t>(k), static_cast<int64_t>(w.k_pad));
        if (!hip_ok(hipGetLastError(), ctx, "hilo residual")) return kExec;
        st = rocknpu_hip_quantize_a8(ctx->d_act.as<float>() + m * k, m, k, k, w.k_pad, ctx->d_a8.as<int8_t>() + m * w.k_pad,
                                     ctx->d_as.as<float>() + m, ctx->stream);
        if (st != kOk) return st;
    }
    st = rocknpu_hip_gemm_w8a8_ws(ctx->d_a8.as<int8_t>(), ctx->d_as.as<float>(), w.w8, w.scales, rows, w.n, w.k_pad,
                                  ctx->d_out.as<float>(), w.n, nullptr, split > 0 ? ctx->d_split.p : nullptr, split,
                                  ctx->stream);
    if (st != kOk) return st;
    // a split GEMM that found dirty counters set the workspace's error word
    if (split > 0 && !hip_ok(hipMemcpyAsync(ctx->h_err.p, ctx->d_split.as<uint32_t>() + rk::kSplitErrorWord,
                                            sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream),
                             ctx, "download"))
        return kExec;
    if (hilo) {
        const int64_t total = static_cast<int64_t>(o_elems);
        hilo_sum_kernel<<<static_cast<unsigned>((total + 255) / 256), 256, 0, ctx->stream>>>(
            ctx->d_out.as<float>(), static_cast<int64_t>(m), static_cast<int64_t>(w.n));
        if (!hip_ok(hipGetLastError(), ctx, "hilo sum")) return kExec;
    }
    if (!hip_ok(hipMemcpyAsync(ctx->h_out.p, ctx->d_out.p, o_elems * sizeof(float), hipMemcpyDeviceToHost,
                               ctx->stream),
                ctx, "download") ||
        !hip_ok(hipMemcpyAsync(ctx->h_as.p, ctx->d_as.p, rows * sizeof(float), hipMemcpyDeviceToHost, ctx->stream),
                ctx, "download"))
        return kExec;
    if (decode) run_overlap(ctx);
    if (!hip_ok(hipStreamSynchronize(ctx->stream), ctx, "execute")) return kExec;
    if (split > 0 && *ctx->h_err.as<uint32_t>() != 0) {
        if (ctx->trace) std::fprintf(stderr, "rocknpu: K-split workspace counters were not zero\n");
        return kExec;
    }
    const float* as = ctx->h_as.as<float>();
    for (size_t r = 0; r < rows; ++r)
        if (!std::isfinite(as[r])) return kInvalid;  // non-finite activation row
    const float* h = ctx->h_out.as<float>();
    size_t col = 0;
    for (size_t i = 0; i < outs.size(); ++i) {
        for (size_t r = 0; r < m; ++r) std::memcpy(outs[i] + r * ns[i], h + r * w.n + col, ns[i] * sizeof(float));
        col += ns[i];
    }
    return kOk;
}

// The int8 GEMM's int32 sums are exact up to K = 133120 (127 * 127 * K < 2^31);
// longer rows are rejected before any weight is uploaded or repacked.
bool w8a8_k_ok(size_t k) { return round_up(k, 64) <= 133120; }

// The cached W8 of one projection (M > 1 -> prompt cache, M = 1 -> decode
// cache), built on a miss.
int single_w8(RockNpuContext* ctx, const Source& src, bool decode, W8Ptr* w, bool* hit) {
    auto& primary = decode ? ctx->m1 : ctx->mtile;
    auto& other = decode ? ctx->mtile : ctx->m1;
    *w = find_w8(primary, other, src.key);
    *hit = *w != nullptr;
    if (*hit) return kOk;
    const int st = build_w8(ctx, {src}, src.key.k, w);
    if (st != kOk) return st;
    primary.emplace(src.key, *w);
    return kOk;
}

// The cached concatenated W8 of a same-input group, built on a miss.
int group_w8(RockNpuContext* ctx, const std::vector<Source>& srcs, bool decode, W8Ptr* w, bool* hit) {
    std::vector<WeightKey> keys;
    for (const auto& s : srcs) keys.push_back(s.key);
    auto& cache = decode ? ctx->m1_groups : ctx->mtile_groups;
    auto it = cache.find(keys);
    *hit = it != cache.end();
    if (*hit) {
        *w = it->second;
        return kOk;
    }
    const int st = build_w8(ctx, srcs, srcs[0].key.k, w);
    if (st != kOk) return st;
    cache.emplace(keys, *w);
    return kOk;
}

// Cached single-projection W8A8 (M > 1 -> prompt cache, M = 1 -> decode cache).
int exec_single(RockNpuContext* ctx, const Source& src, const float* act, float* out, size_t m,
                bool hilo_ok = false) {
    if (!w8a8_k_ok(src.key.k)) return kInvalid;
    const bool decode = m == 1;
    const uint64_t t0 = now_ns();
    W8Ptr w;
    bool hit = false;
    if (const int st0 = single_w8(ctx, src, decode, &w, &hit); st0 != kOk) return st0;
    const uint64_t t1 = now_ns();
    const int st = run_w8a8(ctx, *w, act, m, src.key.k, {out}, {src.key.n}, decode, hilo_ok);
    const uint64_t t2 = now_ns();
    Profile& p = decode ? ctx->m1_profile : ctx->mtile_profile;
    p.calls++;
    (hit ? p.cache_hits : p.cache_misses)++;
    p.prepare_ns += t1 - t0;
    p.execute_ns += t2 - t1;
    if (decode) {
        ctx->m1_calls++;
        if (hit) {
            ctx->hits++;
            ctx->hit_ns += t2 - t0;
        } else {
            ctx->misses++;
            ctx->miss_ns += t2 - t0;
        }
    }
    return st;
}

// Cached concatenated-N group: one GEMM, activations quantised once.
int exec_group(RockNpuContext* ctx, const std::vector<Source>& srcs, const float* act, size_t m,
               const std::vector<float*>& outs, bool hilo_ok = false) {
    if (!w8a8_k_ok(srcs[0].key.k)) return kInvalid;
    const bool decode = m == 1;
    std::vector<size_t> ns;
    for (const auto& s : srcs) ns.push_back(s.key.n);
    const uint64_t t0 = now_ns();
    W8Ptr w;
    bool hit = false;
    if (const int st0 = group_w8(ctx, srcs, decode, &w, &hit); st0 != kOk) return st0;
    const int st = run_w8a8(ctx, *w, act, m, srcs[0].key.k, outs, ns, decode, hilo_ok);
    const uint64_t t1 = now_ns();
    if (decode) {
        ctx->m1_calls++;
        if (hit) {
            ctx->hits++;
            ctx->hit_ns += t1 - t0;
        } else {
            ctx->misses++;
            ctx->miss_ns += t1 - t0;
        }
    }
    return st;
}

bool kquant_kind(uint32_t kind) { return kind == 4 || kind == 6; }

// Validate a raw K-quant projection: lib.rs:4944-4975.
bool kquant_shape_ok(uint32_t kind, size_t bytes, size_t k, size_t n) {
    const size_t bb = block_bytes(kind);
    size_t expected;
    return bb != 0 && k != 0 && n != 0 && k % kQK == 0 && mul_ok(n, k / kQK, &expected) &&
           mul_ok(expected, bb, &expected) && expected == bytes;
}

bool scales_ok(const float* s, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(s[i]) || s[i] <= 0.0f) return false;
    return true;
}

Source kquant_source(const uint8_t* w, size_t bytes, uint32_t kind, size_t k, size_t n) {
    return Source{WeightKey{reinterpret_cast<uintptr_t>(w), bytes, k, n, kind}, w, nullptr, nullptr};
}

Source w8_source(const int8_t* w, const float* scales, size_t k, size_t n) {
    return Source{WeightKey{reinterpret_cast<uintptr_t>(w), k * n, k, n, 8}, nullptr, w, scales};
}

int matmul_kquant(rocknpu_context* ctx, uint32_t kind, const uint8_t* w, size_t bytes, const float* act,
                  float* out, size_t m, size_t k, size_t n) {
    if (!ctx || !w || !act || !out || m == 0 || k == 0 || n == 0 || k % kQK != 0) return kInvalid;
    size_t tmp;
    if (!mul_ok(m, k, &tmp) || !mul_ok(n, k, &tmp) || !mul_ok(m, n, &tmp)) return kInvalid;
    if (!kquant_shape_ok(kind, bytes, k, n)) return kInvalid;
    if (kind == 5 && m == 1) return kInvalid;  // Q5_K is a prompt-path format (lib.rs:5300)
    // the two-part encoding serves the Q4_K and Q6_K entries (lib.rs:4981, 5428)
    return exec_single(ctx, kquant_source(w, bytes, kind, k, n), act, out, m, kind != 5);
}

// Minimal FP16 bridge kernel: activations rounded to f16 (RNE), f16 weights,
// f32 accumulation; one thread per output.
__global__ void f16_matmul_kernel(const _Float16* __restrict__ w, const float* __restrict__ a, float* __restrict__ out,
                                  int64_t m, int64_t k, int64_t n) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= m * n) return;
    const int64_t r = idx / n, c = idx % n;
    float acc = 0.0f;
    for (int64_t t = 0; t < k; ++t) {
        const float x = static_cast<float>(static_cast<_Float16>(a[r * k + t]));
        acc += x * static_cast<float>(w[c * k + t]);
    }
    out[idx] = acc;
}

}  // namespace

namespace rk {

void route_print_summary(const RockNpuContext* ctx);  // route.hip

// K-quant blocks (kind 4/5/6) of an [n, k] weight -> host W8 [n, k] + scales,
// repacked on the context's GPU (the conversion half of the W8 sidecar).
int context_repack_to_host(rocknpu_context* ctx, uint32_t kind, const uint8_t* source, size_t bytes, size_t k,
                           size_t n, int8_t* w8, float* scales) {
    if (!ctx || !source || !w8 || !scales || (kind != 4 && kind != 5 && kind != 6) ||
        !kquant_shape_ok(kind, bytes, k, n))
        return kInvalid;
    W8Ptr w = alloc_w8(n, k);
    if (!w) return kExec;
    int st = repack_into(ctx, kind, source, bytes, k, n, *w, 0);
    if (st != kOk) return st;
    if (!hip_ok(hipMemcpy2DAsync(w8, k, w->w8, w->k_pad, k, n, hipMemcpyDeviceToHost, ctx->stream), ctx, "w8") ||
        !hip_ok(hipMemcpyAsync(scales, w->scales, n * sizeof(float), hipMemcpyDeviceToHost, ctx->stream), ctx,
                "scales") ||
        !hip_ok(hipStreamSynchronize(ctx->stream), ctx, "download"))
        return kExec;
    return kOk;
}

}  // namespace rk

namespace {
// The K-quant blocks of a weight, resident on the device under the
// reference's cache key: the raw rows uploaded on first use, and for calls of
// two or more rows (`tiled`) their tile-interleaved copy, written once on the
// device from the raw rows.
std::shared_ptr<DecodeWeight> raw_weights(RockNpuContext* ctx, const uint8_t* w, size_t bytes, size_t k, size_t n,
                                          uint32_t kind, bool tiled, bool* hit) {
    const WeightKey key{reinterpret_cast<uintptr_t>(w), bytes, k, n, kind};
    std::shared_ptr<DecodeWeight> dw;
    auto it = ctx->raw.find(key);
    if (it != ctx->raw.end()) {
        dw = it->second;
    } else {
        *hit = false;
        dw = std::make_shared<DecodeWeight>();
        if (!dw->raw.ensure(bytes) ||
            !hip_ok(hipMemcpyAsync(dw->raw.p, w, bytes, hipMemcpyHostToDevice, ctx->stream), ctx, "raw"))
            return nullptr;
        dw->raw_bytes = bytes;
        ctx->raw.emplace(key, dw);
    }
    if (tiled && dw->tiled_bytes == 0) {
        *hit = false;
        const size_t tb = rocknpu_hip_gemv_tiled_bytes(kind, k, n);
        if (tb == 0 || !dw->tiled.ensure(tb) ||
            rocknpu_hip_gemv_tile_weights(kind, dw->raw.as<uint8_t>(), bytes, k, n, dw->tiled.as<uint8_t>(), tb,
                                          ctx->stream) != kOk)
            return nullptr;
        dw->tiled_bytes = tb;
    }
    return dw;
}

// Whether a decode call reads the tiled copies (rocknpu_hip_gemv_tiled_preferred:
// from two rows, and Q4_K rows of 16 or more blocks at one row).
bool decode_tiled(uint32_t kind, size_t m, size_t k) { return rocknpu_hip_gemv_tiled_preferred(kind, m, k) != 0; }

// The tiled GEMV's K-split workspace for a launch of m rows over `rows` output
// rows: null when that launch does not split. Zeroed when (re)allocated; every
// completed launch leaves it zero, and gemv_split_failed zeroes it again after
// a launch that found it dirty.
bool gemv_split_ws(RockNpuContext* ctx, uint32_t kind, size_t m, size_t k, size_t rows, void** ws, size_t* bytes) {
    *bytes = rocknpu_hip_gemv_tiled_workspace_bytes(kind, m, k, rows);
    *ws = nullptr;
    if (*bytes == 0) return true;
    const size_t before = ctx->d_gemv_split.cap;
    if (!ctx->d_gemv_split.ensure(*bytes) || !ctx->h_err.ensure(sizeof(uint32_t))) return false;
    if (ctx->d_gemv_split.cap != before &&
        !hip_ok(hipMemsetAsync(ctx->d_gemv_split.p, 0, ctx->d_gemv_split.cap, ctx->stream), ctx, "gemv split"))
        return false;
    *ws = ctx->d_gemv_split.p;
    *bytes = ctx->d_gemv_split.cap;
    return true;
}
// Queues the download of the workspace's error word (read after the sync).
bool gemv_split_queue_check(RockNpuContext* ctx) {
    return hip_ok(hipMemcpyAsync(ctx->h_err.p, ctx->d_gemv_split.p, sizeof(uint32_t), hipMemcpyDeviceToHost,
                                 ctx->stream),
                  ctx, "gemv split");
}
// After the sync: whether a split launch found the workspace dirty (its
// results are NaN where it did); the workspace is zeroed again then.
bool gemv_split_failed(RockNpuContext* ctx) {
    if (*ctx->h_err.as<uint32_t>() == 0) return false;
    if (ctx->trace) std::fprintf(stderr, "ROCKNPU DECODE ERROR gemv: K-split workspace was not clear\n");
    (void)hipMemsetAsync(ctx->d_gemv_split.p, 0, ctx->d_gemv_split.cap, ctx->stream);
    (void)hipStreamSynchronize(ctx->stream);
    return true;
}

// Decode-cache accounting of one decode call (the reference's
// decode_cache_hits / misses and their ns, lib.rs:3821-3826): a hit when every
// weight was resident.
void record_decode(RockNpuContext* ctx, bool hit, uint64_t t0) {
    const uint64_t dt = now_ns() - t0;
    ctx->m1_calls++;
    if (hit) {
        ctx->hits++;
        ctx->hit_ns += dt;
    } else {
        ctx->misses++;
        ctx->miss_ns += dt;
    }
}
}  // namespace

extern "C" {

size_t rocknpu_device_count(void) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess) return 0;
    return count > 0 ? 1 : 0;
}

rocknpu_context* rocknpu_context_create(void) {
    if (rocknpu_device_count() == 0) return nullptr;
    auto* ctx = new (std::nothrow) RockNpuContext();
    if (!ctx) return nullptr;
    if (hipGetDevice(&ctx->device) != hipSuccess || hipStreamCreate(&ctx->stream) != hipSuccess) {
        delete ctx;
        return nullptr;
    }
    ctx->profile_mtile = env_enabled("ROCKNPU_MTILE_PROFILE");
    ctx->profile_m1 = env_enabled("ROCKNPU_M1_PROFILE");
    ctx->trace = env_enabled("ROCKNPU_MTILE_TRACE");
    ctx->hilo = hilo_mode_from_env();
    return ctx;
}

int rocknpu_context_decode_cache_stats(const rocknpu_context* ctx, rocknpu_decode_cache_stats* out) {
    if (!ctx || !out) return kInvalid;
    // the decode caches: W8 of the W8A8 M=1 entries and the raw K-quant blocks
    // the Q8_K decode GEMV reads (lib.rs:3785-3848 counts its decode caches)
    size_t resident = 0;
    for (const auto& e : ctx->m1) resident += e.second->resident_bytes();
    for (const auto& e : ctx->m1_groups) resident += e.second->resident_bytes();
    for (const auto& e : ctx->raw) resident += e.second->raw_bytes + e.second->tiled_bytes;
    rocknpu_decode_cache_stats s{};
    s.hits = ctx->hits;
    s.misses = ctx->misses;
    s.entries = ctx->m1.size() + ctx->m1_groups.size() + ctx->raw.size();
    s.resident_bytes = resident;
    s.hit_ns = ctx->hit_ns;
    s.miss_ns = ctx->miss_ns;
    s.tuned_shapes = 0;          // no per-shape worker tuning on the GPU
    s.worker1_calls = ctx->m1_calls;  // one GPU is one worker
    s.worker2_calls = 0;
    s.worker3_calls = 0;
    s.ksplit_calls = 0;
    *out = s;
    return kOk;
}

void rocknpu_context_destroy(rocknpu_context* ctx) {
    if (!ctx) return;
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    rk::route_print_summary(ctx);
    if (ctx->profile_mtile && ctx->mtile_profile.calls)
        std::fprintf(stderr, "ROCKNPU MTILE PROFILE calls=%zu hits=%zu misses=%zu prepare_ms=%.3f execute_ms=%.3f\n",
                     ctx->mtile_profile.calls, ctx->mtile_profile.cache_hits, ctx->mtile_profile.cache_misses,
                     ctx->mtile_profile.prepare_ns / 1e6, ctx->mtile_profile.execute_ns / 1e6);
    if (ctx->profile_m1 && ctx->m1_profile.calls)
        std::fprintf(stderr, "ROCKNPU M1 PROFILE calls=%zu hits=%zu misses=%zu prepare_ms=%.3f execute_ms=%.3f\n",
                     ctx->m1_profile.calls, ctx->m1_profile.cache_hits, ctx->m1_profile.cache_misses,
                     ctx->m1_profile.prepare_ns / 1e6, ctx->m1_profile.execute_ns / 1e6);
    hipStream_t s = ctx->stream;
    delete ctx;  // frees every cached device buffer
    if (s) (void)hipStreamDestroy(s);
}

int rocknpu_context_set_overlap(rocknpu_context* ctx, rocknpu_overlap_fn callback, void* user_data) {
    if (!ctx) return kInvalid;
    ctx->overlap = callback;
    ctx->overlap_user = callback ? user_data : nullptr;
    return kOk;
}

int rocknpu_matmul_q_concat_f32_f32_mtile(rocknpu_context* ctx, size_t count, const uint8_t* const* weights,
                                          const size_t* bytes, const uint32_t* kinds, const size_t* ns,
                                          const float* act, float* const* outputs, size_t m, size_t k) {
    if (!ctx || count < 1 || count > 4 || !weights || !bytes || !kinds || !ns || !act || !outputs || m == 0 ||
        k == 0)
        return kInvalid;
    std::vector<Source> srcs;
    std::vector<float*> outs;
    for (size_t i = 0; i < count; ++i) {
        if (!weights[i] || !outputs[i] || ns[i] == 0 || !kquant_kind(kinds[i])) return kInvalid;
        if (!kquant_shape_ok(kinds[i], bytes[i], k, ns[i])) return kInvalid;
        srcs.push_back(kquant_source(weights[i], bytes[i], kinds[i], k, ns[i]));
        outs.push_back(outputs[i]);
    }
    return exec_group(ctx, srcs, act, m, outs, true);  // two-part encoding: lib.rs:2484
}

int rocknpu_mtile_release(rocknpu_context* ctx, size_t count, const uint8_t* const* weights) {
    if (!ctx || !weights || count < 1 || count > 4) return kInvalid;
    std::vector<uintptr_t> addrs(count);
    for (size_t i = 0; i < count; ++i) addrs[i] = reinterpret_cast<uintptr_t>(weights[i]);
    auto involved = [&](const WeightKey& key) {
        for (uintptr_t a : addrs)
            if (a == key.address) return true;
        return false;
    };
    for (auto it = ctx->mtile.begin(); it != ctx->mtile.end();)
        it = involved(it->first) ? ctx->mtile.erase(it) : std::next(it);
    for (auto it = ctx->mtile_groups.begin(); it != ctx->mtile_groups.end();) {
        const auto& keys = it->first;
        bool exact = keys.size() == addrs.size();
        for (size_t i = 0; exact && i < keys.size(); ++i) exact = keys[i].address == addrs[i];
        bool any = false;
        for (const auto& key : keys) any = any || involved(key);
        it = (!exact && any) ? ctx->mtile_groups.erase(it) : std::next(it);
    }
    return kOk;
}

int rocknpu_prewarm_quantized_m16(rocknpu_context* ctx, const uint8_t* w, size_t bytes, uint32_t kind, size_t k,
                                  size_t n) {
    if (!ctx || !w || k == 0 || n == 0 || !kquant_kind(kind) || k % kQK != 0) return kInvalid;
    if (!kquant_shape_ok(kind, bytes, k, n)) return kInvalid;
    const Source src = kquant_source(w, bytes, kind, k, n);
    if (find_w8(ctx->mtile, ctx->m1, src.key)) return kOk;
    W8Ptr wp;
    const int st = build_w8(ctx, {src}, k, &wp);
    if (st == kOk) ctx->mtile.emplace(src.key, wp);
    return st;
}

int rocknpu_matmul_f16_f32_f32(rocknpu_context* ctx, const uint16_t* w, const float* act, float* out, size_t m,
                               size_t k, size_t n) {
    if (!ctx || !w || !act || !out || m == 0 || k == 0 || n == 0) return kInvalid;
    size_t a_elems, w_elems, o_elems;
    if (!mul_ok(m, k, &a_elems) || !mul_ok(n, k, &w_elems) || !mul_ok(m, n, &o_elems)) return kInvalid;
    if (!ctx->d_act.ensure(a_elems * 4) || !ctx->d_raw.ensure(w_elems * 2) || !ctx->d_out.ensure(o_elems * 4))
        return kExec;
    if (!hip_ok(hipMemcpyAsync(ctx->d_act.p, act, a_elems * 4, hipMemcpyHostToDevice, ctx->stream), ctx, "act") ||
        !hip_ok(hipMemcpyAsync(ctx->d_raw.p, w, w_elems * 2, hipMemcpyHostToDevice, ctx->stream), ctx, "w"))
        return kExec;
    const unsigned threads = 256;
    const size_t blocks = (o_elems + threads - 1) / threads;
    if (blocks > 0x7fffffff) return kInvalid;
    f16_matmul_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(threads), 0, ctx->stream>>>(
        ctx->d_raw.as<_Float16>(), ctx->d_act.as<float>(), ctx->d_out.as<float>(), static_cast<int64_t>(m),
        static_cast<int64_t>(k), static_cast<int64_t>(n));
    if (!hip_ok(hipGetLastError(), ctx, "f16") ||
        !hip_ok(hipMemcpyAsync(out, ctx->d_out.p, o_elems * 4, hipMemcpyDeviceToHost, ctx->stream), ctx, "out") ||
        !hip_ok(hipStreamSynchronize(ctx->stream), ctx, "f16"))
        return kExec;
    return kOk;
}

int rocknpu_matmul_w8a8_f32_f32_m1(rocknpu_context* ctx, const int8_t* w, const float* scales, const float* act,
                                   float* out, size_t k, size_t n) {
    if (!ctx || !w || !scales || !act || !out || k == 0 || n == 0) return kInvalid;
    size_t tmp;
    if (!mul_ok(k, n, &tmp) || !scales_ok(scales, n)) return kInvalid;
    return exec_single(ctx, w8_source(w, scales, k, n), act, out, 1);
}

int rocknpu_matmul_w8a8_f32_f32_m16(rocknpu_context* ctx, const int8_t* w, const float* scales, const float* act,
                                    float* out, size_t k, size_t n) {
    if (!ctx || !w || !scales || !act || !out || k == 0 || n == 0) return kInvalid;
    size_t tmp;
    if (!mul_ok(k, n, &tmp) || !mul_ok(16, k, &tmp) || !mul_ok(16, n, &tmp) || !scales_ok(scales, n))
        return kInvalid;
    return exec_single(ctx, w8_source(w, scales, k, n), act, out, 16);
}

int rocknpu_matmul_w8a8_f32_f32_m1_nsplit(rocknpu_context* ctx, const int8_t* w, const float* scales,
                                          const float* act, float* out, size_t k, size_t n, size_t chunk_n) {
    if (!ctx || !w || !scales || !act || !out || k == 0 || n == 0 || chunk_n == 0 || chunk_n % 32 != 0 ||
        n % 32 != 0)
        return kInvalid;
    for (size_t off = 0; off < n; off += chunk_n) {
        const size_t cur = chunk_n < n - off ? chunk_n : n - off;
        const int st = rocknpu_matmul_w8a8_f32_f32_m1(ctx, w + off * k, scales + off, act, out + off, k, cur);
        if (st != kOk) return st;
    }
    return kOk;
}

int rocknpu_matmul_w8a8_pair_f32_f32_m1(rocknpu_context* ctx, const int8_t* w1, const float* s1, size_t n1,
                                        const int8_t* w2, const float* s2, size_t n2, const float* act, float* o1,
                                        float* o2, size_t k) {
    if (!ctx || !w1 || !s1 || !w2 || !s2 || !act || !o1 || !o2 || k == 0 || n1 == 0 || n2 == 0) return kInvalid;
    size_t tmp;
    if (!mul_ok(k, n1, &tmp) || !mul_ok(k, n2, &tmp) || !scales_ok(s1, n1) || !scales_ok(s2, n2)) return kInvalid;
    return exec_group(ctx, {w8_source(w1, s1, k, n1), w8_source(w2, s2, k, n2)}, act, 1, {o1, o2});
}

int rocknpu_matmul_w8a8_triple_f32_f32_m1(rocknpu_context* ctx, const int8_t* w1, const float* s1, size_t n1,
                                          const int8_t* w2, const float* s2, size_t n2, const int8_t* w3,
                                          const float* s3, size_t n3, const float* act, float* o1, float* o2,
                                          float* o3, size_t k) {
    if (!ctx || !w1 || !s1 || !w2 || !s2 || !w3 || !s3 || !act || !o1 || !o2 || !o3 || k == 0 || n1 == 0 ||
        n2 == 0 || n3 == 0)
        return kInvalid;
    size_t tmp;
    if (!mul_ok(k, n1, &tmp) || !mul_ok(k, n2, &tmp) || !mul_ok(k, n3, &tmp) || !scales_ok(s1, n1) ||
        !scales_ok(s2, n2) || !scales_ok(s3, n3))
        return kInvalid;
    return exec_group(ctx, {w8_source(w1, s1, k, n1), w8_source(w2, s2, k, n2), w8_source(w3, s3, k, n3)}, act, 1,
                      {o1, o2, o3});
}

int rocknpu_matmul_w8a8_swiglu_down_f32(rocknpu_context* ctx, const int8_t* gw, const float* gs, const int8_t* uw,
                                        const float* us, const int8_t* dw, const float* ds, const float* act,
                                        float* out, size_t projection_k, size_t ffn_n, size_t output_n) {
    if (!ctx || !gw || !gs || !uw || !us || !dw || !ds || !act || !out || projection_k == 0 || ffn_n == 0 ||
        output_n == 0)
        return kInvalid;
    size_t tmp;
    if (!mul_ok(projection_k, ffn_n, &tmp) || !mul_ok(ffn_n, output_n, &tmp) || !scales_ok(gs, ffn_n) ||
        !scales_ok(us, ffn_n) || !scales_ok(ds, output_n) || ffn_n > (size_t{1} << 40))
        return kInvalid;
    if (!w8a8_k_ok(projection_k) || !w8a8_k_ok(ffn_n)) return kInvalid;
    // The reference runs the gate/up pair and the down projection as two M = 1
    // calls with the SwiGLU on the host between them (lib.rs:4308-4393); here
    // the intermediate stays on the device: one upload, one download.
    const uint64_t t0 = now_ns();
    W8Ptr wgu, wd;
    bool hit_gu = false, hit_d = false;
    int st = group_w8(ctx, {w8_source(gw, gs, projection_k, ffn_n), w8_source(uw, us, projection_k, ffn_n)}, true,
                      &wgu, &hit_gu);
    if (st != kOk) return st;
    st = single_w8(ctx, w8_source(dw, ds, ffn_n, output_n), true, &wd, &hit_d);
    if (st != kOk) return st;
    const size_t gu_n = 2 * ffn_n, a8_bytes = std::max(wgu->k_pad, wd->k_pad);
    if (!ctx->d_act.ensure((projection_k + ffn_n) * sizeof(float)) || !ctx->d_a8.ensure(2 * a8_bytes) ||
        !ctx->d_as.ensure(2 * sizeof(float)) || !ctx->d_out.ensure((gu_n + output_n) * sizeof(float)) ||
        !ctx->h_as.ensure(2 * sizeof(float)) || !ctx->h_out.ensure(output_n * sizeof(float)))
        return kExec;
    float* d_x = ctx->d_act.as<float>();
    float* d_h = d_x + projection_k;
    float* d_gu = ctx->d_out.as<float>();
    float* d_y = d_gu + gu_n;
    int8_t* a8 = ctx->d_a8.as<int8_t>();
    float* as = ctx->d_as.as<float>();
    if (!hip_ok(hipMemcpyAsync(d_x, act, projection_k * sizeof(float), hipMemcpyHostToDevice, ctx->stream), ctx,
                "act"))
        return kExec;
    st = rocknpu_hip_quantize_a8(d_x, 1, projection_k, projection_k, wgu->k_pad, a8, as, ctx->stream);
    if (st == kOk)
        st = rocknpu_hip_gemm_w8a8(a8, as, wgu->w8, wgu->scales, 1, gu_n, wgu->k_pad, d_gu, gu_n, nullptr,
                                   ctx->stream);
    if (st != kOk) return st;
    swiglu_kernel<<<static_cast<unsigned>((ffn_n + 255) / 256), 256, 0, ctx->stream>>>(d_gu, d_h,
                                                                                      static_cast<int64_t>(ffn_n));
    if (!hip_ok(hipGetLastError(), ctx, "swiglu")) return kExec;
    st = rocknpu_hip_quantize_a8(d_h, 1, ffn_n, ffn_n, wd->k_pad, a8 + a8_bytes, as + 1, ctx->stream);
    if (st == kOk)
        st = rocknpu_hip_gemm_w8a8(a8 + a8_bytes, as + 1, wd->w8, wd->scales, 1, output_n, wd->k_pad, d_y,
                                   output_n, nullptr, ctx->stream);
    if (st != kOk) return st;
    if (!hip_ok(hipMemcpyAsync(ctx->h_out.p, d_y, output_n * sizeof(float), hipMemcpyDeviceToHost, ctx->stream),
                ctx, "download") ||
        !hip_ok(hipMemcpyAsync(ctx->h_as.p, as, 2 * sizeof(float), hipMemcpyDeviceToHost, ctx->stream), ctx,
                "download"))
        return kExec;
    run_overlap(ctx);
    if (!hip_ok(hipStreamSynchronize(ctx->stream), ctx, "execute")) return kExec;
    // two M = 1 calls, as the reference's pair + single
    record_decode(ctx, hit_gu, t0);
    record_decode(ctx, hit_d, t0);
    const float* has = ctx->h_as.as<float>();
    if (!std::isfinite(has[0]) || !std::isfinite(has[1])) return kInvalid;  // non-finite activation row
    std::memcpy(out, ctx->h_out.p, output_n * sizeof(float));
    return kOk;
}

int rocknpu_matmul_q_pair_f32_f32_mtile(rocknpu_context* ctx, const uint8_t* w1, size_t b1, uint32_t k1, size_t n1,
                                        const uint8_t* w2, size_t b2, uint32_t k2, size_t n2, const float* act,
                                        float* o1, float* o2, size_t m, size_t k) {
    if (!ctx || !w1 || !w2 || !act || !o1 || !o2 || m == 0 || k == 0 || n1 == 0 || n2 == 0) return kInvalid;
    if (!kquant_kind(k1) || !kquant_kind(k2)) return kInvalid;
    if (!kquant_shape_ok(k1, b1, k, n1) || !kquant_shape_ok(k2, b2, k, n2)) return kInvalid;
    return exec_group(ctx, {kquant_source(w1, b1, k1, k, n1), kquant_source(w2, b2, k2, k, n2)}, act, m, {o1, o2});
}

int rocknpu_matmul_q_pair_f32_f32_m1(rocknpu_context* ctx, const uint8_t* w1, size_t b1, uint32_t k1, size_t n1,
                                     const uint8_t* w2, size_t b2, uint32_t k2, size_t n2, const float* act,
                                     float* o1, float* o2, size_t k) {
    if (!ctx || !w1 || !w2 || !act || !o1 || !o2 || k == 0 || n1 == 0 || n2 == 0) return kInvalid;
    if (!kquant_kind(k1) || !kquant_kind(k2)) return kInvalid;
    if (!kquant_shape_ok(k1, b1, k, n1) || !kquant_shape_ok(k2, b2, k, n2)) return kInvalid;
    return exec_group(ctx, {kquant_source(w1, b1, k1, k, n1), kquant_source(w2, b2, k2, k, n2)}, act, 1, {o1, o2});
}

int rocknpu_matmul_q_triple_f32_f32_m1(rocknpu_context* ctx, const uint8_t* w1, size_t b1, uint32_t k1, size_t n1,
                                       const uint8_t* w2, size_t b2, uint32_t k2, size_t n2, const uint8_t* w3,
                                       size_t b3, uint32_t k3, size_t n3, const float* act, float* o1, float* o2,
                                       float* o3, size_t k) {
    if (!ctx || !w1 || !w2 || !w3 || !act || !o1 || !o2 || !o3 || k == 0 || n1 == 0 || n2 == 0 || n3 == 0)
        return kInvalid;
    if (!kquant_kind(k1) || !kquant_kind(k2) || !kquant_kind(k3)) return kInvalid;
    if (!kquant_shape_ok(k1, b1, k, n1) || !kquant_shape_ok(k2, b2, k, n2) || !kquant_shape_ok(k3, b3, k, n3))
        return kInvalid;
    return exec_group(ctx,
                      {kquant_source(w1, b1, k1, k, n1), kquant_source(w2, b2, k2, k, n2),
                       kquant_source(w3, b3, k3, k, n3)},
                      act, 1, {o1, o2, o3});
}

int rocknpu_matmul_q4_k_f32_f32(rocknpu_context* ctx, const uint8_t* w, size_t bytes, const float* act, float* out,
                                size_t m, size_t k, size_t n) {
    return matmul_kquant(ctx, 4, w, bytes, act, out, m, k, n);
}

int rocknpu_matmul_q5_k_f32_f32(rocknpu_context* ctx, const uint8_t* w, size_t bytes, const float* act, float* out,
                                size_t m, size_t k, size_t n) {
    return matmul_kquant(ctx, 5, w, bytes, act, out, m, k, n);
}

int rocknpu_matmul_q6_k_f32_f32(rocknpu_context* ctx, const uint8_t* w, size_t bytes, const float* act, float* out,
                                size_t m, size_t k, size_t n) {
    return matmul_kquant(ctx, 6, w, bytes, act, out, m, k, n);
}

// llama.cpp CPU decode semantics on the GPU: Q8_K quantisation of the f32
// activations, then the Q4_K/Q6_K x Q8_K GEMV over device-resident raw blocks.
int rocknpu_matmul_q_q8k_f32_f32(rocknpu_context* ctx, uint32_t kind, const uint8_t* w, size_t bytes,
                                 const float* act, float* out, size_t m, size_t k, size_t n) {
    if (!ctx || !w || !act || !out || m == 0 || k == 0 || n == 0 || !kquant_kind(kind)) return kInvalid;
    if (!kquant_shape_ok(kind, bytes, k, n)) return kInvalid;
    size_t a_elems, o_elems;
    if (!mul_ok(m, k, &a_elems) || !mul_ok(m, n, &o_elems)) return kInvalid;
    for (size_t i = 0; i < a_elems; ++i)
        if (!std::isfinite(act[i])) return kInvalid;
    const uint64_t t0 = now_ns();
    bool hit = true;
    const bool tiled = decode_tiled(kind, m, k);
    const std::shared_ptr<DecodeWeight> dw = raw_weights(ctx, w, bytes, k, n, kind, tiled, &hit);
    if (!dw) return kExec;
    const size_t q8_bytes = m * (k / kQK) * 292;
    if (!ctx->d_act.ensure(a_elems * 4) || !ctx->d_q8k.ensure(q8_bytes) || !ctx->d_out.ensure(o_elems * 4))
        return kExec;
    if (!hip_ok(hipMemcpyAsync(ctx->d_act.p, act, a_elems * 4, hipMemcpyHostToDevice, ctx->stream), ctx, "act"))
        return kExec;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    if (tiled && !gemv_split_ws(ctx, kind, m, k, n, &ws, &ws_bytes)) return kExec;
    int st = rocknpu_hip_quantize_q8_k(ctx->d_act.as<float>(), m, k, k, ctx->d_q8k.as<uint8_t>(), ctx->stream);
    if (st != kOk) return st;
    st = tiled ? rocknpu_hip_gemv_q8_k_tiled(kind, dw->tiled.as<uint8_t>(), dw->tiled_bytes, k, n,
                                             ctx->d_q8k.as<uint8_t>(), m, ctx->d_out.as<float>(), n, ws, ws_bytes,
                                             ctx->stream)
               : rocknpu_hip_gemv_q8_k(kind, dw->raw.as<uint8_t>(), bytes, k, n, ctx->d_q8k.as<uint8_t>(), m,
                                       ctx->d_out.as<float>(), n, nullptr, nullptr, ctx->stream);
    if (st != kOk) return st;
    if (ws && !gemv_split_queue_check(ctx)) return kExec;
    if (!hip_ok(hipMemcpyAsync(out, ctx->d_out.p, o_elems * 4, hipMemcpyDeviceToHost, ctx->stream), ctx, "out") ||
        !hip_ok(hipStreamSynchronize(ctx->stream), ctx, "gemv"))
        return kExec;
    if (ws && gemv_split_failed(ctx)) return kExec;
    record_decode(ctx, hit, t0);
    return kOk;
}

int rocknpu_matmul_q_q8k_group_f32_f32(rocknpu_context* ctx, size_t count, const uint8_t* const* weights,
                                       const size_t* bytes, const uint32_t* kinds, const size_t* ns,
                                       const float* act, float* const* outputs, size_t m, size_t k) {
    if (!ctx || !weights || !bytes || !kinds || !ns || !act || !outputs || count == 0 || count > 4 || m == 0 ||
        k == 0)
        return kInvalid;
    size_t a_elems, total_n = 0;
    if (!mul_ok(m, k, &a_elems)) return kInvalid;
    for (size_t i = 0; i < count; ++i) {
        if (!weights[i] || !outputs[i] || ns[i] == 0 || !kquant_kind(kinds[i]) ||
            !kquant_shape_ok(kinds[i], bytes[i], k, ns[i]))
            return kInvalid;
        total_n += ns[i];
    }
    size_t o_elems;
    if (!mul_ok(m, total_n, &o_elems)) return kInvalid;
    for (size_t i = 0; i < a_elems; ++i)
        if (!std::isfinite(act[i])) return kInvalid;
    const uint64_t t0 = now_ns();
    bool hit = true;
    std::shared_ptr<DecodeWeight> dw[4];
    for (size_t i = 0; i < count; ++i)
        if (!(dw[i] = raw_weights(ctx, weights[i], bytes[i], k, ns[i], kinds[i], decode_tiled(kinds[i], m, k), &hit)))
            return kExec;
    if (!ctx->d_act.ensure(a_elems * 4) || !ctx->d_out.ensure(o_elems * 4)) return kExec;
    if (!hip_ok(hipMemcpyAsync(ctx->d_act.p, act, a_elems * 4, hipMemcpyHostToDevice, ctx->stream), ctx, "act"))
        return kExec;
    // member i's rows at offset m * (n of the members before it); one fused
    // launch per kind over that kind's members, in member order
    size_t off[4];
    for (size_t i = 0, o = 0; i < count; o += m * ns[i], ++i) off[i] = o;
    bool split = false;
    for (uint32_t kind : {4u, 6u}) {
        const bool tiled = decode_tiled(kind, m, k);
        const uint8_t* w[4];
        size_t wb[4], wn[4], ldo[4];
        float* out[4];
        size_t c = 0;
        for (size_t i = 0; i < count; ++i) {
            if (kinds[i] != kind) continue;
            w[c] = tiled ? dw[i]->tiled.as<uint8_t>() : dw[i]->raw.as<uint8_t>();
            wb[c] = tiled ? dw[i]->tiled_bytes : bytes[i];
            wn[c] = ns[i];
            ldo[c] = ns[i];
            out[c] = ctx->d_out.as<float>() + off[i];
            ++c;
        }
        if (c == 0) continue;
        void* ws = nullptr;
        size_t ws_bytes = 0, rows = 0;
        for (size_t i = 0; i < c; ++i) rows += wn[i];
        if (tiled && !gemv_split_ws(ctx, kind, m, k, rows, &ws, &ws_bytes)) return kExec;
        split |= ws != nullptr;
        const int st = tiled ? rocknpu_hip_gemv_q_f32_tiled(kind, c, w, wb, wn, k, ctx->d_act.as<float>(), k, m, out,
                                                            ldo, ws, ws_bytes, ctx->stream)
                             : rocknpu_hip_gemv_q_f32(kind, c, w, wb, wn, k, ctx->d_act.as<float>(), k, m, out, ldo,
                                                      ctx->stream);
        if (st != kOk) return st;
    }
    if (split && !gemv_split_queue_check(ctx)) return kExec;
    for (size_t i = 0; i < count; ++i)
        if (!hip_ok(hipMemcpyAsync(outputs[i], ctx->d_out.as<float>() + off[i], m * ns[i] * 4, hipMemcpyDeviceToHost,
                                   ctx->stream),
                    ctx, "out"))
            return kExec;
    if (!hip_ok(hipStreamSynchronize(ctx->stream), ctx, "gemv")) return kExec;
    if (split && gemv_split_failed(ctx)) return kExec;
    // a fused launch whose wait for its quantising waves gave up wrote NaN
    if (rocknpu_hip_gemv_take_stall()) {
        if (ctx->trace) std::fprintf(stderr, "ROCKNPU DECODE ERROR gemv: activation quantisation wait gave up\n");
        return kExec;
    }
    record_decode(ctx, hit, t0);
    return kOk;
}

}  // extern "C"
