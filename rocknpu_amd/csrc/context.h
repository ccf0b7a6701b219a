// The C ABI's context (struct RockNpuContext, opaque in include/rocknpu.h) and
// the device buffers it owns. Shared by capi.hip (entry points, caches) and
// route.hip (the routing state a plugin's backend context keeps in the
// reference: the cross-partition Q/K/V stash and the dispatch counters).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "rocknpu.h"
#include "rocknpu_route.h"

namespace rk {

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// (address, bytes, k, n, kind): crates/rocknpu-capi/src/lib.rs:33-39. Kind 8
// marks caller-supplied int8 weights (the reference files those under Q4K
// with bytes = k*n).
struct WeightKey {
    uintptr_t address;
    size_t bytes, k, n;
    uint32_t kind;
    bool operator==(const WeightKey& o) const {
        return address == o.address && bytes == o.bytes && k == o.k && n == o.n && kind == o.kind;
    }
    bool operator<(const WeightKey& o) const {
        if (address != o.address) return address < o.address;
        if (bytes != o.bytes) return bytes < o.bytes;
        if (k != o.k) return k < o.k;
        if (n != o.n) return n < o.n;
        return kind < o.kind;
    }
};
struct KeyHash {
    size_t operator()(const WeightKey& w) const {
        size_t h = w.address * 0x9E3779B97F4A7C15ull;
        h ^= w.bytes + 0x632BE59BD9B4E019ull + (h << 6) + (h >> 2);
        h ^= w.k + (w.n << 20) + (static_cast<size_t>(w.kind) << 56) + (h << 6) + (h >> 2);
        return h;
    }
};

// Device-resident W8 matrix [n, k_pad] + scales[n]; freed with the entry.
struct DeviceW8 {
    int8_t* w8 = nullptr;
    float* scales = nullptr;
    size_t n = 0, k = 0, k_pad = 0;
    DeviceW8() = default;
    DeviceW8(const DeviceW8&) = delete;
    DeviceW8& operator=(const DeviceW8&) = delete;
    ~DeviceW8() {
        if (w8) (void)hipFree(w8);
        if (scales) (void)hipFree(scales);
    }
    size_t resident_bytes() const { return n * k_pad + n * sizeof(float); }
};
using W8Ptr = std::shared_ptr<DeviceW8>;

struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    bool ensure(size_t bytes) {
        if (bytes <= cap) return true;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        const size_t want = round_up(bytes, size_t(1) << 20);
        if (hipMalloc(&p, want) != hipSuccess) return false;
        cap = want;
        return true;
    }
    template <class T>
    T* as() const { return static_cast<T*>(p); }
};

// A weight resident for the Q8_K decode GEMV: its raw K-quant rows (read by
// the one-row kernels) and, built on the first call of two or more rows, the
// tile-interleaved copy the matrix-core kernels read with whole-line loads.
struct DecodeWeight {
    DevBuf raw, tiled;
    size_t raw_bytes = 0, tiled_bytes = 0;
};

struct PinnedBuf {
    void* p = nullptr;
    size_t cap = 0;
    PinnedBuf() = default;
    PinnedBuf(const PinnedBuf&) = delete;
    PinnedBuf& operator=(const PinnedBuf&) = delete;
    ~PinnedBuf() {
        if (p) (void)hipHostFree(p);
    }
    bool ensure(size_t bytes) {
        if (bytes <= cap) return true;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        cap = 0;
        const size_t want = round_up(bytes, size_t(1) << 20);
        if (hipHostMalloc(&p, want, hipHostMallocDefault) != hipSuccess) return false;
        cap = want;
        return true;
    }
    template <class T>
    T* as() const { return static_cast<T*>(p); }
};

struct Profile {
    size_t calls = 0, cache_hits = 0, cache_misses = 0;
    uint64_t prepare_ns = 0, execute_ns = 0;
};

// One attention layer's Q/K/V state for the cross-partition stash
// (adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:871-928, the plugin's
// rocknpu_qkv_layer_state): the K and V weights seen for the layer, and the K/V
// outputs a Q-led triple computed ahead of their own nodes.
struct QkvWeight {
    const void* data = nullptr;
    size_t bytes = 0, n = 0, k = 0;
    int32_t type = 0;
};
struct QkvLayer {
    QkvWeight wk, wv;
    std::vector<float> k_out, v_out;
    const float* activation = nullptr;  // input the pending outputs were computed from
    size_t rows = 0;                    // and its M
    bool k_pending = false, v_pending = false, released = false;
};
// Layers the stash tracks (the plugin's ROCKNPU_QKV_MAX_LAYERS bound).
constexpr size_t kQkvMaxLayers = 256;

struct RouteState {
    std::unordered_map<size_t, QkvLayer> qkv;
    rocknpu_route_stats stats{};
    // ROCKNPU_SPLIT_PROFILE: per rocknpu_route_run call, and per shape of a
    // projection run on its own ({calls, ns})
    std::vector<uint64_t> samples_ns;
    std::map<std::string, std::pair<size_t, uint64_t>> shapes;
};

}  // namespace rk

struct RockNpuContext {
    int device = 0;
    hipStream_t stream = nullptr;
    // prompt (M > 1) caches, dropped by rocknpu_mtile_release
    std::unordered_map<rk::WeightKey, rk::W8Ptr, rk::KeyHash> mtile;
    std::map<std::vector<rk::WeightKey>, rk::W8Ptr> mtile_groups;
    // decode (M = 1) caches, kept across releases
    std::unordered_map<rk::WeightKey, rk::W8Ptr, rk::KeyHash> m1;
    std::map<std::vector<rk::WeightKey>, rk::W8Ptr> m1_groups;
    // K-quant weights resident for the Q8_K decode GEMV (raw and tiled)
    std::unordered_map<rk::WeightKey, std::shared_ptr<rk::DecodeWeight>, rk::KeyHash> raw;
    rk::DevBuf d_raw, d_act, d_a8, d_as, d_out, d_q8k;
    rk::DevBuf d_split;  // the W8A8 GEMM's K-split workspace (counters cleared per call)
    rk::DevBuf d_gemv_split;  // the tiled decode GEMV's K-split slots and error word (zero between calls)
    rk::PinnedBuf h_out, h_as, h_err;  // h_err: the K-split workspace's error word
    size_t hits = 0, misses = 0, m1_calls = 0;
    uint64_t hit_ns = 0, miss_ns = 0;
    rk::Profile mtile_profile, m1_profile;
    bool profile_mtile = false, profile_m1 = false, trace = false;
    int hilo = 0;  // ROCKNPU_PREFILL_HILO: 0 off, 1 wide-K projections only, 2 every prompt projection
    rocknpu_overlap_fn overlap = nullptr;
    void* overlap_user = nullptr;
    rk::RouteState route;  // routing over this context (route.hip)
};
