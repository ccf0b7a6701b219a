// The W8 sidecar (include/rocknpu_sidecar.h): repacked int8 weights cached
// on disk with a provenance fingerprint of their GGUF source. Host code; the
// conversion on a miss is the GPU repack of kernel (a).
#include "rocknpu_sidecar.h"

#include "common.h"

#include <cctype>
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace rk {
int context_repack_to_host(rocknpu_context* ctx, uint32_t kind, const uint8_t* source, size_t bytes, size_t k,
                           size_t n, int8_t* w8, float* scales);  // capi.hip
}

namespace {

constexpr uint64_t kFnvOffset = 14695981039346656037ull;
constexpr uint64_t kFnvPrime = 1099511628211ull;
constexpr size_t kSampleBytes = 4096;

std::string base_path(const char* dir, const char* name) { return std::string(dir) + "/" + name; }

// Whole-file read of exactly `bytes` bytes.
bool read_exact(const std::string& path, void* dst, size_t bytes) {
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    bool ok = std::fseek(f, 0, SEEK_END) == 0 && std::ftell(f) == static_cast<long>(bytes) &&
              std::fseek(f, 0, SEEK_SET) == 0 && std::fread(dst, 1, bytes, f) == bytes;
    std::fclose(f);
    return ok;
}

bool write_all(const std::string& path, const void* src, size_t bytes) {
    std::FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = std::fwrite(src, 1, bytes, f) == bytes;
    return std::fclose(f) == 0 && ok;
}

// The 16 hex digits of <name>.source.fnv1a64 (surrounding whitespace allowed).
bool read_fingerprint(const std::string& path, uint64_t* value) {
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    char buf[64] = {};
    const size_t got = std::fread(buf, 1, sizeof(buf) - 1, f);
    std::fclose(f);
    size_t b = 0;
    while (b < got && (buf[b] == ' ' || buf[b] == '\n' || buf[b] == '\r' || buf[b] == '\t')) ++b;
    size_t e = b;
    while (e < got && std::isxdigit(static_cast<unsigned char>(buf[e]))) ++e;
    for (size_t i = e; i < got; ++i)
        if (!(buf[i] == ' ' || buf[i] == '\n' || buf[i] == '\r' || buf[i] == '\t')) return false;
    if (e - b != 16) return false;
    uint64_t v = 0;
    for (size_t i = b; i < e; ++i) {
        const char c = buf[i];
        v = v << 4 | static_cast<uint64_t>(c <= '9' ? c - '0' : (c | 0x20) - 'a' + 10);
    }
    *value = v;
    return true;
}

bool scales_valid(const float* s, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(s[i]) || s[i] <= 0.0f) return false;
    return true;
}

}  // namespace

extern "C" {

uint64_t rocknpu_w8_source_fingerprint(const uint8_t* data, size_t bytes) {
    uint64_t h = kFnvOffset;
    const uint64_t count = bytes;
    for (unsigned shift = 0; shift < 64; shift += 8) {
        h ^= static_cast<uint8_t>(count >> shift);
        h *= kFnvPrime;
    }
    auto update = [&](size_t off, size_t len) {
        for (size_t i = 0; i < len; ++i) {
            h ^= data[off + i];
            h *= kFnvPrime;
        }
    };
    if (bytes <= kSampleBytes * 3) {
        if (bytes) update(0, bytes);
    } else {
        update(0, kSampleBytes);
        update((bytes - kSampleBytes) / 2, kSampleBytes);
        update(bytes - kSampleBytes, kSampleBytes);
    }
    return h;
}

int rocknpu_w8_sidecar_read(const char* dir, const char* name, const uint8_t* source, size_t source_bytes,
                            size_t k, size_t n, int8_t* w8, float* scales) {
    if (!dir || !dir[0] || !name || !name[0] || !source || source_bytes == 0 || k == 0 || n == 0 || !w8 || !scales)
        return rk::kStatusInvalid;
    size_t count;
    if (__builtin_mul_overflow(k, n, &count)) return rk::kStatusInvalid;
    const std::string base = base_path(dir, name);
    uint64_t expected = 0;
    if (!read_fingerprint(base + ".source.fnv1a64", &expected) ||
        expected != rocknpu_w8_source_fingerprint(source, source_bytes))
        return rk::kStatusInvalid;
    if (!read_exact(base + ".w8", w8, count) || !read_exact(base + ".scale.f32", scales, n * sizeof(float)) ||
        !scales_valid(scales, n))
        return rk::kStatusInvalid;
    return rk::kStatusOk;
}

int rocknpu_w8_sidecar_write(const char* dir, const char* name, const uint8_t* source, size_t source_bytes,
                             size_t k, size_t n, const int8_t* w8, const float* scales) {
    if (!dir || !dir[0] || !name || !name[0] || !source || source_bytes == 0 || k == 0 || n == 0 || !w8 || !scales)
        return rk::kStatusInvalid;
    size_t count;
    if (__builtin_mul_overflow(k, n, &count) || !scales_valid(scales, n)) return rk::kStatusInvalid;
    const std::string base = base_path(dir, name);
    char hex[32];
    std::snprintf(hex, sizeof(hex), "%016" PRIx64 "\n", rocknpu_w8_source_fingerprint(source, source_bytes));
    if (!write_all(base + ".w8", w8, count) || !write_all(base + ".scale.f32", scales, n * sizeof(float)) ||
        !write_all(base + ".source.fnv1a64", hex, 17))
        return rk::kStatusDevice;
    return rk::kStatusOk;
}

int rocknpu_w8_sidecar_get(rocknpu_context* ctx, const char* dir, const char* name, uint32_t kind,
                           const uint8_t* source, size_t source_bytes, size_t k, size_t n, int8_t* w8, float* scales,
                           int write_back, int* from_sidecar) {
    if (from_sidecar) *from_sidecar = 0;
    if (!name || !name[0] || !source || !w8 || !scales) return rk::kStatusInvalid;
    if (dir && dir[0] &&
        rocknpu_w8_sidecar_read(dir, name, source, source_bytes, k, n, w8, scales) == rk::kStatusOk) {
        if (from_sidecar) *from_sidecar = 1;
        return rk::kStatusOk;
    }
    const int st = rk::context_repack_to_host(ctx, kind, source, source_bytes, k, n, w8, scales);
    if (st != rk::kStatusOk) return st;
    if (write_back && dir && dir[0]) return rocknpu_w8_sidecar_write(dir, name, source, source_bytes, k, n, w8, scales);
    return rk::kStatusOk;
}

}  // extern "C"
