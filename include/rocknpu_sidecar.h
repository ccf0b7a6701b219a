/*
 * rocknpu_sidecar.h — the W8 sidecar: repacked int8 weights cached on disk.
 *
 * The reference plugin can start its M=1 W8A8 path from precomputed int8
 * weights instead of repacking every GGUF tensor at load
 * (adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:115-259, written by
 * scripts/make_tinyllama_w8_sidecar_gguf.py:23-70,101-158). For a tensor
 * named `name` in directory `dir` the sidecar is three files:
 *   <name>.w8             n*k int8, row-major [n][k] (one row per output)
 *   <name>.scale.f32      n little-endian f32 scales
 *   <name>.source.fnv1a64 16 lowercase hex digits and a newline: the
 *                         fingerprint of the GGUF source bytes it came from
 * and is used only when the fingerprint matches the tensor being loaded and
 * every scale is finite and > 0. These functions read and write that format
 * byte for byte, so a directory made by either side serves the other.
 *
 * Host pointers; 0 = ROCKNPU_STATUS_OK, -1 = invalid argument or a missing,
 * mismatched or invalid sidecar, -2 = device or file-system failure.
 */
#ifndef ROCKNPU_SIDECAR_H
#define ROCKNPU_SIDECAR_H

#include <stddef.h>
#include <stdint.h>

#include "rocknpu.h"

#ifdef __cplusplus
extern "C" {
#endif

/* FNV-1a 64 over the byte count (8 bytes, least significant first), then
 * over all bytes when bytes <= 12288, else over the first 4096, the 4096 at
 * (bytes - 4096) / 2 and the last 4096. Replaces
 * rocknpu_source_sample_fingerprint (ggml-rocknpu.cpp:123-146) and
 * source_sample_fnv1a64 (make_tinyllama_w8_sidecar_gguf.py:23-45). */
uint64_t rocknpu_w8_source_fingerprint(const uint8_t * data, size_t bytes);

/* Load <dir>/<name>.{w8,scale.f32} into w8 [n*k] and scales [n] when
 * <name>.source.fnv1a64 holds the fingerprint of source[0, source_bytes),
 * both files have exactly the expected sizes and every scale is finite and
 * > 0. The file half of rocknpu_w8_sidecar_get (ggml-rocknpu.cpp:209-243). */
int rocknpu_w8_sidecar_read(const char * dir, const char * name, const uint8_t * source, size_t source_bytes,
                            size_t k, size_t n, int8_t * w8, float * scales);

/* Write the three files for w8 [n*k] and scales [n] made from the source
 * bytes (the generator side, make_tinyllama_w8_sidecar_gguf.py:46-70,110-112). */
int rocknpu_w8_sidecar_write(const char * dir, const char * name, const uint8_t * source, size_t source_bytes,
                             size_t k, size_t n, const int8_t * w8, const float * scales);

/* The sidecar when it matches, else the conversion: Q4_K / Q5_K / Q6_K blocks
 * (kind 4/5/6, [n][k/256] blocks) repacked on the context's GPU with the
 * plugin's semantics (dequantise, scale = max|row|/127 or 1, round half away
 * from zero; rocknpu_w8_convert, ggml-rocknpu.cpp:162-207). With write_back
 * nonzero and dir non-NULL a conversion is also written as a sidecar.
 * *from_sidecar (if non-NULL) tells which path served. */
int rocknpu_w8_sidecar_get(rocknpu_context * context, const char * dir, const char * name, uint32_t kind,
                           const uint8_t * source, size_t source_bytes, size_t k, size_t n, int8_t * w8,
                           float * scales, int write_back, int * from_sidecar);

#ifdef __cplusplus
}
#endif

#endif
