/*
 * CPU oracle for the ggml MUL_MAT offload path — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference algorithm, used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.
 * No product code links, loads or calls it.
 *
 * Reference semantics followed (paths relative to the reference repository):
 *   W8A8 prefill route   crates/rocknpu-capi/src/lib.rs
 *       quantize_symmetric_into        :614-654
 *       rescale_i32_row                :692-709  (f32(acc) * a_scale * w_scale)
 *       prepare_q4_k_w8a8              :711-757
 *       prepare_q5_k_w8a8              :759-806
 *       prepare_q6_k_w8a8              :974-994
 *       execute_cached_w8a8_mtile_pool_padded :1731-1989 (quant, i32 GEMM, rescale)
 *   K-quant block formats and the decode dot products are the public ggml
 *   definitions (block_q4_K / block_q5_K / block_q6_K / block_q8_K,
 *   dequantize_row_q{4,5,6}_K, quantize_row_q8_K_ref,
 *   ggml_vec_dot_q{4,6}_K_q8_K generic) at the llama.cpp commit pinned by
 *   adapters/ggml-rocknpu/README.md:48; the dequantisers themselves are in the
 *   un-vendored crate llama-gguf 0.14.0 (Cargo.lock:276-279).
 *
 * Build: -O3 -ffp-contract=off, no fast-math (IEEE division, no FMA
 * contraction), so every float operation is the one written here.
 */
#ifndef ROCKNPU_ORACLE_H
#define ROCKNPU_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    OR_QK_K = 256,
    OR_Q4_K_BYTES = 144,
    OR_Q5_K_BYTES = 176,
    OR_Q6_K_BYTES = 210,
    OR_Q8_K_BYTES = 292,
    OR_OK = 0,
    OR_INVALID = -1,
};

/* Exact IEEE binary16 -> binary32 conversion. */
float or_fp16_to_f32(uint16_t bits);

/* Block sizes by kind: 4 -> 144, 5 -> 176, 6 -> 210, else 0. */
size_t or_block_bytes(uint32_t kind);

/* One 256-value super-block to f32 (ggml dequantize_row_*). */
void or_dequant_q4_k(const uint8_t *block, float *out256);
void or_dequant_q5_k(const uint8_t *block, float *out256);
void or_dequant_q6_k(const uint8_t *block, float *out256);
/* Whole rows: n rows of k values from n*(k/256) blocks of `kind`. */
int or_dequant_rows(uint32_t kind, const uint8_t *blocks, size_t k, size_t n, float *out);

/* Reference per-row symmetric int8 quantisation (lib.rs:614-654).
 * Returns 0 and writes *scale, or -1 if the row holds a non-finite value. */
int or_quantize_symmetric_row(const float *x, size_t k, int8_t *q, float *scale);

/* The aarch64 NEON form (lib.rs:475-541), the reference's default on its
 * RK3588 target: q = round(x * f32(1/scale)) in chunks of 8, the tail of
 * k % 8 values by division. Same scale. */
int or_quantize_symmetric_row_neon(const float *x, size_t k, int8_t *q, float *scale);

/* Weight repack (lib.rs:711-757, 759-806, 974-994): W8 [n,k] + scales[n]. */
int or_repack_w8(uint32_t kind, const uint8_t *blocks, size_t bytes, size_t k, size_t n,
                 int8_t *w8, float *scales);

/* Per-token A8 quantisation of a [m,k] f32 matrix into [m,k_pad] int8 rows
 * (zero-padded from k to k_pad, lib.rs:1776-1791). */
int or_quantize_a8(const float *a, size_t m, size_t k, size_t k_pad, int8_t *a8, float *scales);

/* Exact C[m,n] = sum_k A[m,k] * W[n,k] (i32). `threads` <= 1 runs serially. */
void or_gemm_i32(const int8_t *a8, const int8_t *w8, size_t m, size_t n, size_t k, int32_t *c,
                 int threads);

/* out[m,n] = (f32(c) * a_scale[m]) * w_scale[n] (lib.rs:706-708). */
void or_rescale(const int32_t *c, const float *a_scales, const float *w_scales, size_t m, size_t n,
                float *out);

/* The aarch64 NEON rescale (lib.rs:664-690): (f32(c) * w_scale[n]) * a_scale[m]
 * in chunks of 4 columns, the n % 4 tail in the scalar order. */
void or_rescale_neon(const int32_t *c, const float *a_scales, const float *w_scales, size_t m, size_t n,
                     float *out);

/* Whole W8A8 route of rocknpu_matmul_q{4,5,6}_k_f32_f32 for M > 1. */
int or_matmul_q_w8a8(uint32_t kind, const uint8_t *blocks, size_t bytes, const float *a, size_t m,
                     size_t k, size_t n, float *out, int threads);

/* Two-part activation encoding (lib.rs:2045-2071): stacked[0, m) = a and
 * stacked[m, 2m) = a - f32(q) * scale per row, q/scale from the symmetric
 * row quantisation. Returns -1 on a non-finite row. */
int or_hilo_stack(const float *a, size_t m, size_t k, float *stacked);

/* lib.rs:2073-2082: out[i] = stacked[i] + stacked[len + i]. */
void or_hilo_sum(float *out, const float *stacked, size_t len);

/* FNV-1a 64 over n bytes continuing from hash h (offset basis
 * 14695981039346656037, prime 1099511628211). */
uint64_t or_fnv1a64(uint64_t h, const uint8_t *data, size_t n);

/* W8 sidecar source fingerprint (adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:
 * 123-146; scripts/make_tinyllama_w8_sidecar_gguf.py:23-45): FNV-1a 64 over
 * the 8 bytes of the byte count (least significant first), then over all
 * bytes when bytes <= 3*4096, else over the first 4096, the 4096 at
 * (bytes - 4096) / 2 and the last 4096. */
uint64_t or_source_fingerprint(const uint8_t *data, size_t bytes);

/* ggml quantize_row_q8_K_ref: k/256 blocks of 292 bytes. */
void or_quantize_row_q8_k(const float *x, size_t k, uint8_t *q8k);

/* ggml generic vec_dot_q{4,6}_K_q8_K over k values (one weight row). */
float or_vec_dot_q4_k_q8_k(size_t k, const uint8_t *w_row, const uint8_t *q8k_row);
float or_vec_dot_q6_k_q8_k(size_t k, const uint8_t *w_row, const uint8_t *q8k_row);

/* Decode GEMV: out[mi*n + ni] = vec_dot(w row ni, q8k row mi). kind 4 or 6. */
int or_gemv_q8_k(uint32_t kind, const uint8_t *w, size_t k, size_t n, const uint8_t *q8k, size_t m,
                 float *out, int threads);

/* Integer sub-sums of the decode dot for each (row, block):
 *   isum[r*nb+b] = sum_j scale_j * sum_{l in sub-block j} q8 * q
 *   msum[r*nb+b] = sum_j min_j * (bsum pair of sub-block j)   (Q4_K; 0 for Q6_K)
 * and mag[ni] = sum_b (sum_l |d*aux32_b[l]| + |dmin*msum_b|), the magnitude the
 * generic ggml dot's f32 rounding error scales with (it rounds d*aux32[l] for
 * its 8 lanes l of positions p % 8 == l): results of any f32 evaluation order
 * agree with it to within a small multiple of 2^-24 * (8 + k/256) * mag. */
int or_gemv_block_sums(uint32_t kind, const uint8_t *w, size_t k, size_t n, const uint8_t *q8k_row,
                       int32_t *isum, int32_t *msum, double *mag);

#ifdef __cplusplus
}
#endif

#endif
