/*
 * rocknpu.h — C ABI of the MI355X (gfx950) MUL_MAT offload library.
 *
 * Drop-in for crates/rocknpu-capi/include/rocknpu.h of the reference: every
 * symbol, argument order, type and status code is the same, so the ggml
 * adapter (adapters/ggml-rocknpu/src/ggml-rocknpu.cpp) links against this
 * library unchanged. Each declaration cites the reference header line and the
 * Rust definition it replaces (crates/rocknpu-capi/src/lib.rs).
 *
 * Conventions (as in the reference):
 *   - every pointer is a HOST pointer owned by the caller for the duration of
 *     the synchronous call; weights are raw row-major [N][K/256] GGUF blocks
 *     (kind 4 = Q4_K 144 B, 5 = Q5_K 176 B, 6 = Q6_K 210 B per block) or
 *     row-major [N,K] int8 with f32 per-row scales; activations f32 [M,K];
 *     outputs f32 [M,N]; all row-major;
 *   - weights must stay immutable while the context lives: the device-resident
 *     W8 copy is cached under (address, bytes, k, n, kind);
 *   - a context is not re-entrant; use one per thread / ggml backend.
 * Numerics (W8A8): W8 rows and A8 rows are symmetric int8 with scale
 * max|row|/127, the product is an exact int32 GEMM on int8 MFMA, and the
 * output is (f32(acc) * a_scale) * w_scale.
 */
#ifndef ROCKNPU_H
#define ROCKNPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct RockNpuContext rocknpu_context;

/* Reference include/rocknpu.h:13-25 (RockNpuDecodeCacheStats, lib.rs:274-288). */
typedef struct rocknpu_decode_cache_stats {
    size_t hits;
    size_t misses;
    size_t entries;
    size_t resident_bytes;
    uint64_t hit_ns;
    uint64_t miss_ns;
    size_t tuned_shapes;
    size_t worker1_calls;
    size_t worker2_calls;
    size_t worker3_calls;
    size_t ksplit_calls;
} rocknpu_decode_cache_stats;

/* Reference include/rocknpu.h:27-32. */
enum rocknpu_status {
    ROCKNPU_STATUS_OK = 0,
    ROCKNPU_STATUS_INVALID_ARGUMENT = -1,
    ROCKNPU_STATUS_DEVICE_ERROR = -2,
    ROCKNPU_STATUS_EXECUTION_ERROR = -3,
};

/* Reference :34 (lib.rs:3725-3727): 1 when a HIP device is present, else 0. */
size_t rocknpu_device_count(void);
/* Reference :35 (lib.rs:3730-3777): NULL when no device is usable. */
rocknpu_context * rocknpu_context_create(void);
/* Reference :36-38 (lib.rs:3785-3848). */
int rocknpu_context_decode_cache_stats(
    const rocknpu_context * context,
    rocknpu_decode_cache_stats * out);
/* Reference :39 (lib.rs:3880-3999): NULL is a no-op. */
void rocknpu_context_destroy(rocknpu_context * context);

/* Reference :41-45 (lib.rs:3860-3872): one-shot host callback run after the
 * next M=1 W8 projection has been enqueued on the GPU and before the wait.
 * NULL clears it; a caller whose callback did not run must run the work. */
typedef void (*rocknpu_overlap_fn)(void * user_data);
int rocknpu_context_set_overlap(rocknpu_context * context, rocknpu_overlap_fn callback, void * user_data);

/* Reference :47-53 (lib.rs:2457-2614): 1..4 same-input projections run as one
 * concatenated-N GEMM with the activations quantised once; outputs[i] gets
 * [m, ns[i]]. Bit-identical to separate calls. */
int rocknpu_matmul_q_concat_f32_f32_mtile(
    rocknpu_context * context, size_t count,
    const uint8_t * const * weights, const size_t * bytes, const uint32_t * kinds, const size_t * ns,
    const float * activations_mk_f32, float * const * outputs, size_t m, size_t k);

/* Reference :55-60 (lib.rs:2426-2445): drop prompt-path device copies of these
 * weights and every concatenated group holding one of them, except the group
 * made of exactly these weights in this order. M=1 caches are kept. */
int rocknpu_mtile_release(
    rocknpu_context * context, size_t count, const uint8_t * const * weights);

/* Reference :62-68 (lib.rs:4074-4120): repack into the resident cache only. */
int rocknpu_prewarm_quantized_m16(
    rocknpu_context * context,
    const uint8_t * weights,
    size_t weights_bytes,
    uint32_t quant_kind,
    size_t k,
    size_t n);

/* Reference :70-77 (lib.rs:4134-4196): FP16 bridge, C = A * W^T with the
 * activations rounded to f16 and f32 accumulation. */
int rocknpu_matmul_f16_f32_f32(
    rocknpu_context * context,
    const uint16_t * weights_nk_f16_bits,
    const float * activations_mk_f32,
    float * output_mn_f32,
    size_t m,
    size_t k,
    size_t n);

/* Reference :79-86 (lib.rs:4207-4251): scales must be finite and > 0. */
int rocknpu_matmul_w8a8_f32_f32_m1(
    rocknpu_context * context,
    const int8_t * weights_nk_i8,
    const float * weight_scales_n_f32,
    const float * activations_k_f32,
    float * output_n_f32,
    size_t k,
    size_t n);

/* Reference :88-95 (lib.rs:4395-4447): M is fixed at 16. */
int rocknpu_matmul_w8a8_f32_f32_m16(
    rocknpu_context * context,
    const int8_t * weights_nk_i8,
    const float * weight_scales_n_f32,
    const float * activations_mk_f32,
    float * output_mn_f32,
    size_t k,
    size_t n);

/* Reference :97-105 (lib.rs:4259-4301): N in chunks of chunk_n (multiples of 32). */
int rocknpu_matmul_w8a8_f32_f32_m1_nsplit(
    rocknpu_context * context,
    const int8_t * weights_nk_i8,
    const float * weight_scales_n_f32,
    const float * activations_k_f32,
    float * output_n_f32,
    size_t k,
    size_t n,
    size_t chunk_n);

/* Reference :107-119 (lib.rs:4308-4393): gate/up pair, f32 SwiGLU
 * g * (1 / (1 + exp(-g))) * u, then the down projection. Here the SwiGLU runs
 * on the device between the two W8A8 products (the device expf), so the
 * intermediate never leaves HBM. */
int rocknpu_matmul_w8a8_swiglu_down_f32(
    rocknpu_context * context,
    const int8_t * gate_weights_nk_i8,
    const float * gate_scales_n_f32,
    const int8_t * up_weights_nk_i8,
    const float * up_scales_n_f32,
    const int8_t * down_weights_nk_i8,
    const float * down_scales_n_f32,
    const float * activations_k_f32,
    float * output_n_f32,
    size_t projection_k,
    size_t ffn_n,
    size_t output_n);

/* Reference :121-132 (lib.rs:4449-4523). */
int rocknpu_matmul_w8a8_pair_f32_f32_m1(
    rocknpu_context * context,
    const int8_t * first_weights_nk_i8,
    const float * first_scales_n_f32,
    size_t first_n,
    const int8_t * second_weights_nk_i8,
    const float * second_scales_n_f32,
    size_t second_n,
    const float * activations_k_f32,
    float * first_output_f32,
    float * second_output_f32,
    size_t k);

/* Reference :134-148 (lib.rs:4719-4821). */
int rocknpu_matmul_q_pair_f32_f32_mtile(
    rocknpu_context * context,
    const uint8_t * first_weights,
    size_t first_bytes,
    uint32_t first_kind,
    size_t first_n,
    const uint8_t * second_weights,
    size_t second_bytes,
    uint32_t second_kind,
    size_t second_n,
    const float * activations_mk_f32,
    float * first_output_mn_f32,
    float * second_output_mn_f32,
    size_t m,
    size_t k);

/* Reference :150-157 (lib.rs:4529-4631). */
int rocknpu_matmul_w8a8_triple_f32_f32_m1(
    rocknpu_context * context,
    const int8_t * first_weights_nk_i8, const float * first_scales_n_f32, size_t first_n,
    const int8_t * second_weights_nk_i8, const float * second_scales_n_f32, size_t second_n,
    const int8_t * third_weights_nk_i8, const float * third_scales_n_f32, size_t third_n,
    const float * activations_k_f32,
    float * first_output_f32, float * second_output_f32, float * third_output_f32,
    size_t k);

/* Reference :159-172 (lib.rs:4633-4717). */
int rocknpu_matmul_q_pair_f32_f32_m1(
    rocknpu_context * context,
    const uint8_t * first_weights,
    size_t first_bytes,
    uint32_t first_kind,
    size_t first_n,
    const uint8_t * second_weights,
    size_t second_bytes,
    uint32_t second_kind,
    size_t second_n,
    const float * activations_k_f32,
    float * first_output_f32,
    float * second_output_f32,
    size_t k);

/* Reference :174-192 (lib.rs:4823-4930). */
int rocknpu_matmul_q_triple_f32_f32_m1(
    rocknpu_context * context,
    const uint8_t * first_weights,
    size_t first_bytes,
    uint32_t first_kind,
    size_t first_n,
    const uint8_t * second_weights,
    size_t second_bytes,
    uint32_t second_kind,
    size_t second_n,
    const uint8_t * third_weights,
    size_t third_bytes,
    uint32_t third_kind,
    size_t third_n,
    const float * activations_k_f32,
    float * first_output_f32,
    float * second_output_f32,
    float * third_output_f32,
    size_t k);

/* Reference :194-202 (lib.rs:4933-5256): W8A8 route for every M >= 1. */
int rocknpu_matmul_q4_k_f32_f32(
    rocknpu_context * context,
    const uint8_t * weights_nk_q4_k,
    size_t weights_bytes,
    const float * activations_mk_f32,
    float * output_mn_f32,
    size_t m,
    size_t k,
    size_t n);

/* Reference :204-212 (lib.rs:5270-5378): prompt path only, M == 1 is rejected. */
int rocknpu_matmul_q5_k_f32_f32(
    rocknpu_context * context,
    const uint8_t * weights_nk_q5_k,
    size_t weights_bytes,
    const float * activations_mk_f32,
    float * output_mn_f32,
    size_t m,
    size_t k,
    size_t n);

/* Reference :214-222 (lib.rs:5380-5671). */
int rocknpu_matmul_q6_k_f32_f32(
    rocknpu_context * context,
    const uint8_t * weights_nk_q6_k,
    size_t weights_bytes,
    const float * activations_mk_f32,
    float * output_mn_f32,
    size_t m,
    size_t k,
    size_t n);

#ifdef __cplusplus
}
#endif

#endif
