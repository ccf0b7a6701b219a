/*
 * rocknpu_ggml.h — decode MUL_MAT with llama.cpp CPU numerics, on the GPU.
 *
 * The reference plugin leaves single-token decode to llama.cpp's CPU backend
 * (adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:311-322 ROCKNPU_DECODE=cpu, and
 * :674-679 where supports_op rejects M=1), i.e. ggml_compute_forward_mul_mat
 * with quantize_row_q8_K on the f32 activations and ggml_vec_dot_q4_K_q8_K /
 * ggml_vec_dot_q6_K_q8_K per output (llama.cpp ggml-cpu, commit pinned by
 * adapters/ggml-rocknpu/README.md:48). This entry point runs that computation
 * on the GPU so a plugin built on rocknpu.h can take decode MUL_MATs too.
 *
 * Host pointers, synchronous, same status codes and weight-cache contract as
 * rocknpu.h. kind: 4 = Q4_K, 6 = Q6_K. Non-finite activations are rejected
 * with ROCKNPU_STATUS_INVALID_ARGUMENT.
 */
#ifndef ROCKNPU_GGML_H
#define ROCKNPU_GGML_H

#include <stddef.h>
#include <stdint.h>

#include "rocknpu.h"

#ifdef __cplusplus
extern "C" {
#endif

int rocknpu_matmul_q_q8k_f32_f32(rocknpu_context * context, uint32_t kind, const uint8_t * weights,
                                 size_t weights_bytes, const float * activations_mk_f32,
                                 float * output_mn_f32, size_t m, size_t k, size_t n);

/* 1..4 projections that read the same activations (q/k/v, gate/up) in one
 * call, each output bit-identical to rocknpu_matmul_q_q8k_f32_f32 on that
 * projection. Arguments as rocknpu_matmul_q_concat_f32_f32_mtile (rocknpu.h;
 * reference rocknpu.h:47-53, lib.rs:2457-2614): kinds[i] is 4 or 6 and may
 * differ between members. The reference groups same-input projections this
 * way only on its prompt path (ggml-rocknpu.cpp:856-976). */
int rocknpu_matmul_q_q8k_group_f32_f32(rocknpu_context * context, size_t count,
                                       const uint8_t * const * weights, const size_t * bytes,
                                       const uint32_t * kinds, const size_t * ns,
                                       const float * activations_mk_f32, float * const * outputs,
                                       size_t m, size_t k);

#ifdef __cplusplus
}
#endif

#endif
