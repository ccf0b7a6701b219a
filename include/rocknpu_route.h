/*
 * rocknpu_route.h — MUL_MAT routing of a ggml backend over this C ABI,
 * without ggml.
 *
 * The reference plugin decides per graph node whether the backend takes a
 * MUL_MAT (supports_op, adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:614-715),
 * groups later projections that read the same activations into one call
 * (rocknpu_mtile_group, :856-976), and dispatches each group or node to a
 * rocknpu.h entry point (rocknpu_backend_graph_compute, :978-1650). These
 * functions make the same three decisions from a plain description of each
 * node, so a plugin fills one rocknpu_mul_mat_node per ggml MUL_MAT and calls
 * them; the tests drive them the same way.
 *
 * GPU deviations from the NPU plugin: the NPU tile limits (K % 512,
 * K <= 4096 or 12288, N % 32, N <= 8192 or 3 x 8192, M <= 128 without
 * ROCKNPU_PREFILL_CACHE) and the scheduling experiments behind ROCKNPU_SCHED_*,
 * ROCKNPU_M16_ONLY and ROCKNPU_RUNTIME_* are not applied: every entry point
 * here takes any shape with K % 256 == 0. Groups hold up to 4 projections of
 * any M (the NPU took M >= 32).
 */
#ifndef ROCKNPU_ROUTE_H
#define ROCKNPU_ROUTE_H

#include <stddef.h>
#include <stdint.h>

#include "rocknpu.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type ids (ggml.h enum ggml_type) the routing reads. */
#define ROCKNPU_TYPE_F32 0
#define ROCKNPU_TYPE_F16 1
#define ROCKNPU_TYPE_Q4_K 12
#define ROCKNPU_TYPE_Q5_K 13
#define ROCKNPU_TYPE_Q6_K 14

/* What graph_compute reads of a MUL_MAT node dst = src0 x src1. */
typedef struct rocknpu_mul_mat_node {
    int32_t weight_type;      /* src0->type */
    int32_t activation_type;  /* src1->type */
    int32_t output_type;      /* dst->type */
    int32_t contiguous;       /* ggml_is_contiguous of src0, src1 and dst */
    int64_t weight_ne[4];     /* src0->ne: K, N, 1, 1 */
    int64_t activation_ne[4]; /* src1->ne: K, M, 1, 1 */
    const void * weights;     /* src0->data */
    size_t weight_bytes;      /* ggml_nbytes(src0) */
    const float * activations;/* src1->data: nodes with the same pointer share an input */
    float * output;           /* dst->data, M x N f32 */
    const char * weight_name; /* src0->name ("blk.<layer>.attn_q.weight", ...), or NULL */
} rocknpu_mul_mat_node;

/* Dispatch counters of the routing over one context (the plugin's TRACE
 * summary counters, ggml-rocknpu.cpp:721-736, and its split-profile counters,
 * :758-818). Printed to stderr when the context is destroyed if
 * ROCKNPU_GGML_TRACE or ROCKNPU_DISPATCH_SUMMARY is set.
 *
 * ROCKNPU_SPLIT_PROFILE (ggml-rocknpu.cpp:758-818, :1080-1092, :1623-1632):
 * every rocknpu_route_run call's wall time is kept as a sample, and from the
 * 112th call on every projection run on its own is timed per "M=.. K=.. N=.."
 * shape. At destroy the context prints one "ROCKNPU SHAPE PROFILE" line per
 * shape and one "ROCKNPU SPLIT PROFILE" line: calls, nodes, total and mean
 * times, the counters below, the samples of 5 ms and 20 ms or more, the last
 * 5 ms sample, the longest, the first 111 calls against the rest, and the four
 * quarters of the samples (time and 20 ms samples each), in the plugin's
 * format. The entry points return once the results are in host memory, so
 * the wall times are the GPU work's. */
typedef struct rocknpu_route_stats {
    size_t graph_calls;        /* rocknpu_route_run calls */
    size_t q4_k_mul_mat;       /* projections run, by weight type */
    size_t q5_k_mul_mat;
    size_t q6_k_mul_mat;
    size_t f16_mul_mat;
    size_t q8k_m1_mul_mat;     /* M = 1 projections on the ROCKNPU_DECODE_GGML route */
    size_t w8a8_m1_mul_mat;    /* M = 1 projections on the ROCKNPU_DECODE_W8A8 route */
    size_t mtile_group_calls;  /* same-input group calls (2..4 projections, M > 1) */
    size_t qkv_triple_calls;   /* Q nodes run as Q+K+V with K/V stashed */
    size_t qkv_stash_hits;     /* K/V nodes served from the stash */
    size_t graph_nodes;        /* nodes passed to rocknpu_route_run */
    uint64_t graph_ns;         /* wall time in rocknpu_route_run */
    /* projections by M: single projections of M 4, 8, 12, 16 and any other M;
     * the members of same-input groups with M > 1 count as "other", and
     * single-token groups in none (the plugin's m4 .. m_other counters) */
    size_t m4_mul_mat;
    size_t m8_mul_mat;
    size_t m12_mul_mat;
    size_t m16_mul_mat;
    size_t m_other_mul_mat;
} rocknpu_route_stats;

/* Where single-token (M = 1) MUL_MATs go (ROCKNPU_DECODE, ggml-rocknpu.cpp:305-322). */
enum rocknpu_decode_route {
    ROCKNPU_DECODE_CPU = 0,  /* left to ggml-cpu (the reference default) */
    ROCKNPU_DECODE_GGML = 1, /* GPU, llama.cpp's Q8_K arithmetic (rocknpu_ggml.h) */
    ROCKNPU_DECODE_W8A8 = 2, /* GPU, the reference's NPU route: W8A8 M=1 entries */
};

/* 1 when the backend takes the node, else 0 (supports_op,
 * ggml-rocknpu.cpp:614-715): F16/Q4_K/Q5_K/Q6_K weights, f32 activations and
 * output, all contiguous, 2-D, matching K, weight bytes that match the
 * shape, K % 256 == 0 for K-quants; M = 1 only for Q4_K/Q6_K and
 * a GPU decode route (Q5_K and F16 decode stay on the CPU, as in the
 * reference). */
int rocknpu_route_supported(const rocknpu_mul_mat_node * node, int32_t decode_route);

/* Same-input groups in node order (rocknpu_mtile_group,
 * ggml-rocknpu.cpp:856-887): a supported Q4_K/Q6_K node leads a group and
 * takes up to 3 later supported Q4_K/Q6_K nodes with the same activations
 * pointer, K and M, not already taken; every other node is a group of its
 * own. group_of[i] = index of the lead node of node i's group (group_of has
 * `count` entries; unsupported nodes get -1). Returns the number of groups.
 *
 * A group runs at its lead's position, so a later member j is taken only if
 * that move is invisible: no node between the lead and j writes memory j
 * reads or writes, or reads memory j writes, and j's output overlaps neither
 * the shared activations nor another member's output. The plugin compares
 * ggml tensors (src[1] identity); addresses are what this interface sees, and
 * a buffer ggml-alloc reused for another tensor has the same address. `nodes`
 * must therefore hold every computing node of the split, in graph order
 * (the split's other ops are views). ROCKNPU_MTILE_GROUP=0 turns grouping off. */
size_t rocknpu_route_plan(const rocknpu_mul_mat_node * nodes, size_t count, int32_t decode_route,
                          int32_t * group_of);

/* Runs the nodes' groups in lead order through the entry points (below).
 * With ROCKNPU_MTILE_QKV (default on; ggml-rocknpu.cpp:871-928) and M > 1, a
 * Q projection ("blk.<L>.attn_q.weight") that runs alone while layer L's K and
 * V weights are known from an earlier call runs as one Q+K+V group, its K/V
 * outputs kept in the context; the K and V nodes of a later call (another
 * split) that read the same activations with the same M are then filled from
 * that stash instead of computed again, bit for bit the same values. After a
 * layer's first such triple, the single and pair prompt caches of its three
 * weights are released (rocknpu_mtile_release, :953-962).
 * Entry points, by group:
 *   group of 2..4, M > 1:            rocknpu_matmul_q_concat_f32_f32_mtile
 *   group of 2..4, M = 1, GGML:      rocknpu_matmul_q_q8k_group_f32_f32
 *   group of 2 or 3, M = 1, W8A8:    rocknpu_matmul_q_pair_f32_f32_m1 / _triple_
 *                                    (4: two pairs)
 *   single Q4_K/Q6_K, M = 1, GGML:   rocknpu_matmul_q_q8k_f32_f32
 *   single Q4_K/Q5_K/Q6_K:           rocknpu_matmul_q{4,5,6}_k_f32_f32
 *   single F16:                      rocknpu_matmul_f16_f32_f32
 * ROCKNPU_STATUS_INVALID_ARGUMENT for an unsupported node (the plugin's
 * graph_compute fails the graph the same way, ggml-rocknpu.cpp:1099-1102);
 * otherwise the first failing call's status, or ROCKNPU_STATUS_OK. */
int rocknpu_route_run(rocknpu_context * context, const rocknpu_mul_mat_node * nodes, size_t count,
                      int32_t decode_route);

/* Copies the context's dispatch counters to *out. */
int rocknpu_route_stats_get(const rocknpu_context * context, rocknpu_route_stats * out);

#ifdef __cplusplus
}
#endif

#endif
