// MUL_MAT routing over the C ABI (include/rocknpu_route.h): which nodes the
// backend takes, which same-input projections run as one call, and which
// entry point each group goes to — the decisions of the reference plugin's
// supports_op (adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:614-715),
// rocknpu_mtile_group (:856-976) and graph_compute (:978-1650), made from
// plain node descriptions instead of ggml tensors. Host code only.
#include <cstdint>
#include <vector>

#include "rocknpu.h"
#include "rocknpu_ggml.h"
#include "rocknpu_route.h"

namespace {

constexpr int kOk = ROCKNPU_STATUS_OK;
constexpr int kInvalid = ROCKNPU_STATUS_INVALID_ARGUMENT;
constexpr int64_t kQK = 256;
constexpr size_t kMaxGroup = 4;

bool kquant(int32_t t) { return t == ROCKNPU_TYPE_Q4_K || t == ROCKNPU_TYPE_Q5_K || t == ROCKNPU_TYPE_Q6_K; }
// the K-quants a same-input group may hold (the concat entry's kinds)
bool groupable(int32_t t) { return t == ROCKNPU_TYPE_Q4_K || t == ROCKNPU_TYPE_Q6_K; }
uint32_t kind_of(int32_t t) { return t == ROCKNPU_TYPE_Q4_K ? 4 : t == ROCKNPU_TYPE_Q5_K ? 5 : 6; }
int64_t block_bytes(int32_t t) { return t == ROCKNPU_TYPE_Q4_K ? 144 : t == ROCKNPU_TYPE_Q5_K ? 176 : 210; }

int64_t k_of(const rocknpu_mul_mat_node& nd) { return nd.weight_ne[0]; }
int64_t n_of(const rocknpu_mul_mat_node& nd) { return nd.weight_ne[1]; }
int64_t m_of(const rocknpu_mul_mat_node& nd) { return nd.activation_ne[1]; }

bool supported(const rocknpu_mul_mat_node& nd, int32_t decode) {
    const int32_t wt = nd.weight_type;
    if ((wt != ROCKNPU_TYPE_F16 && !kquant(wt)) || nd.activation_type != ROCKNPU_TYPE_F32 ||
        nd.output_type != ROCKNPU_TYPE_F32 || !nd.contiguous)
        return false;
    if (nd.weight_ne[2] != 1 || nd.weight_ne[3] != 1 || nd.activation_ne[2] != 1 || nd.activation_ne[3] != 1)
        return false;
    const int64_t k = k_of(nd), n = n_of(nd), m = m_of(nd);
    if (k != nd.activation_ne[0] || k <= 0 || n <= 0 || m <= 0) return false;
    if (!nd.weights || !nd.activations || !nd.output) return false;
    if (kquant(wt)) {
        if (k % kQK != 0) return false;
        // ggml_nbytes of a 2-D K-quant tensor
        if (static_cast<int64_t>(nd.weight_bytes) / block_bytes(wt) / (k / kQK) != n ||
            static_cast<int64_t>(nd.weight_bytes) != n * (k / kQK) * block_bytes(wt))
            return false;
    } else if (static_cast<int64_t>(nd.weight_bytes) != n * k * 2) {
        return false;
    }
    if (m == 1) {
        // decode: the CPU route keeps it; Q5_K and F16 decode are CPU-only in
        // the reference too (ggml-rocknpu.cpp:674-698, lib.rs:5300)
        if (decode != ROCKNPU_DECODE_GGML && decode != ROCKNPU_DECODE_W8A8) return false;
        return groupable(wt);
    }
    return true;
}

}  // namespace

extern "C" {

int rocknpu_route_supported(const rocknpu_mul_mat_node* node, int32_t decode_route) {
    return node != nullptr && supported(*node, decode_route) ? 1 : 0;
}

size_t rocknpu_route_plan(const rocknpu_mul_mat_node* nodes, size_t count, int32_t decode_route,
                          int32_t* group_of) {
    if (nodes == nullptr || group_of == nullptr) return 0;
    for (size_t i = 0; i < count; ++i) group_of[i] = -2;  // not yet placed
    size_t groups = 0;
    for (size_t i = 0; i < count; ++i) {
        if (group_of[i] != -2) continue;
        const rocknpu_mul_mat_node& lead = nodes[i];
        if (!supported(lead, decode_route)) {
            group_of[i] = -1;
            continue;
        }
        group_of[i] = static_cast<int32_t>(i);
        ++groups;
        if (!groupable(lead.weight_type)) continue;
        size_t members = 1;
        for (size_t j = i + 1; j < count && members < kMaxGroup; ++j) {
            const rocknpu_mul_mat_node& c = nodes[j];
            if (group_of[j] != -2 || c.activations != lead.activations || !groupable(c.weight_type) ||
                k_of(c) != k_of(lead) || m_of(c) != m_of(lead) || !supported(c, decode_route))
                continue;
            group_of[j] = static_cast<int32_t>(i);
            ++members;
        }
    }
    return groups;
}

int rocknpu_route_run(rocknpu_context* ctx, const rocknpu_mul_mat_node* nodes, size_t count,
                      int32_t decode_route) {
    if (ctx == nullptr || (nodes == nullptr && count > 0)) return kInvalid;
    for (size_t i = 0; i < count; ++i)
        if (!supported(nodes[i], decode_route)) return kInvalid;
    // the plan's groups, walked in lead order
    std::vector<int32_t> group_of(count);
    rocknpu_route_plan(nodes, count, decode_route, group_of.data());
    for (size_t i = 0; i < count; ++i) {
        if (group_of[i] != static_cast<int32_t>(i)) continue;  // not a lead
        const rocknpu_mul_mat_node* g[kMaxGroup];
        size_t c = 0;
        for (size_t j = i; j < count && c < kMaxGroup; ++j)
            if (group_of[j] == static_cast<int32_t>(i)) g[c++] = &nodes[j];
        const rocknpu_mul_mat_node& lead = *g[0];
        const size_t k = static_cast<size_t>(k_of(lead)), m = static_cast<size_t>(m_of(lead));
        int st = kOk;
        if (c > 1) {
            const uint8_t* w[kMaxGroup];
            size_t bytes[kMaxGroup], ns[kMaxGroup];
            uint32_t kinds[kMaxGroup];
            float* outs[kMaxGroup];
            for (size_t t = 0; t < c; ++t) {
                w[t] = static_cast<const uint8_t*>(g[t]->weights);
                bytes[t] = g[t]->weight_bytes;
                ns[t] = static_cast<size_t>(n_of(*g[t]));
                kinds[t] = kind_of(g[t]->weight_type);
                outs[t] = g[t]->output;
            }
            if (m > 1) {
                st = rocknpu_matmul_q_concat_f32_f32_mtile(ctx, c, w, bytes, kinds, ns, lead.activations, outs,
                                                           m, k);
            } else if (decode_route == ROCKNPU_DECODE_GGML) {
                st = rocknpu_matmul_q_q8k_group_f32_f32(ctx, c, w, bytes, kinds, ns, lead.activations, outs, m,
                                                        k);
            } else if (c == 3) {
                st = rocknpu_matmul_q_triple_f32_f32_m1(ctx, w[0], bytes[0], kinds[0], ns[0], w[1], bytes[1],
                                                        kinds[1], ns[1], w[2], bytes[2], kinds[2], ns[2],
                                                        lead.activations, outs[0], outs[1], outs[2], k);
            } else {
                // pairs: members 0-1, then 2-3
                for (size_t t = 0; t + 1 < c && st == kOk; t += 2)
                    st = rocknpu_matmul_q_pair_f32_f32_m1(ctx, w[t], bytes[t], kinds[t], ns[t], w[t + 1],
                                                          bytes[t + 1], kinds[t + 1], ns[t + 1], lead.activations,
                                                          outs[t], outs[t + 1], k);
            }
        } else {
            const size_t n = static_cast<size_t>(n_of(lead));
            const uint8_t* w = static_cast<const uint8_t*>(lead.weights);
            if (lead.weight_type == ROCKNPU_TYPE_F16)
                st = rocknpu_matmul_f16_f32_f32(ctx, static_cast<const uint16_t*>(lead.weights), lead.activations,
                                                lead.output, m, k, n);
            else if (m == 1 && decode_route == ROCKNPU_DECODE_GGML)
                st = rocknpu_matmul_q_q8k_f32_f32(ctx, kind_of(lead.weight_type), w, lead.weight_bytes,
                                                  lead.activations, lead.output, m, k, n);
            else if (lead.weight_type == ROCKNPU_TYPE_Q4_K)
                st = rocknpu_matmul_q4_k_f32_f32(ctx, w, lead.weight_bytes, lead.activations, lead.output, m, k, n);
            else if (lead.weight_type == ROCKNPU_TYPE_Q5_K)
                st = rocknpu_matmul_q5_k_f32_f32(ctx, w, lead.weight_bytes, lead.activations, lead.output, m, k, n);
            else
                st = rocknpu_matmul_q6_k_f32_f32(ctx, w, lead.weight_bytes, lead.activations, lead.output, m, k, n);
        }
        if (st != kOk) return st;
    }
    return kOk;
}

}  // extern "C"
