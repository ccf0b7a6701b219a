// MUL_MAT routing over the C ABI (include/rocknpu_route.h): which nodes the
// backend takes, which same-input projections run as one call, and which
// entry point each group goes to — the decisions of the reference plugin's
// supports_op (adapters/ggml-rocknpu/src/ggml-rocknpu.cpp:614-715),
// rocknpu_mtile_group (:856-976, with the cross-partition Q/K/V stash of
// :871-928) and graph_compute (:978-1650), made from plain node descriptions
// instead of ggml tensors. Host code only.
#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "context.h"
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

// ROCKNPU_MTILE_GROUP / ROCKNPU_MTILE_QKV: on unless set to "0" (the plugin's
// rocknpu_env_enabled_default(..., true)).
bool env_default_on(const char* name) {
    const char* v = std::getenv(name);
    return v == nullptr || v[0] == '\0' || std::strcmp(v, "0") != 0;
}
bool env_on(const char* name) {
    const char* v = std::getenv(name);
    return v != nullptr && v[0] != '\0' && v[0] != '0';
}

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

// Byte ranges a node reads (its activations) and writes (its output).
struct Span {
    uintptr_t lo, hi;
};
Span reads(const rocknpu_mul_mat_node& nd) {
    const uintptr_t p = reinterpret_cast<uintptr_t>(nd.activations);
    return Span{p, p + static_cast<uintptr_t>(m_of(nd) * k_of(nd)) * sizeof(float)};
}
Span writes(const rocknpu_mul_mat_node& nd) {
    const uintptr_t p = reinterpret_cast<uintptr_t>(nd.output);
    return Span{p, p + static_cast<uintptr_t>(m_of(nd) * n_of(nd)) * sizeof(float)};
}
bool overlap(Span a, Span b) { return a.lo < b.hi && b.lo < a.hi; }

// Whether node j may run at lead i's position with the members already taken:
// the move must not reorder j against any node between them that it depends
// on (writes j's input, or reads or writes j's output), and j must not write
// the shared input or another member's output.
bool movable(const rocknpu_mul_mat_node* nodes, size_t i, size_t j, const size_t* members, size_t count) {
    const Span rj = reads(nodes[j]), wj = writes(nodes[j]);
    for (size_t t = i + 1; t < j; ++t) {
        const Span rt = reads(nodes[t]), wt = writes(nodes[t]);
        if (overlap(wt, rj) || overlap(rt, wj) || overlap(wt, wj)) return false;
    }
    if (overlap(wj, rj)) return false;
    for (size_t g = 0; g < count; ++g)
        if (overlap(wj, writes(nodes[members[g]]))) return false;
    return true;
}

void plan_groups(const rocknpu_mul_mat_node* nodes, size_t count, int32_t decode, bool grouping,
                 int32_t* group_of, size_t* groups_out) {
    for (size_t i = 0; i < count; ++i) group_of[i] = -2;  // not yet placed
    size_t groups = 0;
    for (size_t i = 0; i < count; ++i) {
        if (group_of[i] != -2) continue;
        const rocknpu_mul_mat_node& lead = nodes[i];
        if (!supported(lead, decode)) {
            group_of[i] = -1;
            continue;
        }
        group_of[i] = static_cast<int32_t>(i);
        ++groups;
        if (!grouping || !groupable(lead.weight_type) || overlap(writes(lead), reads(lead))) continue;
        size_t members[kMaxGroup] = {i};
        size_t taken = 1;
        for (size_t j = i + 1; j < count && taken < kMaxGroup; ++j) {
            const rocknpu_mul_mat_node& c = nodes[j];
            if (group_of[j] != -2 || c.activations != lead.activations || !groupable(c.weight_type) ||
                k_of(c) != k_of(lead) || m_of(c) != m_of(lead) || !supported(c, decode) ||
                !movable(nodes, i, j, members, taken))
                continue;
            group_of[j] = static_cast<int32_t>(i);
            members[taken++] = j;
        }
    }
    *groups_out = groups;
}

// "blk.<layer>." prefix and the attention weight's suffix (the plugin's
// rocknpu_attention_layer, ggml-rocknpu.cpp:505-516).
bool attention_layer(const rocknpu_mul_mat_node& nd, const char* needle, size_t* layer) {
    if (nd.weight_name == nullptr || std::strstr(nd.weight_name, needle) == nullptr) return false;
    size_t parsed = 0;
    if (std::sscanf(nd.weight_name, "blk.%zu.", &parsed) != 1 || parsed >= rk::kQkvMaxLayers) return false;
    *layer = parsed;
    return true;
}

// A projection run on its own, by M (the plugin counts every M here, 1 included).
void count_m(rocknpu_route_stats& st, int64_t m) {
    (m == 4 ? st.m4_mul_mat : m == 8 ? st.m8_mul_mat : m == 12 ? st.m12_mul_mat : m == 16 ? st.m16_mul_mat
                                                                                        : st.m_other_mul_mat)++;
}

uint64_t since_ns(std::chrono::steady_clock::time_point t0) {
    return static_cast<uint64_t>(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0).count());
}

void count_run(rocknpu_route_stats& st, const rocknpu_mul_mat_node& nd, int32_t decode) {
    switch (nd.weight_type) {
    case ROCKNPU_TYPE_Q4_K: st.q4_k_mul_mat++; break;
    case ROCKNPU_TYPE_Q5_K: st.q5_k_mul_mat++; break;
    case ROCKNPU_TYPE_Q6_K: st.q6_k_mul_mat++; break;
    default: st.f16_mul_mat++; break;
    }
    if (m_of(nd) == 1) (decode == ROCKNPU_DECODE_GGML ? st.q8k_m1_mul_mat : st.w8a8_m1_mul_mat)++;
}

// The cross-partition Q/K/V stash for one prompt group (ggml-rocknpu.cpp:871-962).
// Returns 1 when it handled the group (*status set), 0 when the group runs as usual.
int qkv_stash(rocknpu_context* ctx, const rocknpu_mul_mat_node* const* g, size_t c, int* status) {
    rk::RouteState& rs = ctx->route;
    const rocknpu_mul_mat_node& lead = *g[0];
    const size_t m = static_cast<size_t>(m_of(lead)), k = static_cast<size_t>(k_of(lead));
    // remember each layer's K/V weights; count the members a pending stash holds
    size_t stashed = 0, layer = 0;
    for (size_t t = 0; t < c; ++t) {
        const bool is_k = attention_layer(*g[t], ".attn_k.weight", &layer);
        if (!is_k && !attention_layer(*g[t], ".attn_v.weight", &layer)) continue;
        rk::QkvLayer& st = rs.qkv[layer];
        rk::QkvWeight& w = is_k ? st.wk : st.wv;
        w = rk::QkvWeight{g[t]->weights, g[t]->weight_bytes, static_cast<size_t>(n_of(*g[t])), k, g[t]->weight_type};
        const bool pending = is_k ? st.k_pending : st.v_pending;
        const std::vector<float>& out = is_k ? st.k_out : st.v_out;
        stashed += pending && st.activation == lead.activations && st.rows == m &&
                   out.size() == m * static_cast<size_t>(n_of(*g[t]));
    }
    if (stashed == c) {
        for (size_t t = 0; t < c; ++t) {
            const bool is_k = attention_layer(*g[t], ".attn_k.weight", &layer);
            if (!is_k) attention_layer(*g[t], ".attn_v.weight", &layer);
            rk::QkvLayer& st = rs.qkv[layer];
            const std::vector<float>& out = is_k ? st.k_out : st.v_out;
            std::memcpy(g[t]->output, out.data(), out.size() * sizeof(float));
            (is_k ? st.k_pending : st.v_pending) = false;
            rs.stats.qkv_stash_hits++;
        }
        *status = kOk;
        return 1;
    }
    // a Q projection alone, with its layer's K/V weights known: run Q, K and V together
    if (c != 1 || !attention_layer(lead, ".attn_q.weight", &layer)) return 0;
    rk::QkvLayer& st = rs.qkv[layer];
    st.k_pending = st.v_pending = false;
    if (st.wk.data == nullptr || st.wv.data == nullptr || st.wk.k != k || st.wv.k != k || !groupable(st.wk.type) ||
        !groupable(st.wv.type))
        return 0;
    st.k_out.resize(m * st.wk.n);
    st.v_out.resize(m * st.wv.n);
    const uint8_t* w[3] = {static_cast<const uint8_t*>(lead.weights), static_cast<const uint8_t*>(st.wk.data),
                           static_cast<const uint8_t*>(st.wv.data)};
    size_t bytes[3] = {lead.weight_bytes, st.wk.bytes, st.wv.bytes};
    uint32_t kinds[3] = {kind_of(lead.weight_type), kind_of(st.wk.type), kind_of(st.wv.type)};
    size_t ns[3] = {static_cast<size_t>(n_of(lead)), st.wk.n, st.wv.n};
    float* outs[3] = {lead.output, st.k_out.data(), st.v_out.data()};
    if (rocknpu_matmul_q_concat_f32_f32_mtile(ctx, 3, w, bytes, kinds, ns, lead.activations, outs, m, k) != kOk)
        return 0;  // the plugin then runs Q on its own (:949-951)
    st.activation = lead.activations;
    st.rows = m;
    st.k_pending = st.v_pending = true;
    rs.stats.qkv_triple_calls++;
    rs.stats.m_other_mul_mat += 3;
    for (int32_t t : {lead.weight_type, st.wk.type, st.wv.type})
        (t == ROCKNPU_TYPE_Q4_K ? rs.stats.q4_k_mul_mat : rs.stats.q6_k_mul_mat)++;
    if (!st.released) {
        // the single and pair prompt caches of these weights are now unused
        rocknpu_mtile_release(ctx, 3, w);
        st.released = true;
    }
    if (env_on("ROCKNPU_GGML_TRACE"))
        std::fprintf(stderr, "ROCKNPU GGML TRACE qkv_triple layer=%zu M=%zu K=%zu N=%zu\n", layer, m, k,
                     ns[0] + ns[1] + ns[2]);
    *status = kOk;
    return 1;
}

}  // namespace

namespace rk {
namespace {
// The ROCKNPU_SPLIT_PROFILE report (ggml-rocknpu.cpp:758-818): the shapes,
// then the calls' summary, field for field in the plugin's format, so logs
// read the same. The first 111 calls are the plugin's warm-up batch; the
// shape timings start after it.
constexpr size_t kWarmCalls = 111;
void split_profile_print(const RouteState& rs) {
    const rocknpu_route_stats& s = rs.stats;
    const std::vector<uint64_t>& v = rs.samples_ns;
    size_t slow5 = 0, slow20 = 0, last_slow5 = 0;
    uint64_t max_ns = 0, first_ns = 0, rest_ns = 0, q_ns[4] = {0, 0, 0, 0};
    size_t q_slow20[4] = {0, 0, 0, 0};
    for (size_t i = 0; i < v.size(); ++i) {
        const uint64_t ns = v[i];
        const bool s20 = ns >= 20000000u;
        max_ns = std::max(max_ns, ns);
        if (ns >= 5000000u) {
            ++slow5;
            last_slow5 = i + 1;
        }
        slow20 += s20 ? 1 : 0;
        const size_t q = std::min<size_t>(3, i * 4 / v.size());
        q_ns[q] += ns;
        q_slow20[q] += s20 ? 1 : 0;
        (i < kWarmCalls ? first_ns : rest_ns) += ns;
    }
    for (const auto& e : rs.shapes)
        std::fprintf(stderr, "ROCKNPU SHAPE PROFILE %s calls=%zu total_ms=%.3f avg_ms=%.3f\n", e.first.c_str(),
                     e.second.first, e.second.second / 1e6, e.second.second / 1e6 / static_cast<double>(e.second.first));
    const double graph_ms = s.graph_ns / 1e6, calls = static_cast<double>(s.graph_calls);
    // cpu_fallback and native_w8 stay 0: unsupported nodes never reach this
    // routing (rocknpu_route_run rejects them), and f32 weights are not taken
    std::fprintf(stderr,
                 "ROCKNPU SPLIT PROFILE graph_calls=%zu graph_nodes=%zu graph_ms=%.3f avg_call_ms=%.3f "
                 "avg_nodes=%.2f cpu_fallback=%zu q4=%zu q6=%zu f16=%zu native_w8=%zu "
                 "m=[4:%zu,8:%zu,12:%zu,16:%zu,other:%zu] slow5=%zu slow20=%zu last_slow5=%zu max_ms=%.3f "
                 "first111_ms=%.3f rest_ms=%.3f q_ms=[%.3f,%.3f,%.3f,%.3f] q_slow20=[%zu,%zu,%zu,%zu]\n",
                 s.graph_calls, s.graph_nodes, graph_ms, s.graph_calls ? graph_ms / calls : 0.0,
                 s.graph_calls ? static_cast<double>(s.graph_nodes) / calls : 0.0, size_t{0}, s.q4_k_mul_mat,
                 s.q6_k_mul_mat, s.f16_mul_mat, size_t{0}, s.m4_mul_mat, s.m8_mul_mat, s.m12_mul_mat,
                 s.m16_mul_mat, s.m_other_mul_mat, slow5, slow20, last_slow5, max_ns / 1e6, first_ns / 1e6,
                 rest_ns / 1e6, q_ns[0] / 1e6, q_ns[1] / 1e6, q_ns[2] / 1e6, q_ns[3] / 1e6, q_slow20[0],
                 q_slow20[1], q_slow20[2], q_slow20[3]);
}
}  // namespace

// Called from rocknpu_context_destroy: the plugin's TRACE summary line
// (ggml-rocknpu.cpp:721-736) and the split profile.
void route_print_summary(const RockNpuContext* ctx) {
    const rocknpu_route_stats& s = ctx->route.stats;
    if (env_on("ROCKNPU_SPLIT_PROFILE")) split_profile_print(ctx->route);
    if (!env_on("ROCKNPU_GGML_TRACE") && !env_on("ROCKNPU_DISPATCH_SUMMARY")) return;
    if (s.graph_calls == 0) return;
    std::fprintf(stderr,
                 "ROCKNPU GGML TRACE summary graph_calls=%zu q4_K_mul_mat=%zu q5_K_mul_mat=%zu q6_K_mul_mat=%zu "
                 "f16_mul_mat=%zu q8k_m1_mul_mat=%zu w8a8_m1_mul_mat=%zu mtile_group_calls=%zu "
                 "qkv_triple_calls=%zu qkv_stash_hits=%zu\n",
                 s.graph_calls, s.q4_k_mul_mat, s.q5_k_mul_mat, s.q6_k_mul_mat, s.f16_mul_mat, s.q8k_m1_mul_mat,
                 s.w8a8_m1_mul_mat, s.mtile_group_calls, s.qkv_triple_calls, s.qkv_stash_hits);
}
}  // namespace rk

extern "C" {

int rocknpu_route_supported(const rocknpu_mul_mat_node* node, int32_t decode_route) {
    return node != nullptr && supported(*node, decode_route) ? 1 : 0;
}

size_t rocknpu_route_plan(const rocknpu_mul_mat_node* nodes, size_t count, int32_t decode_route,
                          int32_t* group_of) {
    if (nodes == nullptr || group_of == nullptr) return 0;
    size_t groups = 0;
    plan_groups(nodes, count, decode_route, env_default_on("ROCKNPU_MTILE_GROUP"), group_of, &groups);
    return groups;
}

int rocknpu_route_stats_get(const rocknpu_context* ctx, rocknpu_route_stats* out) {
    if (ctx == nullptr || out == nullptr) return kInvalid;
    *out = ctx->route.stats;
    return kOk;
}

int rocknpu_route_run(rocknpu_context* ctx, const rocknpu_mul_mat_node* nodes, size_t count,
                      int32_t decode_route) {
    if (ctx == nullptr || (nodes == nullptr && count > 0)) return kInvalid;
    for (size_t i = 0; i < count; ++i)
        if (!supported(nodes[i], decode_route)) return kInvalid;
    rocknpu_route_stats& stats = ctx->route.stats;
    stats.graph_calls++;
    stats.graph_nodes += count;
    const bool profile = env_on("ROCKNPU_SPLIT_PROFILE");
    // the call's wall time, on every return
    struct CallTimer {
        rk::RouteState& rs;
        bool keep;
        std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();
        ~CallTimer() {
            const uint64_t ns = since_ns(t0);
            rs.stats.graph_ns += ns;
            if (keep) rs.samples_ns.push_back(ns);
        }
    } timer{ctx->route, profile};
    const bool shape_profile = profile && stats.graph_calls > rk::kWarmCalls;
    const bool trace = env_on("ROCKNPU_GGML_TRACE");
    const bool qkv = env_default_on("ROCKNPU_MTILE_QKV");
    // the plan's groups, walked in lead order
    std::vector<int32_t> group_of(count);
    size_t groups = 0;
    plan_groups(nodes, count, decode_route, env_default_on("ROCKNPU_MTILE_GROUP"), group_of.data(), &groups);
    for (size_t i = 0; i < count; ++i) {
        if (group_of[i] != static_cast<int32_t>(i)) continue;  // not a lead
        const rocknpu_mul_mat_node* g[kMaxGroup];
        size_t c = 0;
        for (size_t j = i; j < count && c < kMaxGroup; ++j)
            if (group_of[j] == static_cast<int32_t>(i)) g[c++] = &nodes[j];
        const rocknpu_mul_mat_node& lead = *g[0];
        const size_t k = static_cast<size_t>(k_of(lead)), m = static_cast<size_t>(m_of(lead));
        int st = kOk;
        if (qkv && m > 1 && groupable(lead.weight_type) && qkv_stash(ctx, g, c, &st)) {
            if (st != kOk) return st;
            continue;
        }
        if (c > 1) {
            const uint8_t* w[kMaxGroup];
            size_t bytes[kMaxGroup], ns[kMaxGroup];
            uint32_t kinds[kMaxGroup];
            float* outs[kMaxGroup];
            size_t total_n = 0;
            for (size_t t = 0; t < c; ++t) {
                w[t] = static_cast<const uint8_t*>(g[t]->weights);
                bytes[t] = g[t]->weight_bytes;
                ns[t] = static_cast<size_t>(n_of(*g[t]));
                kinds[t] = kind_of(g[t]->weight_type);
                outs[t] = g[t]->output;
                total_n += ns[t];
            }
            if (m > 1) {
                st = rocknpu_matmul_q_concat_f32_f32_mtile(ctx, c, w, bytes, kinds, ns, lead.activations, outs,
                                                           m, k);
                stats.mtile_group_calls++;
                if (st == kOk) stats.m_other_mul_mat += c;
                if (trace)
                    std::fprintf(stderr, "ROCKNPU GGML TRACE mtile_group lead=%s count=%zu M=%zu K=%zu N=%zu\n",
                                 lead.weight_name ? lead.weight_name : "?", c, m, k, total_n);
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
            for (size_t t = 0; t < c && st == kOk; ++t) count_run(stats, *g[t], decode_route);
        } else {
            const size_t n = static_cast<size_t>(n_of(lead));
            const uint8_t* w = static_cast<const uint8_t*>(lead.weights);
            const auto t0 = std::chrono::steady_clock::now();
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
            if (st == kOk) {
                count_run(stats, lead, decode_route);
                count_m(stats, static_cast<int64_t>(m));
            }
            if (shape_profile) {
                char key[96];
                std::snprintf(key, sizeof(key), "M=%zu K=%zu N=%zu", m, k, n);
                auto& e = ctx->route.shapes[key];
                e.first++;
                e.second += since_ns(t0);
            }
        }
        if (st != kOk) return st;
    }
    return kOk;
}

}  // extern "C"
