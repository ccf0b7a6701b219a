/*
 * CPU oracle for the ggml MUL_MAT offload path — TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * always as the checker; the product library never links or loads it.
 * Function-level citations are in oracle.h and beside each function below.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

float or_fp16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            /* subnormal half: renormalise into a normal single */
            uint32_t shift = 0;
            while (!(mant & 0x400u)) {
                mant <<= 1;
                shift++;
            }
            mant &= 0x3ffu;
            bits = sign | ((113u - shift) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

size_t or_block_bytes(uint32_t kind) {
    switch (kind) {
    case 4: return OR_Q4_K_BYTES;
    case 5: return OR_Q5_K_BYTES;
    case 6: return OR_Q6_K_BYTES;
    default: return 0;
    }
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ggml get_scale_min_k4: 6-bit scale and min of sub-block j (0..7) from the
 * 12-byte packed field of a Q4_K/Q5_K block. */
static void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Q4_K: d(f16) dmin(f16) scales[12] qs[128]; y = (d*sc)*q - (dmin*m). */
void or_dequant_q4_k(const uint8_t *b, float *y) {
    const float d = or_fp16_to_f32(rd16(b));
    const float dmin = or_fp16_to_f32(rd16(b + 2));
    const uint8_t *scales = b + 4;
    const uint8_t *qs = b + 16;
    for (int j = 0; j < 4; ++j) {
        uint8_t sc, mn;
        scale_min_k4(2 * j, scales, &sc, &mn);
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        scale_min_k4(2 * j + 1, scales, &sc, &mn);
        const float d2 = d * (float)sc, m2 = dmin * (float)mn;
        for (int l = 0; l < 32; ++l) y[64 * j + l] = d1 * (float)(qs[32 * j + l] & 0xF) - m1;
        for (int l = 0; l < 32; ++l) y[64 * j + 32 + l] = d2 * (float)(qs[32 * j + l] >> 4) - m2;
    }
}

/* Q5_K: d dmin scales[12] qh[32] qs[128]; the fifth bit of value l in
 * 64-chunk j comes from qh[l] bit 2j (low nibble) / 2j+1 (high nibble). */
void or_dequant_q5_k(const uint8_t *b, float *y) {
    const float d = or_fp16_to_f32(rd16(b));
    const float dmin = or_fp16_to_f32(rd16(b + 2));
    const uint8_t *scales = b + 4;
    const uint8_t *qh = b + 16;
    const uint8_t *qs = b + 48;
    for (int j = 0; j < 4; ++j) {
        uint8_t sc, mn;
        scale_min_k4(2 * j, scales, &sc, &mn);
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        scale_min_k4(2 * j + 1, scales, &sc, &mn);
        const float d2 = d * (float)sc, m2 = dmin * (float)mn;
        const uint8_t u1 = (uint8_t)(1u << (2 * j)), u2 = (uint8_t)(2u << (2 * j));
        for (int l = 0; l < 32; ++l)
            y[64 * j + l] = d1 * (float)((qs[32 * j + l] & 0xF) + ((qh[l] & u1) ? 16 : 0)) - m1;
        for (int l = 0; l < 32; ++l)
            y[64 * j + 32 + l] = d2 * (float)((qs[32 * j + l] >> 4) + ((qh[l] & u2) ? 16 : 0)) - m2;
    }
}

/* Q6_K value p of a block as a signed 6-bit integer in [-32, 31], with its
 * int8 sub-block scale index (ggml layout: ql[128] qh[64] scales[16] d). */
static int q6_value(const uint8_t *b, int p, int *scale_index) {
    const uint8_t *ql = b, *qh = b + 128;
    const int half = p / 128, r = p % 128, quarter = r / 32, l = r % 32;
    const uint8_t lo_byte = ql[64 * half + l + (quarter & 1) * 32];
    const int lo = (quarter < 2) ? (lo_byte & 0xF) : (lo_byte >> 4);
    const int hi = (qh[32 * half + l] >> (2 * quarter)) & 3;
    *scale_index = 8 * half + l / 16 + 2 * quarter;
    return (lo | (hi << 4)) - 32;
}

/* Q6_K: y = (d*sc)*q. */
void or_dequant_q6_k(const uint8_t *b, float *y) {
    const float d = or_fp16_to_f32(rd16(b + 208));
    const int8_t *sc = (const int8_t *)(b + 192);
    for (int p = 0; p < 256; ++p) {
        int is;
        const int q = q6_value(b, p, &is);
        y[p] = d * (float)sc[is] * (float)q;
    }
}

static void dequant_block(uint32_t kind, const uint8_t *b, float *y) {
    if (kind == 4) or_dequant_q4_k(b, y);
    else if (kind == 5) or_dequant_q5_k(b, y);
    else or_dequant_q6_k(b, y);
}

int or_dequant_rows(uint32_t kind, const uint8_t *blocks, size_t k, size_t n, float *out) {
    const size_t bb = or_block_bytes(kind);
    if (!bb || k % OR_QK_K) return OR_INVALID;
    const size_t nb = k / OR_QK_K;
    for (size_t i = 0; i < n * nb; ++i) dequant_block(kind, blocks + i * bb, out + i * OR_QK_K);
    return OR_OK;
}

/* (value / scale).round().clamp(-127, 127) as i8 — Rust's round() is half
 * away from zero (roundf), and `NaN as i8` is 0. */
static int8_t quant_one(float v, float scale) {
    float r = roundf(v / scale);
    if (r != r) return 0;
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)r;
}

/* crates/rocknpu-capi/src/lib.rs:614-654 (quantize_symmetric_into). */
int or_quantize_symmetric_row(const float *x, size_t k, int8_t *q, float *scale) {
    float max_abs = 0.0f;
    for (size_t i = 0; i < k; ++i) {
        if (!isfinite(x[i])) return OR_INVALID;
        const float a = fabsf(x[i]);
        if (a > max_abs) max_abs = a;
    }
    const float s = (max_abs == 0.0f) ? 1.0f : max_abs / 127.0f;
    for (size_t i = 0; i < k; ++i) q[i] = quant_one(x[i], s);
    *scale = s;
    return OR_OK;
}

/* The aarch64 NEON form of the same quantisation, the reference's default on
 * RK3588 (ROCKNPU_HOST_NEON defaults to the CPU's NEON support, lib.rs:
 * 300-311): quantize_symmetric_neon_into (lib.rs:509-541) multiplies by the
 * f32 reciprocal of the scale in chunks of 8 values, and divides only for the
 * tail of fewer than 8; max_abs_finite_neon (:475-505) is order-free, so the
 * scale is the scalar one. */
int or_quantize_symmetric_row_neon(const float *x, size_t k, int8_t *q, float *scale) {
    float max_abs = 0.0f;
    for (size_t i = 0; i < k; ++i) {
        if (!isfinite(x[i])) return OR_INVALID;
        const float a = fabsf(x[i]);
        if (a > max_abs) max_abs = a;
    }
    const float s = (max_abs == 0.0f) ? 1.0f : max_abs / 127.0f;
    const float inv = 1.0f / s;
    const size_t body = k - k % 8;
    for (size_t i = 0; i < body; ++i) {
        float r = roundf(x[i] * inv);
        if (r < -127.0f) r = -127.0f;
        if (r > 127.0f) r = 127.0f;
        q[i] = (int8_t)r;
    }
    for (size_t i = body; i < k; ++i) q[i] = quant_one(x[i], s);
    *scale = s;
    return OR_OK;
}

/* crates/rocknpu-capi/src/lib.rs:711-757 (Q4_K), :759-806 (Q5_K),
 * :974-994 (Q6_K): dequantise a row, then quantise it symmetrically. */
int or_repack_w8(uint32_t kind, const uint8_t *blocks, size_t bytes, size_t k, size_t n,
                 int8_t *w8, float *scales) {
    const size_t bb = or_block_bytes(kind);
    if (!bb || k == 0 || k % OR_QK_K || bytes != n * (k / OR_QK_K) * bb) return OR_INVALID;
    const size_t nb = k / OR_QK_K;
    int status = OR_OK;
    float *row = (float *)malloc(k * sizeof(float));
    if (!row) return OR_INVALID;
    for (size_t r = 0; r < n && status == OR_OK; ++r) {
        for (size_t b = 0; b < nb; ++b)
            dequant_block(kind, blocks + (r * nb + b) * bb, row + b * OR_QK_K);
        status = or_quantize_symmetric_row(row, k, w8 + r * k, &scales[r]);
    }
    free(row);
    return status;
}

/* lib.rs:1776-1791: each activation row quantised on its own, the int8 row
 * zero-padded to k_pad. */
int or_quantize_a8(const float *a, size_t m, size_t k, size_t k_pad, int8_t *a8, float *scales) {
    if (k_pad < k) return OR_INVALID;
    for (size_t r = 0; r < m; ++r) {
        memset(a8 + r * k_pad, 0, k_pad);
        if (or_quantize_symmetric_row(a + r * k, k, a8 + r * k_pad, &scales[r]) != OR_OK)
            return OR_INVALID;
    }
    return OR_OK;
}

/* lib.rs:2045-2071 (hilo_stack): the rows, then per row the residual
 * `x - f32::from(q) * scale` of its symmetric quantisation, evaluated as a
 * product rounded to f32 and then a difference (no contraction). */
int or_hilo_stack(const float *a, size_t m, size_t k, float *stacked) {
    int8_t *q = (int8_t *)malloc(k ? k : 1);
    if (!q) return OR_INVALID;
    int status = OR_OK;
    memcpy(stacked, a, m * k * sizeof(float));
    for (size_t r = 0; r < m && status == OR_OK; ++r) {
        float scale;
        if (or_quantize_symmetric_row(a + r * k, k, q, &scale) != OR_OK) {
            status = OR_INVALID;
            break;
        }
        for (size_t t = 0; t < k; ++t) {
            const float deq = (float)q[t] * scale;
            stacked[(m + r) * k + t] = a[r * k + t] - deq;
        }
    }
    free(q);
    return status;
}

/* lib.rs:2073-2082 (hilo_sum). */
void or_hilo_sum(float *out, const float *stacked, size_t len) {
    for (size_t i = 0; i < len; ++i) out[i] = stacked[i] + stacked[len + i];
}

uint64_t or_fnv1a64(uint64_t h, const uint8_t *data, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        h ^= data[i];
        h *= 1099511628211ULL;
    }
    return h;
}

/* ggml-rocknpu.cpp:123-146 */
uint64_t or_source_fingerprint(const uint8_t *data, size_t bytes) {
    uint8_t count[8];
    for (int i = 0; i < 8; ++i) count[i] = (uint8_t)((uint64_t)bytes >> (8 * i));
    uint64_t h = or_fnv1a64(14695981039346656037ULL, count, 8);
    const size_t sample = 4096;
    if (bytes <= 3 * sample) return or_fnv1a64(h, data, bytes);
    h = or_fnv1a64(h, data, sample);
    h = or_fnv1a64(h, data + (bytes - sample) / 2, sample);
    return or_fnv1a64(h, data + bytes - sample, sample);
}

void or_gemm_i32(const int8_t *a8, const int8_t *w8, size_t m, size_t n, size_t k, int32_t *c,
                 int threads) {
    const long long total = (long long)(m * n);
#pragma omp parallel for schedule(static) num_threads(threads > 1 ? threads : 1) if (threads > 1)
    for (long long idx = 0; idx < total; ++idx) {
        const size_t i = (size_t)idx / n, j = (size_t)idx % n;
        const int8_t *ar = a8 + i * k, *wr = w8 + j * k;
        int32_t acc = 0;
        for (size_t t = 0; t < k; ++t) acc += (int32_t)ar[t] * (int32_t)wr[t];
        c[idx] = acc;
    }
}

/* lib.rs:706-708: `value as f32 * activation_scale * weight_scale`. */
void or_rescale(const int32_t *c, const float *a_scales, const float *w_scales, size_t m, size_t n,
                float *out) {
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) {
            const float t = (float)c[i * n + j] * a_scales[i];
            out[i * n + j] = t * w_scales[j];
        }
}

/* rescale_i32_row_neon (lib.rs:664-690), the aarch64 default for prompt
 * rows: (f32(c) * w_scale) * a_scale in chunks of 4 columns of the slice,
 * the tail of fewer than 4 as the scalar (f32(c) * a_scale) * w_scale. */
void or_rescale_neon(const int32_t *c, const float *a_scales, const float *w_scales, size_t m, size_t n,
                     float *out) {
    const size_t body = n - n % 4;
    for (size_t i = 0; i < m; ++i) {
        for (size_t j = 0; j < body; ++j) {
            const float t = (float)c[i * n + j] * w_scales[j];
            out[i * n + j] = t * a_scales[i];
        }
        for (size_t j = body; j < n; ++j) {
            const float t = (float)c[i * n + j] * a_scales[i];
            out[i * n + j] = t * w_scales[j];
        }
    }
}

int or_matmul_q_w8a8(uint32_t kind, const uint8_t *blocks, size_t bytes, const float *a, size_t m,
                     size_t k, size_t n, float *out, int threads) {
    int status = OR_INVALID;
    int8_t *w8 = (int8_t *)malloc(n * k), *a8 = (int8_t *)malloc(m * k);
    float *ws = (float *)malloc(n * sizeof(float)), *as = (float *)malloc(m * sizeof(float));
    int32_t *c = (int32_t *)malloc(m * n * sizeof(int32_t));
    if (w8 && a8 && ws && as && c && or_repack_w8(kind, blocks, bytes, k, n, w8, ws) == OR_OK &&
        or_quantize_a8(a, m, k, k, a8, as) == OR_OK) {
        or_gemm_i32(a8, w8, m, n, k, c, threads);
        or_rescale(c, as, ws, m, n, out);
        status = OR_OK;
    }
    free(w8);
    free(a8);
    free(ws);
    free(as);
    free(c);
    return status;
}

/* ggml quantize_row_q8_K_ref: per 256-block, the first value of largest
 * magnitude sets iscale = -127/max; q = min(127, round-half-even(iscale*x));
 * bsums = sums of 16; d = 1/iscale. An all-zero block stores d = 0 and zero
 * quants (ggml leaves its bsums unwritten; they are zeroed here). */
void or_quantize_row_q8_k(const float *x, size_t k, uint8_t *q8k) {
    for (size_t i = 0; i < k / OR_QK_K; ++i) {
        const float *xb = x + i * OR_QK_K;
        uint8_t *yb = q8k + i * OR_Q8_K_BYTES;
        int8_t *qs = (int8_t *)(yb + 4);
        int16_t bsums[16];
        float mx = 0.0f, amax = 0.0f;
        for (int j = 0; j < OR_QK_K; ++j) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) {
                amax = ax;
                mx = xb[j];
            }
        }
        float d = 0.0f;
        if (amax == 0.0f) {
            memset(qs, 0, OR_QK_K);
            memset(bsums, 0, sizeof bsums);
        } else {
            const float iscale = -127.0f / mx;
            for (int j = 0; j < OR_QK_K; ++j) {
                const float p = iscale * xb[j];
                int v = (int)rintf(p); /* == ggml nearest_int for |p| < 2^22 */
                qs[j] = (int8_t)(v < 127 ? v : 127);
            }
            for (int j = 0; j < 16; ++j) {
                int s = 0;
                for (int t = 0; t < 16; ++t) s += qs[16 * j + t];
                bsums[j] = (int16_t)s;
            }
            d = 1.0f / iscale;
        }
        memcpy(yb, &d, 4);
        memcpy(yb + 260, bsums, sizeof bsums);
    }
}

static void q8k_parts(const uint8_t *yb, float *d, const int8_t **qs, int16_t bsums[16]) {
    memcpy(d, yb, 4);
    *qs = (const int8_t *)(yb + 4);
    memcpy(bsums, yb + 260, 32);
}

/* Integer part of one Q4_K x Q8_K block in ggml's generic 8-lane order:
 * aux32[l] collects positions p with p % 8 == l; sumi is the mins term. */
static void q4k_block_ints(const uint8_t *x, const uint8_t *yb, int32_t aux32[8], int32_t *sumi) {
    float yd;
    const int8_t *q8;
    int16_t bsums[16];
    q8k_parts(yb, &yd, &q8, bsums);
    const uint8_t *scales = x + 4, *qs = x + 16;
    int8_t a[256];
    for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) {
            a[64 * j + l] = (int8_t)(qs[32 * j + l] & 0xF);
            a[64 * j + 32 + l] = (int8_t)(qs[32 * j + l] >> 4);
        }
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) scale_min_k4(j, scales, &sc[j], &mn[j]);
    int32_t s = 0;
    for (int j = 0; j < 16; ++j) s += (int32_t)bsums[j] * (int32_t)mn[j / 2];
    *sumi = s;
    memset(aux32, 0, 8 * sizeof(int32_t));
    for (int p = 0; p < 256; ++p) aux32[p % 8] += (int32_t)sc[p / 32] * ((int32_t)q8[p] * a[p]);
}

static void q6k_block_ints(const uint8_t *x, const uint8_t *yb, int32_t aux32[8]) {
    float yd;
    const int8_t *q8;
    int16_t bsums[16];
    q8k_parts(yb, &yd, &q8, bsums);
    const int8_t *sc = (const int8_t *)(x + 192);
    memset(aux32, 0, 8 * sizeof(int32_t));
    for (int p = 0; p < 256; ++p) {
        int is;
        const int q = q6_value(x, p, &is);
        (void)is;
        aux32[p % 8] += (int32_t)sc[p / 16] * ((int32_t)q8[p] * q);
    }
}

/* ggml_vec_dot_q4_K_q8_K generic: sums[l] += d*aux32[l] per block,
 * sumf -= dmin*sumi per block, then sumf += sums[l]. */
float or_vec_dot_q4_k_q8_k(size_t k, const uint8_t *w, const uint8_t *y) {
    float sums[8] = {0}, sumf = 0.0f;
    for (size_t i = 0; i < k / OR_QK_K; ++i) {
        const uint8_t *x = w + i * OR_Q4_K_BYTES, *yb = y + i * OR_Q8_K_BYTES;
        int32_t aux32[8], sumi;
        q4k_block_ints(x, yb, aux32, &sumi);
        float yd;
        memcpy(&yd, yb, 4);
        const float d = or_fp16_to_f32(rd16(x)) * yd;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
        const float dmin = or_fp16_to_f32(rd16(x + 2)) * yd;
        sumf -= dmin * (float)sumi;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* ggml_vec_dot_q6_K_q8_K generic. */
float or_vec_dot_q6_k_q8_k(size_t k, const uint8_t *w, const uint8_t *y) {
    float sums[8] = {0}, sumf = 0.0f;
    for (size_t i = 0; i < k / OR_QK_K; ++i) {
        const uint8_t *x = w + i * OR_Q6_K_BYTES, *yb = y + i * OR_Q8_K_BYTES;
        int32_t aux32[8];
        q6k_block_ints(x, yb, aux32);
        float yd;
        memcpy(&yd, yb, 4);
        const float d = or_fp16_to_f32(rd16(x + 208)) * yd;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

int or_gemv_q8_k(uint32_t kind, const uint8_t *w, size_t k, size_t n, const uint8_t *q8k, size_t m,
                 float *out, int threads) {
    if ((kind != 4 && kind != 6) || k == 0 || k % OR_QK_K) return OR_INVALID;
    const size_t bb = or_block_bytes(kind), nb = k / OR_QK_K;
    const long long total = (long long)(m * n);
#pragma omp parallel for schedule(static) num_threads(threads > 1 ? threads : 1) if (threads > 1)
    for (long long idx = 0; idx < total; ++idx) {
        const size_t mi = (size_t)idx / n, ni = (size_t)idx % n;
        const uint8_t *row = w + ni * nb * bb, *y = q8k + mi * nb * OR_Q8_K_BYTES;
        out[idx] = kind == 4 ? or_vec_dot_q4_k_q8_k(k, row, y) : or_vec_dot_q6_k_q8_k(k, row, y);
    }
    return OR_OK;
}

int or_gemv_block_sums(uint32_t kind, const uint8_t *w, size_t k, size_t n, const uint8_t *y,
                       int32_t *isum, int32_t *msum, double *mag) {
    if ((kind != 4 && kind != 6) || k == 0 || k % OR_QK_K) return OR_INVALID;
    const size_t bb = or_block_bytes(kind), nb = k / OR_QK_K;
    for (size_t r = 0; r < n; ++r) {
        double total = 0.0;
        for (size_t b = 0; b < nb; ++b) {
            const uint8_t *x = w + (r * nb + b) * bb, *yb = y + b * OR_Q8_K_BYTES;
            int32_t aux32[8], sumi = 0, s = 0;
            if (kind == 4) q4k_block_ints(x, yb, aux32, &sumi);
            else q6k_block_ints(x, yb, aux32);
            float yd;
            memcpy(&yd, yb, 4);
            const double d = (double)or_fp16_to_f32(rd16(kind == 4 ? x : x + 208)) * yd;
            for (int l = 0; l < 8; ++l) {
                s += aux32[l];
                total += fabs(d * aux32[l]);  /* the generic dot rounds each d*aux32[l] */
            }
            isum[r * nb + b] = s;
            msum[r * nb + b] = sumi;
            if (kind == 4) total += fabs((double)or_fp16_to_f32(rd16(x + 2)) * yd * sumi);
        }
        mag[r] = total;
    }
    return OR_OK;
}
