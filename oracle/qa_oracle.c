/*
 * qa_oracle.c -- CPU restatement of the Qwen3-ASR text-decoder KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load this library; the product never links or calls it.
 * Every function names the reference lines (andimarafioti/qwenasr.cpp) it follows; the header
 * lists the [ggml-sem] conversion points and what is left unpinned.
 *
 * Build: see oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off; the f32 dot kernels use explicit
 * AVX2 FMA intrinsics so their rounding does not depend on contraction flags).
 */
#include "qa_oracle.h"

#include <float.h>
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ f16 <-> f32 (IEEE binary16)
 * ggml_cpy f32 -> f16 [ggml-sem]: round to nearest, ties to even; overflow -> inf; NaN kept NaN. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
    }
    if (ax >= 0x477ff000u) {                       /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) {                        /* below 2^-14: subnormal or zero */
        float a;
        memcpy(&a, &ax, 4);
        const float units = a * 16777216.0f;       /* exact: |x| / 2^-24 */
        const uint32_t r = (uint32_t)nearbyintf(units);   /* default mode: ties to even */
        return (uint16_t)(sign | r);
    }
    uint32_t h = ((((ax >> 23) - 127u + 15u) & 0x1fu) << 10) | ((ax >> 13) & 0x3ffu);
    const uint32_t rest = ax & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) {
        h += 1u;                                   /* carries into the exponent when needed */
    }
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            float v = (float)m * (1.0f / 16777216.0f);   /* exact */
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

void orc_f32_to_f16_array(const float * x, uint16_t * h, size_t n) {
    for (size_t i = 0; i < n; ++i) h[i] = orc_f32_to_f16(x[i]);
}

/* Every f16 bit pattern's f32 value (the conversion is exact), filled once at load time. */
static float f16_table[65536];

__attribute__((constructor)) static void fill_f16_table(void) {
    for (uint32_t b = 0; b < 65536u; ++b) f16_table[b] = orc_f16_to_f32((uint16_t)b);
}

void orc_f16_to_f32_array(const uint16_t * h, float * x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = f16_table[h[i]];
}

static inline float round_f16(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

int orc_set_threads(int32_t n) {
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
}

/* ------------------------------------------------------------------ RMSNorm
 * rms_norm_row, src/text-decoder.cpp:542-557: mean of squares accumulated in double (double
 * products), scale = 1.0f / sqrt(float(mean) + eps) in float, y = (x * scale) * w.             */
void orc_rms_norm_row(const float * x, int32_t n, const float * w, float eps, float * y) {
    double ms = 0.0;
    for (int32_t i = 0; i < n; ++i) ms += (double)x[i] * (double)x[i];
    ms /= (double)n;
    const float scale = 1.0f / sqrtf((float)ms + eps);
    for (int32_t i = 0; i < n; ++i) y[i] = x[i] * scale * w[i];
}

/* ------------------------------------------------------------------ RoPE (NEOX)
 * apply_rope_position, src/text-decoder.cpp:604-625: for pair i < d/2,
 * inv_freq = exp(-ln(theta) * 2i / d) and angle = pos * inv_freq in double, c/s rounded to float,
 * (a, b) = (row[i], row[i + d/2]) -> (a*c - b*s, b*c + a*s) in float without contraction.      */
void orc_rope_rows(float * rows, int32_t position, int32_t n_heads, int32_t head_dim, float theta) {
    const int32_t half = head_dim / 2;
    const double log_theta = log((double)theta);
    for (int32_t i = 0; i < half; ++i) {
        const double inv_freq = exp(-log_theta * (double)(2 * i) / (double)head_dim);
        const double angle = (double)position * inv_freq;
        const float c = (float)cos(angle);
        const float s = (float)sin(angle);
        for (int32_t h = 0; h < n_heads; ++h) {
            float * row = rows + (size_t)h * head_dim;
            const float a = row[i];
            const float b = row[half + i];
            row[i] = a * c - b * s;
            row[half + i] = b * c + a * s;
        }
    }
}

/* ------------------------------------------------------------------ bookkeeping
 * Slot of (head, pos, dim) in one layer's K or V tensor ne = [d, max_seq, n_kv]
 * (text-decoder.cpp:1451-1462): (head * max_seq + pos) * d + dim.                              */
int64_t orc_slot_index(int32_t head, int32_t pos, int32_t dim, int32_t max_seq, int32_t head_dim) {
    return ((int64_t)head * max_seq + pos) * head_dim + dim;
}

/* positions (text-decoder.cpp:1724-1727) and dense mask (1729-1735). */
void orc_positions(int32_t n_past, int32_t n_tokens, int32_t * out) {
    for (int32_t i = 0; i < n_tokens; ++i) out[i] = n_past + i;
}

void orc_causal_mask(int32_t n_past, int32_t n_tokens, float * mask) {
    const int32_t full = n_past + n_tokens;
    for (int32_t q = 0; q < n_tokens; ++q) {
        for (int32_t k = 0; k < full; ++k) {
            mask[(size_t)q * full + k] = (k <= n_past + q) ? 0.0f : -INFINITY;
        }
    }
}

/* ------------------------------------------------------------------ linear
 * linear / linear_row, src/text-decoder.cpp:561-600 (and linear_ggml 83-90 with PREC_F32):
 * y[r][o] = sum_i x[r][i] * w[o][i].  Order used here: 8 lanes, lane k accumulates i = k mod 8 with
 * FMA in increasing i, then ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)).  Each (r, o) result depends only
 * on its own row pair, never on blocking or thread count.                                       */
static inline float hsum8(__m256 v) {
    const __m128 lo = _mm256_castps256_ps128(v);
    const __m128 hi = _mm256_extractf128_ps(v, 1);
    const __m128 s4 = _mm_add_ps(lo, hi);                       /* l0+l4, l1+l5, l2+l6, l3+l7 */
    const __m128 s2 = _mm_add_ps(s4, _mm_movehl_ps(s4, s4));    /* (l0+l4)+(l2+l6), (l1+l5)+(l3+l7) */
    const __m128 s1 = _mm_add_ss(s2, _mm_shuffle_ps(s2, s2, 1));
    return _mm_cvtss_f32(s1);
}

static float dot_scalar_order(const float * a, const float * b, int32_t n) {
    /* Same order as the vector kernel, for in_dim not a multiple of 8. */
    float l[8] = {0};
    int32_t i = 0;
    for (; i + 8 <= n; i += 8) {
        for (int k = 0; k < 8; ++k) l[k] = fmaf(a[i + k], b[i + k], l[k]);
    }
    for (int k = 0; i + k < n; ++k) l[k] = fmaf(a[i + k], b[i + k], l[k]);
    const float s0 = (l[0] + l[4]) + (l[2] + l[6]);
    const float s1 = (l[1] + l[5]) + (l[3] + l[7]);
    return s0 + s1;
}

/* 4 weight rows x 3 token rows micro-kernel. */
static void mk_4x3(const float * x0, const float * x1, const float * x2,
                   const float * w0, const float * w1, const float * w2, const float * w3,
                   int32_t n, float out[4][3]) {
    __m256 a00 = _mm256_setzero_ps(), a01 = a00, a02 = a00, a10 = a00, a11 = a00, a12 = a00;
    __m256 a20 = a00, a21 = a00, a22 = a00, a30 = a00, a31 = a00, a32 = a00;
    for (int32_t i = 0; i < n; i += 8) {
        const __m256 v0 = _mm256_loadu_ps(x0 + i);
        const __m256 v1 = _mm256_loadu_ps(x1 + i);
        const __m256 v2 = _mm256_loadu_ps(x2 + i);
        __m256 w = _mm256_loadu_ps(w0 + i);
        a00 = _mm256_fmadd_ps(v0, w, a00); a01 = _mm256_fmadd_ps(v1, w, a01); a02 = _mm256_fmadd_ps(v2, w, a02);
        w = _mm256_loadu_ps(w1 + i);
        a10 = _mm256_fmadd_ps(v0, w, a10); a11 = _mm256_fmadd_ps(v1, w, a11); a12 = _mm256_fmadd_ps(v2, w, a12);
        w = _mm256_loadu_ps(w2 + i);
        a20 = _mm256_fmadd_ps(v0, w, a20); a21 = _mm256_fmadd_ps(v1, w, a21); a22 = _mm256_fmadd_ps(v2, w, a22);
        w = _mm256_loadu_ps(w3 + i);
        a30 = _mm256_fmadd_ps(v0, w, a30); a31 = _mm256_fmadd_ps(v1, w, a31); a32 = _mm256_fmadd_ps(v2, w, a32);
    }
    out[0][0] = hsum8(a00); out[0][1] = hsum8(a01); out[0][2] = hsum8(a02);
    out[1][0] = hsum8(a10); out[1][1] = hsum8(a11); out[1][2] = hsum8(a12);
    out[2][0] = hsum8(a20); out[2][1] = hsum8(a21); out[2][2] = hsum8(a22);
    out[3][0] = hsum8(a30); out[3][1] = hsum8(a31); out[3][2] = hsum8(a32);
}

void orc_linear(const float * x, int32_t rows, int32_t in_dim, const float * w, int32_t out_dim, float * y) {
    if (in_dim % 8 != 0) {
#pragma omp parallel for schedule(static)
        for (int64_t ro = 0; ro < (int64_t)rows * out_dim; ++ro) {
            const int64_t r = ro / out_dim, o = ro % out_dim;
            y[ro] = dot_scalar_order(x + r * in_dim, w + o * (int64_t)in_dim, in_dim);
        }
        return;
    }
    const int32_t OB = 64, TB = 48;
    const int32_t n_ob = (out_dim + OB - 1) / OB;
    const int32_t n_tb = (rows + TB - 1) / TB;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int32_t ob = 0; ob < n_ob; ++ob) {
        for (int32_t tb = 0; tb < n_tb; ++tb) {
            const int32_t o_end = (ob + 1) * OB < out_dim ? (ob + 1) * OB : out_dim;
            const int32_t t_end = (tb + 1) * TB < rows ? (tb + 1) * TB : rows;
            for (int32_t o = ob * OB; o < o_end; o += 4) {
                const float * wr[4];
                for (int k = 0; k < 4; ++k) {
                    const int32_t oo = o + k < o_end ? o + k : o_end - 1;
                    wr[k] = w + (int64_t)oo * in_dim;
                }
                for (int32_t t = tb * TB; t < t_end; t += 3) {
                    const float * xr[3];
                    for (int k = 0; k < 3; ++k) {
                        const int32_t tt = t + k < t_end ? t + k : t_end - 1;
                        xr[k] = x + (int64_t)tt * in_dim;
                    }
                    float out[4][3];
                    mk_4x3(xr[0], xr[1], xr[2], wr[0], wr[1], wr[2], wr[3], in_dim, out);
                    for (int a = 0; a < 4 && o + a < o_end; ++a) {
                        for (int b = 0; b < 3 && t + b < t_end; ++b) {
                            y[(int64_t)(t + b) * out_dim + o + a] = out[a][b];
                        }
                    }
                }
            }
        }
    }
}

/* Greedy pick, src/text-decoder.cpp:2266-2274: strict '>' from -inf, so the first maximum wins
 * and NaN never wins; -1 when nothing beats -inf. */
int32_t orc_argmax(const float * logits, int32_t n) {
    int32_t best_id = -1;
    float best = -INFINITY;
    for (int32_t i = 0; i < n; ++i) {
        if (logits[i] > best) {
            best = logits[i];
            best_id = i;
        }
    }
    return best_id;
}

/* Gap between the greedy pick and the runner-up (the first index of the largest other logit). */
static float top2_margin(const float * logits, int32_t n, int32_t best_id, int32_t * second_id) {
    *second_id = -1;
    if (best_id < 0) return 0.0f;
    float second = -INFINITY;
    for (int32_t i = 0; i < n; ++i) {
        if (i != best_id && logits[i] > second) {
            second = logits[i];
            *second_id = i;
        }
    }
    return logits[best_id] - second;
}

/* ------------------------------------------------------------------ q/k preparation
 * text-decoder.cpp:377-408 (graph) / 694-717 and 1007-1024 (scalar): per-head RMSNorm with the
 * q_norm / k_norm weights, then NEOX RoPE at position pos0 + t.                                */
void orc_qk_prep(float * q, float * k, int32_t n_tokens, int32_t n_heads, int32_t n_kv_heads,
                 int32_t head_dim, const float * q_norm_w, const float * k_norm_w, int32_t pos0,
                 float theta, float eps) {
#pragma omp parallel for schedule(static)
    for (int32_t t = 0; t < n_tokens; ++t) {
        float tmp[512];
        float * qt = q + (size_t)t * n_heads * head_dim;
        float * kt = k + (size_t)t * n_kv_heads * head_dim;
        for (int32_t h = 0; h < n_heads; ++h) {
            orc_rms_norm_row(qt + (size_t)h * head_dim, head_dim, q_norm_w, eps, tmp);
            memcpy(qt + (size_t)h * head_dim, tmp, sizeof(float) * head_dim);
        }
        for (int32_t h = 0; h < n_kv_heads; ++h) {
            orc_rms_norm_row(kt + (size_t)h * head_dim, head_dim, k_norm_w, eps, tmp);
            memcpy(kt + (size_t)h * head_dim, tmp, sizeof(float) * head_dim);
        }
        orc_rope_rows(qt, pos0 + t, n_heads, head_dim, theta);
        orc_rope_rows(kt, pos0 + t, n_kv_heads, head_dim, theta);
    }
}

/* ------------------------------------------------------------------ cache write
 * ggml_cpy of cont(permute(k)) / cont(permute(v)) into the cache view at row n_past
 * (text-decoder.cpp:410-433): token t, head h -> slot (h, n_past + t); f16 caches round to
 * nearest even [ggml-sem].                                                                      */
static size_t layer_elems(const orc_cache * c) {
    return (size_t)c->n_kv_heads * c->max_seq * c->head_dim;
}

void orc_cache_write(orc_cache * cache, int32_t layer, const float * k, const float * v,
                     int32_t n_past, int32_t n_tokens) {
    const int32_t d = cache->head_dim;
    const size_t base = (size_t)layer * layer_elems(cache);
    for (int32_t t = 0; t < n_tokens; ++t) {
        for (int32_t h = 0; h < cache->n_kv_heads; ++h) {
            const float * ks = k + ((size_t)t * cache->n_kv_heads + h) * d;
            const float * vs = v + ((size_t)t * cache->n_kv_heads + h) * d;
            const size_t slot = base + (size_t)orc_slot_index(h, n_past + t, 0, cache->max_seq, d);
            if (cache->dtype == 1) {
                orc_f32_to_f16_array(ks, (uint16_t *)cache->k + slot, (size_t)d);
                orc_f32_to_f16_array(vs, (uint16_t *)cache->v + slot, (size_t)d);
            } else {
                memcpy((float *)cache->k + slot, ks, sizeof(float) * d);
                memcpy((float *)cache->v + slot, vs, sizeof(float) * d);
            }
        }
    }
}

/* ------------------------------------------------------------------ attention core
 * One query row against keys [0, n_keys): the GGML graph of text-decoder.cpp:454-461 --
 * scores = mul_mat(K, q) (q rounded to f16 first when K is f16 [ggml-sem]), soft_max_ext with
 * scale (x * scale, max, expf(x - max), sum in double, times (float)(1/sum)) [ggml-sem], then
 * mul_mat(V^T, p) (p rounded to f16 first when V is f16 [ggml-sem]).  Keys past the causal limit
 * carry a -inf mask in the reference and contribute exact zeros, so they are simply not visited. */
static float dot_fixed(const float * a, const float * b, int32_t n) {
    float l[8] = {0};
    for (int32_t i = 0; i < n; i += 8) {
        for (int k = 0; k < 8; ++k) l[k] = fmaf(a[i + k], b[i + k], l[k]);
    }
    return ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
}

/* ORC_PLANT is a test hook for the negative controls of tests/test_oracle.py, which build copies of
 * this file with a planted mistake and check that the attention pin rejects them: 1 rounds p to f16
 * before the normalisation, 2 leaves q unrounded.  The library itself is always built with 0. */
#ifndef ORC_PLANT
#define ORC_PLANT 0
#endif

static void attend_row(const float * q, const float * kf, const float * vf, size_t row_stride,
                       int32_t n_keys, int32_t head_dim, float scale, int round16, float * scores,
                       float * out) {
    float qq[512];
    for (int32_t d = 0; d < head_dim; ++d) qq[d] = (round16 && ORC_PLANT != 2) ? round_f16(q[d]) : q[d];
    float mx = -INFINITY;
    for (int32_t j = 0; j < n_keys; ++j) {
        const float s = dot_fixed(qq, kf + (size_t)j * row_stride, head_dim) * scale;
        scores[j] = s;
        if (s > mx) mx = s;
    }
    double sum = 0.0;
    for (int32_t j = 0; j < n_keys; ++j) {
        const float e = expf(scores[j] - mx);
        scores[j] = e;
        sum += (double)e;
    }
    const float r = (float)(1.0 / sum);
    for (int32_t d = 0; d < head_dim; ++d) out[d] = 0.0f;
    for (int32_t j = 0; j < n_keys; ++j) {
        float p = scores[j] * r;
        if (round16) p = ORC_PLANT == 1 ? round_f16(scores[j]) * r : round_f16(p);
        const float * vr = vf + (size_t)j * row_stride;
        for (int32_t d = 0; d < head_dim; ++d) out[d] = fmaf(p, vr[d], out[d]);
    }
}

void orc_cache_attention(const orc_cache * cache, int32_t layer, const float * q, int32_t n_past,
                         int32_t n_tokens, int32_t n_heads, float scale, float * out) {
    const int32_t d = cache->head_dim;
    const int32_t n_kv = cache->n_kv_heads;
    const int32_t full = n_past + n_tokens;
    const int32_t rep = n_heads / n_kv;
    const size_t base = (size_t)layer * layer_elems(cache);
    /* f32 copies of rows [0, full) of every head: [head][pos][d] */
    float * kf = (float *)malloc(sizeof(float) * (size_t)n_kv * full * d);
    float * vf = (float *)malloc(sizeof(float) * (size_t)n_kv * full * d);
    /* exact widening of the stored rows, in parallel blocks of 64 positions per head */
    const int32_t n_blk = (full + 63) / 64;
#pragma omp parallel for collapse(2) schedule(static)
    for (int32_t h = 0; h < n_kv; ++h) {
        for (int32_t b = 0; b < n_blk; ++b) {
            const int32_t p0 = b * 64, np = full - p0 < 64 ? full - p0 : 64;
            const size_t src = base + (size_t)orc_slot_index(h, p0, 0, cache->max_seq, d);
            const size_t dst = ((size_t)h * full + p0) * d;
            if (cache->dtype == 1) {
                orc_f16_to_f32_array((const uint16_t *)cache->k + src, kf + dst, (size_t)np * d);
                orc_f16_to_f32_array((const uint16_t *)cache->v + src, vf + dst, (size_t)np * d);
            } else {
                memcpy(kf + dst, (const float *)cache->k + src, sizeof(float) * (size_t)np * d);
                memcpy(vf + dst, (const float *)cache->v + src, sizeof(float) * (size_t)np * d);
            }
        }
    }
    const int round16 = cache->dtype == 1;
#pragma omp parallel
    {
        float * scores = (float *)malloc(sizeof(float) * (size_t)full);
#pragma omp for collapse(2) schedule(dynamic, 4)
        for (int32_t t = 0; t < n_tokens; ++t) {
            for (int32_t h = 0; h < n_heads; ++h) {
                const int32_t kvh = h / rep;
                attend_row(q + ((size_t)t * n_heads + h) * d, kf + (size_t)kvh * full * d,
                           vf + (size_t)kvh * full * d, (size_t)d, n_past + t + 1, d, scale, round16,
                           scores, out + ((size_t)t * n_heads + h) * d);
            }
        }
        free(scores);
    }
    free(kf);
    free(vf);
}

/* Non-cached causal attention (text-decoder.cpp:320-334): f32 K/V, ggml_diag_mask_inf(., 0). */
void orc_causal_attention_f32(const float * q, const float * k, const float * v, int32_t n_tokens,
                              int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, float scale,
                              float * out) {
    const int32_t rep = n_heads / n_kv_heads;
    const size_t stride = (size_t)n_kv_heads * head_dim;
#pragma omp parallel
    {
        float * scores = (float *)malloc(sizeof(float) * (size_t)n_tokens);
#pragma omp for collapse(2) schedule(dynamic, 4)
        for (int32_t t = 0; t < n_tokens; ++t) {
            for (int32_t h = 0; h < n_heads; ++h) {
                const int32_t kvh = h / rep;
                attend_row(q + ((size_t)t * n_heads + h) * head_dim, k + (size_t)kvh * head_dim,
                           v + (size_t)kvh * head_dim, stride, t + 1, head_dim, scale, 0, scores,
                           out + ((size_t)t * n_heads + h) * head_dim);
            }
        }
        free(scores);
    }
}

/* ------------------------------------------------------------------ layers */
static void rms_rows(const float * x, int32_t rows, int32_t dim, const float * w, float eps, float * y) {
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < rows; ++r) orc_rms_norm_row(x + (size_t)r * dim, dim, w, eps, y + (size_t)r * dim);
}

/* attention output -> o_proj + residual -> ffn_norm -> SwiGLU FFN + residual
 * (text-decoder.cpp:465-473 / scalar 778-806). silu(x) = x / (1 + expf(-x)) (scalar 602). */
static void layer_tail(const orc_model * m, int32_t layer, const float * x, const float * attn,
                       int32_t n_tokens, float * y) {
    const orc_config * c = &m->cfg;
    const orc_layer * L = &m->layers[layer];
    const int32_t H = c->hidden, I = c->intermediate, QD = c->n_heads * c->head_dim;
    float * proj = (float *)malloc(sizeof(float) * (size_t)n_tokens * H);
    float * hs = (float *)malloc(sizeof(float) * (size_t)n_tokens * H);
    float * nrm = (float *)malloc(sizeof(float) * (size_t)n_tokens * H);
    float * g = (float *)malloc(sizeof(float) * (size_t)n_tokens * I);
    float * u = (float *)malloc(sizeof(float) * (size_t)n_tokens * I);
    orc_linear(attn, n_tokens, QD, L->o, H, proj);
    for (size_t i = 0; i < (size_t)n_tokens * H; ++i) hs[i] = x[i] + proj[i];
    rms_rows(hs, n_tokens, H, L->ffn_norm, c->rms_norm_eps, nrm);
    orc_linear(nrm, n_tokens, H, L->gate, I, g);
    orc_linear(nrm, n_tokens, H, L->up, I, u);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n_tokens * I; ++i) {
        const float a = g[i];
        g[i] = (a / (1.0f + expf(-a))) * u[i];
    }
    orc_linear(g, n_tokens, I, L->down, H, proj);
    for (size_t i = 0; i < (size_t)n_tokens * H; ++i) y[i] = hs[i] + proj[i];
    free(proj); free(hs); free(nrm); free(g); free(u);
}

/* Cached layer, backend_text_layer_forward_cached_ggml (text-decoder.cpp:347-474): RMSNorm ->
 * q/k/v -> q_norm/k_norm -> RoPE at n_past + t -> cache write -> attention over [0, n_past + t]. */
int orc_layer_forward_cached(const orc_model * m, int32_t layer, const float * x, int32_t n_tokens,
                             int32_t n_past, orc_cache * cache, float * y) {
    const orc_config * c = &m->cfg;
    if (n_tokens <= 0 || n_past < 0 || n_past + n_tokens > cache->max_seq) return 2;
    const orc_layer * L = &m->layers[layer];
    const int32_t H = c->hidden, QD = c->n_heads * c->head_dim, KD = c->n_kv_heads * c->head_dim;
    float * nrm = (float *)malloc(sizeof(float) * (size_t)n_tokens * H);
    float * q = (float *)malloc(sizeof(float) * (size_t)n_tokens * QD);
    float * k = (float *)malloc(sizeof(float) * (size_t)n_tokens * KD);
    float * v = (float *)malloc(sizeof(float) * (size_t)n_tokens * KD);
    float * attn = (float *)malloc(sizeof(float) * (size_t)n_tokens * QD);
    rms_rows(x, n_tokens, H, L->attn_norm, c->rms_norm_eps, nrm);
    orc_linear(nrm, n_tokens, H, L->q, QD, q);
    orc_linear(nrm, n_tokens, H, L->k, KD, k);
    orc_linear(nrm, n_tokens, H, L->v, KD, v);
    orc_qk_prep(q, k, n_tokens, c->n_heads, c->n_kv_heads, c->head_dim, L->q_norm, L->k_norm, n_past,
                c->rope_theta, c->rms_norm_eps);
    orc_cache_write(cache, layer, k, v, n_past, n_tokens);
    orc_cache_attention(cache, layer, q, n_past, n_tokens, c->n_heads,
                        1.0f / sqrtf((float)c->head_dim), attn);
    layer_tail(m, layer, x, attn, n_tokens, y);
    free(nrm); free(q); free(k); free(v); free(attn);
    return 0;
}

/* Non-cached layer, backend_text_layer_forward_ggml (text-decoder.cpp:265-345), positions 0..T-1. */
int orc_layer_forward_nocache(const orc_model * m, int32_t layer, const float * x, int32_t n_tokens,
                              float * y) {
    const orc_config * c = &m->cfg;
    const orc_layer * L = &m->layers[layer];
    const int32_t H = c->hidden, QD = c->n_heads * c->head_dim, KD = c->n_kv_heads * c->head_dim;
    float * nrm = (float *)malloc(sizeof(float) * (size_t)n_tokens * H);
    float * q = (float *)malloc(sizeof(float) * (size_t)n_tokens * QD);
    float * k = (float *)malloc(sizeof(float) * (size_t)n_tokens * KD);
    float * v = (float *)malloc(sizeof(float) * (size_t)n_tokens * KD);
    float * attn = (float *)malloc(sizeof(float) * (size_t)n_tokens * QD);
    rms_rows(x, n_tokens, H, L->attn_norm, c->rms_norm_eps, nrm);
    orc_linear(nrm, n_tokens, H, L->q, QD, q);
    orc_linear(nrm, n_tokens, H, L->k, KD, k);
    orc_linear(nrm, n_tokens, H, L->v, KD, v);
    orc_qk_prep(q, k, n_tokens, c->n_heads, c->n_kv_heads, c->head_dim, L->q_norm, L->k_norm, 0,
                c->rope_theta, c->rms_norm_eps);
    orc_causal_attention_f32(q, k, v, n_tokens, c->n_heads, c->n_kv_heads, c->head_dim,
                             1.0f / sqrtf((float)c->head_dim), attn);
    layer_tail(m, layer, x, attn, n_tokens, y);
    free(nrm); free(q); free(k); free(v); free(attn);
    return 0;
}

/* Logits of one state row: backend_text_logits_ggml (text-decoder.cpp:476-493). */
int orc_logits(const orc_model * m, const float * state, float * logits) {
    const orc_config * c = &m->cfg;
    float * nrm = (float *)malloc(sizeof(float) * (size_t)c->hidden);
    orc_rms_norm_row(state, c->hidden, m->output_norm, c->rms_norm_eps, nrm);
    orc_linear(nrm, 1, c->hidden, m->output, c->vocab, logits);
    free(nrm);
    return 0;
}

/* text_decoder_backend_cached_logits (text-decoder.cpp:1641-1755): capacity check, 28 cached
 * layers, logits of the last token, cur_len = n_past + T. */
int orc_forward_cached(const orc_model * m, const float * x, int32_t n_tokens, int32_t n_past,
                       orc_cache * cache, float * logits) {
    const orc_config * c = &m->cfg;
    if (n_tokens <= 0 || n_past < 0 || n_past + n_tokens > cache->max_seq) return 2;
    const size_t n = (size_t)n_tokens * c->hidden;
    float * a = (float *)malloc(sizeof(float) * n);
    float * b = (float *)malloc(sizeof(float) * n);
    memcpy(a, x, sizeof(float) * n);
    for (int32_t l = 0; l < c->n_layers; ++l) {
        orc_layer_forward_cached(m, l, a, n_tokens, n_past, cache, b);
        float * t = a; a = b; b = t;
    }
    if (logits) orc_logits(m, a + (size_t)(n_tokens - 1) * c->hidden, logits);
    cache->cur_len = n_past + n_tokens;
    free(a);
    free(b);
    return 0;
}

/* qwenasr_text_generate_cached_backend (text-decoder.cpp:2209-2311). */
int orc_generate_cached(const orc_model * m, const float * x, int32_t n_tokens, int32_t max_new,
                        const int32_t * stop_ids, int32_t n_stop, orc_cache * cache,
                        int32_t * out_ids, int32_t * n_out, int32_t * stopped, int32_t * total_tokens,
                        float * margins, int32_t * runner_up) {
    const orc_config * c = &m->cfg;
    *n_out = 0;
    *stopped = 0;
    *total_tokens = n_tokens;
    if (max_new < 0) return 1;
    if (n_tokens + max_new > cache->max_seq) return 2;
    if (max_new == 0) return 0;
    float * logits = (float *)malloc(sizeof(float) * (size_t)c->vocab);
    cache->cur_len = 0;
    orc_forward_cached(m, x, n_tokens, 0, cache, logits);
    int rc = 0;
    for (int32_t step = 0; step < max_new; ++step) {
        const int32_t id = orc_argmax(logits, c->vocab);
        if (id < 0 || id >= c->vocab) { rc = 6; break; }
        int32_t second = -1;
        const float gap = top2_margin(logits, c->vocab, id, &second);
        if (margins) margins[step] = gap;
        if (runner_up) runner_up[step] = second;
        out_ids[(*n_out)++] = id;
        *total_tokens = n_tokens + *n_out;
        int stop = 0;
        for (int32_t s = 0; s < n_stop; ++s) stop |= (id == stop_ids[s]);
        if (stop) { *stopped = 1; break; }
        if (step + 1 >= max_new) break;
        orc_forward_cached(m, m->token_embd + (size_t)id * c->hidden, 1, cache->cur_len, cache, logits);
    }
    free(logits);
    return rc;
}

int orc_decode_steps(const orc_model * m, orc_cache * cache, int32_t first_id, int32_t n_steps,
                     int32_t * out_ids, float * margins, int32_t * runner_up) {
    const orc_config * c = &m->cfg;
    if (cache->cur_len + n_steps > cache->max_seq) return 2;
    float * logits = (float *)malloc(sizeof(float) * (size_t)c->vocab);
    int32_t id = first_id;
    int rc = 0;
    for (int32_t k = 0; k < n_steps; ++k) {
        if (id < 0 || id >= c->vocab) { rc = 6; break; }
        orc_forward_cached(m, m->token_embd + (size_t)id * c->hidden, 1, cache->cur_len, cache, logits);
        id = orc_argmax(logits, c->vocab);
        out_ids[k] = id;
        int32_t second = -1;
        const float gap = top2_margin(logits, c->vocab, id, &second);
        if (margins) margins[k] = gap;
        if (runner_up) runner_up[k] = second;
    }
    free(logits);
    return rc;
}
