/*
 * qora_oracle.c -- CPU oracle for the QORA-4B token-mixer path.
 *
 * TEST INFRASTRUCTURE ONLY (see qora_oracle.h).  A plain-C restatement of
 * the reference's CPU mixer functions; each function cites the Rust lines
 * it follows.  Built with -O2 -ffp-contract=off -fno-fast-math so every
 * f32 operation rounds exactly where the Rust source rounds.
 */
#include "qora_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>

/* ------------------------------------------------------------------ */
/* f16 / bf16 conversion (half 2.7.1: f16::to_f32 is exact)             */
/* ------------------------------------------------------------------ */
static float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return bits_to_f32(sign);
        /* subnormal: value = man * 2^-24 */
        float v = (float)man * 5.9604644775390625e-08f;
        return (sign ? -v : v);
    }
    if (exp == 31) return bits_to_f32(sign | 0x7f800000u | (man << 13));
    return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t or_f32_to_f16(float f) {
    uint32_t x = f32_to_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* overflow */
    if (ax < 0x38800000u) {                        /* result subnormal/0 */
        /* value / 2^-24, rounded to nearest even integer */
        float a = bits_to_f32(ax);
        float q = a * 16777216.0f;                 /* exact scaling */
        float r = nearbyintf(q);                   /* RNE (default mode) */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float or_bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

uint16_t or_f32_to_bf16(float f) {
    uint32_t x = f32_to_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

/* ------------------------------------------------------------------ */
/* scalar helpers, gemv.rs:565-659                                      */
/* ------------------------------------------------------------------ */

/* gemv.rs:631-633  x / (1 + exp(-x)) */
float or_silu(float x) { return x / (1.0f + expf(-x)); }

/* gemv.rs:637-639  x > 20 ? x : ln(1 + exp(x)) */
float or_softplus(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }

/* gemv.rs:643-649: norm = sqrt(sum x^2); scale by 1/norm only if > 1e-12 */
void or_l2_normalize(float* x, int32_t n) {
    float ss = 0.0f;
    for (int32_t i = 0; i < n; ++i) ss += x[i] * x[i];
    float norm = sqrtf(ss);
    if (norm > 1e-12f) {
        float inv = 1.0f / norm;
        for (int32_t i = 0; i < n; ++i) x[i] *= inv;
    }
}

/* gemv.rs:653-659: max-subtract, exp, multiply by 1/sum */
void or_softmax_raw(float* s, int32_t n) {
    float mx = -INFINITY;
    for (int32_t i = 0; i < n; ++i) mx = fmaxf(mx, s[i]);
    float sum = 0.0f;
    for (int32_t i = 0; i < n; ++i) { s[i] = expf(s[i] - mx); sum += s[i]; }
    float inv = 1.0f / sum;
    for (int32_t i = 0; i < n; ++i) s[i] *= inv;
}

/* gemv.rs:571-579: x * inv_rms * (1 + gamma), eps 1e-6 */
void or_rms_norm(const float* x, int32_t n, const uint16_t* gamma, float* out) {
    float ss = 0.0f;
    for (int32_t i = 0; i < n; ++i) ss += x[i] * x[i];
    float inv_rms = 1.0f / sqrtf(ss / (float)n + 1e-6f);
    for (int32_t i = 0; i < n; ++i)
        out[i] = x[i] * inv_rms * (1.0f + or_f16_to_f32(gamma[i]));
}

/* gemv.rs:586-597: per-head RMSNorm with shared (1 + gamma[head_dim]) */
void or_per_head_rms_norm(float* x, int32_t num_heads, int32_t head_dim,
                          const uint16_t* gamma) {
    for (int32_t h = 0; h < num_heads; ++h) {
        float* hx = x + (size_t)h * head_dim;
        float ss = 0.0f;
        for (int32_t d = 0; d < head_dim; ++d) ss += hx[d] * hx[d];
        float inv_rms = 1.0f / sqrtf(ss / (float)head_dim + 1e-6f);
        for (int32_t d = 0; d < head_dim; ++d)
            hx[d] = hx[d] * inv_rms * (1.0f + or_f16_to_f32(gamma[d]));
    }
}

/* gemv.rs:604-627: split-half RoPE on the first rotary_dim dims; pair
 * (i, i + rotary_dim/2); table row = position, rotary_dim/2 entries. */
void or_apply_partial_rope(float* data, int32_t num_heads, int32_t head_dim,
                           const float* cos_table, const float* sin_table,
                           int32_t rotary_dim, int32_t position) {
    int32_t half = rotary_dim / 2;
    size_t off = (size_t)position * (size_t)half;
    for (int32_t h = 0; h < num_heads; ++h) {
        float* b = data + (size_t)h * head_dim;
        for (int32_t i = 0; i < half; ++i) {
            float x1 = b[i], x2 = b[half + i];
            float c = cos_table[off + i], s = sin_table[off + i];
            b[i] = x1 * c - x2 * s;
            b[half + i] = x2 * c + x1 * s;
        }
    }
}

/* convert.rs:161-176: freq = 1 / theta_f32^(2i/rope_dim) (f32 powf),
 * angle = pos_f32 * freq, tables = cosf/sinf(angle). */
void or_rope_table(double theta, int32_t rope_dim, int32_t max_pos,
                   float* cos_table, float* sin_table) {
    int32_t half = rope_dim / 2;
    float th = (float)theta;
    for (int32_t pos = 0; pos < max_pos; ++pos) {
        for (int32_t i = 0; i < half; ++i) {
            float freq = 1.0f / powf(th, 2.0f * (float)i / (float)rope_dim);
            float angle = (float)pos * freq;
            cos_table[(size_t)pos * half + i] = cosf(angle);
            sin_table[(size_t)pos * half + i] = sinf(angle);
        }
    }
}

/* ------------------------------------------------------------------ */
/* DeltaNet head update                                                 */
/* ------------------------------------------------------------------ */

/* gemv.rs:836-861: decay, retrieve, delta update, output on updated S.
 * S is [v-row r][k-col c] row-major (gemv.rs:813,823-824). */
void or_deltanet_head_update_scalar(float* s, const float* q, const float* k,
                                    const float* v, float alpha, float beta,
                                    int32_t hd, float* y) {
    int32_t n = hd * hd;
    for (int32_t i = 0; i < n; ++i) s[i] *= alpha;
    float* pred = (float*)malloc(sizeof(float) * (size_t)hd);
    for (int32_t r = 0; r < hd; ++r) {
        float dot = 0.0f;
        for (int32_t c = 0; c < hd; ++c) dot += s[r * hd + c] * k[c];
        pred[r] = dot;
    }
    for (int32_t r = 0; r < hd; ++r) {
        float delta = beta * (v[r] - pred[r]);
        for (int32_t c = 0; c < hd; ++c) s[r * hd + c] += delta * k[c];
    }
    for (int32_t r = 0; r < hd; ++r) {
        float dot = 0.0f;
        for (int32_t c = 0; c < hd; ++c) dot += s[r * hd + c] * q[c];
        y[r] = dot;
    }
    free(pred);
}

int32_t or_has_avx512(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") ? 1 : 0;
}

/* simd.rs:33-50 hsum_ps: fold 512->128 as (a+b)+(c+d) over the four
 * 128-bit quarters, then (l0+l2)+(l1+l3). */
static float hsum16_emul(const float v[16]) {
    float s[4];
    for (int i = 0; i < 4; ++i) s[i] = (v[i] + v[4 + i]) + (v[8 + i] + v[12 + i]);
    return (s[0] + s[2]) + (s[1] + s[3]);
}

/* simd.rs:292-362 restated lane by lane with fmaf (one rounding, like
 * _mm512_fmadd_ps).  Bit-identical to the intrinsic version. */
void or_deltanet_head_update_avx512_emul(float* s, const float* q,
                                         const float* k, const float* v,
                                         float alpha, float beta, int32_t hd,
                                         float* y) {
    int32_t hd16 = hd / 16 * 16;
    for (int32_t i = 0; i < hd * hd; ++i) s[i] = s[i] * alpha;
    float* pred = (float*)malloc(sizeof(float) * (size_t)hd);
    for (int32_t r = 0; r < hd; ++r) {
        float acc[16] = {0};
        for (int32_t c = 0; c < hd16; c += 16)
            for (int l = 0; l < 16; ++l) acc[l] = fmaf(s[r * hd + c + l], k[c + l], acc[l]);
        pred[r] = hsum16_emul(acc);
    }
    for (int32_t r = 0; r < hd; ++r) {
        float delta = beta * (v[r] - pred[r]);
        if (delta == 0.0f) continue;               /* simd.rs:332 */
        for (int32_t c = 0; c < hd16; ++c)
            s[r * hd + c] = fmaf(delta, k[c], s[r * hd + c]);
    }
    for (int32_t r = 0; r < hd; ++r) {
        float acc[16] = {0};
        for (int32_t c = 0; c < hd16; c += 16)
            for (int l = 0; l < 16; ++l) acc[l] = fmaf(s[r * hd + c + l], q[c + l], acc[l]);
        y[r] = hsum16_emul(acc);
    }
    free(pred);
}

__attribute__((target("avx512f")))
static float hsum_ps(__m512 v) {
    __m128 a = _mm512_extractf32x4_ps(v, 0);
    __m128 b = _mm512_extractf32x4_ps(v, 1);
    __m128 c = _mm512_extractf32x4_ps(v, 2);
    __m128 d = _mm512_extractf32x4_ps(v, 3);
    __m128 sum = _mm_add_ps(_mm_add_ps(a, b), _mm_add_ps(c, d));
    __m128 hi = _mm_movehl_ps(sum, sum);
    __m128 sum2 = _mm_add_ps(sum, hi);
    __m128 hi2 = _mm_shuffle_ps(sum2, sum2, 1);
    __m128 sum3 = _mm_add_ss(sum2, hi2);
    return _mm_cvtss_f32(sum3);
}

__attribute__((target("avx512f")))
static void head_update_avx512_impl(float* s, const float* q, const float* k,
                                    const float* v, float alpha, float beta,
                                    int32_t hd, float* y, float* pred) {
    int32_t hd16 = hd / 16 * 16;
    __m512 al = _mm512_set1_ps(alpha);
    int32_t total = hd * hd;
    for (int32_t i = 0; i < total; i += 16)
        _mm512_storeu_ps(s + i, _mm512_mul_ps(_mm512_loadu_ps(s + i), al));
    for (int32_t r = 0; r < hd; ++r) {
        __m512 acc = _mm512_setzero_ps();
        for (int32_t c = 0; c < hd16; c += 16)
            acc = _mm512_fmadd_ps(_mm512_loadu_ps(s + r * hd + c), _mm512_loadu_ps(k + c), acc);
        pred[r] = hsum_ps(acc);
    }
    for (int32_t r = 0; r < hd; ++r) {
        float delta = beta * (v[r] - pred[r]);
        if (delta == 0.0f) continue;
        __m512 dv = _mm512_set1_ps(delta);
        for (int32_t c = 0; c < hd16; c += 16)
            _mm512_storeu_ps(s + r * hd + c,
                             _mm512_fmadd_ps(dv, _mm512_loadu_ps(k + c), _mm512_loadu_ps(s + r * hd + c)));
    }
    for (int32_t r = 0; r < hd; ++r) {
        __m512 acc = _mm512_setzero_ps();
        for (int32_t c = 0; c < hd16; c += 16)
            acc = _mm512_fmadd_ps(_mm512_loadu_ps(s + r * hd + c), _mm512_loadu_ps(q + c), acc);
        y[r] = hsum_ps(acc);
    }
}

int32_t or_deltanet_head_update_avx512(float* s, const float* q,
                                       const float* k, const float* v,
                                       float alpha, float beta, int32_t hd,
                                       float* y) {
    if (!or_has_avx512()) return -1;
    float pred_stack[512];
    float* pred = hd <= 512 ? pred_stack : (float*)malloc(sizeof(float) * (size_t)hd);
    head_update_avx512_impl(s, q, k, v, alpha, beta, hd, y, pred);
    if (pred != pred_stack) free(pred);
    return 0;
}

static void head_update(int32_t kind, float* s, const float* q, const float* k,
                        const float* v, float al, float be, int32_t hd, float* y) {
    if (kind == OR_UPDATE_AUTO) kind = or_has_avx512() ? OR_UPDATE_AVX512 : OR_UPDATE_SCALAR;
    if (kind == OR_UPDATE_AVX512 && or_deltanet_head_update_avx512(s, q, k, v, al, be, hd, y) == 0)
        return;
    if (kind == OR_UPDATE_AVX512 || kind == OR_UPDATE_AVX512_EMUL)
        or_deltanet_head_update_avx512_emul(s, q, k, v, al, be, hd, y);
    else
        or_deltanet_head_update_scalar(s, q, k, v, al, be, hd, y);
}

/* ------------------------------------------------------------------ */
/* DeltaNet mixer slices                                                */
/* ------------------------------------------------------------------ */

/* gemv.rs:744-769 (decode) / :1132-1147 (prefill): depthwise causal conv
 * with the old buffer, then shift and append the raw input.  Buffer is
 * [ch][K-1] oldest->newest; weights [ch][K], tap K-1 multiplies x_t. */
void or_conv1d_step(int32_t qkv_dim, int32_t ks, float* conv_buf,
                    const float* conv_w, const float* x, float* out) {
    int32_t bl = ks - 1;
    for (int32_t ch = 0; ch < qkv_dim; ++ch) {
        float sum = 0.0f;
        for (int32_t t = 0; t < bl; ++t) sum += conv_buf[ch * bl + t] * conv_w[ch * ks + t];
        sum += x[ch] * conv_w[ch * ks + bl];
        out[ch] = sum;
    }
    for (int32_t ch = 0; ch < qkv_dim; ++ch) {
        for (int32_t t = 0; t < bl - 1; ++t) conv_buf[ch * bl + t] = conv_buf[ch * bl + t + 1];
        conv_buf[ch * bl + bl - 1] = x[ch];
    }
}

/* gemv.rs:865-883 (decode) / :1205-1219 (prefill): per-head RMSNorm with
 * plain gamma (not 1+gamma), then multiply by silu(z). */
static void gated_norm(int32_t num_v, int32_t hd, const float* y, const float* z,
                       const uint16_t* norm_w, float* out) {
    for (int32_t h = 0; h < num_v; ++h) {
        const float* yh = y + (size_t)h * hd;
        float ss = 0.0f;
        for (int32_t j = 0; j < hd; ++j) ss += yh[j] * yh[j];
        float inv_rms = 1.0f / sqrtf(ss / (float)hd + 1e-6f);
        for (int32_t j = 0; j < hd; ++j) {
            float yn = yh[j] * inv_rms * or_f16_to_f32(norm_w[j]);
            out[(size_t)h * hd + j] = yn * or_silu(z[(size_t)h * hd + j]);
        }
    }
}

/* Shared body of one token: activation, split, L2 norm + q scale, gates,
 * GVA map vh -> vh / (num_v/num_qk), head updates, gated norm. */
static void deltanet_token(const or_config* cfg, float* act /* [qkv_dim], mutated */,
                           const float* a, const float* b, const float* a_log,
                           const float* dt_bias, const float* z,
                           const uint16_t* norm_w, float* s, float* out,
                           int32_t update_kind, float* y /* [v_dim] scratch */,
                           int32_t nthreads) {
    int32_t num_qk = cfg->num_qk_heads, num_v = cfg->num_v_heads, hd = cfg->dn_head_dim;
    int32_t q_dim = num_qk * hd, k_dim = num_qk * hd;
    int32_t v_per_qk = num_v / num_qk;
    float scale = 1.0f / sqrtf((float)hd);
    float* q = act;
    float* k = act + q_dim;
    const float* v = act + q_dim + k_dim;
    /* gemv.rs:780-785 */
    for (int32_t h = 0; h < num_qk; ++h) {
        or_l2_normalize(q + (size_t)h * hd, hd);
        or_l2_normalize(k + (size_t)h * hd, hd);
        for (int32_t j = 0; j < hd; ++j) q[(size_t)h * hd + j] *= scale;
    }
    /* gemv.rs:817 runs the heads serially; nthreads > 1 runs them in
     * parallel (each head's arithmetic is unchanged, so the result is too) */
    if (nthreads < 1) nthreads = 1;
    #pragma omp parallel for num_threads(nthreads) schedule(static) if(nthreads > 1)
    for (int32_t vh = 0; vh < num_v; ++vh) {
        /* gemv.rs:788-800: alpha = exp(-exp(A_log) * softplus(a + dt_bias)) */
        float a_exp = expf(a_log[vh]);
        float sp = or_softplus(a[vh] + dt_bias[vh]);
        float al = expf(-a_exp * sp);
        float be = 1.0f / (1.0f + expf(-b[vh]));
        int32_t qk_h = vh / v_per_qk;             /* gemv.rs:806 */
        head_update(update_kind, s + (size_t)vh * hd * hd, q + (size_t)qk_h * hd,
                    k + (size_t)qk_h * hd, v + (size_t)vh * hd, al, be, hd,
                    y + (size_t)vh * hd);
    }
    gated_norm(num_v, hd, y, z, norm_w, out);
}

void or_deltanet_decode_step(const or_config* cfg, const float* qkv,
                             int32_t preact, float* conv_buf,
                             const float* conv_w, const float* a,
                             const float* b, const float* a_log,
                             const float* dt_bias, const float* z,
                             const uint16_t* norm_w, float* s, float* out,
                             int32_t update_kind) {
    or_deltanet_decode_step_mt(cfg, qkv, preact, conv_buf, conv_w, a, b, a_log, dt_bias, z,
                               norm_w, s, out, update_kind, 1);
}

void or_deltanet_decode_step_mt(const or_config* cfg, const float* qkv,
                                int32_t preact, float* conv_buf,
                                const float* conv_w, const float* a,
                                const float* b, const float* a_log,
                                const float* dt_bias, const float* z,
                                const uint16_t* norm_w, float* s, float* out,
                                int32_t update_kind, int32_t nthreads) {
    int32_t hd = cfg->dn_head_dim;
    int32_t qkv_dim = (2 * cfg->num_qk_heads + cfg->num_v_heads) * hd;
    int32_t v_dim = cfg->num_v_heads * hd;
    float* act = (float*)malloc(sizeof(float) * (size_t)qkv_dim);
    float* y = (float*)malloc(sizeof(float) * (size_t)v_dim);
    if (preact) {
        or_conv1d_step(qkv_dim, cfg->conv_kernel, conv_buf, conv_w, qkv, act);
        for (int32_t i = 0; i < qkv_dim; ++i) act[i] = or_silu(act[i]); /* gemv.rs:772 */
    } else {
        memcpy(act, qkv, sizeof(float) * (size_t)qkv_dim);
    }
    deltanet_token(cfg, act, a, b, a_log, dt_bias, z, norm_w, s, out, update_kind, y, nthreads);
    free(act);
    free(y);
}

/* gemv.rs:1119-1219: sequential per-token loop with the scalar update
 * (the prefill path never dispatches to AVX-512). */
void or_deltanet_prefill(const or_config* cfg, int32_t T,
                         const float* qkv_all, const float* a_all,
                         const float* b_all, const float* z_all,
                         float* conv_buf, const float* conv_w,
                         const float* a_log, const float* dt_bias,
                         const uint16_t* norm_w, float* s, float* out_all) {
    int32_t hd = cfg->dn_head_dim, num_v = cfg->num_v_heads;
    int32_t qkv_dim = (2 * cfg->num_qk_heads + num_v) * hd;
    int32_t v_dim = num_v * hd;
    float* act = (float*)malloc(sizeof(float) * (size_t)qkv_dim);
    float* y = (float*)malloc(sizeof(float) * (size_t)v_dim);
    for (int32_t t = 0; t < T; ++t) {
        or_conv1d_step(qkv_dim, cfg->conv_kernel, conv_buf, conv_w,
                       qkv_all + (size_t)t * qkv_dim, act);
        for (int32_t i = 0; i < qkv_dim; ++i) act[i] = or_silu(act[i]);
        deltanet_token(cfg, act, a_all + (size_t)t * num_v, b_all + (size_t)t * num_v,
                       a_log, dt_bias, z_all + (size_t)t * v_dim, norm_w, s,
                       out_all + (size_t)t * v_dim, OR_UPDATE_SCALAR, y, 1);
    }
    free(act);
    free(y);
}

/* ------------------------------------------------------------------ */
/* GQA mixer slices                                                     */
/* ------------------------------------------------------------------ */

/* One head's softmax attention over rows 0..len-1 of a [seq][num_kv][D]
 * cache (gemv.rs:964-986 / :1409-1427).  out is accumulated into. */
static void attend_head(const float* qv, const float* kc, const float* vc,
                        int32_t len, int32_t kv_stride, int32_t kv_off, int32_t D,
                        float scale, float* scores, float* out) {
    for (int32_t t = 0; t < len; ++t) {
        const float* kr = kc + (size_t)t * kv_stride + kv_off;
        float dot = 0.0f;
        for (int32_t d = 0; d < D; ++d) dot += qv[d] * kr[d];
        scores[t] = dot * scale;
    }
    or_softmax_raw(scores, len);
    for (int32_t t = 0; t < len; ++t) {
        const float* vr = vc + (size_t)t * kv_stride + kv_off;
        float sc = scores[t];
        for (int32_t d = 0; d < D; ++d) out[d] += sc * vr[d];
    }
}

int32_t or_attn_decode_step(const or_config* cfg, const float* q_gate,
                            const float* k_new, const float* v_new,
                            const uint16_t* q_norm, const uint16_t* k_norm,
                            const float* rope_cos, const float* rope_sin,
                            int32_t rope_len, float* k_cache, float* v_cache,
                            int32_t seq_len, int32_t round_kv_f16, float* out,
                            int32_t nthreads) {
    int32_t H = cfg->num_heads, KV = cfg->num_kv_heads, D = cfg->attn_head_dim;
    int32_t groups = H / KV, rot = cfg->rope_dim;
    int32_t offset = seq_len;
    if (offset >= rope_len) return -1;
    float* q = (float*)malloc(sizeof(float) * (size_t)H * D);
    float* gate = (float*)malloc(sizeof(float) * (size_t)H * D);
    float* kn = (float*)malloc(sizeof(float) * (size_t)KV * D);
    /* gemv.rs:927-938 split interleaved [q_h | gate_h] */
    for (int32_t h = 0; h < H; ++h) {
        memcpy(q + (size_t)h * D, q_gate + (size_t)h * 2 * D, sizeof(float) * (size_t)D);
        memcpy(gate + (size_t)h * D, q_gate + (size_t)h * 2 * D + D, sizeof(float) * (size_t)D);
    }
    memcpy(kn, k_new, sizeof(float) * (size_t)KV * D);
    or_per_head_rms_norm(q, H, D, q_norm);                 /* :945 */
    or_per_head_rms_norm(kn, KV, D, k_norm);               /* :946 */
    or_apply_partial_rope(q, H, D, rope_cos, rope_sin, rot, offset);  /* :949 */
    or_apply_partial_rope(kn, KV, D, rope_cos, rope_sin, rot, offset); /* :950 */
    /* :953-956 append */
    float* krow = k_cache + (size_t)seq_len * KV * D;
    float* vrow = v_cache + (size_t)seq_len * KV * D;
    for (int32_t i = 0; i < KV * D; ++i) {
        krow[i] = round_kv_f16 ? or_f16_to_f32(or_f32_to_f16(kn[i])) : kn[i];
        vrow[i] = round_kv_f16 ? or_f16_to_f32(or_f32_to_f16(v_new[i])) : v_new[i];
    }
    int32_t L = seq_len + 1;
    float scale = 1.0f / sqrtf((float)D);
    memset(out, 0, sizeof(float) * (size_t)H * D);
    if (nthreads < 1) nthreads = 1;
    #pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int32_t h = 0; h < H; ++h) {
        float* scores = (float*)malloc(sizeof(float) * (size_t)L);
        attend_head(q + (size_t)h * D, k_cache, v_cache, L, KV * D, (h / groups) * D, D,
                    scale, scores, out + (size_t)h * D);
        free(scores);
    }
    /* :1008-1011 output gate */
    for (int32_t j = 0; j < H * D; ++j) out[j] *= 1.0f / (1.0f + expf(-gate[j]));
    free(q); free(gate); free(kn);
    return 0;
}

int32_t or_attn_prefill(const or_config* cfg, int32_t S, const float* q_gate_all,
                        const float* k_all, const float* v_all,
                        const uint16_t* q_norm, const uint16_t* k_norm,
                        const float* rope_cos, const float* rope_sin,
                        int32_t rope_len, float* k_cache, float* v_cache,
                        float* out, const int32_t* rows, int32_t n_rows,
                        int32_t nthreads) {
    int32_t H = cfg->num_heads, KV = cfg->num_kv_heads, D = cfg->attn_head_dim;
    int32_t groups = H / KV, rot = cfg->rope_dim;
    int32_t q_dim = H * D, kv_dim = KV * D;
    if (S > rope_len) return -1;
    float* q_all = (float*)malloc(sizeof(float) * (size_t)S * q_dim);
    float* g_all = (float*)malloc(sizeof(float) * (size_t)S * q_dim);
    /* gemv.rs:1364-1381 split */
    for (int32_t t = 0; t < S; ++t)
        for (int32_t h = 0; h < H; ++h) {
            const float* src = q_gate_all + (size_t)t * 2 * q_dim + (size_t)h * 2 * D;
            memcpy(q_all + (size_t)t * q_dim + (size_t)h * D, src, sizeof(float) * (size_t)D);
            memcpy(g_all + (size_t)t * q_dim + (size_t)h * D, src + D, sizeof(float) * (size_t)D);
        }
    memcpy(k_cache, k_all, sizeof(float) * (size_t)S * kv_dim);
    memcpy(v_cache, v_all, sizeof(float) * (size_t)S * kv_dim);
    /* gemv.rs:1387-1395 QK norm + RoPE at position t */
    for (int32_t t = 0; t < S; ++t) {
        or_per_head_rms_norm(q_all + (size_t)t * q_dim, H, D, q_norm);
        or_per_head_rms_norm(k_cache + (size_t)t * kv_dim, KV, D, k_norm);
        or_apply_partial_rope(q_all + (size_t)t * q_dim, H, D, rope_cos, rope_sin, rot, t);
        or_apply_partial_rope(k_cache + (size_t)t * kv_dim, KV, D, rope_cos, rope_sin, rot, t);
    }
    float scale = 1.0f / sqrtf((float)D);
    int32_t nr = rows ? n_rows : S;
    if (nthreads < 1) nthreads = 1;
    /* gemv.rs:1406-1429: heads in parallel, causal rows t1, keys t2 <= t1 */
    #pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int32_t h = 0; h < H; ++h) {
        float* scores = (float*)malloc(sizeof(float) * (size_t)S);
        float* acc = (float*)malloc(sizeof(float) * (size_t)D);
        for (int32_t i = 0; i < nr; ++i) {
            int32_t t1 = rows ? rows[i] : i;
            memset(acc, 0, sizeof(float) * (size_t)D);
            attend_head(q_all + (size_t)t1 * q_dim + (size_t)h * D, k_cache, v_cache, t1 + 1,
                        kv_dim, (h / groups) * D, D, scale, scores, acc);
            /* :1441-1444 gate */
            float* o = out + (size_t)t1 * q_dim + (size_t)h * D;
            const float* g = g_all + (size_t)t1 * q_dim + (size_t)h * D;
            for (int32_t d = 0; d < D; ++d) o[d] = acc[d] * (1.0f / (1.0f + expf(-g[d])));
        }
        free(scores);
        free(acc);
    }
    free(q_all); free(g_all);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Q4 projections                                                       */
/* ------------------------------------------------------------------ */
/* Rust `(v).round() as i32`: half away from zero, NaN -> 0, saturating. */
static int32_t rust_round_i32(float v) {
    if (v != v) return 0;
    float r = roundf(v);
    if (r >= 2147483647.0f) return 2147483647;
    if (r <= -2147483648.0f) return (int32_t)-2147483647 - 1;
    return (int32_t)r;
}

/* convert.rs:437-467 */
void or_q4_quantize(const float* data, int32_t k, int32_t n, uint8_t* packed,
                    uint16_t* scales) {
    const int32_t gs = 32, groups = n / gs;
    size_t pi = 0, si = 0;
    for (int32_t ki = 0; ki < k; ++ki)
        for (int32_t g = 0; g < groups; ++g) {
            const float* grp = data + (size_t)ki * n + (size_t)g * gs;
            /* :448-449 absmax via f32::max (a NaN operand is ignored) */
            float absmax = 0.0f;
            for (int32_t j = 0; j < gs; ++j) {
                float a = fabsf(grp[j]);
                absmax = (a != a) ? absmax : (absmax != absmax ? a : (a > absmax ? a : absmax));
            }
            float scale = absmax > 0.0f ? absmax / 7.0f : 0.0f;   /* :450 */
            scales[si++] = or_f32_to_f16(scale);                   /* :451 */
            float inv = scale > 0.0f ? 1.0f / scale : 0.0f;        /* :454 */
            for (int32_t j = 0; j < gs; j += 2) {                  /* :455-459 */
                int32_t q0 = rust_round_i32(grp[j] * inv);
                int32_t q1 = rust_round_i32(grp[j + 1] * inv);
                q0 = (q0 < -8 ? -8 : (q0 > 7 ? 7 : q0)) + 8;
                q1 = (q1 < -8 ? -8 : (q1 > 7 ? 7 : q1)) + 8;
                packed[pi++] = (uint8_t)((uint32_t)q0 | ((uint32_t)q1 << 4));
            }
        }
}

/* gemv.rs:412-445, k range [0, k) */
void or_q4_gemv(const float* x, const uint8_t* packed, const uint16_t* scales,
                int32_t k, int32_t n, float* y) {
    const int32_t groups = n / 32, ppg = 16, ppr = groups * ppg;
    for (int32_t j = 0; j < n; ++j) y[j] = 0.0f;
    for (int32_t ki = 0; ki < k; ++ki) {
        float val = x[ki];
        if (val == 0.0f) continue;
        for (int32_t g = 0; g < groups; ++g) {
            float s = or_f16_to_f32(scales[(size_t)ki * groups + g]) * val;
            if (s == 0.0f) continue;
            float lut[16];
            for (int32_t i = 0; i < 16; ++i) lut[i] = s * (float)(i - 8);
            lut[8] = 0.0f;                /* the reference's literal 0.0 (s * 0 could be -0) */
            lut[9] = s;                   /* the literal s (s * 1.0 is s) */
            const uint8_t* po = packed + (size_t)ki * ppr + (size_t)g * ppg;
            float* oo = y + (size_t)g * 32;
            for (int32_t j = 0; j < ppg; ++j) {
                uint8_t b = po[j];
                oo[2 * j] += lut[b & 0x0F];
                oo[2 * j + 1] += lut[b >> 4];
            }
        }
    }
}

/* gemv.rs:529-542 */
void or_q4_gemm(const float* x, int32_t m, const uint8_t* packed,
                const uint16_t* scales, int32_t k, int32_t n, float* y,
                int32_t nthreads) {
    if (nthreads < 1) nthreads = 1;
    #pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int32_t t = 0; t < m; ++t)
        or_q4_gemv(x + (size_t)t * k, packed, scales, k, n, y + (size_t)t * n);
}

/* gemv.rs:469-526: the scalar fallback over one k chunk, then
 * out = (g / (1 + exp(-g))) * u (:523-524) */
void or_q4_gate_up(const float* x, const uint8_t* g_packed,
                   const uint16_t* g_scales, const uint8_t* u_packed,
                   const uint16_t* u_scales, int32_t k, int32_t n, float* out) {
    float* g = (float*)malloc(sizeof(float) * (size_t)n);
    float* u = (float*)malloc(sizeof(float) * (size_t)n);
    or_q4_gemv(x, g_packed, g_scales, k, n, g);
    or_q4_gemv(x, u_packed, u_scales, k, n, u);
    for (int32_t j = 0; j < n; ++j) out[j] = (g[j] / (1.0f + expf(-g[j]))) * u[j];
    free(g);
    free(u);
}

/* gemv.rs:678-708: rows in parallel (rayon chunks of 256 rows there), each
 * row's dot product sequential over its groups and bytes */
void or_q4_lm_head(const float* x, const uint8_t* packed, const uint16_t* scales,
                   int32_t vocab, int32_t hidden, float* out, int32_t nthreads) {
    const int32_t gpr = hidden / 32, ppg = 16, ppr = gpr * ppg;
    if (nthreads < 1) nthreads = 1;
    #pragma omp parallel for num_threads(nthreads) schedule(static, 256)
    for (int32_t v = 0; v < vocab; ++v) {
        float dot = 0.0f;
        const size_t sb = (size_t)v * gpr, pb = (size_t)v * ppr;
        for (int32_t g = 0; g < gpr; ++g) {
            const float scale = or_f16_to_f32(scales[sb + g]);
            if (scale == 0.0f) continue;
            const size_t po = pb + (size_t)g * ppg;
            const int32_t io = g * 32;
            float lut[16];
            for (int q = 0; q < 16; ++q) lut[q] = scale * (float)(q - 8);
            for (int32_t j = 0; j < ppg; ++j) {
                const uint8_t byte = packed[po + j];
                dot += x[io + j * 2] * lut[byte & 0x0F];
                dot += x[io + j * 2 + 1] * lut[byte >> 4];
            }
        }
        out[v] = dot;
    }
}

/* gemv.rs:544-563 */
void or_q4_embed(const uint8_t* packed, const uint16_t* scales, int32_t hidden,
                 int32_t id, float* out) {
    const int32_t gpr = hidden / 32;
    const size_t sb = (size_t)id * gpr, pb = (size_t)id * gpr * 16;
    for (int32_t g = 0; g < gpr; ++g) {
        const float scale = or_f16_to_f32(scales[sb + g]);
        const size_t po = pb + (size_t)g * 16;
        for (int32_t j = 0; j < 16; ++j) {
            const uint8_t byte = packed[po + j];
            out[g * 32 + j * 2] = scale * (float)((int32_t)(byte & 0x0F) - 8);
            out[g * 32 + j * 2 + 1] = scale * (float)((int32_t)((byte >> 4) & 0x0F) - 8);
        }
    }
}

/* ---- sampling ---------------------------------------------------------- */
/* generate.rs:46-54 */
float or_rng_next_f32(uint64_t* state) {
    uint64_t s = *state;
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    *state = s;
    return (float)(s >> 40) / 16777216.0f;
}

/* generate.rs:58-69 */
void or_apply_repetition_penalty(float* logits, int32_t vocab, const int32_t* generated,
                                 int32_t n, float penalty) {
    if (penalty <= 1.0f) return;
    const int32_t window = n < 64 ? n : 64;
    for (int32_t i = n - window; i < n; ++i) {
        const int32_t idx = generated[i];
        if (idx >= 0 && idx < vocab) {
            if (logits[idx] > 0.0f) logits[idx] /= penalty;
            else logits[idx] *= penalty;
        }
    }
}

/* generate.rs:72-82 */
void or_apply_presence_penalty(float* logits, int32_t vocab, const int32_t* generated,
                               int32_t n, float penalty) {
    if (penalty <= 0.0f || n == 0) return;
    unsigned char* seen = (unsigned char*)calloc((size_t)vocab, 1);
    for (int32_t i = 0; i < n; ++i)
        if (generated[i] >= 0 && generated[i] < vocab) seen[generated[i]] = 1;
    for (int32_t i = 0; i < vocab; ++i)
        if (seen[i]) logits[i] -= penalty;
    free(seen);
}

typedef struct { uint32_t id; float v; } or_idx_logit;

/* the stable descending sort_by of generate.rs:350 / gpu_inference.rs:879:
 * equal logits keep index order */
static int or_cmp_desc(const void* a, const void* b) {
    const or_idx_logit* x = (const or_idx_logit*)a;
    const or_idx_logit* y = (const or_idx_logit*)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return x->id < y->id ? -1 : (x->id > y->id);
}

int32_t or_sample_top_k(const float* logits, int32_t vocab, float temperature, float top_p,
                        int32_t top_k, uint64_t* rng_state, int32_t wgpu,
                        int32_t* out_ids, float* out_probs) {
    if (temperature <= 0.0f) {
        int32_t best = 0;
        if (!wgpu) {                       /* generate.rs:336-341: first maximum */
            float max_val = -INFINITY;
            for (int32_t i = 0; i < vocab; ++i)
                if (logits[i] > max_val) { max_val = logits[i]; best = i; }
        } else {                           /* max_by: the last maximum */
            for (int32_t i = 1; i < vocab; ++i)
                if (!(logits[i] < logits[best])) best = i;
        }
        if (out_ids) out_ids[0] = best;
        return best;
    }
    const float inv_temp = 1.0f / temperature;
    or_idx_logit* ix = (or_idx_logit*)malloc(sizeof(or_idx_logit) * (size_t)vocab);
    float max_logit = -INFINITY;
    for (int32_t i = 0; i < vocab; ++i) {
        ix[i].id = (uint32_t)i;
        ix[i].v = logits[i];
        if (logits[i] > max_logit) max_logit = logits[i];     /* f32::max fold */
    }
    qsort(ix, (size_t)vocab, sizeof(or_idx_logit), or_cmp_desc);
    const int32_t k = top_k > 0 ? (top_k < vocab ? top_k : vocab) : vocab;
    if (wgpu) max_logit = ix[0].v;
    float* p = (float*)malloc(sizeof(float) * (size_t)k);
    for (int32_t i = 0; i < k; ++i) p[i] = expf((ix[i].v - max_logit) * inv_temp);
    float sum = 0.0f;
    for (int32_t i = 0; i < k; ++i) sum += p[i];
    int32_t tok;
    if (!wgpu && sum <= 0.0f) {
        tok = (int32_t)ix[0].id;
        goto done;
    }
    if (wgpu) {
        for (int32_t i = 0; i < k; ++i) p[i] /= sum;
    } else {
        const float inv = 1.0f / sum;
        for (int32_t i = 0; i < k; ++i) p[i] *= inv;
    }
    {
        float cumsum = 0.0f;
        int32_t cutoff = k;
        for (int32_t i = 0; i < k; ++i) {
            cumsum += p[i];
            if (cumsum >= top_p) { cutoff = i + 1; break; }
        }
        float total = 0.0f;
        for (int32_t i = 0; i < cutoff; ++i) total += p[i];
        if (!wgpu && total <= 0.0f) {
            tok = (int32_t)ix[0].id;
            goto done;
        }
        const float rand_val = or_rng_next_f32(rng_state) * total;
        float accum = 0.0f;
        tok = (int32_t)ix[0].id;
        for (int32_t i = 0; i < cutoff; ++i) {
            accum += p[i];
            if (accum >= rand_val) { tok = (int32_t)ix[i].id; break; }
        }
    }
done:
    if (out_ids) for (int32_t i = 0; i < k; ++i) out_ids[i] = (int32_t)ix[i].id;
    if (out_probs) for (int32_t i = 0; i < k; ++i) out_probs[i] = p[i];
    free(p);
    free(ix);
    return tok;
}
