/*
 * qora_oracle.h -- CPU oracle for the QORA-4B token-mixer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the
 * reference CPU path (Rust crate qor4b, src/gemv.rs, src/simd.rs,
 * src/convert.rs), written from reading that source.  It is the oracle
 * that the HIP kernels are compared against and the CPU baseline that the
 * benchmark times.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links it.
 *
 * Numerics follow the reference's scalar Rust semantics: f32 arithmetic
 * evaluated left to right, no FMA contraction (built with
 * -ffp-contract=off), glibc expf/logf/powf/cosf/sinf (what Rust's f32
 * methods lower to on x86_64 Linux), sequential left-fold sums.  The
 * AVX-512 head update restates simd.rs with the same intrinsics and the
 * same horizontal-sum tree; a lane-exact scalar emulation of it exists for
 * hosts without AVX-512.
 *
 * Every function is pinned by tests/test_oracle.py (invariants, closed
 * forms, brute force, fp64 shadows, chunked == recurrent).  None of the
 * reference's own tests can pin it: the reference has no tests, fixtures or
 * golden vectors, and its Rust toolchain is not available here.
 */
#ifndef QORA_ORACLE_H
#define QORA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mixer dimensions (config.rs:42-79 default_4b; helpers config.rs:82-97). */
typedef struct {
    int32_t num_qk_heads;   /* DeltaNet q/k heads (16) */
    int32_t num_v_heads;    /* DeltaNet v heads (32) */
    int32_t dn_head_dim;    /* DeltaNet head dim (128) */
    int32_t conv_kernel;    /* causal conv1d taps (4) */
    int32_t num_heads;      /* GQA query heads (16) */
    int32_t num_kv_heads;   /* GQA kv heads (4) */
    int32_t attn_head_dim;  /* GQA head dim (256) */
    int32_t rope_dim;       /* rotated dims per head (64) */
} or_config;

/* --- scalar helpers (gemv.rs:565-659) --------------------------------- */
float    or_f16_to_f32(uint16_t h);            /* half 2.7 to_f32: exact   */
uint16_t or_f32_to_f16(float f);               /* IEEE RNE                 */
float    or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);              /* RNE                      */
float    or_silu(float x);                     /* gemv.rs:631-633          */
float    or_softplus(float x);                 /* gemv.rs:637-639          */
void     or_l2_normalize(float* x, int32_t n); /* gemv.rs:643-649          */
void     or_softmax_raw(float* s, int32_t n);  /* gemv.rs:653-659          */
void     or_rms_norm(const float* x, int32_t n, const uint16_t* gamma,
                     float* out);              /* gemv.rs:571-579 (1+g)    */
void     or_per_head_rms_norm(float* x, int32_t num_heads, int32_t head_dim,
                              const uint16_t* gamma); /* gemv.rs:586-597   */
void     or_apply_partial_rope(float* data, int32_t num_heads,
                               int32_t head_dim, const float* cos_table,
                               const float* sin_table, int32_t rotary_dim,
                               int32_t position); /* gemv.rs:604-627       */
/* RoPE tables [max_pos][rope_dim/2] (convert.rs:161-176). */
void     or_rope_table(double theta, int32_t rope_dim, int32_t max_pos,
                       float* cos_table, float* sin_table);

/* --- DeltaNet head update --------------------------------------------- */
/* Scalar path, gemv.rs:836-861 (decode) == gemv.rs:1174-1201 (prefill). */
void or_deltanet_head_update_scalar(float* s, const float* q, const float* k,
                                    const float* v, float alpha, float beta,
                                    int32_t hd, float* y);
/* AVX-512 path, simd.rs:292-362 (hd % 16 == 0).  Returns 0 on success,
 * -1 when the host has no AVX-512F (nothing is written then). */
int32_t or_deltanet_head_update_avx512(float* s, const float* q,
                                       const float* k, const float* v,
                                       float alpha, float beta, int32_t hd,
                                       float* y);
/* Lane-exact scalar emulation of the AVX-512 path (any host). */
void or_deltanet_head_update_avx512_emul(float* s, const float* q,
                                         const float* k, const float* v,
                                         float alpha, float beta, int32_t hd,
                                         float* y);
int32_t or_has_avx512(void);                   /* simd.rs:18-27            */

/* Head-update variants selectable by the layer functions below. */
enum { OR_UPDATE_SCALAR = 0, OR_UPDATE_AVX512 = 1, OR_UPDATE_AVX512_EMUL = 2,
       OR_UPDATE_AUTO = 3 /* AVX-512 when present, else scalar (gemv.rs:814) */ };

/* --- causal depthwise conv1d step (gemv.rs:744-769 / :1132-1147) ------ */
/* out[ch] = sum_{t<K-1} buf[ch][t] w[ch][t] + x[ch] w[ch][K-1]; then the
 * buffer [qkv_dim][K-1] (oldest..newest) shifts left and takes x.  No SiLU. */
void or_conv1d_step(int32_t qkv_dim, int32_t ks, float* conv_buf,
                    const float* conv_w, const float* x, float* out);

/* --- DeltaNet mixer slice: one decode step (gemv.rs:744-883) ---------- */
/* qkv   [qkv_dim]: with preact=1 the raw in_proj_qkv output (conv1d +
 *       SiLU applied here, conv_buf [qkv_dim][K-1] shifted); with preact=0
 *       the already-activated stream (conv and SiLU skipped, conv_buf
 *       untouched).
 * a, b  [num_v]: in_proj_a / in_proj_b outputs.
 * z     [v_dim]: in_proj_z output (silu applied here, gemv.rs:880-882).
 * s     [num_v][hd][hd] state, updated in place.
 * out   [v_dim]: gated, normed mixer output (the out_proj input).       */
void or_deltanet_decode_step(const or_config* cfg, const float* qkv,
                             int32_t preact, float* conv_buf,
                             const float* conv_w, const float* a,
                             const float* b, const float* a_log,
                             const float* dt_bias, const float* z,
                             const uint16_t* norm_w, float* s, float* out,
                             int32_t update_kind);
/* The same step with the v-head loop split over nthreads OpenMP threads
 * (the reference runs it serially, gemv.rs:817); results are identical. */
void or_deltanet_decode_step_mt(const or_config* cfg, const float* qkv,
                                int32_t preact, float* conv_buf,
                                const float* conv_w, const float* a,
                                const float* b, const float* a_log,
                                const float* dt_bias, const float* z,
                                const uint16_t* norm_w, float* s, float* out,
                                int32_t update_kind, int32_t nthreads);

/* --- DeltaNet mixer slice: sequential prefill (gemv.rs:1119-1219) ----- */
/* qkv_all [T][qkv_dim] raw projections, a_all/b_all [T][num_v],
 * z_all [T][v_dim]; out_all [T][v_dim].  State and conv_buf in place.   */
void or_deltanet_prefill(const or_config* cfg, int32_t T,
                         const float* qkv_all, const float* a_all,
                         const float* b_all, const float* z_all,
                         float* conv_buf, const float* conv_w,
                         const float* a_log, const float* dt_bias,
                         const uint16_t* norm_w, float* s, float* out_all);

/* --- GQA mixer slice: one decode step (gemv.rs:927-1011) -------------- */
/* q_gate [num_heads][2*D] interleaved q|gate per head (gemv.rs:927-937),
 * k_new/v_new [num_kv][D] projection outputs.  k_cache/v_cache hold
 * [seq_len + 1][num_kv][D] f32 (reference layout, gemv.rs:164-168); rows
 * 0..seq_len-1 are the past, row seq_len is written here (the append).
 * round_kv_f16 != 0 rounds the appended k/v rows to f16 first (the cache
 * dtype of the MI355X build).  out [num_heads][D] = gated attention.
 * nthreads > 1 splits heads over OpenMP threads exactly as rayon splits
 * them (gemv.rs:963); per-head arithmetic is identical either way.
 * Returns 0, or -1 when a RoPE position is beyond the table (the
 * reference panics on the slice index there, gemv.rs:620-621).          */
int32_t or_attn_decode_step(const or_config* cfg, const float* q_gate,
                         const float* k_new, const float* v_new,
                         const uint16_t* q_norm, const uint16_t* k_norm,
                         const float* rope_cos, const float* rope_sin,
                         int32_t rope_len, float* k_cache, float* v_cache,
                         int32_t seq_len, int32_t round_kv_f16, float* out,
                         int32_t nthreads);

/* --- GQA mixer slice: causal prefill (gemv.rs:1364-1444) -------------- */
/* q_gate_all [S][num_heads][2*D]; k_all, v_all [S][num_kv][D] raw
 * projections.  k_cache/v_cache [S][num_kv][D] receive the normed+roped K
 * and V (the cache replacement, gemv.rs:1397-1400).  out [S][num_heads][D].
 * rows: if non-NULL, only query rows rows[0..n_rows) are computed (the
 * others of out are left untouched); NULL computes all S rows.
 * Returns 0, or -1 when S exceeds the RoPE table.                       */
int32_t or_attn_prefill(const or_config* cfg, int32_t S, const float* q_gate_all,
                     const float* k_all, const float* v_all,
                     const uint16_t* q_norm, const uint16_t* k_norm,
                     const float* rope_cos, const float* rope_sin,
                     int32_t rope_len, float* k_cache, float* v_cache,
                     float* out, const int32_t* rows, int32_t n_rows,
                     int32_t nthreads);

/* --- Q4 projections ------------------------------------------------- */
/* quantize_q4, convert.rs:437-467: data [k][n] f32 (n % 32 == 0) ->
 * packed [k][n/2] (per 32-column group: 16 bytes, low nibble = even
 * column) and scales [k][n/32] f16 = absmax/7.                          */
void or_q4_quantize(const float* data, int32_t k, int32_t n, uint8_t* packed,
                    uint16_t* scales);
/* gemv_q4_inner over the full k range, gemv.rs:412-445 (scalar path; the
 * AVX-512 twin simd.rs:73-139 forms the same lut values and sums in the
 * same order): y[n] = x[k] @ W.                                          */
void or_q4_gemv(const float* x, const uint8_t* packed, const uint16_t* scales,
                int32_t k, int32_t n, float* y);
/* gemm_q4, gemv.rs:529-542: each of the m rows of x [m][k] independently
 * through gemv_q4_inner; y [m][n].                                      */
void or_q4_gemm(const float* x, int32_t m, const uint8_t* packed,
                const uint16_t* scales, int32_t k, int32_t n, float* y,
                int32_t nthreads);
/* fused_gate_up_q4, gemv.rs:469-526 (one k chunk): out[j] =
 * silu(g[j]) * u[j] with g = x @ Wg, u = x @ Wu.                         */
void or_q4_gate_up(const float* x, const uint8_t* g_packed,
                   const uint16_t* g_scales, const uint8_t* u_packed,
                   const uint16_t* u_scales, int32_t k, int32_t n, float* out);

/* --- vocabulary side: embedding lookup and lm_head ------------------- */
/* The embedding is a Q4Weight with k = vocab rows, n = hidden columns
 * (convert.rs:390-415): packed [vocab][hidden/2], scales [vocab][hidden/32]. */
/* lm_head_parallel, Q4 arm, gemv.rs:678-708: out[v] = x . row v, per row
 * a 16-entry lut of scale * (q - 8) per group, groups with scale 0
 * skipped, products summed in column order.                              */
void or_q4_lm_head(const float* x, const uint8_t* packed, const uint16_t* scales,
                   int32_t vocab, int32_t hidden, float* out, int32_t nthreads);
/* embed_lookup_q4, gemv.rs:544-563: out[hidden] = row id dequantized.    */
void or_q4_embed(const uint8_t* packed, const uint16_t* scales, int32_t hidden,
                 int32_t id, float* out);

/* --- sampling (generate.rs:41-82,334-384; wgpu twin gpu_inference.rs:
 * 855-931) -------------------------------------------------------------- */
/* Rng::next_f32, generate.rs:46-54 (xorshift64 13/7/17, top 24 bits).    */
float or_rng_next_f32(uint64_t* state);
/* apply_repetition_penalty / apply_presence_penalty, generate.rs:58-82.  */
void or_apply_repetition_penalty(float* logits, int32_t vocab, const int32_t* generated,
                                 int32_t n, float penalty);
void or_apply_presence_penalty(float* logits, int32_t vocab, const int32_t* generated,
                               int32_t n, float penalty);
/* sample_token_top_k: wgpu = 0 follows generate.rs:334-384, wgpu = 1
 * gpu_inference.rs:867-906.  top_k = 0 means all logits (generate.rs only).
 * If out_ids / out_probs are non-null they receive the first k sorted ids
 * and (when sampling) their normalized probabilities.                    */
int32_t or_sample_top_k(const float* logits, int32_t vocab, float temperature, float top_p,
                        int32_t top_k, uint64_t* rng_state, int32_t wgpu,
                        int32_t* out_ids, float* out_probs);

#ifdef __cplusplus
}
#endif
#endif
