/*
 * qora_mixer.h -- C ABI of the MI355X token-mixer library (libqora_mixer.so).
 *
 * The library runs the two halves of the QORA-4B token mixer on one
 * MI355X (gfx950) with hand-written HIP kernels loaded from code objects:
 *   - Gated DeltaNet: recurrent decode step and chunked prefill;
 *   - full-attention GQA: decode step over an f16 KV cache and causal
 *     prefill that writes that cache.
 * Each mixer entry replaces the middle of one reference layer-forward
 * (cited per entry).  Around the mixer the library also exports the
 * neighbouring steps of a decode or prefill layer, each a separate entry
 * the caller may use or not: the Q4 projections (GEMV for decode with the
 * RMSNorm, residual, SiLU gate/up and DeltaNet conv fused; an MFMA GEMM for
 * prefill), lm_head and the embedding lookup, and next-token sampling.
 * F16 projections stay with the caller.
 *
 * Conventions
 *   - Every entry returns int32_t status (QM_OK == 0); qm_status_string()
 *     names a code and qm_last_error() gives the detail of the last failure
 *     on that context.  The reference panics on the same conditions
 *     (gemv.rs:1049, gemv.rs:620-621) and its GPU thread turns panics into
 *     Err (gpu_inference.rs:950-975); a Rust caller maps non-zero to Err.
 *   - All pointers named *_dev are device pointers (from qm_alloc or any
 *     hipMalloc); sizes are element counts unless named *bytes.  Device
 *     pointers given to the mixer calls must be 16-byte aligned (the
 *     kernels move 16-byte vectors); others are refused with
 *     QM_ERR_INVALID_ARG.
 *   - Kernels are enqueued asynchronously on `stream` (a hipStream_t; NULL
 *     means the context's own stream).  Nothing synchronises the host
 *     except qm_sync and the d2h copy.
 *   - A context is not thread-safe and owns one workspace: enqueue one
 *     context's mixer calls on one stream at a time (the reference calls
 *     its layer-forwards from one thread, gpu_inference.rs:946-948).
 *   - Mixer calls never allocate device memory once qm_reserve() has sized
 *     the workspace for the largest batch / KV length the caller will use;
 *     without it the first larger call grows the workspace (not allowed
 *     while the stream is being captured into a graph: QM_ERR_WORKSPACE).
 *     A grown-out-of workspace is kept, not freed, until qm_destroy: a graph
 *     captured before the growth still holds its address and stays valid
 *     to replay.  Graphs and eager calls of one context share the current
 *     workspace, so they must not run concurrently (one stream at a time,
 *     as above).
 *   - f16 / bf16 values are passed as uint16_t bit patterns.
 *
 * Shapes are those of Qor4bConfig::default_4b (config.rs:42-79):
 *   DeltaNet  num_qk_heads 16, num_v_heads 32, head_dim 128, conv k=4,
 *             qkv_dim 8192 = [q 2048 | k 2048 | v 4096], v_dim 4096;
 *   GQA       16 query heads, 4 kv heads, head_dim 256, rope_dim 64.
 * qm_create() rejects any other qm_config with QM_ERR_SHAPE.
 */
#ifndef QORA_MIXER_H
#define QORA_MIXER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------- */
enum {
    QM_OK = 0,
    QM_ERR_NO_DEVICE = 1,      /* no HIP device / bad device index        */
    QM_ERR_CODE_OBJECT = 2,    /* gfx950 code object missing or unusable  */
    QM_ERR_INVALID_ARG = 3,    /* null pointer, non-positive size, ...    */
    QM_ERR_SHAPE = 4,          /* dimensions other than the 4B mixer's    */
    QM_ERR_ROPE_RANGE = 5,     /* position beyond the RoPE table          */
    QM_ERR_CAPACITY = 6,       /* KV position beyond the cache capacity   */
    QM_ERR_HIP = 7,            /* HIP runtime error (launch, copy, ...)   */
    QM_ERR_OUT_OF_MEMORY = 8,
    QM_ERR_WORKSPACE = 9       /* workspace would have to grow in capture */
};

typedef struct qm_context qm_context;
typedef struct qm_graph qm_graph;
typedef struct qm_event qm_event;
typedef void* qm_stream;       /* hipStream_t */

/* Mixer dimensions, mirroring Qor4bConfig's mixer fields (config.rs:4-32). */
typedef struct {
    int32_t num_qk_heads;      /* 16  */
    int32_t num_v_heads;       /* 32  */
    int32_t dn_head_dim;       /* 128 */
    int32_t conv_kernel;       /* 4   */
    int32_t num_heads;         /* 16  */
    int32_t num_kv_heads;      /* 4   */
    int32_t attn_head_dim;     /* 256 */
    int32_t rope_dim;          /* 64 = attn_head_dim * partial_rotary_factor */
} qm_config;

/* ---- context ------------------------------------------------------ */
/* The default 4B mixer config (config.rs:42-79, rope_dim config.rs:82-85). */
void        qm_default_config(qm_config* cfg);
/* Create a context on `device`.  cfg may be NULL (default config).
 * code_object_dir holds the gfx950 code objects (qm_*.hsaco); NULL means
 * the directory libqora_mixer.so was loaded from. */
int32_t     qm_create(qm_context** ctx, const qm_config* cfg,
                      const char* code_object_dir, int32_t device);
int32_t     qm_destroy(qm_context* ctx);
const char* qm_status_string(int32_t status);
/* Detail of the last failure on ctx (or of the last qm_create failure on
 * this thread when ctx is NULL).  Valid until the next call on ctx. */
const char* qm_last_error(const qm_context* ctx);
int32_t     qm_device_count(int32_t* count);
/* Size the workspace for batches up to max_batch and KV lengths up to
 * max_kv_len (and DeltaNet and GQA prefill up to max_prefill_tokens) so
 * that later mixer calls do not allocate (e.g. under graph capture). */
int32_t     qm_reserve(qm_context* ctx, int32_t max_batch, int32_t max_kv_len,
                       int32_t max_prefill_tokens);
/* Launch-shape overrides for tests and tuning (0 = automatic).  Results do
 * not depend on them beyond fp32 reassociation. */
enum {
    QM_OPT_DN_DECODE_THREADS = 1,  /* threads per v-head workgroup: 256, 512, 1024 */
    QM_OPT_GQA_DECODE_CHUNK = 2,   /* keys per split-K workgroup (mult. 64)*/
    QM_OPT_GQA_PREFILL_ORDER = 3   /* row-block order of the causal prefill:
                                      1 longest first, 2 packed; results are
                                      bit-identical */
};
int32_t     qm_set_option(qm_context* ctx, int32_t option, int64_t value);

/* ---- device memory, streams, events, graphs (caller plumbing) ----- */
/* The reference's GPU path gets its device from the wgpu backend
 * (gpu_inference.rs:987-991) and allocates through tensor constructors
 * (GpuHybridCache::new, gpu_inference.rs:45-70); these entries are the
 * explicit HIP equivalents a caller uses to own state, KV caches and
 * streams.  qm_create / qm_reserve above play the part of that device
 * set-up. */
int32_t qm_alloc(qm_context* ctx, uint64_t bytes, void** dev);
int32_t qm_free(qm_context* ctx, void* dev);
int32_t qm_memcpy_h2d(qm_context* ctx, void* dst_dev, const void* src_host,
                      uint64_t bytes, qm_stream stream);
int32_t qm_memcpy_d2h(qm_context* ctx, void* dst_host, const void* src_dev,
                      uint64_t bytes, qm_stream stream); /* synchronous */
int32_t qm_memcpy_d2d(qm_context* ctx, void* dst_dev, const void* src_dev,
                      uint64_t bytes, qm_stream stream);
int32_t qm_memset(qm_context* ctx, void* dst_dev, int32_t byte_value,
                  uint64_t bytes, qm_stream stream);
int32_t qm_stream_create(qm_context* ctx, qm_stream* stream);
int32_t qm_stream_destroy(qm_context* ctx, qm_stream stream);
int32_t qm_sync(qm_context* ctx, qm_stream stream);
int32_t qm_event_create(qm_context* ctx, qm_event** ev);
int32_t qm_event_destroy(qm_context* ctx, qm_event* ev);
int32_t qm_event_record(qm_context* ctx, qm_event* ev, qm_stream stream);
int32_t qm_event_elapsed_ms(qm_context* ctx, qm_event* start, qm_event* stop,
                            float* ms);
/* Capture everything enqueued on `stream` between begin and end into a
 * replayable graph (amortises launch cost of per-token decode loops). */
int32_t qm_graph_begin(qm_context* ctx, qm_stream stream);
int32_t qm_graph_end(qm_context* ctx, qm_stream stream, qm_graph** graph);
int32_t qm_graph_launch(qm_context* ctx, qm_graph* graph, qm_stream stream);
int32_t qm_graph_destroy(qm_context* ctx, qm_graph* graph);

/* ---- host helpers --------------------------------------------------- */
/* RoPE tables [max_pos][rope_dim/2] in host memory, the formula of
 * convert.rs:161-176 (f32 powf/cosf/sinf); max_pos may exceed the 8192
 * rows the reference stores. */
int32_t qm_rope_table(double theta, int32_t rope_dim, int32_t max_pos,
                      float* cos_host, float* sin_host);
/* Fill `count` elements with mean + std * N(0,1) from a counter-based
 * generator (seed, element index); dtype QM_F32 / QM_F16 / QM_BF16.
 * Synthetic-data plumbing for benchmarks; not a mixer op. */
enum { QM_F32 = 0, QM_F16 = 1, QM_BF16 = 2 };
int32_t qm_fill_normal(qm_context* ctx, void* dst_dev, int32_t dtype,
                       uint64_t count, float mean, float std, uint64_t seed,
                       qm_stream stream);

/* ---- DeltaNet decode step ------------------------------------------- */
/* Replaces the mixer slice of forward_deltanet_decode, gemv.rs:744-883
 * (wgpu twin forward_deltanet_decode_gpu, gpu_inference.rs:149-227), for
 * `batch` independent sequences:
 *   [conv1d k=4 + state shift, SiLU] -> split q|k|v -> per-head L2 norm,
 *   q *= 1/sqrt(128) -> alpha = exp(-exp(A_log) softplus(a + dt_bias)),
 *   beta = sigmoid(b) -> per v-head vh (q/k head vh/2):
 *   S = alpha S; S += beta (v - S k) k^T; y = S q -> per-head RMSNorm
 *   (plain gamma, eps 1e-6) * silu(z).
 * flags: QM_DN_PREACT  qkv_dev is the raw in_proj_qkv output; conv1d+SiLU
 *                      run here and conv_buf_dev is shifted (layer mode);
 *        QM_DN_POSTACT qkv_dev is already activated; conv_buf_dev unused.
 * qkv_dev      f32 [batch][8192]
 * conv_buf_dev f32 [batch][8192][3]   (DeltaNetState.conv_buf layout)
 * conv_w_dev   f32 [8192][4]          (tap 3 multiplies the new token)
 * a_dev, b_dev f32 [batch][32]; a_log_dev, dt_bias_dev f32 [32]
 * z_dev        f32 [batch][4096]      (in_proj_z output, pre-silu)
 * norm_w_dev   f16 [128]              (attn_norm_weight)
 * state_dev    f32 [batch] x state_stride, each [32][128 v][128 k]
 *              (DeltaNetState.s layout), updated in place
 * out_dev      f32 [batch][4096]      (gated output, the out_proj input) */
enum { QM_DN_POSTACT = 0, QM_DN_PREACT = 1 };
int32_t qm_deltanet_decode(qm_context* ctx, qm_stream stream, int32_t batch,
                           int32_t flags, const float* qkv_dev,
                           float* conv_buf_dev, const float* conv_w_dev,
                           const float* a_dev, const float* b_dev,
                           const float* a_log_dev, const float* dt_bias_dev,
                           const float* z_dev, const uint16_t* norm_w_dev,
                           float* state_dev, int64_t state_stride,
                           float* out_dev);

/* ---- DeltaNet chunked prefill --------------------------------------- */
/* Replaces the sequential mixer loop of prefill_deltanet_layer,
 * gemv.rs:1119-1219 (wgpu twin prefill_deltanet_layer_gpu's host loop,
 * gpu_inference.rs:488-588, and its device<->host round trip), for one
 * sequence of seq_len tokens, computed in chunks of 64 tokens (WY/UT form)
 * with the same result as seq_len recurrent steps.
 * qkv_dev   bf16 [seq_len][8192]  raw in_proj_qkv outputs
 * conv_buf_dev f32 [8192][3] in/out; conv_w_dev f32 [8192][4]
 * a_dev, b_dev f32 [seq_len][32]; a_log_dev, dt_bias_dev f32 [32]
 * z_dev     bf16 [seq_len][4096]; norm_w_dev f16 [128]
 * state_dev f32 [32][128][128] in/out
 * out_dev   bf16 [seq_len][4096]  gated output */
int32_t qm_deltanet_prefill(qm_context* ctx, qm_stream stream, int32_t seq_len,
                            const uint16_t* qkv_dev, float* conv_buf_dev,
                            const float* conv_w_dev, const float* a_dev,
                            const float* b_dev, const float* a_log_dev,
                            const float* dt_bias_dev, const uint16_t* z_dev,
                            const uint16_t* norm_w_dev, float* state_dev,
                            uint16_t* out_dev);

/* ---- GQA decode step ------------------------------------------------- */
/* Replaces the mixer slice of forward_attn_decode, gemv.rs:927-1011
 * (wgpu twin forward_attn_decode_gpu, gpu_inference.rs:271-349):
 * split q|gate per head -> per-head RMSNorm (1+gamma) of q and k ->
 * partial RoPE (dims 0..63, pairs (i, i+32)) at position pos -> append
 * k, v to the cache at pos (f16) -> softmax(q K^T / 16) V over positions
 * 0..pos with kv head h/4 -> * sigmoid(gate).
 * q_gate_dev   f32 [batch][16][512]  interleaved [q_h | gate_h]
 * k_new_dev, v_new_dev f32 [batch][4][256]
 * q_norm_dev, k_norm_dev f16 [256]
 * rope_cos_dev, rope_sin_dev f32 [rope_len][32]
 * pos_dev      int32 [batch] positions (= cached length before the append)
 *              or NULL: every sequence is at position max_pos
 * max_pos      upper bound of the positions; must be < rope_len and
 *              < cache_capacity (else QM_ERR_ROPE_RANGE / QM_ERR_CAPACITY);
 *              device positions above it are clamped to it
 * k_cache_dev, v_cache_dev f16 [batch][4][cache_capacity][256]
 * out_dev      f32 [batch][16][256]  gated attention (the o_proj input) */
int32_t qm_gqa_decode(qm_context* ctx, qm_stream stream, int32_t batch,
                      const float* q_gate_dev, const float* k_new_dev,
                      const float* v_new_dev, const uint16_t* q_norm_dev,
                      const uint16_t* k_norm_dev, const float* rope_cos_dev,
                      const float* rope_sin_dev, int32_t rope_len,
                      const int32_t* pos_dev, int32_t max_pos,
                      uint16_t* k_cache_dev, uint16_t* v_cache_dev,
                      int64_t cache_capacity, float* out_dev);

/* qm_gqa_decode without any device allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory at call time
 * (code under HIP graph capture without a prior qm_reserve, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, kernels, launch
 * shapes and results as qm_gqa_decode, bit for bit; the split partials go to
 * a fixed 32 MiB scratch array each GPU holds for the life of the process
 * (batch x 4 x splits <= 8065, i.e. e.g. batch 64 up to ~63K positions at
 * the automatic split size), and a call that needs more is refused with
 * QM_ERR_WORKSPACE before anything is enqueued.  The first context that
 * calls it on a GPU holds that GPU's array until qm_destroy; a call from
 * any other context on the same GPU is refused with QM_ERR_WORKSPACE, since
 * two contexts' calls could overlap on the device and race in the array.
 * Calls from the holding context on different streams share it too: they
 * must not overlap in time (order them by events or synchronisation). */
int32_t qm_gqa_decode_noalloc(qm_context* ctx, qm_stream stream, int32_t batch,
                              const float* q_gate_dev, const float* k_new_dev,
                              const float* v_new_dev, const uint16_t* q_norm_dev,
                              const uint16_t* k_norm_dev, const float* rope_cos_dev,
                              const float* rope_sin_dev, int32_t rope_len,
                              const int32_t* pos_dev, int32_t max_pos,
                              uint16_t* k_cache_dev, uint16_t* v_cache_dev,
                              int64_t cache_capacity, float* out_dev);

/* ---- GQA causal prefill ---------------------------------------------- */
/* Replaces the mixer slice of prefill_attn_layer, gemv.rs:1364-1444
 * (wgpu twin prefill_attn_layer_gpu, gpu_inference.rs:679-766): per-token
 * QK RMSNorm + RoPE at positions 0..S-1, the KV cache replaced by the
 * normed/roped K and V (rows 0..S-1, f16), causal softmax attention, gate.
 * q_gate_dev bf16 [S][16][512]; k_dev, v_dev bf16 [S][4][256]
 * k_cache_dev, v_cache_dev f16 [4][cache_capacity][256] (S <= capacity)
 * out_dev bf16 [S][16][256] */
int32_t qm_gqa_prefill(qm_context* ctx, qm_stream stream, int32_t seq_len,
                       const uint16_t* q_gate_dev, const uint16_t* k_dev,
                       const uint16_t* v_dev, const uint16_t* q_norm_dev,
                       const uint16_t* k_norm_dev, const float* rope_cos_dev,
                       const float* rope_sin_dev, int32_t rope_len,
                       uint16_t* k_cache_dev, uint16_t* v_cache_dev,
                       int64_t cache_capacity, uint16_t* out_dev);

/* ---- Q4 projections --------------------------------------------------- */
/* A Q4Weight (gemv.rs:29-34, written by quantize_q4, convert.rs:437-467)
 * maps k inputs to n outputs, n a multiple of 32 (the reference stores
 * narrower matrices as f16, convert.rs:360-364; QM_ERR_SHAPE here):
 *   W[i][j] = scale[i][j/32] * (q[i][j] - 8),
 * reference layout: packed u8 [k][n/2], row i byte 16 g + t holding the
 * codes of columns 32 g + 2t (low nibble) and 32 g + 2t + 1 (high nibble);
 * scales f16 [k][n/32].
 * On the device a weight lives tile-major: codes u8 [n/T][k][T/2] and
 * gscales f16 [n/32][k], T = 8 columns when n < 4096, else 16 (each column
 * tile one contiguous stream; sizes as in the reference layout).
 * qm_q4_repack converts once at load time, as the reference's wgpu loader
 * repacks Q4 weights for its backend (q4_weight_to_gpu, gpu_loader.rs:
 * 82-106).  packed/scales/codes/gscales are device pointers. */
int32_t qm_q4_repack(qm_context* ctx, qm_stream stream, int32_t k, int32_t n,
                     const uint8_t* packed_dev, const uint16_t* scales_dev,
                     uint8_t* codes_dev, uint16_t* gscales_dev);

/* y = x W for one input row: replaces gemv_q4, gemv.rs:451-467 (inner loop
 * gemv_q4_inner :412-445, AVX-512 twin gemv_q4_avx512 simd.rs:73-139), the
 * Weight::Q4 arm of gemv() (gemv.rs:286-291) that the decode projections
 * call: in_proj_qkv/a/b/z and out_proj (gemv.rs:742,788-789,865,886),
 * q/k/v/o_proj (:928,941-942,1014) and down_proj (:895,1021).
 * x_dev f32 [k]; codes_dev, gscales_dev the repacked weight; y_dev f32 [n].
 * Sums run in fp32 in a fixed order (bit-reproducible run to run); they
 * differ from the reference's k-ordered sums by fp32 reassociation only. */
int32_t qm_q4_gemv(qm_context* ctx, qm_stream stream, int32_t k, int32_t n,
                   const float* x_dev, const uint8_t* codes_dev,
                   const uint16_t* gscales_dev, float* y_dev);

/* Up to four projections of the same input row in one launch (a launch
 * has a fixed cost of a few microseconds, comparable to streaming a
 * 2560x4096 Q4 weight), with the reference's neighbouring steps fused:
 *   norm_w_dev  NULL, or f16 [k]: x is first replaced by rms_norm(x, norm_w)
 *               (1 + gamma, eps 1e-6; gemv.rs:571-579), as the decode layers
 *               do before their input projections (gemv.rs:740, and the
 *               attention layer's equivalent) -- x_dev itself is not written;
 *   residual_dev NULL, or f32 [n]: y = residual + x W (the residual adds
 *               after out_proj / o_proj and down_proj, gemv.rs:889-890,896);
 *               may alias y_dev.
 * E.g. the four gemv() calls on x_norm at the top of the DeltaNet decode
 * (in_proj_qkv, in_proj_a, in_proj_b, in_proj_z, gemv.rs:742,788-789,865)
 * are one call with norm_w = input_norm; the three of the attention decode
 * (q/k/v_proj, gemv.rs:928,941-942) another. */
typedef struct {
    int32_t n;                   /* outputs of weight i (multiple of 32) */
    const uint8_t* codes_dev;    /* [n/T][k][T/2] */
    const uint16_t* gscales_dev; /* f16 [n/32][k] */
    float* y_dev;                /* f32 [n] */
    const float* residual_dev;   /* NULL or f32 [n] */
} qm_q4_out;
int32_t qm_q4_gemv_multi(qm_context* ctx, qm_stream stream, int32_t k,
                         const float* x_dev, const uint16_t* norm_w_dev,
                         int32_t count, const qm_q4_out* outs);

/* qm_q4_gemv_multi with the DeltaNet decode's conv1d step + SiLU fused
 * onto outs[0], the in_proj_qkv output (gemv.rs:744-772): y_0 =
 * silu(sum_{j<3} buf[c][j] w[c][j] + v w[c][3]) with v = (x W_0)[c], and
 * the buffer shifted in place (buf[c] <- {buf[c][1], buf[c][2], v}).
 * conv_buf_dev f32 [n_0][3] (oldest .. newest), conv_w_dev f32 [n_0][4];
 * outs[0] takes no residual.  qm_deltanet_decode then runs with
 * QM_DN_POSTACT (conv skipped), one launch fewer per layer than
 * QM_DN_PREACT. */
int32_t qm_q4_gemv_multi_conv(qm_context* ctx, qm_stream stream, int32_t k, const float* x_dev,
                              const uint16_t* norm_w_dev, int32_t count, const qm_q4_out* outs,
                              float* conv_buf_dev, const float* conv_w_dev);

/* The MLP's first half: out = silu(xn Wg) * (xn Wu) with xn = x, or
 * rms_norm(x, norm_w) when norm_w_dev is not NULL (replaces rms_norm +
 * fused_gate_up_q4, gemv.rs:893-894 and :469-526).  Both weights k x n,
 * device layout; out_dev f32 [n]. */
int32_t qm_q4_gate_up(qm_context* ctx, qm_stream stream, int32_t k, int32_t n,
                      const float* x_dev, const uint16_t* norm_w_dev,
                      const uint8_t* gate_codes_dev, const uint16_t* gate_gscales_dev,
                      const uint8_t* up_codes_dev, const uint16_t* up_gscales_dev,
                      float* out_dev);

/* ---- Q4 projections for prefill (seq_len > 1) ------------------------- */
/* The f16 input of qm_q4_gemm: each of the m rows of x_dev (f32 [m][k]) as
 * rms_norm(row, norm_w) (1 + gamma, eps 1e-6; gemv.rs:571-579), or simply
 * converted when norm_w_dev is NULL.  out_dev f16 [m][k]; k % 4 == 0. */
int32_t qm_rms_norm_f16(qm_context* ctx, qm_stream stream, int32_t m, int32_t k,
                        const float* x_dev, const uint16_t* norm_w_dev,
                        uint16_t* out_dev);

/* y = x W (+ residual) for m input rows on MFMA: replaces gemm_q4,
 * gemv.rs:529-542 (gemm() on a Q4 weight, :295-300), which the prefill
 * layers call for every projection (gemv.rs:1114-1117,1222,1231-1239,
 * 1366-1385,1447-1467).  x_dev [m][k] (k % 32 == 0, else QM_ERR_SHAPE) of
 * x_dtype QM_F16 (from qm_rms_norm_f16) or QM_BF16 (a mixer prefill output
 * or the MLP's silu(g) * u); codes_dev/gscales_dev a weight in the device
 * layout (qm_q4_repack); residual_dev NULL or f32 [m][n] (may alias y_dev);
 * exactly one of y_dev (f32 [m][n]) and y_bf16_dev (bf16 [m][n], e.g. the
 * in_proj_qkv / in_proj_z outputs that qm_deltanet_prefill reads) is
 * non-NULL.  Products accumulate in fp32.  An f16 x multiplies W rounded to
 * f16 per element (s * (q - 8), one rounding): within 1e-3 of
 * sum_k |x_k W_kj| of the fp32 reference per element.  A bf16 x is used as
 * it is (bf16's range: outliers stay finite) and multiplies W rounded on to
 * bf16: within 2^-8 + 2^-11 (+ the fp32 accumulation) of that sum. */
int32_t qm_q4_gemm(qm_context* ctx, qm_stream stream, int32_t m, int32_t k, int32_t n,
                   const uint16_t* x_dev, int32_t x_dtype, const uint8_t* codes_dev,
                   const uint16_t* gscales_dev, const float* residual_dev,
                   float* y_dev, uint16_t* y_bf16_dev);

/* The prefill MLP's gate and up projections and their SiLU product
 * (gemv.rs:1231-1237: gemm(gate_proj), gemm(up_proj), then
 * silu(g) * u per element) in one launch: out_dev bf16 [m][n] =
 * bf16(silu(x Wg) * (x Wu)), the input of the down_proj qm_q4_gemm
 * (x_dtype QM_BF16).  bf16 holds any product of the fp32 accumulators (the
 * reference keeps this intermediate in f32, gemv.rs:469-526), so outlier
 * activations stay finite.  Both weights are k x n in the device layout; x
 * as for qm_q4_gemm. */
int32_t qm_q4_gemm_gate_up(qm_context* ctx, qm_stream stream, int32_t m, int32_t k, int32_t n,
                           const uint16_t* x_dev, int32_t x_dtype,
                           const uint8_t* gate_codes_dev, const uint16_t* gate_gscales_dev,
                           const uint8_t* up_codes_dev, const uint16_t* up_gscales_dev,
                           uint16_t* out_dev);

/* ---- vocabulary side of a step: embedding lookup and lm_head ---------- */
/* The embedding (tied to lm_head) stays in the reference layout, a
 * Q4Weight with k = vocab rows and n = hidden columns
 * (write_embedding_weight, convert.rs:390-415): packed_dev u8
 * [vocab][hidden/2], scales_dev f16 [vocab][hidden/32]. */

/* logits_dev f32 [vocab] = rms_norm(x, final_norm) . row v for every v:
 * replaces the final rms_norm + lm_head_parallel (Q4 arm, gemv.rs:678-708;
 * called at gemv.rs:1074-1076, 1280-1282), which the reference's wgpu path
 * keeps on the CPU (lm_head_cpu, gpu_inference.rs:425-427,818-842).
 * x_dev f32 [hidden] (hidden % 512 == 0, at most 8192, else QM_ERR_SHAPE);
 * norm_w_dev f16 [hidden], the (1 + gamma) final norm, or NULL for none.
 * fp32 throughout: within 1e-5 of sum_j |xn_j W_vj| of the reference. */
int32_t qm_q4_lm_head(qm_context* ctx, qm_stream stream, int32_t vocab, int32_t hidden,
                      const float* x_dev, const uint16_t* norm_w_dev,
                      const uint8_t* packed_dev, const uint16_t* scales_dev,
                      float* logits_dev);

/* out_dev f32 [count][hidden] = the embedding rows of ids_dev [count]
 * (embed_lookup_q4, gemv.rs:544-563; used at gemv.rs:1040,1063,1260):
 * bit-identical to the reference's rows.  An id outside [0, vocab), a
 * slice-index panic in the reference, yields a row of NaN. */
int32_t qm_q4_embed(qm_context* ctx, qm_stream stream, int32_t count, int32_t vocab,
                    int32_t hidden, const int32_t* ids_dev, const uint8_t* packed_dev,
                    const uint16_t* scales_dev, float* out_dev);

/* ---- next-token sampling ------------------------------------------------ */
/* The sampling settings of GenerateParams (generate.rs:9-21) plus the
 * per-step choices of the decode loop (generate.rs:185-198). */
enum { QM_SAMPLE_WGPU = 1 };  /* follow the wgpu path's sample_token_top_k,
                                 gpu_inference.rs:867-906: probabilities
                                 divided by the sum, no zero-sum exits,
                                 greedy keeps the last of equal maxima */
typedef struct qm_sample_params {
    float temperature;         /* <= 0: greedy (the top_k etc. are unused) */
    float top_p;
    int32_t top_k;             /* 1 .. 1024 when sampling */
    float repetition_penalty;  /* applied when > 1 (last 64 ids) */
    float presence_penalty;    /* applied when > 0, once per distinct id */
    int32_t banned_id;         /* set to -inf after the penalties, or -1
                                  (the EOS ban inside a think block,
                                  generate.rs:191) */
    int32_t flags;             /* 0 or QM_SAMPLE_WGPU */
} qm_sample_params;

/* Next token from logits_dev f32 [vocab], on the device: replaces
 * apply_repetition_penalty + apply_presence_penalty (generate.rs:58-82,
 * applied in place to logits_dev as the reference mutates its logits) and
 * sample_token_top_k (generate.rs:334-384), so the logits need not be
 * copied to the host.  generated_dev int32 [n_generated] (oldest first);
 * rng_state_dev the Rng's xorshift64 state (generate.rs:41-55), advanced
 * exactly when the reference draws.  token_out_dev int32 [1].  Optional
 * top_ids_dev int32 [k] / top_probs_dev f32 [k] receive the sorted top-k
 * ids and their probabilities.  Given the same logits and state, the token
 * and the new state equal the reference's (the one difference: exp is the
 * correctly rounded one, libm's expf can differ by one ulp in rare cases).
 * Logits must not be NaN (the reference's sort has no defined order for
 * them).  top_k = 0 (all logits) is not supported: QM_ERR_INVALID_ARG;
 * vocab at most 262144 (QM_ERR_SHAPE).  Uses 64 KB of the context's
 * workspace (reserved by qm_reserve). */
int32_t qm_sample(qm_context* ctx, qm_stream stream, int32_t vocab, float* logits_dev,
                  const int32_t* generated_dev, int32_t n_generated,
                  const qm_sample_params* params, uint64_t* rng_state_dev,
                  int32_t* token_out_dev, int32_t* top_ids_dev, float* top_probs_dev);

#ifdef __cplusplus
}
#endif
#endif /* QORA_MIXER_H */
