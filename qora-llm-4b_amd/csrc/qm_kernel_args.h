// qm_kernel_args.h -- argument blocks passed by value to the gfx950 kernels.
// Shared by the host runtime (g++) and the device code (hipcc --genco), so
// it uses only fixed-width integer and pointer members.
#pragma once
#include <stdint.h>

// Mixer shape (Qor4bConfig::default_4b, config.rs:42-97).
#define QM_DN_QK_HEADS   16
#define QM_DN_V_HEADS    32
#define QM_DN_HD         128
#define QM_DN_CONV_K     4
#define QM_DN_QKV_DIM    8192      // 2*16*128 + 32*128
#define QM_DN_QK_DIM     2048      // 16*128: q (and k) part of qkv
#define QM_DN_V_DIM      4096
#define QM_DN_HEAD_ELEMS 16384     // 128*128 state floats per v-head
#define QM_GQA_HEADS     16
#define QM_GQA_KV_HEADS  4
#define QM_GQA_HD        256
#define QM_GQA_ROT       64
#define QM_GQA_GROUP     4         // query heads per kv head

// Causal conv1d + SiLU pre-pass of the layer-mode DeltaNet decode step.
struct DnConvArgs {
    const float* qkv;        // [B][8192] raw projection
    float* conv_buf;         // [B][8192][3]
    const float* conv_w;     // [8192][4]
    float* act;              // [B][8192] activated output
    int32_t batch;
};

// DeltaNet decode step on activated inputs.
struct DnDecodeArgs {
    const float* act;        // [B][8192] activated q|k|v (q,k not yet L2-normed)
    const float* a;          // [B][32]
    const float* b;          // [B][32]
    const float* a_log;      // [32]
    const float* dt_bias;    // [32]
    const float* z;          // [B][4096]
    const uint16_t* norm_w;  // [128] f16
    float* state;            // [B] x state_stride floats
    int64_t state_stride;
    float* out;              // [B][4096]
    int32_t batch;
};

// GQA decode step (split-K attention with fused q/k prep, then merge).
struct GqaDecodeArgs {
    const float* q_gate;     // [B][16][512]
    const float* k_new;      // [B][4][256]
    const float* v_new;      // [B][4][256]
    const uint16_t* q_norm;  // [256] f16
    const uint16_t* k_norm;  // [256] f16
    const float* rope_cos;   // [rope_len][32]
    const float* rope_sin;
    const int32_t* pos;      // [B] or null
    uint16_t* k_cache;       // [B][4][cap][256] f16
    uint16_t* v_cache;
    float* out;              // [B][16][256]
    float* partial;          // [B][4][nsplit][4 heads][260]: acc[256], m, l, pad
    int64_t cap;
    int32_t max_pos;
    int32_t chunk;           // keys per split
    int32_t nsplit;          // splits per (b, kv head)
    int32_t batch;
};

// DeltaNet chunked prefill (chunk 64).  Workspace tensors, per (v-head,
// chunk) block, nc = ceil(T / 64):
//   Wn, Qt  f16 [32][nc][8192]     -W = -T diag(beta*gamma) K and
//                                   Q~ = diag(gamma) Q - P W
//   Ut, Y0t f16 [32][nc][8192]     U~ = T diag(beta) V and Y0 = P U~
//   Ktt     f16 [16][nc][8192]     K^T per qk-head (normalised keys)
//   Dt      f32 [32][nc][64]       gamma_C / gamma_t per token
//   gC      f32 [32][nc]           gamma_C = prod of the chunk's decays
//   Yt      f16 [32][nc][8][64][16] pre-norm outputs of the chunked path,
//                                   per 16-row slice, token-major
// The other per-(head, chunk) blocks are stored in the MFMA fragment order
// the scan kernel loads them in (described there).
#define QM_DN_CHUNK 64
#define QM_DN_CHUNK_THREADS 256   // chunk kernel: one 4-wave workgroup per (chunk, qk-head)
struct DnPrefillArgs {
    const uint16_t* qkv;     // bf16 [T][8192]
    float* conv_buf;         // [8192][3]
    const float* conv_w;     // [8192][4]
    const float* a;          // [T][32]
    const float* b;          // [T][32]
    const float* a_log;      // [32]
    const float* dt_bias;    // [32]
    const uint16_t* z;       // bf16 [T][4096]
    const uint16_t* norm_w;  // f16 [128]
    float* state;            // [32][128][128]
    uint16_t* out;           // bf16 [T][4096]
    uint16_t* Wn;
    uint16_t* Qt;
    uint16_t* Ut;
    uint16_t* Y0t;
    uint16_t* Ktt;
    float* Dt;
    float* gC;
    // the scan's outputs Y (pre-norm) in f16, per (v-head, chunk) 8 slices x
    // 4 token tiles x 64 lanes x 4 tokens (fragment order)
    uint16_t* Yt;
    // pre-norm outputs of slices run exactly: per (v-head, chunk) 32 KB, the
    // 4 KB at 4096 * slice holding f32 [64 tokens][16 rows]
    float* Yx;
    // Precision guard: vstat f32 [32][nc + 1][128] holds, per (v-head,
    // chunk), each v channel's max |v| after conv1d + SiLU (+inf in entry 0
    // if any f16 operand of that chunk would overflow); slot nc holds the
    // entering state's row maxima.  mode int32 [32][8]: per (v-head, 16-row
    // slice) 0 = chunked f16 path (outputs in Yt), 1 = exact fp32 recurrence
    // (outputs in Yx).
    float* vstat;
    int32_t* mode;
    int32_t T;
    int32_t nc;
};

// GQA causal prefill.  kvf is a workspace copy of the f16 K and V, per kv
// head and 64-key tile (s_pad = S rounded up to 64, zero padded), in the
// attention's MFMA fragment order: f16 [4][s_pad / 64][64 blocks][64 lanes][8],
// blocks 0..31 K, 32..63 V transposed.
struct GqaPrefillArgs {
    const uint16_t* q_gate;  // bf16 [S][16][512]
    const uint16_t* k;       // bf16 [S][4][256]
    const uint16_t* v;       // bf16 [S][4][256]
    const uint16_t* q_norm;  // f16 [256]
    const uint16_t* k_norm;  // f16 [256]
    const float* rope_cos;   // [rope_len][32]
    const float* rope_sin;
    uint16_t* k_cache;       // f16 [4][cap][256]
    uint16_t* v_cache;
    uint16_t* kvf;           // f16 [4][s_pad / 64][64][64][8]
    uint16_t* out;           // bf16 [S][16][256]
    int32_t* queue;          // [4] next row block per kv head (zeroed by the kv kernel)
    int64_t cap;
    int32_t S;
    int32_t s_pad;
};

// The attention kernel's arguments: the shared ones plus the order in which
// each kv group's queue hands out its 48-row blocks (block 0 = rows 0..47).
// ordered = 0: the n-th draw is the n-th longest block (nblk - 1 - n).
#define QM_GQA_PREFILL_ORDER_MAX 1024
struct GqaPrefillAttnArgs {
    GqaPrefillArgs a;
    int32_t ordered;
    uint16_t order[QM_GQA_PREFILL_ORDER_MAX];
};

// Q4 GEMV (one input row) on the tile-major device layout, for up to
// QM_Q4_MAX_OUT weights sharing x: one workgroup per column tile, weight p
// taking workgroups wstart[p] .. wstart[p+1]-1 with tiles of tile[p]
// columns.  The gate/up kernel takes gate = weight 0, up = weight 1 (same
// shape), y[0] = silu(x Wg) * (x Wu).
#define QM_Q4_MAX_OUT 4
// Column-tile width of the device layout of a weight with n outputs.
#define QM_Q4_TILE(n) ((n) < 4096 ? 8 : 16)
struct Q4GemvArgs {
    const float* x;                        // [k]
    const uint16_t* norm_w;                // null, or f16 [k]: x <- rms_norm(x, 1 + norm_w)
    const uint8_t* codes[QM_Q4_MAX_OUT];   // [n_p/T][k][T/2]
    const uint16_t* gscales[QM_Q4_MAX_OUT];// f16 [n_p/32][k]
    float* y[QM_Q4_MAX_OUT];               // [n_p]
    const float* residual[QM_Q4_MAX_OUT];  // null, or f32 [n_p]: y = residual + x W
    int32_t tile[QM_Q4_MAX_OUT];           // T of weight p (8 or 16)
    int32_t wstart[QM_Q4_MAX_OUT + 1];
    int32_t k;
    int32_t count;
    float* conv_buf;                       // null, or f32 [n_0][3]: y_0 <- silu(conv1d(y_0)), buffer shifted
    const float* conv_w;                   // f32 [n_0][4]
};

// Reference Q4Weight layout -> tile-major device layout.
struct Q4RepackArgs {
    const uint8_t* packed;   // [k][n/2]
    const uint16_t* scales;  // f16 [k][n/32]
    uint8_t* codes;          // [n/T][k][T/2]
    uint16_t* gscales;       // f16 [n/32][k]
    int32_t k;
    int32_t n;
    int32_t tile;            // T = QM_Q4_TILE(n)
};

// Q4 prefill GEMM: y[m][n] = x[m][k] W (+ residual), x f16 or bf16, W in
// the device layout; output f32 (y) or bf16 (y_bf16 non-null).  The gate/up
// form reads two weights (codes/gscales the gate, codes2/gscales2 the up
// weight) and writes y_bf16 = silu(x Wg) * (x Wu).  k % 32 == 0.
struct Q4GemmArgs {
    const uint16_t* x;       // f16 or bf16 [m][k]
    const uint8_t* codes;    // [n/T][k][T/2]
    const uint16_t* gscales; // f16 [n/32][k]
    const uint8_t* codes2;   // gate/up form: the up weight
    const uint16_t* gscales2;
    float* y;                // f32 [m][n]
    uint16_t* y_bf16;        // or bf16 [m][n] (the gate/up form's output)
    const float* residual;   // null, or f32 [m][n]
    int32_t m;
    int32_t k;
    int32_t n;
    int32_t tile;            // QM_Q4_TILE(n)
};

// lm_head on the vocab-major Q4 embedding: logits[v] = (rms_norm(x) or x) . row v.
struct LmHeadArgs {
    const float* x;          // f32 [k]
    const uint16_t* norm_w;  // null or f16 [k] (1 + gamma)
    const uint8_t* codes;    // [vocab][k/2]
    const uint16_t* scales;  // f16 [vocab][k/32]
    float* logits;           // f32 [vocab]
    int32_t vocab;
    int32_t k;               // % 512 == 0, <= 8192
};

// Embedding rows of count token ids, dequantized to f32.
struct EmbedArgs {
    const int32_t* ids;      // [count]
    const uint8_t* codes;    // [vocab][k/2]
    const uint16_t* scales;  // f16 [vocab][k/32]
    float* out;              // f32 [count][k]
    int32_t vocab;
    int32_t k;               // % 32 == 0
};

// Next-token sampling (one workgroup per kernel).
#define QMK_SAMPLE_WGPU 1          // follow gpu_inference.rs:867-906 instead of generate.rs:334-384
struct SampleArgs {
    float* logits;            // [vocab]; the penalties are applied in place
    const int32_t* generated; // [n_generated] ids generated so far, oldest first
    uint64_t* rng_state;      // xorshift64 state, advanced when a draw is made
    int32_t* token_out;       // [1]
    int32_t* top_ids;         // null, or [k] the sorted top-k ids
    float* top_probs;         // null, or [k] their probabilities after the softmax
    int32_t vocab;
    int32_t n_generated;
    int32_t top_k;            // 1 .. 1024 (ignored when greedy)
    int32_t banned;           // id set to -inf after the penalties, or -1
    int32_t flags;
    float temperature;        // <= 0: greedy
    float top_p;
    float repetition_penalty; // applied when > 1
    float presence_penalty;   // applied when > 0
    uint64_t* cand;           // workspace: [n_cand] stage-1 candidates
    int32_t chunk;            // vocabulary slice per stage-1 workgroup (multiple of 256)
    int32_t n_cand;           // slices x k (<= 8192)
};

// Per-row RMSNorm (or plain conversion) of f32 [m][k] into f16.
struct RmsNormArgs {
    const float* x;          // [m][k]
    const uint16_t* norm_w;  // null or f16 [k]
    uint16_t* out;           // f16 [m][k]
    int32_t m;
    int32_t k;
};

// Counter-based normal generator fill.
struct FillArgs {
    void* dst;
    uint64_t count;
    uint64_t seed;
    float mean;
    float stdev;
    int32_t dtype;
};
