// sample.hip -- next-token sampling on the device for gfx950: penalties,
// top-k, temperature softmax, top-p and the xorshift64 draw, so that the
// logits never leave HBM (generate.rs:58-82,334-384; the wgpu path's twin,
// gpu_inference.rs:867-931).
//
// qm_sample_penalties (one workgroup): the repetition penalty over the last
// 64 generated ids in order (repeats apply again, as the reference's loop
// does), the presence penalty once per distinct generated id, then an
// optional banned id set to -inf (generate.rs:189-195).
//
// The top k of the reference's stable descending sort (logit desc, index
// asc) without sorting the vocabulary:
//   qm_sample_select: each workgroup finds the first k of its slice of the
//      vocabulary by a radix select over an order-preserving 32-bit key (-0
//      folded onto +0, which compare equal in the reference's sort; NaN
//      below -inf): four 8-bit digits, LDS histograms with integer atomics
//      (order-independent), then every key above the threshold and, of the
//      keys equal to it, the lowest indices (a block scan of the per-thread
//      counts makes that choice deterministic).
//      The slice's candidates are sorted (bitonic, in LDS).
//   qm_sample_top_k (one workgroup of 1024 threads): merge of the slices'
//      sorted lists up to k elements; then the reference's sequential f32
//      arithmetic on one thread: the softmax sum, the top-p cutoff, the
//      total and the cumulative draw, in the reference's order and rounding
//      (contraction off in these kernels).  exp is taken in double and rounded to f32 (the
//      reference calls libm expf, correctly rounded but for rare half-way
//      cases).
// Greedy (temperature <= 0) is the same selection with k = 1.
#include "qm_device.h"
#include "qm_kernel_args.h"

#define SMP_THREADS 1024
#define SMP_MAX_K 1024
#define SMP_MAX_CAND 8192          // stage-1 candidates (slices x k), merged in LDS
#define SMP_MAX_LISTS 256          // stage-1 slices (vocabulary / 1024 at most)
#define SMP_MAX_VOCAB 262144       // the presence bitmap in LDS (32 KB)

// Larger logit -> larger key; -0 == +0; NaN below every number.
QM_DEV uint32_t logit_key(float v) {
    uint32_t u = __float_as_uint(v);
    if (v != v) return 0u;
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

QM_DEV float key_logit(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

extern "C" __global__ __launch_bounds__(SMP_THREADS) void qm_sample_penalties(SampleArgs A) {
#pragma clang fp contract(off)
    __shared__ uint32_t seen[(SMP_MAX_VOCAB + 31) / 32];
    const int tid = threadIdx.x;
    const int n = A.n_generated;
    // generate.rs:58-69
    if (A.repetition_penalty > 1.0f && tid == 0) {
        const int window = min(n, 64);
        for (int i = n - window; i < n; ++i) {
            const int tok = A.generated[i];
            if (tok < 0 || tok >= A.vocab) continue;
            const float l = A.logits[tok];
            A.logits[tok] = l > 0.0f ? __fdiv_rn(l, A.repetition_penalty) : __fmul_rn(l, A.repetition_penalty);
        }
    }
    // generate.rs:72-82: once per distinct id, by the thread whose bit-set
    // in an LDS bitmap of the vocabulary finds the bit clear
    const bool presence = A.presence_penalty > 0.0f && n > 0;
    if (presence)
        for (int i = tid; i < (A.vocab + 31) / 32; i += SMP_THREADS) seen[i] = 0u;
    __syncthreads();
    if (presence) {
        for (int i = tid; i < n; i += SMP_THREADS) {
            const int tok = A.generated[i];
            if (tok < 0 || tok >= A.vocab) continue;
            const uint32_t bit = 1u << (tok & 31);
            if (!(atomicOr(&seen[tok >> 5], bit) & bit)) A.logits[tok] = __fsub_rn(A.logits[tok], A.presence_penalty);
        }
    }
    __syncthreads();
    if (tid == 0 && A.banned >= 0 && A.banned < A.vocab) A.logits[A.banned] = -__builtin_inff();
}

// Candidate order: key descending, then index ascending (descending for
// tie_last).  Zero sorts last.
QM_DEV uint64_t cand_pack(uint32_t key, int i, bool tie_last) {
    return ((uint64_t)key << 32) | (tie_last ? (uint32_t)i : 0xffffffffu - (uint32_t)i);
}
QM_DEV int32_t cand_id(uint64_t c, bool tie_last) {
    return tie_last ? (int32_t)(uint32_t)c : (int32_t)(0xffffffffu - (uint32_t)c);
}

// The radix digit of one pass, by wave 0: the largest d with
// sum(hist[e], e > d) + hist[d] >= rank.  Lane l holds bins 4l .. 4l + 3;
// suffix sums over lanes by shuffles.  Writes the digit and the count above
// it to out[0], out[1].
QM_DEV void radix_pick(const uint32_t* hist, uint32_t rank, uint32_t* out) {
    const int l = threadIdx.x;
    uint32_t h[4], s = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) s += (h[b] = hist[4 * l + b]);
    uint32_t incl = s;                     // sum over lanes >= l
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t v = __shfl_down(incl, off);
        if (l + off < 64) incl += v;
    }
    uint32_t above = incl - s;             // bins of the lanes above this one
    int found = -1;
    uint32_t found_above = 0;
#pragma unroll
    for (int b = 3; b >= 0; --b) {
        if (found < 0 && above + h[b] >= rank) {
            found = 4 * l + b;
            found_above = above;
        }
        above += h[b];
    }
    const uint64_t any = __ballot(found >= 0);
    const int top = 63 - __builtin_clzll(any);   // the highest lane holding the answer
    if (l == top) {
        out[0] = (uint32_t)found;
        out[1] = found_above;
    }
}

// Radix select over the keys logit_key(x[lo .. hi)) of the workgroup's
// threads: the key of the rank0-th largest, and how many keys equal to it
// are within the top rank0.
QM_DEV void radix_select(const float* x, int lo, int hi, uint32_t rank0, uint32_t* hist, uint32_t* pick,
                         uint32_t& prefix, uint32_t& rank) {
    const int tid = threadIdx.x;
    uint32_t mask = 0;
    prefix = 0;
    rank = rank0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += blockDim.x) hist[i] = 0;
        __syncthreads();
        for (int i = lo; i < hi; ++i) {
            const uint32_t key = logit_key(x[i]);
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 64) radix_pick(hist, rank, pick);
        __syncthreads();
        prefix |= pick[0] << shift;
        rank -= pick[1];
        mask |= 255u << shift;
        __syncthreads();
    }
}

// In-place bitonic sort of c[0 .. P) (P a power of two), descending.
QM_DEV void bitonic_desc(uint64_t* c, int P) {
    for (int size = 2; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < P; i += blockDim.x) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0;
                    const uint64_t a = c[i], b = c[j];
                    if (desc ? a < b : a > b) {
                        c[i] = b;
                        c[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// Stage 1: workgroup w (256 threads) takes the slice [w CH, (w + 1) CH) of
// the vocabulary, thread t the contiguous elements t * per .. + per - 1 of
// it, and writes the slice's first min(k, slice length) elements of the
// global order, sorted, to cand[w k ..] (zeros after them).  Every element
// of the global top k is among its slice's top k.
extern "C" __global__ __launch_bounds__(256) void qm_sample_select(SampleArgs A) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t scan[256];
    __shared__ uint32_t pick[2], ncand;
    __shared__ uint64_t loc[SMP_MAX_K];
    const int tid = threadIdx.x, w = blockIdx.x;
    const int V = A.vocab;
    const bool greedy = !(A.temperature > 0.0f);
    const int k = greedy ? 1 : min(A.top_k, V);
    const bool tie_last = greedy && (A.flags & QMK_SAMPLE_WGPU);
    const int per = A.chunk / 256;
    const int s0 = w * A.chunk, s1 = min(s0 + A.chunk, V);
    const int lo = min(s0 + tid * per, s1), hi = min(lo + per, s1);
    const int kk = min(k, s1 - s0);

    uint32_t prefix, rank;
    radix_select(A.logits, lo, hi, (uint32_t)kk, hist, pick, prefix, rank);
    // keys above the threshold, then `rank` of the equal keys in index order
    // (reversed for tie_last), ranked by a block scan of per-thread counts
    uint32_t eq = 0;
    for (int i = lo; i < hi; ++i) eq += logit_key(A.logits[i]) == prefix;
    scan[tid] = eq;
    if (tid == 0) ncand = 0;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const uint32_t v = tid >= off ? scan[tid - off] : 0u;
        __syncthreads();
        scan[tid] += v;
        __syncthreads();
    }
    uint32_t before = tie_last ? scan[255] - scan[tid] : scan[tid] - eq;
    for (int j = 0; j < hi - lo; ++j) {
        const int i = tie_last ? hi - 1 - j : lo + j;
        const uint32_t key = logit_key(A.logits[i]);
        bool take = key > prefix;
        if (key == prefix) take = before++ < rank;
        if (take) {
            const uint32_t slot = atomicAdd(&ncand, 1u);
            if (slot < (uint32_t)kk) loc[slot] = cand_pack(key, i, tie_last);
        }
    }
    int P = 1;
    while (P < k) P <<= 1;
    __syncthreads();
    for (int i = kk + tid; i < P; i += 256) loc[i] = 0;
    __syncthreads();
    bitonic_desc(loc, P);
    uint64_t* out = A.cand + (size_t)w * k;
    for (int i = tid; i < k; i += 256) out[i] = loc[i];
}

// Stage 2 (one workgroup): merge the slices' sorted lists into the first k
// of the global order (wave 0 repeatedly takes the largest list head), and
// draw.
extern "C" __global__ __launch_bounds__(SMP_THREADS) void qm_sample_top_k(SampleArgs A) {
#pragma clang fp contract(off)
    __shared__ uint64_t cand[SMP_MAX_CAND];
    __shared__ uint64_t top[SMP_MAX_K];
    __shared__ float prob[SMP_MAX_K];
    __shared__ float sh_sum;

    const int tid = threadIdx.x;
    const int V = A.vocab;
    const bool greedy = !(A.temperature > 0.0f);
    const int k = greedy ? 1 : min(A.top_k, V);
    const bool tie_last = greedy && (A.flags & QMK_SAMPLE_WGPU);
    const int n = A.n_cand, nl = n / k;    // lists of k
    for (int i = tid; i < n; i += SMP_THREADS) cand[i] = A.cand[i];
    __syncthreads();
    if (tid < 64) {
        // lane l owns lists l, l + 64, ... (at most SMP_MAX_LISTS / 64)
        int head[SMP_MAX_LISTS / 64];
        uint64_t hv[SMP_MAX_LISTS / 64];     // current head values; 0 when exhausted
#pragma unroll
        for (int j = 0; j < SMP_MAX_LISTS / 64; ++j) {
            const int list = tid + 64 * j;
            head[j] = 0;
            hv[j] = list < nl ? cand[list * k] : 0;
        }
        for (int r = 0; r < k; ++r) {
            uint64_t best = hv[0];
            int best_j = 0;
#pragma unroll
            for (int j = 1; j < SMP_MAX_LISTS / 64; ++j)
                if (hv[j] > best) {
                    best = hv[j];
                    best_j = j;
                }
            uint64_t m = best;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const uint64_t o = __shfl_xor(m, off);
                m = o > m ? o : m;
            }
            // non-zero composites are distinct; the lowest lane holding the
            // maximum advances that list
            const uint64_t holders = __ballot(best == m);
            if (tid == __builtin_ctzll(holders)) {
#pragma unroll
                for (int j = 0; j < SMP_MAX_LISTS / 64; ++j)
                    if (j == best_j) {
                        const int list = tid + 64 * j;
                        head[j]++;
                        hv[j] = head[j] < k ? cand[list * k + head[j]] : 0;
                    }
            }
            if (tid == 0) top[r] = m;
        }
    }
    __syncthreads();
    if (A.top_ids && tid < k) A.top_ids[tid] = cand_id(top[tid], tie_last);
    if (greedy) {                      // generate.rs:335-342 (first maximum; last for the wgpu twin)
        if (tid == 0) A.token_out[0] = cand_id(top[0], tie_last);
        return;
    }

    // generate.rs:345-383 (the wgpu twin, gpu_inference.rs:874-905,
    // divides by the sum instead of multiplying by its inverse and has no
    // zero-sum exits)
    const float inv_temp = __fdiv_rn(1.0f, A.temperature);
    const float max_logit = key_logit((uint32_t)(top[0] >> 32));
    if (tid < k) {
        const float l = key_logit((uint32_t)(top[tid] >> 32));
        prob[tid] = (float)exp((double)__fmul_rn(__fsub_rn(l, max_logit), inv_temp));
    }
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int i = 0; i < k; ++i) sum = __fadd_rn(sum, prob[i]);
        sh_sum = sum;
    }
    __syncthreads();
    const float sum = sh_sum;
    const bool wgpu = A.flags & QMK_SAMPLE_WGPU;
    if (!wgpu && sum <= 0.0f) {
        if (tid == 0) A.token_out[0] = cand_id(top[0], false);
        return;
    }
    if (tid < k) prob[tid] = wgpu ? __fdiv_rn(prob[tid], sum) : __fmul_rn(prob[tid], __fdiv_rn(1.0f, sum));
    __syncthreads();
    if (A.top_probs && tid < k) A.top_probs[tid] = prob[tid];
    if (tid != 0) return;
    float cumsum = 0.0f;
    int cutoff = k;
    for (int i = 0; i < k; ++i) {
        cumsum = __fadd_rn(cumsum, prob[i]);
        if (cumsum >= A.top_p) {
            cutoff = i + 1;
            break;
        }
    }
    float total = 0.0f;
    for (int i = 0; i < cutoff; ++i) total = __fadd_rn(total, prob[i]);
    if (!wgpu && total <= 0.0f) {
        A.token_out[0] = cand_id(top[0], false);
        return;
    }
    // Rng::next_f32, generate.rs:46-54
    uint64_t s = A.rng_state[0];
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    A.rng_state[0] = s;
    const float rand_val = __fmul_rn((float)(uint32_t)(s >> 40) / 16777216.0f, total);
    float accum = 0.0f;
    int32_t tok = cand_id(top[0], false);
    for (int i = 0; i < cutoff; ++i) {
        accum = __fadd_rn(accum, prob[i]);
        if (accum >= rand_val) {
            tok = cand_id(top[i], false);
            break;
        }
    }
    A.token_out[0] = tok;
}
