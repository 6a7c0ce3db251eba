// qm_runtime.cpp -- host side of libqora_mixer.so (the C ABI in
// include/qora_mixer.h).
//
// Loads the gfx950 code objects (qm_*.hsaco) with hipModuleLoad, validates
// every argument before anything is enqueued (so bad shapes, positions and
// null pointers come back as status codes instead of faults), picks launch
// shapes and enqueues the kernels with hipModuleLaunchKernel.  Device memory
// for the mixer's own scratch (split-K partials, the activated qkv of
// layer-mode decode) lives in a per-context workspace that only grows
// outside stream capture.
#include "qora_mixer.h"
#include "qm_kernel_args.h"
#include "qm_gqa_plan.h"
#include "qm_noalloc.h"

#include <hip/hip_runtime_api.h>
#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <initializer_list>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace {

thread_local std::string g_create_error;

}  // namespace

struct qm_context {
    int device = 0;
    qm_config cfg{};
    hipStream_t stream = nullptr;
    std::vector<hipModule_t> modules;
    hipFunction_t f_conv = nullptr;
    hipFunction_t f_dn[3] = {nullptr, nullptr, nullptr};  // 256, 512, 1024 threads
    hipFunction_t f_gqa_split[5] = {};      // 4 .. 8 waves per workgroup
    hipFunction_t f_gqa_merge = nullptr;
    hipFunction_t f_fill = nullptr;
    hipFunction_t f_dnp_chunk = nullptr;
    hipFunction_t f_dnp_scan = nullptr;
    hipFunction_t f_dnp_out = nullptr;
    hipFunction_t f_gqp_kv = nullptr;
    hipFunction_t f_gqp_attn = nullptr;
    hipFunction_t f_q4_gemv = nullptr;
    hipFunction_t f_q4_gemv_hidden = nullptr;  // k <= 2560 (the hidden size)
    hipFunction_t f_q4_gemv_inter = nullptr;   // 4096 < k <= 9216 (the MLP's intermediate size)
    hipFunction_t f_q4_repack = nullptr;
    hipFunction_t f_q4_gate_up = nullptr;
    hipFunction_t f_q4_gemm[2][2] = {};  // [x bf16][gate/up form]
    hipFunction_t f_q4_gemm_n128[2] = {}; // [x bf16]: 128 x 128 tiles for narrow outputs
    hipFunction_t f_q4_gemm_m64[2] = {};  // [x bf16]: 64 x 128 tiles
    hipFunction_t f_q4_gemm_n32[2] = {};  // [x bf16]: n = 32, 16 rows per 4-wave workgroup, k split over the waves
    hipFunction_t f_rms_f16 = nullptr;
    hipFunction_t f_lm_head = nullptr;
    hipFunction_t f_embed = nullptr;
    hipFunction_t f_sample_pen = nullptr;
    hipFunction_t f_sample = nullptr;
    hipFunction_t f_sample_select = nullptr;
    int lm_head_hidden = 0;              // the hidden size lm_head_wg_per_cu was computed for
    int lm_head_wg_per_cu = 1;
    int dnp_chunk_threads = 0;     // the DeltaNet prefill chunk kernel's workgroup size (its launch bounds)
    int gqp_kv_threads = 0;        // the GQA prefill K/V kernel's workgroup size (its launch bounds)
    int q4_threads = 0;            // the Q4 kernels' workgroup sizes (their launch bounds)
    int q4_gu_threads = 0;
    int q4_hidden_threads = 0, q4_inter_threads = 0;
    void* ws = nullptr;            // general workspace
    size_t ws_bytes = 0;
    // whether a call that used `ws` ran under stream capture: a graph may
    // then hold its address in kernel arguments
    bool ws_captured = false;
    // Workspaces replaced by a larger one after a capture had used them.  A
    // graph captured earlier holds their addresses in its kernel arguments,
    // so they stay allocated until qm_destroy.
    std::vector<void*> retired_ws;
    std::string err;
    int64_t opt_dn_threads = 0;
    int64_t opt_gqa_chunk = 0;
    int64_t opt_gqp_order = 0;
    // the GQA prefill attention's queue orders of the last few sequence
    // lengths (a plan costs 0.1-2.7 ms on the host), least recently used
    // evicted; each entry is for seq_len S over `bins` workgroups per kv
    // group under order option `mode` (ordered = 0: longest first)
    struct GqpPlan {
        int32_t S = -1, bins = -1;
        int64_t mode = -1;
        uint64_t used = 0;
        int32_t ordered = 0;
        uint16_t order[QM_GQA_PREFILL_ORDER_MAX];
    };
    static constexpr int kGqpPlans = 8;
    GqpPlan gqp_plans[kGqpPlans];
    uint64_t gqp_clock = 0;
    GqaPrefillAttnArgs gqp_args{};
    bool noalloc_owner = false;    // this context holds its device's no-alloc scratch
    int num_cu = 0;                // compute units of the device
    // this device's copy of the fixed scratch array of the allocation-free
    // entry point (qm_noalloc.hip), resolved at qm_create; null if that failed
    void* noalloc_scratch = nullptr;
    std::string noalloc_err;
};

struct qm_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

struct qm_event {
    hipEvent_t ev = nullptr;
};

namespace {

int32_t fail(qm_context* c, int32_t code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (c) c->err = buf; else g_create_error = buf;
    return code;
}

// Mixer kernels move data in 16-byte vectors: every device pointer they take
// must be 16-byte aligned (hipMalloc returns 256-byte aligned memory).
bool all_aligned16(std::initializer_list<const void*> ptrs) {
    for (const void* p : ptrs)
        if (p && (reinterpret_cast<uintptr_t>(p) & 15u) != 0) return false;
    return true;
}

bool aligned_to(const void* p, uintptr_t a) { return !p || (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

constexpr int32_t kSampleMaxVocab = 262144;      // the presence bitmap of qm_sample_penalties (LDS)
constexpr size_t kSampleWsBytes = 8192 * sizeof(uint64_t);   // stage-1 sampling candidates

#define QM_HIP(c, call)                                                              \
    do {                                                                             \
        hipError_t e_ = (call);                                                      \
        if (e_ != hipSuccess)                                                        \
            return fail((c), e_ == hipErrorOutOfMemory ? QM_ERR_OUT_OF_MEMORY : QM_ERR_HIP, \
                        "%s: %s", #call, hipGetErrorString(e_));                     \
    } while (0)

hipStream_t pick(qm_context* c, qm_stream s) { return s ? static_cast<hipStream_t>(s) : c->stream; }

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) return false;
    return st != hipStreamCaptureStatusNone;
}

// Grow the workspace (every call that uses it comes through here first).
// Growth is refused while the stream is being captured.  If a capture has
// used the old buffer, it is retired, not freed: the graph keeps its address
// in kernel arguments and may be replayed later.  Otherwise it is freed once
// the device has finished the work queued on it.  Growth on demand is
// geometric (at least 1.5x) so that callers who never call qm_reserve grow
// O(log) times, not once per KV-length step; qm_reserve asks for its exact
// size.
int32_t ensure(qm_context* c, hipStream_t s, size_t ws_bytes, bool exact = false) {
    const bool cap = capturing(s);
    if (cap) c->ws_captured = true;
    if (ws_bytes <= c->ws_bytes) return QM_OK;
    if (cap)
        return fail(c, QM_ERR_WORKSPACE,
                    "workspace must grow to %zu bytes during graph capture; "
                    "call qm_reserve() before capturing", ws_bytes);
    size_t want = ws_bytes;
    if (c->ws_bytes > 0 && !exact) want = std::max(want, c->ws_bytes + c->ws_bytes / 2);
    want = (want + 4095) & ~static_cast<size_t>(4095);
    if (c->ws && !c->ws_captured) {
        // queued kernels on any stream may still read it
        QM_HIP(c, hipDeviceSynchronize());
        QM_HIP(c, hipFree(c->ws));
        c->ws = nullptr;
        c->ws_bytes = 0;
    }
    void* fresh = nullptr;
    QM_HIP(c, hipMalloc(&fresh, want));
    if (c->ws) c->retired_ws.push_back(c->ws);
    c->ws = fresh;
    c->ws_bytes = want;
    c->ws_captured = false;
    return QM_OK;
}

template <class Args>
int32_t launch(qm_context* c, hipFunction_t f, uint32_t grid, uint32_t block, const Args& args,
               hipStream_t s, const char* what) {
    Args copy = args;
    void* params[] = {static_cast<void*>(&copy)};
    hipError_t e = hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, 0, s, params, nullptr);
    if (e != hipSuccess) return fail(c, QM_ERR_HIP, "launch %s: %s", what, hipGetErrorString(e));
    return QM_OK;
}

std::string library_dir() {
    Dl_info info;
    if (dladdr(reinterpret_cast<void*>(&qm_create), &info) && info.dli_fname) {
        std::string p = info.dli_fname;
        size_t k = p.find_last_of('/');
        if (k != std::string::npos) return p.substr(0, k);
    }
    return ".";
}

bool same_config(const qm_config& a, const qm_config& b) {
    return a.num_qk_heads == b.num_qk_heads && a.num_v_heads == b.num_v_heads &&
           a.dn_head_dim == b.dn_head_dim && a.conv_kernel == b.conv_kernel &&
           a.num_heads == b.num_heads && a.num_kv_heads == b.num_kv_heads &&
           a.attn_head_dim == b.attn_head_dim && a.rope_dim == b.rope_dim;
}

int32_t load_function(qm_context* c, hipModule_t m, const char* name, hipFunction_t* f) {
    hipError_t e = hipModuleGetFunction(f, m, name);
    if (e != hipSuccess)
        return fail(c, QM_ERR_CODE_OBJECT, "kernel %s not found in code object: %s", name,
                    hipGetErrorString(e));
    return QM_OK;
}

}  // namespace

namespace {
struct DnPrefillLayout {
    size_t Wn, Qt, Ut, Y0t, Ktt, Dt, gC, Yt, Yx, vstat, mode, total;
};

// GQA prefill workspace: the fragment-ordered K and V tile copy, then the
// row-block queue.
size_t gqa_prefill_kvf_bytes(size_t s_pad) {
    return (static_cast<size_t>(QM_GQA_KV_HEADS) * QM_GQA_HD * s_pad * 2 * 2 + 255) & ~static_cast<size_t>(255);
}

DnPrefillLayout dn_prefill_layout(int64_t T) {
    const int64_t nc = (T + QM_DN_CHUNK - 1) / QM_DN_CHUNK;
    auto al = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    DnPrefillLayout L{};
    size_t o = 0;
    const size_t blk = static_cast<size_t>(QM_DN_V_HEADS) * nc * QM_DN_CHUNK * QM_DN_HD * 2;
    L.Wn = o; o += al(blk);
    L.Qt = o; o += al(blk);
    L.Ut = o; o += al(blk);
    L.Y0t = o; o += al(blk);
    L.Ktt = o; o += al(blk / 2);
    L.Dt = o; o += al(static_cast<size_t>(QM_DN_V_HEADS) * nc * QM_DN_CHUNK * 4);
    L.gC = o; o += al(static_cast<size_t>(QM_DN_V_HEADS) * nc * 4);
    L.Yt = o; o += al(blk);
    L.Yx = o; o += al(2 * blk);
    L.vstat = o; o += al(static_cast<size_t>(QM_DN_V_HEADS) * (nc + 1) * QM_DN_HD * 4);
    L.mode = o; o += al(static_cast<size_t>(QM_DN_V_HEADS) * 8 * 4);
    L.total = o;
    return L;
}
}  // namespace

extern "C" {

void qm_default_config(qm_config* cfg) {
    if (!cfg) return;
    cfg->num_qk_heads = QM_DN_QK_HEADS;
    cfg->num_v_heads = QM_DN_V_HEADS;
    cfg->dn_head_dim = QM_DN_HD;
    cfg->conv_kernel = QM_DN_CONV_K;
    cfg->num_heads = QM_GQA_HEADS;
    cfg->num_kv_heads = QM_GQA_KV_HEADS;
    cfg->attn_head_dim = QM_GQA_HD;
    cfg->rope_dim = QM_GQA_ROT;
}

const char* qm_status_string(int32_t status) {
    switch (status) {
        case QM_OK: return "ok";
        case QM_ERR_NO_DEVICE: return "no HIP device";
        case QM_ERR_CODE_OBJECT: return "gfx950 code object missing or unusable";
        case QM_ERR_INVALID_ARG: return "invalid argument";
        case QM_ERR_SHAPE: return "unsupported mixer shape";
        case QM_ERR_ROPE_RANGE: return "position beyond the RoPE table";
        case QM_ERR_CAPACITY: return "position beyond the KV cache capacity";
        case QM_ERR_HIP: return "HIP runtime error";
        case QM_ERR_OUT_OF_MEMORY: return "out of device memory";
        case QM_ERR_WORKSPACE: return "workspace growth during graph capture";
        default: return "unknown status";
    }
}

const char* qm_last_error(const qm_context* ctx) {
    return ctx ? ctx->err.c_str() : g_create_error.c_str();
}

int32_t qm_device_count(int32_t* count) {
    if (!count) return QM_ERR_INVALID_ARG;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = (e == hipSuccess) ? n : 0;
    return QM_OK;
}

int32_t qm_create(qm_context** out, const qm_config* cfg, const char* code_object_dir,
                  int32_t device) {
    if (!out) return fail(nullptr, QM_ERR_INVALID_ARG, "qm_create: out is null");
    *out = nullptr;
    qm_config want;
    qm_default_config(&want);
    if (cfg && !same_config(*cfg, want))
        return fail(nullptr, QM_ERR_SHAPE,
                    "kernels are built for the 4B mixer (16/32 heads x 128, conv 4; "
                    "16q/4kv x 256, rope 64)");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return fail(nullptr, QM_ERR_NO_DEVICE, "no HIP device visible");
    if (device < 0 || device >= n)
        return fail(nullptr, QM_ERR_NO_DEVICE, "device %d out of range (%d devices)", device, n);
    if (hipSetDevice(device) != hipSuccess)
        return fail(nullptr, QM_ERR_NO_DEVICE, "hipSetDevice(%d) failed", device);

    qm_context* c = new qm_context();
    c->device = device;
    c->cfg = want;
    if (hipDeviceGetAttribute(&c->num_cu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        c->num_cu <= 0)
        c->num_cu = 256;
    std::string dir = code_object_dir ? code_object_dir : library_dir();
    const char* files[] = {"qm_dn_decode.hsaco", "qm_gqa_decode.hsaco", "qm_util.hsaco",
                           "qm_dn_prefill.hsaco", "qm_gqa_prefill.hsaco", "qm_q4_proj.hsaco",
                           "qm_q4_vocab.hsaco", "qm_sample.hsaco"};
    constexpr int kModules = 8;
    hipModule_t mods[kModules] = {};
    for (int i = 0; i < kModules; ++i) {
        std::string path = dir + "/" + files[i];
        hipError_t e = hipModuleLoad(&mods[i], path.c_str());
        if (e != hipSuccess) {
            for (int j = 0; j < i; ++j) hipModuleUnload(mods[j]);
            delete c;
            return fail(nullptr, QM_ERR_CODE_OBJECT, "cannot load %s: %s", path.c_str(),
                        hipGetErrorString(e));
        }
        c->modules.push_back(mods[i]);
    }
    int32_t st = QM_OK;
    const char* dn_names[3] = {"qm_dn_decode_t256", "qm_dn_decode_t512", "qm_dn_decode_t1024"};
    if (st == QM_OK) st = load_function(c, mods[0], "qm_dn_conv_silu", &c->f_conv);
    for (int i = 0; i < 3 && st == QM_OK; ++i) st = load_function(c, mods[0], dn_names[i], &c->f_dn[i]);
    if (st == QM_OK) st = load_function(c, mods[1], "qm_gqa_decode_split", &c->f_gqa_split[0]);
    if (st == QM_OK) st = load_function(c, mods[1], "qm_gqa_decode_split_w5", &c->f_gqa_split[1]);
    if (st == QM_OK) st = load_function(c, mods[1], "qm_gqa_decode_split_w6", &c->f_gqa_split[2]);
    if (st == QM_OK) st = load_function(c, mods[1], "qm_gqa_decode_split_w7", &c->f_gqa_split[3]);
    if (st == QM_OK) st = load_function(c, mods[1], "qm_gqa_decode_split_w8", &c->f_gqa_split[4]);
    if (st == QM_OK) st = load_function(c, mods[1], "qm_gqa_decode_merge", &c->f_gqa_merge);
    if (st == QM_OK) st = load_function(c, mods[2], "qm_fill_normal", &c->f_fill);
    if (st == QM_OK) st = load_function(c, mods[3], "qm_dn_prefill_chunk", &c->f_dnp_chunk);
    if (st == QM_OK) st = load_function(c, mods[3], "qm_dn_prefill_scan", &c->f_dnp_scan);
    if (st == QM_OK) st = load_function(c, mods[3], "qm_dn_prefill_out", &c->f_dnp_out);
    if (st == QM_OK) st = load_function(c, mods[4], "qm_gqa_prefill_kv", &c->f_gqp_kv);
    if (st == QM_OK) st = load_function(c, mods[4], "qm_gqa_prefill_attn", &c->f_gqp_attn);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemv", &c->f_q4_gemv);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemv_hidden", &c->f_q4_gemv_hidden);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemv_inter", &c->f_q4_gemv_inter);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_repack", &c->f_q4_repack);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gate_up", &c->f_q4_gate_up);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemm", &c->f_q4_gemm[0][0]);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemm_xbf16", &c->f_q4_gemm[1][0]);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemm_gu", &c->f_q4_gemm[0][1]);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemm_gu_xbf16", &c->f_q4_gemm[1][1]);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemm_n128", &c->f_q4_gemm_n128[0]);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemm_xbf16_n128", &c->f_q4_gemm_n128[1]);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemm_m64", &c->f_q4_gemm_m64[0]);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemm_xbf16_m64", &c->f_q4_gemm_m64[1]);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemm_n32", &c->f_q4_gemm_n32[0]);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_q4_gemm_xbf16_n32", &c->f_q4_gemm_n32[1]);
    if (st == QM_OK) st = load_function(c, mods[5], "qm_rms_norm_f16", &c->f_rms_f16);
    if (st == QM_OK) st = load_function(c, mods[6], "qm_q4_lm_head", &c->f_lm_head);
    if (st == QM_OK) st = load_function(c, mods[6], "qm_q4_embed", &c->f_embed);
    if (st == QM_OK) st = load_function(c, mods[7], "qm_sample_penalties", &c->f_sample_pen);
    if (st == QM_OK) st = load_function(c, mods[7], "qm_sample_top_k", &c->f_sample);
    if (st == QM_OK) st = load_function(c, mods[7], "qm_sample_select", &c->f_sample_select);
    if (st == QM_OK &&
        (hipFuncGetAttribute(&c->q4_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, c->f_q4_gemv) != hipSuccess ||
         hipFuncGetAttribute(&c->q4_gu_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, c->f_q4_gate_up) !=
             hipSuccess ||
         hipFuncGetAttribute(&c->q4_hidden_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, c->f_q4_gemv_hidden) !=
             hipSuccess ||
         hipFuncGetAttribute(&c->q4_inter_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, c->f_q4_gemv_inter) !=
             hipSuccess))
        st = fail(c, QM_ERR_CODE_OBJECT, "qm_q4_gemv: cannot read its workgroup size");
    if (st == QM_OK && hipFuncGetAttribute(&c->dnp_chunk_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK,
                                           c->f_dnp_chunk) != hipSuccess)
        st = fail(c, QM_ERR_CODE_OBJECT, "qm_dn_prefill_chunk: cannot read its workgroup size");
    if (st == QM_OK && hipFuncGetAttribute(&c->gqp_kv_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK,
                                           c->f_gqp_kv) != hipSuccess)
        st = fail(c, QM_ERR_CODE_OBJECT, "qm_gqa_prefill_kv: cannot read its workgroup size");
    if (st == QM_OK && hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess)
        st = fail(c, QM_ERR_HIP, "hipStreamCreate failed");
    if (st == QM_OK) {
        // once per device, with the device current (set above): the address
        // of its copy of the no-alloc scratch array
        const int e = qm_noalloc_scratch(device, &c->noalloc_scratch);
        if (e != 0) {
            c->noalloc_scratch = nullptr;
            c->noalloc_err = std::string("hipGetSymbolAddress(scratch): ") +
                             hipGetErrorString(static_cast<hipError_t>(e));
        }
    }
    if (st != QM_OK) {
        g_create_error = c->err;
        qm_destroy(c);
        return st;
    }
    *out = c;
    return QM_OK;
}

int32_t qm_destroy(qm_context* c) {
    if (!c) return QM_ERR_INVALID_ARG;
    hipSetDevice(c->device);
    hipDeviceSynchronize();
    if (c->ws) hipFree(c->ws);
    for (void* p : c->retired_ws) hipFree(p);
    if (c->noalloc_owner) qm_noalloc_release(c->device, c);
    if (c->stream) hipStreamDestroy(c->stream);
    for (hipModule_t m : c->modules) hipModuleUnload(m);
    delete c;
    return QM_OK;
}

int32_t qm_set_option(qm_context* c, int32_t option, int64_t value) {
    if (!c) return QM_ERR_INVALID_ARG;
    switch (option) {
        case QM_OPT_DN_DECODE_THREADS:
            if (value != 0 && value != 256 && value != 512 && value != 1024)
                return fail(c, QM_ERR_INVALID_ARG, "DN decode threads must be 0, 256, 512 or 1024");
            c->opt_dn_threads = value;
            return QM_OK;
        case QM_OPT_GQA_DECODE_CHUNK:
            if (value < 0 || value % 64 != 0 || value > (1 << 20))
                return fail(c, QM_ERR_INVALID_ARG, "GQA decode chunk must be a multiple of 64");
            c->opt_gqa_chunk = value;
            return QM_OK;
        case QM_OPT_GQA_PREFILL_ORDER:
            if (value < 0 || value > 2)
                return fail(c, QM_ERR_INVALID_ARG, "GQA prefill order must be 0, 1 or 2");
            c->opt_gqp_order = value;
            return QM_OK;
        default:
            return fail(c, QM_ERR_INVALID_ARG, "unknown option %d", option);
    }
}

// ---- plumbing --------------------------------------------------------------
int32_t qm_alloc(qm_context* c, uint64_t bytes, void** dev) {
    if (!c || !dev || bytes == 0) return c ? fail(c, QM_ERR_INVALID_ARG, "qm_alloc: bad args") : QM_ERR_INVALID_ARG;
    *dev = nullptr;
    QM_HIP(c, hipMalloc(dev, bytes));
    return QM_OK;
}

int32_t qm_free(qm_context* c, void* dev) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (dev) QM_HIP(c, hipFree(dev));
    return QM_OK;
}

int32_t qm_memcpy_h2d(qm_context* c, void* dst, const void* src, uint64_t bytes, qm_stream s) {
    if (!c || ((!dst || !src) && bytes)) return c ? fail(c, QM_ERR_INVALID_ARG, "qm_memcpy_h2d: null") : QM_ERR_INVALID_ARG;
    if (!bytes) return QM_OK;
    QM_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, pick(c, s)));
    QM_HIP(c, hipStreamSynchronize(pick(c, s)));   // src may be pageable / temporary
    return QM_OK;
}

int32_t qm_memcpy_d2h(qm_context* c, void* dst, const void* src, uint64_t bytes, qm_stream s) {
    if (!c || ((!dst || !src) && bytes)) return c ? fail(c, QM_ERR_INVALID_ARG, "qm_memcpy_d2h: null") : QM_ERR_INVALID_ARG;
    if (!bytes) return QM_OK;
    QM_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, pick(c, s)));
    QM_HIP(c, hipStreamSynchronize(pick(c, s)));
    return QM_OK;
}

int32_t qm_memcpy_d2d(qm_context* c, void* dst, const void* src, uint64_t bytes, qm_stream s) {
    if (!c || ((!dst || !src) && bytes)) return c ? fail(c, QM_ERR_INVALID_ARG, "qm_memcpy_d2d: null") : QM_ERR_INVALID_ARG;
    if (!bytes) return QM_OK;
    QM_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, pick(c, s)));
    return QM_OK;
}

int32_t qm_memset(qm_context* c, void* dst, int32_t v, uint64_t bytes, qm_stream s) {
    if (!c || (!dst && bytes)) return c ? fail(c, QM_ERR_INVALID_ARG, "qm_memset: null") : QM_ERR_INVALID_ARG;
    if (!bytes) return QM_OK;
    QM_HIP(c, hipMemsetAsync(dst, v, bytes, pick(c, s)));
    return QM_OK;
}

int32_t qm_stream_create(qm_context* c, qm_stream* s) {
    if (!c || !s) return QM_ERR_INVALID_ARG;
    hipStream_t h = nullptr;
    QM_HIP(c, hipStreamCreateWithFlags(&h, hipStreamNonBlocking));
    *s = h;
    return QM_OK;
}

int32_t qm_stream_destroy(qm_context* c, qm_stream s) {
    if (!c || !s) return QM_ERR_INVALID_ARG;
    QM_HIP(c, hipStreamDestroy(static_cast<hipStream_t>(s)));
    return QM_OK;
}

int32_t qm_sync(qm_context* c, qm_stream s) {
    if (!c) return QM_ERR_INVALID_ARG;
    QM_HIP(c, hipStreamSynchronize(pick(c, s)));
    return QM_OK;
}

int32_t qm_event_create(qm_context* c, qm_event** ev) {
    if (!c || !ev) return QM_ERR_INVALID_ARG;
    qm_event* e = new qm_event();
    hipError_t r = hipEventCreate(&e->ev);
    if (r != hipSuccess) { delete e; return fail(c, QM_ERR_HIP, "hipEventCreate: %s", hipGetErrorString(r)); }
    *ev = e;
    return QM_OK;
}

int32_t qm_event_destroy(qm_context* c, qm_event* ev) {
    if (!c || !ev) return QM_ERR_INVALID_ARG;
    hipEventDestroy(ev->ev);
    delete ev;
    return QM_OK;
}

int32_t qm_event_record(qm_context* c, qm_event* ev, qm_stream s) {
    if (!c || !ev) return QM_ERR_INVALID_ARG;
    QM_HIP(c, hipEventRecord(ev->ev, pick(c, s)));
    return QM_OK;
}

int32_t qm_event_elapsed_ms(qm_context* c, qm_event* a, qm_event* b, float* ms) {
    if (!c || !a || !b || !ms) return QM_ERR_INVALID_ARG;
    QM_HIP(c, hipEventSynchronize(b->ev));
    QM_HIP(c, hipEventElapsedTime(ms, a->ev, b->ev));
    return QM_OK;
}

int32_t qm_graph_begin(qm_context* c, qm_stream s) {
    if (!c) return QM_ERR_INVALID_ARG;
    QM_HIP(c, hipStreamBeginCapture(pick(c, s), hipStreamCaptureModeThreadLocal));
    return QM_OK;
}

int32_t qm_graph_end(qm_context* c, qm_stream s, qm_graph** out) {
    if (!c || !out) return QM_ERR_INVALID_ARG;
    qm_graph* g = new qm_graph();
    hipError_t e = hipStreamEndCapture(pick(c, s), &g->graph);
    if (e != hipSuccess) { delete g; return fail(c, QM_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e)); }
    e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        hipGraphDestroy(g->graph);
        delete g;
        return fail(c, QM_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    *out = g;
    return QM_OK;
}

int32_t qm_graph_launch(qm_context* c, qm_graph* g, qm_stream s) {
    if (!c || !g) return QM_ERR_INVALID_ARG;
    QM_HIP(c, hipGraphLaunch(g->exec, pick(c, s)));
    return QM_OK;
}

int32_t qm_graph_destroy(qm_context* c, qm_graph* g) {
    if (!c || !g) return QM_ERR_INVALID_ARG;
    if (g->exec) hipGraphExecDestroy(g->exec);
    if (g->graph) hipGraphDestroy(g->graph);
    delete g;
    return QM_OK;
}

// ---- host helpers ------------------------------------------------------------
// convert.rs:161-176 (built with -ffp-contract=off: plain f32 rounding).
int32_t qm_rope_table(double theta, int32_t rope_dim, int32_t max_pos, float* cos_host,
                      float* sin_host) {
    if (!cos_host || !sin_host || rope_dim <= 0 || rope_dim % 2 || max_pos <= 0 || !(theta > 0.0))
        return QM_ERR_INVALID_ARG;
    const int32_t half = rope_dim / 2;
    const float th = static_cast<float>(theta);
    for (int32_t i = 0; i < half; ++i) {
        const float freq = 1.0f / powf(th, 2.0f * static_cast<float>(i) / static_cast<float>(rope_dim));
        for (int32_t pos = 0; pos < max_pos; ++pos) {
            const float angle = static_cast<float>(pos) * freq;
            cos_host[static_cast<size_t>(pos) * half + i] = cosf(angle);
            sin_host[static_cast<size_t>(pos) * half + i] = sinf(angle);
        }
    }
    return QM_OK;
}

int32_t qm_fill_normal(qm_context* c, void* dst, int32_t dtype, uint64_t count, float mean,
                       float stdev, uint64_t seed, qm_stream s) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (!dst || count == 0 || dtype < QM_F32 || dtype > QM_BF16)
        return fail(c, QM_ERR_INVALID_ARG, "qm_fill_normal: bad args");
    FillArgs a{dst, count, seed, mean, stdev, dtype};
    uint64_t blocks = (count + 255) / 256;
    uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>(blocks, 1u << 16));
    return launch(c, c->f_fill, grid, 256, a, pick(c, s), "qm_fill_normal");
}

// ---- DeltaNet decode ---------------------------------------------------------------
// Threads per (sequence, v-head) workgroup.  Small batches leave most CUs
// idle, so they take wider workgroups (more loads in flight per head), up
// to 512: with 1024 (4 waves per SIMD) the per-wave fixed VALU work (gates,
// q/k norms) is paid four times per SIMD, and batch 1 measured 3.68 us per
// step against 3.54 us with 512.
static int dn_auto_threads(int32_t batch) {
    const int64_t heads = static_cast<int64_t>(batch) * QM_DN_V_HEADS;
    if (heads >= 512) return 256;
    return 512;
}

int32_t qm_deltanet_decode(qm_context* c, qm_stream stream, int32_t batch, int32_t flags,
                           const float* qkv, float* conv_buf, const float* conv_w,
                           const float* a, const float* b, const float* a_log,
                           const float* dt_bias, const float* z, const uint16_t* norm_w,
                           float* state, int64_t state_stride, float* out) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (batch <= 0) return fail(c, QM_ERR_INVALID_ARG, "qm_deltanet_decode: batch %d", batch);
    if (flags != QM_DN_PREACT && flags != QM_DN_POSTACT)
        return fail(c, QM_ERR_INVALID_ARG, "qm_deltanet_decode: flags %d", flags);
    if (!qkv || !a || !b || !a_log || !dt_bias || !z || !norm_w || !state || !out)
        return fail(c, QM_ERR_INVALID_ARG, "qm_deltanet_decode: null pointer");
    if (!all_aligned16({qkv, conv_buf, conv_w, a, b, a_log, dt_bias, z, norm_w, state, out}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_deltanet_decode: device pointers must be 16-byte aligned");
    if (flags == QM_DN_PREACT && (!conv_buf || !conv_w))
        return fail(c, QM_ERR_INVALID_ARG, "qm_deltanet_decode: layer mode needs conv_buf and conv_w");
    if (state_stride < static_cast<int64_t>(QM_DN_V_HEADS) * QM_DN_HEAD_ELEMS || state_stride % 4)
        return fail(c, QM_ERR_INVALID_ARG, "qm_deltanet_decode: state_stride %lld",
                    static_cast<long long>(state_stride));
    const uint64_t grid = static_cast<uint64_t>(batch) * QM_DN_V_HEADS;
    if (grid > 0x7fffffffull) return fail(c, QM_ERR_INVALID_ARG, "qm_deltanet_decode: batch too large");
    hipStream_t s = pick(c, stream);
    const int threads = c->opt_dn_threads ? static_cast<int>(c->opt_dn_threads) : dn_auto_threads(batch);
    const size_t act_bytes = flags == QM_DN_PREACT ? static_cast<size_t>(batch) * QM_DN_QKV_DIM * 4 : 0;
    int32_t st = ensure(c, s, act_bytes);
    if (st != QM_OK) return st;
    const float* act = qkv;
    if (flags == QM_DN_PREACT) {
        DnConvArgs ca{qkv, conv_buf, conv_w, static_cast<float*>(c->ws), batch};
        const uint64_t n = static_cast<uint64_t>(batch) * QM_DN_QKV_DIM;
        st = launch(c, c->f_conv, static_cast<uint32_t>((n + 255) / 256), 256, ca, s, "qm_dn_conv_silu");
        if (st != QM_OK) return st;
        act = static_cast<const float*>(c->ws);
    }
    DnDecodeArgs da{act, a, b, a_log, dt_bias, z, norm_w, state, state_stride, out, batch};
    const int fi = threads == 256 ? 0 : threads == 512 ? 1 : 2;
    return launch(c, c->f_dn[fi], static_cast<uint32_t>(grid), threads, da, s, "qm_dn_decode");
}

// ---- GQA decode --------------------------------------------------------------------
// Keys per split workgroup, a multiple of 16 (one wave round): enough that
// a launch has at most about 2048 workgroups (8 per CU) and the merge folds
// at most 64 splits per head in one pass (at most 56 per memory round
// trip), at most 2048.  Small batches thus
// get the shortest chunks that still fit (batch 1 at position 4096: 80 keys,
// 208 workgroups), since each wave's rounds run one after another.
static int64_t gqa_auto_chunk(int64_t len, int32_t batch) {
    const int64_t want = std::max<int64_t>((len + 63) / 64, (len * batch * QM_GQA_KV_HEADS + 2047) / 2048);
    const int64_t ch = ((want + 15) / 16) * 16;
    return std::max<int64_t>(16, std::min<int64_t>(ch, 2048));
}

}  // extern "C"

namespace {
// qm_gqa_decode and qm_gqa_decode_noalloc: the same checks, launch shapes and
// kernels; the split partials go to the context's workspace (grown if
// needed) or to the device's fixed scratch array (never allocated here).
int32_t gqa_decode_impl(qm_context* c, qm_stream stream, int32_t batch, const float* q_gate,
                        const float* k_new, const float* v_new, const uint16_t* q_norm,
                        const uint16_t* k_norm, const float* rope_cos, const float* rope_sin,
                        int32_t rope_len, const int32_t* pos, int32_t max_pos, uint16_t* k_cache,
                        uint16_t* v_cache, int64_t cap, float* out, bool noalloc) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (batch <= 0) return fail(c, QM_ERR_INVALID_ARG, "qm_gqa_decode: batch %d", batch);
    if (!q_gate || !k_new || !v_new || !q_norm || !k_norm || !rope_cos || !rope_sin || !k_cache ||
        !v_cache || !out)
        return fail(c, QM_ERR_INVALID_ARG, "qm_gqa_decode: null pointer");
    if (!all_aligned16({q_gate, k_new, v_new, q_norm, k_norm, rope_cos, rope_sin, pos, k_cache, v_cache, out}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_gqa_decode: device pointers must be 16-byte aligned");
    if (max_pos < 0) return fail(c, QM_ERR_INVALID_ARG, "qm_gqa_decode: max_pos %d", max_pos);
    if (max_pos >= rope_len)
        return fail(c, QM_ERR_ROPE_RANGE, "position %d beyond RoPE table of %d rows", max_pos, rope_len);
    if (cap <= 0 || max_pos >= cap)
        return fail(c, QM_ERR_CAPACITY, "position %d beyond cache capacity %lld", max_pos,
                    static_cast<long long>(cap));
    hipStream_t s = pick(c, stream);
    const int64_t len = static_cast<int64_t>(max_pos) + 1;
    const int64_t chunk = c->opt_gqa_chunk ? c->opt_gqa_chunk : gqa_auto_chunk(len, batch);
    const int64_t nsplit = (len + chunk - 1) / chunk;
    const uint64_t grid = static_cast<uint64_t>(batch) * QM_GQA_KV_HEADS * nsplit;
    if (grid > 0x7fffffffull) return fail(c, QM_ERR_INVALID_ARG, "qm_gqa_decode: grid too large");
    const size_t part_bytes = nsplit > 1 ? static_cast<size_t>(grid) * 4 * 260 * sizeof(float) : 0;
    float* partials = nullptr;
    if (noalloc) {
        if (!c->noalloc_scratch)
            return fail(c, QM_ERR_HIP, "qm_gqa_decode_noalloc: the device scratch is unavailable (%s)",
                        c->noalloc_err.c_str());
        if (part_bytes > QM_NOALLOC_SCRATCH_BYTES)
            return fail(c, QM_ERR_WORKSPACE,
                        "qm_gqa_decode_noalloc: %lld splits of %lld keys for batch %d need %zu bytes of "
                        "partials; the fixed scratch holds %u (batch x 4 x splits <= %u)",
                        static_cast<long long>(nsplit), static_cast<long long>(chunk), batch, part_bytes,
                        QM_NOALLOC_SCRATCH_BYTES, QM_NOALLOC_SCRATCH_BYTES / (4 * 260 * 4));
        if (!c->noalloc_owner) {
            // one context per GPU may use the scratch: calls from two
            // contexts could overlap on the device and race in it
            const int e = qm_noalloc_claim(c->device, c);
            if (e != 0)
                return fail(c, QM_ERR_WORKSPACE,
                            "qm_gqa_decode_noalloc: the fixed scratch of device %d is held by another context "
                            "(calls from two contexts could overlap and race in it)", c->device);
            c->noalloc_owner = true;
        }
        partials = static_cast<float*>(c->noalloc_scratch);
    } else {
        const int32_t st = ensure(c, s, part_bytes);
        if (st != QM_OK) return st;
        partials = static_cast<float*>(c->ws);
    }
    GqaDecodeArgs ga{q_gate, k_new, v_new, q_norm, k_norm, rope_cos, rope_sin, pos, k_cache, v_cache,
                     out, partials, cap, max_pos,
                     static_cast<int32_t>(chunk), static_cast<int32_t>(nsplit), batch};
    // a split of 80..128 keys gets one wave per 16-key round, so no wave
    // runs two rounds one after the other; longer splits stream on 4 waves
    const int nw = (chunk >= 80 && chunk <= 128) ? static_cast<int>(chunk / 16) : 4;
    int32_t st = launch(c, c->f_gqa_split[nw - 4], static_cast<uint32_t>(grid), 64 * nw, ga, s,
                        "qm_gqa_decode_split");
    if (st != QM_OK || nsplit == 1) return st;
    return launch(c, c->f_gqa_merge, static_cast<uint32_t>(batch) * QM_GQA_KV_HEADS * 16, 64, ga, s,
                  "qm_gqa_decode_merge");
}
}  // namespace

extern "C" {

int32_t qm_gqa_decode(qm_context* c, qm_stream stream, int32_t batch, const float* q_gate,
                      const float* k_new, const float* v_new, const uint16_t* q_norm,
                      const uint16_t* k_norm, const float* rope_cos, const float* rope_sin,
                      int32_t rope_len, const int32_t* pos, int32_t max_pos, uint16_t* k_cache,
                      uint16_t* v_cache, int64_t cap, float* out) {
    return gqa_decode_impl(c, stream, batch, q_gate, k_new, v_new, q_norm, k_norm, rope_cos, rope_sin, rope_len,
                           pos, max_pos, k_cache, v_cache, cap, out, false);
}

int32_t qm_gqa_decode_noalloc(qm_context* c, qm_stream stream, int32_t batch, const float* q_gate,
                              const float* k_new, const float* v_new, const uint16_t* q_norm,
                              const uint16_t* k_norm, const float* rope_cos, const float* rope_sin,
                              int32_t rope_len, const int32_t* pos, int32_t max_pos, uint16_t* k_cache,
                              uint16_t* v_cache, int64_t cap, float* out) {
    return gqa_decode_impl(c, stream, batch, q_gate, k_new, v_new, q_norm, k_norm, rope_cos, rope_sin, rope_len,
                           pos, max_pos, k_cache, v_cache, cap, out, true);
}

int32_t qm_reserve(qm_context* c, int32_t max_batch, int32_t max_kv_len, int32_t max_prefill_tokens) {
    if (!c || max_batch <= 0 || max_kv_len < 0 || max_prefill_tokens < 0)
        return c ? fail(c, QM_ERR_INVALID_ARG, "qm_reserve: bad args") : QM_ERR_INVALID_ARG;
    size_t ws = static_cast<size_t>(max_batch) * QM_DN_QKV_DIM * 4;
    if (max_kv_len > 0) {
        // Bound on batch * nsplit over every batch <= max_batch and length
        // <= max_kv_len.  Automatic chunks: below the 2048 cap a chunk holds
        // at least len*batch/512 keys, so nsplit <= ceil(512/batch), and at
        // least len/64, so nsplit <= 64; at the cap nsplit = ceil(len/2048);
        // and always nsplit <= ceil(len/16).
        const int64_t L = max_kv_len, B = max_batch;
        int64_t bn;
        if (c->opt_gqa_chunk) {
            bn = B * ((L + c->opt_gqa_chunk - 1) / c->opt_gqa_chunk);
        } else {
            const int64_t per_seq = std::min<int64_t>((L + 15) / 16, std::max<int64_t>(64, (L + 2047) / 2048));
            bn = std::min<int64_t>(B * per_seq, std::max<int64_t>(512 + B, B * ((L + 2047) / 2048)));
        }
        ws = std::max(ws, static_cast<size_t>(bn) * QM_GQA_KV_HEADS * 4 * 260 * sizeof(float));
    }
    if (max_prefill_tokens > 0) {
        ws = std::max(ws, dn_prefill_layout(max_prefill_tokens).total);
        const size_t s_pad = (static_cast<size_t>(max_prefill_tokens) + 63) / 64 * 64;
        ws = std::max(ws, gqa_prefill_kvf_bytes(s_pad) + 256);
    }
    ws = std::max(ws, kSampleWsBytes);
    return ensure(c, c->stream, ws, true);
}

// ---- DeltaNet chunked prefill --------------------------------------------------------

int32_t qm_deltanet_prefill(qm_context* c, qm_stream stream, int32_t seq_len, const uint16_t* qkv,
                            float* conv_buf, const float* conv_w, const float* a, const float* b,
                            const float* a_log, const float* dt_bias, const uint16_t* z,
                            const uint16_t* norm_w, float* state, uint16_t* out) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (seq_len <= 0) return fail(c, QM_ERR_INVALID_ARG, "qm_deltanet_prefill: seq_len %d", seq_len);
    if (!qkv || !conv_buf || !conv_w || !a || !b || !a_log || !dt_bias || !z || !norm_w || !state || !out)
        return fail(c, QM_ERR_INVALID_ARG, "qm_deltanet_prefill: null pointer");
    if (!all_aligned16({qkv, conv_buf, conv_w, a, b, a_log, dt_bias, z, norm_w, state, out}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_deltanet_prefill: device pointers must be 16-byte aligned");
    hipStream_t s = pick(c, stream);
    const DnPrefillLayout L = dn_prefill_layout(seq_len);
    int32_t st = ensure(c, s, L.total);
    if (st != QM_OK) return st;
    char* ws = static_cast<char*>(c->ws);
    const int32_t nc = (seq_len + QM_DN_CHUNK - 1) / QM_DN_CHUNK;
    DnPrefillArgs pa{qkv, conv_buf, conv_w, a, b, a_log, dt_bias, z, norm_w, state, out,
                     reinterpret_cast<uint16_t*>(ws + L.Wn),
                     reinterpret_cast<uint16_t*>(ws + L.Qt), reinterpret_cast<uint16_t*>(ws + L.Ut),
                     reinterpret_cast<uint16_t*>(ws + L.Y0t), reinterpret_cast<uint16_t*>(ws + L.Ktt),
                     reinterpret_cast<float*>(ws + L.Dt),
                     reinterpret_cast<float*>(ws + L.gC), reinterpret_cast<uint16_t*>(ws + L.Yt),
                     reinterpret_cast<float*>(ws + L.Yx),
                     reinterpret_cast<float*>(ws + L.vstat), reinterpret_cast<int32_t*>(ws + L.mode), seq_len, nc};
    st = launch(c, c->f_dnp_chunk, static_cast<uint32_t>(nc) * QM_DN_QK_HEADS, c->dnp_chunk_threads, pa, s,
                "qm_dn_prefill_chunk");
    if (st != QM_OK) return st;
    st = launch(c, c->f_dnp_scan, QM_DN_V_HEADS * 8, 256, pa, s, "qm_dn_prefill_scan");
    if (st != QM_OK) return st;
    return launch(c, c->f_dnp_out, static_cast<uint32_t>(nc) * QM_DN_V_HEADS, 256, pa, s, "qm_dn_prefill_out");
}

// ---- GQA causal prefill ------------------------------------------------------------

int32_t qm_gqa_prefill(qm_context* c, qm_stream stream, int32_t seq_len, const uint16_t* q_gate,
                       const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                       const uint16_t* k_norm, const float* rope_cos, const float* rope_sin,
                       int32_t rope_len, uint16_t* k_cache, uint16_t* v_cache, int64_t cap,
                       uint16_t* out) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (seq_len <= 0) return fail(c, QM_ERR_INVALID_ARG, "qm_gqa_prefill: seq_len %d", seq_len);
    if (!q_gate || !k || !v || !q_norm || !k_norm || !rope_cos || !rope_sin || !k_cache || !v_cache || !out)
        return fail(c, QM_ERR_INVALID_ARG, "qm_gqa_prefill: null pointer");
    if (!all_aligned16({q_gate, k, v, q_norm, k_norm, rope_cos, rope_sin, k_cache, v_cache, out}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_gqa_prefill: device pointers must be 16-byte aligned");
    if (seq_len > rope_len)
        return fail(c, QM_ERR_ROPE_RANGE, "positions 0..%d beyond RoPE table of %d rows", seq_len - 1, rope_len);
    if (seq_len > cap)
        return fail(c, QM_ERR_CAPACITY, "%d tokens beyond cache capacity %lld", seq_len,
                    static_cast<long long>(cap));
    hipStream_t s = pick(c, stream);
    const int32_t s_pad = (seq_len + 63) / 64 * 64;
    const size_t kvf_bytes = gqa_prefill_kvf_bytes(s_pad);
    int32_t st = ensure(c, s, kvf_bytes + 256);
    if (st != QM_OK) return st;
    GqaPrefillArgs ga{q_gate, k, v, q_norm, k_norm, rope_cos, rope_sin, k_cache, v_cache,
                      static_cast<uint16_t*>(c->ws), out,
                      reinterpret_cast<int32_t*>(static_cast<char*>(c->ws) + kvf_bytes), cap, seq_len, s_pad};
    st = launch(c, c->f_gqp_kv, static_cast<uint32_t>(s_pad / 64) * QM_GQA_KV_HEADS, c->gqp_kv_threads, ga, s,
                "qm_gqa_prefill_kv");
    if (st != QM_OK) return st;
    // persistent: one workgroup per CU (a multiple of the 4 kv groups), no
    // more than there are 48-row blocks
    const int32_t nblk = (seq_len + 47) / 48;
    const int32_t per_group = std::max(1, std::min(c->num_cu / QM_GQA_KV_HEADS, nblk));
    qm_context::GqpPlan* plan = nullptr;
    for (auto& p : c->gqp_plans)
        if (p.S == seq_len && p.bins == per_group && p.mode == c->opt_gqp_order) plan = &p;
    if (!plan) {
        plan = &c->gqp_plans[0];
        for (auto& p : c->gqp_plans)
            if (p.used < plan->used) plan = &p;
        plan->ordered = qm_plan::gqp_set_order(plan->order, seq_len, per_group, c->opt_gqp_order);
        plan->S = seq_len;
        plan->bins = per_group;
        plan->mode = c->opt_gqp_order;
    }
    plan->used = ++c->gqp_clock;
    c->gqp_args.ordered = plan->ordered;
    if (plan->ordered)
        std::memcpy(c->gqp_args.order, plan->order, sizeof(uint16_t) * static_cast<size_t>((seq_len + 47) / 48));
    c->gqp_args.a = ga;
    return launch(c, c->f_gqp_attn, static_cast<uint32_t>(per_group) * QM_GQA_KV_HEADS, 768, c->gqp_args,
                  s, "qm_gqa_prefill_attn");
}

// ---- Q4 projections ---------------------------------------------------------------

namespace {
int32_t q4_check(qm_context* c, const char* what, int32_t k, int32_t n) {
    if (k <= 0 || n <= 0) return fail(c, QM_ERR_INVALID_ARG, "%s: k %d, n %d", what, k, n);
    if (n % 32 != 0)
        return fail(c, QM_ERR_SHAPE, "%s: n = %d is not a multiple of the 32-column group", what, n);
    return QM_OK;
}
}  // namespace

int32_t qm_q4_repack(qm_context* c, qm_stream stream, int32_t k, int32_t n, const uint8_t* packed,
                     const uint16_t* scales, uint8_t* codes, uint16_t* gscales) {
    if (!c) return QM_ERR_INVALID_ARG;
    int32_t st = q4_check(c, "qm_q4_repack", k, n);
    if (st != QM_OK) return st;
    if (!packed || !scales || !codes || !gscales)
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_repack: null pointer");
    if (!all_aligned16({packed, scales, codes, gscales}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_repack: device pointers must be 16-byte aligned");
    Q4RepackArgs ra{packed, scales, codes, gscales, k, n, QM_Q4_TILE(n)};
    const uint32_t grid = static_cast<uint32_t>((n / 32 + 15) / 16) * static_cast<uint32_t>((k + 63) / 64);
    return launch(c, c->f_q4_repack, grid, 256, ra, pick(c, stream), "qm_q4_repack");
}

namespace {
int32_t q4_gemv_multi_impl(qm_context* c, qm_stream stream, int32_t k, const float* x, const uint16_t* norm_w,
                           int32_t count, const qm_q4_out* outs, float* conv_buf, const float* conv_w) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (count < 1 || count > QM_Q4_MAX_OUT || !outs || !x)
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gemv_multi: %d outputs (1..%d) or null pointer", count,
                    QM_Q4_MAX_OUT);
    if (!all_aligned16({x, norm_w}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gemv: device pointers must be 16-byte aligned");
    Q4GemvArgs qa{};
    qa.x = x;
    qa.norm_w = norm_w;
    qa.k = k;
    qa.count = count;
    int32_t tiles = 0;
    for (int32_t i = 0; i < count; ++i) {
        const qm_q4_out& o = outs[i];
        int32_t st = q4_check(c, "qm_q4_gemv", k, o.n);
        if (st != QM_OK) return st;
        if (!o.codes_dev || !o.gscales_dev || !o.y_dev)
            return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gemv: null pointer (output %d)", i);
        if (!all_aligned16({o.codes_dev, o.gscales_dev, o.y_dev, o.residual_dev}))
            return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gemv: device pointers must be 16-byte aligned");
        qa.codes[i] = o.codes_dev;
        qa.gscales[i] = o.gscales_dev;
        qa.y[i] = o.y_dev;
        qa.residual[i] = o.residual_dev;
        qa.tile[i] = QM_Q4_TILE(o.n);
        qa.wstart[i] = tiles;
        tiles += o.n / qa.tile[i];
    }
    for (int32_t i = count; i < QM_Q4_MAX_OUT; ++i) qa.tile[i] = 16;
    for (int32_t i = count; i <= QM_Q4_MAX_OUT; ++i) qa.wstart[i] = tiles;
    qa.conv_buf = conv_buf;
    qa.conv_w = conv_w;
    // the shape-fitted forms: k up to 2560 (the hidden size) and 4097 .. 9216
    // (the MLP's down_proj), each with its own workgroup size
    hipFunction_t f = c->f_q4_gemv;
    int threads = c->q4_threads;
    if (k <= 2560) {
        f = c->f_q4_gemv_hidden;
        threads = c->q4_hidden_threads;
    } else if (k > 4096 && k <= 9216 && !norm_w) {
        f = c->f_q4_gemv_inter;
        threads = c->q4_inter_threads;
    }
    return launch(c, f, static_cast<uint32_t>(tiles), static_cast<uint32_t>(threads), qa, pick(c, stream),
                  "qm_q4_gemv");
}
}  // namespace

int32_t qm_q4_gemv_multi(qm_context* c, qm_stream stream, int32_t k, const float* x, const uint16_t* norm_w,
                         int32_t count, const qm_q4_out* outs) {
    return q4_gemv_multi_impl(c, stream, k, x, norm_w, count, outs, nullptr, nullptr);
}

int32_t qm_q4_gemv_multi_conv(qm_context* c, qm_stream stream, int32_t k, const float* x, const uint16_t* norm_w,
                              int32_t count, const qm_q4_out* outs, float* conv_buf, const float* conv_w) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (!conv_buf || !conv_w || !outs || count < 1)
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gemv_multi_conv: null conv buffer, weights or outputs");
    if (outs[0].residual_dev)
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gemv_multi_conv: the conv output takes no residual");
    if (!all_aligned16({conv_buf, conv_w}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gemv_multi_conv: device pointers must be 16-byte aligned");
    return q4_gemv_multi_impl(c, stream, k, x, norm_w, count, outs, conv_buf, conv_w);
}

int32_t qm_q4_gemv(qm_context* c, qm_stream stream, int32_t k, int32_t n, const float* x,
                   const uint8_t* codes, const uint16_t* gscales, float* y) {
    const qm_q4_out o{n, codes, gscales, y, nullptr};
    return qm_q4_gemv_multi(c, stream, k, x, nullptr, 1, &o);
}

int32_t qm_q4_gate_up(qm_context* c, qm_stream stream, int32_t k, int32_t n, const float* x,
                      const uint16_t* norm_w, const uint8_t* gate_codes, const uint16_t* gate_gscales,
                      const uint8_t* up_codes, const uint16_t* up_gscales, float* out) {
    if (!c) return QM_ERR_INVALID_ARG;
    int32_t st = q4_check(c, "qm_q4_gate_up", k, n);
    if (st != QM_OK) return st;
    if (!x || !gate_codes || !gate_gscales || !up_codes || !up_gscales || !out)
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gate_up: null pointer");
    if (!all_aligned16({x, norm_w, gate_codes, gate_gscales, up_codes, up_gscales, out}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gate_up: device pointers must be 16-byte aligned");
    Q4GemvArgs qa{};
    qa.x = x;
    qa.norm_w = norm_w;
    qa.codes[0] = gate_codes;
    qa.gscales[0] = gate_gscales;
    qa.codes[1] = up_codes;
    qa.gscales[1] = up_gscales;
    qa.y[0] = out;
    qa.tile[0] = qa.tile[1] = QM_Q4_TILE(n);
    qa.k = k;
    qa.count = 2;
    return launch(c, c->f_q4_gate_up, static_cast<uint32_t>(n / qa.tile[0]), static_cast<uint32_t>(c->q4_gu_threads), qa,
                  pick(c, stream), "qm_q4_gate_up");
}

int32_t qm_rms_norm_f16(qm_context* c, qm_stream stream, int32_t m, int32_t k, const float* x,
                        const uint16_t* norm_w, uint16_t* out) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (m <= 0 || k <= 0 || k % 4 != 0)
        return fail(c, QM_ERR_INVALID_ARG, "qm_rms_norm_f16: m %d, k %d (k a multiple of 4)", m, k);
    if (!x || !out) return fail(c, QM_ERR_INVALID_ARG, "qm_rms_norm_f16: null pointer");
    if (!all_aligned16({x, norm_w, out}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_rms_norm_f16: device pointers must be 16-byte aligned");
    RmsNormArgs ra{x, norm_w, out, m, k};
    return launch(c, c->f_rms_f16, static_cast<uint32_t>(m), 256, ra, pick(c, stream), "qm_rms_norm_f16");
}

int32_t qm_q4_lm_head(qm_context* c, qm_stream stream, int32_t vocab, int32_t hidden, const float* x,
                      const uint16_t* norm_w, const uint8_t* packed, const uint16_t* scales, float* logits) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (vocab <= 0 || hidden <= 0 || hidden % 512 != 0 || hidden > 8192)
        return fail(c, QM_ERR_SHAPE, "qm_q4_lm_head: vocab %d, hidden %d (hidden a multiple of 512, at most 8192)",
                    vocab, hidden);
    if (!x || !packed || !scales || !logits) return fail(c, QM_ERR_INVALID_ARG, "qm_q4_lm_head: null pointer");
    if (!all_aligned16({x, norm_w, packed, scales, logits}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_lm_head: device pointers must be 16-byte aligned");
    const int block = hidden / 8;                         // 4 rows x hidden / 32 groups
    if (c->lm_head_hidden != hidden) {
        int n = 0;
        if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, c->f_lm_head, block, 0) != hipSuccess || n <= 0)
            n = 1;
        c->lm_head_hidden = hidden;
        c->lm_head_wg_per_cu = n;
    }
    // super-batches of 32 rows, spread evenly over at most one resident wave of workgroups
    const int64_t nsb = (static_cast<int64_t>(vocab) + 31) / 32;
    const int64_t slots = static_cast<int64_t>(c->num_cu) * c->lm_head_wg_per_cu;
    const int64_t per = (nsb + slots - 1) / slots;
    const int64_t grid = (nsb + per - 1) / per;
    LmHeadArgs la{x, norm_w, packed, scales, logits, vocab, hidden};
    return launch(c, c->f_lm_head, static_cast<uint32_t>(grid), static_cast<uint32_t>(block), la, pick(c, stream),
                  "qm_q4_lm_head");
}

int32_t qm_q4_embed(qm_context* c, qm_stream stream, int32_t count, int32_t vocab, int32_t hidden,
                    const int32_t* ids, const uint8_t* packed, const uint16_t* scales, float* out) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (count <= 0 || vocab <= 0 || hidden <= 0 || hidden % 32 != 0)
        return fail(c, QM_ERR_SHAPE, "qm_q4_embed: count %d, vocab %d, hidden %d (a multiple of 32)", count, vocab,
                    hidden);
    if (!ids || !packed || !scales || !out) return fail(c, QM_ERR_INVALID_ARG, "qm_q4_embed: null pointer");
    if (!all_aligned16({ids, packed, scales, out}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_embed: device pointers must be 16-byte aligned");
    EmbedArgs ea{ids, packed, scales, out, vocab, hidden};
    return launch(c, c->f_embed, static_cast<uint32_t>(count), 64, ea, pick(c, stream), "qm_q4_embed");
}

static_assert(QM_SAMPLE_WGPU == QMK_SAMPLE_WGPU, "sampling flag values");

int32_t qm_sample(qm_context* c, qm_stream stream, int32_t vocab, float* logits, const int32_t* generated,
                  int32_t n_generated, const qm_sample_params* p, uint64_t* rng_state, int32_t* token_out,
                  int32_t* top_ids, float* top_probs) {
    if (!c) return QM_ERR_INVALID_ARG;
    if (!p || !logits || !token_out || vocab <= 0 || n_generated < 0 || (n_generated > 0 && !generated))
        return fail(c, QM_ERR_INVALID_ARG, "qm_sample: null pointer or negative size");
    if (vocab > kSampleMaxVocab)
        return fail(c, QM_ERR_SHAPE, "qm_sample: vocab %d (at most %d)", vocab, kSampleMaxVocab);
    if ((p->flags & ~QM_SAMPLE_WGPU) != 0) return fail(c, QM_ERR_INVALID_ARG, "qm_sample: unknown flags 0x%x", p->flags);
    const bool greedy = !(p->temperature > 0.0f);
    if (!greedy) {
        // generate.rs:353 takes every logit for top_k = 0; the top-k kernel sorts at most 1024 in one workgroup
        if (p->top_k < 1 || p->top_k > 1024)
            return fail(c, QM_ERR_INVALID_ARG, "qm_sample: top_k %d (1 .. 1024 when temperature > 0)", p->top_k);
        if ((p->flags & QM_SAMPLE_WGPU) && vocab < p->top_k)
            return fail(c, QM_ERR_INVALID_ARG, "qm_sample: top_k %d exceeds vocab %d", p->top_k, vocab);
        if (!rng_state) return fail(c, QM_ERR_INVALID_ARG, "qm_sample: null rng state");
    }
    if (!aligned_to(logits, 4) || !aligned_to(generated, 4) || !aligned_to(token_out, 4) ||
        !aligned_to(top_ids, 4) || !aligned_to(top_probs, 4) || !aligned_to(rng_state, 8))
        return fail(c, QM_ERR_INVALID_ARG, "qm_sample: misaligned device pointer");
    hipStream_t s = pick(c, stream);
    int32_t st = ensure(c, s, kSampleWsBytes);
    if (st != QM_OK) return st;
    // stage 1 slices: 1024 m logits each, so that slices x k candidates fit
    // the stage-2 sort (8192)
    const int64_t k = greedy ? 1 : std::min(p->top_k, vocab);
    int64_t m = 1;
    while ((vocab + 1024 * m - 1) / (1024 * m) * k > 8192) ++m;
    const int64_t chunk = 1024 * m, nw = (vocab + chunk - 1) / chunk;
    SampleArgs sa{logits,     generated,     rng_state,      token_out,  top_ids,
                  top_probs,  vocab,         n_generated,    p->top_k,   p->banned_id,
                  p->flags,   p->temperature, p->top_p,      p->repetition_penalty, p->presence_penalty,
                  static_cast<uint64_t*>(c->ws), static_cast<int32_t>(chunk), static_cast<int32_t>(nw * k)};
    if (p->repetition_penalty > 1.0f || (p->presence_penalty > 0.0f && n_generated > 0) || p->banned_id >= 0) {
        st = launch(c, c->f_sample_pen, 1, 1024, sa, s, "qm_sample_penalties");
        if (st != QM_OK) return st;
    }
    st = launch(c, c->f_sample_select, static_cast<uint32_t>(nw), 256, sa, s, "qm_sample_select");
    if (st != QM_OK) return st;
    return launch(c, c->f_sample, 1, 1024, sa, s, "qm_sample_top_k");
}

namespace {
int32_t q4_gemm_check(qm_context* c, const char* name, int32_t m, int32_t k, int32_t n, int32_t x_dtype) {
    int32_t st = q4_check(c, name, k, n);
    if (st != QM_OK) return st;
    if (m <= 0) return fail(c, QM_ERR_INVALID_ARG, "%s: m %d", name, m);
    if (k % 32 != 0) return fail(c, QM_ERR_SHAPE, "%s: k = %d is not a multiple of 32", name, k);
    if (x_dtype != QM_F16 && x_dtype != QM_BF16)
        return fail(c, QM_ERR_INVALID_ARG, "%s: x_dtype %d (QM_F16 or QM_BF16)", name, x_dtype);
    return QM_OK;
}
}  // namespace

int32_t qm_q4_gemm(qm_context* c, qm_stream stream, int32_t m, int32_t k, int32_t n, const uint16_t* x,
                   int32_t x_dtype, const uint8_t* codes, const uint16_t* gscales, const float* residual,
                   float* y, uint16_t* y_bf16) {
    if (!c) return QM_ERR_INVALID_ARG;
    int32_t st = q4_gemm_check(c, "qm_q4_gemm", m, k, n, x_dtype);
    if (st != QM_OK) return st;
    if (!x || !codes || !gscales || (!y) == (!y_bf16))
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gemm: null pointer, or not exactly one of y / y_bf16");
    if (!all_aligned16({x, codes, gscales, residual, y, y_bf16}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gemm: device pointers must be 16-byte aligned");
    Q4GemmArgs ga{x, codes, gscales, nullptr, nullptr, y, y_bf16, residual, m, k, n, QM_Q4_TILE(n)};
    const int xb = x_dtype == QM_BF16;
    auto tiles = [&](int64_t tm, int64_t tn) { return (m + tm - 1) / tm * ((n + tn - 1) / tn); };
    const int64_t two_per_cu = 2 * static_cast<int64_t>(c->num_cu);
    // the widest tile that still gives two workgroups per CU; n = 32 (the
    // DeltaNet a/b projections) a k-split kernel of 16 rows per workgroup
    if (n <= 32)
        return launch(c, c->f_q4_gemm_n32[xb], static_cast<uint32_t>((m + 15) / 16), 256, ga, pick(c, stream),
                      "qm_q4_gemm");
    if (tiles(128, 256) >= two_per_cu)
        return launch(c, c->f_q4_gemm[xb][0], static_cast<uint32_t>(tiles(128, 256)), 256, ga, pick(c, stream),
                      "qm_q4_gemm");
    if (tiles(128, 128) >= two_per_cu)
        return launch(c, c->f_q4_gemm_n128[xb], static_cast<uint32_t>(tiles(128, 128)), 256, ga, pick(c, stream),
                      "qm_q4_gemm");
    return launch(c, c->f_q4_gemm_m64[xb], static_cast<uint32_t>(tiles(64, 128)), 256, ga, pick(c, stream),
                  "qm_q4_gemm");
}

int32_t qm_q4_gemm_gate_up(qm_context* c, qm_stream stream, int32_t m, int32_t k, int32_t n, const uint16_t* x,
                           int32_t x_dtype, const uint8_t* gate_codes, const uint16_t* gate_gscales,
                           const uint8_t* up_codes, const uint16_t* up_gscales, uint16_t* out_bf16) {
    if (!c) return QM_ERR_INVALID_ARG;
    int32_t st = q4_gemm_check(c, "qm_q4_gemm_gate_up", m, k, n, x_dtype);
    if (st != QM_OK) return st;
    if (!x || !gate_codes || !gate_gscales || !up_codes || !up_gscales || !out_bf16)
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gemm_gate_up: null pointer");
    if (!all_aligned16({x, gate_codes, gate_gscales, up_codes, up_gscales, out_bf16}))
        return fail(c, QM_ERR_INVALID_ARG, "qm_q4_gemm_gate_up: device pointers must be 16-byte aligned");
    Q4GemmArgs ga{x, gate_codes, gate_gscales, up_codes, up_gscales, nullptr, out_bf16, nullptr, m, k, n,
                  QM_Q4_TILE(n)};
    const uint32_t grid = static_cast<uint32_t>((m + 127) / 128) * static_cast<uint32_t>((n + 127) / 128);
    return launch(c, c->f_q4_gemm[x_dtype == QM_BF16][1], grid, 256, ga, pick(c, stream), "qm_q4_gemm_gate_up");
}

}  // extern "C"
