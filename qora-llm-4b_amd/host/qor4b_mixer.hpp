// qor4b_mixer.hpp -- C++ mirror of the reference's GPU mixer interface,
// header-only, over the C ABI in include/qora_mixer.h.
//
// Names, ownership and argument meaning follow the reference's wgpu path
// (src/gpu_inference.rs, src/gpu_loader.rs) so a host port reads the same:
//   Qor4bConfig            config.rs:4-32, default_4b config.rs:42-79
//   GpuDeltaNetState       gpu_inference.rs:30-36 (state s, conv_buf, conv_pos)
//   GpuKvCacheEntry        gpu_inference.rs:38-42 (k, v, seq_len), f16 with a
//                          fixed capacity instead of a growing tensor
//   GpuDeltaNetLayer /     gpu_loader.rs:37-66, the mixer parameters only
//   GpuFullAttnLayer
//   forward_deltanet_decode_gpu  gpu_inference.rs:125-130
//   forward_attn_decode_gpu      gpu_inference.rs:247-254
//   prefill_deltanet_layer_gpu   gpu_inference.rs:436-441
//   prefill_attn_layer_gpu       gpu_inference.rs:670-677
//   GpuQ4Weight, gemv_gpu, ...   the Q4 projections around the mixer:
//                                Q4Weight gemv.rs:29-34, gemv() :286-291,
//                                fused_gate_up_gemv :304-315, rms_norm
//                                :571-579, loader repack gpu_loader.rs:82-106
// Each forward takes the projection outputs (the caller keeps in_proj /
// q/k/v_proj) and returns the mixer output (the out_proj / o_proj input).
// State and cache objects are updated in place, as the reference's &mut
// borrows are; conv_pos and seq_len advance as there (gemv.rs:769, :955,
// :1399).  Failures throw MixerError, the counterpart of the reference's
// panics, which its GPU thread turns into Err (gpu_inference.rs:950-975).
#pragma once

#include "qora_mixer.h"

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <stdexcept>
#include <string>
#include <utility>

namespace qor4b {

struct Qor4bConfig {
    std::size_t num_attn_heads = 16;
    std::size_t num_kv_heads = 4;
    std::size_t attn_head_dim = 256;
    std::size_t num_qk_heads = 16;
    std::size_t num_v_heads = 32;
    std::size_t deltanet_head_dim = 128;
    std::size_t conv_kernel_size = 4;
    double rope_theta = 10000000.0;
    float partial_rotary_factor = 0.25f;

    static Qor4bConfig default_4b() { return Qor4bConfig{}; }
    std::size_t rope_dim() const { return static_cast<std::size_t>(static_cast<float>(attn_head_dim) * partial_rotary_factor); }
    std::size_t num_kv_groups() const { return num_attn_heads / num_kv_heads; }
    std::size_t deltanet_q_dim() const { return num_qk_heads * deltanet_head_dim; }
    std::size_t deltanet_v_dim() const { return num_v_heads * deltanet_head_dim; }
    std::size_t deltanet_qkv_dim() const { return 2 * deltanet_q_dim() + deltanet_v_dim(); }
    std::size_t attn_q_dim() const { return num_attn_heads * attn_head_dim; }
    std::size_t attn_kv_dim() const { return num_kv_heads * attn_head_dim; }

    qm_config to_c() const {
        qm_config c;
        c.num_qk_heads = static_cast<int32_t>(num_qk_heads);
        c.num_v_heads = static_cast<int32_t>(num_v_heads);
        c.dn_head_dim = static_cast<int32_t>(deltanet_head_dim);
        c.conv_kernel = static_cast<int32_t>(conv_kernel_size);
        c.num_heads = static_cast<int32_t>(num_attn_heads);
        c.num_kv_heads = static_cast<int32_t>(num_kv_heads);
        c.attn_head_dim = static_cast<int32_t>(attn_head_dim);
        c.rope_dim = static_cast<int32_t>(rope_dim());
        return c;
    }
};

class MixerError : public std::runtime_error {
public:
    MixerError(int32_t code, const std::string& msg)
        : std::runtime_error(std::string(qm_status_string(code)) + ": " + msg), code_(code) {}
    int32_t code() const { return code_; }

private:
    int32_t code_;
};

class Context {
public:
    explicit Context(const Qor4bConfig& cfg = Qor4bConfig::default_4b(), int32_t device = 0,
                     const char* code_object_dir = nullptr) {
        const qm_config c = cfg.to_c();
        const int32_t st = qm_create(&h_, &c, code_object_dir, device);
        if (st != QM_OK) throw MixerError(st, qm_last_error(nullptr));
    }
    ~Context() {
        if (h_) qm_destroy(h_);
    }
    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;

    qm_context* get() const { return h_; }
    void check(int32_t st) const {
        if (st != QM_OK) throw MixerError(st, qm_last_error(h_));
    }
    void sync(qm_stream s = nullptr) const { check(qm_sync(h_, s)); }
    // Size the context's workspace once (qm_reserve), so that no later mixer
    // call allocates or synchronises to grow it.
    void reserve(int32_t max_batch, int32_t max_kv_len, int32_t max_prefill_tokens) const {
        check(qm_reserve(h_, max_batch, max_kv_len, max_prefill_tokens));
    }

private:
    qm_context* h_ = nullptr;
};

// Move-only device allocation.
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    DeviceBuffer(Context& ctx, std::size_t bytes) : ctx_(&ctx), bytes_(bytes) {
        ctx.check(qm_alloc(ctx.get(), bytes, &ptr_));
    }
    ~DeviceBuffer() { reset(); }
    DeviceBuffer(DeviceBuffer&& o) noexcept { *this = std::move(o); }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            reset();
            ctx_ = o.ctx_; ptr_ = o.ptr_; bytes_ = o.bytes_;
            o.ptr_ = nullptr; o.bytes_ = 0;
        }
        return *this;
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    template <class T> T* as() const { return static_cast<T*>(ptr_); }
    std::size_t bytes() const { return bytes_; }
    void upload(const void* host, std::size_t n) { ctx_->check(qm_memcpy_h2d(ctx_->get(), ptr_, host, n, nullptr)); }
    void download(void* host, std::size_t n) const { ctx_->check(qm_memcpy_d2h(ctx_->get(), host, ptr_, n, nullptr)); }
    void zero() { ctx_->check(qm_memset(ctx_->get(), ptr_, 0, bytes_, nullptr)); }

private:
    void reset() {
        if (ptr_ && ctx_) qm_free(ctx_->get(), ptr_);
        ptr_ = nullptr;
    }
    Context* ctx_ = nullptr;
    void* ptr_ = nullptr;
    std::size_t bytes_ = 0;
};

// gpu_inference.rs:30-36; GpuHybridCache::new zero-initialises (:54-58).
struct GpuDeltaNetState {
    DeviceBuffer s;          // f32 [num_v_heads][head_dim][head_dim]
    DeviceBuffer conv_buf;   // f32 [qkv_dim][conv_kernel_size - 1]
    std::size_t conv_pos = 0;

    static GpuDeltaNetState zeros(Context& ctx, const Qor4bConfig& cfg) {
        GpuDeltaNetState st;
        st.s = DeviceBuffer(ctx, cfg.num_v_heads * cfg.deltanet_head_dim * cfg.deltanet_head_dim * 4);
        st.conv_buf = DeviceBuffer(ctx, cfg.deltanet_qkv_dim() * (cfg.conv_kernel_size - 1) * 4);
        st.s.zero();
        st.conv_buf.zero();
        return st;
    }
};

// gpu_inference.rs:38-42, with an f16 [kv_heads][capacity][head_dim] layout.
struct GpuKvCacheEntry {
    DeviceBuffer k, v;
    std::size_t seq_len = 0;
    std::size_t capacity = 0;

    static GpuKvCacheEntry with_capacity(Context& ctx, const Qor4bConfig& cfg, std::size_t capacity) {
        GpuKvCacheEntry e;
        e.capacity = capacity;
        e.k = DeviceBuffer(ctx, cfg.num_kv_heads * capacity * cfg.attn_head_dim * 2);
        e.v = DeviceBuffer(ctx, cfg.num_kv_heads * capacity * cfg.attn_head_dim * 2);
        return e;
    }
};

// gpu_loader.rs:37-66, mixer parameters (device copies).
struct GpuDeltaNetLayer {
    DeviceBuffer conv1d_weight;     // f32 [qkv_dim][conv_kernel_size]
    DeviceBuffer a_log;             // f32 [num_v_heads]
    DeviceBuffer dt_bias;           // f32 [num_v_heads]
    DeviceBuffer attn_norm_weight;  // f16 [head_dim], plain gamma
};

struct GpuFullAttnLayer {
    DeviceBuffer q_norm;            // f16 [head_dim], (1 + gamma)
    DeviceBuffer k_norm;
};

// Mixer slice of forward_deltanet_decode_gpu: qkv is the in_proj_qkv output
// (conv1d + SiLU applied here, conv buffer shifted), a/b/z the in_proj_a/b/z
// outputs; out [v_dim] is the out_proj input.  Device pointers, one sequence.
inline void forward_deltanet_decode_gpu(Context& ctx, const float* qkv, const float* a, const float* b,
                                        const float* z, const GpuDeltaNetLayer& layer,
                                        GpuDeltaNetState& state, const Qor4bConfig& cfg, float* out,
                                        qm_stream stream = nullptr) {
    ctx.check(qm_deltanet_decode(ctx.get(), stream, 1, QM_DN_PREACT, qkv, state.conv_buf.as<float>(),
                                 layer.conv1d_weight.as<float>(), a, b, layer.a_log.as<float>(),
                                 layer.dt_bias.as<float>(), z, layer.attn_norm_weight.as<uint16_t>(),
                                 state.s.as<float>(),
                                 static_cast<int64_t>(cfg.num_v_heads * cfg.deltanet_head_dim * cfg.deltanet_head_dim),
                                 out));
    state.conv_pos += 1;
}

// Mixer slice of forward_attn_decode_gpu: q_gate [heads][2*head_dim]
// interleaved, k_new / v_new [kv_heads][head_dim]; appends at kv.seq_len.
inline void forward_attn_decode_gpu(Context& ctx, const float* q_gate, const float* k_new,
                                    const float* v_new, const GpuFullAttnLayer& layer,
                                    GpuKvCacheEntry& kv, const Qor4bConfig& cfg, const float* rope_cos,
                                    const float* rope_sin, int32_t rope_len, float* out,
                                    qm_stream stream = nullptr) {
    (void)cfg;
    ctx.check(qm_gqa_decode(ctx.get(), stream, 1, q_gate, k_new, v_new, layer.q_norm.as<uint16_t>(),
                            layer.k_norm.as<uint16_t>(), rope_cos, rope_sin, rope_len, nullptr,
                            static_cast<int32_t>(kv.seq_len), kv.k.as<uint16_t>(), kv.v.as<uint16_t>(),
                            static_cast<int64_t>(kv.capacity), out));
    kv.seq_len += 1;
}

// Mixer slice of prefill_deltanet_layer_gpu (bf16 projections in, bf16 out).
inline void prefill_deltanet_layer_gpu(Context& ctx, std::size_t seq_len, const uint16_t* qkv,
                                       const float* a, const float* b, const uint16_t* z,
                                       const GpuDeltaNetLayer& layer, GpuDeltaNetState& state,
                                       const Qor4bConfig& cfg, uint16_t* out, qm_stream stream = nullptr) {
    (void)cfg;
    ctx.check(qm_deltanet_prefill(ctx.get(), stream, static_cast<int32_t>(seq_len), qkv,
                                  state.conv_buf.as<float>(), layer.conv1d_weight.as<float>(), a, b,
                                  layer.a_log.as<float>(), layer.dt_bias.as<float>(), z,
                                  layer.attn_norm_weight.as<uint16_t>(), state.s.as<float>(), out));
    state.conv_pos += seq_len;
}

// Mixer slice of prefill_attn_layer_gpu: the cache is replaced by positions
// 0..seq_len-1 (gemv.rs:1397-1400).
inline void prefill_attn_layer_gpu(Context& ctx, std::size_t seq_len, const uint16_t* q_gate,
                                   const uint16_t* k, const uint16_t* v, const GpuFullAttnLayer& layer,
                                   GpuKvCacheEntry& kv, const Qor4bConfig& cfg, const float* rope_cos,
                                   const float* rope_sin, int32_t rope_len, uint16_t* out,
                                   qm_stream stream = nullptr) {
    (void)cfg;
    ctx.check(qm_gqa_prefill(ctx.get(), stream, static_cast<int32_t>(seq_len), q_gate, k, v,
                             layer.q_norm.as<uint16_t>(), layer.k_norm.as<uint16_t>(), rope_cos, rope_sin,
                             rope_len, kv.k.as<uint16_t>(), kv.v.as<uint16_t>(),
                             static_cast<int64_t>(kv.capacity), out));
    kv.seq_len = seq_len;
}

// ---- Q4 projections ----------------------------------------------------------

// A Q4Weight (gemv.rs:29-34) on the device: uploaded in the reference layout
// (packed [k][n/2], scales f16 [k][n/32]) and repacked there into the
// library's tile-major layout, the role q4_weight_to_gpu plays for the
// reference's backend (gpu_loader.rs:82-106).
struct GpuQ4Weight {
    DeviceBuffer codes, gscales;
    std::size_t k = 0, n = 0;

    // packed / scales are host bytes in any alignment (a file map, say)
    static GpuQ4Weight upload(Context& ctx, const void* packed, const void* scales, std::size_t k, std::size_t n) {
        const std::size_t pb = k * n / 2, sb = k * (n / 32) * 2;
        DeviceBuffer p(ctx, pb), s(ctx, sb < 16 ? 16 : sb);
        p.upload(packed, pb);
        s.upload(scales, sb);
        GpuQ4Weight w;
        w.k = k;
        w.n = n;
        w.codes = DeviceBuffer(ctx, pb);
        w.gscales = DeviceBuffer(ctx, sb < 16 ? 16 : sb);
        ctx.check(qm_q4_repack(ctx.get(), nullptr, static_cast<int32_t>(k), static_cast<int32_t>(n),
                               p.as<uint8_t>(), s.as<uint16_t>(), w.codes.as<uint8_t>(), w.gscales.as<uint16_t>()));
        ctx.sync();   // the staging copies are freed on return
        return w;
    }
    qm_q4_out out(float* y, const float* residual = nullptr) const {
        return qm_q4_out{static_cast<int32_t>(n), codes.as<uint8_t>(), gscales.as<uint16_t>(), y, residual};
    }
};

// gemv(input, &Weight::Q4) (gemv.rs:286-291): y = x W.  Device pointers.
inline void gemv_gpu(Context& ctx, const float* x, const GpuQ4Weight& w, float* y, qm_stream stream = nullptr) {
    ctx.check(qm_q4_gemv(ctx.get(), stream, static_cast<int32_t>(w.k), static_cast<int32_t>(w.n), x,
                         w.codes.as<uint8_t>(), w.gscales.as<uint16_t>(), y));
}

// x_norm = rms_norm(x, norm) followed by the gemv calls on it (up to four),
// as the top of forward_deltanet_decode (gemv.rs:740-742,788-789,865) and
// of forward_attn_decode (:926-942) do: one launch.
inline void rms_norm_gemv_gpu(Context& ctx, const float* x, const uint16_t* norm_w,
                              std::initializer_list<std::pair<const GpuQ4Weight*, float*>> outs,
                              qm_stream stream = nullptr) {
    qm_q4_out o[4];
    int32_t cnt = 0;
    std::size_t k = 0;
    for (const auto& e : outs) {
        if (cnt == 4) throw MixerError(QM_ERR_INVALID_ARG, "rms_norm_gemv_gpu: at most four weights");
        o[cnt++] = e.first->out(e.second);
        k = e.first->k;
    }
    ctx.check(qm_q4_gemv_multi(ctx.get(), stream, static_cast<int32_t>(k), x, norm_w, cnt, o));
}

// hidden += v W: the out_proj / o_proj / down_proj residual adds
// (gemv.rs:886-890,895-896); hidden is updated in place.
inline void gemv_residual_gpu(Context& ctx, const float* v, const GpuQ4Weight& w, float* hidden,
                              qm_stream stream = nullptr) {
    const qm_q4_out o = w.out(hidden, hidden);
    ctx.check(qm_q4_gemv_multi(ctx.get(), stream, static_cast<int32_t>(w.k), v, nullptr, 1, &o));
}

// fused_gate_up_gemv(rms_norm(x, norm), gate, up) (gemv.rs:893-894,304-315):
// out = silu(xn Wg) * (xn Wu); norm_w may be null (no norm).
inline void rms_norm_fused_gate_up_gpu(Context& ctx, const float* x, const uint16_t* norm_w,
                                       const GpuQ4Weight& gate, const GpuQ4Weight& up, float* out,
                                       qm_stream stream = nullptr) {
    ctx.check(qm_q4_gate_up(ctx.get(), stream, static_cast<int32_t>(gate.k), static_cast<int32_t>(gate.n), x,
                            norm_w, gate.codes.as<uint8_t>(), gate.gscales.as<uint16_t>(), up.codes.as<uint8_t>(),
                            up.gscales.as<uint16_t>(), out));
}

}  // namespace qor4b
