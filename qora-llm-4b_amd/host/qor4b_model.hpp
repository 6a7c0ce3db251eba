// qor4b_model.hpp -- a .qor4b model resident on the device and one decode
// step through it, over the C ABI (include/qora_mixer.h):
//   load_gpu_model      load_model (save.rs:247-396) + the device upload of
//                       load_gpu_model (gpu_loader.rs:69-140): every Q4
//                       projection repacked (qm_q4_repack), norms, conv and
//                       gate parameters, the vocab-major embedding and the
//                       RoPE tables copied as they are
//   GpuHybridCache      HybridCache / GpuHybridCache (gemv.rs:171-186,
//                       gpu_inference.rs:44-60): per-layer DeltaNet state or
//                       f16 KV cache of a fixed capacity
//   forward_prefill_gpu prefill (gemv.rs:1243-1283): the prompt through
//                       every layer on MFMA GEMMs and the chunked mixers,
//                       logits of the last token
//   forward_decode_gpu  forward_decode (gemv.rs:1059-1077): embedding row,
//                       the 32 layer-forwards (gemv.rs:719-900, 907-1025)
//                       with their projections, final norm and lm_head, all
//                       on the device; the token id is read from device
//                       memory, so sampling (qm_sample) can feed it directly
//   forward_decode_no_logits_gpu
//                       forward_decode_no_logits (gemv.rs:1033-1053): the
//                       same layers, no final norm and no lm_head, for a
//                       token that is already known (the forced THINK_END
//                       of generate.rs:182)
// The model must have the mixer's shape (Qor4bConfig::default_4b) and Q4
// weights; other files raise MixerError(QM_ERR_SHAPE).
#pragma once

#include "qor4b_file.hpp"
#include "qor4b_mixer.hpp"

#include <algorithm>
#include <vector>

namespace qor4b {

struct GpuDeltaNetLayerWeights {
    GpuQ4Weight in_proj_qkv, in_proj_a, in_proj_b, in_proj_z, out_proj, gate_proj, up_proj, down_proj;
    GpuDeltaNetLayer mixer;
    DeviceBuffer input_norm, post_attn_norm;   // f16 [hidden], (1 + gamma)
};

struct GpuFullAttnLayerWeights {
    GpuQ4Weight q_proj, k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj;
    GpuFullAttnLayer mixer;
    DeviceBuffer input_norm, post_attn_norm;
};

struct GpuEmbedding {
    DeviceBuffer packed, scales;               // [vocab][hidden/2], f16 [vocab][hidden/32]
    std::size_t vocab = 0, hidden = 0;
};

struct GpuModel {
    FileConfig config;
    std::vector<GpuDeltaNetLayerWeights> dn;   // the DeltaNet layers, in order
    std::vector<GpuFullAttnLayerWeights> fa;   // the attention layers, in order
    std::vector<std::size_t> slot;             // layer i -> its index in dn or fa
    GpuEmbedding embed;
    DeviceBuffer final_norm;                   // f16 [hidden]
    DeviceBuffer rope_cos, rope_sin;           // f32 [rope_len][rope_dim / 2]
    int32_t rope_len = 0;
};

namespace detail {

inline GpuQ4Weight upload_q4(Context& ctx, const WeightView& w, uint64_t k, uint64_t n, const char* what) {
    if (w.fmt != 1)
        throw MixerError(QM_ERR_SHAPE, std::string(what) + ": F16 weights are not supported (Q4 only)");
    if (w.k != k || w.n != n || w.packed.len != k * n / 2 || w.scales.len != k * (n / 32))
        throw MixerError(QM_ERR_SHAPE, std::string(what) + ": " + std::to_string(w.k) + " x " + std::to_string(w.n) +
                                           ", expected " + std::to_string(k) + " x " + std::to_string(n));
    return GpuQ4Weight::upload(ctx, w.packed.data, w.scales.data, k, n);
}

inline DeviceBuffer upload_array(Context& ctx, const ArrayView& a, uint64_t len, const char* what) {
    if (a.len != len)
        throw MixerError(QM_ERR_SHAPE, std::string(what) + ": " + std::to_string(a.len) + " elements, expected " +
                                           std::to_string(len));
    DeviceBuffer b(ctx, a.bytes() < 16 ? 16 : a.bytes());
    b.upload(a.data, a.bytes());
    return b;
}

}  // namespace detail

inline GpuModel load_gpu_model(Context& ctx, const ModelView& m) {
    const Qor4bConfig mc = Qor4bConfig::default_4b();
    const FileConfig& c = m.config;
    if (c.num_attn_heads != mc.num_attn_heads || c.num_kv_heads != mc.num_kv_heads ||
        c.attn_head_dim != mc.attn_head_dim || c.num_qk_heads != mc.num_qk_heads ||
        c.num_v_heads != mc.num_v_heads || c.deltanet_head_dim != mc.deltanet_head_dim ||
        c.conv_kernel_size != mc.conv_kernel_size || c.hidden_size % 512 != 0)
        throw MixerError(QM_ERR_SHAPE, "load_gpu_model: the file's layer shapes are not the 4B mixer's");
    const uint64_t H = c.hidden_size, I = c.intermediate_size;
    const uint64_t qkv = mc.deltanet_qkv_dim(), vd = mc.deltanet_v_dim(), nv = mc.num_v_heads;
    const uint64_t qd = mc.attn_q_dim(), kvd = mc.attn_kv_dim();
    GpuModel g;
    g.config = c;
    for (const LayerView& l : m.layers) {
        if (l.deltanet) {
            const DeltaNetLayerView& d = l.dn;
            GpuDeltaNetLayerWeights w;
            w.in_proj_qkv = detail::upload_q4(ctx, d.in_proj_qkv, H, qkv, "in_proj_qkv");
            w.in_proj_a = detail::upload_q4(ctx, d.in_proj_a, H, nv, "in_proj_a");
            w.in_proj_b = detail::upload_q4(ctx, d.in_proj_b, H, nv, "in_proj_b");
            w.in_proj_z = detail::upload_q4(ctx, d.in_proj_z, H, vd, "in_proj_z");
            w.out_proj = detail::upload_q4(ctx, d.out_proj, vd, H, "out_proj");
            w.mixer.conv1d_weight = detail::upload_array(ctx, d.conv1d_weight, qkv * mc.conv_kernel_size, "conv1d_weight");
            w.mixer.a_log = detail::upload_array(ctx, d.a_log, nv, "a_log");
            w.mixer.dt_bias = detail::upload_array(ctx, d.dt_bias, nv, "dt_bias");
            w.mixer.attn_norm_weight = detail::upload_array(ctx, d.attn_norm_weight, mc.deltanet_head_dim, "attn_norm");
            w.gate_proj = detail::upload_q4(ctx, d.gate_proj, H, I, "gate_proj");
            w.up_proj = detail::upload_q4(ctx, d.up_proj, H, I, "up_proj");
            w.down_proj = detail::upload_q4(ctx, d.down_proj, I, H, "down_proj");
            w.input_norm = detail::upload_array(ctx, d.input_norm, H, "input_norm");
            w.post_attn_norm = detail::upload_array(ctx, d.post_attn_norm, H, "post_attn_norm");
            g.slot.push_back(g.dn.size());
            g.dn.push_back(std::move(w));
        } else {
            const FullAttnLayerView& a = l.fa;
            GpuFullAttnLayerWeights w;
            w.q_proj = detail::upload_q4(ctx, a.q_proj, H, 2 * qd, "q_proj");
            w.k_proj = detail::upload_q4(ctx, a.k_proj, H, kvd, "k_proj");
            w.v_proj = detail::upload_q4(ctx, a.v_proj, H, kvd, "v_proj");
            w.o_proj = detail::upload_q4(ctx, a.o_proj, qd, H, "o_proj");
            w.mixer.q_norm = detail::upload_array(ctx, a.q_norm, mc.attn_head_dim, "q_norm");
            w.mixer.k_norm = detail::upload_array(ctx, a.k_norm, mc.attn_head_dim, "k_norm");
            w.gate_proj = detail::upload_q4(ctx, a.gate_proj, H, I, "gate_proj");
            w.up_proj = detail::upload_q4(ctx, a.up_proj, H, I, "up_proj");
            w.down_proj = detail::upload_q4(ctx, a.down_proj, I, H, "down_proj");
            w.input_norm = detail::upload_array(ctx, a.input_norm, H, "input_norm");
            w.post_attn_norm = detail::upload_array(ctx, a.post_attn_norm, H, "post_attn_norm");
            g.slot.push_back(g.fa.size());
            g.fa.push_back(std::move(w));
        }
    }
    // the embedding is used as stored (vocab-major, tied to lm_head)
    const WeightView& e = m.embed;
    if (e.fmt != 1 || e.n != H || e.packed.len != e.k * H / 2 || e.scales.len != e.k * (H / 32))
        throw MixerError(QM_ERR_SHAPE, "embed: a Q4 [vocab][hidden] weight is required");
    g.embed.vocab = e.k;
    g.embed.hidden = H;
    g.embed.packed = detail::upload_array(ctx, e.packed, e.packed.len, "embed");
    g.embed.scales = detail::upload_array(ctx, e.scales, e.scales.len, "embed scales");
    g.final_norm = detail::upload_array(ctx, m.final_norm, H, "final_norm");
    const uint64_t half = mc.rope_dim() / 2;
    if (m.rope_cos.len % half != 0 || m.rope_sin.len != m.rope_cos.len)
        throw MixerError(QM_ERR_SHAPE, "rope tables: not [positions][rope_dim / 2]");
    g.rope_len = static_cast<int32_t>(m.rope_cos.len / half);
    g.rope_cos = detail::upload_array(ctx, m.rope_cos, m.rope_cos.len, "rope_cos");
    g.rope_sin = detail::upload_array(ctx, m.rope_sin, m.rope_sin.len, "rope_sin");
    ctx.sync();
    return g;
}

// HybridCache::new (gemv.rs:175-186): zero DeltaNet states, empty KV caches
// of kv_capacity positions.
struct GpuHybridCache {
    std::vector<GpuDeltaNetState> dn;
    std::vector<GpuKvCacheEntry> kv;

    static GpuHybridCache create(Context& ctx, const GpuModel& m, std::size_t kv_capacity) {
        const Qor4bConfig cfg = Qor4bConfig::default_4b();
        if (kv_capacity < 1 || kv_capacity > 0x7fffffffu)
            throw MixerError(QM_ERR_INVALID_ARG, "GpuHybridCache: kv_capacity " + std::to_string(kv_capacity));
        // decode at any position up to the capacity: the split-K partials'
        // workspace is sized once here, not grown every 128 positions
        ctx.reserve(1, static_cast<int32_t>(kv_capacity), 0);
        GpuHybridCache c;
        for (std::size_t i = 0; i < m.dn.size(); ++i) c.dn.push_back(GpuDeltaNetState::zeros(ctx, cfg));
        for (std::size_t i = 0; i < m.fa.size(); ++i)
            c.kv.push_back(GpuKvCacheEntry::with_capacity(ctx, cfg, kv_capacity));
        return c;
    }
};

// Device buffers one decode step works in.
struct DecodeScratch {
    DeviceBuffer x, proj, a, b, z, k, v, mix, inter;

    static DecodeScratch create(Context& ctx, const GpuModel& m) {
        const Qor4bConfig cfg = Qor4bConfig::default_4b();
        DecodeScratch s;
        s.x = DeviceBuffer(ctx, m.config.hidden_size * 4);
        s.proj = DeviceBuffer(ctx, std::max(cfg.deltanet_qkv_dim(), 2 * cfg.attn_q_dim()) * 4);
        s.a = DeviceBuffer(ctx, 64 * 4);
        s.b = DeviceBuffer(ctx, 64 * 4);
        s.z = DeviceBuffer(ctx, cfg.deltanet_v_dim() * 4);
        s.k = DeviceBuffer(ctx, cfg.attn_kv_dim() * 4);
        s.v = DeviceBuffer(ctx, cfg.attn_kv_dim() * 4);
        s.mix = DeviceBuffer(ctx, std::max(cfg.deltanet_v_dim(), cfg.attn_q_dim()) * 4);
        s.inter = DeviceBuffer(ctx, m.config.intermediate_size * 4);
        return s;
    }
};

namespace detail {

// The embedding row and the 32 layer-forwards of one decode token; the
// hidden state is left in s.x.
inline void decode_layers_gpu(Context& ctx, const GpuModel& m, GpuHybridCache& cache, DecodeScratch& s,
                              const int32_t* token_dev, qm_stream stream) {
    const Qor4bConfig cfg = Qor4bConfig::default_4b();
    const int32_t H = static_cast<int32_t>(m.config.hidden_size);
    const int32_t V = static_cast<int32_t>(m.embed.vocab);
    float* x = s.x.as<float>();
    ctx.check(qm_q4_embed(ctx.get(), stream, 1, V, H, token_dev, m.embed.packed.as<uint8_t>(),
                          m.embed.scales.as<uint16_t>(), x));
    std::size_t di = 0, ai = 0;
    for (std::size_t i = 0; i < m.slot.size(); ++i) {
        if (m.config.layer_types[i] == 0) {
            // forward_deltanet_decode, gemv.rs:719-900
            const GpuDeltaNetLayerWeights& w = m.dn[m.slot[i]];
            GpuDeltaNetState& st = cache.dn[di++];
            // input norm + the four projections, with the conv1d step + SiLU
            // on in_proj_qkv (its buffer shifted there), then the mixer on
            // the activated stream
            const qm_q4_out outs[4] = {w.in_proj_qkv.out(s.proj.as<float>()), w.in_proj_z.out(s.z.as<float>()),
                                       w.in_proj_a.out(s.a.as<float>()), w.in_proj_b.out(s.b.as<float>())};
            ctx.check(qm_q4_gemv_multi_conv(ctx.get(), stream, H, x, w.input_norm.as<uint16_t>(), 4, outs,
                                            st.conv_buf.as<float>(), w.mixer.conv1d_weight.as<float>()));
            ctx.check(qm_deltanet_decode(ctx.get(), stream, 1, QM_DN_POSTACT, s.proj.as<float>(), nullptr, nullptr,
                                         s.a.as<float>(), s.b.as<float>(), w.mixer.a_log.as<float>(),
                                         w.mixer.dt_bias.as<float>(), s.z.as<float>(),
                                         w.mixer.attn_norm_weight.as<uint16_t>(), st.s.as<float>(),
                                         static_cast<int64_t>(cfg.num_v_heads * cfg.deltanet_head_dim *
                                                              cfg.deltanet_head_dim),
                                         s.mix.as<float>()));
            st.conv_pos += 1;
            gemv_residual_gpu(ctx, s.mix.as<float>(), w.out_proj, x, stream);
            rms_norm_fused_gate_up_gpu(ctx, x, w.post_attn_norm.as<uint16_t>(), w.gate_proj, w.up_proj,
                                       s.inter.as<float>(), stream);
            gemv_residual_gpu(ctx, s.inter.as<float>(), w.down_proj, x, stream);
        } else {
            // forward_attn_decode, gemv.rs:907-1025
            const GpuFullAttnLayerWeights& w = m.fa[m.slot[i]];
            rms_norm_gemv_gpu(ctx, x, w.input_norm.as<uint16_t>(),
                              {{&w.q_proj, s.proj.as<float>()}, {&w.k_proj, s.k.as<float>()},
                               {&w.v_proj, s.v.as<float>()}},
                              stream);
            forward_attn_decode_gpu(ctx, s.proj.as<float>(), s.k.as<float>(), s.v.as<float>(), w.mixer,
                                    cache.kv[ai++], cfg, m.rope_cos.as<float>(), m.rope_sin.as<float>(),
                                    m.rope_len, s.mix.as<float>(), stream);
            gemv_residual_gpu(ctx, s.mix.as<float>(), w.o_proj, x, stream);
            rms_norm_fused_gate_up_gpu(ctx, x, w.post_attn_norm.as<uint16_t>(), w.gate_proj, w.up_proj,
                                       s.inter.as<float>(), stream);
            gemv_residual_gpu(ctx, s.inter.as<float>(), w.down_proj, x, stream);
        }
    }
}

}  // namespace detail

// forward_decode (gemv.rs:1059-1077): logits [vocab] for the token whose id
// is at token_dev (device int32), with every layer's state / KV cache
// advanced by one position.
inline void forward_decode_gpu(Context& ctx, const GpuModel& m, GpuHybridCache& cache, DecodeScratch& s,
                               const int32_t* token_dev, float* logits_dev, qm_stream stream = nullptr) {
    if (!logits_dev) throw MixerError(QM_ERR_INVALID_ARG, "forward_decode_gpu: null logits");
    detail::decode_layers_gpu(ctx, m, cache, s, token_dev, stream);
    const int32_t H = static_cast<int32_t>(m.config.hidden_size);
    const int32_t V = static_cast<int32_t>(m.embed.vocab);
    ctx.check(qm_q4_lm_head(ctx.get(), stream, V, H, s.x.as<float>(), m.final_norm.as<uint16_t>(),
                            m.embed.packed.as<uint8_t>(), m.embed.scales.as<uint16_t>(), logits_dev));
}

// forward_decode_no_logits (gemv.rs:1033-1053): every layer's state / KV
// cache advanced by the token at token_dev, without the final norm and the
// 248,320-row lm_head (the caller already knows the next token).
inline void forward_decode_no_logits_gpu(Context& ctx, const GpuModel& m, GpuHybridCache& cache,
                                         DecodeScratch& s, const int32_t* token_dev, qm_stream stream = nullptr) {
    detail::decode_layers_gpu(ctx, m, cache, s, token_dev, stream);
}

// Device buffers a prefill of up to max_tokens works in.
struct PrefillScratch {
    DeviceBuffer x, xn16, proj16, z16, a, b, k16, v16, mix16, inter_bf16;
    std::size_t max_tokens = 0;

    static PrefillScratch create(Context& ctx, const GpuModel& m, std::size_t max_tokens) {
        const Qor4bConfig cfg = Qor4bConfig::default_4b();
        const std::size_t T = max_tokens, H = m.config.hidden_size;
        if (T < 1 || T > 0x7fffffffu)
            throw MixerError(QM_ERR_INVALID_ARG, "PrefillScratch: max_tokens " + std::to_string(T));
        ctx.reserve(1, 0, static_cast<int32_t>(T));   // the chunked mixers' workspace
        PrefillScratch s;
        s.max_tokens = T;
        s.x = DeviceBuffer(ctx, T * H * 4);
        s.xn16 = DeviceBuffer(ctx, T * H * 2);
        s.proj16 = DeviceBuffer(ctx, T * std::max(cfg.deltanet_qkv_dim(), 2 * cfg.attn_q_dim()) * 2);
        s.z16 = DeviceBuffer(ctx, T * cfg.deltanet_v_dim() * 2);
        s.a = DeviceBuffer(ctx, T * cfg.num_v_heads * 4);
        s.b = DeviceBuffer(ctx, T * cfg.num_v_heads * 4);
        s.k16 = DeviceBuffer(ctx, T * cfg.attn_kv_dim() * 2);
        s.v16 = DeviceBuffer(ctx, T * cfg.attn_kv_dim() * 2);
        s.mix16 = DeviceBuffer(ctx, T * std::max(cfg.deltanet_v_dim(), cfg.attn_q_dim()) * 2);
        s.inter_bf16 = DeviceBuffer(ctx, T * m.config.intermediate_size * 2);
        return s;
    }
};

// prefill (gemv.rs:1243-1283): the tokens_dev [T] prompt through every
// layer on MFMA (prefill_deltanet_layer, gemv.rs:1086-1240;
// prefill_attn_layer, :1339-1470), each projection one qm_q4_gemm over all
// T rows (f16 inputs from qm_rms_norm_f16, bf16 mixer inputs and outputs
// and MLP intermediate,
// the hidden state f32 with the residuals added in the GEMM epilogues),
// the MLP's gate/up as one launch; then the final norm and lm_head of the
// last token into logits_dev.  DeltaNet states and conv buffers continue
// from where they are; KV caches are replaced by positions 0 .. T-1.
inline void forward_prefill_gpu(Context& ctx, const GpuModel& m, GpuHybridCache& cache, PrefillScratch& s,
                                const int32_t* tokens_dev, int32_t T, float* logits_dev, qm_stream stream = nullptr) {
    if (T < 1 || static_cast<std::size_t>(T) > s.max_tokens)
        throw MixerError(QM_ERR_INVALID_ARG, "forward_prefill_gpu: " + std::to_string(T) + " tokens, scratch holds " +
                                                 std::to_string(s.max_tokens));
    const Qor4bConfig cfg = Qor4bConfig::default_4b();
    const int32_t H = static_cast<int32_t>(m.config.hidden_size), I = static_cast<int32_t>(m.config.intermediate_size);
    const int32_t V = static_cast<int32_t>(m.embed.vocab);
    float* x = s.x.as<float>();
    uint16_t* xn = s.xn16.as<uint16_t>();
    auto gemm = [&](const uint16_t* in, int32_t x_dtype, const GpuQ4Weight& w, float* y, uint16_t* y_bf16,
                    const float* residual) {
        ctx.check(qm_q4_gemm(ctx.get(), stream, T, static_cast<int32_t>(w.k), static_cast<int32_t>(w.n), in, x_dtype,
                             w.codes.as<uint8_t>(), w.gscales.as<uint16_t>(), residual, y, y_bf16));
    };
    auto mlp = [&](const DeviceBuffer& post_norm, const GpuQ4Weight& gate, const GpuQ4Weight& up,
                   const GpuQ4Weight& down) {
        ctx.check(qm_rms_norm_f16(ctx.get(), stream, T, H, x, post_norm.as<uint16_t>(), xn));
        ctx.check(qm_q4_gemm_gate_up(ctx.get(), stream, T, H, I, xn, QM_F16, gate.codes.as<uint8_t>(),
                                     gate.gscales.as<uint16_t>(), up.codes.as<uint8_t>(), up.gscales.as<uint16_t>(),
                                     s.inter_bf16.as<uint16_t>()));
        gemm(s.inter_bf16.as<uint16_t>(), QM_BF16, down, x, nullptr, x);
    };
    ctx.check(qm_q4_embed(ctx.get(), stream, T, V, H, tokens_dev, m.embed.packed.as<uint8_t>(),
                          m.embed.scales.as<uint16_t>(), x));
    std::size_t di = 0, ai = 0;
    for (std::size_t i = 0; i < m.slot.size(); ++i) {
        if (m.config.layer_types[i] == 0) {
            const GpuDeltaNetLayerWeights& w = m.dn[m.slot[i]];
            GpuDeltaNetState& st = cache.dn[di++];
            ctx.check(qm_rms_norm_f16(ctx.get(), stream, T, H, x, w.input_norm.as<uint16_t>(), xn));
            gemm(xn, QM_F16, w.in_proj_qkv, nullptr, s.proj16.as<uint16_t>(), nullptr);
            gemm(xn, QM_F16, w.in_proj_z, nullptr, s.z16.as<uint16_t>(), nullptr);
            gemm(xn, QM_F16, w.in_proj_a, s.a.as<float>(), nullptr, nullptr);
            gemm(xn, QM_F16, w.in_proj_b, s.b.as<float>(), nullptr, nullptr);
            prefill_deltanet_layer_gpu(ctx, static_cast<std::size_t>(T), s.proj16.as<uint16_t>(), s.a.as<float>(),
                                       s.b.as<float>(), s.z16.as<uint16_t>(), w.mixer, st, cfg,
                                       s.mix16.as<uint16_t>(), stream);
            gemm(s.mix16.as<uint16_t>(), QM_BF16, w.out_proj, x, nullptr, x);
            mlp(w.post_attn_norm, w.gate_proj, w.up_proj, w.down_proj);
        } else {
            const GpuFullAttnLayerWeights& w = m.fa[m.slot[i]];
            ctx.check(qm_rms_norm_f16(ctx.get(), stream, T, H, x, w.input_norm.as<uint16_t>(), xn));
            gemm(xn, QM_F16, w.q_proj, nullptr, s.proj16.as<uint16_t>(), nullptr);
            gemm(xn, QM_F16, w.k_proj, nullptr, s.k16.as<uint16_t>(), nullptr);
            gemm(xn, QM_F16, w.v_proj, nullptr, s.v16.as<uint16_t>(), nullptr);
            prefill_attn_layer_gpu(ctx, static_cast<std::size_t>(T), s.proj16.as<uint16_t>(), s.k16.as<uint16_t>(),
                                   s.v16.as<uint16_t>(), w.mixer, cache.kv[ai++], cfg, m.rope_cos.as<float>(),
                                   m.rope_sin.as<float>(), m.rope_len, s.mix16.as<uint16_t>(), stream);
            gemm(s.mix16.as<uint16_t>(), QM_BF16, w.o_proj, x, nullptr, x);
            mlp(w.post_attn_norm, w.gate_proj, w.up_proj, w.down_proj);
        }
    }
    ctx.check(qm_q4_lm_head(ctx.get(), stream, V, H, x + static_cast<std::size_t>(T - 1) * H,
                            m.final_norm.as<uint16_t>(), m.embed.packed.as<uint8_t>(), m.embed.scales.as<uint16_t>(),
                            logits_dev));
}

}  // namespace qor4b
