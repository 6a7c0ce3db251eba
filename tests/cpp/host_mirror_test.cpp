// host_mirror_test.cpp -- runs the reference's layer flow through the C++
// mirror (qor4b_mixer.hpp): a DeltaNet layer and a GQA layer each prefill a
// prompt and then decode tokens, carrying state / conv buffer / KV cache
// from prefill into decode as generate.rs does (prefill at :243, decode
// loop at :126).  Every output is checked against the CPU oracle
// (test infrastructure, linked only here).  Exit status 0 = all checks pass.
#include "qor4b_model.hpp"
#include "qor4b_writer.hpp"
#include "qora_oracle.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unistd.h>
#include <vector>

using namespace qor4b;

namespace {

struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
    float normal() { return static_cast<float>(std::sqrt(-2.0 * std::log(uniform())) * std::cos(6.283185307179586 * uniform())); }
};

std::vector<float> normals(Rng& r, std::size_t n, float std = 1.0f) {
    std::vector<float> v(n);
    for (auto& x : v) x = std * r.normal();
    return v;
}
std::vector<uint16_t> to_bf16(const std::vector<float>& v) {
    std::vector<uint16_t> o(v.size());
    for (std::size_t i = 0; i < v.size(); ++i) o[i] = or_f32_to_bf16(v[i]);
    return o;
}
std::vector<float> from_bf16(const std::vector<uint16_t>& v) {
    std::vector<float> o(v.size());
    for (std::size_t i = 0; i < v.size(); ++i) o[i] = or_bf16_to_f32(v[i]);
    return o;
}
std::vector<uint16_t> to_f16(const std::vector<float>& v) {
    std::vector<uint16_t> o(v.size());
    for (std::size_t i = 0; i < v.size(); ++i) o[i] = or_f32_to_f16(v[i]);
    return o;
}
template <class T>
DeviceBuffer upload(Context& ctx, const std::vector<T>& v) {
    DeviceBuffer b(ctx, v.size() * sizeof(T));
    b.upload(v.data(), v.size() * sizeof(T));
    return b;
}
double rel_err(const float* got, const float* ref, std::size_t n) {
    double e = 0, m = 0;
    for (std::size_t i = 0; i < n; ++i) {
        e = std::fmax(e, std::fabs((double)got[i] - ref[i]));
        m = std::fmax(m, std::fabs((double)ref[i]));
    }
    return m > 0 ? e / m : e;
}
double abs_err(const float* got, const float* ref, std::size_t n) {
    double e = 0;
    for (std::size_t i = 0; i < n; ++i) e = std::fmax(e, std::fabs((double)got[i] - ref[i]));
    return e;
}

int failures = 0;
void expect(bool ok, const char* what, double v, double bar) {
    std::printf("%-52s %.3e (bar %.0e) %s\n", what, v, bar, ok ? "ok" : "FAIL");
    if (!ok) ++failures;
}

or_config oracle_cfg(const Qor4bConfig& c) {
    or_config o;
    o.num_qk_heads = (int32_t)c.num_qk_heads; o.num_v_heads = (int32_t)c.num_v_heads;
    o.dn_head_dim = (int32_t)c.deltanet_head_dim; o.conv_kernel = (int32_t)c.conv_kernel_size;
    o.num_heads = (int32_t)c.num_attn_heads; o.num_kv_heads = (int32_t)c.num_kv_heads;
    o.attn_head_dim = (int32_t)c.attn_head_dim; o.rope_dim = (int32_t)c.rope_dim();
    return o;
}

void deltanet_flow(Context& ctx, const Qor4bConfig& cfg) {
    const std::size_t T = 100, steps = 4;
    const std::size_t qkv_dim = cfg.deltanet_qkv_dim(), v_dim = cfg.deltanet_v_dim(), nv = cfg.num_v_heads;
    Rng r(11);
    std::vector<float> conv_w = normals(r, qkv_dim * 4, 0.5f);
    std::vector<float> a_log(nv), dt_bias(nv, 0.0f);
    for (auto& x : a_log) x = std::log(0.01f + 0.09f * (float)r.uniform());
    std::vector<float> gamma = normals(r, cfg.deltanet_head_dim, 0.1f);
    for (auto& x : gamma) x += 1.0f;
    std::vector<uint16_t> norm_w = to_f16(gamma);

    GpuDeltaNetLayer layer{upload(ctx, conv_w), upload(ctx, a_log), upload(ctx, dt_bias), upload(ctx, norm_w)};
    GpuDeltaNetState state = GpuDeltaNetState::zeros(ctx, cfg);

    // prefill (bf16 projections)
    std::vector<uint16_t> qkv_p = to_bf16(normals(r, T * qkv_dim)), z_p = to_bf16(normals(r, T * v_dim));
    std::vector<float> a_p = normals(r, T * nv), b_p = normals(r, T * nv);
    DeviceBuffer d_qkv = upload(ctx, qkv_p), d_z = upload(ctx, z_p), d_a = upload(ctx, a_p), d_b = upload(ctx, b_p);
    DeviceBuffer d_out(ctx, T * v_dim * 2);
    prefill_deltanet_layer_gpu(ctx, T, d_qkv.as<uint16_t>(), d_a.as<float>(), d_b.as<float>(), d_z.as<uint16_t>(),
                               layer, state, cfg, d_out.as<uint16_t>());
    std::vector<uint16_t> out_p(T * v_dim);
    d_out.download(out_p.data(), out_p.size() * 2);

    const or_config oc = oracle_cfg(cfg);
    std::vector<float> S(nv * cfg.deltanet_head_dim * cfg.deltanet_head_dim, 0.0f), buf(qkv_dim * 3, 0.0f);
    std::vector<float> ref_p(T * v_dim);
    std::vector<float> qkv_pf = from_bf16(qkv_p), z_pf = from_bf16(z_p);
    or_deltanet_prefill(&oc, (int32_t)T, qkv_pf.data(), a_p.data(), b_p.data(), z_pf.data(), buf.data(),
                        conv_w.data(), a_log.data(), dt_bias.data(), norm_w.data(), S.data(), ref_p.data());
    std::vector<float> got_p = from_bf16(out_p);
    const double ep = rel_err(got_p.data(), ref_p.data(), got_p.size());
    expect(ep <= 2e-2, "deltanet prefill T=100: rel out", ep, 2e-2);

    // decode steps continue from the prefilled state and conv buffer
    double ed = 0;
    for (std::size_t s = 0; s < steps; ++s) {
        std::vector<float> qkv = normals(r, qkv_dim), a = normals(r, nv), b = normals(r, nv), z = normals(r, v_dim);
        DeviceBuffer dq = upload(ctx, qkv), da = upload(ctx, a), db = upload(ctx, b), dz = upload(ctx, z);
        DeviceBuffer dout(ctx, v_dim * 4);
        forward_deltanet_decode_gpu(ctx, dq.as<float>(), da.as<float>(), db.as<float>(), dz.as<float>(), layer,
                                    state, cfg, dout.as<float>());
        std::vector<float> got(v_dim), ref(v_dim);
        dout.download(got.data(), got.size() * 4);
        or_deltanet_decode_step(&oc, qkv.data(), 1, buf.data(), conv_w.data(), a.data(), b.data(), a_log.data(),
                                dt_bias.data(), z.data(), norm_w.data(), S.data(), ref.data(), OR_UPDATE_AUTO);
        ed = std::fmax(ed, rel_err(got.data(), ref.data(), v_dim));
    }
    expect(ed <= 2e-2, "deltanet decode x4 after prefill: rel out", ed, 2e-2);
    std::vector<float> Sg(S.size()), bufg(buf.size());
    state.s.download(Sg.data(), Sg.size() * 4);
    state.conv_buf.download(bufg.data(), bufg.size() * 4);
    expect(rel_err(Sg.data(), S.data(), S.size()) <= 2e-2, "deltanet state after prefill+decode: rel",
           rel_err(Sg.data(), S.data(), S.size()), 2e-2);
    expect(std::memcmp(bufg.data(), buf.data(), buf.size() * 4) == 0, "deltanet conv buffer exact (mismatch = 1)",
           std::memcmp(bufg.data(), buf.data(), buf.size() * 4) != 0, 0.5);
    expect(state.conv_pos == T + steps, "deltanet conv_pos advanced (error = |diff|)",
           std::fabs((double)state.conv_pos - (double)(T + steps)), 0.5);
}

void attention_flow(Context& ctx, const Qor4bConfig& cfg) {
    const std::size_t S = 50, steps = 3, cap = 64;
    const std::size_t H = cfg.num_attn_heads, KV = cfg.num_kv_heads, D = cfg.attn_head_dim;
    Rng r(12);
    const int32_t rope_len = 128;
    std::vector<float> cos_t(rope_len * cfg.rope_dim() / 2), sin_t(cos_t.size());
    ctx.check(qm_rope_table(cfg.rope_theta, (int32_t)cfg.rope_dim(), rope_len, cos_t.data(), sin_t.data()));
    DeviceBuffer d_cos = upload(ctx, cos_t), d_sin = upload(ctx, sin_t);
    std::vector<uint16_t> qn = to_f16(normals(r, D, 0.1f)), kn = to_f16(normals(r, D, 0.1f));
    GpuFullAttnLayer layer{upload(ctx, qn), upload(ctx, kn)};
    GpuKvCacheEntry kv = GpuKvCacheEntry::with_capacity(ctx, cfg, cap);

    std::vector<uint16_t> qg = to_bf16(normals(r, S * H * 2 * D)), k = to_bf16(normals(r, S * KV * D)),
                          v = to_bf16(normals(r, S * KV * D));
    DeviceBuffer d_qg = upload(ctx, qg), d_k = upload(ctx, k), d_v = upload(ctx, v);
    DeviceBuffer d_out(ctx, S * H * D * 2);
    prefill_attn_layer_gpu(ctx, S, d_qg.as<uint16_t>(), d_k.as<uint16_t>(), d_v.as<uint16_t>(), layer, kv, cfg,
                           d_cos.as<float>(), d_sin.as<float>(), rope_len, d_out.as<uint16_t>());
    std::vector<uint16_t> out_b(S * H * D);
    d_out.download(out_b.data(), out_b.size() * 2);

    const or_config oc = oracle_cfg(cfg);
    std::vector<float> qgf = from_bf16(qg), kf = from_bf16(k), vf = from_bf16(v);
    std::vector<float> Kc(cap * KV * D, 0.0f), Vc(cap * KV * D, 0.0f), ref(S * H * D);
    or_attn_prefill(&oc, (int32_t)S, qgf.data(), kf.data(), vf.data(), qn.data(), kn.data(), cos_t.data(),
                    sin_t.data(), rope_len, Kc.data(), Vc.data(), ref.data(), nullptr, 0, 4);
    std::vector<float> got = from_bf16(out_b);
    const double ep = rel_err(got.data(), ref.data(), got.size());
    expect(ep <= 2e-2, "gqa prefill S=50: rel out", ep, 2e-2);
    // the MI355X cache holds f16: decode in the oracle reads the same rounding
    for (std::size_t i = 0; i < S * KV * D; ++i) {
        Kc[i] = or_f16_to_f32(or_f32_to_f16(Kc[i]));
        Vc[i] = or_f16_to_f32(or_f32_to_f16(Vc[i]));
    }
    double ed = 0;
    for (std::size_t s = 0; s < steps; ++s) {
        std::vector<float> q_gate = normals(r, H * 2 * D), k_new = normals(r, KV * D), v_new = normals(r, KV * D);
        DeviceBuffer dq = upload(ctx, q_gate), dk = upload(ctx, k_new), dv = upload(ctx, v_new);
        DeviceBuffer dout(ctx, H * D * 4);
        const std::size_t pos = kv.seq_len;
        forward_attn_decode_gpu(ctx, dq.as<float>(), dk.as<float>(), dv.as<float>(), layer, kv, cfg,
                                d_cos.as<float>(), d_sin.as<float>(), rope_len, dout.as<float>());
        std::vector<float> g(H * D), rf(H * D);
        dout.download(g.data(), g.size() * 4);
        or_attn_decode_step(&oc, q_gate.data(), k_new.data(), v_new.data(), qn.data(), kn.data(), cos_t.data(),
                            sin_t.data(), rope_len, Kc.data(), Vc.data(), (int32_t)pos, 1, rf.data(), 4);
        ed = std::fmax(ed, abs_err(g.data(), rf.data(), g.size()));
    }
    expect(ed <= 1e-3, "gqa decode x3 after prefill: max-abs out", ed, 1e-3);
    expect(kv.seq_len == S + steps, "gqa kv seq_len advanced (error = |diff|)",
           std::fabs((double)kv.seq_len - (double)(S + steps)), 0.5);
    // a position past the RoPE table is an error, not a fault (gemv.rs:620-621 panics)
    bool raised = false;
    try {
        kv.seq_len = rope_len;
        std::vector<float> z(H * 2 * D, 0.0f);
        DeviceBuffer dz = upload(ctx, z);
        forward_attn_decode_gpu(ctx, dz.as<float>(), dz.as<float>(), dz.as<float>(), layer, kv, cfg,
                                d_cos.as<float>(), d_sin.as<float>(), rope_len, dz.as<float>());
    } catch (const MixerError& e) {
        raised = e.code() == QM_ERR_ROPE_RANGE;
    }
    expect(raised, "gqa decode past the RoPE table raises (missing = 1)", raised ? 0 : 1, 0.5);
}

// The Q4 projections of one DeltaNet decode layer through the mirror
// (gemv.rs:740-742,788-789,865,886-897) against the oracle's rms_norm and
// gemv_q4_inner restatements: qkv/z/a/b of the normed input, the out_proj
// residual, and the MLP (normed gate/up, down residual).
void q4_layer_flow(Context& ctx) {
    Rng r(23);
    const std::size_t H = 2560;
    struct Shape { std::size_t k, n; };
    const Shape sh[8] = {{H, 8192}, {H, 4096}, {H, 32}, {H, 32}, {4096, H}, {H, 9216}, {H, 9216}, {9216, H}};
    std::vector<std::vector<uint8_t>> packed(8);
    std::vector<std::vector<uint16_t>> scales(8);
    std::vector<GpuQ4Weight> w;
    for (int i = 0; i < 8; ++i) {
        std::vector<float> f = normals(r, sh[i].k * sh[i].n, 0.02f);
        packed[i].resize(sh[i].k * sh[i].n / 2);
        scales[i].resize(sh[i].k * sh[i].n / 32);
        or_q4_quantize(f.data(), (int32_t)sh[i].k, (int32_t)sh[i].n, packed[i].data(), scales[i].data());
        w.push_back(GpuQ4Weight::upload(ctx, packed[i].data(), scales[i].data(), sh[i].k, sh[i].n));
    }
    std::vector<float> x = normals(r, H), mix = normals(r, 4096);
    std::vector<float> g1 = normals(r, H, 0.1f), g2 = normals(r, H, 0.1f);
    std::vector<uint16_t> n1 = to_f16(g1), n2 = to_f16(g2);
    DeviceBuffer dx = upload(ctx, x), dmix = upload(ctx, mix), dn1 = upload(ctx, n1), dn2 = upload(ctx, n2);
    DeviceBuffer y0(ctx, 8192 * 4), y1(ctx, 4096 * 4), y2(ctx, 32 * 4), y3(ctx, 32 * 4), inter(ctx, 9216 * 4);
    DeviceBuffer h = upload(ctx, x);

    rms_norm_gemv_gpu(ctx, dx.as<float>(), dn1.as<uint16_t>(),
                      {{&w[0], y0.as<float>()}, {&w[1], y1.as<float>()}, {&w[2], y2.as<float>()},
                       {&w[3], y3.as<float>()}});
    gemv_residual_gpu(ctx, dmix.as<float>(), w[4], h.as<float>());
    rms_norm_fused_gate_up_gpu(ctx, h.as<float>(), dn2.as<uint16_t>(), w[5], w[6], inter.as<float>());
    // down_proj residual is checked against the GPU's own MLP input
    std::vector<float> inter_g(9216), h_mid(H);
    inter.download(inter_g.data(), 9216 * 4);
    h.download(h_mid.data(), H * 4);
    gemv_residual_gpu(ctx, inter.as<float>(), w[7], h.as<float>());
    ctx.sync();

    std::vector<float> xn(H), ref(9216), got(9216);
    or_rms_norm(x.data(), (int32_t)H, n1.data(), xn.data());
    DeviceBuffer* ys[4] = {&y0, &y1, &y2, &y3};
    const char* names[4] = {"q4 rms_norm + in_proj_qkv (rel)", "q4 rms_norm + in_proj_z (rel)",
                            "q4 rms_norm + in_proj_a (rel)", "q4 rms_norm + in_proj_b (rel)"};
    for (int i = 0; i < 4; ++i) {
        or_q4_gemv(xn.data(), packed[i].data(), scales[i].data(), (int32_t)H, (int32_t)sh[i].n, ref.data());
        ys[i]->download(got.data(), sh[i].n * 4);
        const double e = rel_err(got.data(), ref.data(), sh[i].n);
        expect(e <= 1e-5, names[i], e, 1e-5);
    }
    // out_proj residual: h = x + mix W
    or_q4_gemv(mix.data(), packed[4].data(), scales[4].data(), 4096, (int32_t)H, ref.data());
    for (std::size_t j = 0; j < H; ++j) ref[j] += x[j];
    double e = rel_err(h_mid.data(), ref.data(), H);
    expect(e <= 1e-5, "q4 out_proj + residual (rel)", e, 1e-5);
    // MLP gate/up on rms_norm(h)
    std::vector<float> hn(H);
    or_rms_norm(h_mid.data(), (int32_t)H, n2.data(), hn.data());
    or_q4_gate_up(hn.data(), packed[5].data(), scales[5].data(), packed[6].data(), scales[6].data(), (int32_t)H,
                  9216, ref.data());
    e = rel_err(inter_g.data(), ref.data(), 9216);
    expect(e <= 1e-4, "q4 rms_norm + gate/up + silu (rel)", e, 1e-4);
    // down_proj residual
    or_q4_gemv(inter_g.data(), packed[7].data(), scales[7].data(), 9216, (int32_t)H, ref.data());
    for (std::size_t j = 0; j < H; ++j) ref[j] += h_mid[j];
    h.download(got.data(), H * 4);
    e = rel_err(got.data(), ref.data(), H);
    expect(e <= 1e-5, "q4 down_proj + residual (rel)", e, 1e-5);
}

// A two-layer model of the 4B's shapes (one DeltaNet layer, one attention
// layer, a 4096-token vocabulary) written as a .qor4b file, loaded onto the
// device (load_gpu_model) and decoded for a few tokens with forward_decode_gpu
// and greedy qm_sample, the sampled id feeding the next step on the device.
// Each step's logits are checked against the oracle's forward_decode
// (gemv.rs:1059-1077) composed from its restatements.
void model_flow(Context& ctx, const Qor4bConfig& cfg) {
    using namespace qor4b_test;
    Rng r(31);
    const uint32_t H = 2560, I = 9216, V = 4096;
    auto q4w = [&](uint64_t k, uint64_t n) {
        W w;
        w.k = k;
        w.n = n;
        w.packed.resize(k * n / 2);
        w.scales.resize(k * (n / 32));
        for (std::size_t i = 0; i < w.packed.size(); i += 8) {
            const uint64_t b = r.next();
            std::memcpy(&w.packed[i], &b, std::min<std::size_t>(8, w.packed.size() - i));
        }
        for (auto& x : w.scales) x = or_f32_to_f16(0.006f * (1.0f + 0.2f * r.normal()));
        return w;
    };
    auto f16v = [&](std::size_t n, float mean, float sd) {
        std::vector<uint16_t> v(n);
        for (auto& x : v) x = or_f32_to_f16(mean + sd * r.normal());
        return v;
    };
    Model m;
    m.vocab = V;
    m.hidden = H;
    m.intermediate = I;
    m.layer_types = {0, 1};
    DnLayer d;
    d.in_proj_qkv = q4w(H, cfg.deltanet_qkv_dim());
    d.in_proj_a = q4w(H, cfg.num_v_heads);
    d.in_proj_b = q4w(H, cfg.num_v_heads);
    d.in_proj_z = q4w(H, cfg.deltanet_v_dim());
    d.out_proj = q4w(cfg.deltanet_v_dim(), H);
    d.conv1d_weight = normals(r, cfg.deltanet_qkv_dim() * 4, 0.5f);
    d.a_log.resize(cfg.num_v_heads);
    for (auto& x : d.a_log) x = std::log(0.01f + 0.09f * (float)r.uniform());
    d.dt_bias.assign(cfg.num_v_heads, 0.0f);
    d.attn_norm_weight = f16v(cfg.deltanet_head_dim, 1.0f, 0.1f);
    d.gate_proj = q4w(H, I);
    d.up_proj = q4w(H, I);
    d.down_proj = q4w(I, H);
    d.input_norm = f16v(H, 0.0f, 0.1f);
    d.post_attn_norm = f16v(H, 0.0f, 0.1f);
    m.dn.push_back(std::move(d));
    FaLayer a;
    a.q_proj = q4w(H, 2 * cfg.attn_q_dim());
    a.k_proj = q4w(H, cfg.attn_kv_dim());
    a.v_proj = q4w(H, cfg.attn_kv_dim());
    a.o_proj = q4w(cfg.attn_q_dim(), H);
    a.q_norm = f16v(cfg.attn_head_dim, 0.0f, 0.1f);
    a.k_norm = f16v(cfg.attn_head_dim, 0.0f, 0.1f);
    a.gate_proj = q4w(H, I);
    a.up_proj = q4w(H, I);
    a.down_proj = q4w(I, H);
    a.input_norm = f16v(H, 0.0f, 0.1f);
    a.post_attn_norm = f16v(H, 0.0f, 0.1f);
    m.fa.push_back(std::move(a));
    m.embed = q4w(V, H);
    for (auto& x : m.embed.scales) x = or_f32_to_f16(0.02f * (1.0f + 0.2f * r.normal()));
    m.final_norm = f16v(H, 0.0f, 0.1f);
    const int32_t rope_len = 8192, half = (int32_t)cfg.rope_dim() / 2;
    m.rope_cos.resize((std::size_t)rope_len * half);
    m.rope_sin.resize((std::size_t)rope_len * half);
    or_rope_table(m.rope_theta, (int32_t)cfg.rope_dim(), rope_len, m.rope_cos.data(), m.rope_sin.data());

    const char* tmp = std::getenv("TMPDIR");
    std::string path = std::string(tmp && *tmp ? tmp : "/tmp") + "/qor4b_model_flow_XXXXXX";
    std::vector<char> pbuf(path.begin(), path.end());
    pbuf.push_back('\0');
    const int fd = mkstemp(pbuf.data());
    if (fd < 0) throw std::runtime_error("model_flow: no temporary file");
    close(fd);
    path = pbuf.data();
    const bool written = write_file(path, serialize(m));
    expect(written, "model file written (failed = 1)", written ? 0 : 1, 0.5);
    GpuModel gm;
    {
        MappedFile f(path);
        gm = load_gpu_model(ctx, parse_qor4b(f.data(), f.size()));
    }
    unlink(path.c_str());
    GpuHybridCache cache = GpuHybridCache::create(ctx, gm, 64);
    DecodeScratch scratch = DecodeScratch::create(ctx, gm);
    DeviceBuffer tok(ctx, 16), logits(ctx, V * 4);
    const int32_t first = 1234;
    tok.upload(&first, 4);

    // the oracle's forward_decode over the same weights
    const or_config oc = oracle_cfg(cfg);
    const DnLayer& od = m.dn[0];
    const FaLayer& oa = m.fa[0];
    std::vector<float> S(cfg.num_v_heads * cfg.deltanet_head_dim * cfg.deltanet_head_dim, 0.0f);
    std::vector<float> buf(cfg.deltanet_qkv_dim() * 3, 0.0f);
    std::vector<float> Kc, Vc;
    auto gemv = [](const std::vector<float>& x, const W& w) {
        std::vector<float> y(w.n);
        or_q4_gemv(x.data(), w.packed.data(), w.scales.data(), (int32_t)w.k, (int32_t)w.n, y.data());
        return y;
    };
    auto rms = [](const std::vector<float>& x, const std::vector<uint16_t>& g) {
        std::vector<float> y(x.size());
        or_rms_norm(x.data(), (int32_t)x.size(), g.data(), y.data());
        return y;
    };
    auto mlp = [&](std::vector<float>& x, const std::vector<uint16_t>& norm, const W& g, const W& u, const W& dw) {
        const std::vector<float> xn = rms(x, norm);
        std::vector<float> inter(I);
        or_q4_gate_up(xn.data(), g.packed.data(), g.scales.data(), u.packed.data(), u.scales.data(), (int32_t)H,
                      (int32_t)I, inter.data());
        const std::vector<float> y = gemv(inter, dw);
        for (uint32_t j = 0; j < H; ++j) x[j] += y[j];
    };
    double worst = 0;
    int32_t id = first;
    bool greedy_ok = true;
    const int steps = 4;
    for (int step = 0; step < steps; ++step) {
        forward_decode_gpu(ctx, gm, cache, scratch, tok.as<int32_t>(), logits.as<float>());
        std::vector<float> got(V);
        logits.download(got.data(), V * 4);

        std::vector<float> x(H);
        or_q4_embed(m.embed.packed.data(), m.embed.scales.data(), (int32_t)H, id, x.data());
        {   // forward_deltanet_decode
            const std::vector<float> xn = rms(x, od.input_norm);
            const std::vector<float> qkv = gemv(xn, od.in_proj_qkv), av = gemv(xn, od.in_proj_a),
                                     bv = gemv(xn, od.in_proj_b), zv = gemv(xn, od.in_proj_z);
            std::vector<float> out(cfg.deltanet_v_dim());
            or_deltanet_decode_step(&oc, qkv.data(), 1, buf.data(), od.conv1d_weight.data(), av.data(), bv.data(),
                                    od.a_log.data(), od.dt_bias.data(), zv.data(), od.attn_norm_weight.data(),
                                    S.data(), out.data(), OR_UPDATE_AUTO);
            const std::vector<float> h = gemv(out, od.out_proj);
            for (uint32_t j = 0; j < H; ++j) x[j] += h[j];
            mlp(x, od.post_attn_norm, od.gate_proj, od.up_proj, od.down_proj);
        }
        {   // forward_attn_decode
            const std::vector<float> xn = rms(x, oa.input_norm);
            const std::vector<float> qg = gemv(xn, oa.q_proj), kn = gemv(xn, oa.k_proj), vn = gemv(xn, oa.v_proj);
            Kc.resize((std::size_t)(step + 1) * cfg.attn_kv_dim());
            Vc.resize((std::size_t)(step + 1) * cfg.attn_kv_dim());
            std::vector<float> out(cfg.attn_q_dim());
            or_attn_decode_step(&oc, qg.data(), kn.data(), vn.data(), oa.q_norm.data(), oa.k_norm.data(),
                                m.rope_cos.data(), m.rope_sin.data(), rope_len, Kc.data(), Vc.data(), step, 1,
                                out.data(), 4);
            const std::vector<float> h = gemv(out, oa.o_proj);
            for (uint32_t j = 0; j < H; ++j) x[j] += h[j];
            mlp(x, oa.post_attn_norm, oa.gate_proj, oa.up_proj, oa.down_proj);
        }
        const std::vector<float> xf = rms(x, m.final_norm);
        std::vector<float> ref(V);
        or_q4_lm_head(xf.data(), m.embed.packed.data(), m.embed.scales.data(), (int32_t)V, (int32_t)H, ref.data(), 4);
        worst = std::fmax(worst, rel_err(got.data(), ref.data(), V));

        // greedy next token on the device, fed back through tok
        qm_sample_params sp{0.0f, 1.0f, 1, 1.0f, 0.0f, -1, 0};
        ctx.check(qm_sample(ctx.get(), nullptr, (int32_t)V, logits.as<float>(), nullptr, 0, &sp, nullptr,
                            tok.as<int32_t>(), nullptr, nullptr));
        int32_t next = 0;
        tok.download(&next, 4);
        std::size_t best = 0, second = 1;
        if (ref[second] > ref[best]) std::swap(best, second);
        for (std::size_t i = 2; i < V; ++i) {
            if (ref[i] > ref[best]) { second = best; best = i; }
            else if (ref[i] > ref[second]) second = i;
        }
        if (ref[best] - ref[second] > 1e-3 * std::fabs(ref[best]) && (std::size_t)next != best) greedy_ok = false;
        id = next;
    }
    expect(worst <= 2e-3, "qor4b file -> device model, 4 decode steps: logits rel", worst, 2e-3);

    // forward_decode_no_logits (gemv.rs:1033-1053): a forced token advances
    // every state and cache exactly as a full decode step does, so the next
    // step's logits are bit-identical either way
    {
        GpuHybridCache ca = GpuHybridCache::create(ctx, gm, 64), cb = GpuHybridCache::create(ctx, gm, 64);
        DeviceBuffer la(ctx, V * 4), lb(ctx, V * 4);
        const int32_t forced = 77, after = 4321;
        tok.upload(&forced, 4);
        forward_decode_gpu(ctx, gm, ca, scratch, tok.as<int32_t>(), la.as<float>());
        forward_decode_no_logits_gpu(ctx, gm, cb, scratch, tok.as<int32_t>());
        tok.upload(&after, 4);
        forward_decode_gpu(ctx, gm, ca, scratch, tok.as<int32_t>(), la.as<float>());
        forward_decode_gpu(ctx, gm, cb, scratch, tok.as<int32_t>(), lb.as<float>());
        std::vector<float> ga(V), gb(V);
        la.download(ga.data(), V * 4);
        lb.download(gb.data(), V * 4);
        const std::size_t ns = cfg.num_v_heads * cfg.deltanet_head_dim * cfg.deltanet_head_dim;
        std::vector<float> sa(ns), sb(ns);
        ca.dn[0].s.download(sa.data(), ns * 4);
        cb.dn[0].s.download(sb.data(), ns * 4);
        const bool same = std::memcmp(ga.data(), gb.data(), V * 4) == 0 &&
                          std::memcmp(sa.data(), sb.data(), ns * 4) == 0;
        expect(same, "forward_decode_no_logits then a decode step == two decode steps (bit-identical; 1 = differs)",
               same ? 0 : 1, 0.5);
    }

    // prefill (gemv.rs:1243-1283) of a 37-token prompt on a fresh cache, on
    // MFMA with f16 / bf16 activations, against the oracle's f32 prefill
    // composed from its restatements; then one decode step continuing from
    // the prefilled state, conv buffer and KV cache
    {
        const int32_t T = 37;
        std::vector<int32_t> ids(T);
        for (auto& v : ids) v = static_cast<int32_t>(r.next() % V);
        DeviceBuffer dids = upload(ctx, ids);
        GpuHybridCache pc = GpuHybridCache::create(ctx, gm, 64);
        PrefillScratch ps = PrefillScratch::create(ctx, gm, T);
        forward_prefill_gpu(ctx, gm, pc, ps, dids.as<int32_t>(), T, logits.as<float>());
        std::vector<float> got(V);
        logits.download(got.data(), V * 4);

        auto gemm_rows = [&](const std::vector<float>& X, const W& w) {
            std::vector<float> Y((std::size_t)T * w.n);
            or_q4_gemm(X.data(), T, w.packed.data(), w.scales.data(), (int32_t)w.k, (int32_t)w.n, Y.data(), 8);
            return Y;
        };
        auto rms_rows = [&](const std::vector<float>& X, const std::vector<uint16_t>& g) {
            std::vector<float> Y(X.size());
            for (int32_t t = 0; t < T; ++t) or_rms_norm(&X[(std::size_t)t * H], (int32_t)H, g.data(), &Y[(std::size_t)t * H]);
            return Y;
        };
        auto add = [](std::vector<float>& X, const std::vector<float>& D) {
            for (std::size_t i = 0; i < X.size(); ++i) X[i] += D[i];
        };
        auto mlp_rows = [&](std::vector<float>& X, const std::vector<uint16_t>& norm, const W& g, const W& u,
                            const W& dw) {
            const std::vector<float> XN = rms_rows(X, norm);
            std::vector<float> G = gemm_rows(XN, g);
            const std::vector<float> U = gemm_rows(XN, u);
            for (std::size_t i = 0; i < G.size(); ++i) G[i] = (G[i] / (1.0f + std::exp(-G[i]))) * U[i];   // gemv.rs:1235
            add(X, gemm_rows(G, dw));
        };
        std::vector<float> X((std::size_t)T * H);
        for (int32_t t = 0; t < T; ++t)
            or_q4_embed(m.embed.packed.data(), m.embed.scales.data(), (int32_t)H, ids[t], &X[(std::size_t)t * H]);
        std::vector<float> S2(S.size(), 0.0f), buf2(buf.size(), 0.0f);
        {   // prefill_deltanet_layer
            const std::vector<float> XN = rms_rows(X, od.input_norm);
            const std::vector<float> qkv = gemm_rows(XN, od.in_proj_qkv), z = gemm_rows(XN, od.in_proj_z),
                                     av = gemm_rows(XN, od.in_proj_a), bv = gemm_rows(XN, od.in_proj_b);
            std::vector<float> out((std::size_t)T * cfg.deltanet_v_dim());
            or_deltanet_prefill(&oc, T, qkv.data(), av.data(), bv.data(), z.data(), buf2.data(),
                                od.conv1d_weight.data(), od.a_log.data(), od.dt_bias.data(), od.attn_norm_weight.data(),
                                S2.data(), out.data());
            add(X, gemm_rows(out, od.out_proj));
            mlp_rows(X, od.post_attn_norm, od.gate_proj, od.up_proj, od.down_proj);
        }
        std::vector<float> Kp((std::size_t)(T + 1) * cfg.attn_kv_dim()), Vp(Kp.size());
        {   // prefill_attn_layer
            const std::vector<float> XN = rms_rows(X, oa.input_norm);
            const std::vector<float> qg = gemm_rows(XN, oa.q_proj), kk = gemm_rows(XN, oa.k_proj),
                                     vv = gemm_rows(XN, oa.v_proj);
            std::vector<float> out((std::size_t)T * cfg.attn_q_dim());
            or_attn_prefill(&oc, T, qg.data(), kk.data(), vv.data(), oa.q_norm.data(), oa.k_norm.data(),
                            m.rope_cos.data(), m.rope_sin.data(), rope_len, Kp.data(), Vp.data(), out.data(),
                            nullptr, 0, 4);
            add(X, gemm_rows(out, oa.o_proj));
            mlp_rows(X, oa.post_attn_norm, oa.gate_proj, oa.up_proj, oa.down_proj);
        }
        std::vector<float> xl(X.end() - H, X.end()), xf(H), ref(V);
        or_rms_norm(xl.data(), (int32_t)H, m.final_norm.data(), xf.data());
        or_q4_lm_head(xf.data(), m.embed.packed.data(), m.embed.scales.data(), (int32_t)V, (int32_t)H, ref.data(), 4);
        double e = rel_err(got.data(), ref.data(), V);
        expect(e <= 2e-2, "device prefill T=37 (MFMA, f16/bf16 activations): logits rel", e, 2e-2);
        std::vector<float> Sg(S2.size());
        pc.dn[0].s.download(Sg.data(), Sg.size() * 4);
        e = rel_err(Sg.data(), S2.data(), S2.size());
        expect(e <= 2e-2, "device prefill: DeltaNet state rel", e, 2e-2);
        expect(pc.kv[0].seq_len == (std::size_t)T && pc.dn[0].conv_pos == (std::size_t)T,
               "prefill cache positions (error = 1)", 0, 0.5);

        // one decode step continuing from the prefill
        const int32_t nid = 77;
        tok.upload(&nid, 4);
        forward_decode_gpu(ctx, gm, pc, scratch, tok.as<int32_t>(), logits.as<float>());
        logits.download(got.data(), V * 4);
        std::vector<float> x(H);
        or_q4_embed(m.embed.packed.data(), m.embed.scales.data(), (int32_t)H, nid, x.data());
        {
            const std::vector<float> xn = rms(x, od.input_norm);
            const std::vector<float> qkv = gemv(xn, od.in_proj_qkv), av = gemv(xn, od.in_proj_a),
                                     bv = gemv(xn, od.in_proj_b), zv = gemv(xn, od.in_proj_z);
            std::vector<float> out(cfg.deltanet_v_dim());
            or_deltanet_decode_step(&oc, qkv.data(), 1, buf2.data(), od.conv1d_weight.data(), av.data(), bv.data(),
                                    od.a_log.data(), od.dt_bias.data(), zv.data(), od.attn_norm_weight.data(),
                                    S2.data(), out.data(), OR_UPDATE_AUTO);
            const std::vector<float> h = gemv(out, od.out_proj);
            for (uint32_t j = 0; j < H; ++j) x[j] += h[j];
            mlp(x, od.post_attn_norm, od.gate_proj, od.up_proj, od.down_proj);
        }
        {
            const std::vector<float> xn = rms(x, oa.input_norm);
            const std::vector<float> qg = gemv(xn, oa.q_proj), kn = gemv(xn, oa.k_proj), vn = gemv(xn, oa.v_proj);
            std::vector<float> out(cfg.attn_q_dim());
            or_attn_decode_step(&oc, qg.data(), kn.data(), vn.data(), oa.q_norm.data(), oa.k_norm.data(),
                                m.rope_cos.data(), m.rope_sin.data(), rope_len, Kp.data(), Vp.data(), T, 1,
                                out.data(), 4);
            const std::vector<float> h = gemv(out, oa.o_proj);
            for (uint32_t j = 0; j < H; ++j) x[j] += h[j];
            mlp(x, oa.post_attn_norm, oa.gate_proj, oa.up_proj, oa.down_proj);
        }
        or_rms_norm(x.data(), (int32_t)H, m.final_norm.data(), xf.data());
        or_q4_lm_head(xf.data(), m.embed.packed.data(), m.embed.scales.data(), (int32_t)V, (int32_t)H, ref.data(), 4);
        e = rel_err(got.data(), ref.data(), V);
        expect(e <= 2e-2, "decode step after the device prefill: logits rel", e, 2e-2);
    }
    expect(greedy_ok, "greedy qm_sample = oracle argmax (mismatch = 1)", greedy_ok ? 0 : 1, 0.5);
    expect(cache.kv[0].seq_len == (std::size_t)steps && cache.dn[0].conv_pos == (std::size_t)steps,
           "cache positions advanced (error = 1)", 0, 0.5);
}

}  // namespace

int main() {
    try {
        const Qor4bConfig cfg = Qor4bConfig::default_4b();
        Context ctx(cfg);
        deltanet_flow(ctx, cfg);
        attention_flow(ctx, cfg);
        q4_layer_flow(ctx);
        model_flow(ctx, cfg);
    } catch (const std::exception& e) {
        std::printf("exception: %s\n", e.what());
        return 2;
    }
    std::printf("%s\n", failures ? "FAILED" : "all checks passed");
    return failures ? 1 : 0;
}
