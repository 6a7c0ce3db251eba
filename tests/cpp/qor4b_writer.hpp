// qor4b_writer.hpp -- writes .qor4b files field for field as save_model does
// (save.rs:135-240), for the loader tests (test infrastructure).  A model is
// given as host arrays; weights are Q4 (packed [k][n/2] + f16 scales
// [k][n/32]) or F16 ([k][n]).
#pragma once

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

namespace qor4b_test {

struct W {
    uint64_t k = 0, n = 0;
    uint8_t fmt = 1;
    std::vector<uint8_t> packed;
    std::vector<uint16_t> scales, f16;
};

struct DnLayer {
    W in_proj_qkv, in_proj_a, in_proj_b, in_proj_z, out_proj;
    std::vector<float> conv1d_weight, a_log, dt_bias;
    std::vector<uint16_t> attn_norm_weight;
    W gate_proj, up_proj, down_proj;
    std::vector<uint16_t> input_norm, post_attn_norm;
};

struct FaLayer {
    W q_proj, k_proj, v_proj, o_proj;
    std::vector<uint16_t> q_norm, k_norm;
    W gate_proj, up_proj, down_proj;
    std::vector<uint16_t> input_norm, post_attn_norm;
};

struct Model {
    uint32_t version = 2;
    uint8_t format_id = 1;
    uint32_t vocab = 0, hidden = 0, heads = 16, kv_heads = 4, attn_head_dim = 256, qk_heads = 16, v_heads = 32,
             dn_head_dim = 128, conv_kernel = 4, intermediate = 0;
    double rope_theta = 1e7;
    float partial_rotary = 0.25f;
    double eps = 1e-6;
    uint32_t eos = 248044;
    uint8_t tie = 1, has_vision = 0;
    std::vector<uint8_t> layer_types;     // 0 DeltaNet, 1 full attention
    std::vector<DnLayer> dn;              // in order of the DeltaNet layers
    std::vector<FaLayer> fa;
    W embed;
    std::vector<uint16_t> final_norm;
    std::vector<float> rope_cos, rope_sin;
    std::vector<uint8_t> vision_tail;     // bytes written after the globals when has_vision
};

class Out {
public:
    std::vector<uint8_t> bytes;
    template <class T> void put(T v) {
        const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
        bytes.insert(bytes.end(), p, p + sizeof(T));
    }
    template <class T> void vec(const std::vector<T>& v) {
        put<uint64_t>(v.size());
        const uint8_t* p = reinterpret_cast<const uint8_t*>(v.data());
        bytes.insert(bytes.end(), p, p + v.size() * sizeof(T));
    }
    void weight(const W& w) {
        put<uint64_t>(w.k);
        put<uint64_t>(w.n);
        put<uint8_t>(w.fmt);
        if (w.fmt == 0) {
            vec(w.f16);
        } else {
            vec(w.packed);
            vec(w.scales);
        }
    }
};

inline std::vector<uint8_t> serialize(const Model& m) {
    Out o;
    o.bytes.insert(o.bytes.end(), {'Q', 'O', 'R', '4'});
    o.put<uint32_t>(m.version);
    o.put<uint8_t>(m.format_id);
    for (uint32_t v : {m.vocab, m.hidden, static_cast<uint32_t>(m.layer_types.size()), m.heads, m.kv_heads,
                       m.attn_head_dim, m.qk_heads, m.v_heads, m.dn_head_dim, m.conv_kernel, m.intermediate})
        o.put<uint32_t>(v);
    o.put<double>(m.rope_theta);
    o.put<float>(m.partial_rotary);
    o.put<double>(m.eps);
    o.put<uint32_t>(m.eos);
    o.put<uint8_t>(m.tie);
    o.put<uint8_t>(m.has_vision);
    for (uint8_t t : m.layer_types) o.put<uint8_t>(t);
    std::size_t di = 0, ai = 0;
    for (uint8_t t : m.layer_types) {
        if (t == 0) {
            const DnLayer& d = m.dn[di++];
            o.weight(d.in_proj_qkv);
            o.weight(d.in_proj_a);
            o.weight(d.in_proj_b);
            o.weight(d.in_proj_z);
            o.weight(d.out_proj);
            o.vec(d.conv1d_weight);
            o.vec(d.a_log);
            o.vec(d.dt_bias);
            o.vec(d.attn_norm_weight);
            o.weight(d.gate_proj);
            o.weight(d.up_proj);
            o.weight(d.down_proj);
            o.vec(d.input_norm);
            o.vec(d.post_attn_norm);
        } else {
            const FaLayer& a = m.fa[ai++];
            o.weight(a.q_proj);
            o.weight(a.k_proj);
            o.weight(a.v_proj);
            o.weight(a.o_proj);
            o.vec(a.q_norm);
            o.vec(a.k_norm);
            o.weight(a.gate_proj);
            o.weight(a.up_proj);
            o.weight(a.down_proj);
            o.vec(a.input_norm);
            o.vec(a.post_attn_norm);
        }
    }
    o.weight(m.embed);
    o.vec(m.final_norm);
    o.vec(m.rope_cos);
    o.vec(m.rope_sin);
    o.bytes.insert(o.bytes.end(), m.vision_tail.begin(), m.vision_tail.end());
    return o.bytes;
}

inline bool write_file(const std::string& path, const std::vector<uint8_t>& b) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = std::fwrite(b.data(), 1, b.size(), f) == b.size();
    return std::fclose(f) == 0 && ok;
}

}  // namespace qor4b_test
