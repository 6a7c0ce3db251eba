// qor4b_file_test.cpp -- the .qor4b parser (qor4b_file.hpp) on the CPU: small
// synthetic models written field for field as save_model does
// (qor4b_writer.hpp) are parsed from memory and through the file map, every
// view compared with what was written; then the load errors of load_model
// (save.rs:247-260,127): bad magic, unsupported version, unknown weight
// format, and truncation at every byte.  Exit status 0 = all checks pass.
#include "qor4b_file.hpp"
#include "qor4b_writer.hpp"

#include <cstdio>
#include <cstring>
#include <unistd.h>

using namespace qor4b;
using namespace qor4b_test;

namespace {

int failures = 0;
void expect(bool ok, const char* what) {
    if (!ok) {
        std::printf("FAIL %s\n", what);
        ++failures;
    }
}

uint64_t lcg = 88172645463325252ull;
uint32_t rnd() {
    lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
    return static_cast<uint32_t>(lcg >> 33);
}

W q4(uint64_t k, uint64_t n) {
    W w;
    w.k = k;
    w.n = n;
    w.fmt = 1;
    w.packed.resize(k * n / 2);
    w.scales.resize(k * (n / 32));
    for (auto& b : w.packed) b = static_cast<uint8_t>(rnd());
    for (auto& s : w.scales) s = static_cast<uint16_t>(rnd());
    return w;
}
W f16w(uint64_t k, uint64_t n) {
    W w;
    w.k = k;
    w.n = n;
    w.fmt = 0;
    w.f16.resize(k * n);
    for (auto& s : w.f16) s = static_cast<uint16_t>(rnd());
    return w;
}
template <class T> std::vector<T> vals(std::size_t n) {
    std::vector<T> v(n);
    for (auto& x : v) {
        const uint32_t r = rnd();
        std::memcpy(&x, &r, sizeof(T) < 4 ? sizeof(T) : 4);
    }
    return v;
}

// A model of made-up small shapes: the parser does not depend on them.
Model small_model(const std::vector<uint8_t>& types, bool f16_weights, bool vision) {
    Model m;
    m.vocab = 96;
    m.hidden = 64;
    m.intermediate = 128;
    m.layer_types = types;
    m.has_vision = vision;
    auto w = [&](uint64_t k, uint64_t n) { return f16_weights ? f16w(k, n) : q4(k, n); };
    m.format_id = f16_weights ? 0 : 1;
    for (uint8_t t : types) {
        if (t == 0) {
            DnLayer d;
            d.in_proj_qkv = w(64, 256);
            d.in_proj_a = w(64, 32);
            d.in_proj_b = w(64, 32);
            d.in_proj_z = w(64, 128);
            d.out_proj = w(128, 64);
            d.conv1d_weight = vals<float>(256 * 4);
            d.a_log = vals<float>(4);
            d.dt_bias = vals<float>(4);
            d.attn_norm_weight = vals<uint16_t>(32);
            d.gate_proj = w(64, 128);
            d.up_proj = w(64, 128);
            d.down_proj = w(128, 64);
            d.input_norm = vals<uint16_t>(64);
            d.post_attn_norm = vals<uint16_t>(64);
            m.dn.push_back(d);
        } else {
            FaLayer a;
            a.q_proj = w(64, 256);
            a.k_proj = w(64, 64);
            a.v_proj = w(64, 64);
            a.o_proj = w(128, 64);
            a.q_norm = vals<uint16_t>(32);
            a.k_norm = vals<uint16_t>(32);
            a.gate_proj = w(64, 128);
            a.up_proj = w(64, 128);
            a.down_proj = w(128, 64);
            a.input_norm = vals<uint16_t>(64);
            a.post_attn_norm = vals<uint16_t>(64);
            m.fa.push_back(a);
        }
    }
    m.embed = q4(96, 64);
    m.final_norm = vals<uint16_t>(64);
    m.rope_cos = vals<float>(10 * 8);
    m.rope_sin = vals<float>(10 * 8);
    if (vision) m.vision_tail = std::vector<uint8_t>(333, 0xAB);
    return m;
}

template <class T> bool same(const ArrayView& a, const std::vector<T>& v) {
    return a.len == v.size() && a.elem == sizeof(T) && std::memcmp(a.data, v.data(), v.size() * sizeof(T)) == 0;
}
bool same(const WeightView& a, const W& w) {
    if (a.k != w.k || a.n != w.n || a.fmt != w.fmt) return false;
    return w.fmt == 0 ? same(a.f16, w.f16) : same(a.packed, w.packed) && same(a.scales, w.scales);
}

void check_model(const ModelView& v, const Model& m, const char* tag) {
    char what[160];
    std::snprintf(what, sizeof what, "%s: header and config", tag);
    const FileConfig& c = v.config;
    expect(v.version == m.version && v.format_id == m.format_id && c.vocab_size == m.vocab &&
               c.hidden_size == m.hidden && c.num_layers == m.layer_types.size() && c.num_attn_heads == m.heads &&
               c.num_kv_heads == m.kv_heads && c.attn_head_dim == m.attn_head_dim && c.num_qk_heads == m.qk_heads &&
               c.num_v_heads == m.v_heads && c.deltanet_head_dim == m.dn_head_dim && c.conv_kernel_size == m.conv_kernel &&
               c.intermediate_size == m.intermediate && c.rope_theta == m.rope_theta &&
               c.partial_rotary_factor == m.partial_rotary && c.rms_norm_eps == m.eps && c.eos_token_id == m.eos &&
               c.tie_word_embeddings == (m.tie != 0) && c.has_vision == (m.has_vision != 0) &&
               c.layer_types == m.layer_types,
           what);
    std::size_t di = 0, ai = 0;
    for (std::size_t i = 0; i < m.layer_types.size(); ++i) {
        const LayerView& l = v.layers[i];
        std::snprintf(what, sizeof what, "%s: layer %zu", tag, i);
        if (m.layer_types[i] == 0) {
            const DnLayer& d = m.dn[di++];
            const DeltaNetLayerView& x = l.dn;
            expect(l.deltanet && same(x.in_proj_qkv, d.in_proj_qkv) && same(x.in_proj_a, d.in_proj_a) &&
                       same(x.in_proj_b, d.in_proj_b) && same(x.in_proj_z, d.in_proj_z) && same(x.out_proj, d.out_proj) &&
                       same(x.conv1d_weight, d.conv1d_weight) && same(x.a_log, d.a_log) && same(x.dt_bias, d.dt_bias) &&
                       same(x.attn_norm_weight, d.attn_norm_weight) && same(x.gate_proj, d.gate_proj) &&
                       same(x.up_proj, d.up_proj) && same(x.down_proj, d.down_proj) &&
                       same(x.input_norm, d.input_norm) && same(x.post_attn_norm, d.post_attn_norm),
                   what);
        } else {
            const FaLayer& a = m.fa[ai++];
            const FullAttnLayerView& x = l.fa;
            expect(!l.deltanet && same(x.q_proj, a.q_proj) && same(x.k_proj, a.k_proj) && same(x.v_proj, a.v_proj) &&
                       same(x.o_proj, a.o_proj) && same(x.q_norm, a.q_norm) && same(x.k_norm, a.k_norm) &&
                       same(x.gate_proj, a.gate_proj) && same(x.up_proj, a.up_proj) &&
                       same(x.down_proj, a.down_proj) && same(x.input_norm, a.input_norm) &&
                       same(x.post_attn_norm, a.post_attn_norm),
                   what);
        }
    }
    std::snprintf(what, sizeof what, "%s: globals", tag);
    expect(same(v.embed, m.embed) && same(v.final_norm, m.final_norm) && same(v.rope_cos, m.rope_cos) &&
               same(v.rope_sin, m.rope_sin),
           what);
}

template <class F> bool throws(F f, const char* needle) {
    try {
        f();
    } catch (const FormatError& e) {
        return std::strstr(e.what(), needle) != nullptr;
    }
    return false;
}

}  // namespace

int main() {
    // a hybrid stack (the 4B's 3:1 pattern), an all-DeltaNet one, F16 weights,
    // a trailing vision section and a version-1 header
    struct Case { std::vector<uint8_t> types; bool f16, vision; uint32_t version; const char* tag; };
    const Case cases[] = {{{0, 0, 0, 1, 0, 0, 0, 1}, false, false, 2, "hybrid q4"},
                          {{0, 0}, false, false, 2, "deltanet only"},
                          {{1, 0}, true, false, 2, "f16 weights"},
                          {{0, 1}, false, true, 2, "vision tail"},
                          {{0, 1}, false, false, 1, "version 1"}};
    for (const Case& cs : cases) {
        Model m = small_model(cs.types, cs.f16, cs.vision);
        m.version = cs.version;
        const std::vector<uint8_t> b = serialize(m);
        const ModelView v = parse_qor4b(b.data(), b.size());
        check_model(v, m, cs.tag);
        expect(v.vision_offset == b.size() - m.vision_tail.size(), "vision section offset");
    }

    // through a file map
    {
        const Model m = small_model({0, 0, 0, 1}, false, false);
        const std::vector<uint8_t> b = serialize(m);
        char path[] = "/tmp/qor4b_file_test_XXXXXX";
        const int fd = mkstemp(path);
        expect(fd >= 0, "temporary file");
        if (fd >= 0) {
            close(fd);
            expect(write_file(path, b), "write file");
            {
                MappedFile f(path);
                expect(f.size() == b.size(), "mapped size");
                check_model(parse_qor4b(f.data(), f.size()), m, "mapped file");
            }
            unlink(path);
        }
        expect(throws([] { MappedFile f("/nonexistent/model.qor4b"); }, "cannot open"), "missing file");
    }

    // errors
    const Model m = small_model({0, 1}, false, false);
    const std::vector<uint8_t> good = serialize(m);
    {
        std::vector<uint8_t> b = good;
        b[0] = 'X';
        expect(throws([&] { parse_qor4b(b.data(), b.size()); }, "Invalid magic"), "bad magic");
    }
    {
        std::vector<uint8_t> b = good;
        b[4] = 3;
        expect(throws([&] { parse_qor4b(b.data(), b.size()); }, "Unsupported version 3"), "bad version");
    }
    {
        // the first weight's format byte: after magic, version, format, 11 u32,
        // f64, f32, f64, u32, 2 u8, 2 layer types, k u64, n u64
        const std::size_t at = 4 + 4 + 1 + 44 + 8 + 4 + 8 + 4 + 2 + 2 + 16;
        std::vector<uint8_t> b = good;
        expect(b[at] == 1, "format byte located");
        b[at] = 7;
        expect(throws([&] { parse_qor4b(b.data(), b.size()); }, "Unknown weight format 7"), "bad weight format");
    }
    {
        // a huge element count must not wrap the bounds check
        std::vector<uint8_t> b = good;
        const std::size_t at = 4 + 4 + 1 + 44 + 8 + 4 + 8 + 4 + 2 + 2 + 17;
        const uint64_t huge = ~0ull / 2;
        std::memcpy(&b[at], &huge, 8);
        expect(throws([&] { parse_qor4b(b.data(), b.size()); }, "unexpected end of file"), "huge count");
    }
    int truncated_ok = 0;
    for (std::size_t n = 0; n < good.size(); n += (n < 200 ? 1 : 97)) {
        truncated_ok += throws([&] { parse_qor4b(good.data(), n); }, "") ? 1 : 0;
        if (!throws([&] { parse_qor4b(good.data(), n); }, "")) {
            std::printf("FAIL truncation at %zu parsed\n", n);
            ++failures;
            break;
        }
    }
    std::printf("truncations rejected: %d\n", truncated_ok);
    std::printf("%s\n", failures ? "FAILED" : "all checks passed");
    return failures ? 1 : 0;
}
