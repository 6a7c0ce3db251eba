// qor4b_file.hpp -- the .qor4b model file (save.rs:135-396) read in place:
// a parser over a read-only memory map that returns views of every field,
// with no copies and no device dependency.  qor4b_model.hpp uploads the
// views to the device.
//
// Layout (all little-endian; save_model, save.rs:135-240):
//   "QOR4", version u32 (1 or 2), format u8 (0 = F16, 1 = Q4)
//   config: vocab, hidden, layers, attn heads, kv heads, attn head dim,
//           qk heads, v heads, deltanet head dim, conv kernel,
//           intermediate (u32 each), rope_theta f64, partial_rotary f32,
//           rms_norm_eps f64, eos u32, tie_word_embeddings u8, has_vision u8
//   layer types: u8 per layer (0 = DeltaNet, else full attention)
//   per layer, in order (save.rs:171-200):
//     DeltaNet:  in_proj_qkv, in_proj_a, in_proj_b, in_proj_z, out_proj (W),
//                conv1d_weight, a_log, dt_bias (f32 vec), attn_norm (f16 vec),
//                gate, up, down (W), input_norm, post_attn_norm (f16 vec)
//     full attn: q, k, v, o (W), q_norm, k_norm (f16 vec), gate, up, down (W),
//                input_norm, post_attn_norm (f16 vec)
//   embed (W, vocab-major), final_norm (f16 vec), rope_cos, rope_sin (f32 vec)
//   vision encoder when has_vision (not read here: nothing follows it)
// W (write_weight, save.rs:103-113): k u64, n u64, fmt u8, then for fmt 0 an
// f16 vec of k*n, for fmt 1 a byte vec (packed [k][n/2]) and an f16 vec
// (scales [k][n/32]).  A vec is a u64 element count and the elements.
// Errors (bad magic, version, weight format, a truncated file) throw
// FormatError, where load_model returns io::Error (save.rs:247-260,127).
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace qor4b {

class FormatError : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};

// Elements in the file are not aligned: views hold bytes and counts, and
// readers copy (memcpy or a device upload).
struct ArrayView {
    const uint8_t* data = nullptr;
    uint64_t len = 0;          // elements
    uint32_t elem = 0;         // bytes per element
    uint64_t bytes() const { return len * elem; }
};

struct WeightView {
    uint64_t k = 0, n = 0;     // in and out dimension (gemv.rs:17-34)
    uint8_t fmt = 0;           // 0 = F16, 1 = Q4
    ArrayView f16;             // fmt 0: f16 [k][n]
    ArrayView packed;          // fmt 1: u8 [k][n/2]
    ArrayView scales;          // fmt 1: f16 [k][n/32]
};

struct FileConfig {
    uint32_t vocab_size = 0, hidden_size = 0, num_layers = 0, num_attn_heads = 0, num_kv_heads = 0,
             attn_head_dim = 0, num_qk_heads = 0, num_v_heads = 0, deltanet_head_dim = 0, conv_kernel_size = 0,
             intermediate_size = 0;
    double rope_theta = 0;
    float partial_rotary_factor = 0;
    double rms_norm_eps = 0;
    uint32_t eos_token_id = 0;
    bool tie_word_embeddings = false, has_vision = false;
    std::vector<uint8_t> layer_types;   // 0 = DeltaNet, else full attention
};

struct DeltaNetLayerView {
    WeightView in_proj_qkv, in_proj_a, in_proj_b, in_proj_z, out_proj;
    ArrayView conv1d_weight, a_log, dt_bias, attn_norm_weight;
    WeightView gate_proj, up_proj, down_proj;
    ArrayView input_norm, post_attn_norm;
};

struct FullAttnLayerView {
    WeightView q_proj, k_proj, v_proj, o_proj;
    ArrayView q_norm, k_norm;
    WeightView gate_proj, up_proj, down_proj;
    ArrayView input_norm, post_attn_norm;
};

struct LayerView {
    bool deltanet = true;
    DeltaNetLayerView dn;      // when deltanet
    FullAttnLayerView fa;      // otherwise
};

struct ModelView {
    uint32_t version = 0;
    uint8_t format_id = 0;
    FileConfig config;
    std::vector<LayerView> layers;
    WeightView embed;
    ArrayView final_norm, rope_cos, rope_sin;
    uint64_t vision_offset = 0;   // where the vision section starts (has_vision)
};

namespace detail {

class Reader {
public:
    Reader(const uint8_t* p, std::size_t n) : base_(p), size_(n) {}
    uint64_t offset() const { return off_; }

    const uint8_t* take(uint64_t bytes, const char* what) {
        if (bytes > size_ - off_)
            throw FormatError("unexpected end of file reading " + std::string(what) + " at byte " +
                              std::to_string(off_) + " (" + std::to_string(bytes) + " bytes needed, " +
                              std::to_string(size_ - off_) + " left)");
        const uint8_t* p = base_ + off_;
        off_ += bytes;
        return p;
    }
    template <class T>
    T scalar(const char* what) {
        T v;
        std::memcpy(&v, take(sizeof(T), what), sizeof(T));
        return v;
    }
    // read_f16_vec / read_f32_vec / read_bytes_vec (save.rs:64-96)
    ArrayView vec(uint32_t elem, const char* what) {
        const uint64_t len = scalar<uint64_t>(what);
        if (len > (size_ - off_) / elem)
            throw FormatError("unexpected end of file reading " + std::string(what) + " at byte " +
                              std::to_string(off_) + " (" + std::to_string(len) + " elements of " +
                              std::to_string(elem) + " bytes)");
        ArrayView a;
        a.len = len;
        a.elem = elem;
        a.data = take(len * elem, what);
        return a;
    }
    // read_weight, save.rs:115-129
    WeightView weight(const char* what) {
        WeightView w;
        w.k = scalar<uint64_t>(what);
        w.n = scalar<uint64_t>(what);
        w.fmt = scalar<uint8_t>(what);
        if (w.fmt == 0) {
            w.f16 = vec(2, what);
        } else if (w.fmt == 1) {
            w.packed = vec(1, what);
            w.scales = vec(2, what);
        } else {
            throw FormatError("Unknown weight format " + std::to_string(w.fmt) + " in " + what);
        }
        return w;
    }

private:
    const uint8_t* base_;
    std::size_t size_;
    uint64_t off_ = 0;
};

}  // namespace detail

// load_model's parse (save.rs:247-396) over bytes in memory.
inline ModelView parse_qor4b(const uint8_t* data, std::size_t size) {
    detail::Reader r(data, size);
    ModelView m;
    if (std::memcmp(r.take(4, "magic"), "QOR4", 4) != 0) throw FormatError("Invalid magic (expected QOR4)");
    m.version = r.scalar<uint32_t>("version");
    if (m.version != 1 && m.version != 2)
        throw FormatError("Unsupported version " + std::to_string(m.version) + " (expected 1 or 2)");
    m.format_id = r.scalar<uint8_t>("format");
    FileConfig& c = m.config;
    c.vocab_size = r.scalar<uint32_t>("config");
    c.hidden_size = r.scalar<uint32_t>("config");
    c.num_layers = r.scalar<uint32_t>("config");
    c.num_attn_heads = r.scalar<uint32_t>("config");
    c.num_kv_heads = r.scalar<uint32_t>("config");
    c.attn_head_dim = r.scalar<uint32_t>("config");
    c.num_qk_heads = r.scalar<uint32_t>("config");
    c.num_v_heads = r.scalar<uint32_t>("config");
    c.deltanet_head_dim = r.scalar<uint32_t>("config");
    c.conv_kernel_size = r.scalar<uint32_t>("config");
    c.intermediate_size = r.scalar<uint32_t>("config");
    c.rope_theta = r.scalar<double>("config");
    c.partial_rotary_factor = r.scalar<float>("config");
    c.rms_norm_eps = r.scalar<double>("config");
    c.eos_token_id = r.scalar<uint32_t>("config");
    c.tie_word_embeddings = r.scalar<uint8_t>("config") != 0;
    c.has_vision = r.scalar<uint8_t>("config") != 0;
    c.layer_types.resize(c.num_layers);
    for (auto& t : c.layer_types) t = r.scalar<uint8_t>("layer types");
    m.layers.resize(c.num_layers);
    for (std::size_t i = 0; i < c.num_layers; ++i) {
        LayerView& l = m.layers[i];
        l.deltanet = c.layer_types[i] == 0;
        if (l.deltanet) {
            DeltaNetLayerView& d = l.dn;
            d.in_proj_qkv = r.weight("in_proj_qkv");
            d.in_proj_a = r.weight("in_proj_a");
            d.in_proj_b = r.weight("in_proj_b");
            d.in_proj_z = r.weight("in_proj_z");
            d.out_proj = r.weight("out_proj");
            d.conv1d_weight = r.vec(4, "conv1d_weight");
            d.a_log = r.vec(4, "a_log");
            d.dt_bias = r.vec(4, "dt_bias");
            d.attn_norm_weight = r.vec(2, "attn_norm_weight");
            d.gate_proj = r.weight("gate_proj");
            d.up_proj = r.weight("up_proj");
            d.down_proj = r.weight("down_proj");
            d.input_norm = r.vec(2, "input_norm");
            d.post_attn_norm = r.vec(2, "post_attn_norm");
        } else {
            FullAttnLayerView& a = l.fa;
            a.q_proj = r.weight("q_proj");
            a.k_proj = r.weight("k_proj");
            a.v_proj = r.weight("v_proj");
            a.o_proj = r.weight("o_proj");
            a.q_norm = r.vec(2, "q_norm");
            a.k_norm = r.vec(2, "k_norm");
            a.gate_proj = r.weight("gate_proj");
            a.up_proj = r.weight("up_proj");
            a.down_proj = r.weight("down_proj");
            a.input_norm = r.vec(2, "input_norm");
            a.post_attn_norm = r.vec(2, "post_attn_norm");
        }
    }
    m.embed = r.weight("embed");
    m.final_norm = r.vec(2, "final_norm");
    m.rope_cos = r.vec(4, "rope_cos");
    m.rope_sin = r.vec(4, "rope_sin");
    m.vision_offset = r.offset();
    return m;
}

// A read-only private memory map of a whole file.
class MappedFile {
public:
    explicit MappedFile(const std::string& path) {
        const int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) throw FormatError("cannot open " + path);
        struct stat st;
        if (::fstat(fd, &st) != 0) {
            ::close(fd);
            throw FormatError("cannot stat " + path);
        }
        size_ = static_cast<std::size_t>(st.st_size);
        if (size_ > 0) {
            void* p = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
            if (p == MAP_FAILED) {
                ::close(fd);
                throw FormatError("cannot map " + path);
            }
            data_ = static_cast<const uint8_t*>(p);
        }
        ::close(fd);
    }
    ~MappedFile() {
        if (data_) ::munmap(const_cast<uint8_t*>(data_), size_);
    }
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;

    const uint8_t* data() const { return data_; }
    std::size_t size() const { return size_; }

private:
    const uint8_t* data_ = nullptr;
    std::size_t size_ = 0;
};

}  // namespace qor4b
