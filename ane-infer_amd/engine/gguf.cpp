// gguf.cpp — GGUF reader of the C++ engine API (see gguf.hpp for the
// reference functions each piece mirrors).
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>

namespace ane {
namespace gguf {

namespace {

constexpr uint32_t kMagic = 0x46554747;  // "GGUF" read as a little-endian u32

[[noreturn]] void bad(const std::string &msg) { throw Error(ANEHIP_EINVAL, "gguf: " + msg); }

// Bounds-checked little-endian cursor over the file's bytes.
class Reader {
  public:
    Reader(const uint8_t *p, size_t n) : p_(p), n_(n) {}
    size_t pos() const { return pos_; }
    template <typename T> T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p_ + pos_, sizeof(T));
        pos_ += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        need(len);
        std::string s(reinterpret_cast<const char *>(p_ + pos_), (size_t)len);
        pos_ += (size_t)len;
        return s;
    }

  private:
    void need(uint64_t k) const {
        if (k > n_ - pos_) bad("truncated at byte " + std::to_string(pos_));
    }
    const uint8_t *p_;
    size_t n_, pos_ = 0;
};

GgufType value_type(uint32_t v) {
    if (v > 12) bad("unknown GGUF type: " + std::to_string(v));
    return (GgufType)v;
}

GgmlType tensor_type(uint32_t v) {
    switch (v) {
        case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 12: case 13: case 14: return (GgmlType)v;
        default: throw Error(ANEHIP_EUNSUPPORTED, "gguf: unsupported GGML type: " + std::to_string(v));
    }
}

MetadataValue read_value(Reader &r, GgufType t, int depth) {
    MetadataValue m;
    m.type = t;
    switch (t) {
        case GgufType::U8: m.v = (uint64_t)r.get<uint8_t>(); break;
        case GgufType::I8: m.v = (int64_t)r.get<int8_t>(); break;
        case GgufType::U16: m.v = (uint64_t)r.get<uint16_t>(); break;
        case GgufType::I16: m.v = (int64_t)r.get<int16_t>(); break;
        case GgufType::U32: m.v = (uint64_t)r.get<uint32_t>(); break;
        case GgufType::I32: m.v = (int64_t)r.get<int32_t>(); break;
        case GgufType::F32: m.v = (double)r.get<float>(); break;
        case GgufType::U64: m.v = r.get<uint64_t>(); break;
        case GgufType::I64: m.v = r.get<int64_t>(); break;
        case GgufType::F64: m.v = r.get<double>(); break;
        case GgufType::Bool: m.v = r.get<uint8_t>() != 0; break;
        case GgufType::String: m.v = r.str(); break;
        case GgufType::Array: {
            if (depth > 8) bad("arrays nested too deep");
            const GgufType et = value_type(r.get<uint32_t>());
            const uint64_t count = r.get<uint64_t>();
            auto arr = std::make_shared<MetadataArray>();
            // every element takes at least one byte, so count is bounded by the file
            arr->reserve((size_t)std::min<uint64_t>(count, 1u << 16));
            for (uint64_t i = 0; i < count; i++) arr->push_back(read_value(r, et, depth + 1));
            m.v = std::move(arr);
            break;
        }
    }
    return m;
}

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1f, f = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (f == 0) {
            bits = sign;
        } else {  // subnormal: f * 2^-24, exact in fp32
            const float v = std::ldexp((float)f, -24);
            std::memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (f << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (f << 13);
    }
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

}  // namespace

size_t block_size(GgmlType t) {
    switch (t) {
        case GgmlType::F32: case GgmlType::F16: return 1;
        case GgmlType::Q4_0: case GgmlType::Q4_1: case GgmlType::Q5_0: case GgmlType::Q5_1: case GgmlType::Q8_0:
            return 32;
        case GgmlType::Q4K: case GgmlType::Q5K: case GgmlType::Q6K: return 256;
    }
    return 1;
}

size_t bytes_per_block(GgmlType t) {
    switch (t) {
        case GgmlType::F32: return 4;
        case GgmlType::F16: return 2;
        case GgmlType::Q4_0: return 18;
        case GgmlType::Q4_1: return 20;
        case GgmlType::Q5_0: return 22;
        case GgmlType::Q5_1: return 24;
        case GgmlType::Q8_0: return 34;
        case GgmlType::Q4K: return 144;
        case GgmlType::Q5K: return 176;
        case GgmlType::Q6K: return 210;
    }
    return 0;
}

bool MetadataValue::as_u32(uint32_t &out) const {
    if (type != GgufType::U32) return false;
    out = (uint32_t)std::get<uint64_t>(v);
    return true;
}
bool MetadataValue::as_u64(uint64_t &out) const {
    if (type != GgufType::U64) return false;
    out = std::get<uint64_t>(v);
    return true;
}
bool MetadataValue::as_f32(float &out) const {
    if (type != GgufType::F32) return false;
    out = (float)std::get<double>(v);
    return true;
}
const std::string *MetadataValue::as_str() const {
    return type == GgufType::String ? &std::get<std::string>(v) : nullptr;
}
const MetadataArray *MetadataValue::as_array() const {
    return type == GgufType::Array ? std::get<std::shared_ptr<MetadataArray>>(v).get() : nullptr;
}

uint64_t TensorInfo::n_elements() const {
    uint64_t n = 1;
    for (uint64_t d : dimensions) n *= d;
    return n;
}

uint64_t TensorInfo::data_size() const {
    const uint64_t bs = block_size(typ), bpb = bytes_per_block(typ);
    return (n_elements() + bs - 1) / bs * bpb;
}

GgufFile GgufFile::parse(const uint8_t *data, size_t size) {
    Reader r(data, size);
    const uint32_t magic = r.get<uint32_t>();
    if (magic != kMagic) {
        char buf[96];
        std::snprintf(buf, sizeof buf, "not a GGUF file (magic: 0x%08x, expected 0x%08x)", magic, kMagic);
        bad(buf);
    }
    GgufFile g;
    g.version = r.get<uint32_t>();
    if (g.version < 2 || g.version > 3) bad("unsupported GGUF version: " + std::to_string(g.version));
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key = r.str();
        const GgufType t = value_type(r.get<uint32_t>());
        g.metadata[key] = read_value(r, t, 0);
    }
    g.tensors.reserve((size_t)std::min<uint64_t>(n_tensors, 1u << 16));
    for (uint64_t i = 0; i < n_tensors; i++) {
        TensorInfo ti;
        ti.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        if (nd > 4) bad("tensor " + ti.name + " has " + std::to_string(nd) + " dimensions");
        for (uint32_t k = 0; k < nd; k++) ti.dimensions.push_back(r.get<uint64_t>());
        ti.typ = tensor_type(r.get<uint32_t>());
        ti.offset = r.get<uint64_t>();
        g.tensors.push_back(std::move(ti));
    }
    // tensor data starts at the next multiple of general.alignment (default 32)
    uint32_t align = 32;
    auto it = g.metadata.find("general.alignment");
    if (it != g.metadata.end()) it->second.as_u32(align);
    if (align == 0) bad("general.alignment is 0");
    const uint64_t pos = r.pos();
    g.tensor_data_offset = (pos + align - 1) / align * align;
    return g;
}

const TensorInfo *GgufFile::get_tensor(const std::string &name) const {
    for (const TensorInfo &t : tensors)
        if (t.name == name) return &t;
    return nullptr;
}

const std::string *GgufFile::architecture() const {
    auto it = metadata.find("general.architecture");
    return it == metadata.end() ? nullptr : it->second.as_str();
}

bool GgufFile::arch_u32(const char *key, uint32_t &out) const {
    const std::string *arch = architecture();
    if (!arch) return false;
    auto it = metadata.find(*arch + "." + key);
    return it != metadata.end() && it->second.as_u32(out);
}

bool GgufFile::arch_f32(const char *key, float &out) const {
    const std::string *arch = architecture();
    if (!arch) return false;
    auto it = metadata.find(*arch + "." + key);
    return it != metadata.end() && it->second.as_f32(out);
}

bool GgufFile::vocab_size(uint32_t &out) const {
    auto it = metadata.find("tokenizer.ggml.tokens");
    if (it == metadata.end() || !it->second.as_array()) return false;
    out = (uint32_t)it->second.as_array()->size();
    return true;
}

bool GgufFile::is_deltanet_layer(size_t layer) const {
    return get_tensor("blk." + std::to_string(layer) + ".ssm_a") != nullptr;
}

MappedFile::MappedFile(const std::string &path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw Error(ANEHIP_EINVAL, "gguf: cannot open " + path + ": " + std::strerror(errno));
    struct stat st;
    if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
        ::close(fd);
        throw Error(ANEHIP_EINVAL, "gguf: cannot read the size of " + path);
    }
    void *p = ::mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) throw Error(ANEHIP_EINVAL, "gguf: cannot map " + path + ": " + std::strerror(errno));
    data_ = static_cast<const uint8_t *>(p);
    size_ = (size_t)st.st_size;
}

MappedFile::~MappedFile() {
    if (data_) ::munmap(const_cast<uint8_t *>(data_), size_);
}

std::vector<float> dequantize_tensor(const uint8_t *data, size_t size, GgmlType typ, size_t n) {
    const size_t bs = block_size(typ), bpb = bytes_per_block(typ);
    if ((n + bs - 1) / bs * bpb > size) bad("tensor data shorter than its elements");
    std::vector<float> out(n);
    switch (typ) {
        case GgmlType::F32:
            std::memcpy(out.data(), data, n * 4);
            break;
        case GgmlType::F16:
            for (size_t i = 0; i < n; i++) {
                uint16_t h;
                std::memcpy(&h, data + 2 * i, 2);
                out[i] = half_to_float(h);
            }
            break;
        case GgmlType::Q4_0:
        case GgmlType::Q8_0:
            for (size_t b = 0; b * 32 < n; b++) {
                const uint8_t *blk = data + b * bpb;
                uint16_t hs;
                std::memcpy(&hs, blk, 2);
                const float scale = half_to_float(hs);
                float tmp[32];
                if (typ == GgmlType::Q8_0) {
                    for (int i = 0; i < 32; i++) tmp[i] = (float)(int8_t)blk[2 + i] * scale;
                } else {  // element i: low nibble of byte i, element i + 16: high nibble
                    for (int i = 0; i < 16; i++) {
                        tmp[i] = (float)((int)(blk[2 + i] & 0x0f) - 8) * scale;
                        tmp[i + 16] = (float)((int)((blk[2 + i] >> 4) & 0x0f) - 8) * scale;
                    }
                }
                const size_t k = std::min<size_t>(32, n - b * 32);
                std::memcpy(&out[b * 32], tmp, k * 4);
            }
            break;
        default:
            throw Error(ANEHIP_EUNSUPPORTED,
                        "gguf: unsupported quantization type for dequantization: " + std::to_string((uint32_t)typ));
    }
    return out;
}

namespace {
const TensorInfo &find(const GgufFile &g, const std::string &name, const uint8_t **bytes, const uint8_t *file,
                       size_t file_size) {
    const TensorInfo *t = g.get_tensor(name);
    if (!t) bad("tensor not found: " + name);
    const uint64_t off = g.tensor_data_offset + t->offset, n = t->data_size();
    if (off > file_size || n > file_size - off) bad("tensor " + name + " lies past the end of the file");
    *bytes = file + off;
    return *t;
}
}  // namespace

RawTensor extract_tensor_raw(const GgufFile &g, const uint8_t *file, size_t file_size, const std::string &name) {
    const uint8_t *p;
    const TensorInfo &t = find(g, name, &p, file, file_size);
    RawTensor r;
    r.data.assign(p, p + t.data_size());
    r.ne0 = t.dimensions.empty() ? 0 : (size_t)t.dimensions[0];
    r.ne1 = t.dimensions.size() > 1 ? (size_t)t.dimensions[1] : 1;
    r.typ = t.typ;
    return r;
}

std::vector<float> extract_tensor_f32(const GgufFile &g, const uint8_t *file, size_t file_size,
                                      const std::string &name) {
    const uint8_t *p;
    const TensorInfo &t = find(g, name, &p, file, file_size);
    return dequantize_tensor(p, t.data_size(), t.typ, (size_t)t.n_elements());
}

}  // namespace gguf

Qwen35Config qwen35_config_from_gguf(const gguf::GgufFile &g) {
    Qwen35Config c;
    ModelConfig &b = c.base;
    uint32_t v = 0;
    auto need = [&](const char *key) -> size_t {
        uint32_t x;
        if (!g.arch_u32(key, x)) throw Error(ANEHIP_EINVAL, std::string("gguf: missing ") + key);
        return x;
    };
    b.dim = need("embedding_length");
    b.n_heads = need("attention.head_count");
    b.n_kv_heads = g.arch_u32("attention.head_count_kv", v) ? v : b.n_heads;
    b.n_layers = need("block_count");
    b.hidden_dim = need("feed_forward_length");
    b.vocab_size = g.vocab_size(v) ? v : 32000;
    float f;
    b.rope_freq_base = g.arch_f32("rope.freq_base", f) ? f : 10000.0f;
    // model.rs:38,50: context length (default 2048) capped at 4096
    b.max_seq_len = std::min<size_t>(g.arch_u32("context_length", v) ? v : 2048, 4096);
    b.rms_norm_eps = g.arch_f32("attention.layer_norm_rms_epsilon", f) ? f : 1e-6f;
    if (b.n_heads == 0) throw Error(ANEHIP_EINVAL, "gguf: head_count is 0");
    b.head_dim = g.arch_u32("attention.key_length", v) ? v : b.dim / b.n_heads;
    c.full_attention_interval = g.arch_u32("full_attention_interval", v) ? v : 4;
    c.ssm_state_size = g.arch_u32("ssm.state_size", v) ? v : 128;
    c.ssm_conv_kernel = g.arch_u32("ssm.conv_kernel", v) ? v : 4;
    c.ssm_group_count = g.arch_u32("ssm.group_count", v) ? v : 16;
    c.ssm_inner_size = g.arch_u32("ssm.inner_size", v) ? v : b.dim;
    for (size_t l = 0; l < b.n_layers; l++)
        c.layer_types.push_back(g.is_deltanet_layer(l) ? LayerType::DeltaNet : LayerType::FullAttention);
    return c;
}

Qwen35ModelWeights load_qwen35_q8(const gguf::GgufFile &g, const uint8_t *file, size_t file_size,
                                  const Qwen35Config &config) {
    using namespace gguf;
    auto f32 = [&](const std::string &name) { return extract_tensor_f32(g, file, file_size, name); };
    auto quant = [&](const std::string &name) {
        RawTensor r = extract_tensor_raw(g, file, file_size, name);
        if (r.typ != GgmlType::Q8_0 && r.typ != GgmlType::Q4_0)
            throw Error(ANEHIP_EUNSUPPORTED,
                        "gguf: unsupported quantization type: " + std::to_string((uint32_t)r.typ) + " (" + name + ")");
        return Q8Tensor::from_raw(std::move(r.data), r.ne0, r.ne1,
                                  r.typ == GgmlType::Q8_0 ? QuantType::Q8_0 : QuantType::Q4_0);
    };
    Qwen35ModelWeights w;
    w.config = config;
    w.embedding = f32("token_embd.weight");
    w.final_norm = f32("output_norm.weight");
    w.lm_head = g.get_tensor("output.weight") ? quant("output.weight") : quant("token_embd.weight");
    for (size_t l = 0; l < config.base.n_layers; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        FfnWeights ffn{quant(p + "ffn_gate.weight"), quant(p + "ffn_up.weight"), quant(p + "ffn_down.weight")};
        if (config.layer_types[l] == LayerType::DeltaNet) {
            DeltaNetLayerWeights d;
            d.attn_norm = f32(p + "attn_norm.weight");
            d.post_attn_norm = f32(p + "post_attention_norm.weight");
            d.qkv = quant(p + "attn_qkv.weight");
            d.attn_gate = quant(p + "attn_gate.weight");
            d.ssm_a = f32(p + "ssm_a");
            d.ssm_alpha = quant(p + "ssm_alpha.weight");
            d.ssm_beta = quant(p + "ssm_beta.weight");
            d.ssm_conv1d = f32(p + "ssm_conv1d.weight");
            d.ssm_dt_bias = f32(p + "ssm_dt.bias");
            d.ssm_norm = f32(p + "ssm_norm.weight");
            d.ssm_out = quant(p + "ssm_out.weight");
            d.ffn = std::move(ffn);
            w.layers.emplace_back(std::move(d));
        } else {
            FullAttnLayerWeights a;
            a.attn_norm = f32(p + "attn_norm.weight");
            a.post_attn_norm = f32(p + "post_attention_norm.weight");
            a.wq = quant(p + "attn_q.weight");
            a.wk = quant(p + "attn_k.weight");
            a.wv = quant(p + "attn_v.weight");
            a.wo = quant(p + "attn_output.weight");
            a.q_norm = f32(p + "attn_q_norm.weight");
            a.k_norm = f32(p + "attn_k_norm.weight");
            a.ffn = std::move(ffn);
            w.layers.emplace_back(std::move(a));
        }
    }
    return w;
}

}  // namespace ane
