// gguf.hpp — GGUF v2/v3 reader of the C++ engine API: parses the header,
// metadata and tensor index of a GGUF file and hands out tensors as raw
// blocks (Q8_0 / Q4_0, for the quantised projections) or dequantised fp32
// (norms, conv weights, the embedding table).  Mirrors crates/gguf:
//
//   GgufType, GgmlType (block sizes)       crates/gguf/src/parser.rs:17-136
//   MetadataValue, TensorInfo              parser.rs:138-206
//   GgufFile::parse, get_tensor and the    parser.rs:208-536
//     metadata accessors
//   dequantize_tensor (F32, F16, Q4_0,     crates/gguf/src/dequant.rs:12-38
//     Q8_0)
//   extract_tensor_raw, extract_tensor_f32 crates/gguf/src/to_ane.rs:11-44
//
// Errors (the reference's anyhow::bail!) are thrown as ane::Error with
// ANEHIP_EINVAL (malformed file) or ANEHIP_EUNSUPPORTED (a type this path
// does not handle).  All integers are little endian, as in the format.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <variant>
#include <vector>

#include "ane_engine.hpp"

namespace ane {
namespace gguf {

// Metadata value types (parser.rs:19-34).
enum class GgufType : uint32_t {
    U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, Bool = 7, String = 8, Array = 9,
    U64 = 10, I64 = 11, F64 = 12
};

// Tensor element types the parser accepts (parser.rs:96-113); only F32, F16,
// Q4_0 and Q8_0 can be loaded.
enum class GgmlType : uint32_t {
    F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q4K = 12, Q5K = 13, Q6K = 14
};
size_t block_size(GgmlType t);       // elements per block (parser.rs:117-126)
size_t bytes_per_block(GgmlType t);  // parser.rs:129-142

struct MetadataValue;
using MetadataArray = std::vector<MetadataValue>;
struct MetadataValue {
    GgufType type = GgufType::U32;
    std::variant<uint64_t, int64_t, double, bool, std::string, std::shared_ptr<MetadataArray>> v;
    // the reference's as_u32 / as_u64 / as_f32 / as_str: only the exact type
    bool as_u32(uint32_t &out) const;
    bool as_u64(uint64_t &out) const;
    bool as_f32(float &out) const;
    const std::string *as_str() const;
    const MetadataArray *as_array() const;
};

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dimensions;  // ne0 (fastest) first
    GgmlType typ = GgmlType::F32;
    uint64_t offset = 0;  // from the start of the tensor data section
    uint64_t n_elements() const;
    uint64_t data_size() const;  // bytes: whole blocks (parser.rs:198-205)
};

class GgufFile {
  public:
    uint32_t version = 0;
    std::map<std::string, MetadataValue> metadata;
    std::vector<TensorInfo> tensors;
    uint64_t tensor_data_offset = 0;  // absolute file offset of the tensor data

    // Parses the header, metadata and tensor index from the first `size`
    // bytes of a file (the tensor data itself is not needed).
    static GgufFile parse(const uint8_t *data, size_t size);

    const TensorInfo *get_tensor(const std::string &name) const;
    const std::string *architecture() const;  // general.architecture
    // {arch}.<key> as u32 / f32 (absent or of another type: false)
    bool arch_u32(const char *key, uint32_t &out) const;
    bool arch_f32(const char *key, float &out) const;
    bool vocab_size(uint32_t &out) const;  // length of tokenizer.ggml.tokens
    // DeltaNet layer iff blk.<l>.ssm_a exists (parser.rs:483-486)
    bool is_deltanet_layer(size_t layer) const;
};

// A GGUF file mapped read-only into memory (the reference reads the file
// into a Vec<u8>; mapping avoids a copy of a multi-GB checkpoint).
class MappedFile {
  public:
    explicit MappedFile(const std::string &path);
    ~MappedFile();
    MappedFile(const MappedFile &) = delete;
    MappedFile &operator=(const MappedFile &) = delete;
    const uint8_t *data() const { return data_; }
    size_t size() const { return size_; }

  private:
    const uint8_t *data_ = nullptr;
    size_t size_ = 0;
};

// n elements of a tensor's bytes -> fp32 (dequant.rs:12-38 for the quants;
// F16 is the IEEE half conversion).
std::vector<float> dequantize_tensor(const uint8_t *data, size_t size, GgmlType typ, size_t n_elements);

// The tensor's blocks as stored (to_ane.rs:11-30): ne0 = fast dim (input),
// ne1 = slow dim (output rows).
struct RawTensor {
    std::vector<uint8_t> data;
    size_t ne0 = 0, ne1 = 1;
    GgmlType typ = GgmlType::F32;
};
RawTensor extract_tensor_raw(const GgufFile &g, const uint8_t *file, size_t file_size, const std::string &name);
std::vector<float> extract_tensor_f32(const GgufFile &g, const uint8_t *file, size_t file_size,
                                      const std::string &name);

}  // namespace gguf

// Qwen35Config::from_gguf (crates/engine/src/model.rs:21-98): the shape from
// the {arch}.* metadata with the reference's defaults, layer types from the
// presence of blk.<l>.ssm_a.
Qwen35Config qwen35_config_from_gguf(const gguf::GgufFile &g);

// load_qwen35_q8 (crates/cli/src/main.rs:1875-1994): the embedding and norms
// as fp32, every projection as raw Q8_0 / Q4_0 blocks; lm_head is
// output.weight, else the tied token_embd.weight.
Qwen35ModelWeights load_qwen35_q8(const gguf::GgufFile &g, const uint8_t *file, size_t file_size,
                                  const Qwen35Config &config);

}  // namespace ane
