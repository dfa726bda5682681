// GGUF v3 reader: the weight source for the resident store
// (crates/strata-gguf/src/reader.rs:1-445, metadata.rs). Memory-maps one
// file read-only, parses the header, the metadata and the tensor directory
// with bounds checks, and hands out bounds-checked payload slices. Host code
// only (internal to libstrata_hip).
#pragma once

#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace sh {

// reader.rs:123-176: every value type is parsed; scalars keep their payload
// (integers as i64, u64 as its own field, f32 widened to f64), strings their
// text, arrays their element type and true count.
struct GgufMeta {
  uint32_t ty = 0;
  int64_t i = 0;
  uint64_t u = 0;
  double f = 0.0;
  std::string s;
  uint32_t elem = 0;
  uint64_t count = 0;
};

struct GgufTensor {
  std::string name;
  std::vector<uint64_t> shape;  // GGUF order: dim 0 fastest
  uint32_t ty = 0;
  uint64_t offset = 0;  // from the start of the data section
};

// Error kinds of crates/strata-gguf/src/error.rs that the reader returns.
enum class GgufErr {
  kOk,
  kIo,
  kBadMagic,
  kUnsupportedVersion,
  kBadKeyLength,
  kStringNotUtf8,
  kBadValueType,
  kDuplicateTensor,  // Error::TensorNotFound { name } in the reference (reader.rs:290-292)
  kWrongTensorDims,
  kTruncated,
  kUnsupportedQuant,
};

struct GgufFile {
  const uint8_t* map = nullptr;
  uint64_t size = 0;
  uint32_t version = 0;
  uint64_t alignment = 32;
  uint64_t data_start = 0;
  uint64_t n_kv = 0;
  std::vector<GgufTensor> tensors;
  std::unordered_map<std::string, size_t> index;
  std::unordered_map<std::string, GgufMeta> meta;
  ~GgufFile();
};

// Opens and parses `path`; on failure returns the error kind and a message.
GgufErr gguf_open(const char* path, GgufFile** out, std::string* msg);

// quant.rs:125-164 for every type id the reference knows: (block elements,
// block bytes); {0, 0} for an unknown id.
void gguf_type_geometry(uint32_t ty, uint64_t* block, uint64_t* bytes);

// reader.rs:399-423 (tensor_payload_bytes) and :425-445 (tensor_data).
GgufErr gguf_payload_bytes(const GgufTensor& t, uint64_t* bytes, std::string* msg);
GgufErr gguf_tensor_data(const GgufFile& f, const GgufTensor& t, const uint8_t** data, uint64_t* bytes,
                         std::string* msg);

// split_paths (reader.rs:524-572): the shards of `<name>-NNNNN-of-MMMMM.gguf`
// in split order; any other path is a single-shard model. A missing shard is
// kIo with a message naming it.
GgufErr gguf_split_paths(const std::string& any, std::vector<std::string>* out, std::string* msg);

// GgufModel (reader.rs:450-522): every shard, one name index across them (a
// name in two shards is kDuplicateTensor).
struct GgufModel {
  std::vector<GgufFile*> shards;
  std::unordered_map<std::string, std::pair<size_t, size_t>> index;  // name -> (shard, tensor)
  ~GgufModel();
};
GgufErr gguf_model_open(const char* any_shard, GgufModel** out, std::string* msg);

}  // namespace sh
