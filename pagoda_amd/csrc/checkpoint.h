// checkpoint.h — readers for the two checkpoint formats the reference loads:
// an MLX model directory (config.json + safetensors shards of 8-bit affine,
// group-64 matrices; pagoda-hf/src/qwen3_5.rs:338-452, 1587-1698) and a Qwen2
// GGUF file (pagoda-hf/src/qwen2_gguf.rs:65-140). Files are memory-mapped;
// tensors are located by name and copied out on demand.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/pagoda_hip.h"
#include "json.h"

namespace pgd {

// read-only memory map of a whole file
class MappedFile {
 public:
  explicit MappedFile(const std::string& path);
  ~MappedFile();
  MappedFile(const MappedFile&) = delete;
  MappedFile& operator=(const MappedFile&) = delete;
  const uint8_t* data() const { return p_; }
  size_t size() const { return n_; }
  const std::string& path() const { return path_; }

 private:
  std::string path_;
  const uint8_t* p_ = nullptr;
  size_t n_ = 0;
};

// element types of checkpoint tensors
enum class DType { U32, BF16, F16, F32, Q4K, Q6K, Q8_0, Q5_0 };

struct TensorView {
  DType dtype;
  std::vector<uint64_t> shape;  // outermost first (safetensors order; GGUF dims reversed to match)
  const uint8_t* data = nullptr;
  size_t bytes = 0;
  uint64_t numel() const {
    uint64_t n = 1;
    for (uint64_t d : shape) n *= d;
    return n;
  }
};

// the safetensors shards of an MLX model directory
class SafetensorsStore {
 public:
  explicit SafetensorsStore(const std::string& dir);
  const TensorView* find(const std::string& name) const;
  const TensorView& at(const std::string& name) const;  // throws kErrFormat "missing ..."

 private:
  std::vector<std::unique_ptr<MappedFile>> files_;
  std::map<std::string, TensorView> tensors_;
  void add_file(const std::string& path, const std::map<std::string, std::string>* owner);
};

// one GGUF file (versions 2 and 3)
class GgufFile {
 public:
  explicit GgufFile(const std::string& path);
  const TensorView* find(const std::string& name) const;
  const TensorView& at(const std::string& name) const;
  // metadata scalars; throw kErrFormat when the key is missing or not numeric / string
  bool has(const std::string& key) const { return meta_.count(key) != 0; }
  double num(const std::string& key) const;
  std::string str(const std::string& key) const;

 private:
  struct Meta {
    bool is_str = false;
    double num = 0.0;
    std::string s;
  };
  std::unique_ptr<MappedFile> file_;
  std::map<std::string, Meta> meta_;
  std::map<std::string, TensorView> tensors_;
  std::map<std::string, uint32_t> other_types_;  // tensors in block types not stored here
};

// Model configuration of a checkpoint. max_pos <= 0 takes the file's context
// length; kv_blocks must be > 0. full (hybrid model): layer kinds in order.
pgd_model_config mlx_config(const std::string& dir, int max_pos, int kv_blocks, std::vector<bool>* full);
pgd_model_config gguf_config(const GgufFile& f, int max_pos, int kv_blocks);

// f32 copy of a plain tensor (F32, BF16 or F16)
std::vector<float> tensor_f32(const TensorView& t, const std::string& name);

}  // namespace pgd
