// checkpoint.cpp — MLX safetensors directories and Qwen2 GGUF files: mapping,
// tensor directories, configuration (see checkpoint.h).
#include "checkpoint.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <sstream>

#include "common.h"

namespace pgd {

namespace {

[[noreturn]] void bad(const std::string& msg) { throw Error{kErrFormat, msg}; }

bool file_exists(const std::string& p) {
  struct stat st;
  return ::stat(p.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

std::string read_text(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) bad("cannot open " + path);
  std::ostringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

// element count of a shape, rejecting products past 2^48 (no file holds more;
// this keeps every byte count below computed exactly in 64 bits)
uint64_t checked_numel(const std::vector<uint64_t>& shape, const std::string& what) {
  uint64_t n = 1;
  for (uint64_t d : shape) {
    if (d > (1ull << 48) || (d && n > (1ull << 48) / d)) bad(what + ": shape too large");
    n *= d;
  }
  return n;
}

size_t dtype_size(DType t) {
  switch (t) {
    case DType::U32:
    case DType::F32: return 4;
    case DType::BF16:
    case DType::F16: return 2;
    default: return 0;
  }
}

int json_int(const json::Value& v, const char* key) {
  const json::Value* x = v.get(key);
  if (!x || !x->is_num()) bad(std::string("config.json: missing integer ") + key);
  if (x->num != std::floor(x->num) || x->num < 0 || x->num > 2147483647.0) bad(std::string("config.json: bad ") + key);
  return (int)x->num;
}

double json_num(const json::Value& v, const char* key) {
  const json::Value* x = v.get(key);
  if (!x || !x->is_num()) bad(std::string("config.json: missing number ") + key);
  return x->num;
}

}  // namespace

// ---------------------------------------------------------------------------
MappedFile::MappedFile(const std::string& path) : path_(path) {
  int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) bad("cannot open " + path);
  struct stat st;
  if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
    ::close(fd);
    bad("empty or unreadable file " + path);
  }
  n_ = (size_t)st.st_size;
  void* p = ::mmap(nullptr, n_, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (p == MAP_FAILED) bad("cannot map " + path);
  p_ = (const uint8_t*)p;
}

MappedFile::~MappedFile() {
  if (p_) ::munmap((void*)p_, n_);
}

std::vector<float> tensor_f32(const TensorView& t, const std::string& name) {
  const uint64_t n = t.numel();
  std::vector<float> out(n);
  switch (t.dtype) {
    case DType::F32: memcpy(out.data(), t.data, n * 4); break;
    case DType::BF16:
      for (uint64_t i = 0; i < n; ++i) {
        uint16_t h;
        memcpy(&h, t.data + 2 * i, 2);
        out[i] = bf16_to_f32(h);
      }
      break;
    case DType::F16:
      for (uint64_t i = 0; i < n; ++i) {
        uint16_t h;
        memcpy(&h, t.data + 2 * i, 2);
        out[i] = f16_to_f32(h);
      }
      break;
    default: bad(name + " is not a plain float tensor");
  }
  return out;
}

// ---------------------------------------------------------------------------
// safetensors: u64 header length, JSON header, data
// (qwen3_5.rs:1587-1645, 1686-1692)
// ---------------------------------------------------------------------------
void SafetensorsStore::add_file(const std::string& path, const std::map<std::string, std::string>* owner) {
  files_.push_back(std::make_unique<MappedFile>(path));
  const MappedFile& f = *files_.back();
  if (f.size() < 8) bad(path + ": safetensors too small");
  uint64_t hn;
  memcpy(&hn, f.data(), 8);
  if (hn > f.size() - 8) bad(path + ": header length past the end of the file");
  json::Value hdr = json::parse((const char*)f.data() + 8, (size_t)hn);
  if (hdr.kind != json::Value::Object) bad(path + ": header is not an object");
  const uint8_t* base = f.data() + 8 + hn;
  const size_t avail = f.size() - 8 - hn;
  const std::string fname = path.substr(path.find_last_of('/') + 1);
  for (const auto& kv : hdr.obj) {
    if (kv.first == "__metadata__") continue;
    if (owner) {  // the index names one shard per tensor
      auto it = owner->find(kv.first);
      if (it == owner->end() || it->second != fname) continue;
    }
    const json::Value& m = kv.second;
    const json::Value* dt = m.get("dtype");
    const json::Value* shape = m.get("shape");
    const json::Value* offs = m.get("data_offsets");
    if (!dt || dt->kind != json::Value::String || !shape || shape->kind != json::Value::Array || !offs ||
        offs->kind != json::Value::Array || offs->arr.size() != 2)
      bad(path + ": bad entry for " + kv.first);
    TensorView t;
    if (dt->str == "U32") t.dtype = DType::U32;
    else if (dt->str == "BF16") t.dtype = DType::BF16;
    else if (dt->str == "F16") t.dtype = DType::F16;
    else if (dt->str == "F32") t.dtype = DType::F32;
    else bad("unsupported dtype " + dt->str + " for " + kv.first);
    for (const auto& d : shape->arr) {
      if (!d.is_num() || d.num < 0) bad(path + ": bad shape for " + kv.first);
      t.shape.push_back((uint64_t)d.num);
    }
    const double b0 = offs->arr[0].num, b1 = offs->arr[1].num;
    if (!offs->arr[0].is_num() || !offs->arr[1].is_num() || b0 < 0 || b1 < b0 || b1 > (double)avail)
      bad(path + ": data offsets out of range for " + kv.first);
    t.data = base + (size_t)b0;
    t.bytes = (size_t)(b1 - b0);
    if (t.bytes != checked_numel(t.shape, kv.first) * dtype_size(t.dtype))
      bad(path + ": size does not match shape for " + kv.first);
    tensors_[kv.first] = t;
  }
}

SafetensorsStore::SafetensorsStore(const std::string& dir) {
  const std::string index = dir + "/model.safetensors.index.json";
  if (file_exists(index)) {
    json::Value idx = json::parse(read_text(index));
    const json::Value* wm = idx.get("weight_map");
    if (!wm || wm->kind != json::Value::Object) bad(index + ": no weight_map");
    std::map<std::string, std::string> owner;
    std::vector<std::string> shards;
    for (const auto& kv : wm->obj) {
      if (kv.second.kind != json::Value::String) bad(index + ": bad weight_map entry " + kv.first);
      owner[kv.first] = kv.second.str;
      shards.push_back(kv.second.str);
    }
    std::sort(shards.begin(), shards.end());
    shards.erase(std::unique(shards.begin(), shards.end()), shards.end());
    for (const auto& s : shards) {
      if (s.find('/') != std::string::npos) bad(index + ": shard names must be plain file names");
      add_file(dir + "/" + s, &owner);
    }
  } else if (file_exists(dir + "/model.safetensors")) {
    add_file(dir + "/model.safetensors", nullptr);  // one shard, no index
  } else {
    bad("no safetensors index or model.safetensors in " + dir);
  }
}

const TensorView* SafetensorsStore::find(const std::string& name) const {
  auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

const TensorView& SafetensorsStore::at(const std::string& name) const {
  const TensorView* t = find(name);
  if (!t) bad("missing " + name);
  return *t;
}

// ---------------------------------------------------------------------------
// GGUF (v2/v3): magic, version, tensor count, metadata count, metadata
// key/values, tensor infos, alignment padding, data
// ---------------------------------------------------------------------------
namespace {

enum GgufType {
  G_U8 = 0, G_I8 = 1, G_U16 = 2, G_I16 = 3, G_U32 = 4, G_I32 = 5, G_F32 = 6, G_BOOL = 7, G_STR = 8, G_ARR = 9,
  G_U64 = 10, G_I64 = 11, G_F64 = 12
};

// ggml tensor types the backend stores
enum { GGML_F32 = 0, GGML_F16 = 1, GGML_Q5_0 = 6, GGML_Q8_0 = 8, GGML_Q4_K = 12, GGML_Q6_K = 14 };

struct Cursor {
  const uint8_t* p;
  const uint8_t* end;
  const std::string& path;
  template <typename T>
  T get() {
    if ((size_t)(end - p) < sizeof(T)) bad(path + ": truncated GGUF header");
    T v;
    memcpy(&v, p, sizeof(T));
    p += sizeof(T);
    return v;
  }
  std::string str() {
    uint64_t n = get<uint64_t>();
    if ((uint64_t)(end - p) < n) bad(path + ": truncated GGUF string");
    std::string s((const char*)p, (size_t)n);
    p += n;
    return s;
  }
  void skip(uint64_t n) {
    if ((uint64_t)(end - p) < n) bad(path + ": truncated GGUF value");
    p += n;
  }
};

size_t gguf_scalar_size(uint32_t t) {
  switch (t) {
    case G_U8: case G_I8: case G_BOOL: return 1;
    case G_U16: case G_I16: return 2;
    case G_U32: case G_I32: case G_F32: return 4;
    case G_U64: case G_I64: case G_F64: return 8;
    default: return 0;
  }
}

double gguf_scalar(Cursor& c, uint32_t t) {
  switch (t) {
    case G_U8: return c.get<uint8_t>();
    case G_I8: return c.get<int8_t>();
    case G_BOOL: return c.get<uint8_t>();
    case G_U16: return c.get<uint16_t>();
    case G_I16: return c.get<int16_t>();
    case G_U32: return c.get<uint32_t>();
    case G_I32: return c.get<int32_t>();
    case G_F32: return c.get<float>();
    case G_U64: return (double)c.get<uint64_t>();
    case G_I64: return (double)c.get<int64_t>();
    case G_F64: return c.get<double>();
  }
  bad(c.path + ": unknown GGUF value type " + std::to_string(t));
}

}  // namespace

GgufFile::GgufFile(const std::string& path) : file_(std::make_unique<MappedFile>(path)) {
  Cursor c{file_->data(), file_->data() + file_->size(), path};
  if (c.get<uint32_t>() != 0x46554747u) bad(path + ": not a GGUF file");
  const uint32_t version = c.get<uint32_t>();
  if (version != 2 && version != 3) bad(path + ": GGUF version " + std::to_string(version) + " (2 or 3 supported)");
  const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
  if (n_tensors > (1u << 24) || n_kv > (1u << 24)) bad(path + ": implausible GGUF counts");
  for (uint64_t i = 0; i < n_kv; ++i) {
    std::string key = c.str();
    const uint32_t t = c.get<uint32_t>();
    Meta m;
    if (t == G_STR) {
      m.is_str = true;
      m.s = c.str();
    } else if (t == G_ARR) {  // arrays (tokenizer tables) are skipped
      const uint32_t et = c.get<uint32_t>();
      const uint64_t n = c.get<uint64_t>();
      if (et == G_STR) {
        for (uint64_t j = 0; j < n; ++j) c.str();
      } else {
        const size_t es = gguf_scalar_size(et);
        if (!es) bad(path + ": unsupported GGUF array type for " + key);
        if (n > file_->size() / es) bad(path + ": GGUF array too long for " + key);
        c.skip(n * es);
      }
      continue;
    } else {
      m.num = gguf_scalar(c, t);
    }
    meta_[key] = m;
  }
  uint64_t align = 32;
  if (has("general.alignment")) {
    align = (uint64_t)num("general.alignment");
    if (align == 0 || (align & (align - 1))) bad(path + ": general.alignment must be a power of two");
  }
  struct Info {
    std::string name;
    std::vector<uint64_t> ne;
    uint32_t type;
    uint64_t off;
  };
  std::vector<Info> infos;
  for (uint64_t i = 0; i < n_tensors; ++i) {
    Info in;
    in.name = c.str();
    const uint32_t nd = c.get<uint32_t>();
    if (nd == 0 || nd > 4) bad(path + ": bad dimension count for " + in.name);
    for (uint32_t d = 0; d < nd; ++d) in.ne.push_back(c.get<uint64_t>());
    in.type = c.get<uint32_t>();
    in.off = c.get<uint64_t>();
    infos.push_back(in);
  }
  const size_t head = (size_t)(c.p - file_->data());
  const size_t data0 = (head + align - 1) / align * align;
  if (data0 > file_->size()) bad(path + ": no tensor data");
  const size_t avail = file_->size() - data0;
  for (const Info& in : infos) {
    TensorView t;
    // GGUF lists ne[0] (innermost) first; the view keeps outermost first
    for (size_t d = in.ne.size(); d-- > 0;) t.shape.push_back(in.ne[d]);
    const uint64_t inner = in.ne[0];
    const uint64_t outer = checked_numel(t.shape, in.name) / std::max<uint64_t>(inner, 1);
    uint64_t bytes = 0;
    switch (in.type) {
      case GGML_F32: t.dtype = DType::F32; bytes = t.numel() * 4; break;
      case GGML_F16: t.dtype = DType::F16; bytes = t.numel() * 2; break;
      case GGML_Q4_K:
      case GGML_Q6_K:
        if (inner % 256) bad(path + ": " + in.name + " rows are not whole 256-weight super-blocks");
        t.dtype = in.type == GGML_Q4_K ? DType::Q4K : DType::Q6K;
        bytes = outer * (inner / 256) * (in.type == GGML_Q4_K ? 144 : 210);
        break;
      case GGML_Q8_0:
      case GGML_Q5_0:
        if (inner % 32) bad(path + ": " + in.name + " rows are not whole 32-weight blocks");
        t.dtype = in.type == GGML_Q8_0 ? DType::Q8_0 : DType::Q5_0;
        bytes = outer * (inner / 32) * (in.type == GGML_Q8_0 ? 34 : 22);
        break;
      default:
        // other block types are tolerated until a tensor of that type is asked for
        other_types_[in.name] = in.type;
        continue;
    }
    if (in.off % align || in.off > avail || bytes > avail - in.off) bad(path + ": data of " + in.name + " out of range");
    t.data = file_->data() + data0 + in.off;
    t.bytes = (size_t)bytes;
    tensors_[in.name] = t;
  }
}

const TensorView* GgufFile::find(const std::string& name) const {
  auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

const TensorView& GgufFile::at(const std::string& name) const {
  const TensorView* t = find(name);
  if (t) return *t;
  auto it = other_types_.find(name);
  if (it != other_types_.end())
    bad(name + " has ggml type " + std::to_string(it->second) + "; the backend stores F32, F16, Q4_K, Q6_K, Q8_0 and Q5_0 tensors");
  bad("missing " + name);
}

double GgufFile::num(const std::string& key) const {
  auto it = meta_.find(key);
  if (it == meta_.end() || it->second.is_str) bad("GGUF metadata: missing number " + key);
  return it->second.num;
}

std::string GgufFile::str(const std::string& key) const {
  auto it = meta_.find(key);
  if (it == meta_.end() || !it->second.is_str) bad("GGUF metadata: missing string " + key);
  return it->second.s;
}

// ---------------------------------------------------------------------------
// configurations
// ---------------------------------------------------------------------------
pgd_model_config mlx_config(const std::string& dir, int max_pos, int kv_blocks, std::vector<bool>* full) {
  // qwen3_5.rs:339-383
  json::Value cfg = json::parse(read_text(dir + "/config.json"));
  const json::Value* tc = cfg.get("text_config");
  const json::Value& text = tc ? *tc : cfg;
  pgd_model_config c{};
  c.arch = PGD_ARCH_QWEN35;
  c.hidden = json_int(text, "hidden_size");
  c.n_layers = json_int(text, "num_hidden_layers");
  c.intermediate = json_int(text, "intermediate_size");
  c.vocab = json_int(text, "vocab_size");
  c.heads = json_int(text, "num_attention_heads");
  c.kv_heads = json_int(text, "num_key_value_heads");
  c.head_dim = json_int(text, "head_dim");
  c.k_heads = json_int(text, "linear_num_key_heads");
  c.v_heads = json_int(text, "linear_num_value_heads");
  c.k_dim = json_int(text, "linear_key_head_dim");
  c.v_dim = json_int(text, "linear_value_head_dim");
  c.conv_kernel = json_int(text, "linear_conv_kernel_dim");
  c.eps = (float)json_num(text, "rms_norm_eps");
  const json::Value* rp = text.get("rope_parameters");
  const json::Value* theta = rp ? rp->get("rope_theta") : nullptr;
  if (!theta || !theta->is_num()) bad("config.json: missing rope_parameters.rope_theta");
  c.rope_theta = (float)theta->num;
  const json::Value* prf = rp->get("partial_rotary_factor");
  const float partial = prf && prf->is_num() ? (float)prf->num : 0.25f;
  c.rotary_dim = (int)((float)c.head_dim * partial);
  const json::Value* kinds = text.get("layer_types");
  if (!kinds || kinds->kind != json::Value::Array) bad("config.json: missing layer_types");
  if ((int)kinds->arr.size() != c.n_layers) bad("config.json: layer_types length");
  full->assign(c.n_layers, false);
  for (int i = 0; i < c.n_layers; ++i) {
    const json::Value& k = kinds->arr[i];
    if (k.kind != json::Value::String) bad("config.json: layer type");
    if (k.str == "full_attention") (*full)[i] = true;
    else if (k.str != "linear_attention") bad("unknown layer type " + k.str);
  }
  // the repeating pattern, when there is one (layer i full iff i % P == P - 1)
  c.full_every = 0;
  for (int P = 1; P <= c.n_layers && !c.full_every; ++P) {
    bool ok = true;
    for (int i = 0; i < c.n_layers && ok; ++i) ok = (*full)[i] == (i % P == P - 1);
    if (ok) c.full_every = P;
  }
  const json::Value* q = cfg.get("quantization_config");
  if (!q) bad("config.json: missing quantization_config");
  if (json_int(*q, "bits") != 8) bad("only 8-bit affine quantization is supported");
  if (json_int(*q, "group_size") != 64) bad("only group size 64 is supported");
  const json::Value* mode = q->get("mode");
  if (!mode || mode->kind != json::Value::String || mode->str != "affine") bad("only affine quantization is supported");
  if (max_pos <= 0) {
    const json::Value* mp = text.get("max_position_embeddings");
    if (!mp || !mp->is_num()) bad("config.json has no max_position_embeddings: pass max_pos");
    max_pos = (int)mp->num;
  }
  c.max_pos = max_pos;
  c.kv_block = 16;
  PGD_CHECK(kv_blocks > 0, kErrArg, "kv_blocks must be > 0");
  c.kv_blocks = kv_blocks;
  return c;
}

pgd_model_config gguf_config(const GgufFile& f, int max_pos, int kv_blocks) {
  // qwen2_gguf.rs:67-91
  const std::string arch = f.str("general.architecture");
  if (arch != "qwen2") bad("only Qwen2 GGUF is supported (general.architecture = " + arch + ")");
  pgd_model_config c{};
  c.arch = PGD_ARCH_QWEN2;
  c.heads = (int)f.num("qwen2.attention.head_count");
  c.kv_heads = (int)f.num("qwen2.attention.head_count_kv");
  c.hidden = (int)f.num("qwen2.embedding_length");
  c.n_layers = (int)f.num("qwen2.block_count");
  c.eps = (float)f.num("qwen2.attention.layer_norm_rms_epsilon");
  c.rope_theta = f.has("qwen2.rope.freq_base") ? (float)f.num("qwen2.rope.freq_base") : 1000000.0f;
  if (c.heads <= 0 || c.hidden % c.heads) bad("hidden size not divisible by the head count");
  c.head_dim = c.hidden / c.heads;
  c.rotary_dim = c.head_dim;
  const TensorView& emb = f.at("token_embd.weight");
  if (emb.shape.size() != 2) bad("token_embd.weight is not a matrix");
  c.vocab = (int)emb.shape[0];
  const TensorView& gate = f.at("blk.0.ffn_gate.weight");
  c.intermediate = f.has("qwen2.feed_forward_length") ? (int)f.num("qwen2.feed_forward_length") : (int)gate.shape[0];
  c.full_every = 1;
  if (max_pos <= 0) max_pos = (int)f.num("qwen2.context_length");
  c.max_pos = max_pos;
  c.kv_block = 16;
  PGD_CHECK(kv_blocks > 0, kErrArg, "kv_blocks must be > 0");
  c.kv_blocks = kv_blocks;
  return c;
}

}  // namespace pgd
