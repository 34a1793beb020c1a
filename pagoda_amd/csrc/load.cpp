// load.cpp — models from checkpoints: MLX 8-bit affine directories (hybrid
// model, pagoda-hf/src/qwen3_5.rs:338-452) and Qwen2 GGUF files
// (pagoda-hf/src/qwen2_gguf.rs:65-140), behind the pgd_model C ABI.
#include <sys/stat.h>

#include <cstring>
#include <string>

#include "checkpoint.h"
#include "common.h"
#include "model.h"

namespace pgd {

namespace {

[[noreturn]] void bad(const std::string& msg) { throw Error{kErrFormat, msg}; }

void upload_floats(float* dst, const std::vector<float>& v, hipStream_t s) {
  PGD_HIP(hipMemcpyAsync(dst, v.data(), v.size() * 4, hipMemcpyHostToDevice, s));
  PGD_HIP(hipStreamSynchronize(s));
}

// ---------------------------------------------------------------------------
// MLX directory: `language_model.*` tensors (qwen3_5.rs:384-450); matrices
// are `<name>.weight` (u32 [out, in / 4]), `.scales` and `.biases` (bf16
// [out, in / 64]) (qwen3_5.rs:1651-1672)
// ---------------------------------------------------------------------------
class MlxSource : public WeightSource {
 public:
  MlxSource(const std::string& dir, std::vector<bool> full) : st_(dir), full_(std::move(full)) {}
  bool full_layer(int i) const override { return full_[i]; }
  bool tied_head() const override { return false; }

  void matrix(QMat& q, int fmt, int n_out, int n_in, int li, int kind, hipStream_t s) override {
    (void)fmt;
    Affine a = affine(name(li, kind), n_out, n_in);
    qmat_alloc(q, FMT_A8, n_out, n_in, s);
    qmat_upload_a8(q, a.packed, a.scales, a.biases, s);
  }

  bool stacked(QMat& q, int fmt, int n_in, const std::vector<std::pair<int, int>>& parts, int li,
               hipStream_t s) override {
    if (fmt != FMT_A8) return false;
    int n = 0;
    for (auto& p : parts) n += p.second;
    const size_t G = (size_t)n_in / 64;
    std::vector<uint32_t> packed((size_t)n * n_in / 4);
    std::vector<uint16_t> scales((size_t)n * G), biases((size_t)n * G);
    size_t r = 0;
    for (auto& p : parts) {
      Affine a = affine(name(li, p.first), p.second, n_in);
      memcpy(packed.data() + r * n_in / 4, a.packed, (size_t)p.second * n_in);
      memcpy(scales.data() + r * G, a.scales, (size_t)p.second * G * 2);
      memcpy(biases.data() + r * G, a.biases, (size_t)p.second * G * 2);
      r += p.second;
    }
    qmat_alloc(q, FMT_A8, n, n_in, s);
    qmat_upload_a8(q, packed.data(), scales.data(), biases.data(), s);
    return true;
  }

  void vec(float* dst, size_t n, int li, int kind, hipStream_t s) override {
    const std::string nm = name(li, kind);
    std::vector<float> v = tensor_f32(st_.at(nm), nm);
    if (v.size() != n) bad(nm + ": expected " + std::to_string(n) + " values, found " + std::to_string(v.size()));
    upload_floats(dst, v, s);
  }

 private:
  struct Affine {
    const uint32_t* packed;
    const uint16_t* scales;
    const uint16_t* biases;
  };
  SafetensorsStore st_;
  std::vector<bool> full_;

  // qwen3_5.rs:1651-1672: codes u32 [out, in / 4], bf16 scales / biases [out, in / 64]
  Affine affine(const std::string& nm, int n_out, int n_in) const {
    const TensorView& w = st_.at(nm + ".weight");
    const TensorView& sc = st_.at(nm + ".scales");
    const TensorView& bi = st_.at(nm + ".biases");
    if (w.dtype != DType::U32) bad(nm + " weight is not packed u32");
    if (sc.dtype != DType::BF16 || bi.dtype != DType::BF16) bad(nm + " scales / biases are not bf16");
    if (w.shape.size() != 2 || w.shape[0] != (uint64_t)n_out || w.shape[1] * 4 != (uint64_t)n_in)
      bad(nm + ": expected " + std::to_string(n_out) + " x " + std::to_string(n_in) + " codes");
    const std::vector<uint64_t> g{(uint64_t)n_out, (uint64_t)n_in / 64};
    if (sc.shape != g || bi.shape != g) bad(nm + " group mismatch");
    return {reinterpret_cast<const uint32_t*>(w.data), reinterpret_cast<const uint16_t*>(sc.data),
            reinterpret_cast<const uint16_t*>(bi.data)};
  }

  static std::string name(int li, int kind) {
    const std::string pre = "language_model.model";
    if (li < 0) {
      switch (kind) {
        case K_EMBED: return pre + ".embed_tokens";
        case K_HEAD: return "language_model.lm_head";
        case K_FINAL_NORM: return pre + ".norm.weight";
      }
      bad("no MLX tensor for kind " + std::to_string(kind));
    }
    const std::string p = pre + ".layers." + std::to_string(li);
    switch (kind) {
      case K_IN_NORM: return p + ".input_layernorm.weight";
      case K_POST_NORM: return p + ".post_attention_layernorm.weight";
      case K_GATE: return p + ".mlp.gate_proj";
      case K_UP: return p + ".mlp.up_proj";
      case K_DOWN: return p + ".mlp.down_proj";
      case K_QKV: return p + ".linear_attn.in_proj_qkv";
      case K_Z: return p + ".linear_attn.in_proj_z";
      case K_A: return p + ".linear_attn.in_proj_a";
      case K_B: return p + ".linear_attn.in_proj_b";
      case K_OUT: return p + ".linear_attn.out_proj";
      case K_CONV: return p + ".linear_attn.conv1d.weight";
      case K_ALOG: return p + ".linear_attn.A_log";
      case K_DTB: return p + ".linear_attn.dt_bias";
      case K_GNORM: return p + ".linear_attn.norm.weight";
      case K_Q: return p + ".self_attn.q_proj";
      case K_K: return p + ".self_attn.k_proj";
      case K_V: return p + ".self_attn.v_proj";
      case K_O: return p + ".self_attn.o_proj";
      case K_QNORM: return p + ".self_attn.q_norm.weight";
      case K_KNORM: return p + ".self_attn.k_norm.weight";
    }
    bad("no MLX tensor for kind " + std::to_string(kind));
  }
};

// ---------------------------------------------------------------------------
// Qwen2 GGUF (qwen2_gguf.rs:88-124): Q4_K / Q6_K / Q8_0 / Q5_0 matrices, F32 / F16 vectors;
// lm_head is output.weight, else the embedding (qwen2_gguf.rs:96-99)
// ---------------------------------------------------------------------------
class GgufSource : public WeightSource {
 public:
  explicit GgufSource(const GgufFile& f) : f_(f) {}
  bool full_layer(int) const override { return true; }
  bool tied_head() const override { return f_.find("output.weight") == nullptr; }

  void matrix(QMat& q, int fmt, int n_out, int n_in, int li, int kind, hipStream_t s) override {
    (void)fmt;
    const std::string nm = name(li, kind);
    const TensorView& t = f_.at(nm);
    const int f = fmt_of(t, nm);
    if (t.shape.size() != 2 || t.shape[0] != (uint64_t)n_out || t.shape[1] != (uint64_t)n_in)
      bad(nm + ": expected " + std::to_string(n_out) + " x " + std::to_string(n_in));
    qmat_alloc(q, f, n_out, n_in, s);
    qmat_upload_kq(q, t.data, s);
  }

  // row-major GGML blocks of the same type concatenate into one matrix
  bool stacked(QMat& q, int, int n_in, const std::vector<std::pair<int, int>>& parts, int li,
               hipStream_t s) override {
    std::vector<const TensorView*> ts;
    int n = 0;
    for (auto& p : parts) {
      const std::string nm = name(li, p.first);
      const TensorView& t = f_.at(nm);
      if (t.shape.size() != 2 || t.shape[0] != (uint64_t)p.second || t.shape[1] != (uint64_t)n_in)
        bad(nm + ": expected " + std::to_string(p.second) + " x " + std::to_string(n_in));
      if (!ts.empty() && t.dtype != ts[0]->dtype) return false;
      ts.push_back(&t);
      n += p.second;
    }
    const int f = fmt_of(*ts[0], name(li, parts[0].first));
    std::vector<uint8_t> blocks;
    for (const TensorView* t : ts) blocks.insert(blocks.end(), t->data, t->data + t->bytes);
    qmat_alloc(q, f, n, n_in, s);
    qmat_upload_kq(q, blocks.data(), s);
    return true;
  }

  void vec(float* dst, size_t n, int li, int kind, hipStream_t s) override {
    const std::string nm = name(li, kind);
    std::vector<float> v = tensor_f32(f_.at(nm), nm);
    if (v.size() != n) bad(nm + ": expected " + std::to_string(n) + " values, found " + std::to_string(v.size()));
    upload_floats(dst, v, s);
  }

 private:
  const GgufFile& f_;

  static int fmt_of(const TensorView& t, const std::string& nm) {
    switch (t.dtype) {
      case DType::Q4K: return FMT_Q4K;
      case DType::Q6K: return FMT_Q6K;
      case DType::Q8_0: return FMT_Q8_0;
      case DType::Q5_0: return FMT_Q5_0;
      default: bad(nm + " must be Q4_K, Q6_K, Q8_0 or Q5_0");
    }
  }

  static std::string name(int li, int kind) {
    if (li < 0) {
      switch (kind) {
        case K_EMBED: return "token_embd.weight";
        case K_HEAD: return "output.weight";
        case K_FINAL_NORM: return "output_norm.weight";
      }
      bad("no GGUF tensor for kind " + std::to_string(kind));
    }
    const std::string p = "blk." + std::to_string(li);
    switch (kind) {
      case K_IN_NORM: return p + ".attn_norm.weight";
      case K_POST_NORM: return p + ".ffn_norm.weight";
      case K_Q: return p + ".attn_q.weight";
      case K_K: return p + ".attn_k.weight";
      case K_V: return p + ".attn_v.weight";
      case K_O: return p + ".attn_output.weight";
      case K_QB: return p + ".attn_q.bias";
      case K_KB: return p + ".attn_k.bias";
      case K_VB: return p + ".attn_v.bias";
      case K_GATE: return p + ".ffn_gate.weight";
      case K_UP: return p + ".ffn_up.weight";
      case K_DOWN: return p + ".ffn_down.weight";
    }
    bad("no GGUF tensor for kind " + std::to_string(kind));
  }
};

bool is_dir(const char* p) {
  struct stat st;
  return ::stat(p, &st) == 0 && S_ISDIR(st.st_mode);
}

template <typename F>
int load_with(pgd_dev* dev, pgd_model** out, F&& fill) {
  pgd_model* held = nullptr;
  int rc = guard([&] {
    PGD_CHECK(dev && out, kErrArg, "null argument");
    DeviceScope scope(dev);
    held = new pgd_model();
    held->m.dev = dev;
    fill(held->m);
    *out = held;
  });
  if (rc && held) delete held;
  return rc;
}

}  // namespace

}  // namespace pgd

using namespace pgd;

extern "C" {

int pgd_model_load_mlx(pgd_dev* dev, const char* dir, int max_pos, int kv_blocks, pgd_model** out) {
  return load_with(dev, out, [&](Model& m) {
    PGD_CHECK(dir, kErrArg, "null path");
    std::vector<bool> full;
    m.cfg = mlx_config(dir, max_pos, kv_blocks, &full);
    validate_config(m.cfg, false);
    MlxSource src(dir, std::move(full));
    build_model(m, src);
  });
}

int pgd_model_load_gguf(pgd_dev* dev, const char* path, int max_pos, int kv_blocks, pgd_model** out) {
  return load_with(dev, out, [&](Model& m) {
    PGD_CHECK(path, kErrArg, "null path");
    GgufFile f(path);
    m.cfg = gguf_config(f, max_pos, kv_blocks);
    validate_config(m.cfg, false);
    GgufSource src(f);
    build_model(m, src);
  });
}

int pgd_checkpoint_config(const char* path, int max_pos, int kv_blocks, pgd_model_config* cfg) {
  return guard([&] {
    PGD_CHECK(path && cfg, kErrArg, "null argument");
    if (is_dir(path)) {
      std::vector<bool> full;
      *cfg = mlx_config(path, max_pos, kv_blocks, &full);
      // parse every shard header; the embedding must match the config
      SafetensorsStore st(path);
      const TensorView& e = st.at("language_model.model.embed_tokens.weight");
      if (e.shape.size() != 2 || e.shape[0] != (uint64_t)cfg->vocab || e.shape[1] * 4 != (uint64_t)cfg->hidden)
        throw Error{kErrFormat, "embed_tokens does not match vocab_size x hidden_size"};
    } else {
      GgufFile f(path);
      *cfg = gguf_config(f, max_pos, kv_blocks);
    }
    validate_config(*cfg, false);
  });
}

int pgd_model_config_get(const pgd_model* m, pgd_model_config* cfg) {
  return guard([&] {
    PGD_CHECK(m && cfg, kErrArg, "null argument");
    *cfg = m->m.cfg;
  });
}

}  // extern "C"
