// model.h — decode runtime: model weights on the device, paged KV pool,
// per-session recurrent state and the ragged step that drives every forward.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <set>
#include <utility>
#include <vector>

#include "../../include/pagoda_hip.h"
#include "device.h"
#include "ops.h"
#include "quant.h"

namespace pgd {

struct Layer {
  bool full = false;
  float* in_norm = nullptr;
  float* post_norm = nullptr;
  QMat gate, up, down;
  // hybrid model: the projections that read the normed input, stacked into
  // one matrix (rows [qkv | z | b | a] or [q | k | v]), one launch
  QMat proj;
  // gated-delta (linear attention) layer
  QMat qkv, z, a, b, out;
  float* conv = nullptr;
  float* a_log = nullptr;
  float* dt_bias = nullptr;
  float* gnorm = nullptr;
  int lin_index = -1;
  // full-attention layer
  QMat q, k, v, o;
  float* q_norm = nullptr;
  float* k_norm = nullptr;
  float* qb = nullptr;
  float* kb = nullptr;
  float* vb = nullptr;
  int full_index = -1;
  float* k_pool = nullptr;  // [kv_blocks][kv_heads][block][head_dim]
  float* v_pool = nullptr;
};

struct Session;

struct Model {
  pgd_dev* dev = nullptr;
  pgd_model_config cfg{};
  int conv_dim = 0, key_dim = 0, value_dim = 0, q_out = 0, kv_width = 0;
  int proj_lin = 0, proj_full = 0;  // stacked projection widths (hybrid model)
  QMat embed, head;
  bool tied = false;
  float* final_norm = nullptr;
  std::vector<Layer> layers;
  int n_lin = 0, n_full = 0;
  size_t conv_floats = 0, state_floats = 0;  // per linear layer
  size_t rec_floats = 0;                     // per session (all linear layers)
  std::vector<void*> allocs;                 // small device vectors, KV pools

  // KV page allocator (block ids shared by all full-attention layers)
  std::vector<int> free_blocks;
  std::vector<int> refcount;

  // host rope tables, grown on demand
  std::vector<float> cos_tab, sin_tab;
  int rope_rows = 0;

  // per-step workspace
  DevBuf ws;
  size_t ws_rows = 0;
  DevBuf meta_dev;
  size_t meta_cap = 0;
  void* meta_host = nullptr;  // pinned
  size_t meta_host_cap = 0;
  std::vector<int> plan_host, plan_seq, plan_pos, plan_bt;  // attention plan of the current step
  DevBuf out_dev;  // ids / values / non-finite counts
  size_t out_cap = 0;
  void* out_host = nullptr;
  size_t out_host_cap = 0;
  int live_sessions = 0;
  // arithmetic of the GGML-format (Qwen2) matrices: 1 = candle's CPU quantized
  // matmul (activations quantized to Q8_K / Q8_0), 0 = f32 dequant-then-dot
  int q8act = 0;
  // captured decode steps (pgd_model_set_graphs): one executable graph per
  // launch signature, the signatures seen once, replays so far
  struct Graph {
    hipGraphExec_t exec;
    uint64_t epoch;
  };
  bool use_graphs = false;
  std::map<std::vector<long long>, Graph> graphs;
  std::set<std::vector<long long>> graph_seen;
  long long graph_launches = 0;
  void drop_graphs();

  ~Model();
  void ensure_rope(int pos);
  int alloc_block();
  void release_block(int b);
  void copy_block(int dst, int src);
};

struct Session {
  Model* model = nullptr;
  int len = 0;
  std::vector<int> blocks;
  float* rec = nullptr;  // [n_lin][conv_floats + state_floats]
  std::vector<float> last_logits;
  bool has_logits = false;
  // a step failed after it began writing this session's state in place
  // (GDN state, KV pages): every later use is refused
  bool poisoned = false;
  ~Session();
};

// Tensor kinds: model-level (layer -1) and per-layer tensors. The synthetic
// generator keys its streams by (layer << 8) | kind.
enum TensorKind {
  K_EMBED = 1, K_HEAD = 2, K_FINAL_NORM = 3,
  K_IN_NORM = 10, K_POST_NORM = 11, K_GATE = 12, K_UP = 13, K_DOWN = 14,
  K_QKV = 20, K_Z = 21, K_A = 22, K_B = 23, K_OUT = 24, K_CONV = 25, K_ALOG = 26, K_DTB = 27, K_GNORM = 28,
  K_Q = 30, K_K = 31, K_V = 32, K_O = 33, K_QNORM = 34, K_KNORM = 35, K_QB = 36, K_KB = 37, K_VB = 38
};

// Where a model's tensors come from: seeded synthesis or a checkpoint.
struct WeightSource {
  virtual ~WeightSource() = default;
  virtual bool full_layer(int layer) const = 0;
  // lm_head shares the embedding matrix
  virtual bool tied_head() const = 0;
  // allocate q and fill it; fmt is the synthetic model's format, which a
  // checkpoint replaces by the stored one
  virtual void matrix(QMat& q, int fmt, int n_out, int n_in, int layer, int kind, hipStream_t s) = 0;
  // one matrix of row ranges taken from several tensors: parts = {kind, rows};
  // fmt as for matrix(). Returns false, allocating nothing, when the tensors
  // cannot share one matrix (a checkpoint storing them in different formats).
  virtual bool stacked(QMat& q, int fmt, int n_in, const std::vector<std::pair<int, int>>& parts, int layer,
                       hipStream_t s) = 0;
  // fill n device floats
  virtual void vec(float* dst, size_t n, int layer, int kind, hipStream_t s) = 0;
};

// Allocate and fill every tensor of m (m.dev and m.cfg set, cfg validated).
void build_model(Model& m, WeightSource& src);
// Checks of a configuration; synthetic models also need the layer pattern.
void validate_config(const pgd_model_config& c, bool synthetic);

// Output request of a step.
struct StepOut {
  // rows whose logits are computed: 0 = last row of each sequence, 1 = every row
  int all_rows = 0;
  int last_max = 0;           // argmax tie rule
  uint32_t* ids = nullptr;    // host [n_logit_rows]
  float* vals = nullptr;      // host [n_logit_rows] (max logit), nullable
  float* logits = nullptr;    // host [n_logit_rows][vocab], nullable
};

// One forward over a ragged batch: sequence i feeds n[i] tokens. On a
// validation error nothing is modified.
void step(Model& m, Session* const* sess, const uint32_t* toks, const int* n, int nseq, StepOut& out);

}  // namespace pgd

// the opaque handles of the C ABI
struct pgd_model {
  pgd::Model m;
};

struct pgd_session {
  pgd::Session s;
};
