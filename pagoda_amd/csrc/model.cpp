// model.cpp — decode runtime behind the pgd_model / pgd_session C ABI.
//
// One HIP stream per device handle; every call is serialized by the caller
// (the reference engine is single-threaded per instance, engine.rs:1404).
// A forward is one ragged step: token rows of all sequences go through the
// projections together; the causal conv, Gated-DeltaNet recurrence and
// attention run per sequence in token order (qwen3_5.rs:1193-1479,
// qwen2_gguf.rs:142-266, llama.rs:734-886).
#include "model.h"

#include <atomic>
#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <string>
#include <unordered_map>
#include <unordered_set>

#include "common.h"

namespace pgd {

namespace {

uint64_t tkey(int layer, int kind) { return ((uint64_t)(layer < 0 ? 0xFFFF : layer) << 8) | (uint64_t)kind; }

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

float* dev_floats(Model& m, size_t n) {
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(float));
  if (e != hipSuccess) throw Error{kErrAlloc, std::string("hipMalloc: ") + hipGetErrorString(e)};
  m.allocs.push_back(p);
  return (float*)p;
}

}  // namespace

void validate_config(const pgd_model_config& c, bool synthetic) {
  PGD_CHECK(c.arch == PGD_ARCH_QWEN35 || c.arch == PGD_ARCH_QWEN2, kErrArg, "unknown arch");
  PGD_CHECK(c.n_layers > 0 && c.hidden > 0 && c.intermediate > 0 && c.vocab > 0, kErrShape, "model dims");
  PGD_CHECK(c.heads > 0 && c.kv_heads > 0 && c.heads % c.kv_heads == 0, kErrShape, "heads / kv_heads");
  PGD_CHECK(c.head_dim == 64 || c.head_dim == 128 || c.head_dim == 256, kErrShape, "head_dim must be 64/128/256");
  PGD_CHECK(c.rotary_dim > 0 && c.rotary_dim % 2 == 0 && c.rotary_dim <= c.head_dim, kErrShape, "rotary_dim");
  PGD_CHECK(c.kv_block > 0 && c.kv_blocks > 0, kErrShape, "kv pool");
  PGD_CHECK(c.max_pos > 0, kErrShape, "max_pos");
  int kmul = c.arch == PGD_ARCH_QWEN35 ? 64 : 32;
  PGD_CHECK(c.hidden % kmul == 0 && c.intermediate % kmul == 0 && (c.heads * c.head_dim) % kmul == 0, kErrShape,
            "GEMV input widths must be multiples of the quant group");
  if (c.arch == PGD_ARCH_QWEN35) {
    PGD_CHECK(!synthetic || c.full_every >= 1, kErrShape, "full_every");
    PGD_CHECK(c.k_dim == 128 && c.v_dim == 128, kErrShape, "gated delta needs k_dim == v_dim == 128");
    PGD_CHECK(c.k_heads > 0 && c.v_heads % c.k_heads == 0, kErrShape, "v_heads % k_heads");
    PGD_CHECK(c.conv_kernel >= 2 && c.conv_kernel <= 8, kErrShape, "conv kernel");
  }
}

// ---------------------------------------------------------------------------
void Model::drop_graphs() {
  for (auto& g : graphs) (void)hipGraphExecDestroy(g.second.exec);
  graphs.clear();
}

Model::~Model() {
  drop_graphs();
  if (dev) {
    DeviceScope scope(dev);
    (void)hipStreamSynchronize(dev->stream);
    qmat_free(embed);
    if (!tied) qmat_free(head);
    for (auto& L : layers) {
      for (QMat* q : {&L.gate, &L.up, &L.down, &L.proj, &L.qkv, &L.z, &L.a, &L.b, &L.out, &L.q, &L.k, &L.v, &L.o})
        qmat_free(*q);
    }
    for (void* p : allocs) (void)hipFree(p);
    if (meta_host) (void)hipHostFree(meta_host);
    if (out_host) (void)hipHostFree(out_host);
    ws.reset();
    meta_dev.reset();
    out_dev.reset();
  }
}

void Model::ensure_rope(int pos) {
  // pagoda-hf/src/qwen3_5.rs:1855-1870 (rope_cos_sin); equal to the Qwen2
  // tables of qwen2_gguf.rs:327-344 when rotary_dim == head_dim.
  const int rd = cfg.rotary_dim, half = rd / 2;
  if (pos < rope_rows) return;
  int rows = std::max(pos + 1, std::max(2 * rope_rows, 256));
  rows = std::min(rows, std::max(cfg.max_pos, pos + 1));
  cos_tab.resize((size_t)rows * rd);
  sin_tab.resize((size_t)rows * rd);
  std::vector<float> freq(half);
  for (int i = 0; i < half; ++i) freq[i] = 1.0f / powf(cfg.rope_theta, (float)(2 * i) / (float)rd);
  for (int p = rope_rows; p < rows; ++p) {
    for (int i = 0; i < half; ++i) {
      float ang = (float)p * freq[i];
      float c = cosf(ang), s = sinf(ang);
      cos_tab[(size_t)p * rd + i] = c;
      cos_tab[(size_t)p * rd + half + i] = c;
      sin_tab[(size_t)p * rd + i] = s;
      sin_tab[(size_t)p * rd + half + i] = s;
    }
  }
  rope_rows = rows;
}

int Model::alloc_block() {
  PGD_CHECK(!free_blocks.empty(), kErrAlloc, "KV page pool exhausted");
  int b = free_blocks.back();
  free_blocks.pop_back();
  refcount[b] = 1;
  return b;
}

void Model::release_block(int b) {
  if (--refcount[b] == 0) free_blocks.push_back(b);
}

void Model::copy_block(int dst, int src) {
  size_t per = (size_t)cfg.kv_heads * cfg.kv_block * cfg.head_dim;
  for (auto& L : layers) {
    if (!L.full) continue;
    PGD_HIP(hipMemcpyAsync(L.k_pool + (size_t)dst * per, L.k_pool + (size_t)src * per, per * 4,
                           hipMemcpyDeviceToDevice, dev->stream));
    PGD_HIP(hipMemcpyAsync(L.v_pool + (size_t)dst * per, L.v_pool + (size_t)src * per, per * 4,
                           hipMemcpyDeviceToDevice, dev->stream));
  }
}

Session::~Session() {
  if (!model) return;
  for (int b : blocks) model->release_block(b);
  if (rec) {
    DeviceScope scope(model->dev);
    (void)hipStreamSynchronize(model->dev->stream);
    (void)hipFree(rec);
  }
  model->live_sessions--;
}

// ---------------------------------------------------------------------------
// model build (from any weight source) and the synthetic source
// ---------------------------------------------------------------------------
void build_model(Model& m, WeightSource& src) {
  // GGUF (Qwen2) models default to the reference CPU path's arithmetic
  m.q8act = m.cfg.arch == PGD_ARCH_QWEN2 ? 1 : 0;
  const pgd_model_config& c = m.cfg;
  hipStream_t s = m.dev->stream;
  const int H = c.hidden;
  m.kv_width = c.kv_heads * c.head_dim;
  auto vec = [&](size_t n, int li, int kind) {
    float* p = dev_floats(m, n);
    src.vec(p, n, li, kind, s);
    return p;
  };
  if (c.arch == PGD_ARCH_QWEN35) {
    m.key_dim = c.k_heads * c.k_dim;
    m.value_dim = c.v_heads * c.v_dim;
    m.conv_dim = 2 * m.key_dim + m.value_dim;
    m.q_out = c.heads * c.head_dim * 2;
    m.proj_lin = m.conv_dim + m.value_dim + 2 * c.v_heads;
    m.proj_full = m.q_out + 2 * m.kv_width;
    src.matrix(m.embed, FMT_A8, c.vocab, H, -1, K_EMBED, s);
  } else {
    m.q_out = c.heads * c.head_dim;
    m.proj_full = m.q_out + 2 * m.kv_width;  // q | k | v outputs side by side
    src.matrix(m.embed, FMT_Q6K, c.vocab, H, -1, K_EMBED, s);
  }
  if (src.tied_head()) {
    m.head = m.embed;  // tied lm_head (qwen2_gguf.rs:96-99)
    m.tied = true;
  } else {
    src.matrix(m.head, m.embed.fmt, c.vocab, H, -1, K_HEAD, s);
  }
  m.final_norm = vec(H, -1, K_FINAL_NORM);
  m.layers.resize(c.n_layers);
  size_t kv_per_layer = (size_t)c.kv_blocks * c.kv_heads * c.kv_block * c.head_dim;
  for (int i = 0; i < c.n_layers; ++i) {
    Layer& L = m.layers[i];
    L.in_norm = vec(H, i, K_IN_NORM);
    L.post_norm = vec(H, i, K_POST_NORM);
    if (c.arch == PGD_ARCH_QWEN35) {
      L.full = src.full_layer(i);
      src.matrix(L.gate, FMT_A8, c.intermediate, H, i, K_GATE, s);
      src.matrix(L.up, FMT_A8, c.intermediate, H, i, K_UP, s);
      src.matrix(L.down, FMT_A8, H, c.intermediate, i, K_DOWN, s);
      if (!L.full) {
        L.lin_index = m.n_lin++;
        // [qkv | z | b | a] stacked, one launch
        PGD_CHECK(src.stacked(L.proj, FMT_A8, H,
                              {{K_QKV, m.conv_dim}, {K_Z, m.value_dim}, {K_B, c.v_heads}, {K_A, c.v_heads}}, i, s),
                  kErrFormat, "GDN projections must share one format");
        src.matrix(L.out, FMT_A8, H, m.value_dim, i, K_OUT, s);
        L.conv = vec((size_t)m.conv_dim * c.conv_kernel, i, K_CONV);
        L.a_log = vec(c.v_heads, i, K_ALOG);
        L.dt_bias = vec(c.v_heads, i, K_DTB);
        L.gnorm = vec(c.v_dim, i, K_GNORM);
      } else {
        L.full_index = m.n_full++;
        PGD_CHECK(src.stacked(L.proj, FMT_A8, H, {{K_Q, m.q_out}, {K_K, m.kv_width}, {K_V, m.kv_width}}, i, s),
                  kErrFormat, "attention projections must share one format");
        src.matrix(L.o, FMT_A8, H, c.heads * c.head_dim, i, K_O, s);
        L.q_norm = vec(c.head_dim, i, K_QNORM);
        L.k_norm = vec(c.head_dim, i, K_KNORM);
      }
    } else {
      L.full = true;
      L.full_index = m.n_full++;
      // q and k in one matrix (one launch) when they share a format
      if (!src.stacked(L.proj, FMT_Q4K, H, {{K_Q, m.q_out}, {K_K, m.kv_width}}, i, s)) {
        src.matrix(L.q, FMT_Q4K, m.q_out, H, i, K_Q, s);
        src.matrix(L.k, FMT_Q4K, m.kv_width, H, i, K_K, s);
      }
      src.matrix(L.v, FMT_Q6K, m.kv_width, H, i, K_V, s);
      src.matrix(L.o, FMT_Q4K, H, c.heads * c.head_dim, i, K_O, s);
      src.matrix(L.gate, FMT_Q4K, c.intermediate, H, i, K_GATE, s);
      src.matrix(L.up, FMT_Q4K, c.intermediate, H, i, K_UP, s);
      src.matrix(L.down, i % 2 == 0 ? FMT_Q6K : FMT_Q4K, H, c.intermediate, i, K_DOWN, s);
      L.qb = vec(m.q_out, i, K_QB);
      L.kb = vec(m.kv_width, i, K_KB);
      L.vb = vec(m.kv_width, i, K_VB);
    }
    if (L.full) {
      L.k_pool = dev_floats(m, kv_per_layer);
      L.v_pool = dev_floats(m, kv_per_layer);
    }
  }
  if (c.arch == PGD_ARCH_QWEN35) {
    m.conv_floats = (size_t)m.conv_dim * (c.conv_kernel - 1);
    m.conv_floats = align_up(m.conv_floats, 64);
    m.state_floats = (size_t)c.v_heads * c.k_dim * c.v_dim;
    m.rec_floats = (size_t)m.n_lin * (m.conv_floats + m.state_floats);
  }
  m.refcount.assign(c.kv_blocks, 0);
  m.free_blocks.resize(c.kv_blocks);
  for (int b = 0; b < c.kv_blocks; ++b) m.free_blocks[b] = c.kv_blocks - 1 - b;
  PGD_HIP(hipStreamSynchronize(s));
}

namespace {

// Seeded synthetic weights, generated on the device: matrices N(0, 0.02)
// quantized in their format, norms 1, conv N(0, 0.2), A_log ln(16) U(0,1),
// dt_bias N(0, 0.1), q/k/v biases N(0, 0.02).
class SynthSource : public WeightSource {
 public:
  SynthSource(const pgd_model_config& c, uint64_t seed) : c_(c), seed_(seed) {}
  bool full_layer(int i) const override { return (i % c_.full_every) == c_.full_every - 1; }
  bool tied_head() const override { return c_.arch == PGD_ARCH_QWEN2; }
  void matrix(QMat& q, int fmt, int n_out, int n_in, int li, int kind, hipStream_t s) override {
    qmat_alloc(q, fmt, n_out, n_in, s);
    qmat_synth(q, seed_, tkey(li, kind), 0.02f, s);
  }
  bool stacked(QMat& q, int fmt, int n_in, const std::vector<std::pair<int, int>>& parts, int li,
               hipStream_t s) override {
    int n = 0;
    for (auto& p : parts) n += p.second;
    qmat_alloc(q, fmt, n, n_in, s);
    int r = 0;
    for (auto& p : parts) {  // each range keeps its own tensor key
      qmat_synth_rows(q, r, p.second, seed_, tkey(li, p.first), 0.02f, s);
      r += p.second;
    }
    return true;
  }
  void vec(float* p, size_t n, int li, int kind, hipStream_t s) override {
    switch (kind) {
      case K_CONV: synth_normal_f32(p, n, seed_, tkey(li, kind), 0.2f, s); break;
      case K_ALOG: synth_uniform_f32(p, n, seed_, tkey(li, kind), 2.7725887f, s); break;
      case K_DTB: synth_normal_f32(p, n, seed_, tkey(li, kind), 0.1f, s); break;
      case K_QB:
      case K_KB:
      case K_VB: synth_normal_f32(p, n, seed_, tkey(li, kind), 0.02f, s); break;
      default: fill_f32(p, n, 1.0f, s);  // norm weights
    }
  }

 private:
  pgd_model_config c_;
  uint64_t seed_;
};

}  // namespace

// ---------------------------------------------------------------------------
// ragged step
// ---------------------------------------------------------------------------
namespace {

struct Ws {
  float *x, *xn, *A, *B, *C0, *C1, *D, *E, *F, *G, *logits;
  void* act;   // prepared A8 activation operands
  void* act2;  // second set: the SwiGLU product feeding the down projection
  void* act3;  // third set: the post-mixer norm's input, written by the mixer's
               // output projection while it reads act
  size_t lda, ldb, ldd, lde;
};

Ws carve_ws(Model& m, int rows, int lrows) {
  const pgd_model_config& c = m.cfg;
  size_t H = c.hidden;
  size_t lda = std::max<size_t>(std::max<size_t>(m.conv_dim, m.q_out), std::max(m.proj_lin, m.proj_full));
  size_t ldb = std::max<size_t>(m.value_dim, m.kv_width);
  size_t ldc = std::max<size_t>(align_up(std::max(c.v_heads, 1), 8), m.kv_width);
  size_t ldd = std::max<size_t>(m.conv_dim, (size_t)c.heads * c.head_dim);
  size_t lde = std::max<size_t>(m.value_dim, (size_t)c.heads * c.head_dim);
  size_t act_floats = 0, act2_floats = 0, act3_floats = 0;
  if (c.arch == PGD_ARCH_QWEN35) {
    int kmax = std::max(std::max(c.hidden, c.intermediate), std::max(m.value_dim, c.heads * c.head_dim));
    act_floats = (a8_act_bytes(rows, kmax) + 3) / 4;
    act2_floats = (a8_act_bytes(rows, c.intermediate) + 3) / 4;
    act3_floats = (a8_act_bytes(rows, c.hidden) + 3) / 4;
  }
  size_t sizes[] = {rows * H, rows * H, rows * lda, rows * ldb, rows * ldc, rows * ldc, rows * ldd, rows * lde,
                    rows * (size_t)c.heads * c.head_dim, rows * (size_t)c.intermediate, (size_t)lrows * c.vocab,
                    act_floats, act2_floats, act3_floats};
  size_t total = 0;
  for (size_t v : sizes) total += align_up(v, 64);
  if (m.ws.bytes < total * 4) {
    PGD_HIP(hipStreamSynchronize(m.dev->stream));
    m.ws = DevBuf(total * 4);
  }
  float* p = m.ws.as<float>();
  float* ptrs[14];
  for (int i = 0; i < 14; ++i) {
    ptrs[i] = p;
    p += align_up(sizes[i], 64);
  }
  Ws w{ptrs[0], ptrs[1], ptrs[2], ptrs[3], ptrs[4], ptrs[5], ptrs[6], ptrs[7], ptrs[8], ptrs[9], ptrs[10],
       (void*)ptrs[11], (void*)ptrs[12], (void*)ptrs[13], lda, ldb, ldd, lde};
  return w;
}

}  // namespace

// Replays the captured graph of a step whose launches are keyed by `key`;
// the first step with a key runs eagerly (it sizes every scratch buffer),
// the second is captured and replayed. A capture that fails (a buffer grew
// during it) is dropped and the step runs eagerly: nothing executes while a
// stream is being captured.
void run_graphed(Model& m, const std::vector<long long>& key, const std::function<void()>& forward) {
  hipStream_t st = m.dev->stream;
  const uint64_t epoch = gemv::scratch_epoch();
  auto it = m.graphs.find(key);
  if (it != m.graphs.end() && it->second.epoch == epoch) {
    PGD_HIP(hipGraphLaunch(it->second.exec, st));
    m.graph_launches++;
    return;
  }
  if (it != m.graphs.end()) {
    (void)hipGraphExecDestroy(it->second.exec);
    m.graphs.erase(it);
  }
  if (!m.graph_seen.insert(key).second || m.graph_seen.size() > 4096) {
    if (m.graph_seen.size() > 4096) m.graph_seen.clear();
    if (m.graphs.size() >= 64) m.drop_graphs();
    hipGraph_t g = nullptr;
    PGD_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    bool ok = true;
    try {
      forward();
    } catch (...) {
      ok = false;
    }
    hipError_t e = hipStreamEndCapture(st, &g);
    ok = ok && e == hipSuccess && g && gemv::scratch_epoch() == epoch;
    hipGraphExec_t ex = nullptr;
    if (ok) ok = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0) == hipSuccess;
    if (g) (void)hipGraphDestroy(g);
    (void)hipGetLastError();  // a failed capture's error is not this step's
    if (ok) {
      m.graphs[key] = {ex, epoch};
      PGD_HIP(hipGraphLaunch(ex, st));
      m.graph_launches++;
      return;
    }
    if (ex) (void)hipGraphExecDestroy(ex);
  }
  forward();
}

void step(Model& m, Session* const* sess, const uint32_t* toks, const int* n, int nseq, StepOut& out) {
  const pgd_model_config& c = m.cfg;
  hipStream_t st = m.dev->stream;
  PGD_CHECK(nseq > 0 && sess && toks && n, kErrArg, "empty step");
  // ---- validation (nothing is modified before this block passes) ----
  int rows = 0;
  {
    std::unordered_set<const Session*> seen;
    for (int i = 0; i < nseq; ++i) {
      PGD_CHECK(sess[i] && sess[i]->model == &m, kErrArg, "session does not belong to this model");
      PGD_CHECK(seen.insert(sess[i]).second, kErrArg, "a session appears twice in one step");
      PGD_CHECK(!sess[i]->poisoned, kErrState, "session state is undefined after a failed step");
      PGD_CHECK(n[i] >= 1, kErrArg, "every session must feed at least one token");
      PGD_CHECK((long long)sess[i]->len + n[i] <= c.max_pos, kErrShape,
                "context " + std::to_string(sess[i]->len) + " + " + std::to_string(n[i]) + " exceeds max_pos");
      rows += n[i];
    }
    for (int r = 0; r < rows; ++r)
      PGD_CHECK(toks[r] < (uint32_t)c.vocab, kErrArg, "token " + std::to_string(toks[r]) + " out of vocab");
  }
  const int lrows = out.all_rows ? rows : nseq;
  // From here on the step writes session state in place (KV pages, the GDN
  // recurrent and conv state). A device error past this point leaves that
  // state half-advanced, so the sessions are marked unusable instead of
  // silently continuing from it (a batched step commits all or nothing,
  // pagoda-hf/src/llama.rs:750-778).
  // Armed just before the first kernel that writes session state, so that a
  // capacity or allocation error before it (page pool, rope tables,
  // workspace, metadata buffers) leaves every session usable.
  struct PoisonOnThrow {
    Session* const* s;
    int n;
    bool armed = false;
    ~PoisonOnThrow() {
      if (armed)
        for (int i = 0; i < n; ++i) s[i]->poisoned = true;
    }
  } poison{sess, nseq};
  // GEMVs of f32 activations (the Qwen2 path) in the model's arithmetic
  auto gemv = [&](const QMat& q, const float* x, int ldx, int nr, float* y, int ldy, const float* res, int ldres) {
    if (m.q8act && q.fmt != FMT_A8) qmat_gemv_q8act(q, x, ldx, nr, y, ldy, res, ldres, st);
    else qmat_gemv(q, x, 0, ldx, nr, y, ldy, res, ldres, st);
  };
  // ---- KV pages: count, then allocate (copy-on-write for a shared tail) ----
  if (m.n_full > 0) {
    size_t need = 0;
    for (int i = 0; i < nseq; ++i) {
      const Session* s = sess[i];
      size_t want = (size_t)(s->len + n[i] + c.kv_block - 1) / c.kv_block;
      // a step that failed after this allocation may have left pages past len
      if (want > s->blocks.size()) need += want - s->blocks.size();
      // the partly filled page holding position len, when another holder shares it
      if (s->len % c.kv_block && m.refcount[s->blocks[s->len / c.kv_block]] > 1) need += 1;
    }
    PGD_CHECK(need <= m.free_blocks.size(), kErrAlloc, "KV page pool exhausted");
    for (int i = 0; i < nseq; ++i) {
      Session* s = sess[i];
      if (s->len % c.kv_block) {
        int& tail = s->blocks[s->len / c.kv_block];
        if (m.refcount[tail] > 1) {
          int nb = m.alloc_block();
          m.copy_block(nb, tail);
          m.release_block(tail);
          tail = nb;
        }
      }
      size_t want = (size_t)(s->len + n[i] + c.kv_block - 1) / c.kv_block;
      while (s->blocks.size() < want) s->blocks.push_back(m.alloc_block());
    }
  }
  int max_pos = 0, max_n = 0;
  size_t max_blocks = 1;
  for (int i = 0; i < nseq; ++i) max_n = std::max(max_n, n[i]);
  for (int i = 0; i < nseq; ++i) {
    max_pos = std::max(max_pos, sess[i]->len + n[i] - 1);
    max_blocks = std::max(max_blocks, sess[i]->blocks.size());
  }
  // block-table stride rounded up to 16 pages: it is a launch argument, and a
  // captured step stays valid while contexts grow by up to 256 positions
  max_blocks = align_up(max_blocks, 16);
  m.ensure_rope(max_pos);
  const int rd = c.rotary_dim;
  // ---- attention plan (same for every full-attention layer) ----
  std::vector<int>& plan = m.plan_host;
  {
    std::vector<int>& p_seq = m.plan_seq;
    std::vector<int>& p_pos = m.plan_pos;
    std::vector<int>& p_bt = m.plan_bt;
    p_seq.resize(rows);
    p_pos.resize(rows);
    p_bt.assign((size_t)nseq * max_blocks, 0);
    int r = 0;
    for (int i = 0; i < nseq; ++i) {
      const Session* ss = sess[i];
      for (size_t b = 0; b < ss->blocks.size(); ++b) p_bt[i * max_blocks + b] = ss->blocks[b];
      for (int t = 0; t < n[i]; ++t, ++r) {
        p_seq[r] = i;
        p_pos[r] = ss->len + t;
      }
    }
    build_attn_plan(p_seq.data(), p_pos.data(), rows, p_bt.data(), (int)max_blocks, c.kv_block, c.heads / c.kv_heads,
                    c.head_dim, plan);
  }
  // ---- host metadata, one upload ----
  size_t off_seq = 0;
  size_t off_pos = align_up(off_seq + rows * 4, 256);
  size_t off_rs = align_up(off_pos + rows * 4, 256);
  size_t off_rc = align_up(off_rs + nseq * 4, 256);
  size_t off_bt = align_up(off_rc + nseq * 4, 256);
  size_t off_lr = align_up(off_bt + nseq * max_blocks * 4, 256);
  size_t off_tok = align_up(off_lr + lrows * 4, 256);
  size_t off_sb = align_up(off_tok + rows * 4, 256);
  size_t off_cos = align_up(off_sb + nseq * 8, 256);
  size_t off_sin = align_up(off_cos + (size_t)rows * rd * 4, 256);
  size_t off_plan = align_up(off_sin + (size_t)rows * rd * 4, 256);
  size_t meta_bytes = align_up(off_plan + plan.size() * 4, 256);
  if (m.meta_host_cap < meta_bytes) {
    if (m.meta_host) {
      PGD_HIP(hipStreamSynchronize(st));
      PGD_HIP(hipHostFree(m.meta_host));
      m.meta_host = nullptr;
    }
    PGD_HIP(hipHostMalloc(&m.meta_host, meta_bytes * 2));
    m.meta_host_cap = meta_bytes * 2;
  }
  if (m.meta_dev.bytes < meta_bytes) {
    PGD_HIP(hipStreamSynchronize(st));
    m.meta_dev = DevBuf(meta_bytes * 2);
  }
  PGD_HIP(hipStreamSynchronize(st));  // host staging buffer reuse
  uint8_t* hb = (uint8_t*)m.meta_host;
  int* h_seq = (int*)(hb + off_seq);
  int* h_pos = (int*)(hb + off_pos);
  int* h_rs = (int*)(hb + off_rs);
  int* h_rc = (int*)(hb + off_rc);
  int* h_bt = (int*)(hb + off_bt);
  int* h_lr = (int*)(hb + off_lr);
  uint32_t* h_tok = (uint32_t*)(hb + off_tok);
  float** h_sb = (float**)(hb + off_sb);
  float* h_cos = (float*)(hb + off_cos);
  float* h_sin = (float*)(hb + off_sin);
  memcpy(hb + off_plan, plan.data(), plan.size() * 4);
  {
    int r = 0, lr = 0;
    for (int i = 0; i < nseq; ++i) {
      Session* s = sess[i];
      h_rs[i] = r;
      h_rc[i] = n[i];
      h_sb[i] = s->rec;
      for (size_t b = 0; b < max_blocks; ++b) h_bt[i * max_blocks + b] = b < s->blocks.size() ? s->blocks[b] : 0;
      for (int t = 0; t < n[i]; ++t, ++r) {
        h_seq[r] = i;
        h_pos[r] = s->len + t;
        h_tok[r] = toks[r];
        memcpy(h_cos + (size_t)r * rd, m.cos_tab.data() + (size_t)(s->len + t) * rd, rd * 4);
        memcpy(h_sin + (size_t)r * rd, m.sin_tab.data() + (size_t)(s->len + t) * rd, rd * 4);
        if (out.all_rows) h_lr[lr++] = r;
      }
      if (!out.all_rows) h_lr[lr++] = r - 1;
    }
  }
  PGD_HIP(hipMemcpyAsync(m.meta_dev.p, m.meta_host, meta_bytes, hipMemcpyHostToDevice, st));
  uint8_t* db = (uint8_t*)m.meta_dev.p;
  const int* d_seq = (const int*)(db + off_seq);
  const int* d_pos = (const int*)(db + off_pos);
  SeqMeta sm{(const int*)(db + off_rs), (const int*)(db + off_rc)};
  const int* d_lr = (const int*)(db + off_lr);
  const uint32_t* d_tok = (const uint32_t*)(db + off_tok);
  float* const* d_sb = (float* const*)(db + off_sb);
  RowMeta rm{d_seq, d_pos, (const int*)(db + off_bt), (int)max_blocks, (const float*)(db + off_cos),
             (const float*)(db + off_sin)};
  const AttnPlan ap = attn_plan_view(plan.data(), (const int*)(db + off_plan));

  // ---- forward ----
  Ws w = carve_ws(m, rows, lrows);
  const int H = c.hidden;
  const int norm_mode = c.arch == PGD_ARCH_QWEN35 ? 0 : m.q8act ? 2 : 1;
  const float eps = c.arch == PGD_ARCH_QWEN35 ? 1e-6f : c.eps;
  // step outputs: ids, max values, non-finite counts
  size_t out_bytes = (size_t)lrows * 12;
  if (m.out_dev.bytes < out_bytes) {
    PGD_HIP(hipStreamSynchronize(st));
    m.out_dev = DevBuf(out_bytes * 2);
  }
  if (m.out_host_cap < out_bytes) {
    PGD_HIP(hipStreamSynchronize(st));
    if (m.out_host) PGD_HIP(hipHostFree(m.out_host));
    m.out_host = nullptr;
    m.out_host_cap = 0;
    PGD_HIP(hipHostMalloc(&m.out_host, out_bytes * 2));
    m.out_host_cap = out_bytes * 2;
  }
  uint32_t* d_ids = m.out_dev.as<uint32_t>();
  float* d_vals = (float*)(d_ids + lrows);
  int* d_nf = (int*)(d_vals + lrows);
  // every launch of the forward, from the embedding rows to the argmax; the
  // same launches with the same arguments whenever graph_key() is the same
  auto forward = [&]() {
    qmat_embed(m.embed, d_tok, rows, w.x, H, st);
    const size_t per_lin = m.conv_floats + m.state_floats;
    const bool hybrid = c.arch == PGD_ARCH_QWEN35;
    // the next input norm's deferred input, when the last residual GEMV wrote it
    A8Act next_in;
    bool have_next_in = false;
    for (size_t li = 0; li < m.layers.size(); ++li) {
      auto& L = m.layers[li];
      A8Act post_in;  // the post-mixer norm's deferred input
      bool conv_done = false;  // the projection GEMV ran the causal conv
      // ---- projections of the normed input ----
      const float *q_raw = nullptr, *k_raw = nullptr, *v_raw = nullptr;
      int ld_q = 0, ld_kv = 0;
      if (hybrid) {
        // the input norm's deferred operands: written by the previous layer's down
        // projection, or prepared here for the first layer; one GEMV for all projections
        A8Act act = have_next_in ? next_in : a8_gnorm_prep(w.x, H, rows, H, L.in_norm, eps, w.act, st);
        // one token per sequence: the GEMV's epilogue (1..4 rows, and the
        // per-wave kernels) or its range reduction also runs the causal conv,
        // row r on sequence r's state
        conv_done = !L.full && rows == nseq;
        if (conv_done)
          qmat_gemv_a8_conv(L.proj, act, w.A, (int)w.lda, L.conv, d_sb, (size_t)L.lin_index * per_lin, m.conv_dim,
                            c.conv_kernel, w.D, (int)w.ldd, st);
        else
          qmat_gemv_a8(L.proj, act, w.A, (int)w.lda, nullptr, 0, st);
        if (L.full) {
          q_raw = w.A;
          k_raw = w.A + m.q_out;
          v_raw = w.A + m.q_out + m.kv_width;
          ld_q = ld_kv = (int)w.lda;
        }
      } else {
        rmsnorm_rows(w.x, H, nullptr, rows, H, L.in_norm, eps, norm_mode, w.xn, H, st);
        // q | k | v side by side in A (q and k from one stacked launch when they share a format)
        float* yv = w.A + m.q_out + m.kv_width;
        if (L.proj.base && m.q8act && qmat_q8act_pairable(L.proj, L.v)) {
          // stacked q|k and v in one launch (one activation quantization)
          qmat_gemv_q8act_pair(L.proj, w.A, L.v, yv, w.xn, H, rows, (int)w.lda, st);
        } else {
          if (L.proj.base) {
            gemv(L.proj, w.xn, H, rows, w.A, (int)w.lda, nullptr, 0);
          } else {
            gemv(L.q, w.xn, H, rows, w.A, (int)w.lda, nullptr, 0);
            gemv(L.k, w.xn, H, rows, w.A + m.q_out, (int)w.lda, nullptr, 0);
          }
          gemv(L.v, w.xn, H, rows, yv, (int)w.lda, nullptr, 0);
        }
        q_raw = w.A;
        k_raw = w.A + m.q_out;
        v_raw = w.A + m.q_out + m.kv_width;
        ld_q = ld_kv = (int)w.lda;
      }
      if (!L.full) {
        // stacked rows: [qkv (conv_dim) | z (value_dim) | b (v_heads) | a (v_heads)]
        const float* P = w.A;
        const int ldp = (int)w.lda;
        if (!conv_done)
          conv_step(P, ldp, w.D, (int)w.ldd, m.conv_dim, c.conv_kernel, L.conv, d_sb, (size_t)L.lin_index * per_lin,
                    sm, nseq, max_n, st);
        GdnParams gp{};
        gp.k_heads = c.k_heads;
        gp.v_heads = c.v_heads;
        gp.k_dim = c.k_dim;
        gp.v_dim = c.v_dim;
        gp.conv_out = w.D;
        gp.ld_conv = (int)w.ldd;
        gp.z = P + m.conv_dim;
        gp.ld_z = ldp;
        gp.b = P + m.conv_dim + m.value_dim;
        gp.a = P + m.conv_dim + m.value_dim + c.v_heads;
        gp.ld_ab = ldp;
        gp.a_log = L.a_log;
        gp.dt_bias = L.dt_bias;
        gp.norm = L.gnorm;
        // the gated norm writes the out projection's operands itself
        const A8Act act = a8_act_view(w.act, rows, m.value_dim);
        gp.out = nullptr;
        gp.act = a8_act_dst(act);
        gp.state_base = d_sb;
        gp.state_off = (size_t)L.lin_index * per_lin + m.conv_floats;
        gdn_step(gp, sm, nseq, rows, max_n, st);
        // the residual GEMV also writes the post-mixer norm's input (act3)
        post_in = qmat_gemv_a8_res_norm(L.out, act, w.x, H, L.post_norm, eps, w.act3, st);
      } else {
        AttnLayout al{c.heads, c.kv_heads, c.head_dim, c.rotary_dim, c.kv_block, L.k_pool, L.v_pool};
        QkvPrep qp{};
        qp.variant = hybrid ? 0 : 1;
        qp.q_raw = q_raw;
        qp.ld_q = ld_q;
        qp.k_raw = k_raw;
        qp.v_raw = v_raw;
        qp.ld_kv = ld_kv;
        qp.q_norm = L.q_norm;
        qp.k_norm = L.k_norm;
        qp.q_bias = L.qb;
        qp.k_bias = L.kb;
        qp.v_bias = L.vb;
        qp.q = w.D;
        qp.gate = w.F;
        qkv_prep(qp, al, rm, rows, st);
        if (hybrid) {
          // attention writes the o projection's operands itself
          const A8Act act = a8_act_view(w.act, rows, c.heads * c.head_dim);
          const a8act::Dst dst = a8_act_dst(act);
          attn_decode(w.D, w.F, nullptr, al, rm, ap, rows, st, &dst);
          post_in = qmat_gemv_a8_res_norm(L.o, act, w.x, H, L.post_norm, eps, w.act3, st);
        } else {
          // candle's CPU arithmetic: attention in the CPU path's order too, so
          // the whole forward is bit-equal to the reference restatement (its
          // LDS holds the block tables' capacity, a launch argument that
          // changes only with max_blocks)
          if (m.q8act) attn_exact(w.D, w.E, al, rm, rows, (int)max_blocks * c.kv_block, st);
          else attn_decode(w.D, nullptr, w.E, al, rm, ap, rows, st);
          gemv(L.o, w.E, c.heads * c.head_dim, rows, w.x, H, w.x, H);
        }
      }
      // ---- SwiGLU MLP ----
      if (hybrid) {
        const A8Act act = post_in;
        // the SwiGLU epilogue writes the down projection's operands itself
        const A8Act mid = a8_act_view(w.act2, rows, c.intermediate);
        qmat_gemv_a8_swiglu(L.gate, L.up, act, nullptr, 0, st, &mid);
        // the residual GEMV also writes the next layer's input norm (act)
        if (li + 1 < m.layers.size()) {
          next_in = qmat_gemv_a8_res_norm(L.down, mid, w.x, H, m.layers[li + 1].in_norm, eps, w.act, st);
          have_next_in = true;
        } else {
          qmat_gemv_a8(L.down, mid, w.x, H, w.x, H, st);
        }
      } else {
        rmsnorm_rows(w.x, H, nullptr, rows, H, L.post_norm, eps, norm_mode, w.xn, H, st);
        if (m.q8act) qmat_gemv_swiglu_q8act(L.gate, L.up, w.xn, H, rows, w.G, c.intermediate, st);
        else qmat_gemv_swiglu(L.gate, L.up, w.xn, H, rows, w.G, c.intermediate, st);
        gemv(L.down, w.G, c.intermediate, rows, w.x, H, w.x, H);
      }
    }
    // ---- head ----
    if (hybrid) {
      A8Act act = a8_norm_prep(w.x, H, d_lr, lrows, H, m.final_norm, eps, nullptr, 0, w.act, st);
      qmat_gemv_a8(m.head, act, w.logits, c.vocab, nullptr, 0, st);
    } else {
      rmsnorm_rows(w.x, H, d_lr, lrows, H, m.final_norm, eps, norm_mode, w.xn, H, st);
      gemv(m.head, w.xn, H, lrows, w.logits, c.vocab, nullptr, 0);
    }
    argmax_rows(w.logits, c.vocab, lrows, c.vocab, out.last_max, d_ids, d_vals, d_nf, st);
  };
  poison.armed = true;
  if (m.use_graphs) {
    // Everything a launch argument depends on besides the model: shapes,
    // workspace / metadata / output buffers, the attention plan's header and
    // section offsets (its page list comes last, so it may grow), and the
    // scratch buffers' allocation epoch.
    std::vector<long long> key = {rows, nseq, lrows, out.all_rows, out.last_max, max_n, (long long)max_blocks,
                                  (long long)(uintptr_t)m.ws.p, (long long)m.ws.bytes,
                                  (long long)(uintptr_t)m.meta_dev.p, (long long)(uintptr_t)m.out_dev.p, m.q8act};
    for (int i = 0; i < 8; ++i) key.push_back(plan[i]);
    run_graphed(m, key, forward);
  } else {
    forward();
  }
  PGD_HIP(hipMemcpyAsync(m.out_host, m.out_dev.p, out_bytes, hipMemcpyDeviceToHost, st));
  if (out.logits)
    PGD_HIP(hipMemcpyAsync(out.logits, w.logits, (size_t)lrows * c.vocab * 4, hipMemcpyDeviceToHost, st));
  PGD_HIP(hipStreamSynchronize(st));
  const uint32_t* h_ids = (const uint32_t*)m.out_host;
  const float* h_vals = (const float*)(h_ids + lrows);
  const int* h_nf = (const int*)(h_vals + lrows);
  if (out.ids) {
    // the engine faults a request on any non-finite logit
    // (pagoda/src/engine.rs:1278-1280): such a row returns no token
    for (int r = 0; r < lrows; ++r) out.ids[r] = h_nf[r] > 0 ? 0xFFFFFFFFu : h_ids[r];
  }
  if (out.vals) memcpy(out.vals, h_vals, (size_t)lrows * 4);
  for (int i = 0; i < nseq; ++i) sess[i]->len += n[i];
  poison.armed = false;
}

}  // namespace pgd

using namespace pgd;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int pgd_model_synth(pgd_dev* dev, const pgd_model_config* cfg, uint64_t seed, pgd_model** out) {
  pgd_model* held = nullptr;
  int rc = guard([&] {
    PGD_CHECK(dev && cfg && out, kErrArg, "null argument");
    validate_config(*cfg, true);
    DeviceScope scope(dev);
    held = new pgd_model();
    held->m.dev = dev;
    held->m.cfg = *cfg;
    SynthSource src(*cfg, seed);
    build_model(held->m, src);
    *out = held;
  });
  if (rc && held) delete held;
  return rc;
}

int pgd_model_set_kquant_arith(pgd_model* pm, int mode) {
  return guard([&] {
    PGD_CHECK(pm, kErrArg, "null model");
    PGD_CHECK(mode == PGD_ARITH_DEQUANT_F32 || mode == PGD_ARITH_CPU_Q8, kErrArg, "unknown arithmetic mode");
    pm->m.q8act = mode == PGD_ARITH_CPU_Q8 ? 1 : 0;
  });
}

int pgd_model_set_graphs(pgd_model* pm, int on) {
  return guard([&] {
    PGD_CHECK(pm, kErrArg, "null argument");
    Model& m = pm->m;
    DeviceScope scope(m.dev);
    PGD_HIP(hipStreamSynchronize(m.dev->stream));
    m.use_graphs = on != 0;
    if (!m.use_graphs) {
      m.drop_graphs();
      m.graph_seen.clear();
    }
  });
}

int pgd_model_graph_stats(const pgd_model* pm, int* graphs, long long* launches) {
  return guard([&] {
    PGD_CHECK(pm, kErrArg, "null argument");
    if (graphs) *graphs = (int)pm->m.graphs.size();
    if (launches) *launches = pm->m.graph_launches;
  });
}

int pgd_model_free(pgd_model* m) {
  return guard([&] {
    if (!m) return;
    PGD_CHECK(m->m.live_sessions == 0, kErrState, "free every session before its model");
    delete m;
  });
}

int pgd_model_info(const pgd_model* pm, size_t* weight_bytes, double* algo, int* kv_free) {
  return guard([&] {
    PGD_CHECK(pm, kErrArg, "null model");
    const Model& m = pm->m;
    size_t wb = m.embed.bytes + (m.tied ? 0 : m.head.bytes);
    double ab = qmat_algo_bytes(m.head);  // one embedding row is negligible
    for (auto& L : m.layers)
      for (const QMat* q :
           {&L.gate, &L.up, &L.down, &L.proj, &L.qkv, &L.z, &L.a, &L.b, &L.out, &L.q, &L.k, &L.v, &L.o}) {
        wb += q->bytes;
        ab += q->base ? qmat_algo_bytes(*q) : 0.0;
      }
    if (weight_bytes) *weight_bytes = wb;
    if (algo) *algo = ab;
    if (kv_free) *kv_free = (int)m.free_blocks.size();
  });
}

int pgd_session_new(pgd_model* pm, pgd_session** out) {
  pgd_session* held = nullptr;
  int rc = guard([&] {
    PGD_CHECK(pm && out, kErrArg, "null argument");
    Model& m = pm->m;
    DeviceScope scope(m.dev);
    held = new pgd_session();
    held->s.model = &m;
    m.live_sessions++;
    if (m.rec_floats) {
      void* p = nullptr;
      hipError_t e = hipMalloc(&p, m.rec_floats * 4);
      PGD_CHECK(e == hipSuccess, kErrAlloc, std::string("hipMalloc session state: ") + hipGetErrorString(e));
      held->s.rec = (float*)p;
      PGD_HIP(hipMemsetAsync(p, 0, m.rec_floats * 4, m.dev->stream));
      PGD_HIP(hipStreamSynchronize(m.dev->stream));
    }
    *out = held;
  });
  if (rc && held) delete held;
  return rc;
}

int pgd_session_fork(const pgd_session* ps, pgd_session** out) {
  pgd_session* held = nullptr;
  int rc = guard([&] {
    PGD_CHECK(ps && out, kErrArg, "null argument");
    const Session& s = ps->s;
    PGD_CHECK(!s.poisoned, kErrState, "session state is undefined after a failed step");
    Model& m = *s.model;
    DeviceScope scope(m.dev);
    held = new pgd_session();
    held->s.model = &m;
    m.live_sessions++;
    held->s.len = s.len;
    // only the pages holding positions [0, len): a failed step may have left
    // pages past them, which stay the parent's own
    const size_t used = ((size_t)s.len + m.cfg.kv_block - 1) / m.cfg.kv_block;
    held->s.blocks.assign(s.blocks.begin(), s.blocks.begin() + std::min(used, s.blocks.size()));
    for (int b : held->s.blocks) m.refcount[b]++;
    held->s.last_logits = s.last_logits;
    held->s.has_logits = s.has_logits;
    if (m.rec_floats) {
      void* p = nullptr;
      hipError_t e = hipMalloc(&p, m.rec_floats * 4);
      PGD_CHECK(e == hipSuccess, kErrAlloc, std::string("hipMalloc session state: ") + hipGetErrorString(e));
      held->s.rec = (float*)p;
      PGD_HIP(hipMemcpyAsync(p, s.rec, m.rec_floats * 4, hipMemcpyDeviceToDevice, m.dev->stream));
      PGD_HIP(hipStreamSynchronize(m.dev->stream));
    }
    *out = held;
  });
  if (rc && held) delete held;
  return rc;
}

int pgd_session_fork_prefix(const pgd_session* ps, int n, pgd_session** out) {
  pgd_session* held = nullptr;
  int rc = guard([&] {
    PGD_CHECK(ps && out, kErrArg, "null argument");
    const Session& s = ps->s;
    PGD_CHECK(!s.poisoned, kErrState, "session state is undefined after a failed step");
    Model& m = *s.model;
    // recurrent (GDN) state summarizes the whole context and cannot be cut
    // back to a shorter prefix; such backends offer no prefix graft
    // (CandleCausalLM::cache_prefix default None, pagoda-hf/src/lib.rs:224)
    PGD_CHECK(m.rec_floats == 0, kErrState, "a recurrent-state session cannot be sliced to a prefix");
    PGD_CHECK(n >= 0 && n <= s.len, kErrArg, "prefix length " + std::to_string(n) + " outside 0.." +
                                                 std::to_string(s.len));
    held = new pgd_session();
    held->s.model = &m;
    m.live_sessions++;
    held->s.len = n;
    // pages wholly or partly below n are shared; the partial last page is
    // copied on the first write (step's copy-on-write of a shared tail), and
    // its slots at or past n are never read before they are rewritten
    const size_t keep = ((size_t)n + m.cfg.kv_block - 1) / m.cfg.kv_block;
    held->s.blocks.assign(s.blocks.begin(), s.blocks.begin() + keep);
    for (int b : held->s.blocks) m.refcount[b]++;
    *out = held;
  });
  if (rc && held) delete held;
  return rc;
}

// ---- engine-addressable KV pages ----
// The engine's paged cache hands out physical block ids with reference counts
// and copy-on-write (pagoda/src/kv_cache.rs:1-8, 65-125); its radix cache maps
// each cached token to a (block, offset) slot (pagoda/src/radix_cache.rs:17-18).
// These entry points expose this backend's KV pages under the same scheme: a
// page id names the same page in every full-attention layer's K and V pools.

int pgd_model_kv_pool(const pgd_model* pm, int* n_pages, int* page_tokens, int* n_free) {
  return guard([&] {
    PGD_CHECK(pm, kErrArg, "null argument");
    const Model& m = pm->m;
    if (n_pages) *n_pages = (int)m.refcount.size();
    if (page_tokens) *page_tokens = m.cfg.kv_block;
    if (n_free) *n_free = (int)m.free_blocks.size();
  });
}

int pgd_session_pages(const pgd_session* ps, int32_t* ids, int cap, int* n) {
  return guard([&] {
    PGD_CHECK(ps && n, kErrArg, "null argument");
    const Session& s = ps->s;
    PGD_CHECK(!s.poisoned, kErrState, "session state is undefined after a failed step");
    const Model& m = *s.model;
    PGD_CHECK(m.n_full > 0, kErrState, "model has no KV pages");
    // a failed step may have allocated pages past len: only the ones holding
    // positions [0, len) are the session's KV
    const int used = (s.len + m.cfg.kv_block - 1) / m.cfg.kv_block;
    *n = used;
    if (!ids) return;
    PGD_CHECK(cap >= used, kErrArg, "page id buffer holds " + std::to_string(cap) + " of " + std::to_string(used));
    for (int i = 0; i < used; ++i) ids[i] = s.blocks[i];
  });
}

namespace {
void check_held_pages(const Model& m, const int32_t* ids, int n) {
  PGD_CHECK(n >= 0 && (n == 0 || ids), kErrArg, "bad page list");
  for (int i = 0; i < n; ++i) {
    PGD_CHECK(ids[i] >= 0 && ids[i] < (int)m.refcount.size(), kErrArg,
              "page id " + std::to_string(ids[i]) + " outside the pool");
    PGD_CHECK(m.refcount[ids[i]] > 0, kErrState, "page " + std::to_string(ids[i]) + " is free");
  }
}
}  // namespace

int pgd_page_retain(pgd_model* pm, const int32_t* ids, int n) {
  return guard([&] {
    PGD_CHECK(pm, kErrArg, "null argument");
    Model& m = pm->m;
    check_held_pages(m, ids, n);
    for (int i = 0; i < n; ++i) m.refcount[ids[i]]++;
  });
}

int pgd_page_release(pgd_model* pm, const int32_t* ids, int n) {
  return guard([&] {
    PGD_CHECK(pm, kErrArg, "null argument");
    Model& m = pm->m;
    check_held_pages(m, ids, n);
    // a page listed twice must hold two references
    std::unordered_map<int, int> count;
    for (int i = 0; i < n; ++i) count[ids[i]]++;
    for (auto& kv : count)
      PGD_CHECK(m.refcount[kv.first] >= kv.second, kErrState,
                "page " + std::to_string(kv.first) + " released more often than held");
    for (int i = 0; i < n; ++i) m.release_block(ids[i]);
  });
}

int pgd_page_refcount(const pgd_model* pm, int32_t id, int* count) {
  return guard([&] {
    PGD_CHECK(pm && count, kErrArg, "null argument");
    const Model& m = pm->m;
    PGD_CHECK(id >= 0 && id < (int)m.refcount.size(), kErrArg, "page id outside the pool");
    *count = m.refcount[id];
  });
}

int pgd_session_from_pages(pgd_model* pm, const int32_t* ids, int n_pages, int n_pos, pgd_session** out) {
  pgd_session* held = nullptr;
  int rc = guard([&] {
    PGD_CHECK(pm && out, kErrArg, "null argument");
    Model& m = pm->m;
    // a recurrent (GDN) state is not a function of KV pages: a hybrid session
    // cannot be rebuilt from them (CandleCausalLM::cache_prefix default None,
    // pagoda-hf/src/lib.rs:224)
    PGD_CHECK(m.rec_floats == 0, kErrState, "a recurrent-state model cannot build a session from KV pages");
    PGD_CHECK(m.n_full > 0, kErrState, "model has no KV pages");
    PGD_CHECK(n_pos >= 0 && n_pos <= m.cfg.max_pos, kErrArg, "length outside 0..max_pos");
    const int need = (n_pos + m.cfg.kv_block - 1) / m.cfg.kv_block;
    PGD_CHECK(n_pages == need, kErrArg,
              std::to_string(n_pos) + " positions take " + std::to_string(need) + " pages, not " +
                  std::to_string(n_pages));
    check_held_pages(m, ids, n_pages);
    {
      std::unordered_set<int> seen;
      for (int i = 0; i < n_pages; ++i)
        PGD_CHECK(seen.insert(ids[i]).second, kErrArg, "page " + std::to_string(ids[i]) + " listed twice");
    }
    held = new pgd_session();
    held->s.model = &m;
    m.live_sessions++;
    held->s.len = n_pos;
    held->s.blocks.assign(ids, ids + n_pages);
    // the session takes its own reference on every page; a page another
    // holder keeps (refcount > 1) is copied before the session's first write
    // into it (the step's copy-on-write of a shared tail)
    for (int b : held->s.blocks) m.refcount[b]++;
    *out = held;
  });
  if (rc && held) delete held;
  return rc;
}

int pgd_session_free(pgd_session* s) {
  return guard([&] { delete s; });
}

int pgd_session_len(const pgd_session* s, int* len) {
  return guard([&] {
    PGD_CHECK(s && len, kErrArg, "null argument");
    *len = s->s.len;
  });
}

int pgd_forward(pgd_session* ps, const uint32_t* toks, int n, float* logits) {
  return guard([&] {
    PGD_CHECK(ps && logits && n >= 0, kErrArg, "bad argument");
    Session& s = ps->s;
    Model& m = *s.model;
    if (n == 0) {
      PGD_CHECK(!s.poisoned, kErrState, "session state is undefined after a failed step");
      PGD_CHECK(s.has_logits, kErrState, "empty feed before any forward");
      memcpy(logits, s.last_logits.data(), (size_t)m.cfg.vocab * 4);
      return;
    }
    PGD_CHECK(toks, kErrArg, "null tokens");
    DeviceScope scope(m.dev);
    Session* sp = &s;
    uint32_t id = 0;
    StepOut o;
    o.ids = &id;
    o.logits = logits;
    step(m, &sp, toks, &n, 1, o);
    s.last_logits.assign(logits, logits + m.cfg.vocab);
    s.has_logits = true;
  });
}

int pgd_forward_greedy(pgd_session* ps, uint32_t tok, uint32_t* id, float* logit) {
  return guard([&] {
    PGD_CHECK(ps && id, kErrArg, "null argument");
    Session& s = ps->s;
    Model& m = *s.model;
    DeviceScope scope(m.dev);
    Session* sp = &s;
    int n = 1;
    float v = 0.0f;
    StepOut o;
    o.last_max = 1;
    o.ids = id;
    o.vals = &v;
    step(m, &sp, &tok, &n, 1, o);
    s.has_logits = false;
    if (logit) *logit = v;
  });
}

int pgd_forward_verify(pgd_session* ps, const uint32_t* toks, int n, uint32_t* ids, float* logits_max) {
  return guard([&] {
    PGD_CHECK(ps && toks && ids, kErrArg, "null argument");
    PGD_CHECK(n >= 1 && n <= 4, kErrArg, "verify batch must be 1..4 tokens");
    Session& s = ps->s;
    Model& m = *s.model;
    DeviceScope scope(m.dev);
    Session* sp = &s;
    StepOut o;
    o.all_rows = 1;
    o.last_max = 1;
    o.ids = ids;
    o.vals = logits_max;
    step(m, &sp, toks, &n, 1, o);
    s.has_logits = false;
  });
}

int pgd_step_ragged(pgd_model* pm, pgd_session* const* sessions, const uint32_t* toks, const int* n_per_seq,
                    int nseq, int all_rows, uint32_t* ids, float* logits) {
  return guard([&] {
    PGD_CHECK(pm && sessions && toks && n_per_seq && ids && nseq > 0, kErrArg, "null argument");
    Model& m = pm->m;
    DeviceScope scope(m.dev);
    std::vector<Session*> ss(nseq);
    for (int i = 0; i < nseq; ++i) {
      PGD_CHECK(sessions[i], kErrArg, "null session");
      ss[i] = &sessions[i]->s;
    }
    StepOut o;
    o.all_rows = all_rows ? 1 : 0;
    o.ids = ids;
    o.logits = logits;
    step(m, ss.data(), toks, n_per_seq, nseq, o);
    for (int i = 0; i < nseq; ++i) {
      if (logits && !all_rows) {
        ss[i]->last_logits.assign(logits + (size_t)i * m.cfg.vocab, logits + (size_t)(i + 1) * m.cfg.vocab);
        ss[i]->has_logits = true;
      } else {
        ss[i]->has_logits = false;
      }
    }
  });
}

// ---- cache bytes v1 (pagoda-hf/src/qwen3_5.rs:177-255) ----
}  // extern "C"

namespace {
void put(std::vector<uint8_t>& b, const void* p, size_t n) {
  const uint8_t* c = (const uint8_t*)p;
  b.insert(b.end(), c, c + n);
}
void put_u32(std::vector<uint8_t>& b, uint32_t v) { put(b, &v, 4); }
void put_vec(std::vector<uint8_t>& b, const float* v, size_t n) {
  put_u32(b, (uint32_t)n);
  put(b, v, n * 4);
}
struct Reader {
  const uint8_t* p;
  size_t n, at = 0;
  void need(size_t k) { PGD_CHECK(at + k <= n, kErrFormat, "kv truncated"); }
  uint8_t u8() {
    need(1);
    return p[at++];
  }
  uint32_t u32() {
    need(4);
    uint32_t v;
    memcpy(&v, p + at, 4);
    at += 4;
    return v;
  }
  uint64_t u64() {
    need(8);
    uint64_t v;
    memcpy(&v, p + at, 8);
    at += 8;
    return v;
  }
  std::vector<float> vec() {
    uint32_t k = u32();
    need((size_t)k * 4);
    std::vector<float> v(k);
    memcpy(v.data(), p + at, (size_t)k * 4);
    at += (size_t)k * 4;
    return v;
  }
};

// IEEE binary16 with round to nearest even; NaN -> quiet NaN keeping the
// sign, overflow -> infinity (the f16 wire encoding of
// pagoda-hf/src/llama.rs:139-172).
uint16_t f32_to_f16_rne(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  const uint32_t sign = (b >> 16) & 0x8000u;
  const int e32 = (int)((b >> 23) & 0xffu);
  uint32_t man = b & 0x7fffffu;
  if (e32 == 0xff) return (uint16_t)(sign | (man ? 0x7e00u : 0x7c00u));
  const int e = e32 - 112;  // rebias 127 -> 15
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {  // subnormal half (or zero)
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const int sh = 14 - e;
    uint32_t h = man >> sh, rest = man & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (rest > half || (rest == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rest = man & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;  // a carry into the exponent is correct
  return (uint16_t)(sign | h);
}

float f16_to_f32_exact(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu, bits;
  if (e == 0) {
    if (!man) {
      bits = sign;
    } else {
      int k = 0;
      while (!(man & 0x400u)) {
        man <<= 1;
        ++k;
      }
      bits = sign | ((uint32_t)(113 - k) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((e + 112) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

// process-wide wire dtype of the SessionKv export (llama.rs:128-136)
std::atomic<int> g_kv_wire_f16{0};

constexpr uint32_t kKvWireMagic = 0x50444B56u;

// One KV pool as [kv_heads][len][head_dim] f32 on the host.
std::vector<float> gather_kv_head_major(const Model& m, const Session& s, const float* pool) {
  const pgd_model_config& c = m.cfg;
  const size_t per_blk = (size_t)c.kv_heads * c.kv_block * c.head_dim;
  std::vector<float> out((size_t)c.kv_heads * s.len * c.head_dim), page(per_blk);
  for (size_t bi = 0; bi < s.blocks.size(); ++bi) {
    PGD_HIP(hipMemcpy(page.data(), pool + (size_t)s.blocks[bi] * per_blk, per_blk * 4, hipMemcpyDeviceToHost));
    for (int h = 0; h < c.kv_heads; ++h)
      for (int sl = 0; sl < c.kv_block; ++sl) {
        const size_t p = bi * c.kv_block + sl;
        if (p >= (size_t)s.len) break;
        memcpy(&out[((size_t)h * s.len + p) * c.head_dim], &page[((size_t)h * c.kv_block + sl) * c.head_dim],
               (size_t)c.head_dim * 4);
      }
  }
  return out;
}

// SessionKv::export_bytes (pagoda-hf/src/llama.rs:215-266)
std::vector<uint8_t> export_sessionkv(const Model& m, const Session& s) {
  const pgd_model_config& c = m.cfg;
  const bool f16 = g_kv_wire_f16.load() != 0;
  std::vector<uint8_t> b;
  put_u32(b, kKvWireMagic);
  put_u32(b, 2);
  put_u32(b, (uint32_t)s.len);
  put_u32(b, (uint32_t)c.n_layers);
  if (s.has_logits)
    put_vec(b, s.last_logits.data(), s.last_logits.size());
  else
    put_u32(b, 0);
  for (const Layer& L : m.layers) {
    if (s.len == 0) {  // no forward yet: the reference's layers are None
      put_u32(b, 0);
      continue;
    }
    put_u32(b, 1);
    put_u32(b, (uint32_t)c.kv_heads);
    put_u32(b, (uint32_t)c.head_dim);
    put_u32(b, f16 ? 1u : 0u);
    for (const float* pool : {L.k_pool, L.v_pool}) {
      const std::vector<float> kv = gather_kv_head_major(m, s, pool);
      if (f16) {
        for (float x : kv) {
          const uint16_t h = f32_to_f16_rne(x);
          put(b, &h, 2);
        }
      } else {
        put(b, kv.data(), kv.size() * 4);
      }
    }
  }
  return b;
}
}  // namespace

extern "C" {

int pgd_set_kv_wire_f16(int on) {
  g_kv_wire_f16.store(on ? 1 : 0);
  return 0;
}

int pgd_session_export(const pgd_session* ps, uint8_t* buf, size_t cap, size_t* len) {
  return guard([&] {
    PGD_CHECK(ps && len, kErrArg, "null argument");
    const Session& s = ps->s;
    PGD_CHECK(!s.poisoned, kErrState, "session state is undefined after a failed step");
    const Model& m = *s.model;
    const pgd_model_config& c = m.cfg;
    DeviceScope scope(m.dev);
    PGD_HIP(hipStreamSynchronize(m.dev->stream));
    if (c.arch == PGD_ARCH_QWEN2) {
      const std::vector<uint8_t> b = export_sessionkv(m, s);
      *len = b.size();
      if (buf) {
        PGD_CHECK(cap >= b.size(), kErrArg, "export buffer too small");
        memcpy(buf, b.data(), b.size());
      }
      return;
    }
    std::vector<uint8_t> b;
    put_u32(b, 1);
    uint64_t L64 = (uint64_t)s.len;
    put(b, &L64, 8);
    put_u32(b, (uint32_t)c.n_layers);
    const size_t per_blk = (size_t)c.kv_heads * c.kv_block * c.head_dim;
    const size_t per_lin = m.conv_floats + m.state_floats;
    std::vector<float> tmp;
    for (const Layer& L : m.layers) {
      if (L.full) {
        b.push_back(2);
        put_u32(b, (uint32_t)s.len);
        put_u32(b, (uint32_t)c.kv_heads);
        put_u32(b, (uint32_t)c.head_dim);
        for (int which = 0; which < 2; ++which) {
          const float* pool = which == 0 ? L.k_pool : L.v_pool;
          std::vector<float> out((size_t)s.len * c.kv_heads * c.head_dim);
          tmp.resize(per_blk);
          for (size_t bi = 0; bi < s.blocks.size(); ++bi) {
            PGD_HIP(hipMemcpy(tmp.data(), pool + (size_t)s.blocks[bi] * per_blk, per_blk * 4, hipMemcpyDeviceToHost));
            for (int sl = 0; sl < c.kv_block; ++sl) {
              size_t p = bi * c.kv_block + sl;
              if (p >= (size_t)s.len) break;
              for (int h = 0; h < c.kv_heads; ++h)
                memcpy(&out[(p * c.kv_heads + h) * c.head_dim], &tmp[((size_t)h * c.kv_block + sl) * c.head_dim],
                       (size_t)c.head_dim * 4);
            }
          }
          put_vec(b, out.data(), out.size());
        }
      } else {
        b.push_back(1);
        size_t cf = (size_t)m.conv_dim * (c.conv_kernel - 1);
        tmp.resize(std::max(cf, m.state_floats));
        const float* base = s.rec + (size_t)L.lin_index * per_lin;
        PGD_HIP(hipMemcpy(tmp.data(), base, cf * 4, hipMemcpyDeviceToHost));
        put_vec(b, tmp.data(), cf);
        PGD_HIP(hipMemcpy(tmp.data(), base + m.conv_floats, m.state_floats * 4, hipMemcpyDeviceToHost));
        put_vec(b, tmp.data(), m.state_floats);
      }
    }
    *len = b.size();
    if (buf) {
      PGD_CHECK(cap >= b.size(), kErrArg, "export buffer too small");
      memcpy(buf, b.data(), b.size());
    }
  });
}

}  // extern "C"

namespace {
// SessionKv::import_bytes (pagoda-hf/src/llama.rs:268-345): version 1
// (payload f32 whatever the dtype field says) or 2 (dtype 1 = f16 payload);
// the logits become the session's cached last logits (replayed on an empty
// feed, lib.rs:644-667). This cache needs every layer present with the
// model's kv_heads/head_dim (or none, at length 0) and logits of vocab
// entries or none. Trailing bytes are ignored, as in the reference reader.
pgd_session* import_sessionkv(Model& m, const uint8_t* buf, size_t len) {
  const pgd_model_config& c = m.cfg;
  Reader rd{buf, len};
  PGD_CHECK(rd.u32() == kKvWireMagic, kErrFormat, "bad kv payload magic");
  const uint32_t version = rd.u32();
  PGD_CHECK(version == 1 || version == 2, kErrFormat, "unsupported kv payload version " + std::to_string(version));
  const uint32_t slen = rd.u32();
  PGD_CHECK(rd.u32() == (uint32_t)c.n_layers, kErrFormat, "layer count mismatch");
  PGD_CHECK(slen <= (uint32_t)c.max_pos, kErrFormat, "length exceeds max_pos");
  const uint32_t nl = rd.u32();
  PGD_CHECK(nl == 0 || nl == (uint32_t)c.vocab, kErrFormat, "logits count is neither 0 nor vocab");
  rd.need((size_t)nl * 4);
  std::vector<float> logits(nl);
  if (nl) memcpy(logits.data(), buf + rd.at, (size_t)nl * 4);
  rd.at += (size_t)nl * 4;
  const size_t count = (size_t)c.kv_heads * slen * c.head_dim;
  std::vector<std::vector<float>> kv((size_t)m.n_full * 2);
  for (const Layer& L : m.layers) {
    const uint32_t present = rd.u32();
    if (!present) {
      PGD_CHECK(slen == 0, kErrFormat, "missing layer in a non-empty kv payload");
      continue;
    }
    const uint32_t kvh = rd.u32(), hd = rd.u32(), dt = rd.u32();
    PGD_CHECK(kvh == (uint32_t)c.kv_heads && hd == (uint32_t)c.head_dim, kErrFormat, "kv shape");
    const bool f16 = version >= 2 && dt == 1;
    for (int which = 0; which < 2; ++which) {
      std::vector<float>& dst = kv[(size_t)L.full_index * 2 + which];
      dst.resize(count);
      rd.need(count * (f16 ? 2 : 4));
      if (f16) {
        for (size_t i = 0; i < count; ++i) {
          uint16_t h;
          memcpy(&h, buf + rd.at + 2 * i, 2);
          dst[i] = f16_to_f32_exact(h);
        }
        rd.at += count * 2;
      } else {
        memcpy(dst.data(), buf + rd.at, count * 4);
        rd.at += count * 4;
      }
    }
  }
  const size_t nblk = ((size_t)slen + c.kv_block - 1) / c.kv_block;
  PGD_CHECK(nblk <= m.free_blocks.size(), kErrAlloc, "KV page pool exhausted");
  DeviceScope scope(m.dev);
  pgd_session* held = new pgd_session();
  Session& s = held->s;
  s.model = &m;
  m.live_sessions++;
  try {
    for (size_t i = 0; i < nblk; ++i) s.blocks.push_back(m.alloc_block());
    const size_t per_blk = (size_t)c.kv_heads * c.kv_block * c.head_dim;
    std::vector<float> page(per_blk);
    for (const Layer& L : m.layers) {
      if (slen == 0) break;
      for (int which = 0; which < 2; ++which) {
        const std::vector<float>& src = kv[(size_t)L.full_index * 2 + which];
        float* pool = which == 0 ? L.k_pool : L.v_pool;
        for (size_t bi = 0; bi < nblk; ++bi) {
          std::fill(page.begin(), page.end(), 0.0f);
          for (int h = 0; h < c.kv_heads; ++h)
            for (int sl = 0; sl < c.kv_block; ++sl) {
              const size_t p = bi * c.kv_block + sl;
              if (p >= slen) break;
              memcpy(&page[((size_t)h * c.kv_block + sl) * c.head_dim], &src[((size_t)h * slen + p) * c.head_dim],
                     (size_t)c.head_dim * 4);
            }
          PGD_HIP(hipMemcpy(pool + (size_t)s.blocks[bi] * per_blk, page.data(), per_blk * 4, hipMemcpyHostToDevice));
        }
      }
    }
  } catch (...) {
    delete held;
    throw;
  }
  s.len = (int)slen;
  if (nl) {
    s.last_logits = std::move(logits);
    s.has_logits = true;
  }
  return held;
}
}  // namespace

extern "C" {

int pgd_session_import(pgd_model* pm, const uint8_t* buf, size_t len, pgd_session** out) {
  pgd_session* held = nullptr;
  int rc = guard([&] {
    PGD_CHECK(pm && buf && out, kErrArg, "null argument");
    Model& m = pm->m;
    const pgd_model_config& c = m.cfg;
    if (c.arch == PGD_ARCH_QWEN2) {
      held = import_sessionkv(m, buf, len);
      *out = held;
      return;
    }
    Reader rd{buf, len};
    PGD_CHECK(rd.u32() == 1, kErrFormat, "kv version");
    uint64_t slen = rd.u64();
    PGD_CHECK(rd.u32() == (uint32_t)c.n_layers, kErrFormat, "layer count mismatch");
    PGD_CHECK(slen <= (uint64_t)c.max_pos, kErrFormat, "length exceeds max_pos");
    size_t nblk = (slen + c.kv_block - 1) / c.kv_block;
    PGD_CHECK(nblk <= m.free_blocks.size() || m.n_full == 0, kErrAlloc, "KV page pool exhausted");
    const size_t per_blk = (size_t)c.kv_heads * c.kv_block * c.head_dim;
    const size_t per_lin = m.conv_floats + m.state_floats;
    // parse everything first
    std::vector<std::vector<float>> conv(m.n_lin), state(m.n_lin), kk(m.n_full), vv(m.n_full);
    for (const Layer& L : m.layers) {
      uint8_t tag = rd.u8();
      if (L.full) {
        PGD_CHECK(tag == 2, kErrFormat, "layer kind mismatch");
        uint32_t kv_len = rd.u32(), kvh = rd.u32(), hd = rd.u32();
        PGD_CHECK(kv_len == slen && kvh == (uint32_t)c.kv_heads && hd == (uint32_t)c.head_dim, kErrFormat, "kv shape");
        kk[L.full_index] = rd.vec();
        vv[L.full_index] = rd.vec();
        PGD_CHECK(kk[L.full_index].size() == (size_t)kv_len * kvh * hd && vv[L.full_index].size() == kk[L.full_index].size(),
                  kErrFormat, "kv shape");
      } else {
        PGD_CHECK(tag == 1, kErrFormat, "layer kind mismatch");
        conv[L.lin_index] = rd.vec();
        state[L.lin_index] = rd.vec();
        PGD_CHECK(conv[L.lin_index].size() == (size_t)m.conv_dim * (c.conv_kernel - 1) &&
                      state[L.lin_index].size() == m.state_floats,
                  kErrFormat, "recurrent state shape");
      }
    }
    PGD_CHECK(rd.at == len, kErrFormat, "kv trailing bytes");
    DeviceScope scope(m.dev);
    held = new pgd_session();
    Session& s = held->s;
    s.model = &m;
    m.live_sessions++;
    if (m.rec_floats) {
      void* p = nullptr;
      hipError_t e = hipMalloc(&p, m.rec_floats * 4);
      PGD_CHECK(e == hipSuccess, kErrAlloc, "hipMalloc session state");
      s.rec = (float*)p;
      PGD_HIP(hipMemsetAsync(p, 0, m.rec_floats * 4, m.dev->stream));
      PGD_HIP(hipStreamSynchronize(m.dev->stream));
    }
    if (m.n_full) {
      for (size_t i = 0; i < nblk; ++i) s.blocks.push_back(m.alloc_block());
    }
    std::vector<float> page(per_blk);
    for (const Layer& L : m.layers) {
      if (L.full) {
        for (int which = 0; which < 2; ++which) {
          const std::vector<float>& src = which == 0 ? kk[L.full_index] : vv[L.full_index];
          float* pool = which == 0 ? L.k_pool : L.v_pool;
          for (size_t bi = 0; bi < nblk; ++bi) {
            std::fill(page.begin(), page.end(), 0.0f);
            for (int sl = 0; sl < c.kv_block; ++sl) {
              size_t p = bi * c.kv_block + sl;
              if (p >= slen) break;
              for (int h = 0; h < c.kv_heads; ++h)
                memcpy(&page[((size_t)h * c.kv_block + sl) * c.head_dim], &src[(p * c.kv_heads + h) * c.head_dim],
                       (size_t)c.head_dim * 4);
            }
            PGD_HIP(hipMemcpy(pool + (size_t)s.blocks[bi] * per_blk, page.data(), per_blk * 4, hipMemcpyHostToDevice));
          }
        }
      } else {
        float* base = s.rec + (size_t)L.lin_index * per_lin;
        PGD_HIP(hipMemcpy(base, conv[L.lin_index].data(), conv[L.lin_index].size() * 4, hipMemcpyHostToDevice));
        PGD_HIP(hipMemcpy(base + m.conv_floats, state[L.lin_index].data(), m.state_floats * 4, hipMemcpyHostToDevice));
      }
    }
    s.len = (int)slen;
    *out = held;
  });
  if (rc && held) delete held;
  return rc;
}

}  // extern "C"
