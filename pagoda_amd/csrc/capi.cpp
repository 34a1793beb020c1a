// capi.cpp — extern "C" surface: devices, matrices and the error channel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/pagoda_hip.h"
#include "common.h"
#include "device.h"
#include "ops.h"
#include "quant.h"

namespace pgd {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
const std::string& last_error() { return g_last_error; }

}  // namespace pgd

using namespace pgd;

struct pgd_matrix {
  pgd_dev* dev;
  QMat m;
};

struct pgd_event {
  pgd_dev* dev;
  hipEvent_t ev;
};

extern "C" {

int pgd_last_error(char* buf, size_t len) {
  const std::string& e = last_error();
  if (buf && len) {
    size_t n = e.size() < len - 1 ? e.size() : len - 1;
    memcpy(buf, e.data(), n);
    buf[n] = 0;
  }
  return (int)e.size();
}

int pgd_version(void) { return 100; }

int pgd_device_open(const char* spec, pgd_dev** out) {
  return guard([&] {
    PGD_CHECK(spec && out, kErrArg, "pgd_device_open: null argument");
    std::string s(spec);
    int ordinal = 0;
    if (s == "hip") {
      ordinal = 0;
    } else if (s.rfind("hip:", 0) == 0 && s.size() > 4) {
      char* end = nullptr;
      long v = strtol(s.c_str() + 4, &end, 10);
      PGD_CHECK(end && *end == 0 && v >= 0, kErrArg, "bad PAGODA_DEVICE index in \"" + s + "\"");
      ordinal = (int)v;
    } else {
      throw Error{kErrArg, "unknown device spec \"" + s + "\" (want hip or hip:N)"};
    }
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    PGD_CHECK(e == hipSuccess && count > 0, kErrDevice, "no HIP device available");
    PGD_CHECK(ordinal < count, kErrDevice, "no HIP device " + std::to_string(ordinal));
    *out = new pgd_dev(ordinal);
  });
}

int pgd_device_close(pgd_dev* dev) {
  return guard([&] {
    if (!dev) return;
    delete dev;
  });
}

int pgd_device_sync(pgd_dev* dev) {
  return guard([&] {
    PGD_CHECK(dev, kErrArg, "null device");
    DeviceScope scope(dev);
    PGD_HIP(hipStreamSynchronize(dev->stream));
  });
}

void* pgd_device_stream(pgd_dev* dev) { return dev ? (void*)dev->stream : nullptr; }

int pgd_device_malloc(pgd_dev* dev, size_t bytes, void** out) {
  return guard([&] {
    PGD_CHECK(dev && out, kErrArg, "null argument");
    DeviceScope scope(dev);
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    PGD_CHECK(e == hipSuccess, kErrAlloc, std::string("hipMalloc: ") + hipGetErrorString(e));
    *out = p;
  });
}

int pgd_device_free(pgd_dev* dev, void* ptr) {
  return guard([&] {
    PGD_CHECK(dev, kErrArg, "null device");
    DeviceScope scope(dev);
    if (ptr) PGD_HIP(hipFree(ptr));
  });
}

int pgd_device_memcpy(pgd_dev* dev, void* dst, const void* src, size_t bytes, int kind) {
  return guard([&] {
    PGD_CHECK(dev, kErrArg, "null device");
    PGD_CHECK(kind >= 0 && kind <= 2, kErrArg, "memcpy kind");
    DeviceScope scope(dev);
    hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice : kind == 1 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    if (bytes) PGD_HIP(hipMemcpyAsync(dst, src, bytes, k, dev->stream));
    PGD_HIP(hipStreamSynchronize(dev->stream));
  });
}

int pgd_device_copy_dev(pgd_dev* dev, void* dst, const void* src, size_t bytes) {
  return guard([&] {
    PGD_CHECK(dev && (bytes == 0 || (dst && src)), kErrArg, "null argument");
    DeviceScope scope(dev);
    if (bytes) PGD_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, dev->stream));
  });
}

int pgd_event_new(pgd_dev* dev, pgd_event** out) {
  return guard([&] {
    PGD_CHECK(dev && out, kErrArg, "null argument");
    DeviceScope scope(dev);
    hipEvent_t e;
    PGD_HIP(hipEventCreate(&e));
    *out = new pgd_event{dev, e};
  });
}

int pgd_event_record(pgd_event* ev) {
  return guard([&] {
    PGD_CHECK(ev, kErrArg, "null event");
    DeviceScope scope(ev->dev);
    PGD_HIP(hipEventRecord(ev->ev, ev->dev->stream));
  });
}

int pgd_event_elapsed_ms(pgd_event* start, pgd_event* end, float* ms) {
  return guard([&] {
    PGD_CHECK(start && end && ms, kErrArg, "null argument");
    DeviceScope scope(end->dev);
    PGD_HIP(hipEventSynchronize(end->ev));
    PGD_HIP(hipEventElapsedTime(ms, start->ev, end->ev));
  });
}

int pgd_event_free(pgd_event* ev) {
  return guard([&] {
    if (!ev) return;
    DeviceScope scope(ev->dev);
    (void)hipEventDestroy(ev->ev);
    delete ev;
  });
}

static int new_matrix(pgd_dev* dev, int fmt, int n_out, int n_in, pgd_matrix** out, pgd_matrix** held) {
  PGD_CHECK(dev && out, kErrArg, "null argument");
  auto* m = new pgd_matrix{dev, QMat{}};
  *held = m;
  qmat_alloc(m->m, fmt, n_out, n_in, dev->stream);
  return 0;
}

int pgd_matrix_upload_a8(pgd_dev* dev, const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                         int n_out, int n_in, pgd_matrix** out) {
  pgd_matrix* held = nullptr;
  int rc = guard([&] {
    PGD_CHECK(packed && scales && biases, kErrArg, "null argument");
    DeviceScope scope(dev);
    new_matrix(dev, FMT_A8, n_out, n_in, out, &held);
    qmat_upload_a8(held->m, packed, scales, biases, dev->stream);
    *out = held;
  });
  if (rc && held) pgd_matrix_free(held);
  return rc;
}

static int upload_kq(pgd_dev* dev, int fmt, const void* blocks, int n_out, int n_in, pgd_matrix** out) {
  pgd_matrix* held = nullptr;
  int rc = guard([&] {
    PGD_CHECK(blocks, kErrArg, "null argument");
    DeviceScope scope(dev);
    new_matrix(dev, fmt, n_out, n_in, out, &held);
    qmat_upload_kq(held->m, (const uint8_t*)blocks, dev->stream);
    *out = held;
  });
  if (rc && held) pgd_matrix_free(held);
  return rc;
}

int pgd_matrix_upload_q4k(pgd_dev* dev, const void* blocks, int n_out, int n_in, pgd_matrix** out) {
  return upload_kq(dev, FMT_Q4K, blocks, n_out, n_in, out);
}

int pgd_matrix_upload_q6k(pgd_dev* dev, const void* blocks, int n_out, int n_in, pgd_matrix** out) {
  return upload_kq(dev, FMT_Q6K, blocks, n_out, n_in, out);
}

int pgd_matrix_upload_q8_0(pgd_dev* dev, const void* blocks, int n_out, int n_in, pgd_matrix** out) {
  return upload_kq(dev, FMT_Q8_0, blocks, n_out, n_in, out);
}

int pgd_matrix_upload_q5_0(pgd_dev* dev, const void* blocks, int n_out, int n_in, pgd_matrix** out) {
  return upload_kq(dev, FMT_Q5_0, blocks, n_out, n_in, out);
}

int pgd_matrix_synth(pgd_dev* dev, int fmt, int n_out, int n_in, uint64_t seed, uint64_t key, float std,
                     pgd_matrix** out) {
  pgd_matrix* held = nullptr;
  int rc = guard([&] {
    PGD_CHECK(fmt >= 0 && fmt <= 2, kErrFormat, "unknown matrix format");
    DeviceScope scope(dev);
    new_matrix(dev, fmt, n_out, n_in, out, &held);
    qmat_synth(held->m, seed, key, std, dev->stream);
    PGD_HIP(hipStreamSynchronize(dev->stream));
    *out = held;
  });
  if (rc && held) pgd_matrix_free(held);
  return rc;
}

int pgd_matrix_free(pgd_matrix* m) {
  return guard([&] {
    if (!m) return;
    DeviceScope scope(m->dev);
    (void)hipStreamSynchronize(m->dev->stream);
    qmat_free(m->m);
    delete m;
  });
}

int pgd_matrix_info(const pgd_matrix* m, int* fmt, int* n_out, int* n_in, size_t* dev_bytes, double* algo) {
  return guard([&] {
    PGD_CHECK(m, kErrArg, "null matrix");
    if (fmt) *fmt = m->m.fmt;
    if (n_out) *n_out = m->m.n_out;
    if (n_in) *n_in = m->m.n_in;
    if (dev_bytes) *dev_bytes = m->m.bytes;
    if (algo) *algo = qmat_algo_bytes(m->m);
  });
}

int pgd_matrix_dequant(const pgd_matrix* m, int row0, int rows, float* out) {
  return guard([&] {
    PGD_CHECK(m && out, kErrArg, "null argument");
    PGD_CHECK(row0 >= 0 && rows >= 0 && row0 + rows <= m->m.n_out, kErrShape, "dequant row range");
    if (!rows) return;
    DeviceScope scope(m->dev);
    DevBuf buf((size_t)rows * m->m.n_in * 4);
    qmat_dequant(m->m, row0, rows, (float*)buf.p, m->dev->stream);
    PGD_HIP(hipMemcpyAsync(out, buf.p, buf.bytes, hipMemcpyDeviceToHost, m->dev->stream));
    PGD_HIP(hipStreamSynchronize(m->dev->stream));
  });
}

int pgd_matrix_gemv(const pgd_matrix* m, const float* x, int nrows, float* y) {
  return guard([&] {
    PGD_CHECK(m && x && y, kErrArg, "null argument");
    PGD_CHECK(nrows >= 1 && nrows <= 64, kErrShape, "gemv rows must be in 1..64");
    DeviceScope scope(m->dev);
    int ldx = (m->m.n_in + 7) & ~7;
    DevBuf xb((size_t)nrows * ldx * 4), yb((size_t)nrows * m->m.n_out * 4);
    hipStream_t s = m->dev->stream;
    PGD_HIP(hipMemcpy2DAsync(xb.p, (size_t)ldx * 4, x, (size_t)m->m.n_in * 4, (size_t)m->m.n_in * 4, nrows,
                             hipMemcpyHostToDevice, s));
    qmat_gemv(m->m, xb.p, 0, ldx, nrows, (float*)yb.p, m->m.n_out, nullptr, 0, s);
    PGD_HIP(hipMemcpyAsync(y, yb.p, yb.bytes, hipMemcpyDeviceToHost, s));
    PGD_HIP(hipStreamSynchronize(s));
  });
}

int pgd_matrix_gemv_dev(const pgd_matrix* m, const void* x, int x_f16, int ldx, int nrows, float* y, int ldy,
                        const float* res, int ldres) {
  return guard([&] {
    PGD_CHECK(m && x && y, kErrArg, "null argument");
    PGD_CHECK(ldy >= m->m.n_out && (!res || ldres >= m->m.n_out), kErrShape, "gemv output stride");
    DeviceScope scope(m->dev);
    qmat_gemv(m->m, x, x_f16, ldx, nrows, y, ldy, res, ldres, m->dev->stream);
  });
}

int pgd_matrix_gemv_swiglu_dev(const pgd_matrix* gate, const pgd_matrix* up, const float* x, int ldx, int nrows,
                               float* mid, int ldm) {
  return guard([&] {
    PGD_CHECK(gate && up && x && mid, kErrArg, "null argument");
    PGD_CHECK(gate->dev == up->dev, kErrArg, "gate and up live on different devices");
    PGD_CHECK(ldm >= gate->m.n_out, kErrShape, "swiglu output stride");
    DeviceScope scope(gate->dev);
    qmat_gemv_swiglu(gate->m, up->m, x, ldx, nrows, mid, ldm, gate->dev->stream);
  });
}

namespace {
int gdn_call(pgd_dev* dev, int k_heads, int v_heads, const float* conv_out, const float* a, const float* b,
             const float* z, const float* a_log, const float* dt_bias, const float* norm, float* const* states,
             const int* row_start, const int* row_count, int nseq, int rows, int max_rows, float* out) {
  return guard([&] {
    PGD_CHECK(dev && conv_out && a && b && z && a_log && dt_bias && norm && states && row_start && row_count && out,
              kErrArg, "null argument");
    PGD_CHECK(nseq >= 0 && rows >= 0 && max_rows >= 0, kErrArg, "nseq, rows, max_rows");
    DeviceScope scope(dev);
    GdnParams p{};
    p.k_heads = k_heads;
    p.v_heads = v_heads;
    p.k_dim = 128;
    p.v_dim = 128;
    p.conv_out = conv_out;
    p.ld_conv = 2 * k_heads * 128 + v_heads * 128;
    p.a = a;
    p.b = b;
    p.ld_ab = v_heads;
    p.z = z;
    p.ld_z = v_heads * 128;
    p.a_log = a_log;
    p.dt_bias = dt_bias;
    p.norm = norm;
    p.out = out;
    p.ld_out = v_heads * 128;
    p.state_base = states;
    p.state_off = 0;
    gdn_step(p, SeqMeta{row_start, row_count}, nseq, rows, max_rows, dev->stream);
  });
}
}  // namespace

int pgd_gdn_step_dev(pgd_dev* dev, int k_heads, int v_heads, const float* conv_out, const float* a, const float* b,
                     const float* z, const float* a_log, const float* dt_bias, const float* norm, float* const* states,
                     const int* row_start, const int* row_count, int nseq, float* out) {
  return gdn_call(dev, k_heads, v_heads, conv_out, a, b, z, a_log, dt_bias, norm, states, row_start, row_count, nseq,
                  0, 0, out);
}

int pgd_gdn_prefill_dev(pgd_dev* dev, int k_heads, int v_heads, const float* conv_out, const float* a,
                        const float* b, const float* z, const float* a_log, const float* dt_bias, const float* norm,
                        float* const* states, const int* row_start, const int* row_count, int nseq, int rows,
                        int max_rows, float* out) {
  return gdn_call(dev, k_heads, v_heads, conv_out, a, b, z, a_log, dt_bias, norm, states, row_start, row_count, nseq,
                  rows, max_rows, out);
}

int pgd_attn_decode_dev(pgd_dev* dev, int heads, int kv_heads, int head_dim, int block, const float* q,
                        const float* gate, const float* k_pool, const float* v_pool, const int* seq_of_row,
                        const int* pos_of_row, const int* block_tables, int max_blocks, int rows, float* out) {
  return guard([&] {
    PGD_CHECK(dev && q && k_pool && v_pool && seq_of_row && pos_of_row && block_tables && out, kErrArg,
              "null argument");
    PGD_CHECK(block > 0 && max_blocks > 0 && rows >= 0, kErrArg, "bad page geometry");
    DeviceScope scope(dev);
    AttnLayout L{heads, kv_heads, head_dim, head_dim, block, const_cast<float*>(k_pool), const_cast<float*>(v_pool)};
    RowMeta m{seq_of_row, pos_of_row, block_tables, max_blocks, nullptr, nullptr};
    if (rows == 0) return;
    PGD_CHECK(kv_heads > 0 && heads % kv_heads == 0, kErrShape, "heads must be a multiple of kv_heads");
    // the plan is built from the row metadata on the host
    std::vector<int> h_seq(rows), h_pos(rows);
    PGD_HIP(hipStreamSynchronize(dev->stream));
    PGD_HIP(hipMemcpy(h_seq.data(), seq_of_row, rows * sizeof(int), hipMemcpyDeviceToHost));
    PGD_HIP(hipMemcpy(h_pos.data(), pos_of_row, rows * sizeof(int), hipMemcpyDeviceToHost));
    int nseq = 0;
    for (int v : h_seq) {
      PGD_CHECK(v >= 0, kErrArg, "negative sequence index");
      nseq = std::max(nseq, v + 1);
    }
    std::vector<int> h_bt((size_t)nseq * max_blocks);
    PGD_HIP(hipMemcpy(h_bt.data(), block_tables, h_bt.size() * sizeof(int), hipMemcpyDeviceToHost));
    std::vector<int> plan;
    build_attn_plan(h_seq.data(), h_pos.data(), rows, h_bt.data(), max_blocks, block, heads / kv_heads, head_dim,
                    plan);
    DevBuf d_plan(plan.size() * sizeof(int));
    PGD_HIP(hipMemcpy(d_plan.p, plan.data(), plan.size() * sizeof(int), hipMemcpyHostToDevice));
    attn_decode(q, gate, out, L, m, attn_plan_view(plan.data(), d_plan.as<int>()), rows, dev->stream);
    PGD_HIP(hipStreamSynchronize(dev->stream));
  });
}

size_t pgd_act_bytes(int nrows, int k) { return nrows > 0 && k > 0 ? a8_act_bytes(nrows, k) : 0; }

int pgd_act_prep_dev(pgd_dev* dev, const float* x, int ldx, int nrows, int k, void* act) {
  return guard([&] {
    PGD_CHECK(dev && x && act && nrows > 0, kErrArg, "bad argument");
    PGD_CHECK(k % 64 == 0 && ldx >= k && ldx % 4 == 0, kErrShape, "activation width must be a multiple of 64");
    DeviceScope scope(dev);
    a8_act_prep(x, ldx, nrows, k, act, dev->stream);
  });
}

int pgd_matrix_gemv_act_dev(const pgd_matrix* m, const void* act, int nrows, float* y, int ldy, const float* res,
                            int ldres) {
  return guard([&] {
    PGD_CHECK(m && act && y && nrows > 0, kErrArg, "bad argument");
    PGD_CHECK(m->m.fmt == FMT_A8, kErrFormat, "prepared activations feed A8 matrices");
    PGD_CHECK(ldy >= m->m.n_out && (!res || ldres >= m->m.n_out), kErrShape, "gemv output stride");
    DeviceScope scope(m->dev);
    A8Act a = a8_act_view(const_cast<void*>(act), nrows, m->m.n_in);
    qmat_gemv_a8(m->m, a, y, ldy, res, ldres, m->dev->stream);
  });
}

int pgd_matrix_gemv_q8act_dev(const pgd_matrix* m, const float* x, int ldx, int nrows, float* y, int ldy,
                              const float* res, int ldres) {
  return guard([&] {
    PGD_CHECK(m && x && y && nrows > 0, kErrArg, "bad argument");
    PGD_CHECK(m->m.fmt != FMT_A8, kErrFormat, "quantized activations are for GGML-format matrices");
    PGD_CHECK(ldy >= m->m.n_out && (!res || ldres >= m->m.n_out), kErrShape, "gemv output stride");
    DeviceScope scope(m->dev);
    qmat_gemv_q8act(m->m, x, ldx, nrows, y, ldy, res, ldres, m->dev->stream);
  });
}

int pgd_matrix_gemv_q8act_pair_dev(const pgd_matrix* a, float* ya, const pgd_matrix* b, float* yb, const float* x,
                                   int ldx, int nrows, int ldy) {
  return guard([&] {
    PGD_CHECK(a && b && ya && yb && x && nrows > 0 && a->dev == b->dev, kErrArg, "bad argument");
    PGD_CHECK(a->m.n_in == b->m.n_in, kErrShape, "paired matrices need one input width");
    PGD_CHECK(qmat_q8act_pairable(a->m, b->m), kErrFormat, "paired matrices need one activation type");
    DeviceScope scope(a->dev);
    qmat_gemv_q8act_pair(a->m, ya, b->m, yb, x, ldx, nrows, ldy, a->dev->stream);
  });
}

int pgd_matrix_gemv_swiglu_act_dev(const pgd_matrix* gate, const pgd_matrix* up, const void* act, int nrows,
                                   float* mid, int ldm) {
  return guard([&] {
    PGD_CHECK(gate && up && act && mid && nrows > 0, kErrArg, "bad argument");
    PGD_CHECK(gate->dev == up->dev, kErrArg, "gate and up live on different devices");
    PGD_CHECK(ldm >= gate->m.n_out, kErrShape, "swiglu output stride");
    DeviceScope scope(gate->dev);
    A8Act a = a8_act_view(const_cast<void*>(act), nrows, gate->m.n_in);
    qmat_gemv_a8_swiglu(gate->m, up->m, a, mid, ldm, gate->dev->stream);
  });
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free A8 GEMV: the kernels' scratch (split-K and stream-K partial
// sums, per-row scales) comes from one fixed device array per GPU instead of
// the growing per-stream buffers, for callers that cannot allocate device
// memory (code under graph capture, tight serving loops).
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kScratchBytes = (size_t)40 << 20;
// host-side name of the per-GPU array; its device address comes from
// hipGetSymbolAddress on each device
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// One GPU's copy of scratch and its last user: calls queued on different
// streams are ordered through `done`, an event recorded after each call, so
// a call on another stream never overwrites partial sums still being read.
struct ScratchSlot {
  uint8_t* ptr = nullptr;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
};
std::mutex g_scratch_mu;
std::map<int, ScratchSlot> g_scratch;  // device ordinal -> that GPU's slot

// the current device's slot, set up once per device
ScratchSlot& scratch_on_current_device() {
  int dev = 0;
  PGD_HIP(hipGetDevice(&dev));
  auto it = g_scratch.find(dev);
  if (it != g_scratch.end()) return it->second;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  PGD_CHECK(e == hipSuccess && p, kErrState, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
  ScratchSlot sl;
  sl.ptr = static_cast<uint8_t*>(p);
  PGD_HIP(hipEventCreateWithFlags(&sl.done, hipEventDisableTiming));
  return g_scratch[dev] = sl;
}

struct ArenaScope {
  gemv::ScratchArena arena;
  gemv::ScratchArena* prev;
  explicit ArenaScope(uint8_t* base, size_t cap) {
    arena.base = base;
    arena.cap = cap;
    prev = gemv::set_scratch_arena(&arena);
  }
  ~ArenaScope() { gemv::set_scratch_arena(prev); }
};
}  // namespace

extern "C" {

size_t pgd_noalloc_scratch_bytes(void) { return kScratchBytes; }

int pgd_matrix_gemv_act_dev_noalloc(const pgd_matrix* m, const void* act, int nrows, float* y, int ldy,
                                    const float* res, int ldres) {
  return guard([&] {
    PGD_CHECK(m && act && y && nrows > 0, kErrArg, "bad argument");
    PGD_CHECK(m->m.fmt == FMT_A8, kErrFormat, "prepared activations feed A8 matrices");
    PGD_CHECK(ldy >= m->m.n_out && (!res || ldres >= m->m.n_out), kErrShape, "gemv output stride");
    const size_t need = qmat_gemv_a8_scratch(m->m, nrows, res != nullptr);
    PGD_CHECK(need <= kScratchBytes, kErrShape,
              std::to_string(nrows) + " rows of a " + std::to_string(m->m.n_out) + " x " + std::to_string(m->m.n_in) +
                  " matrix need " + std::to_string(need) + " bytes of scratch, above the fixed " +
                  std::to_string(kScratchBytes >> 20) + " MiB");
    DeviceScope scope(m->dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ScratchSlot& sl = scratch_on_current_device();
    hipStream_t st = m->dev->stream;
    // the previous call was queued on another stream: wait for it on the GPU
    if (sl.last && sl.last != st) PGD_HIP(hipStreamWaitEvent(st, sl.done, 0));
    ArenaScope arena(sl.ptr, kScratchBytes);
    A8Act a = a8_act_view(const_cast<void*>(act), nrows, m->m.n_in);
    qmat_gemv_a8(m->m, a, y, ldy, res, ldres, st);
    PGD_HIP(hipEventRecord(sl.done, st));
    sl.last = st;
  });
}

}  // extern "C"
