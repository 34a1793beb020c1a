// ops.hip — RMSNorm, causal conv step, Gated-DeltaNet recurrence, q/k/v
// preparation with paged KV writes and argmax (attention: attn.hip).
#include "common.h"
#include "ops.h"
#include "gemv_impl.h"

namespace pgd {

namespace {

// ---------------------------------------------------------------------------
// block reductions (256 threads = 4 waves)
// ---------------------------------------------------------------------------
__device__ inline float block_sum256(float v, float* red4) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red4[w] = v;
  __syncthreads();
  float t = red4[0] + red4[1] + red4[2] + red4[3];
  __syncthreads();
  return t;
}

// ---------------------------------------------------------------------------
// RMSNorm
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, int ldx, const int* rows_idx,
                                                      int n, const float* __restrict__ w, float eps, int mode,
                                                      float* __restrict__ y, int ldy) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const int src = rows_idx ? rows_idx[r] : r;
  const float* xr = x + (size_t)src * ldx;
  float ss = 0.0f;
  if (mode != 2) {
    for (int i = threadIdx.x; i < n; i += 256) ss += xr[i] * xr[i];
    ss = block_sum256(ss, red);
  } else {
    // candle's CPU rms_norm sums the squares left to right in f32; the same
    // order makes the normed values (and so their Q8 quantization, where an
    // embedding row's grid values can sit exactly on a rounding tie) agree
    // bit for bit. The squares are formed in parallel (each rounds the same
    // wherever it is computed) and staged in LDS; one lane adds them in order.
    __shared__ float sq[8192];
    for (int i = threadIdx.x; i < n; i += 256) sq[i] = xr[i] * xr[i];
    __syncthreads();
    if (threadIdx.x == 0) {
      int i = 0;
      for (; i + 4 <= n; i += 4) {
        const float4 v = *reinterpret_cast<const float4*>(sq + i);
        ss += v.x;
        ss += v.y;
        ss += v.z;
        ss += v.w;
      }
      for (; i < n; ++i) ss += sq[i];
      red[0] = ss;
    }
    __syncthreads();
    ss = red[0];
  }
  float* yr = y + (size_t)r * ldy;
  if (mode == 0) {
    float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) yr[i] = xr[i] * inv * w[i];
  } else {
    float m = sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) yr[i] = xr[i] / m * w[i];
  }
}

// ---------------------------------------------------------------------------
// causal conv step (sequential over a sequence's rows)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void conv_step_kernel(const float* __restrict__ x, int ldx, float* __restrict__ out,
                                                        int ldo, int channels, int kernel,
                                                        const float* __restrict__ weight, float* const* state_base,
                                                        size_t state_off, const int* row_start, const int* row_count) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int s = blockIdx.y;
  if (c >= channels) return;
  const int hist = kernel - 1;
  float* st = state_base[s] + state_off + (size_t)c * hist;
  float win[8];
  float wt[8];
  for (int k = 0; k < hist; ++k) win[k] = st[k];
  for (int k = 0; k < kernel; ++k) wt[k] = weight[(size_t)c * kernel + k];
  const int r0 = row_start[s], n = row_count[s];
  // inputs loaded eight rows ahead (the steps are sequential; the loads are not)
  constexpr int PF = 8;
  float xr[PF];
#pragma unroll
  for (int k = 0; k < PF; ++k) xr[k] = k < n ? x[(size_t)(r0 + k) * ldx + c] : 0.0f;
  for (int t = 0; t < n; ++t) {
    const float xv = xr[0];
#pragma unroll
    for (int k = 0; k + 1 < PF; ++k) xr[k] = xr[k + 1];
    xr[PF - 1] = t + PF < n ? x[(size_t)(r0 + t + PF) * ldx + c] : 0.0f;
    float acc = 0.0f;
    for (int k = 0; k < hist; ++k) acc += win[k] * wt[k];
    acc += xv * wt[hist];
    out[(size_t)(r0 + t) * ldo + c] = acc / (1.0f + expf(-acc));
    for (int k = 0; k + 1 < hist; ++k) win[k] = win[k + 1];
    if (hist > 0) win[hist - 1] = xv;
  }
  for (int k = 0; k < hist; ++k) st[k] = win[k];
}

// ---------------------------------------------------------------------------
// Gated-DeltaNet
// ---------------------------------------------------------------------------
// One workgroup per (value head, sequence); 256 threads. Thread (rg, cg)
// holds state rows 16rg..16rg+15, columns 4cg..4cg+3 in 64 registers for the
// whole sequence chunk. Column sums over rows (S^T k, S^T q) are folded
// through LDS across the 8 row groups.
__device__ inline float softplus_f(float x) {
  if (x > 20.0f) return x;
  if (x < -20.0f) return expf(x);
  return logf(1.0f + expf(x));
}

__global__ __launch_bounds__(256) void gdn_kernel(GdnParams p, const int* row_start, const int* row_count) {
  constexpr int D = 128;
  __shared__ float qs[D], ks[D], delta[D];
  __shared__ float red[8][D];
  __shared__ float part[4];
  __shared__ float obuf[D];
  const int h = blockIdx.x, s = blockIdx.y, tid = threadIdx.x;
  const int cg = tid & 31, rg = tid >> 5;
  const int repeat = p.v_heads / p.k_heads;
  const int kh = h / repeat;
  const int key_dim = p.k_heads * D;
  float* st = p.state_base[s] + p.state_off + (size_t)h * D * D;
  float S[16][4];
#pragma unroll
  for (int ii = 0; ii < 16; ++ii) {
    float4 v = *reinterpret_cast<const float4*>(st + (size_t)(16 * rg + ii) * D + 4 * cg);
    S[ii][0] = v.x;
    S[ii][1] = v.y;
    S[ii][2] = v.z;
    S[ii][3] = v.w;
  }
  const float a_log = p.a_log[h], dtb = p.dt_bias[h];
  const float qscale = sqrtf((float)D);
  const int r0 = row_start[s], n = row_count[s];
  // the gate input z and the norm weight are loaded with the step's other
  // inputs, not after the reductions that need them
  const float nw = tid < D ? p.norm[tid] : 0.0f;
  // a step's inputs (gate z, v, this thread's q or k element, the a / b gate
  // inputs) are loaded one step ahead, so a prefill's sequential steps do
  // not wait for memory each
  struct In {
    float zg, vv, v, ar, br;
  };
  auto load_in = [&](int row) {
    const float* cv = p.conv_out + (size_t)row * p.ld_conv;
    In x;
    x.zg = tid < D ? p.z[(size_t)row * p.ld_z + h * D + tid] : 0.0f;
    x.vv = tid < D ? cv[2 * key_dim + h * D + tid] : 0.0f;
    x.v = tid < D ? cv[kh * D + tid] : cv[key_dim + kh * D + (tid - D)];
    x.ar = p.a[(size_t)row * p.ld_ab + h];
    x.br = p.b[(size_t)row * p.ld_ab + h];
    return x;
  };
  In nxt = load_in(r0);
  for (int t = 0; t < n; ++t) {
    const int row = r0 + t;
    const In cur = nxt;
    if (t + 1 < n) nxt = load_in(row + 1);
    const float zg = cur.zg, vv = cur.vv;
    // q (threads 0..127) and k (128..255), L2-normalized per head
    float v = cur.v;
    float ss = wave_sum(v * v);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    if (tid < D) {
      float inv = 1.0f / sqrtf(part[0] + part[1] + 1e-6f);
      qs[tid] = (v * inv) / qscale;
    } else {
      float inv = 1.0f / sqrtf(part[2] + part[3] + 1e-6f);
      ks[tid - D] = v * inv;
    }
    const float g = -expf(a_log) * softplus_f(cur.ar + dtb);
    const float decay = expf(g);
    const float beta = 1.0f / (1.0f + expf(-cur.br));
    __syncthreads();
    // S *= decay; mem = S^T k (partial over this thread's 16 rows)
    float m4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) {
      const float kv = ks[16 * rg + ii];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        S[ii][c] = S[ii][c] * decay;
        m4[c] += S[ii][c] * kv;
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) red[rg][4 * cg + c] = m4[c];
    __syncthreads();
    if (tid < D) {
      float mem = 0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q) mem += red[q][tid];
      delta[tid] = (vv - mem) * beta;
    }
    __syncthreads();
    // S += k delta^T ; o = S^T q (partial)
    float o4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float dl[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) dl[c] = delta[4 * cg + c];
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) {
      const float kv = ks[16 * rg + ii], qv = qs[16 * rg + ii];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        S[ii][c] = S[ii][c] + kv * dl[c];
        o4[c] += S[ii][c] * qv;
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) red[rg][4 * cg + c] = o4[c];
    __syncthreads();
    // gated RMSNorm over the head (qwen3_5.rs:1747-1756)
    float o = 0.0f;
    if (tid < D) {
#pragma unroll
      for (int q = 0; q < 8; ++q) o += red[q][tid];
    }
    float oss = wave_sum(tid < D ? o * o : 0.0f);
    if ((tid & 63) == 0) part[tid >> 6] = oss;
    __syncthreads();
    if (tid < D) {
      const float inv = 1.0f / sqrtf((part[0] + part[1]) / (float)D + 1e-6f);
      const float val = o * inv * nw * (zg / (1.0f + expf(-zg)));
      if (p.out) p.out[(size_t)row * p.ld_out + h * D + tid] = val;
      obuf[tid] = val;
    }
    __syncthreads();
    if (p.act.XA && tid < D / 16) {
      // the head's 128 outputs are two whole groups of the out projection's input
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = obuf[16 * tid + e];
      a8act::emit_slice(p.act, row, (h * D + 16 * tid) >> 6, tid & 3, v, true);
    }
    __syncthreads();
  }
#pragma unroll
  for (int ii = 0; ii < 16; ++ii)
    *reinterpret_cast<float4*>(st + (size_t)(16 * rg + ii) * D + 4 * cg) = make_float4(S[ii][0], S[ii][1], S[ii][2], S[ii][3]);
}

// ---------------------------------------------------------------------------
// q/k/v preparation + paged KV write; one wave per (head or kv head, row)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void qkv_prep_kernel(QkvPrep p, AttnLayout L, RowMeta m) {
  __shared__ float buf[512];
  const int r = blockIdx.y;
  const int hidx = blockIdx.x;
  const int lane = threadIdx.x;
  const int hd = L.head_dim, rd = L.rotary_dim, half = rd / 2;
  const int E = hd / 64;
  const bool is_q = hidx < L.heads;
  const int h = is_q ? hidx : hidx - L.heads;
  const float* src;
  const float* bias = nullptr;
  const float* nw = nullptr;
  if (is_q) {
    src = p.q_raw + (size_t)r * p.ld_q + (size_t)h * hd * (p.variant == 0 ? 2 : 1);
    bias = p.variant == 1 ? p.q_bias + (size_t)h * hd : nullptr;
    nw = p.variant == 0 ? p.q_norm : nullptr;
  } else {
    src = p.k_raw + (size_t)r * p.ld_kv + (size_t)h * hd;
    bias = p.variant == 1 ? p.k_bias + (size_t)h * hd : nullptr;
    nw = p.variant == 0 ? p.k_norm : nullptr;
  }
  float v[4], cs_v[4], sn_v[4];
  float ss = 0.0f;
  // the RoPE table entries are loaded with the row (one round trip)
  const float* cs = m.cos + (size_t)r * rd;
  const float* sn = m.sin + (size_t)r * rd;
  for (int e = 0; e < E; ++e) {
    const int d = lane + 64 * e;
    v[e] = src[d];
    cs_v[e] = d < rd ? cs[d] : 0.0f;
    sn_v[e] = d < rd ? sn[d] : 0.0f;
    if (bias) v[e] = v[e] + bias[d];
    ss += v[e] * v[e];
  }
  if (nw) {
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)hd + 1e-6f);
    for (int e = 0; e < E; ++e) v[e] = v[e] * inv * nw[lane + 64 * e];
  }
  for (int e = 0; e < E; ++e) buf[lane + 64 * e] = v[e];
  __syncthreads();
  for (int e = 0; e < E; ++e) {
    const int d = lane + 64 * e;
    if (d < rd) {
      const float rot = d < half ? -buf[d + half] : buf[d - half];
      v[e] = buf[d] * cs_v[e] + rot * sn_v[e];
    }
  }
  if (is_q) {
    float* qd = p.q + ((size_t)r * L.heads + h) * hd;
    for (int e = 0; e < E; ++e) qd[lane + 64 * e] = v[e];
    if (p.variant == 0) {
      float* gd = p.gate + ((size_t)r * L.heads + h) * hd;
      for (int e = 0; e < E; ++e) gd[lane + 64 * e] = src[hd + lane + 64 * e];
    }
  } else {
    const int seq = m.seq_of_row[r], pos = m.pos_of_row[r];
    const int blk = m.block_tables[(size_t)seq * m.max_blocks + pos / L.block];
    const size_t off = (((size_t)blk * L.kv_heads + h) * L.block + (pos % L.block)) * hd;
    const float* vs = p.v_raw + (size_t)r * p.ld_kv + (size_t)h * hd;
    const float* vb = p.variant == 1 ? p.v_bias + (size_t)h * hd : nullptr;
    for (int e = 0; e < E; ++e) {
      const int d = lane + 64 * e;
      L.k_pool[off + d] = v[e];
      L.v_pool[off + d] = vb ? vs[d] + vb[d] : vs[d];
    }
  }
}


// ---------------------------------------------------------------------------
// argmax
// ---------------------------------------------------------------------------
__device__ inline bool better(float v, int i, float bv, int bi, int last_max) {
  if (bi < 0) return true;
  if (v > bv) return true;
  if (v < bv) return false;
  return last_max ? i > bi : i < bi;
}

// Row argmax in two passes: kArgChunks workgroups per row each reduce one
// contiguous chunk, then one wave per row merges the chunk winners. better()
// is a total order on (value, index), so the merge order does not matter.
constexpr int kArgChunks = 64;
struct ArgPart {
  float v;
  int i, nf;
};

__device__ inline void arg_merge(float& bv, int& bi, int& nf, float v, int i, int n2, int last_max) {
  if (i >= 0 && better(v, i, bv, bi, last_max)) {
    bv = v;
    bi = i;
  }
  nf += n2;
}

__global__ __launch_bounds__(256) void argmax_part_kernel(const float* __restrict__ x, int ld, int n, int last_max,
                                                          ArgPart* __restrict__ part) {
  __shared__ ArgPart sp[4];
  const int r = blockIdx.y, b = blockIdx.x, tid = threadIdx.x;
  const int len = (n + kArgChunks - 1) / kArgChunks;
  const int lo = b * len, hi = min(n, lo + len);
  const float* xr = x + (size_t)r * ld;
  float bv = -INFINITY;
  int bi = -1, nf = 0;
  for (int i = lo + tid; i < hi; i += 256) {
    const float v = xr[i];
    if (!isfinite(v)) nf++;
    else if (better(v, i, bv, bi, last_max)) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v = __shfl_xor(bv, o, 64);
    const int i = __shfl_xor(bi, o, 64);
    const int f = __shfl_xor(nf, o, 64);
    arg_merge(bv, bi, nf, v, i, f, last_max);
  }
  if ((tid & 63) == 0) sp[tid >> 6] = ArgPart{bv, bi, nf};
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) arg_merge(bv, bi, nf, sp[w].v, sp[w].i, sp[w].nf, last_max);
    part[(size_t)r * kArgChunks + b] = ArgPart{bv, bi, nf};
  }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const ArgPart* __restrict__ part, int last_max,
                                                          uint32_t* ids, float* vals, int* nonfinite) {
  const int r = blockIdx.x, lane = threadIdx.x;
  ArgPart p = part[(size_t)r * kArgChunks + lane];
  float bv = p.v;
  int bi = p.i, nf = p.nf;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v = __shfl_xor(bv, o, 64);
    const int i = __shfl_xor(bi, o, 64);
    const int f = __shfl_xor(nf, o, 64);
    arg_merge(bv, bi, nf, v, i, f, last_max);
  }
  if (lane == 0) {
    ids[r] = bi < 0 ? 0xFFFFFFFFu : (uint32_t)bi;
    if (vals) vals[r] = bv;
    if (nonfinite) nonfinite[r] = nf;
  }
}

__global__ void gather_kernel(const float* src, int lds, const int* idx, int n, float* dst, int ldd) {
  const int r = blockIdx.y;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[(size_t)r * ldd + i] = src[(size_t)idx[r] * lds + i];
}

}  // namespace

// ---------------------------------------------------------------------------
void rmsnorm_rows(const float* x, int ldx, const int* rows_idx, int rows, int n, const float* w, float eps, int mode,
                  float* y, int ldy, hipStream_t s) {
  if (rows <= 0) return;
  PGD_CHECK(mode != 2 || n <= 8192, kErrShape, "ordered-sum RMSNorm rows are at most 8192 wide");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, s, x, ldx, rows_idx, n, w, eps, mode, y, ldy);
  PGD_HIP(hipGetLastError());
}

void conv_step(const float* x, int ldx, float* out, int ldo, int channels, int kernel, const float* weight,
               float* const* state_base, size_t state_off, SeqMeta meta, int nseq, hipStream_t s) {
  PGD_CHECK(kernel >= 1 && kernel <= 8, kErrShape, "conv kernel must be in 1..8");
  if (nseq <= 0) return;
  hipLaunchKernelGGL(conv_step_kernel, dim3((channels + 255) / 256, nseq), dim3(256), 0, s, x, ldx, out, ldo, channels,
                     kernel, weight, state_base, state_off, meta.row_start, meta.row_count);
  PGD_HIP(hipGetLastError());
}

void gdn_step(const GdnParams& p, SeqMeta meta, int nseq, hipStream_t s) {
  PGD_CHECK(p.k_dim == 128 && p.v_dim == 128, kErrShape, "gated delta kernel needs k_dim == v_dim == 128");
  PGD_CHECK(p.k_heads > 0 && p.v_heads % p.k_heads == 0, kErrShape, "v_heads must be a multiple of k_heads");
  if (nseq <= 0) return;
  hipLaunchKernelGGL(gdn_kernel, dim3(p.v_heads, nseq), dim3(256), 0, s, p, meta.row_start, meta.row_count);
  PGD_HIP(hipGetLastError());
}

void qkv_prep(const QkvPrep& p, const AttnLayout& L, const RowMeta& m, int rows, hipStream_t s) {
  PGD_CHECK(L.head_dim % 64 == 0 && L.head_dim <= 256, kErrShape, "head_dim must be 64, 128, 192 or 256");
  PGD_CHECK(L.rotary_dim % 2 == 0 && L.rotary_dim <= L.head_dim, kErrShape, "rotary_dim");
  if (rows <= 0) return;
  hipLaunchKernelGGL(qkv_prep_kernel, dim3(L.heads + L.kv_heads, rows), dim3(64), 0, s, p, L, m);
  PGD_HIP(hipGetLastError());
}

void argmax_rows(const float* x, int ld, int rows, int n, int last_max, uint32_t* ids, float* vals, int* nonfinite,
                 hipStream_t s) {
  if (rows <= 0) return;
  static_assert(kArgChunks == 64, "one wave merges the chunks");
  auto* part = static_cast<ArgPart*>(gemv::gemv_scratch(s, (size_t)rows * kArgChunks * sizeof(ArgPart)));
  hipLaunchKernelGGL(argmax_part_kernel, dim3(kArgChunks, rows), dim3(256), 0, s, x, ld, n, last_max, part);
  hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, s, part, last_max, ids, vals, nonfinite);
  PGD_HIP(hipGetLastError());
}

void gather_rows(const float* src, int lds, const int* idx, int rows, int n, float* dst, int ldd, hipStream_t s) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(gather_kernel, dim3((n + 255) / 256, rows), dim3(256), 0, s, src, lds, idx, n, dst, ldd);
  PGD_HIP(hipGetLastError());
}

}  // namespace pgd
