// ops.hip — RMSNorm, causal conv step, Gated-DeltaNet recurrence, q/k/v
// preparation with paged KV writes and argmax (attention: attn.hip).
#include "common.h"
#include "ops.h"
#include "gemv_impl.h"

namespace pgd {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

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
// The output of row t reads inputs t-k+1..t only (earlier rows' inputs come
// from the state), so a sequence is cut into segments of kConvSeg rows along
// grid z; each thread runs one channel through one segment. Segment 0 alone
// reads the old state and alone writes the new one (the last k-1 inputs of
// old state ++ x), so no segment reads a state another has rewritten.
constexpr int kConvSeg = 64;

// KW: the conv kernel length (a compile-time constant, so the window lives in
// registers rather than in per-lane scratch memory)
template <int KW>
__global__ __launch_bounds__(256) void conv_step_kernel(const float* __restrict__ x, int ldx, float* __restrict__ out,
                                                        int ldo, int channels, const float* __restrict__ weight,
                                                        float* const* state_base, size_t state_off,
                                                        const int* row_start, const int* row_count) {
  constexpr int kernel = KW;
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int s = blockIdx.y;
  if (c >= channels) return;
  const int r0 = row_start[s], n = row_count[s];
  const int t_beg = blockIdx.z * kConvSeg;
  if (t_beg >= n && (blockIdx.z > 0 || n > 0)) return;
  const int t_end = gridDim.z == 1 ? n : min(n, t_beg + kConvSeg);
  constexpr int hist = kernel - 1, HA = hist > 0 ? hist : 1;
  float* st = state_base[s] + state_off + (size_t)c * hist;
  float win[HA];
  float wt[kernel];
  float old[HA];
#pragma unroll
  for (int k = 0; k < hist; ++k) {
    // window before row t_beg: inputs t_beg-hist..t_beg-1, from the state before row 0
    const int t = t_beg - hist + k;
    win[k] = t < 0 ? st[hist + t] : x[(size_t)(r0 + t) * ldx + c];
  }
  const bool whole = gridDim.z == 1;  // this thread runs every row: the last window is the new state
  if (!whole)
#pragma unroll
    for (int k = 0; k < hist; ++k) old[k] = win[k];
#pragma unroll
  for (int k = 0; k < kernel; ++k) wt[k] = weight[(size_t)c * kernel + k];
  // inputs loaded eight rows ahead (the steps are sequential; the loads are not)
  constexpr int PF = 8;
  float xr[PF];
#pragma unroll
  for (int k = 0; k < PF; ++k) xr[k] = t_beg + k < t_end ? x[(size_t)(r0 + t_beg + k) * ldx + c] : 0.0f;
  for (int t = t_beg; t < t_end; ++t) {
    const float xv = xr[0];
#pragma unroll
    for (int k = 0; k + 1 < PF; ++k) xr[k] = xr[k + 1];
    xr[PF - 1] = t + PF < t_end ? x[(size_t)(r0 + t + PF) * ldx + c] : 0.0f;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < hist; ++k) acc += win[k] * wt[k];
    acc += xv * wt[hist];
    out[(size_t)(r0 + t) * ldo + c] = acc / (1.0f + expf(-acc));
#pragma unroll
    for (int k = 0; k + 1 < hist; ++k) win[k] = win[k + 1];
    if constexpr (hist > 0) win[hist - 1] = xv;
  }
  if (whole) {
#pragma unroll
    for (int k = 0; k < hist; ++k) st[k] = win[k];
    return;
  }
  if (blockIdx.z != 0) return;
#pragma unroll
  for (int k = 0; k < hist; ++k) {
    // new state: inputs n-hist..n-1 of old state ++ x (old[] picked with
    // compile-time indices, so it stays in registers)
    const int t = n - hist + k;
    float v = 0.0f;
    if (t < 0) {
#pragma unroll
      for (int jj = 0; jj < hist; ++jj)
        if (jj == hist + t) v = old[jj];
    } else {
      v = x[(size_t)(r0 + t) * ldx + c];
    }
    st[k] = v;
  }
}

// ---------------------------------------------------------------------------
// Gated-DeltaNet
// ---------------------------------------------------------------------------
// One workgroup per (value head, sequence) of 32 RG threads. Thread (rg, cg)
// holds state rows RPT rg .. RPT rg + RPT - 1 (RPT = 128 / RG), columns
// 4cg..4cg+3 in registers for the whole sequence chunk. Column sums over rows
// (S^T k, S^T q) are folded through LDS across the RG row groups, in order.
// RG = 16 (512 threads, 32 state registers each) measured ~3% faster than 8
// at 1..64 sequences and 32 much slower from 32 sequences on (16 waves per
// workgroup, one workgroup per compute unit).
__device__ inline float softplus_f(float x) {
  if (x > 20.0f) return x;
  if (x < -20.0f) return expf(x);
  return logf(1.0f + expf(x));
}

constexpr int kGdnRowGroups = 16;

template <int RG>
__global__ __launch_bounds__(32 * RG) void gdn_kernel(GdnParams p, const int* row_start, const int* row_count) {
  constexpr int D = 128, RPT = D / RG;  // row groups, rows per thread
  __shared__ float qs[D], ks[D], delta[D];
  __shared__ float red[RG][D];
  __shared__ float part[4];
  __shared__ float obuf[D];
  const int h = blockIdx.x, s = blockIdx.y, tid = threadIdx.x;
  const int cg = tid & 31, rg = tid >> 5;
  const int repeat = p.v_heads / p.k_heads;
  const int kh = h / repeat;
  const int key_dim = p.k_heads * D;
  float* st = p.state_base[s] + p.state_off + (size_t)h * D * D;
  float S[RPT][4];
#pragma unroll
  for (int ii = 0; ii < RPT; ++ii) {
    float4 v = *reinterpret_cast<const float4*>(st + (size_t)(RPT * rg + ii) * D + 4 * cg);
    S[ii][0] = v.x;
    S[ii][1] = v.y;
    S[ii][2] = v.z;
    S[ii][3] = v.w;
  }
  const float a_log = p.a_log[h], dtb = p.dt_bias[h];
  const float qscale = sqrtf((float)D);
  const int r0 = row_start[s], n = row_count[s];
  if (p.o_raw && n >= kGdnLongRows) return;  // gdn_chunk_kernel's
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
    x.v = tid < D ? cv[kh * D + tid] : tid < 2 * D ? cv[key_dim + kh * D + (tid - D)] : 0.0f;
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
    if ((tid & 63) == 0 && tid < 2 * D) part[tid >> 6] = ss;
    __syncthreads();
    if (tid < D) {
      float inv = 1.0f / sqrtf(part[0] + part[1] + 1e-6f);
      qs[tid] = (v * inv) / qscale;
    } else if (tid < 2 * D) {
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
    for (int ii = 0; ii < RPT; ++ii) {
      const float kv = ks[RPT * rg + ii];
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
      for (int q = 0; q < RG; ++q) mem += red[q][tid];
      delta[tid] = (vv - mem) * beta;
    }
    __syncthreads();
    // S += k delta^T ; o = S^T q (partial)
    float o4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float dl[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) dl[c] = delta[4 * cg + c];
#pragma unroll
    for (int ii = 0; ii < RPT; ++ii) {
      const float kv = ks[RPT * rg + ii], qv = qs[RPT * rg + ii];
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
      for (int q = 0; q < RG; ++q) o += red[q][tid];
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
  for (int ii = 0; ii < RPT; ++ii)
    *reinterpret_cast<float4*>(st + (size_t)(RPT * rg + ii) * D + 4 * cg) = make_float4(S[ii][0], S[ii][1], S[ii][2], S[ii][3]);
}

// Prefill form of the recurrence, chunkwise (the published chunked form of
// the gated delta rule, in exact arithmetic the same recurrence). Over a
// chunk of m tokens from state S0, with G_t the running sum of the log decay
// g from the chunk start, gamma_t = exp(G_t), and the sequential recurrence
// S_t = a_t S_{t-1} + k_t d_t^T, d_t = beta_t (v_t - (a_t S_{t-1})^T k_t):
//   d_t = U_t - sum_{i<t} L_ti d_i,  U_t = beta_t (v_t - gamma_t S0^T k_t),
//                                    L_ti = beta_t exp(G_t - G_i) (k_t . k_i)
//   o_t = gamma_t S0^T q_t + sum_{i<=t} exp(G_t - G_i) (q_t . k_i) d_i
//   S_m = gamma_m S0 + sum_i exp(G_m - G_i) k_i d_i^T
// (every decay factor exp(G_t - G_i) with t >= i is at most 1). A column of S
// (one value dimension) evolves on its own, so a head's 128 columns are split
// over kGdnColGroups workgroups (grid x = value head * groups + group), each
// holding its 128 x 32 slice of S in LDS and repeating the 32 x 32 token
// products. q and k are L2 normalized per token as in the step kernel and
// kept transposed ([k index][token]) for float4 reads in the register-blocked
// products. The recurrence outputs go to o_raw; gdn_norm_kernel applies the
// gated RMSNorm.
constexpr int kGdnColGroups = 4;
constexpr int kGdnCols = 128 / kGdnColGroups;                  // 32 columns of S per workgroup
constexpr int kGdnCP = kGdnCols + 4, kGdnTP = kGdnChunk + 4;  // padded LDS row strides
constexpr size_t kGdnChunkLds =
    (size_t)(3 * 128 * kGdnTP + 2 * kGdnChunk * kGdnCP + 2 * kGdnChunk * kGdnTP + 2 * kGdnChunk) * sizeof(float);

__global__ __launch_bounds__(256) void gdn_chunk_kernel(GdnParams p, const int* row_start, const int* row_count) {
  constexpr int D = 128, C = kGdnChunk, NCOL = kGdnCols, CP = kGdnCP, TP = kGdnTP;
  static_assert(C == 32 && NCOL == 32 && CP == TP, "thread mappings assume 32 tokens x 32 columns");
  extern __shared__ __attribute__((aligned(16))) float gsm[];
  float* S = gsm;            // [D][CP]  this group's columns of the state (k index major)
  float* KT = S + D * CP;    // [D][TP]  normalized k, transposed
  float* QT = KT + D * TP;   // [D][TP]  normalized, scaled q, transposed
  float* Uc = QT + D * TP;   // [C][CP]  v, then U, then exp(G_m - G_i) d_i
  float* Zc = Uc + C * CP;   // [C][CP]  gamma_t S0^T q_t
  float* Lm = Zc + C * CP;   // [C][TP]
  float* Bm = Lm + C * TP;   // [C][TP]
  float* Gs = Bm + C * TP;   // [C] running log decay
  float* Bs = Gs + C;        // [C] beta
  const int h = blockIdx.x / kGdnColGroups, col0 = (blockIdx.x % kGdnColGroups) * NCOL;
  const int s = blockIdx.y, tid = threadIdx.x;
  const int n = row_count[s];
  if (n < kGdnLongRows) return;
  const int r0 = row_start[s];
  const int repeat = p.v_heads / p.k_heads, kh = h / repeat, key_dim = p.k_heads * D;
  const int ldo = p.v_heads * D;
  float* st = p.state_base[s] + p.state_off + (size_t)h * D * D + col0;
  for (int i = tid; i < D * NCOL / 4; i += 256)
    *reinterpret_cast<float4*>(S + (i >> 3) * CP + (i & 7) * 4) =
        *reinterpret_cast<const float4*>(st + (size_t)(i >> 3) * D + (i & 7) * 4);
  const float a_log = p.a_log[h], dtb = p.dt_bias[h];
  const float qscale = sqrtf((float)D);
  const int c = tid & (NCOL - 1), tq = tid >> 5;  // column phases: column c, tokens 4 tq ..
  // a chunk's q, k (token (tid / 32) + 8 jj, elements 4 (tid % 32)..) and v
  // (token tid / 8, columns 4 (tid % 8)..) in registers, loaded one chunk
  // ahead so that no chunk waits for its inputs; zeros past the sequence
  float4 qn[4], kn[4], vn;
  auto load_chunk = [&](int tc) {
    const int mc = min(C, n - tc);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int t = (tid >> 5) + 8 * jj, e = (tid & 31) * 4;
      qn[jj] = make_float4(0.f, 0.f, 0.f, 0.f);
      kn[jj] = qn[jj];
      if (t < mc) {
        const float* cv = p.conv_out + (size_t)(r0 + tc + t) * p.ld_conv;
        qn[jj] = *reinterpret_cast<const float4*>(cv + kh * D + e);
        kn[jj] = *reinterpret_cast<const float4*>(cv + key_dim + kh * D + e);
      }
    }
    const int t = tid >> 3, e = (tid & 7) * 4;
    vn = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < mc)
      vn = *reinterpret_cast<const float4*>(p.conv_out + (size_t)(r0 + tc + t) * p.ld_conv + 2 * key_dim + h * D +
                                            col0 + e);
  };
  load_chunk(0);

  for (int t0 = 0; t0 < n; t0 += C) {
    const int m = min(C, n - t0);
    __syncthreads();  // the previous chunk is done with every buffer
    // q and k of the chunk (zeros past m): 32 lanes per token, 4 elements each
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int t = (tid >> 5) + 8 * jj, e = (tid & 31) * 4;
      const float4 q4 = qn[jj], k4 = kn[jj];
      float sq = q4.x * q4.x + q4.y * q4.y + q4.z * q4.z + q4.w * q4.w;
      float sk = k4.x * k4.x + k4.y * k4.y + k4.z * k4.z + k4.w * k4.w;
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) {
        sq += __shfl_xor(sq, o, 64);
        sk += __shfl_xor(sk, o, 64);
      }
      const float iq = 1.0f / sqrtf(sq + 1e-6f), ik = 1.0f / sqrtf(sk + 1e-6f);
      QT[(e + 0) * TP + t] = (q4.x * iq) / qscale;
      QT[(e + 1) * TP + t] = (q4.y * iq) / qscale;
      QT[(e + 2) * TP + t] = (q4.z * iq) / qscale;
      QT[(e + 3) * TP + t] = (q4.w * iq) / qscale;
      KT[(e + 0) * TP + t] = k4.x * ik;
      KT[(e + 1) * TP + t] = k4.y * ik;
      KT[(e + 2) * TP + t] = k4.z * ik;
      KT[(e + 3) * TP + t] = k4.w * ik;
    }
    {
      // v of this group's columns: token tid / 8, 4 columns
      const int t = tid >> 3, e = (tid & 7) * 4;
      *reinterpret_cast<float4*>(Uc + t * CP + e) = vn;
    }
    if (t0 + C < n) load_chunk(t0 + C);
    if (tid < 64) {
      // decay and beta per token, then the running sum of the log decay
      float g = 0.f, beta = 0.f;
      if (tid < m) {
        const size_t row = (size_t)(r0 + t0 + tid) * p.ld_ab + h;
        g = -expf(a_log) * softplus_f(p.a[row] + dtb);
        beta = 1.0f / (1.0f + expf(-p.b[row]));
      }
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) {
        const float y = __shfl_up(g, o, 64);
        if ((tid & 31) >= o) g += y;
      }
      if (tid < C) {
        Gs[tid] = g;
        Bs[tid] = beta;
      }
    }
    __syncthreads();
    // fp32 MFMA tiles (v_mfma_f32_16x16x4_f32): lane l supplies A[row l % 16]
    // [k l / 16] and B[k l / 16][col l % 16] and holds D[4 (l / 16) + r][l % 16].
    const int lane = tid & 63, wave = tid >> 6, lr = lane & 15, lk = lane >> 4;
    {
      // L (t x i, i < t) and B (i <= t) from K K^T and Q K^T over the 128 k:
      // waves 0..2 take the three nonzero 16x16 tiles of both, wave 3 writes
      // the zero tile above the diagonal
      if (wave < 3) {
        const int tb = wave == 0 ? 0 : 16, ib = wave == 2 ? 16 : 0;
        f4 aL = {0.f, 0.f, 0.f, 0.f}, aB = aL;
#pragma unroll 8
        for (int k0 = 0; k0 < D; k0 += 4) {
          const float* kr = KT + (k0 + lk) * TP;
          const float ki = kr[ib + lr];
          aL = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[tb + lr], ki, aL, 0, 0, 0);
          aB = __builtin_amdgcn_mfma_f32_16x16x4f32(QT[(k0 + lk) * TP + tb + lr], ki, aB, 0, 0, 0);
        }
        const int i = ib + lr;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = tb + 4 * lk + r;
          float vl = 0.f, vb = 0.f;
          if (t < m && i <= t) {
            const float w = expf(Gs[t] - Gs[i]);
            vb = w * aB[r];
            if (i < t) vl = Bs[t] * (w * aL[r]);
          }
          Lm[t * TP + i] = vl;
          Bm[t * TP + i] = vb;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 4 * lk + r, i = 16 + lr;
          Lm[t * TP + i] = 0.f;
          Bm[t * TP + i] = 0.f;
        }
      }
    }
    {
      // W = K S0 and Z = Q S0: wave w takes tokens 16 (w / 2).., columns
      // 16 (w % 2)..; then U = beta (v - gamma W) and gamma Z
      const int tb = 16 * (wave >> 1), cb = 16 * (wave & 1);
      f4 aW = {0.f, 0.f, 0.f, 0.f}, aZ = aW;
#pragma unroll 8
      for (int k0 = 0; k0 < D; k0 += 4) {
        const float sv = S[(k0 + lk) * CP + cb + lr];
        aW = __builtin_amdgcn_mfma_f32_16x16x4f32(KT[(k0 + lk) * TP + tb + lr], sv, aW, 0, 0, 0);
        aZ = __builtin_amdgcn_mfma_f32_16x16x4f32(QT[(k0 + lk) * TP + tb + lr], sv, aZ, 0, 0, 0);
      }
      const int cc = cb + lr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = tb + 4 * lk + r;
        const float gam = expf(Gs[t]), bet = Bs[t];
        Uc[t * CP + cc] = bet * (Uc[t * CP + cc] - gam * aW[r]);
        Zc[t * CP + cc] = gam * aZ[r];
      }
    }
    __syncthreads();
    // d = (I + L)^-1 U for column c, in registers (every thread of the column
    // solves it; L is zero on and above the diagonal and past the chunk)
    float d[C];
#pragma unroll
    for (int t = 0; t < C; ++t) d[t] = Uc[t * CP + c];
#pragma unroll
    for (int t = 1; t < C; ++t) {
      float acc = d[t];
#pragma unroll
      for (int i = 0; i < t; ++i) acc = fmaf(-Lm[t * TP + i], d[i], acc);
      d[t] = acc;
    }
    // outputs of tokens 4 tq .. for column c: B is zero above the diagonal
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 4 * tq + j;
      float o = Zc[t * CP + c];
#pragma unroll
      for (int i4 = 0; i4 < C; i4 += 4) {
        const float4 b4 = *reinterpret_cast<const float4*>(Bm + t * TP + i4);
        o = fmaf(b4.x, d[i4], o);
        o = fmaf(b4.y, d[i4 + 1], o);
        o = fmaf(b4.z, d[i4 + 2], o);
        o = fmaf(b4.w, d[i4 + 3], o);
      }
      if (t < m && r0 + t0 + t < p.o_rows) p.o_raw[(size_t)(r0 + t0 + t) * ldo + h * D + col0 + c] = o;
    }
    const float gl = Gs[m - 1];
#pragma unroll
    for (int i = 0; i < C; ++i) d[i] = i < m ? expf(gl - Gs[i]) * d[i] : 0.f;
    __syncthreads();  // every column's U is read
    if (tq == 0) {
#pragma unroll
      for (int i = 0; i < C; ++i) Uc[i * CP + c] = d[i];
    }
    __syncthreads();
    {
      // S = gamma_m S0 + K^T (weighted d): wave w takes k rows 32 w .. 32 w + 31
      // (two 16-row tiles) by both 16-column tiles, 8 MFMA steps over the tokens
      const float gm = expf(gl);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          const int kb = 32 * wave + 16 * kt, cb = 16 * ct;
          f4 acc;
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = gm * S[(kb + 4 * lk + r) * CP + cb + lr];
#pragma unroll
          for (int i0 = 0; i0 < C; i0 += 4)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(KT[(kb + lr) * TP + i0 + lk], Uc[(i0 + lk) * CP + cb + lr], acc,
                                                       0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) S[(kb + 4 * lk + r) * CP + cb + lr] = acc[r];
        }
    }
  }
  __syncthreads();
  for (int i = tid; i < D * NCOL / 4; i += 256)
    *reinterpret_cast<float4*>(st + (size_t)(i >> 3) * D + (i & 7) * 4) =
        *reinterpret_cast<const float4*>(S + (i >> 3) * CP + (i & 7) * 4);
}

// Gated RMSNorm of the chunkwise outputs (rows of long sequences only),
// exactly the step kernel's tail: out and / or the prepared activations.
__device__ inline void gdn_norm_row(const GdnParams& p, int row, int h, int tid, float* part, float* obuf) {
  constexpr int D = 128;
  const float o = p.o_raw[(size_t)row * p.v_heads * D + h * D + tid];
  const float zg = p.z[(size_t)row * p.ld_z + h * D + tid];
  const float oss = wave_sum(o * o);
  if ((tid & 63) == 0) part[tid >> 6] = oss;
  __syncthreads();
  const float inv = 1.0f / sqrtf((part[0] + part[1]) / (float)D + 1e-6f);
  const float val = o * inv * p.norm[tid] * (zg / (1.0f + expf(-zg)));
  if (p.out) p.out[(size_t)row * p.ld_out + h * D + tid] = val;
  obuf[tid] = val;
  __syncthreads();
  if (p.act.XA && tid < D / 16) {
    float v[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = obuf[16 * tid + e];
    a8act::emit_slice(p.act, row, (h * D + 16 * tid) >> 6, tid & 3, v, true);
  }
}

// grid (row blocks, sequence, value head); a workgroup strides over its
// sequence's rows
__global__ __launch_bounds__(128) void gdn_norm_kernel(GdnParams p, const int* row_start, const int* row_count) {
  __shared__ float part[2];
  __shared__ float obuf[128];
  const int s = blockIdx.y, h = blockIdx.z, tid = threadIdx.x;
  const int n = row_count[s];
  if (n < kGdnLongRows) return;
  // (rows at or past o_rows were never staged: a caller's rows bound was too small)
  const int r0 = row_start[s], t_end = min(n, p.o_rows - r0);
  for (int t = blockIdx.x; t < t_end; t += gridDim.x) {
    __syncthreads();  // part and obuf of the previous row are consumed
    gdn_norm_row(p, r0 + t, h, tid, part, obuf);
  }
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
               float* const* state_base, size_t state_off, SeqMeta meta, int nseq, int max_rows, hipStream_t s) {
  PGD_CHECK(kernel >= 1 && kernel <= 8, kErrShape, "conv kernel must be in 1..8");
  if (nseq <= 0) return;
  const int segs = max_rows > kConvSeg ? (max_rows + kConvSeg - 1) / kConvSeg : 1;
  const dim3 grid((channels + 255) / 256, nseq, segs);
#define PGD_CONV_CASE(K)                                                                                            \
  case K:                                                                                                          \
    hipLaunchKernelGGL(conv_step_kernel<K>, grid, dim3(256), 0, s, x, ldx, out, ldo, channels, weight, state_base, \
                       state_off, meta.row_start, meta.row_count);                                                 \
    break;
  switch (kernel) {
    PGD_CONV_CASE(1)
    PGD_CONV_CASE(2)
    PGD_CONV_CASE(3)
    PGD_CONV_CASE(4)
    PGD_CONV_CASE(5)
    PGD_CONV_CASE(6)
    PGD_CONV_CASE(7)
    PGD_CONV_CASE(8)
  }
#undef PGD_CONV_CASE
  PGD_HIP(hipGetLastError());
}

void gdn_step(const GdnParams& p, SeqMeta meta, int nseq, int rows, int max_rows, hipStream_t s) {
  PGD_CHECK(p.k_dim == 128 && p.v_dim == 128, kErrShape, "gated delta kernel needs k_dim == v_dim == 128");
  PGD_CHECK(p.k_heads > 0 && p.v_heads % p.k_heads == 0, kErrShape, "v_heads must be a multiple of k_heads");
  if (nseq <= 0) return;
  const bool chunked = rows > 0 && max_rows >= kGdnLongRows;
  GdnParams q = p;
  q.o_rows = chunked ? rows : 0;
  q.o_raw = chunked ? static_cast<float*>(gemv::gemv_scratch(s, (size_t)rows * p.v_heads * 128 * sizeof(float), 7))
                    : nullptr;
  hipLaunchKernelGGL(gdn_kernel<kGdnRowGroups>, dim3(p.v_heads, nseq), dim3(32 * kGdnRowGroups), 0, s, q,
                     meta.row_start, meta.row_count);
  PGD_HIP(hipGetLastError());
  if (!chunked) return;
  PGD_CHECK(p.ld_conv % 4 == 0, kErrShape, "chunked gated delta kernel needs 16-byte aligned conv rows");
  constexpr size_t lds = kGdnChunkLds;
  static bool attr = false;
  if (!attr) {
    PGD_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&gdn_chunk_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr = true;
  }
  hipLaunchKernelGGL(gdn_chunk_kernel, dim3(p.v_heads * kGdnColGroups, nseq), dim3(256), lds, s, q, meta.row_start,
                     meta.row_count);
  PGD_HIP(hipGetLastError());
  hipLaunchKernelGGL(gdn_norm_kernel, dim3(std::min(max_rows, 4096), nseq, p.v_heads), dim3(128), 0, s, q,
                     meta.row_start, meta.row_count);
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
