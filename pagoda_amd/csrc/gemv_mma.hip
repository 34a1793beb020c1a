// gemv_mma.hip — MLX affine-8 (group 64) GEMV / skinny GEMM on the matrix cores.
//
// Y[b, n] = sum_k x[b, k] * (s[n, g] * c[n, k] + bias[n, g]),  g = k / 64,
// for up to 32 batch rows per launch, in two 16-row batch tiles. Per group:
//   P[b, n] = sum_k (c[n,k] - 128) * (xh[b,k] + xl[b,k])     4 x v_mfma_f32_16x16x32_f16
//   Y[b, n] += s[n,g] * (P[b, n] + 128 * XSP[b,g]) + bias[n,g] * XS[b,g]
// xh = f16(x) and xl = f16(x - xh) carry x to ~22 bits, codes - 128 are
// exact in f16, XS = sum x and XSP = sum (xh + xl) over the group in f32.
// The batch row is the MFMA's M index and the weight row its N index: a lane
// owns one weight row (one scale/bias load per group) and four batch rows,
// and every batch row goes through the same instruction sequence whatever the
// batch size, so a batched call is bitwise equal to single-row calls.
//
// Activations are converted once (a8_xprep_kernel, or fused into the RMSNorm
// that produces them, a8_norm_prep_kernel) into the MFMA operand order;
// weights are stored tiled (32 rows x 64 codes per 2 KiB block), so a wave's
// 128-bit loads read 512 B runs. A workgroup of KS waves shares one 32-row
// tile and splits the groups between its waves; each wave keeps PF groups of
// loads in flight; partial sums meet in LDS in a fixed order.
//
// Counterpart of affine_gemv / affine_gemm4 / gemv2_silu / gemv_res
// (pagoda-hf/src/qwen3_gemv.rs:54-306, 414-567).
#include "common.h"
#include "gemv_impl.h"
#include "quant.h"

namespace pgd {
namespace gemv {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

// four codes (one u32) -> two f16 pairs holding (code - 128)
__device__ inline void codes_to_h(uint32_t w, uint32_t& lo, uint32_t& hi) {
  // bytes [c, 0x64] form the f16 1024 + c; subtracting 1152 leaves c - 128
  const uint32_t a = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
  const h2 ha = __builtin_bit_cast(h2, a) - (h2){(_Float16)1152.0f, (_Float16)1152.0f};
  const h2 hb = __builtin_bit_cast(h2, b) - (h2){(_Float16)1152.0f, (_Float16)1152.0f};
  lo = __builtin_bit_cast(uint32_t, ha);
  hi = __builtin_bit_cast(uint32_t, hb);
}

__device__ inline h8 codes8(uint32_t w0, uint32_t w1) {
  uint32_t c0, c1, c2, c3;
  codes_to_h(w0, c0, c1);
  codes_to_h(w1, c2, c3);
  return __builtin_bit_cast(h8, make_uint4(c0, c1, c2, c3));
}

// ---- activation prep --------------------------------------------------------
// Rows are cut into chunks of 32 (two 16-row batch tiles). For chunk c,
// group g, batch tile bt, item = (c * G + g) * 2 + bt:
//   XA[item][lane] = 64 B: xh step 0 | xh step 1 | xl step 0 | xl step 1,
//     8 halves each, batch row 32c + 16bt + lane % 16, k = 64g + 16(lane/16) + 8 step + e
//   CA[item] = 32 floats: 128 * XSP for the 16 rows, then XS for the 16 rows
// Rows past the end are never written: their MFMA rows only feed discarded
// outputs.
__device__ inline void prep16(const float* v, uint4* o, float& xs, float& xsp) {
  uint32_t hw[8], lw[8];
  xs = 0.0f;
  xsp = 0.0f;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const _Float16 h0 = (_Float16)v[2 * p], h1 = (_Float16)v[2 * p + 1];
    const _Float16 l0 = (_Float16)(v[2 * p] - (float)h0), l1 = (_Float16)(v[2 * p + 1] - (float)h1);
    hw[p] = __builtin_bit_cast(uint32_t, (h2){h0, h1});
    lw[p] = __builtin_bit_cast(uint32_t, (h2){l0, l1});
    xs += v[2 * p] + v[2 * p + 1];
    xsp += ((float)h0 + (float)l0) + ((float)h1 + (float)l1);
  }
  o[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  o[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
  o[2] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  o[3] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
}

__global__ __launch_bounds__(256) void a8_xprep_kernel(const float* __restrict__ x, int ldx, int rows, int G,
                                                       uint4* __restrict__ XA, float* __restrict__ CA) {
  const size_t item = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int bt = (int)(item & 1);
  const size_t cg = item >> 1;
  const int g = (int)(cg % G), c = (int)(cg / G);
  if (32 * c >= rows) return;
  const int row = 32 * c + 16 * bt + (lane & 15), q = lane >> 4;
  float v[16];
  if (row < rows) {
    const float4* xp = reinterpret_cast<const float4*>(x + (size_t)row * ldx + (g << 6) + 16 * q);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 f = xp[i];
      v[4 * i] = f.x;
      v[4 * i + 1] = f.y;
      v[4 * i + 2] = f.z;
      v[4 * i + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = 0.0f;
  }
  float xs, xsp;
  prep16(v, XA + (item * 64 + lane) * 4, xs, xsp);
  // the four lanes of a row (q = 0..3) hold its four 16-wide k slices
  xs += __shfl_xor(xs, 16, 64);
  xs += __shfl_xor(xs, 32, 64);
  xsp += __shfl_xor(xsp, 16, 64);
  xsp += __shfl_xor(xsp, 32, 64);
  if (q == 0) {
    CA[item * 32 + (lane & 15)] = 128.0f * xsp;
    CA[item * 32 + 16 + (lane & 15)] = xs;
  }
}

// Fused RMSNorm (rms_zero, pagoda-hf/src/qwen3_5.rs:1736-1745) + activation
// prep: one workgroup per output row; thread t owns 16-wide slices t, t+256,
// ... (slice u = 4g + q), kept in registers between the two passes.
constexpr int kNormMaxSlices = 8;  // n <= 256 * 16 * 8
__global__ __launch_bounds__(256) void a8_norm_prep_kernel(const float* __restrict__ x, int ldx,
                                                           const int* __restrict__ rows_idx, int rows, int n,
                                                           const float* __restrict__ w, float eps, float* y, int ldy,
                                                           uint4* __restrict__ XA, float* __restrict__ CA) {
  __shared__ float red[4];
  const int r = blockIdx.x, tid = threadIdx.x;
  const int src = rows_idx ? rows_idx[r] : r;
  const float* xr = x + (size_t)src * ldx;
  const int slices = n >> 4, G = n >> 6;
  float v[kNormMaxSlices][16];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormMaxSlices; ++i) {
    const int u = tid + 256 * i;
    if (u < slices) {
      const float4* p = reinterpret_cast<const float4*>(xr + 16 * u);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float4 f = p[e];
        v[i][4 * e] = f.x;
        v[i][4 * e + 1] = f.y;
        v[i][4 * e + 2] = f.z;
        v[i][4 * e + 3] = f.w;
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) ss += v[i][e] * v[i][e];
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)n + eps);
  const int c = r >> 5, bt = (r >> 4) & 1, j = r & 15;
#pragma unroll
  for (int i = 0; i < kNormMaxSlices; ++i) {
    const int u = tid + 256 * i;
    const bool live = u < slices;  // uniform per group of four lanes (slices % 4 == 0)
    float xs = 0.0f, xsp = 0.0f;
    if (live) {
      const float4* wp = reinterpret_cast<const float4*>(w + 16 * u);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float4 f = wp[e];
        v[i][4 * e] = v[i][4 * e] * inv * f.x;
        v[i][4 * e + 1] = v[i][4 * e + 1] * inv * f.y;
        v[i][4 * e + 2] = v[i][4 * e + 2] * inv * f.z;
        v[i][4 * e + 3] = v[i][4 * e + 3] * inv * f.w;
      }
      if (y) {
        float4* yp = reinterpret_cast<float4*>(y + (size_t)r * ldy + 16 * u);
#pragma unroll
        for (int e = 0; e < 4; ++e) yp[e] = make_float4(v[i][4 * e], v[i][4 * e + 1], v[i][4 * e + 2], v[i][4 * e + 3]);
      }
      const int g = u >> 2, q = u & 3;
      const size_t item = ((size_t)c * G + g) * 2 + bt;
      prep16(v[i], XA + (item * 64 + q * 16 + j) * 4, xs, xsp);
    }
    // group sums over the four slices of a group (adjacent lanes)
    xs += __shfl_xor(xs, 1, 64);
    xs += __shfl_xor(xs, 2, 64);
    xsp += __shfl_xor(xsp, 1, 64);
    xsp += __shfl_xor(xsp, 2, 64);
    if (live && (u & 3) == 0) {
      const size_t item = ((size_t)c * G + (u >> 2)) * 2 + bt;
      CA[item * 32 + j] = 128.0f * xsp;
      CA[item * 32 + 16 + j] = xs;
    }
  }
}

template <int NS, int NBT>
struct GroupRaw {
  uint4 w[NS];       // 16 codes per weight subtile
  uint32_t sb[NS];   // scale | bias
  uint4 xa[NBT][4];  // A operands
  float4 cp[NBT];    // 128 * XSP of this lane's 4 batch rows
  float4 xs[NBT];    // XS of this lane's 4 batch rows
};

// NS = 16-row weight subtiles per wave (2 = one 32-row tile; 4 = gate + up)
template <int NBT, int KS, int PF, int EPI>
__global__ __launch_bounds__(64 * KS) void a8_mma_kernel(GemvArgs a, const uint4* __restrict__ XA,
                                                         const float* __restrict__ CA, int nb) {
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr int NS = DUAL ? 4 : 2;
  __shared__ f4 red[KS > 1 ? KS - 1 : 1][NS][NBT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4;  // MFMA column (weight row in subtile), k quarter / row quad
  const int tile = blockIdx.x;
  const int G = a.n_in >> 6;
  const uint8_t* wbase[NS];
  const uint32_t* sbase[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const uint8_t* p = (DUAL && st >= 2) ? a.u0 : a.p0;
    const uint8_t* ps = (DUAL && st >= 2) ? a.u1 : a.p1;
    const int r = 16 * (st & 1) + j;  // row within the 32-row tile
    wbase[st] = p + ((size_t)tile * G << 11) + (q >> 1) * 1024 + r * 32 + (q & 1) * 16;
    sbase[st] = reinterpret_cast<const uint32_t*>(ps) + ((size_t)tile * G << 5) + r;
  }
  const bool bt1 = NBT > 1 && nb > 16;
  f4 Y[NS][NBT];
#pragma unroll
  for (int st = 0; st < NS; ++st)
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) Y[st][bt] = (f4){0.f, 0.f, 0.f, 0.f};

  auto load = [&](int g, GroupRaw<NS, NBT>& R) {
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      R.w[st] = *reinterpret_cast<const uint4*>(wbase[st] + ((size_t)g << 11));
      R.sb[st] = sbase[st][(size_t)g << 5];
    }
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) {
      if (bt == 0 || bt1) {
        const size_t item = (size_t)g * 2 + bt;
        const uint4* xp = XA + (item * 64 + lane) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) R.xa[bt][i] = xp[i];
        R.cp[bt] = *reinterpret_cast<const float4*>(CA + item * 32 + 4 * q);
        R.xs[bt] = *reinterpret_cast<const float4*>(CA + item * 32 + 16 + 4 * q);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) R.xa[bt][i] = make_uint4(0u, 0u, 0u, 0u);
        R.cp[bt] = make_float4(0.f, 0.f, 0.f, 0.f);
        R.xs[bt] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };

  auto compute = [&](const GroupRaw<NS, NBT>& R) {
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      const h8 b0 = codes8(R.w[st].x, R.w[st].y);
      const h8 b1 = codes8(R.w[st].z, R.w[st].w);
      const float sc = bf16_to_f32(R.sb[st] & 0xffffu);
      const float bi = bf16_to_f32(R.sb[st] >> 16);
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        f4 P = {0.f, 0.f, 0.f, 0.f};
        P = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, R.xa[bt][0]), b0, P, 0, 0, 0);
        P = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, R.xa[bt][1]), b1, P, 0, 0, 0);
        P = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, R.xa[bt][2]), b0, P, 0, 0, 0);
        P = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, R.xa[bt][3]), b1, P, 0, 0, 0);
        const float cp[4] = {R.cp[bt].x, R.cp[bt].y, R.cp[bt].z, R.cp[bt].w};
        const float xs[4] = {R.xs[bt].x, R.xs[bt].y, R.xs[bt].z, R.xs[bt].w};
#pragma unroll
        for (int r = 0; r < 4; ++r) Y[st][bt][r] = fmaf(bi, xs[r], fmaf(sc, P[r] + cp[r], Y[st][bt][r]));
      }
    }
  };

  // groups of this wave: a contiguous range, PF groups in flight
  const int per = (G + KS - 1) / KS;
  const int g0 = wave * per, g1 = min(G, g0 + per);
  GroupRaw<NS, NBT> buf[PF];
#pragma unroll
  for (int u = 0; u < PF; ++u)
    if (g0 + u < g1) load(g0 + u, buf[u]);
  for (int g = g0; g < g1; g += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      if (g + u < g1) {
        compute(buf[u]);
        if (g + u + PF < g1) load(g + u + PF, buf[u]);
      }
    }
  }

  // ---- split-K reduction (fixed order: wave 0 + 1 + ... + KS-1) ----
  if constexpr (KS > 1) {
    if (wave > 0) {
#pragma unroll
      for (int st = 0; st < NS; ++st)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) red[wave - 1][st][bt][lane] = Y[st][bt];
    }
    __syncthreads();
    if (wave != 0) return;
    for (int w = 0; w < KS - 1; ++w)
#pragma unroll
      for (int st = 0; st < NS; ++st)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) Y[st][bt] += red[w][st][bt][lane];
  }
  // ---- epilogue: lane holds weight row n for batch rows 16bt + 4q + r ----
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const int n = tile * 32 + 16 * st + j;
    if (n >= a.n_out) continue;
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int b = 16 * bt + 4 * q + r;
        if (b >= nb) continue;
        const size_t o = (size_t)b * a.ldy + n;
        if constexpr (EPI == EPI_STORE) a.y[o] = Y[st][bt][r];
        if constexpr (EPI == EPI_RES) a.y[o] = a.res[(size_t)b * a.ldres + n] + Y[st][bt][r];
        if constexpr (EPI == EPI_SWIGLU) a.y[o] = silu_f(Y[st][bt][r]) * Y[2 + st][bt][r];
      }
  }
}

constexpr int kPF = 2;  // groups of loads in flight per wave

template <int NBT, int KS, int EPI>
void launch_kernel(const GemvArgs& a, const uint4* XA, const float* CA, int nb, hipStream_t s) {
  constexpr int PF = kPF;
  const int tiles = (a.n_out + 31) / 32;
  hipLaunchKernelGGL((a8_mma_kernel<NBT, KS, PF, EPI>), dim3(tiles), dim3(64 * KS), 0, s, a, XA, CA, nb);
}

template <int NBT, int EPI>
void launch_ks(const GemvArgs& a, const uint4* XA, const float* CA, int nb, hipStream_t s) {
  // enough waves to fill the GPU (~8 per CU), each wave keeping its prefetch
  // ring busy. The split depends on the matrix shape only, never on the batch,
  // so every batch size sums a row's groups in the same order.
  const int tiles = (a.n_out + 31) / 32;
  const int G = a.n_in / 64;
  int ks = 1;
  while (ks < 8 && tiles * ks < 2048 && G / (2 * ks) >= 4) ks *= 2;
  switch (ks) {
    case 1: launch_kernel<NBT, 1, EPI>(a, XA, CA, nb, s); break;
    case 2: launch_kernel<NBT, 2, EPI>(a, XA, CA, nb, s); break;
    case 4: launch_kernel<NBT, 4, EPI>(a, XA, CA, nb, s); break;
    default: launch_kernel<NBT, 8, EPI>(a, XA, CA, nb, s); break;
  }
}

template <int EPI>
void launch_prepped(GemvArgs a, const A8Act& act, hipStream_t s) {
  PGD_CHECK(act.K == a.n_in, kErrShape, "prepared activations have the wrong width");
  const int G = a.n_in / 64;
  const uint4* XA = reinterpret_cast<const uint4*>(act.XA);
  int rows = act.rows;
  for (int c = 0; rows > 0; ++c) {
    const int nb = rows < 32 ? rows : 32;
    const uint4* xa = XA + (size_t)c * G * 2 * 64 * 4;
    const float* ca = act.CA + (size_t)c * G * 2 * 32;
    if (nb > 16) launch_ks<2, EPI>(a, xa, ca, nb, s);
    else launch_ks<1, EPI>(a, xa, ca, nb, s);
    PGD_HIP(hipGetLastError());
    rows -= nb;
    a.y += (size_t)nb * a.ldy;
    if (a.res) a.res += (size_t)nb * a.ldres;
  }
}

}  // namespace

void run_a8_mma(const GemvArgs& a, const A8Act& act, int epi, hipStream_t s) {
  if (epi == EPI_SWIGLU) launch_prepped<EPI_SWIGLU>(a, act, s);
  else if (epi == EPI_RES) launch_prepped<EPI_RES>(a, act, s);
  else launch_prepped<EPI_STORE>(a, act, s);
}

}  // namespace gemv

size_t a8_act_bytes(int rows, int K) {
  const size_t chunks = ((size_t)rows + 31) / 32, G = (size_t)K / 64;
  return chunks * G * 2 * (64 * 64 + 32 * 4);
}

A8Act a8_act_view(void* buf, int rows, int K) {
  const size_t chunks = ((size_t)rows + 31) / 32, G = (size_t)K / 64;
  A8Act a;
  a.XA = buf;
  a.CA = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(buf) + chunks * G * 2 * 64 * 64);
  a.rows = rows;
  a.K = K;
  return a;
}

A8Act a8_act_prep(const float* x, int ldx, int rows, int K, void* buf, hipStream_t s) {
  PGD_CHECK(K % 64 == 0 && ldx % 4 == 0, kErrShape, "A8 activation width must be a multiple of 64");
  A8Act a = a8_act_view(buf, rows, K);
  if (rows <= 0) return a;
  const size_t items = ((size_t)rows + 31) / 32 * (K / 64) * 2;
  hipLaunchKernelGGL(gemv::a8_xprep_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, x, ldx, rows, K / 64,
                     reinterpret_cast<uint4*>(buf), const_cast<float*>(a.CA));
  PGD_HIP(hipGetLastError());
  return a;
}

A8Act a8_norm_prep(const float* x, int ldx, const int* rows_idx, int rows, int n, const float* w, float eps, float* y,
                   int ldy, void* buf, hipStream_t s) {
  PGD_CHECK(n % 64 == 0 && n <= 256 * 16 * gemv::kNormMaxSlices && ldx % 4 == 0, kErrShape, "norm prep width");
  A8Act a = a8_act_view(buf, rows, n);
  if (rows <= 0) return a;
  hipLaunchKernelGGL(gemv::a8_norm_prep_kernel, dim3(rows), dim3(256), 0, s, x, ldx, rows_idx, rows, n, w, eps, y,
                     ldy, reinterpret_cast<uint4*>(buf), const_cast<float*>(a.CA));
  PGD_HIP(hipGetLastError());
  return a;
}

namespace gemv {

}  // namespace gemv
}  // namespace pgd
