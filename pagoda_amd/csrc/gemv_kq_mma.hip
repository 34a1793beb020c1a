// gemv_kq_mma.hip — GGML Q4_K GEMV / skinny GEMM on the matrix cores.
//
// Q4_K (pagoda-hf/src/qwen2_gguf.rs:271-289 runs it through candle's
// QMatMul): per 32-element sub-block s of a 256-element super-block,
// w = d * sc[s] * q - dmin * m[s] with q a 4-bit code. Per sub-block:
//   P[b, n] = sum_k (1024 + q[n,k]) * x[b,k]      v_mfma_f32_16x16x32_f16
//   XS[b]   = sum_k x[b,k]                          (MFMA against a ones operand)
//   Y[b, n] += d sc * P - (1024 d sc + dmin m) * XS
// 1024 + q is exact in f16 and is what one byte permute makes of a nibble;
// f32 activations enter as xh = f16(x), xl = f16(x - xh) (two MFMAs, ~22 bits
// of x), f16 activations as themselves. The batch row is the MFMA's M index,
// the weight row its N index, and the split of the groups depends on the
// matrix shape only, so every batch row runs the same instruction sequence:
// a batched call is bitwise equal to single-row calls.
//
// Weights are the tiled Q4K planes (quant.h): a 64-group of 32 rows is one
// 1 KiB run of qs bytes (row-major, 32 B per row); a lane owning rows
// j and 16 + j and k quarter q reads 8 bytes of each, whose low nibbles are
// its 8 codes of sub-block 2 * (g % 4) and high nibbles those of the next.
// Workgroups hold KS waves sharing one 32-row tile (KS from the shape) and
// splitting its groups; each wave keeps PF groups of loads in flight; the
// waves' partial sums meet in LDS in a fixed order. Matrices of few tiles and
// a long K (the 896-row down projection: 28 tiles) also split K over GS
// workgroups per tile (grid y); their sums go to a workspace and
// kq_part_reduce_kernel adds them in part order and applies the epilogue.
// The split depends on the shape only, so batch rows stay bitwise equal.
#include <type_traits>

#include "common.h"
#include "gemv_impl.h"
#include "quant.h"

namespace pgd {
namespace gemv {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

// eight 4-bit codes (the low or high nibbles of 8 bytes) -> f16 1024 + q
__device__ inline h8 nib8(uint32_t w0, uint32_t w1, int hi) {
  const uint32_t a = hi ? (w0 >> 4) & 0x0F0F0F0Fu : w0 & 0x0F0F0F0Fu;
  const uint32_t b = hi ? (w1 >> 4) & 0x0F0F0F0Fu : w1 & 0x0F0F0F0Fu;
  // bytes [n, 0x64] form the f16 1024 + n
  const uint32_t c0 = __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u);
  const uint32_t c1 = __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u);
  const uint32_t c2 = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
  const uint32_t c3 = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
  return __builtin_bit_cast(h8, make_uint4(c0, c1, c2, c3));
}

// 6-bit scale and min of sub-block is (0..7) from the 12 scale bytes
__device__ inline void q4k_sc_m(const uint4& hdr, int is, float& sc, float& m) {
  const uint4 s = make_uint4(hdr.y, hdr.z, hdr.w, 0u);
  auto byte = [&](int i) -> uint32_t {
    const uint32_t w = i < 4 ? s.x : (i < 8 ? s.y : s.z);
    return (w >> (8 * (i & 3))) & 255u;
  };
  uint32_t a, b;
  if (is < 4) {
    a = byte(is) & 63u;
    b = byte(is + 4) & 63u;
  } else {
    a = (byte(is + 4) & 0xFu) | ((byte(is - 4) >> 6) << 4);
    b = (byte(is + 4) >> 4) | ((byte(is) >> 6) << 4);
  }
  sc = (float)a;
  m = (float)b;
}

template <int NBT, int NS, bool XF16>
struct Q4Raw {
  uint2 w[NS];       // 8 qs bytes per 16-row subtile
  uint4 hdr[NS];     // the subtile row's super-block header
  uint4 x[2][NBT][XF16 ? 1 : 2];  // per sub-block half and batch tile: 8 activations (f16: 16 B, f32: 32 B)
};

// KS == 1: a workgroup of kTilesKS1 waves, one tile each (no k split)
constexpr int kTilesKS1 = 4;
// activation rows staged in LDS (the *_lds kernels): at most this many bytes, rows
// padded by 16 B against bank conflicts
constexpr int kXLdsMax = 64 * 1024;
__host__ __device__ inline int x_lds_stride(int K, bool f16) { return K * (f16 ? 2 : 4) + 16; }

// rows 0 .. 16 NBT - 1 of the launch's activations into LDS (rows past the
// batch repeat the last one); every thread of the workgroup takes part
template <int NBT, bool XF16>
__device__ inline void stage_x(char* xs, const GemvArgs& a, int nb) {
  constexpr int XE = XF16 ? 2 : 4;
  const int K = a.n_in, RS = x_lds_stride(K, XF16);
  const int nvec = K * XE / 16, total = 16 * NBT * nvec;
  const uint8_t* xb = reinterpret_cast<const uint8_t*>(a.x);
  for (int i = threadIdx.x; i < total; i += blockDim.x) {
    const int b = i / nvec, c = i - b * nvec;
    const uint4 v = *reinterpret_cast<const uint4*>(xb + ((size_t)min(b, nb - 1) * a.ldx) * XE + c * 16);
    *reinterpret_cast<uint4*>(xs + b * RS + c * 16) = v;
  }
  __syncthreads();
}

// ---- grid k split ----------------------------------------------------------
// Workgroups per tile along K for a matrix of `tiles` tiles and U k units
// (Q4_K: 64-groups, Q6_K: 128-halves): enough workgroups to reach ~128 when
// the tiles alone give fewer, for K of at least min_units (below that a
// matrix is too small to repay the second launch); 1 = no grid split.
inline int grid_split(int tiles, int U, int min_units) {
  if (tiles >= 128 || U < min_units) return 1;
  int gs = 1;
  while (gs < 8 && tiles * gs < 128) gs *= 2;
  return gs;
}
// waves per workgroup under a grid split: each keeps >= 2 k units
inline int grid_split_ks(int U, int gs) {
  int ks = 2;
  while (ks < 8 && 2 * ks * gs * 2 <= U) ks *= 2;
  return ks;
}

// sums of one workgroup (lane: row n of subtile st, batch rows 16 bt + 4 q + r)
// into the workspace [matrix][part][row][n_out]
template <int NS, int NBT, bool DUAL>
__device__ inline void store_part(const GemvArgs& a, int nb, int tile, const f4 (&Y)[NS][NBT]) {
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const int n = tile * 32 + 16 * (st & 1) + j;
    if (n >= a.n_out) continue;
    const int m = (DUAL && st >= 2) ? 1 : 0;
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int b = 16 * bt + 4 * q + r;
        if (b < nb) a.y[(((size_t)m * gridDim.y + blockIdx.y) * nb + b) * a.n_out + n] = Y[st][bt][r];
      }
  }
}

// y = epilogue(sum over parts 0, 1, .. in order) of the workspace
template <int EPI>
__global__ __launch_bounds__(256) void kq_part_reduce_kernel(GemvArgs a, const float* __restrict__ ws, int gs, int nb) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, plane = (size_t)nb * a.n_out;
  if (i >= plane) return;
  const int b = (int)(i / a.n_out), n = (int)(i % a.n_out);
  float v = ws[i];
  for (int p = 1; p < gs; ++p) v += ws[p * plane + i];
  const size_t o = (size_t)b * a.ldy + n;
  if constexpr (EPI == EPI_STORE) a.y[o] = v;
  if constexpr (EPI == EPI_RES) a.y[o] = a.res[(size_t)b * a.ldres + n] + v;
  if constexpr (EPI == EPI_SWIGLU) {
    float u = ws[gs * plane + i];
    for (int p = 1; p < gs; ++p) u += ws[(gs + p) * plane + i];
    a.y[o] = silu_f(v) * u;
  }
}

inline float* part_workspace(const GemvArgs& a, int nb, int gs, bool dual, hipStream_t s) {
  return static_cast<float*>(gemv_scratch(s, (size_t)(dual ? 2 : 1) * gs * nb * a.n_out * sizeof(float), 1));
}

template <int EPI>
void launch_part_reduce(const GemvArgs& a, const float* ws, int gs, int nb, hipStream_t s) {
  const size_t n = (size_t)nb * a.n_out;
  hipLaunchKernelGGL((kq_part_reduce_kernel<EPI>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a, ws, gs, nb);
}

// PART: this workgroup's sums go to the workspace a.y, [matrix][part][row][n_out]
template <int NBT, int KS, int PF, bool XF16, int EPI, bool PART = false>
__global__ __launch_bounds__(64 * (KS == 1 ? kTilesKS1 : KS)) void q4k_mma_kernel(GemvArgs a, int nb) {
  static_assert(!PART || KS > 1, "a grid k split keeps one tile per workgroup");
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr int NS = DUAL ? 4 : 2;
  __shared__ f4 red[KS > 1 ? KS - 1 : 1][NS][NBT][64];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, q = lane >> 4;
  const int G = a.n_in >> 6, nsb = a.nsb, G4 = 4 * nsb;
  // wave = this wave's k range; KS == 1: every wave its own tile
  const int wave = KS == 1 ? 0 : wv;
  const int tile = KS == 1 ? blockIdx.x * kTilesKS1 + wv : blockIdx.x;
  if (tile >= (a.n_out + 31) / 32) return;

  const uint8_t* wbase[NS];
  const uint8_t* hbase[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const uint8_t* p = (DUAL && st >= 2) ? a.u0 : a.p0;
    const uint8_t* ph = (DUAL && st >= 2) ? a.u1 : a.p1;
    const int r = 16 * (st & 1) + j;
    wbase[st] = p + (size_t)tile * G4 * 1024 + r * 32 + 8 * q;
    hbase[st] = ph + (size_t)tile * nsb * 512 + r * 16;
  }
  // activation rows of this lane's A operand (rows past the batch re-read the
  // last one; their MFMA rows only feed discarded outputs)
  const uint8_t* xrow[NBT];
#pragma unroll
  for (int bt = 0; bt < NBT; ++bt) {
    const int b = min(16 * bt + j, nb - 1);
    xrow[bt] = reinterpret_cast<const uint8_t*>(a.x) + (size_t)b * a.ldx * (XF16 ? 2 : 4);
  }

  auto load = [&](int g, Q4Raw<NBT, NS, XF16>& R) {
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      R.w[st] = *reinterpret_cast<const uint2*>(wbase[st] + (size_t)g * 1024);
      R.hdr[st] = *reinterpret_cast<const uint4*>(hbase[st] + (size_t)(g >> 2) * 512);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        const int k0 = 64 * g + 32 * h + 8 * q;
        if constexpr (XF16) {
          R.x[h][bt][0] = *reinterpret_cast<const uint4*>(xrow[bt] + (size_t)k0 * 2);
        } else {
          R.x[h][bt][0] = *reinterpret_cast<const uint4*>(xrow[bt] + (size_t)k0 * 4);
          R.x[h][bt][1] = *reinterpret_cast<const uint4*>(xrow[bt] + (size_t)k0 * 4 + 16);
        }
      }
  };

  f4 Y[NS][NBT];
#pragma unroll
  for (int st = 0; st < NS; ++st)
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) Y[st][bt] = (f4){0.f, 0.f, 0.f, 0.f};
  const h8 ones = {1, 1, 1, 1, 1, 1, 1, 1};

  auto compute = [&](int g, const Q4Raw<NBT, NS, XF16>& R) {
    // A operands and sub-block sums
    h8 xh[2][NBT], xl[2][NBT];
    f4 XS[2][NBT];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        const uint4 x0 = R.x[h][bt][0];
        if constexpr (XF16) {
          xh[h][bt] = __builtin_bit_cast(h8, x0);
          XS[h][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[h][bt], ones, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        } else {
          const uint4 x1 = R.x[h][bt][XF16 ? 0 : 1];
          const float v[8] = {__builtin_bit_cast(float, x0.x), __builtin_bit_cast(float, x0.y),
                              __builtin_bit_cast(float, x0.z), __builtin_bit_cast(float, x0.w),
                              __builtin_bit_cast(float, x1.x), __builtin_bit_cast(float, x1.y),
                              __builtin_bit_cast(float, x1.z), __builtin_bit_cast(float, x1.w)};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const _Float16 hv = (_Float16)v[e];
            xh[h][bt][e] = hv;
            xl[h][bt][e] = (_Float16)(v[e] - (float)hv);
          }
          f4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[h][bt], ones, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          XS[h][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[h][bt], ones, t, 0, 0, 0);
        }
      }
    const int js = 2 * (g & 3);  // sub-blocks js, js + 1 of the super-block
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      const float d = f16_to_f32(R.hdr[st].x & 0xffffu), dmin = f16_to_f32(R.hdr[st].x >> 16);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float sc, m;
        q4k_sc_m(R.hdr[st], js + h, sc, m);
        const float ca = d * sc;
        const float cb = fmaf(1024.0f, ca, dmin * m);
        const h8 bq = nib8(R.w[st].x, R.w[st].y, h);
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
          f4 P = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[h][bt], bq, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          if constexpr (!XF16) P = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[h][bt], bq, P, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) Y[st][bt][r] = fmaf(ca, P[r], fmaf(-cb, XS[h][bt][r], Y[st][bt][r]));
        }
      }
    }
  };

  // this workgroup's groups [gb, ge) (grid part blockIdx.y of gridDim.y), then this wave's
  const int gper = PART ? (G + (int)gridDim.y - 1) / (int)gridDim.y : G;
  const int gb = PART ? min(G, (int)blockIdx.y * gper) : 0, ge = min(G, gb + gper);
  const int per = (ge - gb + KS - 1) / KS;
  const int g0 = min(ge, gb + wave * per), g1 = min(ge, g0 + per);
  Q4Raw<NBT, NS, XF16> buf[PF];
#pragma unroll
  for (int u = 0; u < PF; ++u)
    if (g0 + u < g1) load(g0 + u, buf[u]);
  for (int g = g0; g < g1; g += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      if (g + u < g1) {
        compute(g + u, buf[u]);
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
  if constexpr (PART) {
    store_part<NS, NBT, DUAL>(a, nb, tile, Y);
    return;
  }
  // ---- epilogue: lane holds weight row n for batch rows 16bt + 4q + r ----
#pragma unroll
  for (int st = 0; st < (DUAL ? 2 : NS); ++st) {
    const int n = tile * 32 + 16 * (st & 1) + j;
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

// Tall Q4_K matrices with a short K (no k split, one wave per tile, <= 16
// rows): the staged-activation form of q4k_mma_kernel with units of two
// 64-groups of one super-block, so each row's 16-byte header is loaded once
// per two groups, and a PF-unit register ring whose loads past the last unit
// re-read it (cache hits) instead of branching. Same arithmetic and group
// order as q4k_mma_kernel with KS == 1.
template <int NS>
struct Q4W {
  uint2 w[2][NS];  // 8 qs bytes per group and subtile
  uint4 hdr[NS];   // the unit's super-block header per subtile row
};

template <int NBT, int PF, bool XF16, int EPI>
__global__ __launch_bounds__(64 * kTilesKS1) void q4k_lds_kernel(GemvArgs a, int nb) {
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr int NS = DUAL ? 4 : 2;
  extern __shared__ __attribute__((aligned(16))) char xs[];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, q = lane >> 4;
  const int G = a.n_in >> 6, nsb = a.nsb, G4 = 4 * nsb, UN = (G + 1) / 2;
  stage_x<NBT, XF16>(xs, a, nb);
  const int tile = blockIdx.x * kTilesKS1 + wv;
  if (tile >= (a.n_out + 31) / 32) return;
  const int XRS = x_lds_stride(a.n_in, XF16);

  const uint8_t* wbase[NS];
  const uint8_t* hbase[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const uint8_t* p = (DUAL && st >= 2) ? a.u0 : a.p0;
    const uint8_t* ph = (DUAL && st >= 2) ? a.u1 : a.p1;
    const int r = 16 * (st & 1) + j;
    wbase[st] = p + (size_t)tile * G4 * 1024 + r * 32 + 8 * q;
    hbase[st] = ph + (size_t)tile * nsb * 512 + r * 16;
  }
  using W = Q4W<NS>;
  // unit u: groups 2u, 2u + 1 (one super-block); a missing second group re-reads the first
  auto load = [&](int u, W& R) {
#pragma unroll
    for (int st = 0; st < NS; ++st) {
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
        R.w[h2][st] = *reinterpret_cast<const uint2*>(wbase[st] + (size_t)min(2 * u + h2, G - 1) * 1024);
      R.hdr[st] = *reinterpret_cast<const uint4*>(hbase[st] + (size_t)(u >> 1) * 512);
    }
  };

  f4 Y[NS][NBT];
#pragma unroll
  for (int st = 0; st < NS; ++st)
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) Y[st][bt] = (f4){0.f, 0.f, 0.f, 0.f};
  const h8 ones = {1, 1, 1, 1, 1, 1, 1, 1};

  auto compute_group = [&](int g, const uint2 (&w)[NS], const uint4 (&hdr)[NS]) {
    h8 xh[2][NBT], xl[2][NBT];
    f4 XS[2][NBT];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        const char* xp = xs + (16 * bt + j) * XRS + (64 * g + 32 * h + 8 * q) * (XF16 ? 2 : 4);
        const uint4 x0 = *reinterpret_cast<const uint4*>(xp);
        if constexpr (XF16) {
          xh[h][bt] = __builtin_bit_cast(h8, x0);
          XS[h][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[h][bt], ones, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        } else {
          const uint4 x1 = *reinterpret_cast<const uint4*>(xp + 16);
          const float v[8] = {__builtin_bit_cast(float, x0.x), __builtin_bit_cast(float, x0.y),
                              __builtin_bit_cast(float, x0.z), __builtin_bit_cast(float, x0.w),
                              __builtin_bit_cast(float, x1.x), __builtin_bit_cast(float, x1.y),
                              __builtin_bit_cast(float, x1.z), __builtin_bit_cast(float, x1.w)};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const _Float16 hv = (_Float16)v[e];
            xh[h][bt][e] = hv;
            xl[h][bt][e] = (_Float16)(v[e] - (float)hv);
          }
          f4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[h][bt], ones, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          XS[h][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[h][bt], ones, t, 0, 0, 0);
        }
      }
    const int js = 2 * (g & 3);
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      const float d = f16_to_f32(hdr[st].x & 0xffffu), dmin = f16_to_f32(hdr[st].x >> 16);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float sc, m;
        q4k_sc_m(hdr[st], js + h, sc, m);
        const float ca = d * sc;
        const float cb = fmaf(1024.0f, ca, dmin * m);
        const h8 bq = nib8(w[st].x, w[st].y, h);
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
          f4 P = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[h][bt], bq, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          if constexpr (!XF16) P = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[h][bt], bq, P, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) Y[st][bt][r] = fmaf(ca, P[r], fmaf(-cb, XS[h][bt][r], Y[st][bt][r]));
        }
      }
    }
  };

  W buf[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) load(min(i, UN - 1), buf[i]);
  for (int u = 0; u < UN; u += PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      if (u + i < UN) {
        compute_group(2 * (u + i), buf[i].w[0], buf[i].hdr);
        if (2 * (u + i) + 1 < G) compute_group(2 * (u + i) + 1, buf[i].w[1], buf[i].hdr);
      }
      load(min(u + i + PF, UN - 1), buf[i]);
    }
  }
#pragma unroll
  for (int st = 0; st < (DUAL ? 2 : NS); ++st) {
    const int n = tile * 32 + 16 * (st & 1) + j;
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

// units in flight of q4k_lds_kernel (deeper rings measured slower)
constexpr int kQ4UnitsInFlight = 2;
// split of the groups: depends on the matrix shape only
inline int q4k_split(const GemvArgs& a) {
  const int tiles = (a.n_out + 31) / 32, G = a.n_in / 64;
  int ks = 1;
  while (ks < 8 && tiles * ks < 1024 && G / (2 * ks) >= 2) ks *= 2;
  return ks;
}
// workgroups per tile along K (1: none); ks then re-chosen by grid_split_ks
inline int q4k_grid_split(const GemvArgs& a) { return grid_split((a.n_out + 31) / 32, a.n_in / 64, 32); }

template <int NBT, int KS, bool XF16, int EPI>
void q4k_launch_part(const GemvArgs& a, int nb, int gs, hipStream_t s) {
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  const int tiles = (a.n_out + 31) / 32;
  GemvArgs p = a;
  float* ws = part_workspace(a, nb, gs, DUAL, s);
  p.y = ws;
  hipLaunchKernelGGL((q4k_mma_kernel<NBT, KS, 2, XF16, EPI, true>), dim3(tiles, gs), dim3(64 * KS), 0, s, p, nb);
  launch_part_reduce<EPI>(a, ws, gs, nb, s);
}

template <int NBT, int KS, bool XF16, int EPI>
void q4k_launch(const GemvArgs& a, int nb, hipStream_t s) {
  const int tiles = (a.n_out + 31) / 32;
  const size_t xlds = (size_t)16 * NBT * x_lds_stride(a.n_in, XF16);
  if constexpr (KS == 1) {
    // staged activations pay at <= 16 rows (at 17..32 rows measured no faster)
    if (NBT == 1 && xlds <= kXLdsMax)
      hipLaunchKernelGGL((q4k_lds_kernel<NBT, kQ4UnitsInFlight, XF16, EPI>), dim3((tiles + kTilesKS1 - 1) / kTilesKS1),
                         dim3(64 * kTilesKS1), xlds, s, a, nb);
    else
      hipLaunchKernelGGL((q4k_mma_kernel<NBT, KS, 2, XF16, EPI>), dim3((tiles + kTilesKS1 - 1) / kTilesKS1),
                         dim3(64 * kTilesKS1), 0, s, a, nb);
  } else {
    hipLaunchKernelGGL((q4k_mma_kernel<NBT, KS, 2, XF16, EPI>), dim3(tiles), dim3(64 * KS), 0, s, a, nb);
  }
}

template <int NBT, bool XF16, int EPI>
void q4k_launch_ks(const GemvArgs& a, int nb, hipStream_t s) {
  if (const int gs = q4k_grid_split(a); gs > 1) {
    switch (grid_split_ks(a.n_in / 64, gs)) {
      case 2: return q4k_launch_part<NBT, 2, XF16, EPI>(a, nb, gs, s);
      case 4: return q4k_launch_part<NBT, 4, XF16, EPI>(a, nb, gs, s);
      default: return q4k_launch_part<NBT, 8, XF16, EPI>(a, nb, gs, s);
    }
  }
  switch (q4k_split(a)) {
    case 1: return q4k_launch<NBT, 1, XF16, EPI>(a, nb, s);
    case 2: return q4k_launch<NBT, 2, XF16, EPI>(a, nb, s);
    case 4: return q4k_launch<NBT, 4, XF16, EPI>(a, nb, s);
    default: return q4k_launch<NBT, 8, XF16, EPI>(a, nb, s);
  }
}

template <bool XF16, int EPI>
void q4k_launch_wide(const GemvArgs& a, int nb, hipStream_t s) {
  if constexpr (EPI != EPI_SWIGLU) {
    switch (q4k_split(a)) {
      case 1: return q4k_launch<4, 1, XF16, EPI>(a, nb, s);
      case 2: return q4k_launch<4, 2, XF16, EPI>(a, nb, s);
      default: return q4k_launch<4, 4, XF16, EPI>(a, nb, s);
    }
  }
}

template <bool XF16, int EPI>
void q4k_rows(GemvArgs a, int nrows, hipStream_t s) {
  const size_t xel = XF16 ? 2 : 4;
  while (nrows > 0) {
    // 33..64 rows as one launch of four 16-row batch tiles where the k split
    // keeps them in registers (tall matrices: the weights stream once for all
    // rows); a row's sums do not depend on the batch tiles
    const bool wide = q4k_split(a) <= 4 && q4k_grid_split(a) == 1 && EPI != EPI_SWIGLU;
    const int nb = nrows < (wide ? 64 : 32) ? nrows : (wide ? 64 : 32);
    if (nb > 32) q4k_launch_wide<XF16, EPI>(a, nb, s);
    else if (nb > 16) q4k_launch_ks<2, XF16, EPI>(a, nb, s);
    else q4k_launch_ks<1, XF16, EPI>(a, nb, s);
    PGD_HIP(hipGetLastError());
    nrows -= nb;
    a.x = reinterpret_cast<const uint8_t*>(a.x) + (size_t)nb * a.ldx * xel;
    a.y += (size_t)nb * a.ldy;
    if (a.res) a.res += (size_t)nb * a.ldres;
  }
}


// ---- Q6_K -----------------------------------------------------------------
// GGML block_q6_K (pagoda-hf/src/qwen2_gguf.rs:271-289 via candle's QMatMul):
// per 128-element half of a super-block, element e (0..127) has code
// q = (ql[e % 64] nibble e / 64) | ((qh[e % 32] >> 2 (e / 32)) & 3) << 4 and
// weight d * sc[e / 16] * (q - 32). The scale changes every 16 elements, so
// one v_mfma_f32_16x16x16_f16 covers one 16-element sub-block s:
//   XS[b] = sum x  (MFMA against ones)
//   P[b, n] = -1056 XS + sum (1024 + q) x   (the chain starts from -1056 XS)
//   Y += d sc P
// Lane (j, quarter q) holds elements 16 s + 4 q .. + 3 of every sub-block:
// ql bytes 16 (s % 4) + 4 q (nibble s / 4) and qh bytes 16 (s % 2) + 4 q
// (shift 2 (s / 2)): four ql dwords and two qh dwords per half and row,
// which the tiled planes (quant.h q6k_*_off) hold as 16 + 8 contiguous
// bytes; padding rows are zeros.

// four 6-bit codes (ql nibbles + qh bit pairs of 4 bytes) -> f16 1024 + q
__device__ inline h4 q6_codes(uint32_t ql, uint32_t qh, int hi_nib, int sh) {
  const uint32_t lo = hi_nib ? (ql >> 4) & 0x0F0F0F0Fu : ql & 0x0F0F0F0Fu;
  const uint32_t q = lo | (((qh >> sh) & 0x03030303u) << 4);
  const uint32_t c0 = __builtin_amdgcn_perm(0x64646464u, q, 0x04010400u);
  const uint32_t c1 = __builtin_amdgcn_perm(0x64646464u, q, 0x04030402u);
  return __builtin_bit_cast(h4, make_uint2(c0, c1));
}

template <int NBT, bool XF16>
struct Q6Raw {
  using XT = typename std::conditional<XF16, uint2, uint4>::type;  // 4 activations
  uint32_t ql[2][4];
  uint32_t qh[2][2];
  uint2 sc[2];   // the half's 8 int8 sub-block scales
  uint32_t d[2]; // f16 super-block scale (low half)
  XT x[8][NBT];
};

template <int NBT, int KS, bool XF16, int EPI, bool PART = false>
__global__ __launch_bounds__(64 * (KS == 1 ? kTilesKS1 : KS)) void q6k_mma_kernel(GemvArgs a, int nb) {
  static_assert(EPI != EPI_SWIGLU, "one matrix per wave");
  static_assert(!PART || KS > 1, "a grid k split keeps one tile per workgroup");
  constexpr int NS = 2;
  __shared__ f4 red[KS > 1 ? KS - 1 : 1][NS][NBT][64];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, q = lane >> 4;
  const int H = a.n_in >> 7, nsb = a.nsb;
  // wave = this wave's k range; KS == 1: every wave its own tile
  const int wave = KS == 1 ? 0 : wv;
  const int tile = KS == 1 ? blockIdx.x * kTilesKS1 + wv : blockIdx.x;
  if (tile >= (a.n_out + 31) / 32) return;

  // per half u: block tile * 2 nsb + u of each plane
  const size_t blk0 = (size_t)tile * 2 * nsb;
  const uint8_t* qlb[NS];
  const uint8_t* qhb[NS];
  const uint8_t* scb[NS];
  const uint16_t* db[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const int ln = (4 * st + q) * 16 + j;
    qlb[st] = a.p0 + (blk0 << 11) + ln * 16;
    qhb[st] = a.p1 + (blk0 << 10) + ln * 8;
    scb[st] = a.p2 + (blk0 << 8) + (16 * st + j) * 8;
    db[st] = reinterpret_cast<const uint16_t*>(a.p3) + (size_t)tile * nsb * 32 + 16 * st + j;
  }
  const uint8_t* xrow[NBT];
#pragma unroll
  for (int bt = 0; bt < NBT; ++bt) {
    const int b = min(16 * bt + j, nb - 1);
    xrow[bt] = reinterpret_cast<const uint8_t*>(a.x) + ((size_t)b * a.ldx + 4 * q) * (XF16 ? 2 : 4);
  }
  using Raw = Q6Raw<NBT, XF16>;
  using XT = typename Raw::XT;

  auto load = [&](int u, Raw& R) {
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      const uint4 l = *reinterpret_cast<const uint4*>(qlb[st] + ((size_t)u << 11));
      const uint2 h = *reinterpret_cast<const uint2*>(qhb[st] + ((size_t)u << 10));
      R.ql[st][0] = l.x;
      R.ql[st][1] = l.y;
      R.ql[st][2] = l.z;
      R.ql[st][3] = l.w;
      R.qh[st][0] = h.x;
      R.qh[st][1] = h.y;
      R.sc[st] = *reinterpret_cast<const uint2*>(scb[st] + ((size_t)u << 8));
      R.d[st] = db[st][(u >> 1) * 32];
    }
#pragma unroll
    for (int sb = 0; sb < 8; ++sb)
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt)
        R.x[sb][bt] = *reinterpret_cast<const XT*>(xrow[bt] + (size_t)(128 * u + 16 * sb) * (XF16 ? 2 : 4));
  };

  f4 Y[NS][NBT];
#pragma unroll
  for (int st = 0; st < NS; ++st)
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) Y[st][bt] = (f4){0.f, 0.f, 0.f, 0.f};
  const h4 ones = {1, 1, 1, 1};

  auto compute = [&](const Raw& R) {
    float dv[NS];
#pragma unroll
    for (int st = 0; st < NS; ++st) dv[st] = f16_to_f32(R.d[st] & 0xffffu);
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) {
      h4 xh[NBT], xl[NBT];
      f4 XS[NBT];
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        if constexpr (XF16) {
          xh[bt] = __builtin_bit_cast(h4, R.x[sb][bt]);
          XS[bt] = __builtin_amdgcn_mfma_f32_16x16x16f16(xh[bt], ones, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        } else {
          const float v[4] = {__builtin_bit_cast(float, R.x[sb][bt].x), __builtin_bit_cast(float, R.x[sb][bt].y),
                              __builtin_bit_cast(float, R.x[sb][bt].z), __builtin_bit_cast(float, R.x[sb][bt].w)};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const _Float16 hv = (_Float16)v[e];
            xh[bt][e] = hv;
            xl[bt][e] = (_Float16)(v[e] - (float)hv);
          }
          f4 t = __builtin_amdgcn_mfma_f32_16x16x16f16(xh[bt], ones, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          XS[bt] = __builtin_amdgcn_mfma_f32_16x16x16f16(xl[bt], ones, t, 0, 0, 0);
        }
      }
      f4 NXS[NBT];
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) NXS[bt] = XS[bt] * -1056.0f;
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        const uint32_t scw = sb < 4 ? R.sc[st].x : R.sc[st].y;
        const float sc = (float)(int8_t)((scw >> (8 * (sb & 3))) & 255u);
        const float ca = dv[st] * sc;
        const h4 bq = q6_codes(R.ql[st][sb & 3], R.qh[st][sb & 1], sb >> 2, 2 * (sb >> 1));
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
          // the chain starts from -1056 XS: P = sum (q - 32) x
          f4 P = __builtin_amdgcn_mfma_f32_16x16x16f16(xh[bt], bq, NXS[bt], 0, 0, 0);
          if constexpr (!XF16) P = __builtin_amdgcn_mfma_f32_16x16x16f16(xl[bt], bq, P, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) Y[st][bt][r] = fmaf(ca, P[r], Y[st][bt][r]);
        }
      }
      // one sub-block at a time: keeps the operands of the others out of registers
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // double buffer: the next half's loads are in flight during this one's MFMAs
  // this workgroup's halves [hb, he) (grid part blockIdx.y of gridDim.y), then this wave's
  const int hper = PART ? (H + (int)gridDim.y - 1) / (int)gridDim.y : H;
  const int hb = PART ? min(H, (int)blockIdx.y * hper) : 0, he = min(H, hb + hper);
  const int per = (he - hb + KS - 1) / KS;
  const int u0 = min(he, hb + wave * per), u1 = min(he, u0 + per);
  Raw cur, nxt;
  if (u0 < u1) load(u0, cur);
  for (int u = u0; u < u1; ++u) {
    if (u + 1 < u1) load(u + 1, nxt);
    compute(cur);
    cur = nxt;
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
  if constexpr (PART) {
    store_part<NS, NBT, false>(a, nb, tile, Y);
    return;
  }
#pragma unroll
  for (int st = 0; st < NS; ++st) {
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
      }
  }
}

// Tall matrices with a short K (no k split, one wave per tile): the launch's
// activation rows are staged in LDS once per workgroup (rows padded by 16 B
// against bank conflicts), so the tiles of a workgroup share one copy and
// only the weights stream through a PF-deep register ring. Same arithmetic
// and order as q6k_mma_kernel with KS == 1.

template <int NS>
struct Q6W {
  uint4 ql[NS];
  uint2 qh[NS];
  uint2 sc[NS];
  uint32_t d[NS];
};

template <int NBT, int PF, bool XF16, int EPI>
__global__ __launch_bounds__(64 * kTilesKS1) void q6k_lds_kernel(GemvArgs a, int nb) {
  static_assert(EPI != EPI_SWIGLU, "one matrix per wave");
  constexpr int NS = 2, XE = XF16 ? 2 : 4;
  extern __shared__ __attribute__((aligned(16))) char xs[];
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, q = lane >> 4;
  const int H = a.n_in >> 7, nsb = a.nsb, K = a.n_in;
  const int RS = x_lds_stride(K, XF16);
  stage_x<NBT, XF16>(xs, a, nb);
  const int tile = blockIdx.x * kTilesKS1 + wv;
  if (tile >= (a.n_out + 31) / 32) return;

  const size_t blk0 = (size_t)tile * 2 * nsb;
  const uint8_t* qlb[NS];
  const uint8_t* qhb[NS];
  const uint8_t* scb[NS];
  const uint16_t* db[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const int ln = (4 * st + q) * 16 + j;
    qlb[st] = a.p0 + (blk0 << 11) + ln * 16;
    qhb[st] = a.p1 + (blk0 << 10) + ln * 8;
    scb[st] = a.p2 + (blk0 << 8) + (16 * st + j) * 8;
    db[st] = reinterpret_cast<const uint16_t*>(a.p3) + (size_t)tile * nsb * 32 + 16 * st + j;
  }
  using W = Q6W<NS>;
  auto load = [&](int u, W& R) {
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      R.ql[st] = *reinterpret_cast<const uint4*>(qlb[st] + ((size_t)u << 11));
      R.qh[st] = *reinterpret_cast<const uint2*>(qhb[st] + ((size_t)u << 10));
      R.sc[st] = *reinterpret_cast<const uint2*>(scb[st] + ((size_t)u << 8));
      R.d[st] = db[st][(u >> 1) * 32];
    }
  };

  f4 Y[NS][NBT];
#pragma unroll
  for (int st = 0; st < NS; ++st)
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) Y[st][bt] = (f4){0.f, 0.f, 0.f, 0.f};
  const h4 ones = {1, 1, 1, 1};
  const char* xl0 = xs + j * RS + 4 * q * XE;

  auto compute = [&](int u, const W& R) {
    float dv[NS];
#pragma unroll
    for (int st = 0; st < NS; ++st) dv[st] = f16_to_f32(R.d[st] & 0xffffu);
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) {
      h4 xh[NBT], xlo[NBT];
      f4 XS[NBT];
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        const char* xp = xl0 + 16 * bt * RS + (128 * u + 16 * sb) * XE;
        if constexpr (XF16) {
          xh[bt] = __builtin_bit_cast(h4, *reinterpret_cast<const uint2*>(xp));
          XS[bt] = __builtin_amdgcn_mfma_f32_16x16x16f16(xh[bt], ones, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        } else {
          const float4 v4 = *reinterpret_cast<const float4*>(xp);
          const float v[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const _Float16 hv = (_Float16)v[e];
            xh[bt][e] = hv;
            xlo[bt][e] = (_Float16)(v[e] - (float)hv);
          }
          f4 t = __builtin_amdgcn_mfma_f32_16x16x16f16(xh[bt], ones, (f4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          XS[bt] = __builtin_amdgcn_mfma_f32_16x16x16f16(xlo[bt], ones, t, 0, 0, 0);
        }
      }
      f4 NXS[NBT];
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) NXS[bt] = XS[bt] * -1056.0f;
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        const uint32_t scw = sb < 4 ? R.sc[st].x : R.sc[st].y;
        const float sc = (float)(int8_t)((scw >> (8 * (sb & 3))) & 255u);
        const float ca = dv[st] * sc;
        const uint32_t qlw = (sb & 3) == 0 ? R.ql[st].x : (sb & 3) == 1 ? R.ql[st].y : (sb & 3) == 2 ? R.ql[st].z : R.ql[st].w;
        const h4 bq = q6_codes(qlw, (sb & 1) ? R.qh[st].y : R.qh[st].x, sb >> 2, 2 * (sb >> 1));
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
          // the chain starts from -1056 XS: P = sum (q - 32) x
          f4 P = __builtin_amdgcn_mfma_f32_16x16x16f16(xh[bt], bq, NXS[bt], 0, 0, 0);
          if constexpr (!XF16) P = __builtin_amdgcn_mfma_f32_16x16x16f16(xlo[bt], bq, P, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) Y[st][bt][r] = fmaf(ca, P[r], Y[st][bt][r]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // PF halves in flight; loads past the last half re-read it (cache hits)
  W buf[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) load(min(i, H - 1), buf[i]);
  for (int u = 0; u < H; u += PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      if (u + i < H) compute(u + i, buf[i]);
      load(min(u + i + PF, H - 1), buf[i]);
    }
  }
#pragma unroll
  for (int st = 0; st < NS; ++st) {
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
      }
  }
}

#ifndef Q6_LPF
#define Q6_LPF 2
#endif
// split of the 128-element halves: depends on the matrix shape only
inline int q6k_split(const GemvArgs& a) {
  const int tiles = (a.n_out + 31) / 32, H = a.n_in / 128;
  int ks = 1;
  while (ks < 8 && tiles * ks < 1024 && H / (2 * ks) >= 2) ks *= 2;
  return ks;
}

template <int NBT, int KS, bool XF16, int EPI>
void q6k_launch(const GemvArgs& a, int nb, hipStream_t s) {
  const int tiles = (a.n_out + 31) / 32;
  const size_t xlds = (size_t)16 * NBT * x_lds_stride(a.n_in, XF16);
  if (KS == 1 && xlds <= kXLdsMax)
    hipLaunchKernelGGL((q6k_lds_kernel<NBT, Q6_LPF, XF16, EPI>), dim3((tiles + kTilesKS1 - 1) / kTilesKS1),
                       dim3(64 * kTilesKS1), xlds, s, a, nb);
  else if constexpr (KS == 1)
    hipLaunchKernelGGL((q6k_mma_kernel<NBT, KS, XF16, EPI>), dim3((tiles + kTilesKS1 - 1) / kTilesKS1),
                       dim3(64 * kTilesKS1), 0, s, a, nb);
  else
    hipLaunchKernelGGL((q6k_mma_kernel<NBT, KS, XF16, EPI>), dim3(tiles), dim3(64 * KS), 0, s, a, nb);
}

template <int NBT, int KS, bool XF16, int EPI>
void q6k_launch_part(const GemvArgs& a, int nb, int gs, hipStream_t s) {
  const int tiles = (a.n_out + 31) / 32;
  GemvArgs p = a;
  float* ws = part_workspace(a, nb, gs, false, s);
  p.y = ws;
  hipLaunchKernelGGL((q6k_mma_kernel<NBT, KS, XF16, EPI, true>), dim3(tiles, gs), dim3(64 * KS), 0, s, p, nb);
  launch_part_reduce<EPI>(a, ws, gs, nb, s);
}

template <int NBT, bool XF16, int EPI>
void q6k_launch_ks(const GemvArgs& a, int nb, hipStream_t s) {
  if (const int gs = grid_split((a.n_out + 31) / 32, a.n_in / 128, 16); gs > 1) {
    switch (grid_split_ks(a.n_in / 128, gs)) {
      case 2: return q6k_launch_part<NBT, 2, XF16, EPI>(a, nb, gs, s);
      case 4: return q6k_launch_part<NBT, 4, XF16, EPI>(a, nb, gs, s);
      default: return q6k_launch_part<NBT, 8, XF16, EPI>(a, nb, gs, s);
    }
  }
  switch (q6k_split(a)) {
    case 1: return q6k_launch<NBT, 1, XF16, EPI>(a, nb, s);
    case 2: return q6k_launch<NBT, 2, XF16, EPI>(a, nb, s);
    case 4: return q6k_launch<NBT, 4, XF16, EPI>(a, nb, s);
    default: return q6k_launch<NBT, 8, XF16, EPI>(a, nb, s);
  }
}

template <bool XF16, int EPI>
void q6k_launch_wide(const GemvArgs& a, int nb, hipStream_t s) {
  if constexpr (EPI != EPI_SWIGLU) {
    switch (q6k_split(a)) {
      case 1: return q6k_launch<4, 1, XF16, EPI>(a, nb, s);
      case 2: return q6k_launch<4, 2, XF16, EPI>(a, nb, s);
      default: return q6k_launch<4, 4, XF16, EPI>(a, nb, s);
    }
  }
}

template <bool XF16, int EPI>
void q6k_rows(GemvArgs a, int nrows, hipStream_t s) {
  const size_t xel = XF16 ? 2 : 4;
  while (nrows > 0) {
    // 33..64 rows as one launch of four 16-row batch tiles where the k split
    // keeps them in registers (tall matrices: the weights stream once for all
    // rows); a row's sums do not depend on the batch tiles
    // (not the one-wave-per-tile form of very tall matrices: its four-tile
    // registers measured slower than two 32-row launches)
    const int ks6 = q6k_split(a);
    const bool wide = ks6 >= 2 && ks6 <= 4 && grid_split((a.n_out + 31) / 32, a.n_in / 128, 16) == 1 &&
                      EPI != EPI_SWIGLU;
    const int nb = nrows < (wide ? 64 : 32) ? nrows : (wide ? 64 : 32);
    if (nb > 32) q6k_launch_wide<XF16, EPI>(a, nb, s);
    else if (nb > 16) q6k_launch_ks<2, XF16, EPI>(a, nb, s);
    else q6k_launch_ks<1, XF16, EPI>(a, nb, s);
    PGD_HIP(hipGetLastError());
    nrows -= nb;
    a.x = reinterpret_cast<const uint8_t*>(a.x) + (size_t)nb * a.ldx * xel;
    a.y += (size_t)nb * a.ldy;
    if (a.res) a.res += (size_t)nb * a.ldres;
  }
}

}  // namespace

bool q4k_mma_ok(const GemvArgs& a) { return a.n_in % 64 == 0; }

// whole 128-element halves and 16-byte aligned activation rows
bool q6k_mma_ok(const GemvArgs& a, int epi) { return a.n_in % 128 == 0 && a.ldx % 4 == 0 && epi != EPI_SWIGLU; }

void run_q6k_mma(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s) {
  if (x_f16) {
    if (epi == EPI_RES) q6k_rows<true, EPI_RES>(a, nrows, s);
    else q6k_rows<true, EPI_STORE>(a, nrows, s);
  } else {
    if (epi == EPI_RES) q6k_rows<false, EPI_RES>(a, nrows, s);
    else q6k_rows<false, EPI_STORE>(a, nrows, s);
  }
}

void run_q4k_mma(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s) {
  if (x_f16) {
    if (epi == EPI_SWIGLU) q4k_rows<true, EPI_SWIGLU>(a, nrows, s);
    else if (epi == EPI_RES) q4k_rows<true, EPI_RES>(a, nrows, s);
    else q4k_rows<true, EPI_STORE>(a, nrows, s);
  } else {
    if (epi == EPI_SWIGLU) q4k_rows<false, EPI_SWIGLU>(a, nrows, s);
    else if (epi == EPI_RES) q4k_rows<false, EPI_RES>(a, nrows, s);
    else q4k_rows<false, EPI_STORE>(a, nrows, s);
  }
}

}  // namespace gemv
}  // namespace pgd
