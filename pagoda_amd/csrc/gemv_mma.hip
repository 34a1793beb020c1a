// gemv_mma.hip — MLX affine-8 (group 64) GEMV / skinny GEMM on the matrix cores.
//
// Y[b, n] = sum_k x[b, k] * (s[n, g] * c[n, k] + bias[n, g]),  g = k / 64,
// for up to 32 batch rows per launch, in two 16-row batch tiles. Per group:
//   P[b, n] = sum_k (1024 + c[n,k]) * (xh[b,k] + xl[b,k])    4 x v_mfma_f32_16x16x32_f16
//   Y[b, n] += s[n,g] * (P[b, n] - 1024 * XSP[b,g]) + bias[n,g] * XS[b,g]
// xh = f16(x) and xl = f16(x - xh) carry x to ~22 bits; 1024 + c is exact in
// f16 and is what one byte permute makes of a code; XS = sum x and XSP =
// sum (xh + xl) over the group in f32 (the subtraction cancels the offset to
// ~1e-6 of the group's sum).
// The batch row is the MFMA's M index and the weight row its N index: a lane
// owns one weight row (one scale/bias per group) and four batch rows. Every
// batch row goes through the same instruction sequence and the same split of
// the groups whatever the batch size, so a batched call is bitwise equal to
// single-row calls.
//
// Activations are converted once (a8_xprep_kernel, or fused into the RMSNorm
// that produces them, a8_norm_prep_kernel) into the MFMA operand order;
// weights are stored tiled (32 rows x 64 codes per 2 KiB block).
//
// Streaming: a workgroup of kKS waves shares one 32-row tile (two for wide
// matrices at full batch) and splits its groups between the waves. Each wave
// keeps a private LDS ring of P stages; a stage holds everything one group
// needs and is filled by direct global->LDS loads (weights, scale/bias,
// activation operands, per-row constants). All loads of the loop go to LDS,
// so they retire in issue order and one explicit vmcnt wait per group keeps
// the next P-1 groups in flight; the compiler sees no loaded registers to
// wait on. Only the rows the batch needs are staged (one row, four rows, one
// or two 16-row tiles), which keeps stages small and many waves resident.
// Partial sums of the waves meet in LDS in a fixed order.
//
// Counterpart of affine_gemv / affine_gemm4 / gemv2_silu / gemv_res
// (pagoda-hf/src/qwen3_gemv.rs:54-306, 414-567).
#include "common.h"
#include "gemv_impl.h"
#include "quant.h"
#include "a8_stage_reads.h"
#include "a8_act.h"

namespace pgd {
namespace gemv {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

// four codes (one u32) -> two f16 pairs holding (code - 128)
__device__ inline void codes_to_h(uint32_t w, uint32_t& lo, uint32_t& hi) {
  // bytes [c, 0x64] form the f16 1024 + c
  lo = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
  hi = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
}

__device__ inline h8 codes8(uint32_t w0, uint32_t w1) {
  uint32_t c0, c1, c2, c3;
  codes_to_h(w0, c0, c1);
  codes_to_h(w1, c2, c3);
  return __builtin_bit_cast(h8, make_uint4(c0, c1, c2, c3));
}

// ---- activation prep (layout: a8_act.h) ----------------------------------
// one wave per (chunk, group, batch tile); lane = 4 * row + quarter
__global__ __launch_bounds__(256) void a8_xprep_kernel(const float* __restrict__ x, int ldx, a8act::Dst d,
                                                       int rows_end) {
  const size_t item = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int bt = (int)(item & 1);
  const size_t cg = item >> 1;
  const int g = (int)(cg % d.G), c = (int)(cg / d.G);
  if (32 * c >= d.rows) return;
  if (a8act::chunk_compact(d.rows, c) && bt) return;
  const int jr = lane >> 2, q = lane & 3;
  const int row = 32 * c + 16 * bt + jr;
  float v[16];
  if (row < rows_end) {
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
  // rows past rows_end keep what is there (another kernel writes them)
  const bool live = (a8act::chunk_compact(d.rows, c) ? (jr < 4) : true) && (rows_end == d.rows || row < rows_end);
  a8act::emit_slice(d, row, g, q, v, live);
}

// RMSNorm with a deferred scale (rms_zero, pagoda-hf/src/qwen3_5.rs:1736-1745,
// reordered): operands of x * w, and per (row, 32-wide half group) the sum of
// x^2 (each lane's 16 in order, then quarters 0 + 1 or 2 + 3). Layout and
// lanes as a8_xprep_kernel; rss: [rows][K / 32].
__global__ __launch_bounds__(256) void a8_gnorm_prep_kernel(const float* __restrict__ x, int ldx,
                                                            const float* __restrict__ w, a8act::Dst d,
                                                            float* __restrict__ rss, int rows_end) {
  const size_t item = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int bt = (int)(item & 1);
  const size_t cg = item >> 1;
  const int g = (int)(cg % d.G), c = (int)(cg / d.G);
  if (32 * c >= d.rows) return;
  if (a8act::chunk_compact(d.rows, c) && bt) return;
  const int jr = lane >> 2, q = lane & 3;
  const int row = 32 * c + 16 * bt + jr;
  float v[16], ss = 0.0f;
  if (row < rows_end) {
    const float4* xp = reinterpret_cast<const float4*>(x + (size_t)row * ldx + (g << 6) + 16 * q);
    const float4* wp = reinterpret_cast<const float4*>(w + (g << 6) + 16 * q);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 f = xp[i], h = wp[i];
      v[4 * i] = f.x;
      v[4 * i + 1] = f.y;
      v[4 * i + 2] = f.z;
      v[4 * i + 3] = f.w;
#pragma unroll
      for (int e = 0; e < 4; ++e) ss += v[4 * i + e] * v[4 * i + e];
      v[4 * i] *= h.x;
      v[4 * i + 1] *= h.y;
      v[4 * i + 2] *= h.z;
      v[4 * i + 3] *= h.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = 0.0f;
  }
  ss += __shfl_xor(ss, 1, 64);  // half group: quarters (0 + 1), (2 + 3)
  const bool live = (a8act::chunk_compact(d.rows, c) ? (jr < 4) : true) && (rows_end == d.rows || row < rows_end);
  if (live && (q & 1) == 0 && row < rows_end) rss[(size_t)row * 2 * d.G + 2 * g + (q >> 1)] = ss;
  a8act::emit_slice(d, row, g, q, v, live);
}

// Fused RMSNorm (rms_zero, pagoda-hf/src/qwen3_5.rs:1736-1745) + activation
// prep: one workgroup of NT threads per output row; thread t owns 16-wide
// slices t, t+NT, ... (slice u = 4g + q), kept in registers between the two passes together
// with their norm weights, which are loaded with the row (one round trip).
constexpr int kNormMaxSlices = 8;  // n <= 256 * 16 * 8 (wide rows: 256 threads)
template <int NSL, int NT>
__global__ __launch_bounds__(NT) void a8_norm_prep_kernel(const float* __restrict__ x, int ldx,
                                                          const int* __restrict__ rows_idx, int rows, int n,
                                                          const float* __restrict__ w, float eps, float* y, int ldy,
                                                          a8act::Dst d) {
  constexpr int NW = NT / 64;
  __shared__ float red[NW];
  const int r = blockIdx.x, tid = threadIdx.x;
  const int src = rows_idx ? rows_idx[r] : r;
  const float* xr = x + (size_t)src * ldx;
  const int slices = n >> 4;
  float v[NSL][16], wv[NSL][16];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NSL; ++i) {
    const int u = tid + NT * i;
    if (u < slices) {
      const float4* p = reinterpret_cast<const float4*>(xr + 16 * u);
      const float4* wp = reinterpret_cast<const float4*>(w + 16 * u);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float4 f = p[e], g = wp[e];
        v[i][4 * e] = f.x;
        v[i][4 * e + 1] = f.y;
        v[i][4 * e + 2] = f.z;
        v[i][4 * e + 3] = f.w;
        wv[i][4 * e] = g.x;
        wv[i][4 * e + 1] = g.y;
        wv[i][4 * e + 2] = g.z;
        wv[i][4 * e + 3] = g.w;
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) ss += v[i][e] * v[i][e];
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = red[0];
#pragma unroll
  for (int k = 1; k < NW; ++k) tot += red[k];
  const float inv = 1.0f / sqrtf(tot / (float)n + eps);
#pragma unroll
  for (int i = 0; i < NSL; ++i) {
    const int u = tid + NT * i;
    const bool live = u < slices;  // uniform per group of four lanes (slices % 4 == 0)
    if (live) {
#pragma unroll
      for (int e = 0; e < 16; ++e) v[i][e] = v[i][e] * inv * wv[i][e];
      if (y) {
        float4* yp = reinterpret_cast<float4*>(y + (size_t)r * ldy + 16 * u);
#pragma unroll
        for (int e = 0; e < 4; ++e) yp[e] = make_float4(v[i][4 * e], v[i][4 * e + 1], v[i][4 * e + 2], v[i][4 * e + 3]);
      }
    }
    // slice u = 4 g + q: quarter partners are adjacent lanes
    if (i * NT < slices) a8act::emit_slice(d, r, u >> 2, u & 3, v[i], live);
  }
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

// per-mode stage geometry: activation bytes, constant bytes, loads of both
template <int MODE> struct StageGeo;
template <> struct StageGeo<0> { static constexpr int NBT = 1, XB = 1024, CB = 256, KX = 2; };
template <> struct StageGeo<1> { static constexpr int NBT = 1, XB = 4096, CB = 256, KX = 5; };
template <> struct StageGeo<2> { static constexpr int NBT = 2, XB = 8192, CB = 512, KX = 10; };
template <> struct StageGeo<3> { static constexpr int NBT = 1, XB = 256, CB = 16, KX = 2; };


__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)((const __attribute__((address_space(3))) char*)p);
}
// s_waitcnt vmcnt(N) with expcnt and lgkmcnt left at their maxima
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void dma16(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds((glb_void*)g, (lds_void*)l, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds((glb_void*)g, (lds_void*)l, 4, 0, 0);
}

// KS: ranges the groups are split into (fixed per matrix shape, so every batch
// size sums alike); KP: waves per workgroup, each summing R = KS / KP
// consecutive ranges into separate accumulators; P: ring stages per wave.
template <int MODE, int KS, int KP, int P, int MT, int EPI>
__global__ __launch_bounds__(64 * KP) void a8_mma_kernel(GemvArgs a, const uint4* __restrict__ XA,
                                                         const float* __restrict__ CA, int nb) {
  using Geo = StageGeo<MODE>;
  static_assert(KS % KP == 0, "whole ranges per wave");
  constexpr int R = KS / KP;
  constexpr int NBT = Geo::NBT;
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr int NSM = 2 * MT;              // 16-row subtiles per matrix (MT 32-row tiles)
  constexpr int NS = DUAL ? 2 * NSM : NSM;  // subtiles per wave; SwiGLU: gate ones, then up ones
  constexpr int SBD = (NS + 3) / 4;         // scale/bias loads per group (16 rows x 4 subtiles each)
  static_assert(MODE == 2 || NS <= 4, "wide waves only with 32-row launches");
  constexpr int SBOFF = NS * 1024, XOFF = SBOFF + (MODE == 3 ? NS * 64 : SBD * 256), COFF = XOFF + Geo::XB;
  constexpr int STAGE = COFF + Geo::CB;
  constexpr int NDMA = NS + SBD + Geo::KX;  // loads per group
  constexpr int NWAIT = (P - 1) * NDMA;
  constexpr size_t RING = (size_t)KP * P * STAGE;
  constexpr size_t RED = sizeof(f4) * (KS - 1) * NS * NBT * 64;
  static_assert(RING <= 160 * 1024 && RED <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) char smem[RING > RED ? RING : RED];
  auto& red = *reinterpret_cast<f4(*)[KS - 1][NS][NBT][64]>(smem);

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, q = lane >> 4;  // MFMA column (weight row in subtile), k quarter / row quad
  const int G = a.n_in >> 6;
  const int ntiles = (a.n_out + 31) >> 5;
  char* ring = smem + (size_t)wave * P * STAGE;
  const uint32_t ring_lds = lds_addr(ring);

  // subtile st: matrix (gate / up), tile, row within the tile
  auto sub_src = [&](int st, const uint8_t* g0p, const uint8_t* u0p, int& tile, int& r) -> const uint8_t* {
    const int sl = DUAL ? st % NSM : st;
    // a missing last tile re-reads the last real one; its outputs are dropped
    tile = min(blockIdx.x * MT + (sl >> 1), ntiles - 1);
    r = 16 * (sl & 1) + j;
    return (DUAL && st >= NSM) ? u0p : g0p;
  };
  // weights: each lane stages (and later reads back) its own 16 B of each subtile
  const uint8_t* wsrc[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    int tile, r;
    const uint8_t* p = sub_src(st, a.p0, a.u0, tile, r);
    wsrc[st] = p + ((size_t)tile * G << 11) + (q >> 1) * 1024 + r * 32 + (q & 1) * 16;
  }
  // scale/bias: load d, lane L stages subtile min(4 d + L / 16, NS - 1), row L % 16
  const uint32_t* ssrc[SBD];
#pragma unroll
  for (int d = 0; d < SBD; ++d) {
    int tile, r;
    const uint8_t* ps = sub_src(min(4 * d + (lane >> 4), NS - 1), a.p1, a.u1, tile, r);
    ssrc[d] = reinterpret_cast<const uint32_t*>(ps) + ((size_t)tile * G << 5) + r;
  }
  // activation sources (uint4 / float offsets within an item) and LDS read offsets
  int xsrc, csrc;
  uint32_t xrd, crd;
  if constexpr (MODE == 3) {  // compact; lane L < 16: operand L / 4 of k quarter L % 4, row 0
    xsrc = lane;
    csrc = (lane & 3) * 4;
    xrd = q * 16;
    crd = 0;
  } else if constexpr (MODE == 0) {  // compact; lane L: operand L / 16, k quarter (L / 4) % 4, row L % 4
    xsrc = (lane & 3) * 16 + (lane >> 4) * 4 + ((lane >> 2) & 3);
    csrc = lane & 15;
    xrd = (q * 4 + (j & 3)) * 16;
    crd = 0;
  } else {
    xsrc = lane;
    csrc = lane;
    xrd = lane * 16;
    crd = 16 * q;
  }

  f4 Y[NS][NBT];
  f4 Ys[R > 1 ? R - 1 : 1][NS][NBT];  // finished ranges of this wave
#pragma unroll
  for (int st = 0; st < NS; ++st)
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) {
      Y[st][bt] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < (R > 1 ? R - 1 : 1); ++r) Ys[r][st][bt] = (f4){0.f, 0.f, 0.f, 0.f};
    }

  // stage u <- group g: exactly NDMA loads, whatever the mode's lane masks
  auto issue = [&](int g, int u) {
    char* sb = ring + u * STAGE;
#pragma unroll
    for (int st = 0; st < NS; ++st) dma16(wsrc[st] + ((size_t)g << 11), sb + st * 1024);
#pragma unroll
    for (int d = 0; d < SBD; ++d)
      if (MODE != 3 || lane < 16 * NS) dma4(ssrc[d] + ((size_t)g << 5), sb + SBOFF + d * 256);
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) {
      const size_t item = (size_t)g * 2 + bt;
      if constexpr (MODE == 3) {
        if (lane < 16) dma16(XA + (size_t)g * 64 + xsrc, sb + XOFF);
        if (lane < 4) dma4(CA + (size_t)g * 16 + csrc, sb + COFF);
      } else if constexpr (MODE == 0) {
        dma16(XA + (size_t)g * 64 + xsrc, sb + XOFF);
        dma4(CA + (size_t)g * 16 + csrc, sb + COFF);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16(XA + item * 256 + i * 64 + xsrc, sb + XOFF + bt * 4096 + i * 1024);
        dma4(CA + item * 64 + csrc, sb + COFF + bt * 256);
      }
    }
  };

  auto compute = [&](int u) {
    const uint32_t base = ring_lds + u * STAGE;
    uint4 W[NS];
    uint32_t S[NS];
    uint4 X[NBT][4];
    float CPv[NBT][4], XSv[NBT][4];  // -1024 XSP and XS of batch rows 16 bt + 4 q + r: half A + half B
    if constexpr (MODE == 3) {
      float4 c1;
      StageReads<MODE, NS>::run(base + 16 * lane, base + SBOFF + 4 * j, base + XOFF + xrd, base + COFF + crd, W, S, X,
                                c1);
      const float cp = c1.x + c1.y, xs = c1.z + c1.w;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        CPv[0][r] = cp;
        XSv[0][r] = xs;
      }
    } else {
      float4 CC[NBT][4];
      StageReads<MODE, NS>::run(base + 16 * lane, base + SBOFF + 4 * j, base + XOFF + xrd, base + COFF + crd, W, S, X,
                                CC);
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        CPv[bt][0] = CC[bt][0].x + CC[bt][1].x;
        CPv[bt][1] = CC[bt][0].y + CC[bt][1].y;
        CPv[bt][2] = CC[bt][0].z + CC[bt][1].z;
        CPv[bt][3] = CC[bt][0].w + CC[bt][1].w;
        XSv[bt][0] = CC[bt][2].x + CC[bt][3].x;
        XSv[bt][1] = CC[bt][2].y + CC[bt][3].y;
        XSv[bt][2] = CC[bt][2].z + CC[bt][3].z;
        XSv[bt][3] = CC[bt][2].w + CC[bt][3].w;
      }
    }
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      const h8 b0 = codes8(W[st].x, W[st].y);
      const h8 b1 = codes8(W[st].z, W[st].w);
      const float sc = bf16_to_f32(S[st] & 0xffffu);
      const float bi = bf16_to_f32(S[st] >> 16);
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        // the MFMA adds the codes' dot product to -1024 XSP (the 1024 + c offset)
        f4 Pm = {CPv[bt][0], CPv[bt][1], CPv[bt][2], CPv[bt][3]};
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[bt][0]), b0, Pm, 0, 0, 0);
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[bt][1]), b1, Pm, 0, 0, 0);
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[bt][2]), b0, Pm, 0, 0, 0);
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[bt][3]), b1, Pm, 0, 0, 0);
        // one-row launches keep only row 0 (the rows of the other lanes are
        // never stored)
#pragma unroll
        for (int r = 0; r < (MODE == 3 ? 1 : 4); ++r)
          Y[st][bt][r] = fmaf(bi, XSv[bt][r], fmaf(sc, Pm[r], Y[st][bt][r]));
      }
    }
  };

  // groups of this wave: R consecutive ranges of `per` groups, streamed as one
  // run; prefetches past its end re-read the last group (an L2 hit), so every
  // step issues NDMA loads and the wait count stays fixed
  const int per = (G + KS - 1) / KS;
  const int g0 = min(G, wave * R * per), g1 = min(G, g0 + R * per);
  int rc = 0, rend = g0 + per;  // current range and its end
  auto close_range = [&](int gg) {
    if constexpr (R > 1) {
      if (gg + 1 == rend && rc < R - 1) {
#pragma unroll
        for (int r = 0; r < R - 1; ++r)
          if (r == rc) {
#pragma unroll
            for (int st = 0; st < NS; ++st)
#pragma unroll
              for (int bt = 0; bt < NBT; ++bt) Ys[r][st][bt] = Y[st][bt];
          }
#pragma unroll
        for (int st = 0; st < NS; ++st)
#pragma unroll
          for (int bt = 0; bt < NBT; ++bt) Y[st][bt] = (f4){0.f, 0.f, 0.f, 0.f};
        ++rc;
        rend += per;
      }
    }
  };
  if (g0 < g1) {
#pragma unroll
    for (int u = 0; u < P; ++u) issue(min(g0 + u, g1 - 1), u);
    int g = g0;
    for (; g + P <= g1; g += P) {
#pragma unroll
      for (int u = 0; u < P; ++u) {
        wait_vmcnt<NWAIT>();  // group g + u has landed; the next P - 1 stay in flight
        compute(u);
        close_range(g + u);
        issue(min(g + u + P, g1 - 1), u);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    wait_vmcnt<0>();
#pragma unroll
    for (int u = 0; u < P - 1; ++u)
      if (g + u < g1) {
        compute(u);
        close_range(g + u);
      }
  }

  // deferred RMSNorm of the input: the waves share out the rows' 1/rms
  __shared__ float s_inv[32];
  if (a.rss) {
    for (int b = wave; b < nb; b += KP) {
      const float v = rss_inv(a.rss + (size_t)b * a.rss_nh, a.rss_nh, a.rss_n, a.rss_eps);
      if (lane == 0) s_inv[b] = v;
    }
  }

  // ---- split-K reduction (fixed order: range 0 + 1 + ... + KS-1) ----
  // range wave * R + r holds Ys[r] for r < rc, Y for r == rc, zero after
  wait_vmcnt<0>();
  __syncthreads();  // the reduction buffer overlays the rings
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int v = wave * R + r;
    if (v == 0) continue;
#pragma unroll
    for (int st = 0; st < NS; ++st)
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) {
        f4 val = (f4){0.f, 0.f, 0.f, 0.f};
        if (r == rc) val = Y[st][bt];
        if constexpr (R > 1) {
          if (r < rc && r < R - 1) val = Ys[r < R - 1 ? r : 0][st][bt];
        }
        red[v - 1][st][bt][lane] = val;
      }
  }
  __syncthreads();
  if (wave != 0) return;
  if constexpr (R > 1) {
    // wave 0's own first range
    if (rc > 0) {
#pragma unroll
      for (int st = 0; st < NS; ++st)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) Y[st][bt] = Ys[0][st][bt];
    }
  }
  for (int v = 0; v < KS - 1; ++v)
#pragma unroll
    for (int st = 0; st < NS; ++st)
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) Y[st][bt] += red[v][st][bt][lane];

  if (a.rss) {
#pragma unroll
    for (int st = 0; st < NS; ++st)
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int b = 16 * bt + 4 * q + r;
          Y[st][bt][r] *= b < nb ? s_inv[b] : 1.0f;
        }
  }

  // ---- epilogue: lane holds weight row n for batch rows 16bt + 4q + r ----
  if constexpr (DUAL) {
    if (a.oact.XA) {
      // each tile's 32 products of a batch row are one half of group tile / 2
      // of the down projection's input: transpose through LDS, then lane L
      // prepares 16 of them (row L % 32, quarter pair L / 32)
      float* hb = reinterpret_cast<float*>(smem);  // [32][33]
#pragma unroll
      for (int ti = 0; ti < MT; ++ti) {
        const int tile = blockIdx.x * MT + ti;
        if (tile >= ntiles) break;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int b = 16 * bt + 4 * q + r;
              if (b < nb) hb[b * 33 + 16 * h + j] = silu_f(Y[2 * ti + h][bt][r]) * Y[NSM + 2 * ti + h][bt][r];
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int b = lane & 31, h = lane >> 5;
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = b < nb ? hb[b * 33 + 16 * h + e] : 0.0f;
        a8act::emit_slice<32>(a.oact, a.row0 + b, tile >> 1, (tile & 1) * 2 + h, v, b < nb);
      }
      if (!a.y) return;
    }
  }
  // residual + next RMSNorm's input: the new rows also go to LDS (with one
  // tile per workgroup: 32 outputs = half a group of the next activation)
  const bool emit = EPI == EPI_RES && MT == 1 && a.nact.XA;
  float* hn = reinterpret_cast<float*>(smem);  // [32][33]
#pragma unroll
  for (int st = 0; st < NSM; ++st) {
    const int n = (blockIdx.x * MT + (st >> 1)) * 32 + 16 * (st & 1) + j;
    if (n >= a.n_out) continue;
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int b = 16 * bt + 4 * q + r;
        if (b >= nb) continue;
        const size_t o = (size_t)b * a.ldy + n;
        if constexpr (EPI == EPI_STORE) {
          a.y[o] = Y[st][bt][r];
          if (a.cout && a.conv_k != 4 && n < a.conv_n) conv_channel(a, a.row0 + b, n, Y[st][bt][r]);
        }
        if constexpr (EPI == EPI_RES) {
          const float h = a.res[(size_t)b * a.ldres + n] + Y[st][bt][r];
          a.y[o] = h;
          if (emit) hn[b * 33 + 16 * st + j] = h;
        }
        if constexpr (EPI == EPI_SWIGLU) a.y[o] = silu_f(Y[st][bt][r]) * Y[NSM + st][bt][r];
      }
  }
  if constexpr (EPI == EPI_STORE) {
    if (a.cout && a.conv_k == 4) {
      // causal conv of this lane's (row, channel) pairs, conv_channel's
      // arithmetic and order: every state and weight is loaded before any
      // store, so the loads of all pairs overlap
      constexpr int NR = MODE == 3 ? 1 : 4, NPR = NSM * NBT * NR;
      float sv[NPR][3], wv[NSM][4], xv[NPR];
      float* sp[NPR];
      bool live[NPR];
#pragma unroll
      for (int st = 0; st < NSM; ++st) {
        const int n = (blockIdx.x * MT + (st >> 1)) * 32 + 16 * (st & 1) + j;
        const bool cn = n < a.n_out && n < a.conv_n;
#pragma unroll
        for (int k = 0; k < 4; ++k) wv[st][k] = cn ? a.cw[(size_t)n * 4 + k] : 0.0f;
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            const int i = (st * NBT + bt) * NR + r, b = 16 * bt + 4 * q + r;
            live[i] = cn && b < nb;
            xv[i] = Y[st][bt][r];
            sp[i] = live[i] ? a.cbase[a.row0 + b] + a.coff + (size_t)n * 3 : nullptr;
#pragma unroll
            for (int k = 0; k < 3; ++k) sv[i][k] = live[i] ? sp[i][k] : 0.0f;
          }
      }
#pragma unroll
      for (int st = 0; st < NSM; ++st) {
        const int n = (blockIdx.x * MT + (st >> 1)) * 32 + 16 * (st & 1) + j;
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            const int i = (st * NBT + bt) * NR + r, b = 16 * bt + 4 * q + r;
            if (!live[i]) continue;
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < 3; ++k) acc += sv[i][k] * wv[st][k];
            acc += xv[i] * wv[st][3];
            a.cout[(size_t)(a.row0 + b) * a.ldc + n] = acc / (1.0f + expf(-acc));
            sp[i][0] = sv[i][1];
            sp[i][1] = sv[i][2];
            sp[i][2] = xv[i];
          }
      }
    }
  }
  if constexpr (EPI == EPI_RES && MT == 1) {
    if (emit) {
      // as a8_gnorm_prep_kernel: lane L takes row L % 32, quarter pair L / 32
      // of the tile; sum of h^2 in k order, then operands of h * nw
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int tile = blockIdx.x, b = lane & 31, hh = lane >> 5;
      const bool live = b < nb;
      const float4* wp = reinterpret_cast<const float4*>(a.nw + tile * 32 + 16 * hh);
      float v[16], ss = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 w4 = wp[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * i + e] = live ? hn[b * 33 + 16 * hh + 4 * i + e] : 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) ss += v[4 * i + e] * v[4 * i + e];
        v[4 * i] *= w4.x;
        v[4 * i + 1] *= w4.y;
        v[4 * i + 2] *= w4.z;
        v[4 * i + 3] *= w4.w;
      }
      ss += __shfl_xor(ss, 32, 64);
      if (live && hh == 0) a.nrss[(size_t)(a.row0 + b) * (a.n_out >> 5) + tile] = ss;
      a8act::emit_slice<32>(a.nact, a.row0 + b, tile >> 1, (tile & 1) * 2 + hh, v, live);
    }
  }
}

// ---- 17..32 rows: activation stage shared by the waves of a workgroup ----
// A workgroup holds T waves on T consecutive tiles, all on the same range r
// of the KS-way split of the groups (grid: tile blocks x KS). Each group's
// 32-row operands (8.5 KiB) are staged once per workgroup instead of once
// per tile: every wave loads a quarter of them next to its own weights, and
// one barrier per group publishes the stage. The range's partial sums go to
// part[r][row][n]; a8_reduce_kernel adds the KS ranges in order 0, 1, ...
// (the order of the in-workgroup reduction above), so results equal the
// other modes bit for bit.
// NC = activation chunks of 32 rows per launch (2: a 64-row launch streams
// the weights once for both; the second chunk must hold more than 4 rows,
// i.e. use the full operand layout).
template <int KS, int T, int P, int EPI, int NC>
__global__ __launch_bounds__(64 * T) void a8_mma_shared_kernel(GemvArgs a, const uint4* __restrict__ XA,
                                                               const float* __restrict__ CA, int nb,
                                                               float* __restrict__ part) {
  static_assert(T == 2 || T == 4 || T == 8, "operand quarters per wave");
  static_assert(NC == 1 || NC == 2, "one or two chunks");
  static_assert(T >= 2 * NC, "one constant block per wave");
  constexpr int NBT = 2 * NC;
  static_assert(EPI != EPI_SWIGLU, "one matrix per wave");
  constexpr int NS = 2;
  constexpr int CHUNK = 8192 + 512;         // per chunk: operands + constants of both batch tiles
  constexpr int SHARED = NC * CHUNK;
  constexpr int PERW = NS * 1024 + 256;     // a wave's weights + scale/bias
  constexpr int STAGE = SHARED + T * PERW;
  constexpr int XPW = 8 * NC / T;           // operand loads per wave (8 x 1 KiB per group and chunk)
  constexpr int NDMA = NS + 1 + XPW + 1;    // weights, scale/bias, operands, one constant block
  static_assert(P >= 3, "one stage is refilled while the next is in flight");
  constexpr int NWAIT = (P - 2) * NDMA;
  static_assert((size_t)P * STAGE <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) char smem[P * STAGE];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, q = lane >> 4;
  const int G = a.n_in >> 6;
  const int ntiles = (a.n_out + 31) >> 5;
  const int tile = blockIdx.x * T + wave;
  const int rtile = min(tile, ntiles - 1);  // a missing tile re-reads the last one; nothing is stored
  const int r = blockIdx.y;
  const int per = (G + KS - 1) / KS;
  const int g0 = min(G, r * per), g1 = min(G, g0 + per);
  const uint32_t smem_lds = lds_addr(smem);

  const uint8_t* wsrc[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const int row = 16 * st + j;
    wsrc[st] = a.p0 + ((size_t)rtile * G << 11) + (q >> 1) * 1024 + row * 32 + (q & 1) * 16;
  }
  const uint32_t* ssrc =
      reinterpret_cast<const uint32_t*>(a.p1) + ((size_t)rtile * G << 5) + 16 * min(lane >> 4, NS - 1) + j;
  // this wave's share of the operands: loads XPW * wave .. of the 8 NC (chunk =
  // load / 8, tile bt = load / 4 % 2, operand load % 4)
  const int x0 = XPW * wave;
  const int cbt = wave % (2 * NC);  // constant block (chunk cbt / 2, tile cbt % 2; later waves load copies)

  auto issue = [&](int g, int slot) {
    char* sb = smem + slot * STAGE;
    char* mine = sb + SHARED + wave * PERW;
#pragma unroll
    for (int st = 0; st < NS; ++st) dma16(wsrc[st] + ((size_t)g << 11), mine + st * 1024);
    dma4(ssrc + ((size_t)g << 5), mine + NS * 1024);
#pragma unroll
    for (int i = 0; i < XPW; ++i) {
      const int x = x0 + i, xc = x >> 3, xbt = (x >> 2) & 1, xi = x & 3;
      dma16(XA + (((size_t)xc * G + g) * 2 + xbt) * 256 + xi * 64 + lane, sb + xc * CHUNK + xbt * 4096 + xi * 1024);
    }
    const int cc = cbt >> 1, ct = cbt & 1;
    dma4(CA + (((size_t)cc * G + g) * 2 + ct) * 64 + lane, sb + cc * CHUNK + 8192 + ct * 256);
  };

  f4 Y[NS][NBT];
#pragma unroll
  for (int st = 0; st < NS; ++st)
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) Y[st][bt] = (f4){0.f, 0.f, 0.f, 0.f};

  // one chunk's two batch tiles at a time (the weights are read again per chunk)
  auto compute_chunk = [&](int slot, int c) {
    const uint32_t base = smem_lds + slot * STAGE;
    const uint32_t mine = base + SHARED + wave * PERW;
    const uint32_t cb = base + c * CHUNK;
    uint4 W[NS];
    uint32_t S[NS];
    uint4 X[2][4];
    float4 CC[2][4];
    StageReads<2, NS>::run(mine + 16 * lane, mine + NS * 1024 + 4 * j, cb + 16 * lane, cb + 8192 + 16 * q, W, S, X, CC);
    float CPv[2][4], XSv[2][4];
#pragma unroll
    for (int bt = 0; bt < 2; ++bt) {
      CPv[bt][0] = CC[bt][0].x + CC[bt][1].x;
      CPv[bt][1] = CC[bt][0].y + CC[bt][1].y;
      CPv[bt][2] = CC[bt][0].z + CC[bt][1].z;
      CPv[bt][3] = CC[bt][0].w + CC[bt][1].w;
      XSv[bt][0] = CC[bt][2].x + CC[bt][3].x;
      XSv[bt][1] = CC[bt][2].y + CC[bt][3].y;
      XSv[bt][2] = CC[bt][2].z + CC[bt][3].z;
      XSv[bt][3] = CC[bt][2].w + CC[bt][3].w;
    }
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      const h8 b0 = codes8(W[st].x, W[st].y);
      const h8 b1 = codes8(W[st].z, W[st].w);
      const float sc = bf16_to_f32(S[st] & 0xffffu);
      const float bi = bf16_to_f32(S[st] >> 16);
#pragma unroll
      for (int bt = 0; bt < 2; ++bt) {
        // the MFMA adds the codes' dot product to -1024 XSP (the 1024 + c offset)
        f4 Pm = {CPv[bt][0], CPv[bt][1], CPv[bt][2], CPv[bt][3]};
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[bt][0]), b0, Pm, 0, 0, 0);
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[bt][1]), b1, Pm, 0, 0, 0);
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[bt][2]), b0, Pm, 0, 0, 0);
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[bt][3]), b1, Pm, 0, 0, 0);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          Y[st][2 * c + bt][rr] = fmaf(bi, XSv[bt][rr], fmaf(sc, Pm[rr], Y[st][2 * c + bt][rr]));
      }
    }
  };
  auto compute = [&](int slot) {
#pragma unroll
    for (int c = 0; c < NC; ++c) compute_chunk(slot, c);
  };

  // step i: wait for group g0 + i (P - 2 later groups stay in flight), publish
  // it, refill the stage everyone finished at step i - 1, compute
  if (g0 < g1) {
#pragma unroll
    for (int u = 0; u < P - 1; ++u) issue(min(g0 + u, g1 - 1), u);
    int g = g0;
    for (; g + P <= g1; g += P) {
#pragma unroll
      for (int u = 0; u < P; ++u) {
        wait_vmcnt<NWAIT>();
        __syncthreads();
        issue(min(g + u + P - 1, g1 - 1), (u + P - 1) % P);
        compute(u);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // tail: no more loads; the remaining stages arrive in order
#pragma unroll
    for (int u = 0; u < P - 1; ++u) {
      if (g + u < g1) {
        wait_vmcnt<0>();
        __syncthreads();
        compute(u);
      }
    }
  }
  wait_vmcnt<0>();
  if (tile >= ntiles) return;
  // partial sums of range r: part[r][b][n]
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const int n = tile * 32 + 16 * st + j;
    if (n >= a.n_out) continue;
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int b = 16 * bt + 4 * q + rr;
        if (b < nb) part[((size_t)r * nb + b) * a.n_out + n] = Y[st][bt][rr];
      }
  }
}

// Reduction workgroups are one wave, so a 32-row reduction of a 5120-wide
// matrix spreads over 320 workgroups instead of 96 (measured 5.4 -> 5.2 us;
// the kernel is bound by one load round trip plus launch).
constexpr int kRedT = 64;

// y[b][n] = (res[b][n] +) sum over ranges, in range order; each thread sums 4
// consecutive outputs of one row with all KS loads issued before the adds
template <int KS, int EPI>
__global__ __launch_bounds__(kRedT) void a8_reduce_kernel(GemvArgs a, int nb, const float* __restrict__ part) {
  const int n4 = a.n_out >> 2;
  const int b = blockIdx.y, i4 = blockIdx.x * kRedT + threadIdx.x;
  // deferred RMSNorm of the input (whole waves, before any lane leaves)
  const float inv = a.rss ? rss_inv(a.rss + (size_t)b * a.rss_nh, a.rss_nh, a.rss_n, a.rss_eps) : 1.0f;
  if (i4 >= n4) return;
  const int n = i4 * 4;
  const size_t plane = (size_t)nb * a.n_out, e = (size_t)b * a.n_out + n;
  float4 v[KS];
#pragma unroll
  for (int r = 0; r < KS; ++r) v[r] = *reinterpret_cast<const float4*>(part + r * plane + e);
  float4 y = v[0];
#pragma unroll
  for (int r = 1; r < KS; ++r) {
    y.x += v[r].x;
    y.y += v[r].y;
    y.z += v[r].z;
    y.w += v[r].w;
  }
  if (a.rss) {
    y.x *= inv;
    y.y *= inv;
    y.z *= inv;
    y.w *= inv;
  }
  const size_t o = (size_t)b * a.ldy + n;
  if constexpr (EPI == EPI_RES) {
    const float* rs = a.res + (size_t)b * a.ldres + n;
    y.x = rs[0] + y.x;
    y.y = rs[1] + y.y;
    y.z = rs[2] + y.z;
    y.w = rs[3] + y.w;
  }
  a.y[o] = y.x;
  a.y[o + 1] = y.y;
  a.y[o + 2] = y.z;
  a.y[o + 3] = y.w;
  if constexpr (EPI == EPI_STORE) {
    // causal conv of the conv channels (every row its sequence's only token),
    // as the split-K kernels' epilogue runs it
    if (a.cout && n < a.conv_n) {
      const float v[4] = {y.x, y.y, y.z, y.w};
      const int row = a.row0 + b;
      if (a.conv_k == 4 && n + 4 <= a.conv_n) {
        // the four channels' states and weights are loaded before any store,
        // so the loads overlap (conv_channel's arithmetic and order)
        float* cs = a.cbase[row] + a.coff + (size_t)n * 3;
        const float* wt = a.cw + (size_t)n * 4;
        float sv[12], wv[16];
#pragma unroll
        for (int i = 0; i < 12; ++i) sv[i] = cs[i];
#pragma unroll
        for (int i = 0; i < 16; ++i) wv[i] = wt[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float acc = 0.0f;
#pragma unroll
          for (int k = 0; k < 3; ++k) acc += sv[3 * e + k] * wv[4 * e + k];
          acc += v[e] * wv[4 * e + 3];
          a.cout[(size_t)row * a.ldc + n + e] = acc / (1.0f + expf(-acc));
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          cs[3 * e] = sv[3 * e + 1];
          cs[3 * e + 1] = sv[3 * e + 2];
          cs[3 * e + 2] = v[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < a.conv_n) conv_channel(a, row, n + e, v[e]);
      }
    }
  }
}

// The residual reduction of a8_reduce_kernel that also emits the next
// RMSNorm's deferred input (as a8_gnorm_prep_kernel, bit for bit): a thread
// holds 8 consecutive outputs of row b, lanes 2s and 2s + 1 the two halves of
// 16-wide slice s. Slice sums run in k order: the first half's lane starts
// them, the second continues from its partner's totals.
template <int KS>
__global__ __launch_bounds__(kRedT) void a8_reduce_emit_kernel(GemvArgs a, int nb, const float* __restrict__ part) {
  const int n8 = a.n_out >> 3;
  const int b = blockIdx.y, i8 = blockIdx.x * kRedT + threadIdx.x;
  const bool live = i8 < n8;  // every lane stays for the shuffles
  const int n = (live ? i8 : 0) * 8;
  const size_t plane = (size_t)nb * a.n_out, e = (size_t)b * a.n_out + n;
  float4 v0[KS], v1[KS];
#pragma unroll
  for (int r = 0; r < KS; ++r) {
    v0[r] = *reinterpret_cast<const float4*>(part + r * plane + e);
    v1[r] = *reinterpret_cast<const float4*>(part + r * plane + e + 4);
  }
  const float* rs = a.res + (size_t)b * a.ldres + n;
  const float4 r0 = *reinterpret_cast<const float4*>(rs), r1 = *reinterpret_cast<const float4*>(rs + 4);
  float4 y0 = v0[0], y1 = v1[0];
#pragma unroll
  for (int r = 1; r < KS; ++r) {
    y0.x += v0[r].x;
    y0.y += v0[r].y;
    y0.z += v0[r].z;
    y0.w += v0[r].w;
    y1.x += v1[r].x;
    y1.y += v1[r].y;
    y1.z += v1[r].z;
    y1.w += v1[r].w;
  }
  float h[8] = {r0.x + y0.x, r0.y + y0.y, r0.z + y0.z, r0.w + y0.w, r1.x + y1.x, r1.y + y1.y, r1.z + y1.z, r1.w + y1.w};
  if (live) {
    float* yo = a.y + (size_t)b * a.ldy + n;
    *reinterpret_cast<float4*>(yo) = make_float4(h[0], h[1], h[2], h[3]);
    *reinterpret_cast<float4*>(yo + 4) = make_float4(h[4], h[5], h[6], h[7]);
  }
  // ---- next RMSNorm's input ----
  const int half = i8 & 1, slice = i8 >> 1, g = slice >> 2, q = slice & 3;
  const float4 w0 = *reinterpret_cast<const float4*>(a.nw + n), w1 = *reinterpret_cast<const float4*>(a.nw + n + 4);
  const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  // first half's running sums, handed to the second half
  float ss = 0.0f, xs = 0.0f, xsp = 0.0f;
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = h[k] * w[k];
  if (half == 0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += h[k] * h[k];
  }
  uint4 oh, ol;
  if (half == 0) a8act::prep8(v, oh, ol, xs, xsp);
  const float ss0 = __shfl_xor(ss, 1, 64), xs0 = __shfl_xor(xs, 1, 64), xsp0 = __shfl_xor(xsp, 1, 64);
  if (half == 1) {
    ss = ss0;
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += h[k] * h[k];
    xs = xs0;
    xsp = xsp0;
    a8act::prep8(v, oh, ol, xs, xsp);
  }
  // half group: slices q and q ^ 1 (their second-half lanes are 2 apart)
  const float ssh = ss + __shfl_xor(ss, 2, 64);
  const float xsh = xs + __shfl_xor(xs, 2, 64), xsph = xsp + __shfl_xor(xsp, 2, 64);
  if (!live) return;
  const int row = a.row0 + b;
  a8act::put_operand(a.nact, row, g, q, half, oh);
  a8act::put_operand(a.nact, row, g, q, 2 + half, ol);
  if (half == 1 && (q & 1) == 0) {
    a.nrss[(size_t)row * (a.n_out >> 5) + 2 * g + (q >> 1)] = ssh;
    a8act::put_half(a.nact, row, g, q >> 1, xsh, xsph);
  }
}

template <int MODE, int KS, int KP, int P, int MT, int EPI>
void launch_kernel(const GemvArgs& a, const uint4* XA, const float* CA, int nb, hipStream_t s) {
  const int tiles = (a.n_out + 31) / 32;
  hipLaunchKernelGGL((a8_mma_kernel<MODE, KS, KP, P, MT, EPI>), dim3((tiles + MT - 1) / MT), dim3(64 * KP), 0, s, a,
                     XA, CA, nb);
}

// split of the groups: enough ranges that every matrix puts ~2000+ waves' worth
// of work on the GPU. Depends on the shape only.
inline int split_ranges(const GemvArgs& a) {
  const int tiles = (a.n_out + 31) / 32, G = a.n_in / 64;
  // 16 ranges only where each still streams >= 16 groups (measured on MI355X)
  return tiles >= 512 ? 4 : (tiles >= 256 || G < 256) ? 8 : 16;
}

template <int KS, int T, int P, int EPI, int NC = 1>
void launch_shared(const GemvArgs& a, const uint4* XA, const float* CA, int nb, hipStream_t s) {
  static_assert(EPI != EPI_SWIGLU, "SwiGLU keeps the per-wave kernel");
  const int tiles = (a.n_out + 31) / 32;
  float* part = static_cast<float*>(gemv_scratch(s, (size_t)KS * nb * a.n_out * sizeof(float), 1));
  hipLaunchKernelGGL((a8_mma_shared_kernel<KS, T, P, EPI, NC>), dim3((tiles + T - 1) / T, KS), dim3(64 * T), 0, s, a,
                     XA, CA, nb, part);
  if (EPI == EPI_RES && a.nact.XA) {
    const int n8 = a.n_out / 8;
    hipLaunchKernelGGL((a8_reduce_emit_kernel<KS>), dim3((n8 + kRedT - 1) / kRedT, nb), dim3(kRedT), 0, s, a, nb,
                       part);
    return;
  }
  const int n4 = a.n_out / 4;
  hipLaunchKernelGGL((a8_reduce_kernel<KS, EPI>), dim3((n4 + kRedT - 1) / kRedT, nb), dim3(kRedT), 0, s, a, nb, part);
}

// one launch per chunk of up to 32 rows; the mode stages only the rows present
// and picks waves per workgroup / ring depth within the LDS budget
template <int KS, int EPI>
void launch_chunk_ks(const GemvArgs& a, const uint4* XA, const float* CA, int nb, hipStream_t s) {
  constexpr int KP4 = KS < 4 ? KS : 4, KP8 = KS < 8 ? KS : 8;
  if (nb == 1) {
    // fused gate/up: one wave per tile streams the tile's whole K (its KS
    // ranges one after another, summed as the multi-wave reduction sums them)
    // through a 4-stage ring; 17408 x 5120 measured 40.0 -> 36.3 us against 4
    // waves on a quarter of K each. Plain matrices have too few tiles for one
    // wave per tile (2-3x slower).
    if constexpr (EPI == EPI_SWIGLU) return launch_kernel<3, KS, 1, 4, 1, EPI>(a, XA, CA, nb, s);
    return launch_kernel<3, KS, KP8, 3, 1, EPI>(a, XA, CA, nb, s);
  }
  if (nb <= 4) return launch_kernel<0, KS, KP8, 3, 1, EPI>(a, XA, CA, nb, s);
  // 5..16 rows: the per-wave kernel, except for matrices large enough that one
  // operand stage shared by a workgroup's tiles streams faster (same sums)
  if (nb <= 16 && (EPI == EPI_SWIGLU || a.n_out % 4 != 0 || ((a.n_out + 31) / 32 < 256 && a.n_in / 64 < 256)))
    return launch_kernel<1, KS, KP4, 4, 1, EPI>(a, XA, CA, nb, s);
  if constexpr (EPI == EPI_SWIGLU) {
    // gate + up already give each wave 2 KiB of weights per KiB of operands
    launch_kernel<2, KS, KP4, 3, 1, EPI>(a, XA, CA, nb, s);
  } else if (a.n_out % 4 != 0) {
    launch_kernel<2, KS, KP4, 3, 1, EPI>(a, XA, CA, nb, s);
  } else {
    // one operand stage per workgroup of 4 (narrow) or 8 tiles
    if constexpr (KS == 16) launch_shared<KS, 4, 3, EPI>(a, XA, CA, nb, s);
    else launch_shared<KS, 8, 3, EPI>(a, XA, CA, nb, s);
  }
}

template <int EPI>
void launch_chunk(const GemvArgs& a, const uint4* XA, const float* CA, int nb, hipStream_t s) {
  switch (split_ranges(a)) {
    case 4: return launch_chunk_ks<4, EPI>(a, XA, CA, nb, s);
    case 8: return launch_chunk_ks<8, EPI>(a, XA, CA, nb, s);
    default: return launch_chunk_ks<16, EPI>(a, XA, CA, nb, s);
  }
}

// two 32-row chunks in one launch of the shared-operand kernel
template <int EPI>
void launch_pair(const GemvArgs& a, const uint4* XA, const float* CA, int nb, hipStream_t s) {
  if constexpr (EPI != EPI_SWIGLU) {
    switch (split_ranges(a)) {
      case 4: return launch_shared<4, 8, 3, EPI, 2>(a, XA, CA, nb, s);
      case 8: return launch_shared<8, 8, 3, EPI, 2>(a, XA, CA, nb, s);
      default: return launch_shared<16, 4, 3, EPI, 2>(a, XA, CA, nb, s);
    }
  }
}

// batches of at least two 128-row blocks take the GEMM (weights read once per
// 128 rows) when it has work for most of the chip; below that, the GEMV
// kernels' K splits keep more compute units streaming (measured on MI355X:
// the qkv projection at 128 rows 183 us as 56 GEMM workgroups against 91 us
// as two 64-row GEMV launches; 160-row steps of config 5 ran 13% slower
// through one full and one mostly empty GEMM block)
constexpr int kGemmRows = 128;
constexpr int kGemmMinWorkgroups = 128;

// Rows [0, rows) of a launch through the GEMM, then the prepared-output emits
// the GEMV epilogues would have fused (the next RMSNorm's deferred input, the
// SwiGLU product as the down projection's operands), by the prep kernels.
template <int EPI>
void launch_gemm_rows(const GemvArgs& a, const uint4* XA, const float* CA, int rows, hipStream_t s) {
  GemvArgs g = a;
  g.nact = a8act::Dst{};
  g.oact = a8act::Dst{};
  if (EPI == EPI_SWIGLU && !a.y) {
    g.y = static_cast<float*>(gemv_scratch(s, (size_t)rows * a.n_out * sizeof(float), 6));
    g.ldy = a.n_out;
  }
  run_a8_gemm(g, XA, CA, rows, EPI, s);
  const a8act::Dst& out = EPI == EPI_SWIGLU ? a.oact : a.nact;
  if (!out.XA) return;
  const size_t items = ((size_t)rows + 31) / 32 * out.G * 2;
  // the Dst describes the whole activation; its first rows start at a.row0 == 0
  if (EPI == EPI_SWIGLU)
    hipLaunchKernelGGL(a8_xprep_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, g.y, g.ldy, out, rows);
  else
    hipLaunchKernelGGL(a8_gnorm_prep_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, a.y, a.ldy, a.nw, out,
                       a.nrss, rows);
  PGD_HIP(hipGetLastError());
}

template <int EPI>
void launch_prepped(GemvArgs a, const A8Act& act, hipStream_t s) {
  PGD_CHECK(act.K == a.n_in, kErrShape, "prepared activations have the wrong width");
  const int G = a.n_in / 64;
  const uint4* XA = reinterpret_cast<const uint4*>(act.XA);
  int rows = act.rows;
  if (act.rss) {
    a.rss = act.rss;
    a.rss_nh = act.K / 32;
    a.rss_n = act.K;
    a.rss_eps = act.eps;
  }
  const bool sk = a8_sk_wanted(a, EPI);
  PGD_CHECK(!(a.nact.XA && sk), kErrShape, "norm-emitting residual GEMV on a stream-K matrix");
  // plain matrices stream their weights once per 64 rows when the second
  // chunk of a pair holds more than 4 rows (full operand layout)
  const bool pairs = EPI != EPI_SWIGLU && !sk && a.n_out % 4 == 0;
  int c0 = 0;
  // whole 128-row blocks through the GEMM (a partly filled block costs a
  // full one), the rest through the GEMV kernels
  const int gr = rows / kGemmRows * kGemmRows;
  if (gr >= 2 * kGemmRows && !a.cout && a.row0 == 0 &&
      a8_gemm_workgroups(a.n_out, gr, EPI) >= kGemmMinWorkgroups) {
    launch_gemm_rows<EPI>(a, XA, act.CA, gr, s);
    c0 = gr / 32;
    rows -= gr;
    if (a.y) a.y += (size_t)gr * a.ldy;
    if (a.res) a.res += (size_t)gr * a.ldres;
    if (a.rss) a.rss += (size_t)gr * a.rss_nh;
    a.row0 += gr;
  }
  for (int c = c0; rows > 0;) {
    const uint4* xa = XA + (size_t)c * G * 2 * 256;
    const float* ca = act.CA + (size_t)c * G * 2 * 64;
    int nb;
    if (pairs && rows > 36) {
      nb = rows < 64 ? rows : 64;
      launch_pair<EPI>(a, xa, ca, nb, s);
      c += 2;
    } else if (sk && rows > 36) {
      // two chunks through one stream-K launch (weights streamed once)
      nb = rows < 64 ? rows : 64;
      run_a8_sk_chunk(a, xa, ca, nb, EPI, s);
      c += 2;
    } else {
      nb = rows < 32 ? rows : 32;
      if (sk && nb >= 5) run_a8_sk_chunk(a, xa, ca, nb, EPI, s);
      else launch_chunk<EPI>(a, xa, ca, nb, s);
      c += 1;
    }
    PGD_HIP(hipGetLastError());
    rows -= nb;
    if (a.y) a.y += (size_t)nb * a.ldy;
    if (a.res) a.res += (size_t)nb * a.ldres;
    if (a.rss) a.rss += (size_t)nb * a.rss_nh;
    a.row0 += nb;
  }
}

}  // namespace

void run_a8_mma(const GemvArgs& a, const A8Act& act, int epi, hipStream_t s) {
  if (epi == EPI_SWIGLU) launch_prepped<EPI_SWIGLU>(a, act, s);
  else if (epi == EPI_RES) launch_prepped<EPI_RES>(a, act, s);
  else launch_prepped<EPI_STORE>(a, act, s);
}

size_t a8_scratch_need(const GemvArgs& a, int rows, int epi) {
  PGD_CHECK(epi != EPI_SWIGLU && !a.nact.XA, kErrArg, "scratch bound covers plain and residual GEMVs");
  size_t slot[8] = {};
  auto need = [&](int i, size_t b) { slot[i] = std::max(slot[i], b); };
  const bool sk = a8_sk_wanted(a, epi);
  const bool pairs = !sk && a.n_out % 4 == 0;
  const int tiles = (a.n_out + 31) / 32, G = a.n_in / 64, KS = split_ranges(a);
  // the chunk loop and kernel choice of launch_prepped / launch_chunk_ks
  for (; rows > 0;) {
    int nb;
    if (pairs && rows > 36) {
      nb = rows < 64 ? rows : 64;
      need(1, (size_t)KS * nb * a.n_out * sizeof(float));
    } else if (sk && rows > 36) {
      nb = rows < 64 ? rows : 64;
      size_t s3 = 0, s5 = 0;
      sk_scratch_need(a, nb, epi, &s3, &s5);
      need(3, s3);
      need(5, s5);
    } else {
      nb = rows < 32 ? rows : 32;
      if (sk && nb >= 5) {
        size_t s3 = 0, s5 = 0;
        sk_scratch_need(a, nb, epi, &s3, &s5);
        need(3, s3);
        need(5, s5);
      } else if (nb > 4 && a.n_out % 4 == 0 && !(nb <= 16 && tiles < 256 && G < 256)) {
        need(1, (size_t)KS * nb * a.n_out * sizeof(float));
      }
    }
    rows -= nb;
  }
  size_t total = 0;
  for (size_t b : slot)
    if (b) total = ((total + 255) & ~(size_t)255) + b;
  return total;
}

}  // namespace gemv

// operands | constants | deferred-norm row sums ([rows][K / 32], 256 B aligned)
static size_t rss_offset(int rows, int K) {
  return (a8act::xa_bytes(rows, K / 64) + a8act::ca_bytes(rows, K / 64) + 255) & ~(size_t)255;
}

float* a8_act_rss(void* buf, int rows, int K) {
  return reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(buf) + rss_offset(rows, K));
}

size_t a8_act_bytes(int rows, int K) { return rss_offset(rows, K) + (size_t)rows * (K / 32) * sizeof(float); }

A8Act a8_act_view(void* buf, int rows, int K) {
  A8Act a;
  a.XA = buf;
  a.CA = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(buf) + a8act::xa_bytes(rows, K / 64));
  a.rows = rows;
  a.K = K;
  return a;
}

a8act::Dst a8_act_dst(const A8Act& a) {
  return a8act::Dst{reinterpret_cast<uint4*>(const_cast<void*>(a.XA)), const_cast<float*>(a.CA), a.rows, a.K / 64};
}

A8Act a8_act_prep(const float* x, int ldx, int rows, int K, void* buf, hipStream_t s) {
  PGD_CHECK(K % 64 == 0 && ldx % 4 == 0, kErrShape, "A8 activation width must be a multiple of 64");
  A8Act a = a8_act_view(buf, rows, K);
  if (rows <= 0) return a;
  const size_t items = ((size_t)rows + 31) / 32 * (K / 64) * 2;
  hipLaunchKernelGGL(gemv::a8_xprep_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, x, ldx, a8_act_dst(a),
                     rows);
  PGD_HIP(hipGetLastError());
  return a;
}

A8Act a8_gnorm_prep(const float* x, int ldx, int rows, int n, const float* w, float eps, void* buf, hipStream_t s) {
  PGD_CHECK(n % 64 == 0 && ldx % 4 == 0, kErrShape, "A8 activation width must be a multiple of 64");
  A8Act a = a8_act_view(buf, rows, n);
  float* rss = a8_act_rss(buf, rows, n);
  a.rss = rss;
  a.eps = eps;
  if (rows <= 0) return a;
  const size_t items = ((size_t)rows + 31) / 32 * (n / 64) * 2;
  hipLaunchKernelGGL(gemv::a8_gnorm_prep_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, x, ldx, w,
                     a8_act_dst(a), rss, rows);
  PGD_HIP(hipGetLastError());
  return a;
}

A8Act a8_norm_prep(const float* x, int ldx, const int* rows_idx, int rows, int n, const float* w, float eps, float* y,
                   int ldy, void* buf, hipStream_t s) {
  PGD_CHECK(n % 64 == 0 && n <= 256 * 16 * gemv::kNormMaxSlices && ldx % 4 == 0, kErrShape, "norm prep width");
  A8Act a = a8_act_view(buf, rows, n);
  if (rows <= 0) return a;
  // one 16-wide slice per thread up to 8192 wide
  if (n <= 512 * 16)
    hipLaunchKernelGGL((gemv::a8_norm_prep_kernel<1, 512>), dim3(rows), dim3(512), 0, s, x, ldx, rows_idx, rows, n, w,
                       eps, y, ldy, a8_act_dst(a));
  else
    hipLaunchKernelGGL((gemv::a8_norm_prep_kernel<gemv::kNormMaxSlices, 256>), dim3(rows), dim3(256), 0, s, x, ldx,
                       rows_idx, rows, n, w, eps, y, ldy, a8_act_dst(a));
  PGD_HIP(hipGetLastError());
  return a;
}

namespace gemv {

}  // namespace gemv
}  // namespace pgd
