// gemm_a8.hip — MLX affine-8 (group 64) GEMM for prefill: batches of >= 128
// activation rows, every weight byte read once per 128 rows.
//
// Same per-group arithmetic as the GEMV kernels (gemv_mma.hip): with the
// prepared activations (xh + xl f16 operands, a8_act.h) and codes as the f16
// 1024 + c,
//   P[b, n] = -1024 XSP[b, g] + sum_k (1024 + c[n, k]) (xh + xl)[b, k]   4 x v_mfma_f32_16x16x32_f16
//   Y[b, n] += s[n, g] P[b, n] + bias[n, g] XS[b, g]
// but the groups of a row are summed in order 0..G-1 by one wave (no split-K,
// no partial sums in memory).
//
// Tiling: a workgroup of 8 waves computes 256 weight rows (8 tiles of 32; the
// SwiGLU pair: 4 gate + 4 up tiles) x 128 batch rows (4 activation chunks).
// Wave w = 2 wm + wb owns weight tiles 2 wm, 2 wm + 1 (SwiGLU: gate tile wm
// and up tile wm) and batch chunks 2 wb, 2 wb + 1: 4 weight subtiles x 4
// batch tiles of 16 x 16 accumulators. Per group the workgroup stages in LDS
// the 8 tiles' codes (16 KiB) and scale/bias (1 KiB) and the 4 chunks'
// operands (32 KiB) and constants (2 KiB) by direct global->LDS loads, three
// stages deep: groups g + 1 and g + 2 load while group g computes. Each staged byte
// feeds 2 (weights) or 4 (operands) waves.
//
// Workgroups are numbered so that the batch blocks of one weight block run on
// the same XCD (its L2 serves the weight re-reads).
#include "a8_act.h"
#include "common.h"
#include "gemv_impl.h"
#include "quant.h"

namespace pgd {
namespace gemv {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

constexpr int kGW = 8;            // waves per workgroup
constexpr int kWT = 8;            // weight tiles per workgroup
constexpr int kBC = 4;            // batch chunks (32 rows) per workgroup
constexpr int kStW = kWT * 2048;  // codes per stage
constexpr int kStS = kWT * 128;   // scale/bias per stage
constexpr int kStX = kBC * 8192;  // operands per stage
constexpr int kStC = kBC * 512;   // constants per stage
constexpr int kStage = kStW + kStS + kStX + kStC;
constexpr int kLoads = kStage / 1024;  // 1 KiB wave loads per stage
constexpr int kStages = 3;
static_assert(kStage % 1024 == 0, "stage is whole wave loads");

__device__ __forceinline__ void dma16(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds((glb_void*)g, (lds_void*)l, 16, 0, 0);
}

__device__ inline h8 codes8(uint32_t w0, uint32_t w1) {
  const uint32_t c0 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u);
  const uint32_t c1 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u);
  const uint32_t c2 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u);
  const uint32_t c3 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u);
  return __builtin_bit_cast(h8, make_uint4(c0, c1, c2, c3));
}

// global source of wave load j (0 .. kLoads-1) of group g for this lane: the
// stage is [codes: tile t, 2 KiB] [sb: tile t, 128 B] [operands: chunk c, bt,
// 4 KiB] [constants: chunk c, bt, 256 B]
template <bool DUAL>
__device__ inline const void* load_src(const GemvArgs& a, const uint4* XA, const float* CA, int wblk, int cblk, int G,
                                       int ntiles, int nchunks, int g, int j, int lane) {
  if (j < kWT * 2) {  // codes: tile j / 2, half j % 2
    const int t = j >> 1;
    int tile;
    const uint8_t* p;
    if constexpr (DUAL) {
      tile = wblk * (kWT / 2) + (t & 3);
      p = t < 4 ? a.p0 : a.u0;
    } else {
      tile = wblk * kWT + t;
      p = a.p0;
    }
    tile = min(tile, ntiles - 1);
    return p + (((size_t)tile * G + g) << 11) + (j & 1) * 1024 + lane * 16;
  }
  j -= kWT * 2;
  if (j < 1) {  // scale/bias: lane l -> tile l / 8, 16 B (l % 8)
    const int t = lane >> 3;
    int tile;
    const uint8_t* p;
    if constexpr (DUAL) {
      tile = wblk * (kWT / 2) + (t & 3);
      p = t < 4 ? a.p1 : a.u1;
    } else {
      tile = wblk * kWT + t;
      p = a.p1;
    }
    tile = min(tile, ntiles - 1);
    return p + (((size_t)tile * G + g) << 7) + (lane & 7) * 16;
  }
  j -= 1;
  if (j < kBC * 8) {  // operands: chunk j / 8, tile (j / 4) % 2, operand j % 4
    const int c = min(cblk * kBC + (j >> 3), nchunks - 1), bt = (j >> 2) & 1, i = j & 3;
    const size_t item = ((size_t)c * G + g) * 2 + bt;
    return XA + item * 256 + i * 64 + lane;
  }
  j -= kBC * 8;
  {  // constants: lane l -> item (chunk, bt) = l / 16 of this load's pair of chunks
    const int it = j * 4 + (lane >> 4);  // 0 .. 2 kBC - 1
    const int c = min(cblk * kBC + (it >> 1), nchunks - 1), bt = it & 1;
    const size_t item = ((size_t)c * G + g) * 2 + bt;
    return CA + item * 64 + (lane & 15) * 4;
  }
}

template <int EPI>
__global__ __launch_bounds__(64 * kGW) void a8_gemm_kernel(GemvArgs a, const uint4* __restrict__ XA,
                                                           const float* __restrict__ CA, int rows, int nwblk,
                                                           int ncblk, int per_xcd) {
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  // XCD-aware numbering: workgroups are dealt to the 8 XCDs in turn; XCD x
  // takes the contiguous range [x per_xcd, (x + 1) per_xcd) of (weight block,
  // batch block) pairs, batch block fastest
  const int id = blockIdx.x, xcd = id & 7;
  const int gi = xcd * per_xcd + (id >> 3);
  if (gi >= nwblk * ncblk || (id >> 3) >= per_xcd) return;
  const int wblk = gi / ncblk, cblk = gi % ncblk;
  const int G = a.n_in / 64;
  const int ntiles = (a.n_out + 31) / 32, nchunks = (rows + 31) / 32;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wb = wave & 1;
  const int j16 = lane & 15, q = lane >> 4;

  // this wave's loads: j = wave + 8 k; sources of group 0 and the per-group
  // stride of each (codes 2 KiB, scale/bias 128 B, operands 8 KiB, constants 512 B)
  constexpr int NK = (kLoads + kGW - 1) / kGW;
  const char* src[NK];
  uint32_t step[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int j = min(wave + k * kGW, kLoads - 1);
    src[k] = static_cast<const char*>(load_src<DUAL>(a, XA, CA, wblk, cblk, G, ntiles, nchunks, 0, j, lane));
    step[k] = j < kWT * 2 ? 2048u : j < kWT * 2 + 1 ? 128u : j < kWT * 2 + 1 + kBC * 8 ? 8192u : 512u;
  }
  // every wave issues exactly NK loads per group (a wave with fewer repeats
  // the stage's last load: same bytes to the same place), so one vmcnt wait
  // of NK leaves exactly the newest group in flight
  auto issue = [&](int g, int stage) {
    char* base = smem + stage * kStage;
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      const int j = min(wave + k * kGW, kLoads - 1);
      dma16(src[k] + (size_t)g * step[k], base + j * 1024);
    }
  };

  f4 Y[4][4];  // [subtile][batch tile]
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) Y[st][bt] = (f4){0.f, 0.f, 0.f, 0.f};

  // this wave's subtiles: stage tiles (2 wm, 2 wm + 1), or (wm, 4 + wm) for the SwiGLU pair
  const int t0 = DUAL ? wm : 2 * wm, t1 = DUAL ? 4 + wm : 2 * wm + 1;
  const uint32_t woff = (q >> 1) * 1024 + j16 * 32 + (q & 1) * 16;

  // three stages: group g computes while g + 1 and g + 2 load
  // LDS reads in inline asm: the compiler sees no LDS access after the
  // global->LDS loads, so it adds no vmcnt wait of its own before them (it
  // would wait for the groups still loading); each block waits for its own
  // reads, and the loop waits for the loads with explicit vmcnt counts. The
  // barrier is the bare s_barrier: the loaded bytes are in LDS once each wave
  // has waited for its own loads.
  const uint32_t lbase = (uint32_t)(size_t)((const __attribute__((address_space(3))) char*)smem);
  const uint32_t w_lane = lbase + woff, s_lane = lbase + kStW + j16 * 4, x_lane = lbase + kStW + kStS + lane * 16,
                 c_lane = lbase + kStW + kStS + kStX + q * 16;
  // Loads past the last group re-read it into a stage whose group is already
  // consumed, so every iteration issues and waits alike: no branch in the
  // loop body, and the scheduler can interleave a group's MFMAs with its
  // folding FMAs.
  issue(0, 0);
  issue(min(1, G - 1), 1);
  __builtin_amdgcn_s_waitcnt(NK & 15 | (7 << 4) | (15 << 8) | ((NK >> 4) << 14));  // vmcnt(NK)
  __builtin_amdgcn_s_barrier();
  for (int g = 0; g < G; ++g) {
    const int cur = g % kStages;
    issue(min(g + 2, G - 1), (g + 2) % kStages);
    const uint32_t so = cur * kStage;
    // codes of the 4 subtiles (stage tile t, row half h = st & 1) and their scale/bias
    uint4 W[4];
    uint32_t SV[4];
    {
      const uint32_t a0 = w_lane + so + t0 * 2048, a1 = w_lane + so + t1 * 2048;
      const uint32_t b0 = s_lane + so + t0 * 128, b1 = s_lane + so + t1 * 128;
      asm volatile(
          "ds_read_b128 %0, %[a0]\n\tds_read_b128 %1, %[a0] offset:512\n\t"
          "ds_read_b128 %2, %[a1]\n\tds_read_b128 %3, %[a1] offset:512\n\t"
          "ds_read_b32 %4, %[b0]\n\tds_read_b32 %5, %[b0] offset:64\n\t"
          "ds_read_b32 %6, %[b1]\n\tds_read_b32 %7, %[b1] offset:64\n\ts_waitcnt lgkmcnt(0)"
          : "=&v"(W[0]), "=&v"(W[1]), "=&v"(W[2]), "=&v"(W[3]), "=&v"(SV[0]), "=&v"(SV[1]), "=&v"(SV[2]), "=&v"(SV[3])
          : [a0] "v"(a0), [a1] "v"(a1), [b0] "v"(b0), [b1] "v"(b1)
          : "memory");
    }
    h8 B0[4], B1[4];
    float S[4], Bi[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      B0[st] = codes8(W[st].x, W[st].y);
      B1[st] = codes8(W[st].z, W[st].w);
      S[st] = bf16_to_f32(SV[st] & 0xffffu);
      Bi[st] = bf16_to_f32(SV[st] >> 16);
    }
    // batch tiles in pairs: one block of LDS reads (two tiles' operands and
    // constants) per pair
#pragma unroll
    for (int bp = 0; bp < 2; ++bp) {
      uint4 XR[2][4];
      f4 C[2][4];
      {
        // tiles 2 bp, 2 bp + 1 are the two 16-row halves of chunk bp of this wave
        const int item = (2 * wb + bp) * 2;
        const uint32_t xa = x_lane + so + item * 4096, ca = c_lane + so + item * 256;
        asm volatile(
            "ds_read_b128 %0, %[xa]\n\tds_read_b128 %1, %[xa] offset:1024\n\t"
            "ds_read_b128 %2, %[xa] offset:2048\n\tds_read_b128 %3, %[xa] offset:3072\n\t"
            "ds_read_b128 %4, %[xa] offset:4096\n\tds_read_b128 %5, %[xa] offset:5120\n\t"
            "ds_read_b128 %6, %[xa] offset:6144\n\tds_read_b128 %7, %[xa] offset:7168\n\t"
            "ds_read_b128 %8, %[ca]\n\tds_read_b128 %9, %[ca] offset:64\n\t"
            "ds_read_b128 %10, %[ca] offset:128\n\tds_read_b128 %11, %[ca] offset:192\n\t"
            "ds_read_b128 %12, %[ca] offset:256\n\tds_read_b128 %13, %[ca] offset:320\n\t"
            "ds_read_b128 %14, %[ca] offset:384\n\tds_read_b128 %15, %[ca] offset:448\n\ts_waitcnt lgkmcnt(0)"
            : "=&v"(XR[0][0]), "=&v"(XR[0][1]), "=&v"(XR[0][2]), "=&v"(XR[0][3]), "=&v"(XR[1][0]), "=&v"(XR[1][1]),
              "=&v"(XR[1][2]), "=&v"(XR[1][3]), "=&v"(C[0][0]), "=&v"(C[0][1]), "=&v"(C[0][2]), "=&v"(C[0][3]),
              "=&v"(C[1][0]), "=&v"(C[1][1]), "=&v"(C[1][2]), "=&v"(C[1][3])
            : [xa] "v"(xa), [ca] "v"(ca)
            : "memory");
      }
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        const int bt = 2 * bp + hb;
        // constants: -1024 XSP of quarters (0, 1) + (2, 3), XS likewise
        const f4 cp = C[hb][0] + C[hb][1], xs = C[hb][2] + C[hb][3];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          f4 P = cp;
          P = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, XR[hb][0]), B0[st], P, 0, 0, 0);
          P = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, XR[hb][1]), B1[st], P, 0, 0, 0);
          P = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, XR[hb][2]), B0[st], P, 0, 0, 0);
          P = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, XR[hb][3]), B1[st], P, 0, 0, 0);
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) Y[st][bt][rr] = fmaf(Bi[st], xs[rr], fmaf(S[st], P[rr], Y[st][bt][rr]));
        }
      }
    }
    // group g + 1 landed (g + 2 may still be in flight) and every wave is
    // done with stage cur, which group g + 3 overwrites
    __builtin_amdgcn_s_waitcnt(NK & 15 | (7 << 4) | (15 << 8) | ((NK >> 4) << 14));
    __builtin_amdgcn_s_barrier();
  }
  __builtin_amdgcn_s_waitcnt(0);  // the re-read loads of the last iterations

  // deferred RMSNorm of the input: 1/rms of each batch row (rss_inv needs the
  // whole wave), applied to the accumulators before the epilogue
  if (a.rss) {
#pragma unroll
    for (int bt = 0; bt < 4; ++bt) {
      const int c = cblk * kBC + 2 * wb + (bt >> 1);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        float f = 1.0f;
        for (int qq = 0; qq < 4; ++qq) {
          const int b = c * 32 + 16 * (bt & 1) + 4 * qq + rr;
          const float v = b < rows ? rss_inv(a.rss + (size_t)b * a.rss_nh, a.rss_nh, a.rss_n, a.rss_eps) : 1.0f;
          if (qq == q) f = v;
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) Y[st][bt][rr] *= f;
      }
    }
  }
  // epilogue: lane (j16, q) holds weight row 16 h + j16 of its subtiles and
  // batch rows 16 bh + 4 q + rr of each batch tile
#pragma unroll
  for (int bt = 0; bt < 4; ++bt) {
    const int c = cblk * kBC + 2 * wb + (bt >> 1);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int b = c * 32 + 16 * (bt & 1) + 4 * q + rr;
      if (b >= rows) continue;
      if constexpr (DUAL) {
        const int tile = wblk * (kWT / 2) + wm;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int n = tile * 32 + 16 * h + j16;
          if (n < a.n_out) a.y[(size_t)b * a.ldy + n] = silu_f(Y[h][bt][rr]) * Y[2 + h][bt][rr];
        }
      } else {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const int tile = wblk * kWT + (st < 2 ? t0 : t1);
          const int n = tile * 32 + 16 * (st & 1) + j16;
          if (n >= a.n_out) continue;
          const size_t o = (size_t)b * a.ldy + n;
          if constexpr (EPI == EPI_RES) a.y[o] = a.res[(size_t)b * a.ldres + n] + Y[st][bt][rr];
          else a.y[o] = Y[st][bt][rr];
        }
      }
    }
  }
}

}  // namespace

int a8_gemm_workgroups(int n_out, int rows, int epi) {
  const int ntiles = (n_out + 31) / 32;
  const int nwblk = epi == EPI_SWIGLU ? (ntiles + kWT / 2 - 1) / (kWT / 2) : (ntiles + kWT - 1) / kWT;
  return nwblk * ((rows / 32 + kBC - 1) / kBC);
}

void run_a8_gemm(const GemvArgs& a, const uint4* XA, const float* CA, int rows, int epi, hipStream_t s) {
  PGD_CHECK(rows > 0 && (rows % 32 == 0 || rows % 32 > 4), kErrShape,
            "the A8 GEMM takes activation chunks in the full (not compact) layout");
  PGD_CHECK(a.n_in % 64 == 0, kErrShape, "A8 GEMM width");
  const int ntiles = (a.n_out + 31) / 32;
  const int nwblk = epi == EPI_SWIGLU ? (ntiles + kWT / 2 - 1) / (kWT / 2) : (ntiles + kWT - 1) / kWT;
  const int ncblk = (rows / 32 + kBC - 1) / kBC;
  const int total = nwblk * ncblk, per_xcd = (total + 7) / 8;
  const size_t lds = kStages * (size_t)kStage;
  static bool attr_set = false;
  if (!attr_set) {
    PGD_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(a8_gemm_kernel<EPI_STORE>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    PGD_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(a8_gemm_kernel<EPI_RES>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    PGD_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(a8_gemm_kernel<EPI_SWIGLU>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr_set = true;
  }
  const dim3 grid(8 * per_xcd), block(64 * kGW);
  if (epi == EPI_SWIGLU)
    hipLaunchKernelGGL(a8_gemm_kernel<EPI_SWIGLU>, grid, block, lds, s, a, XA, CA, rows, nwblk, ncblk, per_xcd);
  else if (epi == EPI_RES)
    hipLaunchKernelGGL(a8_gemm_kernel<EPI_RES>, grid, block, lds, s, a, XA, CA, rows, nwblk, ncblk, per_xcd);
  else
    hipLaunchKernelGGL(a8_gemm_kernel<EPI_STORE>, grid, block, lds, s, a, XA, CA, rows, nwblk, ncblk, per_xcd);
  PGD_HIP(hipGetLastError());
}

}  // namespace gemv
}  // namespace pgd
