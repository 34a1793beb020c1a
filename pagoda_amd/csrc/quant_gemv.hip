// quant_gemv.hip — dequant-in-register GEMV / skinny GEMM for MLX affine-8
// (group 64) and GGML Q4_K / Q6_K matrices, plus dequant, embedding and the
// seeded synthetic-weight generator.
//
// GEMV mapping (wave64): a wave owns ROWS consecutive output rows. A row is
// cut into 16-byte chunks of its main plane (A8 codes / Q4K qs / Q6K ql);
// lane l takes chunks l, l+64, ... so every load instruction of the wave
// reads 1 KiB of one row contiguously (128-bit per lane). The activation
// values a chunk needs are loaded once per chunk and reused for the ROWS
// rows; the per-row partials are folded with a fixed wave butterfly, so the
// result is deterministic and the same for every batch size (each batch row
// runs the identical instruction sequence).
//
// Reference kernels whose results this reproduces: affine_gemv / gemm4 /
// gemv2_silu / gemv_res (pagoda-hf/src/qwen3_gemv.rs:54-306, 414-567);
// Q4K/Q6K have no reference GPU kernel (candle QMatMul on CPU,
// pagoda-hf/src/qwen2_gguf.rs:271-289).
#include <algorithm>
#include <vector>

#include "common.h"
#include "quant.h"

namespace pgd {

namespace {

struct GemvArgs {
  const uint8_t* p0;
  const uint8_t* p1;
  const uint8_t* p2;
  const uint8_t* p3;
  const uint8_t* u0;  // second matrix (SwiGLU up)
  const uint8_t* u1;
  const uint8_t* u2;
  const uint8_t* u3;
  int n_out, n_in, nsb;
  const void* x;
  int ldx;
  float* y;
  int ldy;
  const float* res;
  int ldres;
};

enum { EPI_STORE = 0, EPI_RES = 1, EPI_SWIGLU = 2 };

// ---- activation loads ------------------------------------------------------
template <bool XF16>
__device__ inline void load_x16(const void* x, size_t off, float* v) {
  if constexpr (XF16) {
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + off);
    uint4 a = p[0], b = p[1];
    uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[2 * i] = f16_to_f32(w[i] & 0xffffu);
      v[2 * i + 1] = f16_to_f32(w[i] >> 16);
    }
  } else {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 f = p[i];
      v[4 * i] = f.x;
      v[4 * i + 1] = f.y;
      v[4 * i + 2] = f.z;
      v[4 * i + 3] = f.w;
    }
  }
}

__device__ inline float sum16(const float* v) {
  float s = v[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) s += v[i];
  return s;
}

__device__ inline uint32_t byte_of(uint4 q, int i) {
  uint32_t w = i < 4 ? q.x : (i < 8 ? q.y : (i < 12 ? q.z : q.w));
  return (w >> (8 * (i & 3))) & 255u;
}

// ---- per-format chunk logic ------------------------------------------------
// A8: chunk p = codes [16p, 16p+16) of a row; group p/4.
struct A8 {
  struct W {
    uint4 q;
    uint32_t sb;
  };
  static __device__ inline int chunks(const GemvArgs& a) { return a.n_in >> 4; }
  static __device__ inline bool pos(const GemvArgs& a, int p, int& lo, int& hi) {
    lo = p << 4;
    hi = -1;
    return true;
  }
  static __device__ inline W load(const uint8_t* c0, const uint8_t* c1, const uint8_t*, const uint8_t*,
                                  const GemvArgs& a, int row, int p) {
    W w;
    w.q = *reinterpret_cast<const uint4*>(c0 + (size_t)row * a.n_in + ((size_t)p << 4));
    w.sb = reinterpret_cast<const uint32_t*>(c1)[(size_t)row * (a.n_in >> 6) + (p >> 2)];
    return w;
  }
  // pagoda-hf/src/qwen3_gemv.rs:96-99: r = fma(scale, sum(code*x), fma(sum(x), bias, r))
  static __device__ inline float acc(float r, const W& w, const float* xl, const float*, float sl, float) {
    float d = (float)byte_of(w.q, 0) * xl[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) d = fmaf((float)byte_of(w.q, i), xl[i], d);
    float s = bf16_to_f32(w.sb & 0xffffu), b = bf16_to_f32(w.sb >> 16);
    return fmaf(s, d, fmaf(sl, b, r));
  }
};

// Q4K: chunk p = qs bytes [16p, 16p+16): block p/8, part p%8 -> 64-group
// j = part/2, half h = part%2. Low nibbles are elements 64j+16h+i of
// sub-block 2j, high nibbles 64j+32+16h+i of sub-block 2j+1.
struct Q4K {
  struct W {
    uint4 q;
    uint4 hdr;
  };
  static __device__ inline int chunks(const GemvArgs& a) { return a.nsb << 3; }
  static __device__ inline bool pos(const GemvArgs& a, int p, int& lo, int& hi) {
    int sb = p >> 3, part = p & 7;
    lo = (sb << 8) + ((part >> 1) << 6) + ((part & 1) << 4);
    hi = lo + 32;
    if (hi >= a.n_in) hi = -1;
    return lo < a.n_in;
  }
  static __device__ inline W load(const uint8_t* c0, const uint8_t* c1, const uint8_t*, const uint8_t*,
                                  const GemvArgs& a, int row, int p) {
    W w;
    w.q = *reinterpret_cast<const uint4*>(c0 + (size_t)row * a.nsb * 128 + ((size_t)p << 4));
    w.hdr = reinterpret_cast<const uint4*>(c1)[(size_t)row * a.nsb + (p >> 3)];
    return w;
  }
  static __device__ inline void scale_min(const uint4& hdr, int is, float& sc, float& m) {
    // 12 scale bytes are hdr bytes 4..15 (hdr.y, hdr.z, hdr.w)
    uint4 s = make_uint4(hdr.y, hdr.z, hdr.w, 0u);
    uint32_t a, b;
    if (is < 4) {
      a = byte_of(s, is) & 63u;
      b = byte_of(s, is + 4) & 63u;
    } else {
      a = (byte_of(s, is + 4) & 0xFu) | ((byte_of(s, is - 4) >> 6) << 4);
      b = (byte_of(s, is + 4) >> 4) | ((byte_of(s, is) >> 6) << 4);
    }
    sc = (float)a;
    m = (float)b;
  }
  static __device__ inline float acc(float r, const W& w, const float* xl, const float* xh, float sl, float sh,
                                     int p, bool has_hi) {
    int j = (p & 7) >> 1;
    float d = f16_to_f32(w.hdr.x & 0xffffu), dmin = f16_to_f32(w.hdr.x >> 16);
    float sc0, m0, sc1, m1;
    scale_min(w.hdr, 2 * j, sc0, m0);
    scale_min(w.hdr, 2 * j + 1, sc1, m1);
    float dl = 0.0f, dh = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t b = byte_of(w.q, i);
      dl = fmaf((float)(b & 15u), xl[i], dl);
      dh = fmaf((float)(b >> 4), xh[i], dh);
    }
    r = fmaf(d * sc0, dl, r);
    r = fmaf(-(dmin * m0), sl, r);
    if (has_hi) {
      r = fmaf(d * sc1, dh, r);
      r = fmaf(-(dmin * m1), sh, r);
    }
    return r;
  }
};

// Q6K: chunk p = ql bytes [16p, 16p+16): block p/8, part p%8 -> half
// n = part/4, c = part%4. Low nibbles: elements 128n+16c+i, high nibbles
// 128n+64+16c+i; the two high bits come from qh byte 32n+16(c&1)+i at shift
// 2(c>>1) (low) and 4+2(c>>1) (high); scales sc[8n+c] and sc[8n+4+c].
struct Q6K {
  struct W {
    uint4 ql;
    uint4 qh;
    float s_lo, s_hi;
  };
  static __device__ inline int chunks(const GemvArgs& a) { return a.nsb << 3; }
  static __device__ inline bool pos(const GemvArgs& a, int p, int& lo, int& hi) {
    int sb = p >> 3, part = p & 7;
    lo = (sb << 8) + ((part >> 2) << 7) + ((part & 3) << 4);
    hi = lo + 64;
    if (hi >= a.n_in) hi = -1;
    return lo < a.n_in;
  }
  static __device__ inline W load(const uint8_t* c0, const uint8_t* c1, const uint8_t* c2, const uint8_t* c3,
                                  const GemvArgs& a, int row, int p) {
    int sb = p >> 3, part = p & 7, n = part >> 2, c = part & 3;
    W w;
    w.ql = *reinterpret_cast<const uint4*>(c0 + (size_t)row * a.nsb * 128 + ((size_t)p << 4));
    w.qh = *reinterpret_cast<const uint4*>(c1 + (size_t)row * a.nsb * 64 + sb * 64 + 32 * n + 16 * (c & 1));
    const int8_t* sc = reinterpret_cast<const int8_t*>(c2) + (size_t)row * a.nsb * 16 + sb * 16 + 8 * n + c;
    float d = f16_to_f32(reinterpret_cast<const uint16_t*>(c3)[(size_t)row * a.nsb + sb]);
    w.s_lo = d * (float)sc[0];
    w.s_hi = d * (float)sc[4];
    return w;
  }
  static __device__ inline float acc(float r, const W& w, const float* xl, const float* xh, float sl, float sh,
                                     int p, bool has_hi) {
    int c = p & 3;
    int shl = 2 * (c >> 1), shh = 4 + 2 * (c >> 1);
    float dl = 0.0f, dh = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t l = byte_of(w.ql, i), h = byte_of(w.qh, i);
      uint32_t ql = (l & 15u) | (((h >> shl) & 3u) << 4);
      uint32_t qh = (l >> 4) | (((h >> shh) & 3u) << 4);
      dl = fmaf((float)ql, xl[i], dl);
      dh = fmaf((float)qh, xh[i], dh);
    }
    // sum (q-32) x = sum q x - 32 sum x
    r = fmaf(w.s_lo, fmaf(-32.0f, sl, dl), r);
    if (has_hi) r = fmaf(w.s_hi, fmaf(-32.0f, sh, dh), r);
    return r;
  }
};

template <class F>
struct Acc {
  template <class W>
  static __device__ inline float run(float r, const W& w, const float* xl, const float* xh, float sl, float sh,
                                     int p, bool has_hi) {
    return F::acc(r, w, xl, xh, sl, sh, p, has_hi);
  }
};
template <>
struct Acc<A8> {
  template <class W>
  static __device__ inline float run(float r, const W& w, const float* xl, const float* xh, float sl, float sh,
                                     int, bool) {
    return A8::acc(r, w, xl, xh, sl, sh);
  }
};

template <class F, int ROWS, int NB, bool XF16, int EPI>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int row0 = wave * ROWS;
  if (row0 >= a.n_out) return;
  int rows[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) rows[r] = min(row0 + r, a.n_out - 1);
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  float acc[ROWS][NB];
  float acc2[DUAL ? ROWS : 1][DUAL ? NB : 1];
#pragma unroll
  for (int r = 0; r < ROWS; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      acc[r][b] = 0.0f;
      if constexpr (DUAL) acc2[r][b] = 0.0f;
    }
  const int nch = F::chunks(a);
  for (int p = lane; p < nch; p += 64) {
    int lo, hi;
    if (!F::pos(a, p, lo, hi)) continue;
    const bool has_hi = hi >= 0;
    typename F::W w[ROWS];
    typename F::W w2[DUAL ? ROWS : 1];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      w[r] = F::load(a.p0, a.p1, a.p2, a.p3, a, rows[r], p);
      if constexpr (DUAL) w2[r] = F::load(a.u0, a.u1, a.u2, a.u3, a, rows[r], p);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float xl[16], xh[16];
      load_x16<XF16>(a.x, (size_t)b * a.ldx + lo, xl);
      float sl = sum16(xl), sh = 0.0f;
      if (has_hi) {
        load_x16<XF16>(a.x, (size_t)b * a.ldx + hi, xh);
        sh = sum16(xh);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) xh[i] = 0.0f;
      }
#pragma unroll
      for (int r = 0; r < ROWS; ++r) {
        acc[r][b] = Acc<F>::run(acc[r][b], w[r], xl, xh, sl, sh, p, has_hi);
        if constexpr (DUAL) acc2[r][b] = Acc<F>::run(acc2[r][b], w2[r], xl, xh, sl, sh, p, has_hi);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < ROWS; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float v = wave_sum(acc[r][b]);
      float v2 = 0.0f;
      if constexpr (DUAL) v2 = wave_sum(acc2[r][b]);
      if (lane == 0 && row0 + r < a.n_out) {
        size_t o = (size_t)b * a.ldy + row0 + r;
        if constexpr (EPI == EPI_STORE) a.y[o] = v;
        if constexpr (EPI == EPI_RES) a.y[o] = a.res[(size_t)b * a.ldres + row0 + r] + v;
        if constexpr (EPI == EPI_SWIGLU) a.y[o] = silu_f(v) * v2;
      }
    }
}

constexpr int kRows = 4;

template <class F, int NB, bool XF16, int EPI>
void launch_nb(const GemvArgs& a, hipStream_t s) {
  int waves = (a.n_out + kRows - 1) / kRows;
  int blocks = (waves + 3) / 4;
  hipLaunchKernelGGL((gemv_kernel<F, kRows, NB, XF16, EPI>), dim3(blocks), dim3(256), 0, s, a);
}

template <class F, bool XF16, int EPI>
void launch_rows(GemvArgs a, int nrows, hipStream_t s) {
  const size_t xel = XF16 ? 2 : 4;
  while (nrows > 0) {
    int nb = std::min(nrows, 8);
    switch (nb) {
      case 1: launch_nb<F, 1, XF16, EPI>(a, s); break;
      case 2: launch_nb<F, 2, XF16, EPI>(a, s); break;
      case 3: launch_nb<F, 3, XF16, EPI>(a, s); break;
      case 4: launch_nb<F, 4, XF16, EPI>(a, s); break;
      case 5: launch_nb<F, 5, XF16, EPI>(a, s); break;
      case 6: launch_nb<F, 6, XF16, EPI>(a, s); break;
      case 7: launch_nb<F, 7, XF16, EPI>(a, s); break;
      default: launch_nb<F, 8, XF16, EPI>(a, s); break;
    }
    PGD_HIP(hipGetLastError());
    nrows -= nb;
    a.x = reinterpret_cast<const uint8_t*>(a.x) + (size_t)nb * a.ldx * xel;
    a.y += (size_t)nb * a.ldy;
    if (a.res) a.res += (size_t)nb * a.ldres;
  }
}

template <bool XF16, int EPI>
void dispatch_fmt(const QMat& m, GemvArgs a, int nrows, hipStream_t s) {
  switch (m.fmt) {
    case FMT_A8: launch_rows<A8, XF16, EPI>(a, nrows, s); break;
    case FMT_Q4K: launch_rows<Q4K, XF16, EPI>(a, nrows, s); break;
    case FMT_Q6K: launch_rows<Q6K, XF16, EPI>(a, nrows, s); break;
    default: throw Error{kErrFormat, "unknown matrix format"};
  }
}

GemvArgs make_args(const QMat& m) {
  GemvArgs a{};
  a.p0 = m.p0;
  a.p1 = m.p1;
  a.p2 = m.p2;
  a.p3 = m.p3;
  a.n_out = m.n_out;
  a.n_in = m.n_in;
  a.nsb = m.nsb;
  return a;
}

// ---- dequant ----------------------------------------------------------------
// One thread per 16-element run. Formulas are the host ones, evaluated with
// FP contraction off (build flag) so each product rounds like the C code.
__global__ void dequant_a8_kernel(const uint8_t* codes, const uint32_t* sb, int n_in, int row0, int rows,
                                  const uint32_t* ids, float* out, int ldo) {
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  int runs = n_in >> 4;
  if (t >= (size_t)rows * runs) return;
  int r = (int)(t / runs), c = (int)(t % runs);
  int row = ids ? (int)ids[r] : row0 + r;
  uint4 q = *reinterpret_cast<const uint4*>(codes + (size_t)row * n_in + c * 16);
  uint32_t v = sb[(size_t)row * (n_in >> 6) + (c >> 2)];
  float s = bf16_to_f32(v & 0xffffu), b = bf16_to_f32(v >> 16);
  float* o = out + (size_t)r * ldo + c * 16;
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = b + s * (float)byte_of(q, i);
}

__global__ void dequant_q4k_kernel(const uint8_t* qs, const uint4* hdr, int n_in, int nsb, int row0, int rows,
                                   const uint32_t* ids, float* out, int ldo) {
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  int runs = nsb * 8;
  if (t >= (size_t)rows * runs) return;
  int r = (int)(t / runs), p = (int)(t % runs);
  int row = ids ? (int)ids[r] : row0 + r;
  int sb = p >> 3, part = p & 7, j = part >> 1, h = part & 1;
  uint4 q = *reinterpret_cast<const uint4*>(qs + (size_t)row * nsb * 128 + (size_t)p * 16);
  uint4 hd = hdr[(size_t)row * nsb + sb];
  float d = f16_to_f32(hd.x & 0xffffu), dmin = f16_to_f32(hd.x >> 16);
  float sc0, m0, sc1, m1;
  Q4K::scale_min(hd, 2 * j, sc0, m0);
  Q4K::scale_min(hd, 2 * j + 1, sc1, m1);
  float d1 = d * sc0, mm1 = dmin * m0, d2 = d * sc1, mm2 = dmin * m1;
  int lo = sb * 256 + 64 * j + 16 * h, hi = lo + 32;
  float* o = out + (size_t)r * ldo;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    uint32_t b = byte_of(q, i);
    if (lo + i < n_in) o[lo + i] = d1 * (float)(b & 15u) - mm1;
    if (hi + i < n_in) o[hi + i] = d2 * (float)(b >> 4) - mm2;
  }
}

__global__ void dequant_q6k_kernel(const uint8_t* qlp, const uint8_t* qhp, const int8_t* scp, const uint16_t* dp,
                                   int n_in, int nsb, int row0, int rows, const uint32_t* ids, float* out,
                                   int ldo) {
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  int runs = nsb * 8;
  if (t >= (size_t)rows * runs) return;
  int r = (int)(t / runs), p = (int)(t % runs);
  int row = ids ? (int)ids[r] : row0 + r;
  int sb = p >> 3, part = p & 7, n = part >> 2, c = part & 3;
  uint4 ql = *reinterpret_cast<const uint4*>(qlp + (size_t)row * nsb * 128 + (size_t)p * 16);
  uint4 qh = *reinterpret_cast<const uint4*>(qhp + (size_t)row * nsb * 64 + sb * 64 + 32 * n + 16 * (c & 1));
  const int8_t* sc = scp + (size_t)row * nsb * 16 + sb * 16 + 8 * n + c;
  float d = f16_to_f32(dp[(size_t)row * nsb + sb]);
  float slo = (float)sc[0], shi = (float)sc[4];
  int shl = 2 * (c >> 1), shh = 4 + 2 * (c >> 1);
  int lo = sb * 256 + 128 * n + 16 * c, hi = lo + 64;
  float* o = out + (size_t)r * ldo;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    uint32_t l = byte_of(ql, i), h = byte_of(qh, i);
    int q1 = (int)((l & 15u) | (((h >> shl) & 3u) << 4)) - 32;
    int q2 = (int)((l >> 4) | (((h >> shh) & 3u) << 4)) - 32;
    // GGML: y = d * sc * q, left to right
    if (lo + i < n_in) o[lo + i] = d * slo * (float)q1;
    if (hi + i < n_in) o[hi + i] = d * shi * (float)q2;
  }
}

void launch_dequant(const QMat& m, int row0, int rows, const uint32_t* ids, float* out, int ldo, hipStream_t s) {
  if (rows <= 0) return;
  size_t runs = m.fmt == FMT_A8 ? (size_t)(m.n_in >> 4) : (size_t)m.nsb * 8;
  size_t n = runs * rows;
  int blocks = (int)((n + 255) / 256);
  switch (m.fmt) {
    case FMT_A8:
      hipLaunchKernelGGL(dequant_a8_kernel, dim3(blocks), dim3(256), 0, s, m.p0,
                         reinterpret_cast<const uint32_t*>(m.p1), m.n_in, row0, rows, ids, out, ldo);
      break;
    case FMT_Q4K:
      hipLaunchKernelGGL(dequant_q4k_kernel, dim3(blocks), dim3(256), 0, s, m.p0,
                         reinterpret_cast<const uint4*>(m.p1), m.n_in, m.nsb, row0, rows, ids, out, ldo);
      break;
    case FMT_Q6K:
      hipLaunchKernelGGL(dequant_q6k_kernel, dim3(blocks), dim3(256), 0, s, m.p0, m.p1,
                         reinterpret_cast<const int8_t*>(m.p2), reinterpret_cast<const uint16_t*>(m.p3), m.n_in,
                         m.nsb, row0, rows, ids, out, ldo);
      break;
    default: throw Error{kErrFormat, "unknown matrix format"};
  }
  PGD_HIP(hipGetLastError());
}

// ---- synthetic generator ----------------------------------------------------
// Same definition as the CPU checker: splitmix64 counter stream per tensor
// key, N(0,1) = Irwin-Hall sum of 12 16-bit uniforms minus 6 (integers, so
// bit-identical on host and device).
__host__ __device__ inline uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t synth_stream(uint64_t seed, uint64_t key) {
  return splitmix64(seed ^ splitmix64(key));
}

__device__ inline float synth_normal(uint64_t stream, uint64_t idx) {
  uint64_t base = stream + idx * 3u;
  int64_t s = 0;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    uint64_t h = splitmix64(base + (uint64_t)j);
    s += (int64_t)(h & 0xffffu) + (int64_t)((h >> 16) & 0xffffu) + (int64_t)((h >> 32) & 0xffffu) +
         (int64_t)(h >> 48);
  }
  int32_t t = (int32_t)(s - 393210);
  return (float)t * (1.0f / 65536.0f);
}

__device__ inline float synth_uniform(uint64_t stream, uint64_t idx) {
  uint64_t h = splitmix64(stream + idx * 3u);
  return (float)(uint32_t)(h >> 40) * (1.0f / 16777216.0f);
}

__device__ inline float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

// MLX affine quantizer, one thread per (row, group of 64).
__global__ void synth_a8_kernel(uint8_t* codes, uint32_t* sb, int n_out, int n_in, uint64_t stream, float std) {
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  int groups = n_in >> 6;
  if (t >= (size_t)n_out * groups) return;
  size_t r = t / groups;
  int g = (int)(t % groups);
  size_t base = r * n_in + (size_t)g * 64;
  float w[64];
  float mx, mn;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    w[i] = std * synth_normal(stream, base + i);
    if (i == 0) {
      mx = w[0];
      mn = w[0];
    } else {
      if (w[i] > mx) mx = w[i];
      if (w[i] < mn) mn = w[i];
    }
  }
  bool mask = fabsf(mn) > fabsf(mx);
  float scale = (mx - mn) / 255.0f;
  if (scale < 1e-7f) scale = 1e-7f;
  if (!mask) scale = -scale;
  float edge = mask ? mn : mx;
  float q0 = rintf(edge / scale);
  float bias = edge;
  if (q0 != 0.0f) scale = edge / q0;
  else bias = 0.0f;
  uint32_t words[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) words[i] = 0;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    float q = clampf(rintf((w[i] - bias) / scale), 0.0f, 255.0f);
    words[i >> 2] |= (uint32_t)q << (8 * (i & 3));
  }
  uint4* dst = reinterpret_cast<uint4*>(codes + base);
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[i] = make_uint4(words[4 * i], words[4 * i + 1], words[4 * i + 2], words[4 * i + 3]);
  sb[r * groups + g] = (uint32_t)f32_to_bf16(scale) | ((uint32_t)f32_to_bf16(bias) << 16);
}

__device__ inline float synth_w(uint64_t stream, float std, size_t r, int n_in, int k) {
  return k < n_in ? std * synth_normal(stream, r * (size_t)n_in + k) : 0.0f;
}

// Q4K quantizer (same choices as the CPU checker), one thread per block.
__global__ void synth_q4k_kernel(uint8_t* qs, uint4* hdr, int n_out, int n_in, int nsb, uint64_t stream, float std) {
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (size_t)n_out * nsb) return;
  size_t r = t / nsb;
  int b = (int)(t % nsb);
  float scale[8], mins[8], maxs = 0.0f, maxm = 0.0f;
  for (int j = 0; j < 8; ++j) {
    int k0 = b * 256 + 32 * j;
    float mn = 0.0f, mx = synth_w(stream, std, r, n_in, k0);
    for (int i = 0; i < 32; ++i) {
      float v = synth_w(stream, std, r, n_in, k0 + i);
      if (v < mn) mn = v;
      if (v > mx) mx = v;
    }
    scale[j] = (mx - mn) / 15.0f;
    mins[j] = -mn;
    if (scale[j] > maxs) maxs = scale[j];
    if (mins[j] > maxm) maxm = mins[j];
  }
  uint16_t dh = f32_to_f16(maxs / 63.0f), mh = f32_to_f16(maxm / 63.0f);
  float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
  uint8_t sc[12];
  for (int i = 0; i < 12; ++i) sc[i] = 0;
  uint8_t scq[8], mq[8];
  for (int j = 0; j < 8; ++j) {
    scq[j] = d > 0.0f ? (uint8_t)clampf(rintf(scale[j] / d), 0.0f, 63.0f) : 0;
    mq[j] = dmin > 0.0f ? (uint8_t)clampf(rintf(mins[j] / dmin), 0.0f, 63.0f) : 0;
    if (j < 4) {
      sc[j] = (uint8_t)((sc[j] & 0xC0) | (scq[j] & 63));
      sc[j + 4] = (uint8_t)((sc[j + 4] & 0xC0) | (mq[j] & 63));
    } else {
      sc[j + 4] = (uint8_t)((scq[j] & 0xF) | ((mq[j] & 0xF) << 4));
      sc[j - 4] = (uint8_t)((sc[j - 4] & 63) | ((scq[j] >> 4) << 6));
      sc[j] = (uint8_t)((sc[j] & 63) | ((mq[j] >> 4) << 6));
    }
  }
  uint32_t sw[3];
  for (int i = 0; i < 3; ++i)
    sw[i] = (uint32_t)sc[4 * i] | ((uint32_t)sc[4 * i + 1] << 8) | ((uint32_t)sc[4 * i + 2] << 16) |
            ((uint32_t)sc[4 * i + 3] << 24);
  hdr[t] = make_uint4((uint32_t)dh | ((uint32_t)mh << 16), sw[0], sw[1], sw[2]);
  uint8_t* q = qs + t * 128;
  for (int grp = 0; grp < 4; ++grp) {
    int j0 = 2 * grp, j1 = 2 * grp + 1;
    float ds0 = d * (float)scq[j0], dm0 = dmin * (float)mq[j0];
    float ds1 = d * (float)scq[j1], dm1 = dmin * (float)mq[j1];
    for (int l4 = 0; l4 < 32; l4 += 4) {
      uint32_t word = 0;
      for (int e = 0; e < 4; ++e) {
        int l = l4 + e;
        float v0 = synth_w(stream, std, r, n_in, b * 256 + 32 * j0 + l);
        float v1 = synth_w(stream, std, r, n_in, b * 256 + 32 * j1 + l);
        float q0 = ds0 > 0.0f ? clampf(rintf((v0 + dm0) / ds0), 0.0f, 15.0f) : 0.0f;
        float q1 = ds1 > 0.0f ? clampf(rintf((v1 + dm1) / ds1), 0.0f, 15.0f) : 0.0f;
        word |= ((uint32_t)q0 | ((uint32_t)q1 << 4)) << (8 * e);
      }
      *reinterpret_cast<uint32_t*>(q + 32 * grp + l4) = word;
    }
  }
}

// Q6K quantizer, one thread per block.
__global__ void synth_q6k_kernel(uint8_t* qlp, uint8_t* qhp, int8_t* scp, uint16_t* dp, int n_out, int n_in,
                                 int nsb, uint64_t stream, float std) {
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (size_t)n_out * nsb) return;
  size_t r = t / nsb;
  int b = (int)(t % nsb);
  float scale[16], maxs = 0.0f;
  for (int j = 0; j < 16; ++j) {
    float amax = 0.0f;
    for (int i = 0; i < 16; ++i) {
      float v = fabsf(synth_w(stream, std, r, n_in, b * 256 + 16 * j + i));
      if (v > amax) amax = v;
    }
    scale[j] = amax / 31.0f;
    if (scale[j] > maxs) maxs = scale[j];
  }
  uint16_t dh = f32_to_f16(maxs / 127.0f);
  float d = f16_to_f32(dh);
  dp[t] = dh;
  int8_t scq[16];
  for (int j = 0; j < 16; ++j) {
    scq[j] = d > 0.0f ? (int8_t)clampf(rintf(scale[j] / d), 0.0f, 127.0f) : 0;
    scp[t * 16 + j] = scq[j];
  }
  uint8_t* ql = qlp + t * 128;
  uint8_t* qh = qhp + t * 64;
  for (int n = 0; n < 2; ++n) {
    for (int l = 0; l < 32; ++l) {
      uint32_t c[4];
      for (int u = 0; u < 4; ++u) {
        int e = 128 * n + 32 * u + l;
        int j = e / 16;
        float ds = d * (float)scq[j];
        float v = synth_w(stream, std, r, n_in, b * 256 + e);
        float q = ds > 0.0f ? clampf(rintf(v / ds), -32.0f, 31.0f) : 0.0f;
        c[u] = (uint32_t)((int)q + 32);
      }
      ql[64 * n + l] = (uint8_t)((c[0] & 0xF) | ((c[2] & 0xF) << 4));
      ql[64 * n + l + 32] = (uint8_t)((c[1] & 0xF) | ((c[3] & 0xF) << 4));
      qh[32 * n + l] = (uint8_t)((c[0] >> 4) | ((c[1] >> 4) << 2) | ((c[2] >> 4) << 4) | ((c[3] >> 4) << 6));
    }
  }
}

__global__ void synth_vec_kernel(float* out, size_t n, uint64_t stream, float scale, int uniform) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = scale * (uniform ? synth_uniform(stream, i) : synth_normal(stream, i));
}

__global__ void fill_kernel(float* out, size_t n, float v) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = v;
}

}  // namespace

// ---------------------------------------------------------------------------
double qmat_algo_bytes(const QMat& m) {
  double n = (double)m.n_out * (double)m.n_in;
  switch (m.fmt) {
    case FMT_A8: return n * 8.5 / 8.0;
    case FMT_Q4K: return n * 4.5 / 8.0;
    case FMT_Q6K: return n * 6.5625 / 8.0;
  }
  return 0.0;
}

void qmat_alloc(QMat& m, int fmt, int n_out, int n_in) {
  PGD_CHECK(n_out > 0 && n_in > 0, kErrShape, "matrix dims must be positive");
  m.fmt = fmt;
  m.n_out = n_out;
  m.n_in = n_in;
  m.nsb = (n_in + 255) / 256;
  size_t rows = (size_t)n_out;
  size_t off[4] = {0, 0, 0, 0};
  size_t total = 0;
  auto place = [&](int i, size_t bytes) {
    total = (total + 255) & ~(size_t)255;
    off[i] = total;
    total += bytes;
  };
  if (fmt == FMT_A8) {
    PGD_CHECK(n_in % 64 == 0, kErrShape, "A8 n_in must be a multiple of 64");
    place(0, rows * n_in);
    place(1, rows * (n_in / 64) * 4);
  } else if (fmt == FMT_Q4K) {
    PGD_CHECK(n_in % 32 == 0, kErrShape, "Q4K n_in must be a multiple of 32");
    place(0, rows * m.nsb * 128);
    place(1, rows * m.nsb * 16);
  } else if (fmt == FMT_Q6K) {
    PGD_CHECK(n_in % 32 == 0, kErrShape, "Q6K n_in must be a multiple of 32");
    place(0, rows * m.nsb * 128);
    place(1, rows * m.nsb * 64);
    place(2, rows * m.nsb * 16);
    place(3, rows * m.nsb * 2);
  } else {
    throw Error{kErrFormat, "unknown matrix format"};
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, total);
  if (e != hipSuccess) throw Error{kErrAlloc, std::string("hipMalloc matrix: ") + hipGetErrorString(e)};
  m.base = (uint8_t*)p;
  m.bytes = total;
  m.p0 = m.base + off[0];
  m.p1 = m.base + off[1];
  m.p2 = fmt == FMT_Q6K ? m.base + off[2] : nullptr;
  m.p3 = fmt == FMT_Q6K ? m.base + off[3] : nullptr;
}

void qmat_free(QMat& m) {
  if (m.base) (void)hipFree(m.base);
  m = QMat{};
}

void qmat_upload_a8(QMat& m, const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                    hipStream_t s) {
  size_t groups = (size_t)m.n_out * (m.n_in / 64);
  std::vector<uint32_t> sb(groups);
  for (size_t i = 0; i < groups; ++i) sb[i] = (uint32_t)scales[i] | ((uint32_t)biases[i] << 16);
  PGD_HIP(hipMemcpyAsync(m.p0, packed, (size_t)m.n_out * m.n_in, hipMemcpyHostToDevice, s));
  PGD_HIP(hipMemcpyAsync(m.p1, sb.data(), groups * 4, hipMemcpyHostToDevice, s));
  PGD_HIP(hipStreamSynchronize(s));
}

void qmat_upload_kq(QMat& m, const uint8_t* blocks, hipStream_t s) {
  size_t nb = (size_t)m.n_out * m.nsb;
  if (m.fmt == FMT_Q4K) {
    std::vector<uint8_t> qs(nb * 128), hdr(nb * 16);
    for (size_t i = 0; i < nb; ++i) {
      const uint8_t* b = blocks + i * 144;
      std::copy(b, b + 16, hdr.data() + i * 16);
      std::copy(b + 16, b + 144, qs.data() + i * 128);
    }
    PGD_HIP(hipMemcpyAsync(m.p0, qs.data(), qs.size(), hipMemcpyHostToDevice, s));
    PGD_HIP(hipMemcpyAsync(m.p1, hdr.data(), hdr.size(), hipMemcpyHostToDevice, s));
    PGD_HIP(hipStreamSynchronize(s));
  } else if (m.fmt == FMT_Q6K) {
    std::vector<uint8_t> ql(nb * 128), qh(nb * 64), sc(nb * 16), d(nb * 2);
    for (size_t i = 0; i < nb; ++i) {
      const uint8_t* b = blocks + i * 210;
      std::copy(b, b + 128, ql.data() + i * 128);
      std::copy(b + 128, b + 192, qh.data() + i * 64);
      std::copy(b + 192, b + 208, sc.data() + i * 16);
      std::copy(b + 208, b + 210, d.data() + i * 2);
    }
    PGD_HIP(hipMemcpyAsync(m.p0, ql.data(), ql.size(), hipMemcpyHostToDevice, s));
    PGD_HIP(hipMemcpyAsync(m.p1, qh.data(), qh.size(), hipMemcpyHostToDevice, s));
    PGD_HIP(hipMemcpyAsync(m.p2, sc.data(), sc.size(), hipMemcpyHostToDevice, s));
    PGD_HIP(hipMemcpyAsync(m.p3, d.data(), d.size(), hipMemcpyHostToDevice, s));
    PGD_HIP(hipStreamSynchronize(s));
  } else {
    throw Error{kErrFormat, "k-quant upload on a non k-quant matrix"};
  }
}

void qmat_dequant(const QMat& m, int row0, int rows, float* out, hipStream_t s) {
  PGD_CHECK(row0 >= 0 && rows >= 0 && row0 + rows <= m.n_out, kErrShape, "dequant row range");
  launch_dequant(m, row0, rows, nullptr, out, m.n_in, s);
}

void qmat_embed(const QMat& m, const uint32_t* ids, int nrows, float* out, int ldo, hipStream_t s) {
  launch_dequant(m, 0, nrows, ids, out, ldo, s);
}

void qmat_gemv(const QMat& m, const void* x, int x_f16, int ldx, int nrows, float* y, int ldy, const float* res,
               int ldres, hipStream_t s) {
  PGD_CHECK(nrows >= 0, kErrShape, "gemv rows");
  PGD_CHECK(ldx >= m.n_in && ldx % 8 == 0, kErrShape, "gemv ldx must be >= n_in and a multiple of 8");
  if (nrows == 0) return;
  GemvArgs a = make_args(m);
  a.x = x;
  a.ldx = ldx;
  a.y = y;
  a.ldy = ldy;
  a.res = res;
  a.ldres = ldres;
  if (x_f16) {
    if (res) dispatch_fmt<true, EPI_RES>(m, a, nrows, s);
    else dispatch_fmt<true, EPI_STORE>(m, a, nrows, s);
  } else {
    if (res) dispatch_fmt<false, EPI_RES>(m, a, nrows, s);
    else dispatch_fmt<false, EPI_STORE>(m, a, nrows, s);
  }
}

void qmat_gemv_swiglu(const QMat& gate, const QMat& up, const float* x, int ldx, int nrows, float* mid, int ldm,
                      hipStream_t s) {
  PGD_CHECK(gate.fmt == up.fmt && gate.n_out == up.n_out && gate.n_in == up.n_in, kErrShape,
            "swiglu gate/up shapes differ");
  PGD_CHECK(ldx >= gate.n_in && ldx % 8 == 0, kErrShape, "gemv ldx must be >= n_in and a multiple of 8");
  if (nrows == 0) return;
  GemvArgs a = make_args(gate);
  a.u0 = up.p0;
  a.u1 = up.p1;
  a.u2 = up.p2;
  a.u3 = up.p3;
  a.x = x;
  a.ldx = ldx;
  a.y = mid;
  a.ldy = ldm;
  dispatch_fmt<false, EPI_SWIGLU>(gate, a, nrows, s);
}

void qmat_synth(QMat& m, uint64_t seed, uint64_t key, float std, hipStream_t s) {
  uint64_t stream = synth_stream(seed, key);
  if (m.fmt == FMT_A8) {
    size_t n = (size_t)m.n_out * (m.n_in / 64);
    hipLaunchKernelGGL(synth_a8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, m.p0,
                       reinterpret_cast<uint32_t*>(m.p1), m.n_out, m.n_in, stream, std);
  } else if (m.fmt == FMT_Q4K) {
    size_t n = (size_t)m.n_out * m.nsb;
    hipLaunchKernelGGL(synth_q4k_kernel, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, s, m.p0,
                       reinterpret_cast<uint4*>(m.p1), m.n_out, m.n_in, m.nsb, stream, std);
  } else {
    size_t n = (size_t)m.n_out * m.nsb;
    hipLaunchKernelGGL(synth_q6k_kernel, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, s, m.p0, m.p1,
                       reinterpret_cast<int8_t*>(m.p2), reinterpret_cast<uint16_t*>(m.p3), m.n_out, m.n_in, m.nsb,
                       stream, std);
  }
  PGD_HIP(hipGetLastError());
}

void synth_normal_f32(float* out, size_t n, uint64_t seed, uint64_t key, float scale, hipStream_t s) {
  if (!n) return;
  hipLaunchKernelGGL(synth_vec_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, n,
                     synth_stream(seed, key), scale, 0);
  PGD_HIP(hipGetLastError());
}

void synth_uniform_f32(float* out, size_t n, uint64_t seed, uint64_t key, float scale, hipStream_t s) {
  if (!n) return;
  hipLaunchKernelGGL(synth_vec_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, n,
                     synth_stream(seed, key), scale, 1);
  PGD_HIP(hipGetLastError());
}

void fill_f32(float* out, size_t n, float v, hipStream_t s) {
  if (!n) return;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, n, v);
  PGD_HIP(hipGetLastError());
}

}  // namespace pgd
