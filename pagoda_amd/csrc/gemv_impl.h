// gemv_impl.h — GEMV kernel templates shared by the per-format
// instantiation files (gemv_a8.hip, gemv_q4k.hip, gemv_q6k.hip).
//
// Dequant-in-register GEMV / skinny GEMM on the vector ALUs for GGML Q4_K /
// Q6_K / Q8_0 / Q5_0 matrices (MLX affine-8 runs on the matrix cores, gemv_mma.hip).
//
// GEMV mapping (wave64): a wave owns ROWS consecutive output rows. A row is
// cut into 16-byte chunks of its main plane (Q4K qs / Q6K ql);
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
#pragma once
#include <algorithm>

#include "common.h"
#include "quant.h"

namespace pgd {
namespace gemv {


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
  // SwiGLU only: also write the product as prepared A8 activations (XA null:
  // no); row0 = first row of this launch within that activation
  a8act::Dst oact;
  int row0;
  // deferred RMSNorm of the input (null: none): rss rows of this launch,
  // rss_nh partials per row, row width rss_n, eps; outputs are scaled by
  // rss_inv() of their row. inv: optional per-launch-row copy of those
  // factors written by the stream-K kernel for its fix-up kernel.
  const float* rss;
  int rss_nh, rss_n;
  float rss_eps;
  float* inv;
  // residual launches only: also emit the next RMSNorm's deferred input from
  // the new rows h = res + W x (operands of h * nw into nact, per-32-column
  // sums of h^2 into nrss [rows][n_out / 32]); nact.XA null: no
  a8act::Dst nact;
  const float* nw;
  float* nrss;
  // split-K store launches of 1..4 rows, every row one sequence's only token
  // (cout null: none): outputs n < conv_n of row r (absolute, row0 + launch row) also go
  // through the causal conv step of channel n (weights cw [conv_n][conv_k],
  // state at cbase[r] + coff, [conv_n][conv_k - 1], updated) into
  // cout[r * ldc + n]
  const float* cw;
  float* const* cbase;
  size_t coff;
  float* cout;
  int ldc, conv_n, conv_k;
};

// the causal conv step of one channel for one row: conv_step_kernel's
// arithmetic and order, the state shifted in place
__device__ inline void conv_channel(const GemvArgs& a, int row, int n, float xv) {
  const int hist = a.conv_k - 1;
  float* cs = a.cbase[row] + a.coff + (size_t)n * hist;
  const float* wt = a.cw + (size_t)n * a.conv_k;
  float acc = 0.0f;
  for (int k = 0; k < hist; ++k) acc += cs[k] * wt[k];
  acc += xv * wt[hist];
  a.cout[(size_t)row * a.ldc + n] = acc / (1.0f + expf(-acc));
  for (int k = 0; k + 1 < hist; ++k) cs[k] = cs[k + 1];
  if (hist > 0) cs[hist - 1] = xv;
}

// 1/rms of one deferred-norm row from its partial sums of squares: lane l adds
// partials l, l + 64, ... in turn, then a xor butterfly (each step adds the
// same two values on both lanes, so every lane ends with the same sum). The
// whole wave calls it; the same function in every consumer.
__device__ inline float rss_inv(const float* rss_row, int nh, int n, float eps) {
  const int lane = threadIdx.x & 63;
  float s = 0.0f;
  for (int i = lane; i < nh; i += 64) s += rss_row[i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  return 1.0f / sqrtf(s / (float)n + eps);
}

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
      v[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu));
      v[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
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
    w.q = *reinterpret_cast<const uint4*>(c0 + q4k_qs_off(row, p << 4, a.nsb));
    w.hdr = *reinterpret_cast<const uint4*>(c1 + q4k_hdr_off(row, p >> 3, a.nsb));
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
    // tiled planes (quant.h): the 16-byte runs arrive one dword at a time
    uint32_t l[4], h[4];
    const int hq = sb * 64 + 32 * n + 16 * (c & 1);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      l[k] = *reinterpret_cast<const uint32_t*>(c0 + q6k_ql_off(row, 16 * p + 4 * k, a.nsb));
      h[k] = *reinterpret_cast<const uint32_t*>(c1 + q6k_qh_off(row, hq + 4 * k, a.nsb));
    }
    w.ql = make_uint4(l[0], l[1], l[2], l[3]);
    w.qh = make_uint4(h[0], h[1], h[2], h[3]);
    const int8_t* sc = reinterpret_cast<const int8_t*>(c2);
    float d = f16_to_f32(reinterpret_cast<const uint16_t*>(c3)[q6k_d_off(row, sb, a.nsb)]);
    w.s_lo = d * (float)sc[q6k_sc_off(row, sb * 16 + 8 * n + c, a.nsb)];
    w.s_hi = d * (float)sc[q6k_sc_off(row, sb * 16 + 8 * n + c + 4, a.nsb)];
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

// Q8_0: chunk p = half p % 2 of block p / 2 of the row (16 weights, so a
// 896-wide row gives 56 chunks for the wave's 64 lanes); y = q * d.
struct Q80 {
  struct W {
    uint4 q;
    float d;
  };
  static __device__ inline int chunks(const GemvArgs& a) { return a.nsb * 2; }
  static __device__ inline bool pos(const GemvArgs& a, int p, int& lo, int& hi) {
    lo = p << 4;
    hi = -1;
    return true;
  }
  static __device__ inline W load(const uint8_t* c0, const uint8_t* c1, const uint8_t*, const uint8_t*,
                                  const GemvArgs& a, int row, int p) {
    W w;
    w.q = *reinterpret_cast<const uint4*>(c0 + (size_t)row * a.n_in + (p << 4));
    w.d = f16_to_f32(reinterpret_cast<const uint16_t*>(c1)[(size_t)row * a.nsb + (p >> 1)]);
    return w;
  }
  static __device__ inline float acc(float r, const W& w, const float* xl, const float*, float, float, int, bool) {
    float dl = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) dl = fmaf((float)(int8_t)byte_of(w.q, i), xl[i], dl);
    return fmaf(w.d, dl, r);
  }
};

// Q5_0: chunk p = half h = p % 2 of block p / 2; qs byte j holds weight j
// (low nibble) and weight j + 16 (high nibble), qh bit j / j + 16 their fifth
// bit; y = (q - 16) * d.
struct Q50 {
  struct W {
    uint4 q;
    uint32_t qh;
    float d;
  };
  static __device__ inline int chunks(const GemvArgs& a) { return a.nsb * 2; }
  static __device__ inline bool pos(const GemvArgs& a, int p, int& lo, int& hi) {
    lo = p << 4;
    hi = -1;
    return true;
  }
  static __device__ inline W load(const uint8_t* c0, const uint8_t* c1, const uint8_t* c2, const uint8_t*,
                                  const GemvArgs& a, int row, int p) {
    W w;
    const size_t b = (size_t)row * a.nsb + (p >> 1);
    w.q = *reinterpret_cast<const uint4*>(c0 + b * 16);
    w.qh = reinterpret_cast<const uint32_t*>(c1)[b] >> (16 * (p & 1));
    w.d = f16_to_f32(reinterpret_cast<const uint16_t*>(c2)[b]);
    return w;
  }
  static __device__ inline float acc(float r, const W& w, const float* xl, const float*, float sl, float, int p,
                                     bool) {
    const int sh = 4 * (p & 1);  // low or high nibbles
    float dl = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t q = ((byte_of(w.q, i) >> sh) & 15u) | (((w.qh >> i) & 1u) << 4);
      dl = fmaf((float)q, xl[i], dl);
    }
    // sum (q - 16) x = sum q x - 16 sum x
    return fmaf(w.d, fmaf(-16.0f, sl, dl), r);
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


// entry points of the instantiation files
void run_q4k(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s);
void run_q6k(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s);
void run_q80(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s);
void run_q50(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s);
// Q4K on the matrix cores (n_in % 64 == 0)
bool q4k_mma_ok(const GemvArgs& a);
void run_q4k_mma(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s);
bool q6k_mma_ok(const GemvArgs& a, int epi);
void run_q6k_mma(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s);
// Per-stream device scratch that grows on demand (the stream is synchronized
// before a buffer is replaced). Slots are independent buffers: 0 for prepared
// activations and small reductions, 1 for split-K partial sums, 3 for
// stream-K partial sums, 4 for attention chunk states, 5 for per-row scales.
void* gemv_scratch(hipStream_t s, size_t bytes, int slot = 0);
// device scratch bytes (with per-slot alignment) one prepared-activation A8
// GEMV of `rows` rows takes through run_a8_mma (epi EPI_STORE or EPI_RES, no
// norm emission), following launch_prepped's choice of kernels
size_t a8_scratch_need(const GemvArgs& a, int rows, int epi);
// stream-K scratch of one 5..32-row chunk (slots 3 and 5, unaligned sizes)
void sk_scratch_need(const GemvArgs& a, int nb, int epi, size_t* slot3, size_t* slot5);
// GGML formats with candle's CPU arithmetic (activations quantized to Q8_K /
// Q8_0, integer block dots); f32 activations
void run_q8act(int fmt, const GemvArgs& a, int nrows, int epi, hipStream_t s);
// two store GEMVs of one input in one launch (formats of one activation type)
bool q8act_pair_ok(int fmt_a, int fmt_b);
void run_q8act_pair(int fmt_a, const GemvArgs& a, int fmt_b, const GemvArgs& b, int nrows, hipStream_t s);
// A8 on the matrix cores (f32 activations)
void run_a8_mma(const GemvArgs& a, const A8Act& act, int epi, hipStream_t s);
// A8 GEMM for prefill-sized batches: rows [0, rows) of a prepared activation
// (whose chunks there are in the full, not compact, layout), epilogue STORE,
// RES or SWIGLU into a.y (no prepared-output emits, no conv)
void run_a8_gemm(const GemvArgs& a, const uint4* XA, const float* CA, int rows, int epi, hipStream_t s);
// workgroups of that GEMM (256 weight rows, or 128 SwiGLU pairs, by 128 batch rows each)
int a8_gemm_workgroups(int n_out, int rows, int epi);
// Stream-K A8 kernel: whether a matrix takes it for 5..32-row launches, and
// one launch of 5..32 rows (operand chunk XA / CA of the prepared activations)
bool a8_sk_wanted(const GemvArgs& a, int epi);
void run_a8_sk_chunk(const GemvArgs& a, const uint4* XA, const float* CA, int nb, int epi, hipStream_t s);

}  // namespace gemv
}  // namespace pgd
