// quant.hip — quantized matrix storage: allocation, upload, dequant,
// embedding rows, the GEMV front end and the seeded synthetic generator.
#include <atomic>
#include <algorithm>
#include <map>
#include <mutex>
#include <vector>

#include "common.h"
#include "gemv_impl.h"
#include "quant.h"

namespace pgd {

using namespace gemv;

namespace {

void run_fmt(const QMat& m, const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s) {
  switch (m.fmt) {
    case FMT_A8: {
      PGD_CHECK(!x_f16, kErrArg, "A8 matrices take f32 activations");
      void* buf = gemv_scratch(s, a8_act_bytes(nrows, a.n_in));
      A8Act act = a8_act_prep(reinterpret_cast<const float*>(a.x), a.ldx, nrows, a.n_in, buf, s);
      run_a8_mma(a, act, epi, s);
      break;
    }
    case FMT_Q4K:
      if (q4k_mma_ok(a)) run_q4k_mma(a, nrows, x_f16, epi, s);
      else run_q4k(a, nrows, x_f16, epi, s);
      break;
    case FMT_Q6K:
      if (q6k_mma_ok(a, epi)) run_q6k_mma(a, nrows, x_f16, epi, s);
      else run_q6k(a, nrows, x_f16, epi, s);
      break;
    case FMT_Q8_0: run_q80(a, nrows, x_f16, epi, s); break;
    case FMT_Q5_0: run_q50(a, nrows, x_f16, epi, s); break;
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
  const int G = n_in >> 6;
  uint4 q = *reinterpret_cast<const uint4*>(codes + a8_code_off(row, c * 16, G));
  uint32_t v = sb[a8_sb_off(row, c >> 2, G)];
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
  uint4 q = *reinterpret_cast<const uint4*>(qs + q4k_qs_off(row, p * 16, nsb));
  uint4 hd = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(hdr) + q4k_hdr_off(row, sb, nsb));
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
  // ql bytes 16p.., qh bytes 64 sb + 32 n + 16 (c & 1).., one dword at a time
  uint32_t qlw[4], qhw[4];
  const int hq = sb * 64 + 32 * n + 16 * (c & 1);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    qlw[k] = *reinterpret_cast<const uint32_t*>(qlp + q6k_ql_off(row, 16 * p + 4 * k, nsb));
    qhw[k] = *reinterpret_cast<const uint32_t*>(qhp + q6k_qh_off(row, hq + 4 * k, nsb));
  }
  const uint4 ql = make_uint4(qlw[0], qlw[1], qlw[2], qlw[3]);
  const uint4 qh = make_uint4(qhw[0], qhw[1], qhw[2], qhw[3]);
  float d = f16_to_f32(dp[q6k_d_off(row, sb, nsb)]);
  float slo = (float)scp[q6k_sc_off(row, sb * 16 + 8 * n + c, nsb)];
  float shi = (float)scp[q6k_sc_off(row, sb * 16 + 8 * n + c + 4, nsb)];
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

// Q8_0 / Q5_0: one thread per 16-weight half block; y = q * d (GGML order)
__global__ void dequant_q80_kernel(const int8_t* q, const uint16_t* dp, int n_in, int nsb, int row0, int rows,
                                   const uint32_t* ids, float* out, int ldo) {
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int runs = nsb * 2;
  if (t >= (size_t)rows * runs) return;
  const int r = (int)(t / runs), c = (int)(t % runs);
  const int row = ids ? (int)ids[r] : row0 + r;
  const float d = f16_to_f32(dp[(size_t)row * nsb + (c >> 1)]);
  const int8_t* src = q + (size_t)row * n_in + 16 * c;
  float* o = out + (size_t)r * ldo + 16 * c;
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = (float)src[i] * d;
}

__global__ void dequant_q50_kernel(const uint8_t* qs, const uint32_t* qhp, const uint16_t* dp, int n_in, int nsb,
                                   int row0, int rows, const uint32_t* ids, float* out, int ldo) {
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int runs = nsb * 2;
  if (t >= (size_t)rows * runs) return;
  const int r = (int)(t / runs), c = (int)(t % runs), b = c >> 1, h = c & 1;
  const int row = ids ? (int)ids[r] : row0 + r;
  const size_t bi = (size_t)row * nsb + b;
  const float d = f16_to_f32(dp[bi]);
  const uint32_t qh = qhp[bi];
  const uint8_t* src = qs + bi * 16;
  float* o = out + (size_t)r * ldo + 32 * b + 16 * h;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t nib = h ? (uint32_t)(src[j] >> 4) : (uint32_t)(src[j] & 15u);
    const int qv = (int)(nib | (((qh >> (j + 16 * h)) & 1u) << 4)) - 16;
    o[j] = (float)qv * d;
  }
}

void launch_dequant(const QMat& m, int row0, int rows, const uint32_t* ids, float* out, int ldo, hipStream_t s) {
  if (rows <= 0) return;
  size_t runs = m.fmt == FMT_A8                                ? (size_t)(m.n_in >> 4)
                : (m.fmt == FMT_Q8_0 || m.fmt == FMT_Q5_0) ? (size_t)m.nsb * 2
                                                             : (size_t)m.nsb * 8;
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
    case FMT_Q8_0:
      hipLaunchKernelGGL(dequant_q80_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<const int8_t*>(m.p0),
                         reinterpret_cast<const uint16_t*>(m.p1), m.n_in, m.nsb, row0, rows, ids, out, ldo);
      break;
    case FMT_Q5_0:
      hipLaunchKernelGGL(dequant_q50_kernel, dim3(blocks), dim3(256), 0, s, m.p0,
                         reinterpret_cast<const uint32_t*>(m.p1), reinterpret_cast<const uint16_t*>(m.p2), m.n_in,
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
__global__ void synth_a8_kernel(uint8_t* codes, uint32_t* sb, int row0, int nrows, int n_in, uint64_t stream,
                                float std) {
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  int groups = n_in >> 6;
  if (t >= (size_t)nrows * groups) return;
  size_t rl = t / groups;  // row within the tensor (its own element numbering)
  size_t r = rl + row0;    // row within the stored matrix
  int g = (int)(t % groups);
  size_t base = rl * n_in + (size_t)g * 64;
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
  uint4* d0 = reinterpret_cast<uint4*>(codes + a8_code_off((int)r, g * 64, groups));
  uint4* d1 = reinterpret_cast<uint4*>(codes + a8_code_off((int)r, g * 64 + 32, groups));
  d0[0] = make_uint4(words[0], words[1], words[2], words[3]);
  d0[1] = make_uint4(words[4], words[5], words[6], words[7]);
  d1[0] = make_uint4(words[8], words[9], words[10], words[11]);
  d1[1] = make_uint4(words[12], words[13], words[14], words[15]);
  sb[a8_sb_off((int)r, g, groups)] = (uint32_t)f32_to_bf16(scale) | ((uint32_t)f32_to_bf16(bias) << 16);
}

__device__ inline float synth_w(uint64_t stream, float std, size_t r, int n_in, int k) {
  return k < n_in ? std * synth_normal(stream, r * (size_t)n_in + k) : 0.0f;
}

// Q4K quantizer (same choices as the CPU checker), one thread per block.
// rows row0 .. row0 + n_out - 1 of the matrix; the stream is indexed by the row
// within the window
__global__ void synth_q4k_kernel(uint8_t* qs, uint4* hdr, int n_out, int n_in, int nsb, uint64_t stream, float std,
                                 int row0) {
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
  *reinterpret_cast<uint4*>(reinterpret_cast<uint8_t*>(hdr) + q4k_hdr_off((int)r + row0, b, nsb)) =
      make_uint4((uint32_t)dh | ((uint32_t)mh << 16), sw[0], sw[1], sw[2]);
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
      *reinterpret_cast<uint32_t*>(qs + q4k_qs_off((int)r + row0, b * 128 + 32 * grp + l4, nsb)) = word;
    }
  }
}

// Q6K quantizer, one thread per block.
__global__ void synth_q6k_kernel(uint8_t* qlp, uint8_t* qhp, int8_t* scp, uint16_t* dp, int n_out, int n_in,
                                 int nsb, uint64_t stream, float std, int row0) {
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
  const int row = (int)r + row0;
  dp[q6k_d_off(row, b, nsb)] = dh;
  int8_t scq[16];
  for (int j = 0; j < 16; ++j) {
    scq[j] = d > 0.0f ? (int8_t)clampf(rintf(scale[j] / d), 0.0f, 127.0f) : 0;
    scp[q6k_sc_off(row, b * 16 + j, nsb)] = scq[j];
  }
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
      qlp[q6k_ql_off(row, b * 128 + 64 * n + l, nsb)] = (uint8_t)((c[0] & 0xF) | ((c[2] & 0xF) << 4));
      qlp[q6k_ql_off(row, b * 128 + 64 * n + l + 32, nsb)] = (uint8_t)((c[1] & 0xF) | ((c[3] & 0xF) << 4));
      qhp[q6k_qh_off(row, b * 64 + 32 * n + l, nsb)] =
          (uint8_t)((c[0] >> 4) | ((c[1] >> 4) << 2) | ((c[2] >> 4) << 4) | ((c[3] >> 4) << 6));
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
namespace gemv {
namespace {
thread_local ScratchArena* t_arena = nullptr;
}

ScratchArena* set_scratch_arena(ScratchArena* a) {
  ScratchArena* old = t_arena;
  t_arena = a;
  return old;
}

namespace {
std::atomic<uint64_t> g_scratch_epoch{0};
}

uint64_t scratch_epoch() { return g_scratch_epoch.load(std::memory_order_relaxed); }

void* gemv_scratch(hipStream_t s, size_t bytes, int slot) {
  if (ScratchArena* ar = t_arena) {
    PGD_CHECK(slot >= 0 && slot < 8, kErrArg, "scratch slot");
    if (ar->len[slot] < bytes) {
      const size_t at = (ar->used + 255) & ~(size_t)255;
      PGD_CHECK(at + bytes <= ar->cap, kErrShape,
                "launch needs more than the " + std::to_string(ar->cap >> 20) + " MiB of fixed scratch");
      ar->off[slot] = at;
      ar->len[slot] = bytes;
      ar->used = at + bytes;
    }
    return ar->base + ar->off[slot];
  }
  static std::mutex mu;
  static std::map<std::pair<hipStream_t, int>, std::pair<void*, size_t>> bufs;
  std::lock_guard<std::mutex> lock(mu);
  auto& e = bufs[{s, slot}];
  if (e.second < bytes) {
    if (e.first) {
      PGD_HIP(hipStreamSynchronize(s));
      PGD_HIP(hipFree(e.first));
      e.first = nullptr;
      e.second = 0;
    }
    size_t want = std::max(bytes, (size_t)4 << 20);
    g_scratch_epoch.fetch_add(1, std::memory_order_relaxed);
    hipError_t err = hipMalloc(&e.first, want);
    if (err != hipSuccess) throw Error{kErrAlloc, std::string("hipMalloc gemv scratch: ") + hipGetErrorString(err)};
    e.second = want;
  }
  return e.first;
}
}  // namespace gemv

double qmat_algo_bytes(const QMat& m) {
  double n = (double)m.n_out * (double)m.n_in;
  switch (m.fmt) {
    case FMT_A8: return n * 8.5 / 8.0;
    case FMT_Q4K: return n * 4.5 / 8.0;
    case FMT_Q6K: return n * 6.5625 / 8.0;
    case FMT_Q8_0: return n * 8.5 / 8.0;
    case FMT_Q5_0: return n * 5.5 / 8.0;
  }
  return 0.0;
}

void qmat_alloc(QMat& m, int fmt, int n_out, int n_in, hipStream_t s) {
  PGD_CHECK(n_out > 0 && n_in > 0, kErrShape, "matrix dims must be positive");
  m.fmt = fmt;
  m.n_out = n_out;
  m.n_in = n_in;
  m.nsb = (fmt == FMT_Q8_0 || fmt == FMT_Q5_0) ? n_in / 32 : (n_in + 255) / 256;
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
    size_t tiles = (rows + 31) / 32;
    place(0, tiles * (n_in / 64) * 2048);
    place(1, tiles * (n_in / 64) * 128);
  } else if (fmt == FMT_Q4K) {
    PGD_CHECK(n_in % 32 == 0, kErrShape, "Q4K n_in must be a multiple of 32");
    size_t tiles = (rows + 31) / 32;
    place(0, tiles * 4 * m.nsb * 1024);
    place(1, tiles * m.nsb * 512);
  } else if (fmt == FMT_Q6K) {
    PGD_CHECK(n_in % 32 == 0, kErrShape, "Q6K n_in must be a multiple of 32");
    size_t tiles = (rows + 31) / 32;
    place(0, tiles * m.nsb * 4096);
    place(1, tiles * m.nsb * 2048);
    place(2, tiles * m.nsb * 512);
    place(3, tiles * m.nsb * 64);
  } else if (fmt == FMT_Q8_0) {
    PGD_CHECK(n_in % 32 == 0, kErrShape, "Q8_0 n_in must be a multiple of 32");
    place(0, rows * n_in);
    place(1, rows * m.nsb * 2);
  } else if (fmt == FMT_Q5_0) {
    PGD_CHECK(n_in % 32 == 0, kErrShape, "Q5_0 n_in must be a multiple of 32");
    place(0, rows * n_in / 2);
    place(1, rows * m.nsb * 4);
    place(2, rows * m.nsb * 2);
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
  m.p2 = (fmt == FMT_Q6K || fmt == FMT_Q5_0) ? m.base + off[2] : nullptr;
  m.p3 = fmt == FMT_Q6K ? m.base + off[3] : nullptr;
  // zero the padding rows of the last tile, ordered before the writes that
  // follow on the same stream
  PGD_HIP(hipMemsetAsync(m.base, 0, total, s));
}

void qmat_free(QMat& m) {
  if (m.base) (void)hipFree(m.base);
  m = QMat{};
}

void qmat_upload_a8(QMat& m, const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                    hipStream_t s) {
  // MLX row-major packed codes -> tiled blocks (same bytes, permuted)
  const int G = m.n_in / 64;
  const size_t tiles = ((size_t)m.n_out + 31) / 32;
  std::vector<uint8_t> codes(tiles * G * 2048, 0);
  std::vector<uint32_t> sb(tiles * G * 32, 0);
  const uint8_t* src = reinterpret_cast<const uint8_t*>(packed);
  for (int r = 0; r < m.n_out; ++r) {
    for (int k = 0; k < m.n_in; k += 32)
      std::copy(src + (size_t)r * m.n_in + k, src + (size_t)r * m.n_in + k + 32, codes.data() + a8_code_off(r, k, G));
    for (int g = 0; g < G; ++g)
      sb[a8_sb_off(r, g, G)] = (uint32_t)scales[(size_t)r * G + g] | ((uint32_t)biases[(size_t)r * G + g] << 16);
  }
  PGD_HIP(hipMemcpyAsync(m.p0, codes.data(), codes.size(), hipMemcpyHostToDevice, s));
  PGD_HIP(hipMemcpyAsync(m.p1, sb.data(), sb.size() * 4, hipMemcpyHostToDevice, s));
  PGD_HIP(hipStreamSynchronize(s));
}

void qmat_upload_kq(QMat& m, const uint8_t* blocks, hipStream_t s) {
  size_t nb = (size_t)m.n_out * m.nsb;
  if (m.fmt == FMT_Q4K) {
    // GGML blocks (row-major, 144 B each) -> tiled planes (same bytes, permuted)
    const size_t tiles = ((size_t)m.n_out + 31) / 32;
    std::vector<uint8_t> qs(tiles * 4 * m.nsb * 1024, 0), hdr(tiles * m.nsb * 512, 0);
    for (int r = 0; r < m.n_out; ++r)
      for (int sb = 0; sb < m.nsb; ++sb) {
        const uint8_t* b = blocks + ((size_t)r * m.nsb + sb) * 144;
        std::copy(b, b + 16, hdr.data() + q4k_hdr_off(r, sb, m.nsb));
        for (int g = 0; g < 4; ++g)
          std::copy(b + 16 + 32 * g, b + 48 + 32 * g, qs.data() + q4k_qs_off(r, sb * 128 + 32 * g, m.nsb));
      }
    PGD_HIP(hipMemcpyAsync(m.p0, qs.data(), qs.size(), hipMemcpyHostToDevice, s));
    PGD_HIP(hipMemcpyAsync(m.p1, hdr.data(), hdr.size(), hipMemcpyHostToDevice, s));
    PGD_HIP(hipStreamSynchronize(s));
  } else if (m.fmt == FMT_Q6K) {
    // GGML blocks (row-major, 210 B each) -> tiled planes (same bytes, permuted)
    const size_t tiles = ((size_t)m.n_out + 31) / 32;
    const int nsb = m.nsb;
    std::vector<uint8_t> ql(tiles * nsb * 4096, 0), qh(tiles * nsb * 2048, 0), sc(tiles * nsb * 512, 0);
    std::vector<uint16_t> d(tiles * nsb * 32, 0);
    for (int r = 0; r < m.n_out; ++r)
      for (int sb = 0; sb < nsb; ++sb) {
        const uint8_t* b = blocks + ((size_t)r * nsb + sb) * 210;
        for (int i = 0; i < 128; i += 4) std::copy(b + i, b + i + 4, ql.data() + q6k_ql_off(r, sb * 128 + i, nsb));
        for (int i = 0; i < 64; i += 4)
          std::copy(b + 128 + i, b + 132 + i, qh.data() + q6k_qh_off(r, sb * 64 + i, nsb));
        for (int i = 0; i < 16; ++i) sc[q6k_sc_off(r, sb * 16 + i, nsb)] = b[192 + i];
        d[q6k_d_off(r, sb, nsb)] = (uint16_t)(b[208] | (b[209] << 8));
      }
    PGD_HIP(hipMemcpyAsync(m.p0, ql.data(), ql.size(), hipMemcpyHostToDevice, s));
    PGD_HIP(hipMemcpyAsync(m.p1, qh.data(), qh.size(), hipMemcpyHostToDevice, s));
    PGD_HIP(hipMemcpyAsync(m.p2, sc.data(), sc.size(), hipMemcpyHostToDevice, s));
    PGD_HIP(hipMemcpyAsync(m.p3, d.data(), d.size() * 2, hipMemcpyHostToDevice, s));
    PGD_HIP(hipStreamSynchronize(s));
  } else if (m.fmt == FMT_Q8_0 || m.fmt == FMT_Q5_0) {
    // GGML blocks (row-major) -> row-major planes: quants, (Q5_0: high bits), scales
    const bool q8 = m.fmt == FMT_Q8_0;
    const size_t nbk = (size_t)m.n_out * m.nsb, qb = q8 ? 32 : 16;
    std::vector<uint8_t> q(nbk * qb), qh(q8 ? 0 : nbk * 4);
    std::vector<uint16_t> d(nbk);
    for (size_t i = 0; i < nbk; ++i) {
      const uint8_t* b = blocks + i * (q8 ? kQ8_0Bytes : kQ5_0Bytes);
      d[i] = (uint16_t)(b[0] | (b[1] << 8));
      if (q8) {
        std::copy(b + 2, b + 34, q.data() + i * 32);
      } else {
        std::copy(b + 2, b + 6, qh.data() + i * 4);
        std::copy(b + 6, b + 22, q.data() + i * 16);
      }
    }
    PGD_HIP(hipMemcpyAsync(m.p0, q.data(), q.size(), hipMemcpyHostToDevice, s));
    if (q8) {
      PGD_HIP(hipMemcpyAsync(m.p1, d.data(), d.size() * 2, hipMemcpyHostToDevice, s));
    } else {
      PGD_HIP(hipMemcpyAsync(m.p1, qh.data(), qh.size(), hipMemcpyHostToDevice, s));
      PGD_HIP(hipMemcpyAsync(m.p2, d.data(), d.size() * 2, hipMemcpyHostToDevice, s));
    }
    PGD_HIP(hipStreamSynchronize(s));
  } else {
    throw Error{kErrFormat, "block upload on an A8 matrix"};
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
  run_fmt(m, a, nrows, x_f16, res ? EPI_RES : EPI_STORE, s);
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
  run_fmt(gate, a, nrows, 0, EPI_SWIGLU, s);
}

void qmat_gemv_q8act(const QMat& m, const float* x, int ldx, int nrows, float* y, int ldy, const float* res, int ldres,
                     hipStream_t s) {
  PGD_CHECK(nrows >= 0 && ldx >= m.n_in, kErrShape, "gemv rows / ldx");
  if (nrows == 0) return;
  GemvArgs a = make_args(m);
  a.x = x;
  a.ldx = ldx;
  a.y = y;
  a.ldy = ldy;
  a.res = res;
  a.ldres = ldres;
  run_q8act(m.fmt, a, nrows, res ? EPI_RES : EPI_STORE, s);
}

bool qmat_q8act_pairable(const QMat& a, const QMat& b) {
  return a.n_in == b.n_in && gemv::q8act_pair_ok(a.fmt, b.fmt);
}

void qmat_gemv_q8act_pair(const QMat& a, float* ya, const QMat& b, float* yb, const float* x, int ldx, int nrows,
                          int ldy, hipStream_t s) {
  PGD_CHECK(nrows >= 0 && ldx >= a.n_in && ldy >= a.n_out && ldy >= b.n_out, kErrShape, "gemv rows / strides");
  if (nrows == 0) return;
  GemvArgs ga = make_args(a), gb = make_args(b);
  ga.x = gb.x = x;
  ga.ldx = gb.ldx = ldx;
  ga.y = ya;
  gb.y = yb;
  ga.ldy = gb.ldy = ldy;
  run_q8act_pair(a.fmt, ga, b.fmt, gb, nrows, s);
}

void qmat_gemv_swiglu_q8act(const QMat& gate, const QMat& up, const float* x, int ldx, int nrows, float* mid, int ldm,
                            hipStream_t s) {
  PGD_CHECK(gate.fmt == up.fmt && gate.n_out == up.n_out && gate.n_in == up.n_in, kErrShape,
            "swiglu gate/up shapes differ");
  PGD_CHECK(nrows >= 0 && ldx >= gate.n_in, kErrShape, "gemv rows / ldx");
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
  run_q8act(gate.fmt, a, nrows, EPI_SWIGLU, s);
}

void qmat_gemv_a8(const QMat& m, const A8Act& act, float* y, int ldy, const float* res, int ldres, hipStream_t s) {
  PGD_CHECK(m.fmt == FMT_A8, kErrFormat, "prepared activations feed A8 matrices");
  if (act.rows <= 0) return;
  GemvArgs a = make_args(m);
  a.y = y;
  a.ldy = ldy;
  a.res = res;
  a.ldres = ldres;
  run_a8_mma(a, act, res ? EPI_RES : EPI_STORE, s);
}

size_t qmat_gemv_a8_scratch(const QMat& m, int rows, bool res) {
  PGD_CHECK(m.fmt == FMT_A8, kErrFormat, "prepared activations feed A8 matrices");
  return rows > 0 ? a8_scratch_need(make_args(m), rows, res ? EPI_RES : EPI_STORE) : 0;
}

void qmat_gemv_a8_conv(const QMat& m, const A8Act& act, float* y, int ldy, const float* conv_w,
                       float* const* state_base, size_t state_off, int conv_n, int kernel, float* conv_out, int ldc,
                       hipStream_t s) {
  PGD_CHECK(m.fmt == FMT_A8, kErrFormat, "prepared activations feed A8 matrices");
  PGD_CHECK(conv_n <= m.n_out && kernel >= 1 && kernel <= 8 && conv_w && state_base && conv_out, kErrShape,
            "conv epilogue arguments");
  // the split-K kernels' epilogue or the range reduction holds the outputs;
  // every row must be its sequence's only token (row r on state r)
  PGD_CHECK(act.rows >= 1, kErrShape, "the conv epilogue needs rows");
  GemvArgs a = make_args(m);
  a.y = y;
  a.ldy = ldy;
  PGD_CHECK(!a8_sk_wanted(a, EPI_STORE), kErrShape, "the conv epilogue needs the split-K kernel");
  a.cw = conv_w;
  a.cbase = state_base;
  a.coff = state_off;
  a.cout = conv_out;
  a.ldc = ldc;
  a.conv_n = conv_n;
  a.conv_k = kernel;
  run_a8_mma(a, act, EPI_STORE, s);
}

A8Act qmat_gemv_a8_res_norm(const QMat& m, const A8Act& act, float* y, int ldy, const float* nw, float eps,
                            void* nbuf, hipStream_t s) {
  PGD_CHECK(m.fmt == FMT_A8, kErrFormat, "prepared activations feed A8 matrices");
  PGD_CHECK(m.n_out % 32 == 0 && ldy % 4 == 0, kErrShape, "norm-emitting residual GEMV: width");
  A8Act out = a8_act_view(nbuf, act.rows, m.n_out);
  out.rss = a8_act_rss(nbuf, act.rows, m.n_out);
  out.eps = eps;
  if (act.rows <= 0) return out;
  GemvArgs a = make_args(m);
  a.y = y;
  a.ldy = ldy;
  a.res = y;
  a.ldres = ldy;
  a.nact = a8_act_dst(out);
  a.nw = nw;
  a.nrss = const_cast<float*>(out.rss);
  run_a8_mma(a, act, EPI_RES, s);
  return out;
}

void qmat_gemv_a8_swiglu(const QMat& gate, const QMat& up, const A8Act& act, float* mid, int ldm, hipStream_t s,
                         const A8Act* mid_act) {
  PGD_CHECK(gate.fmt == FMT_A8 && up.fmt == FMT_A8 && gate.n_out == up.n_out && gate.n_in == up.n_in, kErrShape,
            "swiglu gate/up shapes differ");
  PGD_CHECK(mid || mid_act, kErrArg, "swiglu needs an output");
  if (act.rows <= 0) return;
  GemvArgs a = make_args(gate);
  a.u0 = up.p0;
  a.u1 = up.p1;
  a.y = mid;
  a.ldy = ldm;
  if (mid_act) {
    PGD_CHECK(gate.n_out % 64 == 0 && mid_act->K == gate.n_out && mid_act->rows == act.rows, kErrShape,
              "prepared SwiGLU output needs n_out % 64 == 0 and matching rows");
    a.oact = a8_act_dst(*mid_act);
  }
  run_a8_mma(a, act, EPI_SWIGLU, s);
}

void qmat_synth(QMat& m, uint64_t seed, uint64_t key, float std, hipStream_t s) {
  uint64_t stream = synth_stream(seed, key);
  if (m.fmt == FMT_A8) {
    qmat_synth_rows(m, 0, m.n_out, seed, key, std, s);
    return;
  } else if (m.fmt == FMT_Q4K) {
    size_t n = (size_t)m.n_out * m.nsb;
    hipLaunchKernelGGL(synth_q4k_kernel, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, s, m.p0,
                       reinterpret_cast<uint4*>(m.p1), m.n_out, m.n_in, m.nsb, stream, std, 0);
  } else if (m.fmt == FMT_Q6K) {
    size_t n = (size_t)m.n_out * m.nsb;
    hipLaunchKernelGGL(synth_q6k_kernel, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, s, m.p0, m.p1,
                       reinterpret_cast<int8_t*>(m.p2), reinterpret_cast<uint16_t*>(m.p3), m.n_out, m.n_in, m.nsb,
                       stream, std, 0);
  } else {
    throw Error{kErrFormat, "no synthetic generator for this format"};
  }
  PGD_HIP(hipGetLastError());
}

void qmat_synth_rows(QMat& m, int row0, int rows, uint64_t seed, uint64_t key, float std, hipStream_t s) {
  PGD_CHECK(row0 >= 0 && rows >= 0 && row0 + rows <= m.n_out, kErrShape, "synth row window");
  if (!rows) return;
  if (m.fmt == FMT_Q4K || m.fmt == FMT_Q6K) {
    const size_t n = (size_t)rows * m.nsb;
    const uint64_t stream = synth_stream(seed, key);
    if (m.fmt == FMT_Q4K)
      hipLaunchKernelGGL(synth_q4k_kernel, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, s, m.p0,
                         reinterpret_cast<uint4*>(m.p1), rows, m.n_in, m.nsb, stream, std, row0);
    else
      hipLaunchKernelGGL(synth_q6k_kernel, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, s, m.p0, m.p1,
                         reinterpret_cast<int8_t*>(m.p2), reinterpret_cast<uint16_t*>(m.p3), rows, m.n_in, m.nsb,
                         stream, std, row0);
    PGD_HIP(hipGetLastError());
    return;
  }
  PGD_CHECK(m.fmt == FMT_A8, kErrFormat, "no row-window synthesis for this format");
  size_t n = (size_t)rows * (m.n_in / 64);
  hipLaunchKernelGGL(synth_a8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, m.p0,
                     reinterpret_cast<uint32_t*>(m.p1), row0, rows, m.n_in, synth_stream(seed, key), std);
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
