// gemv_q8.hip — GGML-format GEMV with the arithmetic of candle's CPU
// quantized matmul (the reference's CPU path keeps QMatMul for the Qwen2 GGUF
// weights, pagoda-hf/src/qwen2_gguf.rs:280-289): every activation row is
// quantized to the weight type's vec_dot_type and each output is an integer
// block dot scaled in f32.
//
//   Q4_K, Q6_K  x  Q8_K  (256-element blocks: f32 d, 256 i8, 16 i16 sums)
//   Q8_0, Q5_0  x  Q8_0  (32-element blocks: f16 d, 32 i8)
//
// Activation quantization (BlockQ8K / BlockQ8_0 ::from_float): Q8_K takes the
// first element of largest magnitude as max, iscale = -128 / max,
// q = min(127, round(iscale x)) (round half away from zero), d = 1 / iscale,
// and the sums of each 16 q; Q8_0 takes d = amax / 127, q = round(x / d)
// with d rounded to f16. Every workgroup quantizes the launch's rows into LDS
// itself (no separate launch); all of them compute the same bytes.
//
// Block dots: integer products through v_dot4 (exact), per weight block
//   Q4_K: d_w d_x sum_j sc_j dot_j - dmin_w d_x sum_j m_j bsum_j
//   Q6_K: d_w d_x sum_j sc_j (dot_j(q) - 32 bsum_j)       (q = 6-bit code)
//   Q8_0: sumi d_w d_x;  Q5_0: (dot(q) - 16 sum(x_q)) d_w d_x   (q = 5-bit code)
// The float arithmetic is GGML's scalar one, term for term and in its order,
// so every output is bit-equal to the CPU restatement: the integer products
// of a 256-block are kept in eight residue classes (element index mod 8,
// GGML's aux32[8] lanes), each scaled by d = d_w d_x and added into its own
// running sum block after block, the Q4_K min terms into a ninth, and the
// eight sums are added at the end; 32-blocks add (sumi d_w) d_x block after
// block. Waves compute their blocks' terms in parallel (exact integers, one
// rounding per product) and leave them in LDS; one lane per output then adds
// them in block order. The per-row arithmetic does not depend on the number
// of rows, so batched rows are bitwise equal to single-row launches.
//
// Work split: one workgroup of NW waves (4 or 8, from the number of K
// blocks) per 32-row tile of the weight matrix; wave w takes K blocks w,
// w + NW, ... (256-element super-blocks, or 32-weight blocks). Weights are
// read once per launch of up to RB activation rows.
#include <type_traits>

#include "common.h"
#include "gemv_impl.h"
#include "quant.h"

namespace pgd {
namespace gemv {

namespace {


typedef uint32_t u2v __attribute__((ext_vector_type(2)));

__device__ inline int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// activations in LDS: q [RB][Kp] i8 | d [RB][nb] f32 | sums [RB][nb][SUMS] i32,
// then the block terms [NM][RB][nb][32 outputs][NT] f32 (NT: 9 for Q4_K, the
// eight residue classes and the min term; 8 for Q6_K; 1 for 32-blocks)
template <int FMT, int RB, int NW>
struct ActLds {
  static constexpr bool K256 = FMT == FMT_Q4K || FMT == FMT_Q6K;
  static constexpr int BLK = K256 ? 256 : 32;
  static constexpr int SUMS = K256 ? 16 : 1;
  static constexpr int NT = FMT == FMT_Q4K ? 9 : FMT == FMT_Q6K ? 8 : 1;
  int Kp, nb;
  int8_t* q;
  float* d;
  int* s;
  float* t;
  __host__ __device__ static size_t act_bytes(int nbh) {
    return ((((size_t)RB * nbh * BLK + 15) & ~(size_t)15) + (size_t)RB * nbh * 4 + (size_t)RB * nbh * SUMS * 4 + 15) &
           ~(size_t)15;
  }
  __device__ ActLds(char* base, int n_in) {
    nb = (n_in + BLK - 1) / BLK;
    Kp = nb * BLK;
    q = reinterpret_cast<int8_t*>(base);
    d = reinterpret_cast<float*>(base + (((size_t)RB * Kp + 15) & ~(size_t)15));
    s = reinterpret_cast<int*>(d + RB * nb);
    t = reinterpret_cast<float*>(base + act_bytes(nb));
  }
  // term slot of matrix m, row r, block b, tile output n
  __device__ float* term(int m, int r, int b, int n) const { return t + ((((size_t)m * RB + r) * nb + b) * 32 + n) * NT; }
  static size_t bytes(int n_in, int nm) {
    const int nbh = (n_in + BLK - 1) / BLK;
    return act_bytes(nbh) + (size_t)nm * RB * nbh * 32 * NT * 4;
  }
};

// Quantize rows [0, rows) of x (the launch's chunk) into LDS; the whole
// workgroup calls it.
template <int FMT, int RB, int NW>
__device__ void quantize_rows(const float* __restrict__ x, int ldx, int rows, int n_in, ActLds<FMT, RB, NW>& L) {
  const int tid = threadIdx.x;
  if constexpr (ActLds<FMT, RB, NW>::K256) {
    // eight lanes per 256-element block, 32 consecutive elements each
    const int s = tid & 7;
    const int units = rows * L.nb;
    for (int u0 = 0; u0 < units; u0 += 8 * NW) {
      const int u = u0 + (tid >> 3);
      const bool live = u < units;
      const int r = live ? u / L.nb : 0, b = live ? u % L.nb : 0;
      const int e0 = b * 256 + s * 32;
      float v[32];
      float amax = 0.0f, mx = 0.0f;
      int idx = 0x7fffffff;
      const float* xr = x + (size_t)r * ldx + e0;
      if (live && e0 + 32 <= n_in && (((uintptr_t)xr) & 15) == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float4 t = reinterpret_cast<const float4*>(xr)[i];
          v[4 * i] = t.x;
          v[4 * i + 1] = t.y;
          v[4 * i + 2] = t.z;
          v[4 * i + 3] = t.w;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = (live && e0 + i < n_in) ? xr[i] : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int e = e0 + i;
        const float ax = fabsf(v[i]);
        if (ax > amax) {
          amax = ax;
          mx = v[i];
          idx = e;
        }
      }
      // the first element of largest magnitude over the block's 8 lanes
#pragma unroll
      for (int o = 1; o < 8; o <<= 1) {
        const float oa = __shfl_xor(amax, o, 64), om = __shfl_xor(mx, o, 64);
        const int oi = __shfl_xor(idx, o, 64);
        if (oa > amax || (oa == amax && oi < idx)) {
          amax = oa;
          mx = om;
          idx = oi;
        }
      }
      if (live) {
        int8_t* q = L.q + (size_t)r * L.Kp + e0;
        int* bs = L.s + (r * L.nb + b) * 16 + 2 * s;
        if (amax == 0.0f) {
#pragma unroll
          for (int i = 0; i < 32; ++i) q[i] = 0;
          bs[0] = bs[1] = 0;
          if (s == 0) L.d[r * L.nb + b] = 0.0f;
        } else {
          const float iscale = -128.0f / mx;
          int s0 = 0, s1 = 0;
#pragma unroll
          for (int i = 0; i < 32; ++i) {
            const float t = roundf(iscale * v[i]);
            const int qi = (int)(t < 127.0f ? t : 127.0f);
            q[i] = (int8_t)qi;
            if (i < 16) s0 += qi;
            else s1 += qi;
          }
          bs[0] = s0;
          bs[1] = s1;
          if (s == 0) L.d[r * L.nb + b] = 1.0f / iscale;
        }
      }
    }
  } else {
    // one lane per 32-element block
    const int units = rows * L.nb;
    for (int u = tid; u < units; u += blockDim.x) {
      const int r = u / L.nb, b = u % L.nb;
      const float* xr = x + (size_t)r * ldx + b * 32;
      float v[32];
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        v[i] = xr[i];
        amax = fmaxf(amax, fabsf(v[i]));
      }
      const float d = amax / 127.0f;
      const float id = d != 0.0f ? 1.0f / d : 0.0f;
      int8_t* q = L.q + (size_t)r * L.Kp + b * 32;
      int sum = 0;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int qi = (int)roundf(v[i] * id);
        q[i] = (int8_t)qi;
        sum += qi;
      }
      L.s[r * L.nb + b] = sum;
      L.d[r * L.nb + b] = (float)(_Float16)d;  // the f16 d of block_q8_0
    }
  }
}

// ---- per-format block terms of one wave over its blocks -------------------

// byte b of a dword, alone in its byte lane (for products of one element)
__device__ inline uint32_t byte_lane(uint32_t v, int b) { return v & (0xFFu << (8 * b)); }

// Q4_K: lane l = output row l >> 1, half h = l & 1 of each 32-byte run. The
// lane's bytes 16 h + 4 i + k of a run hold elements of residue 4 (i & 1) + k
// (mod 8) in both nibbles.
template <int RB, int NW, int NM>
__device__ void dots_q4k(const GemvArgs& a, int tile, int rows, const ActLds<FMT_Q4K, RB, NW>& L) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int jr = lane >> 1, h = lane & 1, row = tile * 32 + jr;
  for (int sb = w; sb < a.nsb; sb += NW) {
    const int nj = min(4, (a.n_in - sb * 256 + 63) / 64);  // 64-element chunks present
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const uint8_t* p0 = m ? a.u0 : a.p0;
      const uint8_t* p1 = m ? a.u1 : a.p1;
      const uint4 hdr = *reinterpret_cast<const uint4*>(p1 + q4k_hdr_off(row, sb, a.nsb));
      uint4 wq[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        wq[j] = j < nj ? *reinterpret_cast<const uint4*>(p0 + q4k_qs_off(row, 32 * (4 * sb + j) + 16 * h, a.nsb))
                       : make_uint4(0, 0, 0, 0);
      // 6-bit scales and mins of the 8 sub-blocks
      const uint32_t sw[3] = {hdr.y, hdr.z, hdr.w};
      auto byte = [&](int i) { return (sw[i >> 2] >> (8 * (i & 3))) & 255u; };
      int sc[8], mn[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (k < 4) {
          sc[k] = (int)(byte(k) & 63u);
          mn[k] = (int)(byte(k + 4) & 63u);
        } else {
          sc[k] = (int)((byte(k + 4) & 0xFu) | ((byte(k - 4) >> 6) << 4));
          mn[k] = (int)((byte(k + 4) >> 4) | ((byte(k) >> 6) << 4));
        }
      }
      const float dw = f16_to_f32(hdr.x & 0xffffu), dmin = f16_to_f32(hdr.x >> 16);
      for (int r = 0; r < rows; ++r) {
        const int8_t* xq = L.q + (size_t)r * L.Kp + sb * 256;
        int aux[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) aux[l] = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (j >= nj) break;
          const uint4 xl = *reinterpret_cast<const uint4*>(xq + 64 * j + 16 * h);
          const uint4 xh = *reinterpret_cast<const uint4*>(xq + 64 * j + 32 + 16 * h);
          const uint32_t qw[4] = {wq[j].x, wq[j].y, wq[j].z, wq[j].w};
          const uint32_t lw[4] = {xl.x, xl.y, xl.z, xl.w}, hw[4] = {xh.x, xh.y, xh.z, xh.w};
          int tl[8], th[8];
#pragma unroll
          for (int l = 0; l < 8; ++l) tl[l] = th[l] = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t lo = qw[i] & 0x0F0F0F0Fu, hi = (qw[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              tl[4 * (i & 1) + k] = dot4(byte_lane(lo, k), lw[i], tl[4 * (i & 1) + k]);
              th[4 * (i & 1) + k] = dot4(byte_lane(hi, k), hw[i], th[4 * (i & 1) + k]);
            }
          }
#pragma unroll
          for (int l = 0; l < 8; ++l) aux[l] += sc[2 * j] * tl[l] + sc[2 * j + 1] * th[l];
        }
#pragma unroll
        for (int l = 0; l < 8; ++l) aux[l] += __shfl_xor(aux[l], 1, 64);
        const int* bs = L.s + (r * L.nb + sb) * 16;
        int msum = 0;
#pragma unroll
        for (int k = 0; k < 16; ++k) msum += bs[k] * mn[k / 2];
        const float d8 = L.d[r * L.nb + sb];
        const float d = dw * d8, dm = dmin * d8;
        float* t = L.term(m, r, sb, jr);
#pragma unroll
        for (int c = 0; c < 4; ++c) t[4 * h + c] = d * (float)aux[4 * h + c];
        if (h == 0) t[8] = dm * (float)msum;
      }
    }
  }
}

// Q6_K: lane l = dword k = l >> 4 of row 16 hh + (l & 15), for row halves hh
// 0 and 1. The lane's elements all have residue 4 (k & 1) + c, c = 0..3.
template <int RB, int NW, int NM>
__device__ void dots_q6k(const GemvArgs& a, int tile, int rows, const ActLds<FMT_Q6K, RB, NW>& L) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int k = lane >> 4, jr = lane & 15;
  for (int sb = w; sb < a.nsb; sb += NW) {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const uint8_t* p0 = m ? a.u0 : a.p0;
      const uint8_t* p1 = m ? a.u1 : a.p1;
      const uint8_t* p2 = m ? a.u2 : a.p2;
      const uint8_t* p3 = m ? a.u3 : a.p3;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int row = tile * 32 + 16 * hh + jr;
        const float dw = f16_to_f32(reinterpret_cast<const uint16_t*>(p3)[q6k_d_off(row, sb, a.nsb)]);
        // codes - 32 (signed bytes) of elements 4k + 16 mm + (0..3) of half u,
        // mm = 0..7, and the sub-block scales
        uint32_t v[2][8];
        int sc[2][8];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const bool live = sb * 256 + 128 * u < a.n_in;
          const uint4 ql = live ? *reinterpret_cast<const uint4*>(p0 + q6k_ql_off(row, 64 * (2 * sb + u) + 4 * k, a.nsb))
                                : make_uint4(0, 0, 0, 0);
          const u2v qh = live ? *reinterpret_cast<const u2v*>(p1 + q6k_qh_off(row, 32 * (2 * sb + u) + 4 * k, a.nsb))
                              : (u2v){0u, 0u};
          const u2v scw = live ? *reinterpret_cast<const u2v*>(p2 + q6k_sc_off(row, 16 * sb + 8 * u, a.nsb))
                               : (u2v){0u, 0u};
          const uint32_t qlw[4] = {ql.x, ql.y, ql.z, ql.w};
#pragma unroll
          for (int mm = 0; mm < 8; ++mm) {
            const uint32_t lo = (qlw[mm & 3] >> (mm >= 4 ? 4 : 0)) & 0x0F0F0F0Fu;
            const uint32_t hq = (mm & 1) ? qh.y : qh.x;
            const uint32_t hb = (hq >> (2 * (mm >> 1))) & 0x03030303u;
            v[u][mm] = (((lo | (hb << 4)) | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
            sc[u][mm] = (int)(int8_t)(((mm < 4 ? scw.x : scw.y) >> (8 * (mm & 3))) & 255u);
          }
        }
        const int nu = sb * 256 + 128 < a.n_in ? 2 : 1;
        for (int r = 0; r < rows; ++r) {
          int iw[4] = {0, 0, 0, 0};
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            if (u >= nu) break;
            const int8_t* xq = L.q + (size_t)r * L.Kp + sb * 256 + 128 * u + 4 * k;
#pragma unroll
            for (int mm = 0; mm < 8; ++mm) {
              const uint32_t xw = *reinterpret_cast<const uint32_t*>(xq + 16 * mm);
#pragma unroll
              for (int c = 0; c < 4; ++c) iw[c] += sc[u][mm] * dot4(byte_lane(v[u][mm], c), xw, 0);
            }
          }
          // dword lanes k and k ^ 2 hold the same residues
#pragma unroll
          for (int c = 0; c < 4; ++c) iw[c] += __shfl_xor(iw[c], 32, 64);
          if (k < 2) {
            const float d = dw * L.d[r * L.nb + sb];
            float* t = L.term(m, r, sb, 16 * hh + jr);
#pragma unroll
            for (int c = 0; c < 4; ++c) t[4 * k + c] = d * (float)iw[c];
          }
        }
      }
    }
  }
}

// Q8_0 / Q5_0 (row-major planes, no row padding): lane l = output row l >> 1,
// half h = l & 1 of each block.
template <int FMT, int RB, int NW, int NM>
__device__ void dots_q32(const GemvArgs& a, int tile, int rows, const ActLds<FMT, RB, NW>& L) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int h = lane & 1;
  const int row = min(tile * 32 + (lane >> 1), a.n_out - 1);
  const int nb = a.n_in / 32;
  for (int b = w; b < nb; b += NW) {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const uint8_t* p0 = m ? a.u0 : a.p0;
      const uint8_t* p1 = m ? a.u1 : a.p1;
      const uint8_t* p2 = m ? a.u2 : a.p2;
      uint32_t v[4];
      float dw;
      if constexpr (FMT == FMT_Q8_0) {
        const uint4 q = *reinterpret_cast<const uint4*>(p0 + (size_t)row * a.n_in + 32 * b + 16 * h);
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
        dw = f16_to_f32(reinterpret_cast<const uint16_t*>(p1)[(size_t)row * nb + b]);
      } else {
        // bytes 8h..8h+7 of the block's 16: low nibbles are weights 8h + i,
        // high nibbles weights 16 + 8h + i; qh bit j is weight j's fifth bit
        const u2v q = *reinterpret_cast<const u2v*>(p0 + (size_t)row * (a.n_in / 2) + 16 * b + 8 * h);
        const uint32_t qh = reinterpret_cast<const uint32_t*>(p1)[(size_t)row * nb + b];
        auto spread = [](uint32_t bits4) {  // 4 bits -> bit 4 of 4 bytes
          return ((bits4 & 1u) | ((bits4 & 2u) << 7) | ((bits4 & 4u) << 14) | ((bits4 & 8u) << 21)) << 4;
        };
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const uint32_t wd = i ? q.y : q.x;
          const int j0 = 8 * h + 4 * i;
          v[i] = (wd & 0x0F0F0F0Fu) | spread((qh >> j0) & 15u);
          v[2 + i] = ((wd >> 4) & 0x0F0F0F0Fu) | spread((qh >> (16 + j0)) & 15u);
        }
        dw = f16_to_f32(reinterpret_cast<const uint16_t*>(p2)[(size_t)row * nb + b]);
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        if (r >= rows) break;
        const int8_t* xq = L.q + (size_t)r * L.Kp + 32 * b;
        int sumi = 0;
        if constexpr (FMT == FMT_Q8_0) {
          const uint4 xv = *reinterpret_cast<const uint4*>(xq + 16 * h);
          sumi = dot4(v[0], xv.x, sumi);
          sumi = dot4(v[1], xv.y, sumi);
          sumi = dot4(v[2], xv.z, sumi);
          sumi = dot4(v[3], xv.w, sumi);
          sumi += __shfl_xor(sumi, 1, 64);
        } else {
          const u2v xl = *reinterpret_cast<const u2v*>(xq + 8 * h);
          const u2v xh = *reinterpret_cast<const u2v*>(xq + 16 + 8 * h);
          sumi = dot4(v[0], xl.x, sumi);
          sumi = dot4(v[1], xl.y, sumi);
          sumi = dot4(v[2], xh.x, sumi);
          sumi = dot4(v[3], xh.y, sumi);
          sumi += __shfl_xor(sumi, 1, 64);
          sumi -= 16 * L.s[r * L.nb + b];
        }
        if (h == 0) L.term(m, r, b, lane >> 1)[0] = (float)sumi * dw * L.d[r * L.nb + b];
      }
    }
  }
}

// Touch one dword of every 128-byte line of [base, base + bytes) across the
// workgroup: the tile's weights are on their way into the cache while the
// activations are quantized (the loads' values only feed `sink`).
__device__ inline void touch(const uint8_t* base, size_t bytes, int nthreads, uint32_t& sink) {
  for (size_t off = (size_t)threadIdx.x * 128; off + 4 <= bytes; off += (size_t)nthreads * 128)
    sink ^= *reinterpret_cast<const uint32_t*>(base + off);
}

template <int FMT>
__device__ inline void prefetch_tile(const GemvArgs& a, bool second, int tile, int nthreads, uint32_t& sink) {
  const uint8_t* p0 = second ? a.u0 : a.p0;
  const uint8_t* p1 = second ? a.u1 : a.p1;
  const uint8_t* p2 = second ? a.u2 : a.p2;
  const uint8_t* p3 = second ? a.u3 : a.p3;
  const size_t nsb = (size_t)a.nsb, t = (size_t)tile;
  if constexpr (FMT == FMT_Q4K) {
    touch(p0 + t * 4 * nsb * 1024, 4 * nsb * 1024, nthreads, sink);
    touch(p1 + t * nsb * 512, nsb * 512, nthreads, sink);
  } else if constexpr (FMT == FMT_Q6K) {
    touch(p0 + t * 2 * nsb * 2048, 2 * nsb * 2048, nthreads, sink);
    touch(p1 + t * 2 * nsb * 1024, 2 * nsb * 1024, nthreads, sink);
    touch(p2 + t * 2 * nsb * 256, 2 * nsb * 256, nthreads, sink);
    touch(p3 + t * nsb * 64, nsb * 64, nthreads, sink);
  } else {
    // row-major planes: the tile's rows
    const size_t r0 = t * 32, nr = (size_t)min(32, a.n_out - tile * 32), nb = (size_t)(a.n_in / 32);
    if constexpr (FMT == FMT_Q8_0) {
      touch(p0 + r0 * a.n_in, nr * a.n_in, nthreads, sink);
      touch(p1 + r0 * nb * 2, nr * nb * 2, nthreads, sink);
    } else {
      touch(p0 + r0 * (a.n_in / 2), nr * (a.n_in / 2), nthreads, sink);
      touch(p1 + r0 * nb * 4, nr * nb * 4, nthreads, sink);
      touch(p2 + r0 * nb * 2, nr * nb * 2, nthreads, sink);
    }
  }
}

// One 32-row weight tile of a launch: block terms over the activations
// already quantized in L, then one lane per (row, output) adds them in block
// order (GGML's scalar sums) and applies the epilogue.
template <int FMT, int RB, int NW, int EPI>
__device__ void q8_tile(const GemvArgs& a, int tile, int rows, const ActLds<FMT, RB, NW>& L) {
  constexpr int NM = EPI == EPI_SWIGLU ? 2 : 1;
  if constexpr (FMT == FMT_Q4K) dots_q4k<RB, NW, NM>(a, tile, rows, L);
  else if constexpr (FMT == FMT_Q6K) dots_q6k<RB, NW, NM>(a, tile, rows, L);
  else dots_q32<FMT, RB, NW, NM>(a, tile, rows, L);
  __syncthreads();
  for (int t = threadIdx.x; t < rows * 32; t += blockDim.x) {
    const int r = t >> 5, j = t & 31, n = tile * 32 + j;
    if (n >= a.n_out) continue;
    float v[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      if constexpr (FMT == FMT_Q4K || FMT == FMT_Q6K) {
        // vec_dot_q4_K_q8_K / vec_dot_q6_K_q8_K: sums[8] over the blocks, the
        // min terms subtracted from sumf block by block, then sumf += sums[l]
        float sums[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, sumf = 0.0f;
        for (int b = 0; b < L.nb; ++b) {
          const float* tb = L.term(m, r, b, j);
#pragma unroll
          for (int l = 0; l < 8; ++l) sums[l] += tb[l];
          if constexpr (FMT == FMT_Q4K) sumf -= tb[8];
        }
#pragma unroll
        for (int l = 0; l < 8; ++l) sumf += sums[l];
        v[m] = sumf;
      } else {
        float sumf = 0.0f;
        for (int b = 0; b < L.nb; ++b) sumf += L.term(m, r, b, j)[0];
        v[m] = sumf;
      }
    }
    const size_t o = (size_t)r * a.ldy + n;
    if constexpr (EPI == EPI_STORE) a.y[o] = v[0];
    if constexpr (EPI == EPI_RES) a.y[o] = a.res[(size_t)r * a.ldres + n] + v[0];
    if constexpr (EPI == EPI_SWIGLU) a.y[o] = silu_f(v[0]) * v[NM - 1];
  }
}

// the prefetch loads' values are never used: a store no launch can reach keeps them
__device__ inline void keep(const GemvArgs& a, int rows, uint32_t sink) {
  if (rows < 0 && sink == 0x9e3779b9u) a.y[0] = 0.0f;
}

// K blocks of a row in units of 256 weights (4 Q8_0 / Q5_0 blocks)
template <int FMT>
__host__ __device__ inline int k_blocks(const GemvArgs& a) {
  return (FMT == FMT_Q4K || FMT == FMT_Q6K) ? a.nsb : a.n_in / 128;
}

template <int FMT, int RB, int NW, int EPI>
__global__ __launch_bounds__(64 * NW) void q8_gemv_kernel(GemvArgs a, int rows) {
  extern __shared__ __attribute__((aligned(16))) char dsm[];
  // long rows (a wave walks several K blocks): the tile's later blocks are in
  // the cache by the time the wave reaches them (measured: the 4864-wide down
  // projection 13.2 -> 11.0 us for Q6_K; tiles of one block per wave lost)
  uint32_t sink = 0;
  if (NW == 8 && k_blocks<FMT>(a) > 8) {
    prefetch_tile<FMT>(a, false, blockIdx.x, 64 * NW, sink);
    if constexpr (EPI == EPI_SWIGLU) prefetch_tile<FMT>(a, true, blockIdx.x, 64 * NW, sink);
  }
  ActLds<FMT, RB, NW> L(dsm, a.n_in);
  quantize_rows<FMT, RB, NW>(reinterpret_cast<const float*>(a.x), a.ldx, rows, a.n_in, L);
  __syncthreads();
  q8_tile<FMT, RB, NW, EPI>(a, blockIdx.x, rows, L);
  keep(a, rows, sink);
}

// Two matrices of one input (the attention's stacked q|k and v, whose formats
// differ in Q4_K_M files) in one launch: both formats take the same
// activation type, quantized once per workgroup; workgroups [0, split) run
// tiles of a, the rest tiles of b. Every tile's arithmetic is that of its own
// single-matrix launch.
template <int FMT, int FMT2, int RB, int NW>
__global__ __launch_bounds__(64 * NW) void q8_pair_kernel(GemvArgs a, GemvArgs b, int split, int rows) {
  static_assert(ActLds<FMT, RB, NW>::K256 == ActLds<FMT2, RB, NW>::K256, "one activation type");
  extern __shared__ __attribute__((aligned(16))) char dsm[];
  const bool first = (int)blockIdx.x < split;
  uint32_t sink = 0;
  if (NW == 8 && k_blocks<FMT>(a) > 8) {
    if (first) prefetch_tile<FMT>(a, false, blockIdx.x, 64 * NW, sink);
    else prefetch_tile<FMT2>(b, false, blockIdx.x - split, 64 * NW, sink);
  }
  ActLds<FMT, RB, NW> L(dsm, a.n_in);
  quantize_rows<FMT, RB, NW>(reinterpret_cast<const float*>(a.x), a.ldx, rows, a.n_in, L);
  __syncthreads();
  if (first) {
    q8_tile<FMT, RB, NW, EPI_STORE>(a, blockIdx.x, rows, L);
  } else {
    const ActLds<FMT2, RB, NW> L2(dsm, a.n_in);
    q8_tile<FMT2, RB, NW, EPI_STORE>(b, blockIdx.x - split, rows, L2);
  }
  keep(a, rows, sink);
}

template <int FMT, int RB, int NW, int EPI>
void launch_q8(GemvArgs a, int nrows, hipStream_t s) {
  const size_t lds = ActLds<FMT, RB, NW>::bytes(a.n_in, EPI == EPI_SWIGLU ? 2 : 1);
  PGD_CHECK(lds <= 160 * 1024, kErrShape, "activation rows too wide for the quantized-activation GEMV");
  if (lds > 64 * 1024) {
    static bool set = false;  // per kernel instance: the largest LDS it may be launched with
    if (!set) {
      PGD_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&q8_gemv_kernel<FMT, RB, NW, EPI>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
      set = true;
    }
  }
  const int tiles = (a.n_out + 31) / 32;
  for (int r0 = 0; r0 < nrows; r0 += RB) {
    const int rows = min(RB, nrows - r0);
    hipLaunchKernelGGL((q8_gemv_kernel<FMT, RB, NW, EPI>), dim3(tiles), dim3(64 * NW), lds, s, a, rows);
    PGD_HIP(hipGetLastError());
    a.x = reinterpret_cast<const float*>(a.x) + (size_t)rows * a.ldx;
    a.y += (size_t)rows * a.ldy;
    if (a.res) a.res += (size_t)rows * a.ldres;
  }
}

// waves per workgroup from the K blocks of a row (the sums do not depend on
// it: every block's terms are added in block order by one lane)
template <int FMT, int RB, int EPI>
void launch_waves(const GemvArgs& a, int nrows, hipStream_t s) {
  if (k_blocks<FMT>(a) <= 4) return launch_q8<FMT, RB, 4, EPI>(a, nrows, s);
  launch_q8<FMT, RB, 8, EPI>(a, nrows, s);
}

// LDS of one launch of RB rows: the quantized rows, or the wave partials of
// the widest (16-wave) workgroup, whichever is larger
template <int FMT, int RB>
size_t lds_need(int n_in, int nm) {
  return ActLds<FMT, RB, 8>::bytes(n_in, nm);
}

// rows per launch: decode steps take 1..8; prefills 16 at a time (weights
// read once per 16 rows). Wide rows whose RB quantized rows do not fit the
// 160 KiB of LDS take fewer rows per launch (the per-row arithmetic does not
// depend on RB, so the results are the same).
template <int FMT, int EPI>
void launch_rows(const GemvArgs& a, int nrows, hipStream_t s) {
  const int nm = EPI == EPI_SWIGLU ? 2 : 1;
  const size_t cap = 160 * 1024;
  if (nrows > 8 && lds_need<FMT, 16>(a.n_in, nm) <= cap) return launch_waves<FMT, 16, EPI>(a, nrows, s);
  if (nrows > 4 && lds_need<FMT, 8>(a.n_in, nm) <= cap) return launch_waves<FMT, 8, EPI>(a, nrows, s);
  if (nrows > 1 && lds_need<FMT, 4>(a.n_in, nm) <= cap) return launch_waves<FMT, 4, EPI>(a, nrows, s);
  launch_waves<FMT, 1, EPI>(a, nrows, s);
}

template <int EPI>
void dispatch(int fmt, const GemvArgs& a, int nrows, hipStream_t s) {
  switch (fmt) {
    case FMT_Q4K: return launch_rows<FMT_Q4K, EPI>(a, nrows, s);
    case FMT_Q6K: return launch_rows<FMT_Q6K, EPI>(a, nrows, s);
    case FMT_Q8_0: return launch_rows<FMT_Q8_0, EPI>(a, nrows, s);
    case FMT_Q5_0: return launch_rows<FMT_Q5_0, EPI>(a, nrows, s);
  }
  throw Error{kErrFormat, "quantized-activation GEMV takes Q4_K, Q6_K, Q8_0 or Q5_0 matrices"};
}

template <int FMT, int FMT2, int RB, int NW>
void launch_pair_q8(GemvArgs a, GemvArgs b, int nrows, hipStream_t s) {
  const size_t l1 = ActLds<FMT, RB, NW>::bytes(a.n_in, 1), l2 = ActLds<FMT2, RB, NW>::bytes(a.n_in, 1);
  const size_t lds = l1 > l2 ? l1 : l2;
  PGD_CHECK(lds <= 160 * 1024, kErrShape, "activation rows too wide for the quantized-activation GEMV");
  if (lds > 64 * 1024) {
    static bool set = false;
    if (!set) {
      PGD_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&q8_pair_kernel<FMT, FMT2, RB, NW>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
      set = true;
    }
  }
  const int ta = (a.n_out + 31) / 32, tb = (b.n_out + 31) / 32;
  for (int r0 = 0; r0 < nrows; r0 += RB) {
    const int rows = min(RB, nrows - r0);
    hipLaunchKernelGGL((q8_pair_kernel<FMT, FMT2, RB, NW>), dim3(ta + tb), dim3(64 * NW), lds, s, a, b, ta, rows);
    PGD_HIP(hipGetLastError());
    a.x = reinterpret_cast<const float*>(a.x) + (size_t)rows * a.ldx;
    a.y += (size_t)rows * a.ldy;
    b.y += (size_t)rows * b.ldy;
  }
}

// the waves and rows per launch of launch_waves / launch_rows (shared by both
// matrices: they have the same K)
template <int FMT, int FMT2>
void pair_rows(const GemvArgs& a, const GemvArgs& b, int nrows, hipStream_t s) {
  const int kb = k_blocks<FMT>(a);
  auto go = [&](auto rb) {
    constexpr int RB = decltype(rb)::value;
    if (kb <= 4) return launch_pair_q8<FMT, FMT2, RB, 4>(a, b, nrows, s);
    launch_pair_q8<FMT, FMT2, RB, 8>(a, b, nrows, s);
  };
  const size_t cap = 160 * 1024;
  auto fits = [&](auto rb) {
    constexpr int RB = decltype(rb)::value;
    return lds_need<FMT, RB>(a.n_in, 1) <= cap && lds_need<FMT2, RB>(a.n_in, 1) <= cap;
  };
  if (nrows > 8 && fits(std::integral_constant<int, 16>{})) return go(std::integral_constant<int, 16>{});
  if (nrows > 4 && fits(std::integral_constant<int, 8>{})) return go(std::integral_constant<int, 8>{});
  if (nrows > 1 && fits(std::integral_constant<int, 4>{})) return go(std::integral_constant<int, 4>{});
  go(std::integral_constant<int, 1>{});
}

}  // namespace

bool q8act_pair_ok(int fmt_a, int fmt_b) {
  auto k256 = [](int f) { return f == FMT_Q4K || f == FMT_Q6K; };
  auto b32 = [](int f) { return f == FMT_Q8_0 || f == FMT_Q5_0; };
  return (k256(fmt_a) && k256(fmt_b)) || (b32(fmt_a) && b32(fmt_b));
}

void run_q8act_pair(int fmt_a, const GemvArgs& a, int fmt_b, const GemvArgs& b, int nrows, hipStream_t s) {
  PGD_CHECK(a.n_in == b.n_in, kErrShape, "paired GEMVs need one input width");
  PGD_CHECK(q8act_pair_ok(fmt_a, fmt_b), kErrFormat, "paired GEMVs need one activation type");
#define PGD_PAIR(F1, F2) \
  if (fmt_a == F1 && fmt_b == F2) return pair_rows<F1, F2>(a, b, nrows, s);
  PGD_PAIR(FMT_Q4K, FMT_Q4K)
  PGD_PAIR(FMT_Q4K, FMT_Q6K)
  PGD_PAIR(FMT_Q6K, FMT_Q4K)
  PGD_PAIR(FMT_Q6K, FMT_Q6K)
  PGD_PAIR(FMT_Q8_0, FMT_Q8_0)
  PGD_PAIR(FMT_Q8_0, FMT_Q5_0)
  PGD_PAIR(FMT_Q5_0, FMT_Q8_0)
  PGD_PAIR(FMT_Q5_0, FMT_Q5_0)
#undef PGD_PAIR
}

void run_q8act(int fmt, const GemvArgs& a, int nrows, int epi, hipStream_t s) {
  if (epi == EPI_SWIGLU) dispatch<EPI_SWIGLU>(fmt, a, nrows, s);
  else if (epi == EPI_RES) dispatch<EPI_RES>(fmt, a, nrows, s);
  else dispatch<EPI_STORE>(fmt, a, nrows, s);
}

}  // namespace gemv
}  // namespace pgd
