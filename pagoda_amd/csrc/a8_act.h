// a8_act.h — prepared activations of the A8 matrix-core GEMV, written by
// the prep kernels and directly by the kernels that produce GEMV inputs
// (gated RMSNorm of the Gated-DeltaNet, attention output, SwiGLU).
//
// For an activation of `rows` rows and K = 64 G columns, rows are cut into
// chunks of 32 (two 16-row batch tiles). Per chunk c, group g, tile bt,
// item = (c G + g) 2 + bt:
//   XA[item][i][lane] = 16 B: operand i = xh step 0 | xh step 1 | xl step 0 |
//     xl step 1 (8 halves), batch row 32c + 16bt + lane % 16,
//     k = 64g + 16(lane / 16) + 8 step + e, with xh = f16(x), xl = f16(x - xh)
//   CA[item][64] = -1024 XSP_A[16] | -1024 XSP_B[16] | XS_A[16] | XS_B[16]
// where A sums k quarters 0-1 of the group and B quarters 2-3, XS = sum x and
// XSP = sum (xh + xl) (the consumer adds A + B, which is the same sum as over
// the four quarters in order). A chunk of at most 4 rows (decode batches
// 1..4) is stored compact instead, at the start of the same region:
//   X4[g][row][i][q] = 16 B (row < 4),   C4[g][16] = -1024 XSP_A[4] | -1024 XSP_B[4] | XS_A[4] | XS_B[4]
// so that one row's operands are one contiguous 256 B run. Rows past the end
// are never written: their MFMA rows only feed discarded outputs.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace pgd {
namespace a8act {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

struct Dst {
  uint4* XA;  // operand region (null: no prepared output)
  float* CA;  // constant region
  int rows;   // rows of the whole activation (fixes chunking and compact chunks)
  int G;      // groups of 64 columns
};

__host__ __device__ inline size_t xa_bytes(int rows, int G) { return ((size_t)rows + 31) / 32 * G * 2 * 4096; }
__host__ __device__ inline size_t ca_bytes(int rows, int G) { return ((size_t)rows + 31) / 32 * G * 2 * 256; }

__device__ inline bool chunk_compact(int rows, int c) { return rows - 32 * c <= 4; }

// half a 16-wide k slice (8 values): its two operand words (xh, xl of the 8
// k) and the running sums, continued from xs / xsp (in slice order)
__device__ inline void prep8(const float* v, uint4& oh, uint4& ol, float& xs, float& xsp) {
  uint32_t hw[4], lw[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const _Float16 h0 = (_Float16)v[2 * p], h1 = (_Float16)v[2 * p + 1];
    const _Float16 l0 = (_Float16)(v[2 * p] - (float)h0), l1 = (_Float16)(v[2 * p + 1] - (float)h1);
    hw[p] = __builtin_bit_cast(uint32_t, (h2){h0, h1});
    lw[p] = __builtin_bit_cast(uint32_t, (h2){l0, l1});
    xs += v[2 * p] + v[2 * p + 1];
    xsp += ((float)h0 + (float)l0) + ((float)h1 + (float)l1);
  }
  oh = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  ol = make_uint4(lw[0], lw[1], lw[2], lw[3]);
}

// the four operands of one 16-wide k slice and its partial sums
__device__ inline void prep16(const float* v, uint4 (&o)[4], float& xs, float& xsp) {
  xs = 0.0f;
  xsp = 0.0f;
  prep8(v, o[0], o[2], xs, xsp);
  prep8(v + 8, o[1], o[3], xs, xsp);
}

// operands of slice (row, g, q)
__device__ inline void put_operands(const Dst& d, int row, int g, int q, const uint4 (&o)[4]) {
  const int c = row >> 5;
  if (chunk_compact(d.rows, c)) {
    uint4* p = d.XA + (size_t)c * d.G * 512 + ((size_t)g * 4 + (row & 31)) * 16 + q;
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i * 4] = o[i];
  } else {
    const size_t item = ((size_t)c * d.G + g) * 2 + ((row >> 4) & 1);
    uint4* p = d.XA + item * 256 + q * 16 + (row & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i * 64] = o[i];
  }
}

// operand i (0..3) alone of slice (row, g, q): for producers whose lanes hold
// half a slice (i = 0, 2: k 0..7; i = 1, 3: k 8..15)
__device__ inline void put_operand(const Dst& d, int row, int g, int q, int i, const uint4& o) {
  const int c = row >> 5;
  if (chunk_compact(d.rows, c)) {
    d.XA[(size_t)c * d.G * 512 + ((size_t)g * 4 + (row & 31)) * 16 + q + i * 4] = o;
  } else {
    const size_t item = ((size_t)c * d.G + g) * 2 + ((row >> 4) & 1);
    d.XA[item * 256 + q * 16 + (row & 15) + i * 64] = o;
  }
}

// half-group sums (half 0: quarters 0-1, half 1: quarters 2-3) of (row, g)
__device__ inline void put_half(const Dst& d, int row, int g, int half, float xs, float xsp) {
  const int c = row >> 5;
  if (chunk_compact(d.rows, c)) {
    float* p = d.CA + (size_t)c * d.G * 128 + (size_t)g * 16 + half * 4 + (row & 31);
    p[0] = -1024.0f * xsp;
    p[8] = xs;
  } else {
    const size_t item = ((size_t)c * d.G + g) * 2 + ((row >> 4) & 1);
    float* p = d.CA + item * 64 + half * 16 + (row & 15);
    p[0] = -1024.0f * xsp;
    p[32] = xs;
  }
}

// One 16-wide slice (k = 64 g + 16 q ...) of `row`. The lane holding quarter
// q ^ 1 of the same (row, g) must be lane ^ PARTNER of the same wave and
// execute this call together (the two quarters of a half are summed with one
// XOR shuffle; fp addition commutes, so both lanes get the same sum).
template <int PARTNER = 1>
__device__ inline void emit_slice(const Dst& d, int row, int g, int q, const float (&v)[16], bool live) {
  uint4 o[4];
  float xs, xsp;
  prep16(v, o, xs, xsp);
  xs += __shfl_xor(xs, PARTNER, 64);
  xsp += __shfl_xor(xsp, PARTNER, 64);
  if (!live) return;
  put_operands(d, row, g, q, o);
  if ((q & 1) == 0) put_half(d, row, g, q >> 1, xs, xsp);
}

}  // namespace a8act
}  // namespace pgd
