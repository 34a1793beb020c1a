// quant.h — device layout of quantized matrices and the GEMV launchers.
//
// Every matrix is [n_out, n_in] with n_in contiguous. One device allocation
// per matrix holds structure-of-arrays planes so each wave streams one plane
// with 128-bit loads:
//
//   A8  (MLX affine, group 64):  codes u8, tiled: for each 32-row tile and
//                                64-wide group a 2 KiB block [k half][row][32 codes]
//                                (the order the matrix-core lanes read it)
//                                sb    u32, tiled [tile][group][32 rows]: bf16 scale | bf16 bias << 16
//                                rows are padded to a multiple of 32 with zeros
//   Q4K (GGML block_q4_K):       qs    u8 [n_out][nsb*128]      the 128 nibble bytes of each block
//                                hdr   16B [n_out][nsb]         d, dmin (f16) + 12 packed scale bytes
//   Q6K (GGML block_q6_K):       ql, qh, sc, d planes, tiled by 32 rows
//                                (q6k_*_off below); rows padded with zeros
//
// The planes hold exactly the bytes of the source blocks (144 B / 210 B per
// 256 weights; 1.0625 B per A8 weight), only regrouped.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "a8_act.h"

namespace pgd {

enum Fmt : int { FMT_A8 = 0, FMT_Q4K = 1, FMT_Q6K = 2, FMT_Q8_0 = 3, FMT_Q5_0 = 4 };

// GGML 32-weight block formats (row-major planes, block b of row r at r * nsb + b)
constexpr int kQ8_0Bytes = 34, kQ5_0Bytes = 22;

struct QMat {
  int fmt = FMT_A8;
  // nsb: 256-weight super-blocks per row (Q4K / Q6K), 32-weight blocks per row (Q8_0 / Q5_0)
  int n_out = 0, n_in = 0, nsb = 0;
  uint8_t* base = nullptr;  // owning device allocation
  size_t bytes = 0;
  // plane pointers (into base)
  uint8_t* p0 = nullptr;  // A8 codes | Q4K qs | Q6K ql | Q8_0 int8 q [n_out][n_in] | Q5_0 qs [n_out][n_in / 2]
  uint8_t* p1 = nullptr;  // A8 sb    | Q4K hdr | Q6K qh | Q8_0 f16 d [n_out][nsb] | Q5_0 u32 qh [n_out][nsb]
  uint8_t* p2 = nullptr;  //                      Q6K sc |                        | Q5_0 f16 d [n_out][nsb]
  uint8_t* p3 = nullptr;  //                      Q6K d
};

// A8 tiled addressing (G = n_in / 64 groups per row)
__host__ __device__ inline size_t a8_code_off(int row, int k, int G) {
  return ((((size_t)(row >> 5) * G + (k >> 6)) << 11) + (size_t)(((k >> 5) & 1) << 10) + (size_t)((row & 31) << 5) +
          (size_t)(k & 31));
}
__host__ __device__ inline size_t a8_sb_off(int row, int g, int G) {
  return (((size_t)(row >> 5) * G + g) << 5) + (size_t)(row & 31);
}

// Q4K tiled addressing: the GGML block bytes, reordered so that the 32 bytes
// of one 64-group of 32 consecutive rows are one 1 KiB run. qs byte i
// (0 <= i < 128 nsb; 64-group g = i / 32) of row r, and the 16-byte header
// (d, dmin, 12 scale bytes) of super-block sb of row r.
__host__ __device__ inline size_t q4k_qs_off(int row, int i, int nsb) {
  return ((size_t)(row >> 5) * (4 * (size_t)nsb) + (size_t)(i >> 5)) * 1024 + (size_t)(row & 31) * 32 + (size_t)(i & 31);
}
__host__ __device__ inline size_t q4k_hdr_off(int row, int sb, int nsb) {
  return ((size_t)(row >> 5) * nsb + (size_t)sb) * 512 + (size_t)(row & 31) * 16;
}

// Q6K tiled addressing. For each 32-row tile and 128-element half u of the
// rows (2 nsb halves): a 2 KiB ql block (64 B per row), a 1 KiB qh block
// (32 B per row) and a 256 B scale block (8 int8 per row); per tile and
// super-block 32 f16 d. Inside the ql / qh blocks, dword k of a row's
// 16-byte runs (bytes 4k..4k+3 of each run) of row 16 h + j lives at
// [4 h + k][j][run]: the four ql dwords (two qh dwords) a matrix-core lane
// needs for one half are 16 (8) contiguous bytes, and 64 lanes read 1 KiB
// (512 B) contiguously. ql byte i of a row (0 <= i < 128 nsb), qh byte i
// (0 <= i < 64 nsb), scale i (0 <= i < 16 nsb), d of super-block sb (in f16
// elements):
__host__ __device__ inline size_t q6k_ql_off(int row, int i, int nsb) {
  const int u = i >> 6, w = i & 63;
  const size_t blk = (size_t)(row >> 5) * 2 * nsb + u;
  const int lane = ((((row & 31) >> 4) << 2) + ((w & 15) >> 2)) * 16 + (row & 15);
  return (blk << 11) + (size_t)lane * 16 + (w >> 4) * 4 + (w & 3);
}
__host__ __device__ inline size_t q6k_qh_off(int row, int i, int nsb) {
  const int u = i >> 5, w = i & 31;
  const size_t blk = (size_t)(row >> 5) * 2 * nsb + u;
  const int lane = ((((row & 31) >> 4) << 2) + ((w & 15) >> 2)) * 16 + (row & 15);
  return (blk << 10) + (size_t)lane * 8 + (w >> 4) * 4 + (w & 3);
}
__host__ __device__ inline size_t q6k_sc_off(int row, int i, int nsb) {
  const size_t blk = (size_t)(row >> 5) * 2 * nsb + (i >> 3);
  return (blk << 8) + (size_t)(row & 31) * 8 + (i & 7);
}
__host__ __device__ inline size_t q6k_d_off(int row, int sb, int nsb) {
  return ((size_t)(row >> 5) * nsb + sb) * 32 + (row & 31);
}

// algorithmic bytes of the weights (what a GEMV must stream at least once;
// unpadded n_in as the measurement plan defines it)
double qmat_algo_bytes(const QMat& m);

// allocate planes for a matrix on the device; A8 padding rows are zeroed on
// stream s (everything else is written by the upload or synth that follows)
void qmat_alloc(QMat& m, int fmt, int n_out, int n_in, hipStream_t s);
void qmat_free(QMat& m);

// host source blocks -> device planes
void qmat_upload_a8(QMat& m, const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                    hipStream_t s);
void qmat_upload_kq(QMat& m, const uint8_t* blocks, hipStream_t s);

// dequantize rows [row0, row0+rows) to f32 [rows, n_in]; bit-exact to the
// host formulas (A8: bias + scale*code; Q4K: d1*q - m1; Q6K: d*sc*q).
void qmat_dequant(const QMat& m, int row0, int rows, float* out, hipStream_t s);

// GEMV / skinny GEMM: y[r, n] = sum_k W[n, k] * x[r, k] for r < nrows.
// x is f32 (x_f16 == 0) or IEEE f16 (x_f16 == 1), row stride ldx elements.
// res (nullable): y = res + W.x (res may alias y).
void qmat_gemv(const QMat& m, const void* x, int x_f16, int ldx, int nrows, float* y, int ldy,
               const float* res, int ldres, hipStream_t s);

// The same products with candle's CPU arithmetic (the reference's CPU path,
// pagoda-hf/src/qwen2_gguf.rs:280-289): each f32 activation row is quantized
// to Q8_K (Q4_K / Q6_K weights) or Q8_0 (Q8_0 / Q5_0 weights) and every
// output is an integer block dot scaled in f32.
void qmat_gemv_q8act(const QMat& m, const float* x, int ldx, int nrows, float* y, int ldy, const float* res, int ldres,
                     hipStream_t s);
void qmat_gemv_swiglu_q8act(const QMat& gate, const QMat& up, const float* x, int ldx, int nrows, float* mid, int ldm,
                            hipStream_t s);
// qmat_gemv_q8act of two matrices over the same input rows in one launch
// (ya = A.x, yb = B.x, both with row stride ldy), bit-equal to two calls;
// qmat_q8act_pairable says whether two matrices can share a launch.
bool qmat_q8act_pairable(const QMat& a, const QMat& b);
void qmat_gemv_q8act_pair(const QMat& a, float* ya, const QMat& b, float* yb, const float* x, int ldx, int nrows,
                          int ldy, hipStream_t s);

// fused SwiGLU: mid[r, n] = silu(gate.x) * (up.x)
void qmat_gemv_swiglu(const QMat& gate, const QMat& up, const float* x, int ldx, int nrows, float* mid,
                      int ldm, hipStream_t s);

// ---- A8 activation operands ------------------------------------------------
// The A8 GEMV consumes activations converted once into matrix-core operands
// (f16 hi/lo pairs + per-group sums), in chunks of 32 rows. One prepared
// buffer can feed every A8 matrix with the same input width.
struct A8Act {
  const void* XA = nullptr;
  const float* CA = nullptr;
  int rows = 0, K = 0;
  // deferred RMSNorm (a8_gnorm_prep): the operands hold x * w without the
  // 1/rms factor, rss holds per row the K/32 partial sums of x^2 (one per
  // 32-wide half group), and the consuming GEMV scales row b's outputs by
  // 1/sqrt(sum / K + eps). Null: the operands are the finished input.
  const float* rss = nullptr;
  float eps = 0.0f;
};
size_t a8_act_bytes(int rows, int K);
A8Act a8_act_view(void* buf, int rows, int K);
// destination descriptor for kernels that write prepared activations directly
a8act::Dst a8_act_dst(const A8Act& a);
// from f32 rows x [rows, ldx]
A8Act a8_act_prep(const float* x, int ldx, int rows, int K, void* buf, hipStream_t s);
// the deferred-norm row sums region of an activation buffer
float* a8_act_rss(void* buf, int rows, int K);
// Residual A8 GEMV y += W act (in place) that also writes the next RMSNorm's
// deferred input from the new rows into nbuf (a8_act_bytes(rows, n_out)):
// operands of y * nw and their row sums, exactly as a8_gnorm_prep would make
// them from y. n_out must be a multiple of 32; matrices that take the
// stream-K kernel are not supported.
A8Act qmat_gemv_a8_res_norm(const QMat& m, const A8Act& act, float* y, int ldy, const float* nw, float eps,
                            void* nbuf, hipStream_t s);
// RMSNorm with the scale deferred to the consumer: operands of x * w and the
// row's partial sums of squares (A8Act.rss); one wave per (32-row chunk,
// group, 16-row tile), no per-row reduction. Feeds A8 GEMVs only.
A8Act a8_gnorm_prep(const float* x, int ldx, int rows, int n, const float* w, float eps, void* buf, hipStream_t s);
// fused RMSNorm (x * rsqrt(mean x^2 + eps) * w) + prep; y (nullable) also
// receives the normalized rows; rows_idx (nullable) selects source rows
A8Act a8_norm_prep(const float* x, int ldx, const int* rows_idx, int rows, int n, const float* w, float eps, float* y,
                   int ldy, void* buf, hipStream_t s);
void qmat_gemv_a8(const QMat& m, const A8Act& act, float* y, int ldy, const float* res, int ldres, hipStream_t s);
// device scratch bytes qmat_gemv_a8 takes for `rows` rows (res: residual form)
size_t qmat_gemv_a8_scratch(const QMat& m, int rows, bool res);
// qmat_gemv_a8 (store) for a step where row r is the only token of sequence
// r: outputs n < conv_n of row r also take the causal conv step of channel n
// (the conv_step arithmetic): weights conv_w [conv_n][kernel], state at
// state_base[r] + state_off, [conv_n][kernel - 1] (updated), SiLU output to
// conv_out[r * ldc + n].
void qmat_gemv_a8_conv(const QMat& m, const A8Act& act, float* y, int ldy, const float* conv_w,
                       float* const* state_base, size_t state_off, int conv_n, int kernel, float* conv_out, int ldc,
                       hipStream_t s);
// mid (nullable when mid_act is given): silu(gate x) * (up x) in f32;
// mid_act (nullable): the same product written as prepared activations
void qmat_gemv_a8_swiglu(const QMat& gate, const QMat& up, const A8Act& act, float* mid, int ldm, hipStream_t s,
                         const A8Act* mid_act = nullptr);

// embedding rows: out[r, :] = dequant(W[ids[r], :]) (ids on device)
void qmat_embed(const QMat& m, const uint32_t* ids, int nrows, float* out, int ldo, hipStream_t s);

// synthetic init: fill the planes with the quantized form of seeded
// N(0, std) weights (counter-based generator, reproduced bit for bit by the
// CPU checker).
void qmat_synth(QMat& m, uint64_t seed, uint64_t key, float std, hipStream_t s);
// rows [row0, row0 + rows) of an A8 matrix from their own key (a stacked
// matrix whose row ranges are separate tensors)
void qmat_synth_rows(QMat& m, int row0, int rows, uint64_t seed, uint64_t key, float std, hipStream_t s);

// seeded f32 vectors
void synth_normal_f32(float* out, size_t n, uint64_t seed, uint64_t key, float scale, hipStream_t s);
void synth_uniform_f32(float* out, size_t n, uint64_t seed, uint64_t key, float scale, hipStream_t s);
void fill_f32(float* out, size_t n, float v, hipStream_t s);

namespace gemv {
// Per-stream device scratch buffers that grow on demand (slots: see gemv_impl.h).
void* gemv_scratch(hipStream_t s, size_t bytes, int slot);
// A caller-provided device region that gemv::gemv_scratch carves its slots from,
// on the calling thread only, instead of allocating: each slot gets one
// 256-byte aligned range on first use and keeps it while it is large enough
// (launches on one stream run in order, so reusing a slot is safe as with the
// allocating path). Exhausting the region throws kErrShape.
struct ScratchArena {
  uint8_t* base = nullptr;
  size_t cap = 0, used = 0;
  size_t off[8] = {}, len[8] = {};
};
// install (nullptr: back to allocating); returns the previous arena
ScratchArena* set_scratch_arena(ScratchArena* a);
// Counts the (re)allocations of the stream scratch buffers: launch arguments
// recorded before a change may point at freed memory.
uint64_t scratch_epoch();
}  // namespace gemv

}  // namespace pgd
