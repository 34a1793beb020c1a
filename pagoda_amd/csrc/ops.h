// ops.h — decode-path kernels other than the quantized GEMVs: RMSNorm,
// causal conv step, Gated-DeltaNet recurrence, q/k preparation with paged KV
// writes, paged GQA decode attention and argmax. All take ragged batches:
// `rows` token rows that belong to `nseq` sequences, sequence s owning rows
// [row_start[s], row_start[s] + row_count[s]) in feed order.
#pragma once
#include <vector>

#include "a8_act.h"
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pgd {

// y[r] = rmsnorm(x[src_row(r)]) * w, eps inside the sqrt.
//   mode 0: x * (1/sqrt(mean(x^2)+eps)) * w   (rms_zero, qwen3_5.rs:1736-1745)
//   mode 1: x / sqrt(mean(x^2)+eps) * w       (candle RmsNorm, qwen2_gguf.rs:92)
//   mode 2: mode 1 with the squares summed left to right, candle's CPU order
//           (n <= 8192)
// rows_idx (device, nullable) selects the source rows.
void rmsnorm_rows(const float* x, int ldx, const int* rows_idx, int rows, int n, const float* w, float eps,
                  int mode, float* y, int ldy, hipStream_t s);

// Per-sequence metadata of a ragged step, on the device.
struct SeqMeta {
  const int* row_start;  // [nseq]
  const int* row_count;  // [nseq]
};

// Depthwise causal conv decode step + SiLU with state shift
// (qwen3_5.rs:1800-1853, kernel k, state [channels, k-1] per sequence).
// x/out [rows, channels]; state_base[s] + state_off is the sequence's state.
// max_rows bounds every sequence's row count (0: one segment per sequence,
// which is right for any row count).
void conv_step(const float* x, int ldx, float* out, int ldo, int channels, int kernel, const float* weight,
               float* const* state_base, size_t state_off, SeqMeta meta, int nseq, int max_rows, hipStream_t s);

struct GdnParams {
  int k_heads, v_heads, k_dim, v_dim;
  const float* conv_out;  // [rows, 2*k_heads*k_dim + v_heads*v_dim]: q | k | v
  int ld_conv;
  const float* a;  // [rows, v_heads]
  const float* b;  // [rows, v_heads]
  int ld_ab;
  const float* z;  // [rows, v_heads*v_dim]
  int ld_z;
  const float* a_log;    // [v_heads]
  const float* dt_bias;  // [v_heads]
  const float* norm;     // [v_dim]
  float* out;            // [rows, v_heads*v_dim] (nullable when act is set)
  int ld_out;
  a8act::Dst act;        // the same output as prepared A8 activations (XA null: no)
  float* const* state_base;  // per sequence; state at state_base[s] + state_off, [v_heads, k_dim, v_dim]
  size_t state_off;
  // set by gdn_step, not by callers: the recurrence outputs of the chunkwise
  // form before their gated norm, [rows, v_heads * v_dim] (null: step kernel only)
  float* o_raw;
  int o_rows;  // rows of o_raw (rows past it are not written or read)
};

// Gated-DeltaNet recurrence over each sequence's rows in order
// (qwen3_5.rs:1330-1383; Metal gated_delta_step, qwen3_fuse.rs:176-279).
// k_dim == v_dim == 128. The fp32 state of a (sequence, head) is read once
// into registers, stepped through all its rows, and written once.
// When max_rows >= kGdnLongRows, sequences of at least kGdnLongRows rows take
// the chunkwise form instead: chunks of kGdnChunk tokens, each a triangular
// solve and small matrix products against the chunk's starting state, then a
// row-parallel gated norm. rows bounds row_start + row_count of every
// sequence (it sizes the outputs' staging); max_rows only selects whether the
// chunkwise kernels run, so any value gives correct results.
constexpr int kGdnLongRows = 32;
constexpr int kGdnChunk = 32;
void gdn_step(const GdnParams& p, SeqMeta meta, int nseq, int rows, int max_rows, hipStream_t s);

struct AttnLayout {
  int heads, kv_heads, head_dim, rotary_dim;
  int block;  // tokens per KV page
  // KV pool of this layer: [num_blocks][kv_heads][block][head_dim] f32, K and V
  float* k_pool;
  float* v_pool;
};

struct RowMeta {
  const int* seq_of_row;      // [rows]
  const int* pos_of_row;      // [rows] absolute position of the row's token
  const int* block_tables;    // [nseq][max_blocks]
  int max_blocks;
  const float* cos;           // [rows][rotary_dim] (host-computed tables)
  const float* sin;
};

// Full-attention q/k/v preparation and KV write.
// qwen35 (variant 0): q_raw row = per head [q(hd) | gate(hd)]; q,k RMSNorm
//   (q_norm/k_norm, eps 1e-6, rms_zero); partial rotate-half RoPE on the
//   first rotary_dim dims (qwen3_5.rs:1389-1432).
// qwen2 (variant 1): q_raw row = q; q/k/v biases added; full-width RoPE
//   (qwen2_gguf.rs:233-250, 346-349).
// Writes q [rows, heads, hd], gate [rows, heads, hd] (variant 0) and K/V
// into the pages at each row's position.
struct QkvPrep {
  int variant;
  const float* q_raw;
  int ld_q;
  const float* k_raw;
  const float* v_raw;
  int ld_kv;
  const float* q_norm;
  const float* k_norm;
  const float* q_bias;
  const float* k_bias;
  const float* v_bias;
  float* q;
  float* gate;
};
void qkv_prep(const QkvPrep& p, const AttnLayout& L, const RowMeta& m, int rows, hipStream_t s);

// Paged GQA decode attention: row r attends to positions [0, pos_of_row[r]]
// of its sequence. out [rows, heads, hd]; gate (nullable) multiplies by
// sigmoid(gate) (qwen3_5.rs:1433-1475; qwen2_gguf.rs:252-266). Work is cut
// into chunks of kChunkPages pages; rows whose chunk holds the same physical
// pages share one work item (the plan), so shared pages are read once.
constexpr int kChunkPages = 16;
struct AttnPlan {
  int n_items, n_slots, max_row_slots;
  const int* items;         // [n_items][6]: page_off, npages, row_off, first query, queries, chunk
  const int* pages;         // page ids of the items' chunks
  const int* item_rows;     // rows of the items; index = partial slot
  const int* row_slot_off;  // [rows + 1]
  const int* row_slots;     // each row's slots in chunk order
};
// Plan of one step as one int array (header + sections); the same array is
// uploaded as is, and attn_plan_view maps the host header onto its device copy.
void build_attn_plan(const int* seq_of_row, const int* pos_of_row, int rows, const int* block_tables,
                     int max_blocks, int block, int group, int head_dim, std::vector<int>& out);
AttnPlan attn_plan_view(const int* host, const int* dev);
// The same attention in the CPU path's exact operation order (sequential dot,
// sum and weighted sum; exp correctly rounded): bit-equal to the CPU
// restatement. out [rows, heads, head_dim]; max_len: the longest context of
// the rows.
void attn_exact(const float* q, float* out, const AttnLayout& L, const RowMeta& m, int rows, int max_len,
                hipStream_t s);
void attn_decode(const float* q, const float* gate, float* out, const AttnLayout& L, const RowMeta& m,
                 const AttnPlan& plan, int rows, hipStream_t s, const a8act::Dst* act = nullptr);

// Row-wise argmax over finite values. last_max = 0: first index among equal
// maxima (pagoda/src/sampler.rs:59-69); 1: last (Iterator::max_by,
// qwen3_5.rs:524-529). ids[r] = 0xFFFFFFFF when a row has no finite value;
// nonfinite[r] counts non-finite entries.
void argmax_rows(const float* x, int ld, int rows, int n, int last_max, uint32_t* ids, float* vals,
                 int* nonfinite, hipStream_t s);

// dst[r] = src[idx[r]] (rows of n floats)
void gather_rows(const float* src, int lds, const int* idx, int rows, int n, float* dst, int ldd, hipStream_t s);

}  // namespace pgd
