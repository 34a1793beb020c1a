/*
 * pagoda_hip.h — C ABI of the MI355X (gfx950) decode backend for pagoda.
 *
 * Plain pointers and sizes only. Every call returns 0 on success or a
 * negative status; pgd_last_error() gives the message of the last failure
 * on the calling thread. Unless a name ends in _dev, pointers are HOST
 * memory and the call is synchronous. _dev calls take DEVICE pointers, are
 * queued on the device handle's stream and return without waiting.
 *
 * Each entry point cites the reference interface it replaces (paths relative
 * to the quantz8a/pagoda tree).
 */
#ifndef PAGODA_HIP_H
#define PAGODA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  PGD_OK = 0,
  PGD_ERR_ARG = -1,
  PGD_ERR_DEVICE = -2,
  PGD_ERR_HIP = -3,
  PGD_ERR_SHAPE = -4,
  PGD_ERR_STATE = -5,
  PGD_ERR_ALLOC = -6,
  PGD_ERR_FORMAT = -7,
};

enum { PGD_FMT_A8 = 0, PGD_FMT_Q4K = 1, PGD_FMT_Q6K = 2 };

typedef struct pgd_dev pgd_dev;
typedef struct pgd_matrix pgd_matrix;

/* ---- errors / version ---------------------------------------------------- */
/* Copies the last error message (NUL terminated, truncated to len). Returns its full length. */
int pgd_last_error(char* buf, size_t len);
/* ABI version (major*10000 + minor*100 + patch). */
int pgd_version(void);

/* ---- device ---------------------------------------------------------------
 * Replaces CandleModel::device_from_env (pagoda-hf/src/lib.rs:409-426) for
 * PAGODA_DEVICE=hip: spec is "hip" or "hip:N". Any other spec is an error;
 * there is no CPU fallback. */
int pgd_device_open(const char* spec, pgd_dev** out);
int pgd_device_close(pgd_dev* dev);
int pgd_device_sync(pgd_dev* dev);
/* The hipStream_t every _dev call of this handle is queued on. */
void* pgd_device_stream(pgd_dev* dev);
int pgd_device_malloc(pgd_dev* dev, size_t bytes, void** out);
int pgd_device_free(pgd_dev* dev, void* ptr);
/* kind: 0 host->device, 1 device->host, 2 device->device (synchronous) */
int pgd_device_memcpy(pgd_dev* dev, void* dst, const void* src, size_t bytes, int kind);

/* Device-to-device copy queued on the handle's stream, not waited for (no
 * reference counterpart: the on-box streaming rate the roofline report
 * quotes beside the HBM specification). */
int pgd_device_copy_dev(pgd_dev* dev, void* dst, const void* src, size_t bytes);

/* ---- timing: HIP events recorded on the device handle's stream --------- */
typedef struct pgd_event pgd_event;
int pgd_event_new(pgd_dev* dev, pgd_event** out);
int pgd_event_record(pgd_event* ev);
/* Waits for `end`, then writes the elapsed milliseconds between the two. */
int pgd_event_elapsed_ms(pgd_event* start, pgd_event* end, float* ms);
int pgd_event_free(pgd_event* ev);

/* ---- quantized matrices ---------------------------------------------------
 * Replaces QuantMatrix::upload (pagoda-hf/src/qwen3_gemv.rs:658-705):
 * MLX affine 8-bit group 64, packed u32 [n_out, n_in/4] (codes little
 * endian), bf16 scales/biases [n_out, n_in/64]. */
int pgd_matrix_upload_a8(pgd_dev* dev, const uint32_t* packed, const uint16_t* scales_bf16,
                         const uint16_t* biases_bf16, int n_out, int n_in, pgd_matrix** out);
/* GGML block_q4_K / block_q6_K rows of ceil(n_in/256) blocks (144 B / 210 B);
 * replaces the QTensor -> QMatMul load of pagoda-hf/src/qwen2_gguf.rs:283-289. */
int pgd_matrix_upload_q4k(pgd_dev* dev, const void* blocks, int n_out, int n_in, pgd_matrix** out);
int pgd_matrix_upload_q6k(pgd_dev* dev, const void* blocks, int n_out, int n_in, pgd_matrix** out);
/* GGML block_q8_0 / block_q5_0 rows of n_in/32 blocks (34 B / 22 B; n_in a
 * multiple of 32): the types a Q4_K_M GGUF holds for rows that are not whole
 * 256-weight super-blocks, loaded by candle at pagoda-hf/src/qwen2_gguf.rs:
 * 283-289 like the k-quants. Format ids 3 and 4 in pgd_matrix_info. */
int pgd_matrix_upload_q8_0(pgd_dev* dev, const void* blocks, int n_out, int n_in, pgd_matrix** out);
int pgd_matrix_upload_q5_0(pgd_dev* dev, const void* blocks, int n_out, int n_in, pgd_matrix** out);
/* Seeded synthetic matrix: N(0, std) weights quantized on the device (no
 * reference counterpart: the reference only loads checkpoints). */
int pgd_matrix_synth(pgd_dev* dev, int fmt, int n_out, int n_in, uint64_t seed, uint64_t key, float std,
                     pgd_matrix** out);
int pgd_matrix_free(pgd_matrix* m);
/* fmt, n_out, n_in, device bytes, algorithmic bytes (bpw * n_out * n_in / 8). */
int pgd_matrix_info(const pgd_matrix* m, int* fmt, int* n_out, int* n_in, size_t* dev_bytes,
                    double* algo_bytes);
/* Dequantize rows to f32 host memory [rows, n_in]; replaces
 * Affine::dequant_rows (pagoda-hf/src/qwen3_5.rs:1546-1584). Bit-exact. */
int pgd_matrix_dequant(const pgd_matrix* m, int row0, int rows, float* out);
/* y[r, :] = W . x[r, :] for r < nrows (nrows 1..64 ragged batch rows), x f32
 * [nrows, n_in], y f32 [nrows, n_out]. Replaces QuantMatrix::gemv and
 * encode_gemm4 (pagoda-hf/src/qwen3_gemv.rs:730-742, 826-846). */
int pgd_matrix_gemv(const pgd_matrix* m, const float* x, int nrows, float* y);
/* Device form. x f32 (x_f16 = 0) or IEEE f16 (x_f16 = 1), row stride ldx
 * elements (multiple of 8); y row stride ldy; res (nullable) adds a residual
 * y = res + W.x (replaces affine_gemv_res, qwen3_gemv.rs:289-306). */
int pgd_matrix_gemv_dev(const pgd_matrix* m, const void* x, int x_f16, int ldx, int nrows, float* y,
                        int ldy, const float* res, int ldres);
/* mid = silu(gate . x) * (up . x); replaces affine_gemv2_silu
 * (qwen3_gemv.rs:256-286). */
int pgd_matrix_gemv_swiglu_dev(const pgd_matrix* gate, const pgd_matrix* up, const float* x, int ldx,
                               int nrows, float* mid, int ldm);
/* A8 activations converted once into matrix-core operands, shared by every
 * A8 matrix of width k (the reference shares one x across several matrices
 * the same way: gemv_shared / affine_gemv_n, qwen3_gemv.rs:149-253).
 * pgd_act_bytes gives the device buffer size for nrows x k. */
size_t pgd_act_bytes(int nrows, int k);
int pgd_act_prep_dev(pgd_dev* dev, const float* x, int ldx, int nrows, int k, void* act);
int pgd_matrix_gemv_act_dev(const pgd_matrix* m, const void* act, int nrows, float* y, int ldy, const float* res,
                            int ldres);
int pgd_matrix_gemv_swiglu_act_dev(const pgd_matrix* gate, const pgd_matrix* up, const void* act, int nrows,
                                   float* mid, int ldm);
/* candle's CPU QMatMul::forward for GGUF weights (called at
 * pagoda-hf/src/qwen2_gguf.rs:271-278, kept on the CPU by qweight at 280-289):
 * each f32 activation row (stride ldx) is quantized to Q8_K (Q4_K / Q6_K
 * weights) or Q8_0 (Q8_0 / Q5_0 weights), every output an integer block dot
 * scaled in f32. res (nullable) adds a residual as in pgd_matrix_gemv_dev. */
int pgd_matrix_gemv_q8act_dev(const pgd_matrix* m, const float* x, int ldx, int nrows, float* y, int ldy,
                              const float* res, int ldres);
/* Two pgd_matrix_gemv_q8act_dev calls over the same input rows in one launch
 * (the Qwen2 attention's q/k and v projections, qwen2_gguf.rs:234-236, whose
 * GGML types differ in Q4_K_M files): ya = a.x and yb = b.x, row stride ldy,
 * bit-equal to the two calls. Both matrices take the same input width and one
 * activation type (Q4_K / Q6_K: Q8_K; Q8_0 / Q5_0: Q8_0), else PGD_ERR_FORMAT. */
int pgd_matrix_gemv_q8act_pair_dev(const pgd_matrix* a, float* ya, const pgd_matrix* b, float* yb, const float* x,
                                   int ldx, int nrows, int ldy);
/* No counterpart in the reference. pgd_matrix_gemv_act_dev for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): the same kernels and results, with
 * their scratch (split-K / stream-K partial sums) taken from one fixed
 * pgd_noalloc_scratch_bytes() (40 MiB) device array per GPU, held until the
 * process ends; calls no hipMalloc / hipFree. A launch needing more scratch
 * (37..64-row launches of matrices over ~41000 rows) is PGD_ERR_SHAPE before anything
 * runs. Every call on one GPU shares that array: a call queued on another
 * device handle's stream than the previous call's first waits (on the GPU,
 * through an event) for that call to finish; calls are serialized on the
 * host. The array keeps the last call's contents. */
size_t pgd_noalloc_scratch_bytes(void);
int pgd_matrix_gemv_act_dev_noalloc(const pgd_matrix* m, const void* act, int nrows, float* y, int ldy,
                                    const float* res, int ldres);

/* ---- decode-step kernels (device pointers, queued on the device stream) ----
 * Gated-DeltaNet recurrence over a ragged batch: sequence i owns rows
 * [row_start[i], row_start[i] + row_count[i]) and its fp32 state
 * states[i] -> [v_heads, 128, 128], updated in place, rows in order.
 * conv_out [rows, 2*k_heads*128 + v_heads*128] (post conv + SiLU: q | k | v),
 * a, b [rows, v_heads], z [rows, v_heads*128], out [rows, v_heads*128].
 * row_start, row_count and states are device arrays.
 * Replaces the per-token loop of LinearAttn::forward (pagoda-hf/src/
 * qwen3_5.rs:1330-1383) and gated_delta_step (qwen3_fuse.rs:176-279). */
int pgd_gdn_step_dev(pgd_dev* dev, int k_heads, int v_heads, const float* conv_out, const float* a,
                     const float* b, const float* z, const float* a_log, const float* dt_bias,
                     const float* norm, float* const* states, const int* row_start, const int* row_count,
                     int nseq, float* out);
/* pgd_gdn_step_dev for prefill: the same recurrence, where sequences of at
 * least 32 rows take the chunkwise form (32-token chunks: a triangular solve
 * and matrix products against each chunk's starting state, the published
 * chunked form of the gated delta rule; equal to the per-token loop in exact
 * arithmetic, to fp32 rounding in practice). rows: every sequence's
 * row_start + row_count is at most rows (rows past it are left unwritten,
 * never written out of bounds). max_rows: the largest row_count, or
 * any bound on it (below 32 every sequence takes the per-token kernel).
 * Replaces the same reference loop as pgd_gdn_step_dev, which it runs one
 * token at a time for prefill too (qwen3_5.rs:1330-1383). */
int pgd_gdn_prefill_dev(pgd_dev* dev, int k_heads, int v_heads, const float* conv_out, const float* a,
                        const float* b, const float* z, const float* a_log, const float* dt_bias,
                        const float* norm, float* const* states, const int* row_start, const int* row_count,
                        int nseq, int rows, int max_rows, float* out);
/* Paged GQA decode attention: row r attends to positions [0, pos_of_row[r]]
 * of sequence seq_of_row[r], whose pages are block_tables[seq * max_blocks
 * + p / block] in pools [pages][kv_heads][block][head_dim]. q, gate, out
 * [rows, heads, head_dim]; gate (nullable) applies sigmoid(gate). Replaces
 * FullAttn::forward's softmax attention (pagoda-hf/src/qwen3_5.rs:1433-1475)
 * and full_attn_heads (qwen3_fuse.rs:384-440) over a contiguous cache. */
int pgd_attn_decode_dev(pgd_dev* dev, int heads, int kv_heads, int head_dim, int block, const float* q,
                        const float* gate, const float* k_pool, const float* v_pool, const int* seq_of_row,
                        const int* pos_of_row, const int* block_tables, int max_blocks, int rows, float* out);

/* ---- models and sessions ---------------------------------------------------
 * Architecture of a model handle. arch 0 is the hybrid Qwen3.5 tower
 * (Gated-DeltaNet + gated full attention, MLX affine-8 weights; Qwen35::load
 * pagoda-hf/src/qwen3_5.rs:338-452); arch 1 is Qwen2 with GGUF Q4_K/Q6_K
 * weights and tied embeddings (Qwen2Gguf::load pagoda-hf/src/qwen2_gguf.rs:65-140). */
enum { PGD_ARCH_QWEN35 = 0, PGD_ARCH_QWEN2 = 1 };

typedef struct pgd_model_config {
  int arch;
  int n_layers, hidden, intermediate, vocab;
  int heads, kv_heads, head_dim, rotary_dim;
  float rope_theta, eps;
  int k_heads, v_heads, k_dim, v_dim, conv_kernel; /* gated-delta layers (arch 0) */
  int full_every; /* arch 0: layer i is full attention iff i % full_every == full_every - 1 */
  int max_pos;    /* context limit (qwen2_gguf.rs:146-150) */
  int kv_block;   /* tokens per KV page (16) */
  int kv_blocks;  /* KV pages per full-attention layer */
} pgd_model_config;

typedef struct pgd_model pgd_model;
typedef struct pgd_session pgd_session;

/* Build a model with seeded synthetic weights generated on the device (the
 * configs use random-init weights; no reference counterpart). */
int pgd_model_synth(pgd_dev* dev, const pgd_model_config* cfg, uint64_t seed, pgd_model** out);
/* Qwen35::load (pagoda-hf/src/qwen3_5.rs:338-452, store 1587-1698): the
 * language model of an MLX directory (config.json; model.safetensors.index.json
 * and its shards, or a single model.safetensors). Matrices are 8-bit affine
 * group 64 (u32 codes, bf16 scales / biases); norms, conv, A_log and dt_bias
 * F32 / BF16 / F16. Layer kinds come from config.json's layer_types.
 * max_pos <= 0: max_position_embeddings; kv_blocks > 0: KV pages per
 * full-attention layer. Errors (missing tensors, shapes, quantization other
 * than 8-bit affine group 64) return kErrFormat and allocate nothing. */
int pgd_model_load_mlx(pgd_dev* dev, const char* dir, int max_pos, int kv_blocks, pgd_model** out);
/* Qwen2 GGUF load (pagoda-hf/src/qwen2_gguf.rs:65-140): GGUF v2/v3,
 * general.architecture "qwen2"; Q4_K / Q6_K / Q8_0 / Q5_0 matrices, F32 / F16 norms and
 * q/k/v biases; lm_head is output.weight or the tied token_embd.weight.
 * Tensors in other ggml block types are an error naming the tensor.
 * max_pos <= 0: qwen2.context_length. */
int pgd_model_load_gguf(pgd_dev* dev, const char* path, int max_pos, int kv_blocks, pgd_model** out);
/* The configuration a loader derives from a checkpoint (a directory: MLX;
 * a file: GGUF), without a device; no reference counterpart. */
int pgd_checkpoint_config(const char* path, int max_pos, int kv_blocks, pgd_model_config* cfg);
/* The configuration of a model (synthetic or loaded). */
int pgd_model_config_get(const pgd_model* m, pgd_model_config* cfg);
/* Arithmetic of a model's GGML-format matrices (the Qwen2 GGUF path). The
 * reference computes them two ways: candle's CPU quantized matmul
 * (PGD_ARITH_CPU_Q8, activations quantized to Q8_K / Q8_0; the default for
 * Qwen2 models, matching the reference CPU path's tokens) or dequantized
 * weights (Metal, qwen2_gguf.rs:280-289), here f32 dequant-then-dot
 * (PGD_ARITH_DEQUANT_F32). A8 (hybrid model) matrices are unaffected. */
enum { PGD_ARITH_DEQUANT_F32 = 0, PGD_ARITH_CPU_Q8 = 1 };
int pgd_model_set_kquant_arith(pgd_model* m, int mode);
/* No reference counterpart (the reference's Metal path encodes every kernel
 * of a token into one command buffer, qwen3_fuse.rs). on != 0: each step's
 * launches (embedding to argmax) are captured once per launch signature
 * (batch shape, buffers, attention plan layout) into a HIP graph and replayed
 * on later steps with the same signature; per-step data (tokens, positions,
 * page tables) is uploaded before the replay. Results are bitwise those of
 * the eager launches. The first step of a signature runs eagerly, the second
 * is captured. graph_stats: graphs held, replays so far. */
int pgd_model_set_graphs(pgd_model* m, int on);
int pgd_model_graph_stats(const pgd_model* m, int* graphs, long long* launches);
int pgd_model_free(pgd_model* m);
/* weight bytes on the device, algorithmic weight bytes per decode step, KV pages free */
int pgd_model_info(const pgd_model* m, size_t* weight_bytes, double* algo_bytes_per_token, int* kv_free);

/* ModelEngine::begin_session (pagoda/src/model.rs:78-80). */
int pgd_session_new(pgd_model* m, pgd_session** out);
/* ModelSession::fork (pagoda/src/model.rs:185-187): KV pages are shared
 * copy-on-write, the recurrent state is copied. */
int pgd_session_fork(const pgd_session* s, pgd_session** out);
int pgd_session_free(pgd_session* s);
/* ModelSession::context_len (pagoda/src/model.rs:165). */
int pgd_session_len(const pgd_session* s, int* len);
/* ModelSession::forward (pagoda/src/model.rs:167): feed n >= 0 tokens, write
 * the last position's logits [vocab] (n == 0 repeats the cached logits). */
int pgd_forward(pgd_session* s, const uint32_t* toks, int n, float* logits);
/* Qwen35::forward_greedy (pagoda-hf/src/qwen3_5.rs:511-530): one token in,
 * greedy id and its logit out (device argmax; ties keep the last max). */
int pgd_forward_greedy(pgd_session* s, uint32_t tok, uint32_t* id, float* logit);
/* Qwen35::forward_verify (pagoda-hf/src/qwen3_5.rs:663-755): n in 1..4
 * teacher-forced tokens, greedy id and logit per position. */
int pgd_forward_verify(pgd_session* s, const uint32_t* toks, int n, uint32_t* ids, float* logits_max);
/* Ragged batched step (ModelEngine::session_forward_batch,
 * pagoda/src/model.rs:88-94, widened to multi-token rows): session i feeds
 * n_per_seq[i] >= 1 tokens from toks (concatenated). ids receive the greedy
 * id (first max, pagoda/src/sampler.rs:59-69) of each session's last position
 * (all_rows = 0) or of every fed position (all_rows = 1); 0xFFFFFFFF marks a
 * row with any non-finite logit, which the engine faults
 * (pagoda/src/engine.rs:1278-1280: only that request, its batch-mates are
 * unaffected). logits (nullable) receive the matching rows [rows][vocab].
 * Atomic on argument errors: no session advances. A device error after the
 * step has begun writing (GDN state and KV pages are updated in place) marks
 * every session of the step unusable: later calls on them return
 * PGD_ERR_STATE instead of continuing from half-advanced state. */
int pgd_step_ragged(pgd_model* m, pgd_session* const* sessions, const uint32_t* toks, const int* n_per_seq,
                    int nseq, int all_rows, uint32_t* ids, float* logits);
/* ModelSession::export_kv / ModelEngine::import_session (pagoda/src/model.rs:
 * 137, 89). Hybrid model (arch 0): Qwen35Cache::to_bytes /
 * from_bytes, cache format v1 (pagoda-hf/src/qwen3_5.rs:177-256). Qwen2 (arch
 * 1): the SessionKv PD payload (CandleCausalLM::cache_export / cache_import,
 * pagoda-hf/src/llama.rs:215-345) with the session's last logits, which an
 * imported session replays on an empty feed (pagoda-hf/src/lib.rs:644-667).
 * export writes *len bytes when buf is large enough (pass buf = NULL to
 * query). */
int pgd_session_export(const pgd_session* s, uint8_t* buf, size_t cap, size_t* len);
int pgd_session_import(pgd_model* m, const uint8_t* buf, size_t len, pgd_session** out);
/* set_kv_wire_f16 (pagoda-hf/src/llama.rs:128-136): process-wide choice of the
 * SessionKv export's K/V encoding, f32 (0, default) or f16 (1). */
int pgd_set_kv_wire_f16(int on);
/* CandleCausalLM::cache_prefix (pagoda-hf/src/lib.rs:219-226;
 * qwen2_gguf.rs:183-185 -> SessionKv::prefix, llama.rs:81-101), used by
 * graft_session (lib.rs:603-616): a new session holding the first n
 * positions of s. KV pages below n are shared; the partial last page is
 * copied on the new session's first write, so appends never disturb s.
 * Cached logits are not carried (a graft has none, lib.rs:613).
 * PGD_ERR_STATE for the hybrid model: GDN state cannot be cut to a prefix
 * (the trait's default None, lib.rs:224). */
int pgd_session_fork_prefix(const pgd_session* s, int n, pgd_session** out);

/* ---- engine-addressable KV pages ------------------------------------------
 * The engine's PagedKvCache hands out physical BlockIds with reference counts
 * and copy-on-write, "exactly what a tensor-backed implementation would swap
 * in" (pagoda/src/kv_cache.rs:1-8, alloc/inc_ref/dec_ref/ref_count 65-105),
 * and its RadixCache maps each cached token to a KvSlot = (BlockId, offset)
 * (pagoda/src/radix_cache.rs:17-18). A page id here names one page of
 * kv_block positions in every full-attention layer's K and V pools; position
 * p of a session lives in slot p % kv_block of its page p / kv_block.
 * Sessions and the engine hold references alike; a page returns to the pool
 * when its count reaches zero, and a session copies a shared, partly filled
 * page before its first write into it. */
/* PagedKvCache::num_blocks / block_size / num_free_blocks (kv_cache.rs:48-56);
 * each output nullable. */
int pgd_model_kv_pool(const pgd_model* m, int* n_pages, int* page_tokens, int* n_free);
/* The page ids holding positions [0, len) of s, in position order. *n gets
 * the count (ids = NULL queries it); cap below it is PGD_ERR_ARG. */
int pgd_session_pages(const pgd_session* s, int32_t* ids, int cap, int* n);
/* PagedKvCache::inc_ref / dec_ref (kv_cache.rs:90-105) on n held pages (a free
 * page or an id outside the pool is an error and changes nothing). */
int pgd_page_retain(pgd_model* m, const int32_t* ids, int n);
int pgd_page_release(pgd_model* m, const int32_t* ids, int n);
/* PagedKvCache::ref_count (kv_cache.rs:74). */
int pgd_page_refcount(const pgd_model* m, int32_t id, int* count);
/* A new session of length n_pos whose KV is the held pages ids[0..n_pages)
 * (n_pages = ceil(n_pos / kv_block), distinct): the radix cache's matched
 * slots become the session's cache without a copy; the session takes its own
 * reference on each page. No cached logits (as a graft, lib.rs:603-616).
 * PGD_ERR_STATE for the hybrid model, whose recurrent state is not a
 * function of KV pages (cache_prefix default None, lib.rs:224). */
int pgd_session_from_pages(pgd_model* m, const int32_t* ids, int n_pages, int n_pos, pgd_session** out);

#ifdef __cplusplus
}
#endif
#endif
