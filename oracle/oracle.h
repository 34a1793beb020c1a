/*
 * oracle.h — CPU restatement of pagoda's decode path (TEST INFRASTRUCTURE).
 *
 * This library is the parity checker for the HIP backend. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only to check or time against; the product library never links it.
 *
 * Citations are path:line under the reference tree (quantz8a/pagoda).
 */
#ifndef PAGODA_ORACLE_H
#define PAGODA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp conversions (round to nearest even) ---- */
uint16_t ora_f32_to_bf16(float x);   /* pagoda-hf/src/qwen3_gemv.rs:570-574 */
float ora_bf16_to_f32(uint16_t h);   /* pagoda-hf/src/qwen3_5.rs:1718 */
uint16_t ora_f32_to_f16(float x);
float ora_f16_to_f32(uint16_t h);

/* ---- synthetic weights (seeded, counter based) ---- */
float ora_synth_normal(uint64_t seed, uint64_t key, uint64_t idx);
float ora_synth_uniform(uint64_t seed, uint64_t key, uint64_t idx);
void ora_synth_normal_fill(uint64_t seed, uint64_t key, float scale, float* out, size_t n);

/* ---- MLX affine 8-bit, group 64 ---- */
void ora_a8_quantize(const float* w, int n_out, int n_in, uint32_t* packed,
                     uint16_t* scales, uint16_t* biases);
void ora_a8_dequant(const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                    int row0, int rows, int n_in, float* out);

/* ---- GGML k-quants: 256-element super-blocks ---- */
#define ORA_QK 256
#define ORA_Q4K_BYTES 144
#define ORA_Q6K_BYTES 210
int ora_kq_blocks(int n_in); /* ceil(n_in / 256) */
void ora_q4k_quantize(const float* w, int n_out, int n_in, uint8_t* blocks);
void ora_q6k_quantize(const float* w, int n_out, int n_in, uint8_t* blocks);
void ora_q4k_dequant(const uint8_t* blocks, int row0, int rows, int n_in, float* out);
void ora_q6k_dequant(const uint8_t* blocks, int row0, int rows, int n_in, float* out);

/* ---- GGML 32-weight blocks (the fallback types of Q4_K_M files for rows
 * that are not whole 256-weight super-blocks) ---- */
#define ORA_Q8_0_BYTES 34
#define ORA_Q5_0_BYTES 22
void ora_q8_0_dequant(const uint8_t* blocks, int row0, int rows, int n_in, float* out);
void ora_q5_0_dequant(const uint8_t* blocks, int row0, int rows, int n_in, float* out);

/* ---- small ops ---- */
void ora_rms_zero(float* x, const float* w, int n);
void ora_rms_gated(float* x, const float* w, const float* gate, int n);
void ora_causal_conv(const float* x, int seq, int channels, int kernel, const float* weight,
                     float* state, float* out);
void ora_rope_cos_sin(int pos, int rotary_dim, float theta, float* cos_out, float* sin_out);
void ora_rope_inplace(float* x, const float* cos_t, const float* sin_t, int n);

/* ---- Gated-DeltaNet recurrent step for `seq` tokens of one sequence ----
 * conv_out [seq, conv_dim] (post conv+SiLU: q | k | v), a,b [seq, v_heads],
 * z [seq, v_heads*v_dim], state [v_heads, k_dim, v_dim] updated in place,
 * out [seq, v_heads*v_dim]. */
void ora_gdn_step(const float* conv_out, const float* a, const float* b, const float* z,
                  const float* a_log, const float* dt_bias, const float* norm, int seq,
                  int k_heads, int v_heads, int k_dim, int v_dim, float* state, float* out);

/* ---- single-query GQA attention over a contiguous [len, kv_heads, hd] cache ----
 * q [heads, hd]; out [heads, hd]; gate (nullable) [heads, hd] sigmoid gate. */
void ora_attn_decode(const float* q, const float* k_cache, const float* v_cache, int len,
                     int heads, int kv_heads, int hd, const float* gate, float* out);

/* ---- models ---- */
typedef struct {
  int n_layers, hidden, intermediate, vocab;
  int heads, kv_heads, head_dim, rotary_dim;
  float rope_theta;
  int k_heads, v_heads, k_dim, v_dim, conv_kernel;
  int full_every; /* layer i is full attention iff i % full_every == full_every-1 */
} ora_qwen35_config;

typedef struct {
  int n_layers, hidden, intermediate, vocab;
  int heads, kv_heads, head_dim, max_pos;
  float rope_theta, eps;
} ora_qwen2_config;

typedef struct ora_qwen35 ora_qwen35;
typedef struct ora_qwen35_cache ora_qwen35_cache;
typedef struct ora_qwen2 ora_qwen2;
typedef struct ora_qwen2_cache ora_qwen2_cache;

ora_qwen35* ora_qwen35_new(const ora_qwen35_config* cfg, uint64_t seed);
void ora_qwen35_free(ora_qwen35* m);
ora_qwen35_cache* ora_qwen35_cache_new(const ora_qwen35* m);
ora_qwen35_cache* ora_qwen35_cache_clone(const ora_qwen35_cache* c);
void ora_qwen35_cache_free(ora_qwen35_cache* c);
int ora_qwen35_cache_len(const ora_qwen35_cache* c);
/* Feed tokens; writes last-position logits [vocab]. Returns 0 on success. */
int ora_qwen35_forward(ora_qwen35* m, const uint32_t* toks, int n, ora_qwen35_cache* c,
                       float* logits);
/* Teacher-forced logits of every fed position, [n, vocab]. */
int ora_qwen35_forward_all(ora_qwen35* m, const uint32_t* toks, int n, ora_qwen35_cache* c,
                           float* logits_all);
/* Cache v1 bytes (pagoda-hf/src/qwen3_5.rs:177-206). Returns size; writes if buf != NULL. */
size_t ora_qwen35_cache_to_bytes(const ora_qwen35_cache* c, uint8_t* buf, size_t cap);
/* Cache v1 bytes -> cache (pagoda-hf/src/qwen3_5.rs:208-256); NULL on a malformed blob. */
ora_qwen35_cache* ora_qwen35_cache_from_bytes(const uint8_t* buf, size_t len);
/* Quantized tensor accessors for tests (pointers into the model). */
const void* ora_qwen35_tensor(const ora_qwen35* m, int layer, int kind, int part);

ora_qwen2* ora_qwen2_new(const ora_qwen2_config* cfg, uint64_t seed);
void ora_qwen2_free(ora_qwen2* m);
ora_qwen2_cache* ora_qwen2_cache_new(const ora_qwen2* m);
void ora_qwen2_cache_free(ora_qwen2_cache* c);
int ora_qwen2_cache_len(const ora_qwen2_cache* c);
/* SessionKv wire payload (pagoda-hf/src/llama.rs:215-345). export returns the
 * size and writes when buf != NULL; f16 selects the f16 wire (version 2,
 * dtype 1). import returns NULL on a malformed payload. */
size_t ora_qwen2_cache_export(const ora_qwen2* m, const ora_qwen2_cache* c, const float* logits, int n_logits,
                              int f16, uint8_t* buf, size_t cap);
ora_qwen2_cache* ora_qwen2_cache_import(const ora_qwen2* m, const uint8_t* buf, size_t len, float* logits_out,
                                        int logits_cap, int* n_logits);
int ora_qwen2_forward(ora_qwen2* m, const uint32_t* toks, int n, ora_qwen2_cache* c,
                      float* logits);
const void* ora_qwen2_tensor(const ora_qwen2* m, int layer, int kind, int part);
/* replace one matrix of the model by GGML blocks of format fmt (1 Q4_K,
 * 2 Q6_K, 3 Q8_0, 4 Q5_0), rows x n_in as before; returns 0 or -1 */
int ora_qwen2_set_matrix(ora_qwen2* m, int layer, int kind, int fmt, const uint8_t* blocks);

/* candle's CPU Q4_K/Q6_K matmul (activations quantized to Q8_K, integer
 * block dots): q8k blocks are 292 bytes (f32 d, 256 i8, 16 i16 bsums). */
void ora_q8k_quantize(const float* x, int n_in, uint8_t* out);
void ora_kq_vec_dot_q8k(int fmt, const uint8_t* blocks, int rows, int n_in, const uint8_t* q8k, float* y);
/* Q8_0 activations (34-byte blocks: f16 d, 32 i8) and the Q8_0 (fmt 3) /
 * Q5_0 (fmt 4) x Q8_0 block dots of the same kernel family. */
void ora_q8_0_quantize_act(const float* x, int n_in, uint8_t* out);
void ora_q8_0_vec_dot(int fmt, const uint8_t* blocks, int rows, int n_in, const uint8_t* q8, float* y);
/* 0: f32 dequant GEMV for every format (default); 1: candle's CPU quantized
 * matmul (Q4_K / Q6_K through Q8_K, Q8_0 / Q5_0 through Q8_0 activations). */
void ora_qwen2_set_kquant_mode(ora_qwen2* m, int mode);

/* greedy tie rule of the engine sampler: first max over finite values
 * (pagoda/src/sampler.rs:59-69). */
uint32_t ora_argmax_first(const float* x, int n);
/* y[i] = e^x[i] as the f32 paths evaluate it: the double exponential rounded once. */
void ora_exp_rows(const float* x, int n, float* y);

int ora_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
