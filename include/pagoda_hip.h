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

#ifdef __cplusplus
}
#endif
#endif
