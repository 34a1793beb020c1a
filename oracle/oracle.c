/*
 * oracle.c — CPU restatement of pagoda's decode path.
 *
 * TEST INFRASTRUCTURE ONLY: this is the parity checker for the HIP backend
 * (pagoda_amd/). It is loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, never by the product library.
 *
 * Each function cites the reference file:line it restates (paths relative to
 * the reference tree). Where the reference delegates to a third-party crate
 * that is absent (candle-core 0.8.4 for GGML k-quants, MLX for the affine
 * quantizer) the published algorithm is restated and marked as such.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off). Contraction is
 * off so every a*b-c in a dequant formula rounds twice, as written in C.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int ora_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------ */
/* fp conversions                                                      */
/* ------------------------------------------------------------------ */

/* pagoda-hf/src/qwen3_gemv.rs:570-574 (f32_to_bf16, round half to even). */
uint16_t ora_f32_to_bf16(float x) {
  uint32_t bits;
  memcpy(&bits, &x, 4);
  uint32_t round = 0x7fffu + ((bits >> 16) & 1u);
  uint64_t s = (uint64_t)bits + round;
  if (s > 0xffffffffull) s = 0xffffffffull; /* saturating_add */
  return (uint16_t)(s >> 16);
}

/* pagoda-hf/src/qwen3_5.rs:1718 (bf16_to_f32). */
float ora_bf16_to_f32(uint16_t h) {
  uint32_t bits = (uint32_t)h << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* IEEE binary16, round to nearest even (textbook; GGML stores d/dmin so). */
uint16_t ora_f32_to_f16(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  uint32_t sign = (b >> 16) & 0x8000u;
  uint32_t exp = (b >> 23) & 0xffu;
  uint32_t man = b & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    int shift = 14 - e;
    uint32_t half = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1u))) half++;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
  return (uint16_t)(sign | half);
}

float ora_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t man = (uint32_t)h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int e = -1;
      do { e++; man <<= 1; } while (!(man & 0x400u));
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* ------------------------------------------------------------------ */
/* synthetic weights                                                   */
/* ------------------------------------------------------------------ */
/* No reference counterpart: the reference loads checkpoints; the configs
 * ask for seeded N(0, s) weights. N(0,1) is the Irwin-Hall sum of 12
 * uniforms minus 6, with 16-bit uniforms drawn from splitmix64, computed in
 * integers so the GPU generator reproduces it bit for bit. */

static uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static uint64_t synth_stream(uint64_t seed, uint64_t key) { return splitmix64(seed ^ splitmix64(key)); }

float ora_synth_normal(uint64_t seed, uint64_t key, uint64_t idx) {
  uint64_t base = synth_stream(seed, key) + idx * 3u;
  int64_t s = 0;
  for (int j = 0; j < 3; ++j) {
    uint64_t h = splitmix64(base + (uint64_t)j);
    s += (int64_t)(h & 0xffffu) + (int64_t)((h >> 16) & 0xffffu) + (int64_t)((h >> 32) & 0xffffu) +
         (int64_t)(h >> 48);
  }
  int32_t t = (int32_t)(s - 393210); /* sum of (u+0.5)/65536 minus 6, times 65536 */
  return (float)t * (1.0f / 65536.0f);
}

float ora_synth_uniform(uint64_t seed, uint64_t key, uint64_t idx) {
  uint64_t h = splitmix64(synth_stream(seed, key) + idx * 3u);
  return (float)(uint32_t)(h >> 40) * (1.0f / 16777216.0f);
}

void ora_synth_normal_fill(uint64_t seed, uint64_t key, float scale, float* out, size_t n) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)n; ++i) out[i] = scale * ora_synth_normal(seed, key, (uint64_t)i);
}

/* ------------------------------------------------------------------ */
/* MLX affine 8-bit, group 64                                          */
/* ------------------------------------------------------------------ */
#define A8_GROUP 64

/* Quantizer: MLX's published affine_quantize algorithm (third-party, not in
 * the reference tree): per group, the larger-magnitude edge is mapped to an
 * exact code, scale = (max-min)/255 signed toward that edge, codes =
 * round-half-even((w - bias) / scale) clamped to [0,255]. Scales/biases are
 * stored as bf16 the way QuantMatrix::upload rounds them
 * (pagoda-hf/src/qwen3_gemv.rs:570-574). Pinned by the reference's MLX vector
 * pagoda-hf/src/qwen3_5.rs:1760-1777 (arange(64) -> 4093115391). */
void ora_a8_quantize(const float* w, int n_out, int n_in, uint32_t* packed, uint16_t* scales,
                     uint16_t* biases) {
  int groups = n_in / A8_GROUP;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < n_out; ++r) {
    for (int g = 0; g < groups; ++g) {
      const float* src = w + (size_t)r * n_in + (size_t)g * A8_GROUP;
      float mx = src[0], mn = src[0];
      for (int i = 1; i < A8_GROUP; ++i) {
        if (src[i] > mx) mx = src[i];
        if (src[i] < mn) mn = src[i];
      }
      int mask = fabsf(mn) > fabsf(mx);
      float scale = (mx - mn) / 255.0f;
      if (scale < 1e-7f) scale = 1e-7f;
      if (!mask) scale = -scale;
      float edge = mask ? mn : mx;
      float q0 = rintf(edge / scale);
      float bias = edge;
      if (q0 != 0.0f) {
        scale = edge / q0;
      } else {
        bias = 0.0f;
      }
      uint8_t* dst = (uint8_t*)(packed) + (size_t)r * n_in + (size_t)g * A8_GROUP;
      for (int i = 0; i < A8_GROUP; ++i) {
        float q = rintf((src[i] - bias) / scale);
        if (q < 0.0f) q = 0.0f;
        if (q > 255.0f) q = 255.0f;
        dst[i] = (uint8_t)q;
      }
      scales[(size_t)r * groups + g] = ora_f32_to_bf16(scale);
      biases[(size_t)r * groups + g] = ora_f32_to_bf16(bias);
    }
  }
}

/* pagoda-hf/src/qwen3_5.rs:1546-1584 (Affine::dequant_rows): codes are the
 * little-endian bytes of the packed u32 words; w = bias + scale * code. */
void ora_a8_dequant(const uint32_t* packed, const uint16_t* scales, const uint16_t* biases, int row0,
                    int rows, int n_in, float* out) {
  int words = n_in / 4, groups = n_in / A8_GROUP;
#pragma omp parallel for schedule(static) if (rows > 64)
  for (int r = 0; r < rows; ++r) {
    const uint32_t* row = packed + (size_t)(row0 + r) * words;
    const uint16_t* srow = scales + (size_t)(row0 + r) * groups;
    const uint16_t* brow = biases + (size_t)(row0 + r) * groups;
    float* o = out + (size_t)r * n_in;
    (void)words;
    /* code i is byte i % 4 of word i / 4, little-endian: on this
     * (little-endian) host, byte i of the row */
    const uint8_t* codes = (const uint8_t*)row;
    for (int g = 0; g < groups; ++g) {
      const float sc = ora_bf16_to_f32(srow[g]), bi = ora_bf16_to_f32(brow[g]);
      const uint8_t* cg = codes + (size_t)g * A8_GROUP;
      float* og = o + (size_t)g * A8_GROUP;
      for (int j = 0; j < A8_GROUP; ++j) og[j] = bi + sc * (float)cg[j];
    }
  }
}

/* ------------------------------------------------------------------ */
/* GGML k-quants (candle-core 0.8.4's k_quants, third party, absent)   */
/* ------------------------------------------------------------------ */
/* Block layouts are the public GGML ones:
 *   block_q4_K { f16 d; f16 dmin; u8 scales[12]; u8 qs[128]; }       144 B
 *   block_q6_K { u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d; }      210 B
 * A row of n_in weights is ceil(n_in/256) blocks; the tail past n_in is
 * quantized as zeros (K = 896 in the configs is 3.5 super-blocks). */

int ora_kq_blocks(int n_in) { return (n_in + ORA_QK - 1) / ORA_QK; }

static void q4k_get_scale_min(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
  }
}

static void q4k_put_scale_min(int j, uint8_t* q, uint8_t sc, uint8_t m) {
  if (j < 4) {
    q[j] = (uint8_t)((q[j] & 0xC0) | (sc & 63));
    q[j + 4] = (uint8_t)((q[j + 4] & 0xC0) | (m & 63));
  } else {
    q[j + 4] = (uint8_t)((sc & 0xF) | ((m & 0xF) << 4));
    q[j - 4] = (uint8_t)((q[j - 4] & 63) | ((sc >> 4) << 6));
    q[j] = (uint8_t)((q[j] & 63) | ((m >> 4) << 6));
  }
}

static float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Quantizer for the synthetic configs (the GGML layout is fixed; the
 * choice of scales is ours): per 32-wide sub-block, scale = (max - min0)/15
 * with min0 = min(0, min), super-scales d = max scale/63 and dmin = max
 * min/63 rounded to f16, 6-bit sub-scales and 4-bit codes rounded half-even. */
void ora_q4k_quantize(const float* w, int n_out, int n_in, uint8_t* blocks) {
  int nb = ora_kq_blocks(n_in);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < n_out; ++r) {
    for (int b = 0; b < nb; ++b) {
      float x[256];
      for (int i = 0; i < 256; ++i) {
        int k = b * 256 + i;
        x[i] = k < n_in ? w[(size_t)r * n_in + k] : 0.0f;
      }
      float scale[8], mins[8], maxs = 0.0f, maxm = 0.0f;
      for (int j = 0; j < 8; ++j) {
        float mn = 0.0f, mx = x[32 * j];
        for (int i = 0; i < 32; ++i) {
          float v = x[32 * j + i];
          if (v < mn) mn = v;
          if (v > mx) mx = v;
        }
        scale[j] = (mx - mn) / 15.0f;
        mins[j] = -mn;
        if (scale[j] > maxs) maxs = scale[j];
        if (mins[j] > maxm) maxm = mins[j];
      }
      uint8_t* blk = blocks + ((size_t)r * nb + b) * ORA_Q4K_BYTES;
      memset(blk, 0, ORA_Q4K_BYTES);
      uint16_t dh = ora_f32_to_f16(maxs / 63.0f), mh = ora_f32_to_f16(maxm / 63.0f);
      float d = ora_f16_to_f32(dh), dmin = ora_f16_to_f32(mh);
      blk[0] = (uint8_t)(dh & 255);
      blk[1] = (uint8_t)(dh >> 8);
      blk[2] = (uint8_t)(mh & 255);
      blk[3] = (uint8_t)(mh >> 8);
      uint8_t* sc = blk + 4;
      uint8_t* qs = blk + 16;
      uint8_t scq[8], mq[8];
      for (int j = 0; j < 8; ++j) {
        scq[j] = d > 0.0f ? (uint8_t)clampf(rintf(scale[j] / d), 0.0f, 63.0f) : 0;
        mq[j] = dmin > 0.0f ? (uint8_t)clampf(rintf(mins[j] / dmin), 0.0f, 63.0f) : 0;
        q4k_put_scale_min(j, sc, scq[j], mq[j]);
      }
      for (int j = 0; j < 8; ++j) {
        float ds = d * (float)scq[j];
        float dm = dmin * (float)mq[j];
        for (int i = 0; i < 32; ++i) {
          float q = ds > 0.0f ? clampf(rintf((x[32 * j + i] + dm) / ds), 0.0f, 15.0f) : 0.0f;
          int l = i, grp = j / 2;
          uint8_t v = (uint8_t)q;
          if (j % 2 == 0) qs[32 * grp + l] |= v;
          else qs[32 * grp + l] |= (uint8_t)(v << 4);
        }
      }
    }
  }
}

/* GGML dequantize_row_q4_K (public; candle-core k_quants restates it):
 * per 64 elements, d1 = d*sc, m1 = dmin*m; low nibbles then high nibbles,
 * y = d1*q - m1. */
void ora_q4k_dequant(const uint8_t* blocks, int row0, int rows, int n_in, float* out) {
  int nb = ora_kq_blocks(n_in);
#pragma omp parallel for schedule(static) if (rows > 64)
  for (int r = 0; r < rows; ++r) {
    float* o = out + (size_t)r * n_in;
    for (int b = 0; b < nb; ++b) {
      const uint8_t* blk = blocks + ((size_t)(row0 + r) * nb + b) * ORA_Q4K_BYTES;
      float d = ora_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
      float dmin = ora_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
      const uint8_t* sc = blk + 4;
      const uint8_t* q = blk + 16;
      int is = 0;
      for (int j = 0; j < 256; j += 64) {
        uint8_t s, m;
        q4k_get_scale_min(is + 0, sc, &s, &m);
        float d1 = d * (float)s, m1 = dmin * (float)m;
        q4k_get_scale_min(is + 1, sc, &s, &m);
        float d2 = d * (float)s, m2 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) {
          int k = b * 256 + j + l;
          if (k < n_in) o[k] = d1 * (float)(q[l] & 0xF) - m1;
        }
        for (int l = 0; l < 32; ++l) {
          int k = b * 256 + j + 32 + l;
          if (k < n_in) o[k] = d2 * (float)(q[l] >> 4) - m2;
        }
        q += 32;
        is += 2;
      }
    }
  }
}

/* Quantizer for the synthetic configs: per 16-wide sub-block scale =
 * max|w|/31, d = max scale/127 (f16), 8-bit sub-scales, 6-bit codes. */
void ora_q6k_quantize(const float* w, int n_out, int n_in, uint8_t* blocks) {
  int nb = ora_kq_blocks(n_in);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < n_out; ++r) {
    for (int b = 0; b < nb; ++b) {
      float x[256];
      for (int i = 0; i < 256; ++i) {
        int k = b * 256 + i;
        x[i] = k < n_in ? w[(size_t)r * n_in + k] : 0.0f;
      }
      float scale[16], maxs = 0.0f;
      for (int j = 0; j < 16; ++j) {
        float amax = 0.0f;
        for (int i = 0; i < 16; ++i) {
          float v = fabsf(x[16 * j + i]);
          if (v > amax) amax = v;
        }
        scale[j] = amax / 31.0f;
        if (scale[j] > maxs) maxs = scale[j];
      }
      uint8_t* blk = blocks + ((size_t)r * nb + b) * ORA_Q6K_BYTES;
      memset(blk, 0, ORA_Q6K_BYTES);
      uint8_t* ql = blk;
      uint8_t* qh = blk + 128;
      int8_t* sc = (int8_t*)(blk + 192);
      uint16_t dh = ora_f32_to_f16(maxs / 127.0f);
      float d = ora_f16_to_f32(dh);
      blk[208] = (uint8_t)(dh & 255);
      blk[209] = (uint8_t)(dh >> 8);
      uint8_t codes[256];
      for (int j = 0; j < 16; ++j) {
        int8_t s = d > 0.0f ? (int8_t)clampf(rintf(scale[j] / d), 0.0f, 127.0f) : 0;
        sc[j] = s;
        float ds = d * (float)s;
        for (int i = 0; i < 16; ++i) {
          float q = ds > 0.0f ? clampf(rintf(x[16 * j + i] / ds), -32.0f, 31.0f) : 0.0f;
          codes[16 * j + i] = (uint8_t)((int)q + 32);
        }
      }
      for (int n = 0; n < 2; ++n) {
        const uint8_t* c = codes + 128 * n;
        for (int l = 0; l < 32; ++l) {
          uint8_t q1 = c[l], q2 = c[l + 32], q3 = c[l + 64], q4 = c[l + 96];
          ql[64 * n + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
          ql[64 * n + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
          qh[32 * n + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
      }
    }
  }
}

/* GGML Q8_0 and Q5_0 blocks of 32 weights (the public GGML block formats,
 * which the reference reads through candle-core 0.8.4, pagoda-hf/Cargo.lock:
 * 165; not under /root/reference). Q8_0: f16 d, int8 q[32], y = q * d.
 * Q5_0: f16 d, 4 bytes qh (one little-endian u32 of high bits), 16 bytes qs;
 * for j < 16, y[j] = (((qs[j] & 15) | (bit j of qh) << 4) - 16) * d and
 * y[j + 16] = (((qs[j] >> 4) | (bit j + 16 of qh) << 4) - 16) * d.
 * Pinned by hand-built blocks with known values (tests/test_oracle_formats.py). */
void ora_q8_0_dequant(const uint8_t* blocks, int row0, int rows, int n_in, float* out) {
  const int nb = n_in / 32;
  for (int r = 0; r < rows; ++r)
    for (int b = 0; b < nb; ++b) {
      const uint8_t* blk = blocks + ((size_t)(row0 + r) * nb + b) * ORA_Q8_0_BYTES;
      const float d = ora_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
      for (int j = 0; j < 32; ++j) out[(size_t)r * n_in + 32 * b + j] = (float)(int8_t)blk[2 + j] * d;
    }
}

void ora_q5_0_dequant(const uint8_t* blocks, int row0, int rows, int n_in, float* out) {
  const int nb = n_in / 32;
  for (int r = 0; r < rows; ++r)
    for (int b = 0; b < nb; ++b) {
      const uint8_t* blk = blocks + ((size_t)(row0 + r) * nb + b) * ORA_Q5_0_BYTES;
      const float d = ora_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
      const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                          ((uint32_t)blk[5] << 24);
      float* o = out + (size_t)r * n_in + 32 * b;
      for (int j = 0; j < 16; ++j) {
        const int lo = (int)((blk[6 + j] & 15u) | (((qh >> j) & 1u) << 4)) - 16;
        const int hi = (int)((blk[6 + j] >> 4) | (((qh >> (j + 16)) & 1u) << 4)) - 16;
        o[j] = (float)lo * d;
        o[j + 16] = (float)hi * d;
      }
    }
}

/* GGML dequantize_row_q6_K (public): y = d * sc * (q - 32), q from the low
 * nibble plane ql and the 2-bit plane qh, 128 elements per half block. */
void ora_q6k_dequant(const uint8_t* blocks, int row0, int rows, int n_in, float* out) {
  int nb = ora_kq_blocks(n_in);
#pragma omp parallel for schedule(static) if (rows > 64)
  for (int r = 0; r < rows; ++r) {
    float* o = out + (size_t)r * n_in;
    for (int b = 0; b < nb; ++b) {
      const uint8_t* blk = blocks + ((size_t)(row0 + r) * nb + b) * ORA_Q6K_BYTES;
      const uint8_t* ql = blk;
      const uint8_t* qh = blk + 128;
      const int8_t* sc = (const int8_t*)(blk + 192);
      float d = ora_f16_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
      for (int n = 0; n < 256; n += 128) {
        for (int l = 0; l < 32; ++l) {
          int is = l / 16;
          int q1 = (int)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
          int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
          int q3 = (int)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
          int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
          int base = b * 256 + n;
          if (base + l < n_in) o[base + l] = d * (float)sc[is + 0] * (float)q1;
          if (base + l + 32 < n_in) o[base + l + 32] = d * (float)sc[is + 2] * (float)q2;
          if (base + l + 64 < n_in) o[base + l + 64] = d * (float)sc[is + 4] * (float)q3;
          if (base + l + 96 < n_in) o[base + l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        ql += 64;
        qh += 32;
        sc += 8;
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* small ops                                                            */
/* ------------------------------------------------------------------ */

/* pagoda-hf/src/qwen3_5.rs:1736-1745 (rms_zero, eps 1e-6). */
void ora_rms_zero(float* x, const float* w, int n) {
  float ss = 0.0f;
  for (int i = 0; i < n; ++i) ss += x[i] * x[i];
  float inv = 1.0f / sqrtf(ss / (float)n + 1e-6f);
  for (int i = 0; i < n; ++i) x[i] = x[i] * inv * w[i];
}

/* e^x for the f32 paths: the double-precision exponential rounded once to
 * f32, i.e. the correctly rounded f32 value (the reference calls the
 * platform's f32 exp, Rust f32::exp -> libm expf, which every libm returns
 * within one ulp of it; glibc's and macOS's expf differ from it by one ulp on
 * a small fraction of inputs). The GPU path evaluates it the same way. */
static float ora_expf(float x) { return (float)exp((double)x); }
void ora_exp_rows(const float* x, int n, float* y) {
  for (int i = 0; i < n; ++i) y[i] = ora_expf(x[i]);
}

static float silu(float x) { return x / (1.0f + ora_expf(-x)); }       /* qwen3_5.rs:1758 */
static float sigmoidf_(float x) { return 1.0f / (1.0f + ora_expf(-x)); } /* qwen3_5.rs:1762 */
static float softplus(float x) {                                     /* qwen3_5.rs:1766-1774 */
  if (x > 20.0f) return x;
  if (x < -20.0f) return ora_expf(x);
  return logf(1.0f + ora_expf(x));
}

/* pagoda-hf/src/qwen3_5.rs:1747-1756 (rms_gated). */
void ora_rms_gated(float* x, const float* w, const float* gate, int n) {
  float ss = 0.0f;
  for (int i = 0; i < n; ++i) ss += x[i] * x[i];
  float inv = 1.0f / sqrtf(ss / (float)n + 1e-6f);
  for (int i = 0; i < n; ++i) x[i] = x[i] * inv * w[i] * silu(gate[i]);
}

/* pagoda-hf/src/qwen3_5.rs:1800-1853 (causal_conv): depthwise conv over
 * [state | x] with weight[c*kernel+k], SiLU, then the last kernel-1 inputs
 * become the state [channels, kernel-1]. */
void ora_causal_conv(const float* x, int seq, int channels, int kernel, const float* weight,
                     float* state, float* out) {
  int hist = kernel - 1;
  for (int t = 0; t < seq; ++t) {
    for (int c = 0; c < channels; ++c) {
      float acc = 0.0f;
      for (int k = 0; k < kernel; ++k) {
        int src = t - hist + k;
        float sample;
        if (src < 0) {
          int idx = hist + src;
          sample = idx < 0 ? 0.0f : state[c * hist + idx];
        } else {
          sample = x[(size_t)src * channels + c];
        }
        acc += sample * weight[c * kernel + k];
      }
      out[(size_t)t * channels + c] = silu(acc);
    }
  }
  if (seq >= hist) {
    for (int c = 0; c < channels; ++c)
      for (int k = 0; k < hist; ++k) state[c * hist + k] = x[(size_t)(seq - hist + k) * channels + c];
  } else {
    int keep = hist;
    float* window = (float*)malloc(sizeof(float) * (size_t)(keep + seq));
    for (int c = 0; c < channels; ++c) {
      for (int k = 0; k < keep; ++k) window[k] = state[c * keep + k];
      for (int t = 0; t < seq; ++t) window[keep + t] = x[(size_t)t * channels + c];
      for (int k = 0; k < keep; ++k) state[c * keep + k] = window[seq + k];
    }
    free(window);
  }
}

/* pagoda-hf/src/qwen3_5.rs:1855-1870 (rope_cos_sin). */
void ora_rope_cos_sin(int pos, int rotary_dim, float theta, float* cos_out, float* sin_out) {
  int half = rotary_dim / 2;
  for (int i = 0; i < half; ++i) {
    float freq = 1.0f / powf(theta, (float)(2 * i) / (float)rotary_dim);
    float ang = (float)pos * freq;
    float c = cosf(ang), s = sinf(ang);
    cos_out[i] = c;
    cos_out[half + i] = c;
    sin_out[i] = s;
    sin_out[half + i] = s;
  }
}

/* pagoda-hf/src/qwen3_5.rs:1872-1883 (rope_inplace, rotate-half over the
 * first n entries). */
void ora_rope_inplace(float* x, const float* cos_t, const float* sin_t, int n) {
  int half = n / 2;
  float rot[512];
  for (int i = 0; i < half; ++i) {
    rot[i] = -x[half + i];
    rot[half + i] = x[i];
  }
  for (int i = 0; i < n; ++i) x[i] = x[i] * cos_t[i] + rot[i] * sin_t[i];
}

static void l2norm_heads(float* x, int heads, int dim) { /* qwen3_5.rs:1786-1798 */
  for (int h = 0; h < heads; ++h) {
    float* row = x + (size_t)h * dim;
    float ss = 0.0f;
    for (int i = 0; i < dim; ++i) ss += row[i] * row[i];
    float inv = 1.0f / sqrtf(ss + 1e-6f);
    for (int i = 0; i < dim; ++i) row[i] *= inv;
  }
}

/* ------------------------------------------------------------------ */
/* Gated-DeltaNet recurrence                                            */
/* ------------------------------------------------------------------ */
/* pagoda-hf/src/qwen3_5.rs:1330-1383 (LinearAttn::forward, per-token loop
 * after the causal conv). */
void ora_gdn_step(const float* conv_out, const float* a, const float* b, const float* z,
                  const float* a_log, const float* dt_bias, const float* norm, int seq, int k_heads,
                  int v_heads, int k_dim, int v_dim, float* state, float* out) {
  int key_dim = k_heads * k_dim, value_dim = v_heads * v_dim;
  int conv_dim = 2 * key_dim + value_dim;
  int repeat = v_heads / k_heads;
  float* qh = (float*)malloc(sizeof(float) * (size_t)v_heads * k_dim);
  float* kh = (float*)malloc(sizeof(float) * (size_t)v_heads * k_dim);
  float* mem = (float*)malloc(sizeof(float) * (size_t)v_dim);
  float* delta = (float*)malloc(sizeof(float) * (size_t)v_dim);
  for (int t = 0; t < seq; ++t) {
    const float* q = conv_out + (size_t)t * conv_dim;
    const float* k = q + key_dim;
    const float* v = q + 2 * key_dim;
    for (int h = 0; h < k_heads; ++h)
      for (int rr = 0; rr < repeat; ++rr) {
        memcpy(qh + (size_t)(h * repeat + rr) * k_dim, q + (size_t)h * k_dim, sizeof(float) * k_dim);
        memcpy(kh + (size_t)(h * repeat + rr) * k_dim, k + (size_t)h * k_dim, sizeof(float) * k_dim);
      }
    l2norm_heads(qh, v_heads, k_dim);
    l2norm_heads(kh, v_heads, k_dim);
    float scale = sqrtf((float)k_dim);
    for (int i = 0; i < v_heads * k_dim; ++i) qh[i] /= scale;
    for (int h = 0; h < v_heads; ++h) {
      float g = -ora_expf(a_log[h]) * softplus(a[t * v_heads + h] + dt_bias[h]);
      float decay = ora_expf(g);
      float beta = sigmoidf_(b[t * v_heads + h]);
      const float* qv = qh + (size_t)h * k_dim;
      const float* kv = kh + (size_t)h * k_dim;
      const float* vv = v + (size_t)h * v_dim;
      float* st = state + (size_t)h * k_dim * v_dim;
      for (int i = 0; i < k_dim * v_dim; ++i) st[i] *= decay;
      for (int j = 0; j < v_dim; ++j) mem[j] = 0.0f;
      for (int ki = 0; ki < k_dim; ++ki)
        for (int j = 0; j < v_dim; ++j) mem[j] += st[ki * v_dim + j] * kv[ki];
      for (int j = 0; j < v_dim; ++j) delta[j] = (vv[j] - mem[j]) * beta;
      for (int ki = 0; ki < k_dim; ++ki)
        for (int j = 0; j < v_dim; ++j) st[ki * v_dim + j] += kv[ki] * delta[j];
      float* o = out + (size_t)t * value_dim + (size_t)h * v_dim;
      for (int j = 0; j < v_dim; ++j) o[j] = 0.0f;
      for (int ki = 0; ki < k_dim; ++ki)
        for (int j = 0; j < v_dim; ++j) o[j] += st[ki * v_dim + j] * qv[ki];
      ora_rms_gated(o, norm, z + (size_t)t * value_dim + (size_t)h * v_dim, v_dim);
    }
  }
  free(qh);
  free(kh);
  free(mem);
  free(delta);
}

/* ------------------------------------------------------------------ */
/* attention                                                            */
/* ------------------------------------------------------------------ */
/* pagoda-hf/src/qwen3_5.rs:1433-1475 (FullAttn::forward scores/softmax/
 * weighted sum, score = dot / sqrt(hd), optional sigmoid gate). With
 * gate == NULL this is the Qwen2 decode row (pagoda-hf/src/qwen2_gguf.rs:
 * 252-266 at one query position). */
void ora_attn_decode(const float* q, const float* k_cache, const float* v_cache, int len, int heads,
                     int kv_heads, int hd, const float* gate, float* out) {
  int groups = heads / kv_heads;
  float scale = sqrtf((float)hd);
  float* scores = (float*)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1));
  for (int h = 0; h < heads; ++h) {
    int kvh = h / groups;
    const float* qh = q + (size_t)h * hd;
    float max_s = -INFINITY;
    for (int p = 0; p < len; ++p) {
      const float* kh = k_cache + ((size_t)p * kv_heads + kvh) * hd;
      float dot = 0.0f;
      for (int i = 0; i < hd; ++i) dot += qh[i] * kh[i];
      float s = dot / scale;
      scores[p] = s;
      if (s > max_s) max_s = s;
    }
    float sum = 0.0f;
    for (int p = 0; p < len; ++p) {
      scores[p] = ora_expf(scores[p] - max_s);
      sum += scores[p];
    }
    float* oh = out + (size_t)h * hd;
    for (int i = 0; i < hd; ++i) oh[i] = 0.0f;
    for (int p = 0; p < len; ++p) {
      const float* vh = v_cache + ((size_t)p * kv_heads + kvh) * hd;
      float w = scores[p] / sum;
      for (int i = 0; i < hd; ++i) oh[i] += w * vh[i];
    }
    if (gate)
      for (int i = 0; i < hd; ++i) oh[i] *= sigmoidf_(gate[(size_t)h * hd + i]);
  }
  free(scores);
}

/* pagoda/src/sampler.rs:59-69 */
uint32_t ora_argmax_first(const float* x, int n) {
  int best = 0;
  float bv = -INFINITY;
  for (int i = 0; i < n; ++i)
    if (isfinite(x[i]) && x[i] > bv) {
      bv = x[i];
      best = i;
    }
  return (uint32_t)best;
}

/* ------------------------------------------------------------------ */
/* candle's CPU k-quant matmul: activations quantized to Q8_K            */
/* ------------------------------------------------------------------ */
/* On the CPU the reference keeps candle's quantized matmul for the Q4_K /
 * Q6_K weights (pagoda-hf/src/qwen2_gguf.rs:280-289, QMatMul::from_qtensor):
 * each activation row is quantized to the weight type's vec_dot_type, Q8_K
 * (block_q8_K { f32 d; i8 qs[256]; i16 bsums[16]; }), and every output is an
 * integer block dot scaled in f32. candle-core 0.8.4 (pagoda-hf/Cargo.lock:
 * 165, not vendored here) restates GGML's published k-quant routines in
 * quantized/k_quants.rs; this follows them:
 *   BlockQ8K::from_float  = quantize_row_q8_K: amax = max|x| (first index
 *     wins), max = the signed value there, iscale = -128/max,
 *     q = min(127, round(iscale*x)) (round half away from zero, Rust's
 *     f32::round), bsums = sums of 16, d = 1/iscale; amax 0 gives d 0, q 0.
 *   BlockQ4K::vec_dot    = ggml_vec_dot_q4_K_q8_K (scalar form);
 *   BlockQ6K::vec_dot    = ggml_vec_dot_q6_K_q8_K (scalar form).
 * The integer parts are exact; SIMD builds (AVX2, NEON) sum the per-block f32
 * terms in other orders, so a CPU build agrees with this to f32 rounding. */
typedef struct {
  float d;
  int8_t qs[256];
  int16_t bsums[16];
} q8k_block;

static void q8k_quantize_block(const float* x, q8k_block* y) {
  float amax = 0.0f, max = 0.0f;
  for (int j = 0; j < 256; ++j) {
    float ax = fabsf(x[j]);
    if (amax < ax) {
      amax = ax;
      max = x[j];
    }
  }
  if (amax == 0.0f) {
    memset(y, 0, sizeof *y);
    return;
  }
  float iscale = -128.0f / max;
  for (int j = 0; j < 256; ++j) {
    float v = roundf(iscale * x[j]);
    y->qs[j] = (int8_t)(v < 127.0f ? v : 127.0f);
  }
  for (int j = 0; j < 16; ++j) {
    int sum = 0;
    for (int i = 0; i < 16; ++i) sum += y->qs[16 * j + i];
    y->bsums[j] = (int16_t)sum;
  }
  y->d = 1.0f / iscale;
}

/* One row of n_in activations (tail past n_in as zeros) -> nb Q8_K blocks,
 * written as d (f32), qs (256 i8), bsums (16 i16) per block, 292 bytes. */
void ora_q8k_quantize(const float* x, int n_in, uint8_t* out) {
  int nb = ora_kq_blocks(n_in);
  for (int b = 0; b < nb; ++b) {
    float t[256];
    for (int i = 0; i < 256; ++i) t[i] = b * 256 + i < n_in ? x[b * 256 + i] : 0.0f;
    q8k_block y;
    q8k_quantize_block(t, &y);
    memcpy(out + (size_t)b * 292, &y.d, 4);
    memcpy(out + (size_t)b * 292 + 4, y.qs, 256);
    memcpy(out + (size_t)b * 292 + 260, y.bsums, 32);
  }
}

static void q8k_unpack(const uint8_t* in, q8k_block* y) {
  memcpy(&y->d, in, 4);
  memcpy(y->qs, in + 4, 256);
  memcpy(y->bsums, in + 260, 32);
}

static float vec_dot_q4k_q8k(const uint8_t* xb, const q8k_block* y, int nb) {
  float sums[8] = {0}, sumf = 0.0f;
  for (int i = 0; i < nb; ++i) {
    const uint8_t* blk = xb + (size_t)i * ORA_Q4K_BYTES;
    const uint8_t* q4 = blk + 16;
    const int8_t* q8 = y[i].qs;
    int8_t aux8[256];
    int32_t aux32[8] = {0};
    for (int j = 0; j < 4; ++j) {
      for (int l = 0; l < 32; ++l) aux8[64 * j + l] = (int8_t)(q4[32 * j + l] & 0xF);
      for (int l = 0; l < 32; ++l) aux8[64 * j + 32 + l] = (int8_t)(q4[32 * j + l] >> 4);
    }
    uint8_t scales[8], mins[8];
    for (int j = 0; j < 8; ++j) q4k_get_scale_min(j, blk + 4, &scales[j], &mins[j]);
    int sumi = 0;
    for (int j = 0; j < 16; ++j) sumi += y[i].bsums[j] * mins[j / 2];
    const int8_t* a = aux8;
    for (int j = 0; j < 8; ++j) {
      int32_t scale = scales[j];
      for (int part = 0; part < 4; ++part) {
        for (int l = 0; l < 8; ++l) aux32[l] += scale * (int16_t)(q8[l] * a[l]);
        q8 += 8;
        a += 8;
      }
    }
    float d = ora_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8))) * y[i].d;
    for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
    float dmin = ora_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8))) * y[i].d;
    sumf -= dmin * (float)sumi;
  }
  for (int l = 0; l < 8; ++l) sumf += sums[l];
  return sumf;
}

static float vec_dot_q6k_q8k(const uint8_t* xb, const q8k_block* y, int nb) {
  float sums[8] = {0}, sumf = 0.0f;
  for (int i = 0; i < nb; ++i) {
    const uint8_t* blk = xb + (size_t)i * ORA_Q6K_BYTES;
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    const int8_t* q8 = y[i].qs;
    int8_t aux8[256];
    int32_t aux32[8] = {0};
    for (int h = 0; h < 2; ++h) {
      int8_t* a = aux8 + 128 * h;
      const uint8_t* q4 = ql + 64 * h;
      const uint8_t* qq = qh + 32 * h;
      for (int l = 0; l < 32; ++l) {
        a[l + 0] = (int8_t)(((q4[l + 0] & 0xF) | (((qq[l] >> 0) & 3) << 4)) - 32);
        a[l + 32] = (int8_t)(((q4[l + 32] & 0xF) | (((qq[l] >> 2) & 3) << 4)) - 32);
        a[l + 64] = (int8_t)(((q4[l + 0] >> 4) | (((qq[l] >> 4) & 3) << 4)) - 32);
        a[l + 96] = (int8_t)(((q4[l + 32] >> 4) | (((qq[l] >> 6) & 3) << 4)) - 32);
      }
    }
    const int8_t* a = aux8;
    for (int j = 0; j < 16; ++j) {
      int scale = sc[j];
      for (int part = 0; part < 2; ++part) {
        for (int l = 0; l < 8; ++l) aux32[l] += scale * (int16_t)(q8[l] * a[l]);
        q8 += 8;
        a += 8;
      }
    }
    uint16_t dh;
    memcpy(&dh, blk + 208, 2);
    float d = ora_f16_to_f32(dh) * y[i].d;
    for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
  }
  for (int l = 0; l < 8; ++l) sumf += sums[l];
  return sumf;
}

/* fmt 1 (Q4_K) / 2 (Q6_K): y[r] = vec_dot(row r's blocks, q8k) for rows rows. */
void ora_kq_vec_dot_q8k(int fmt, const uint8_t* blocks, int rows, int n_in, const uint8_t* q8k, float* y) {
  int nb = ora_kq_blocks(n_in);
  q8k_block* yb = (q8k_block*)malloc(sizeof(q8k_block) * (size_t)nb);
  for (int b = 0; b < nb; ++b) q8k_unpack(q8k + (size_t)b * 292, &yb[b]);
  size_t bb = fmt == 1 ? ORA_Q4K_BYTES : ORA_Q6K_BYTES;
  for (int r = 0; r < rows; ++r)
    y[r] = fmt == 1 ? vec_dot_q4k_q8k(blocks + (size_t)r * nb * bb, yb, nb)
                    : vec_dot_q6k_q8k(blocks + (size_t)r * nb * bb, yb, nb);
  free(yb);
}

/* The 32-weight types' vec_dot_type is Q8_0 (block_q8_0 { f16 d; i8 qs[32]; }):
 * BlockQ8_0::from_float = quantize_row_q8_0: amax = max|x|, d = amax/127,
 * id = 1/d (0 when d is 0), q = round(x*id) (half away from zero), d stored
 * as f16. vec_dot_q8_0_q8_0 / vec_dot_q5_0_q8_0 (scalar forms): per block
 * sumi = integer dot (Q5_0 codes are the nibble with its qh bit as bit 4,
 * minus 16), then sumf += sumi * d_w * d_x in f32 over the blocks in order. */
static void q8_0_quantize_block(const float* x, uint16_t* dh, int8_t* qs) {
  float amax = 0.0f;
  for (int j = 0; j < 32; ++j) {
    float ax = fabsf(x[j]);
    if (ax > amax) amax = ax;
  }
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  for (int j = 0; j < 32; ++j) qs[j] = (int8_t)roundf(x[j] * id);
  *dh = ora_f32_to_f16(d);
}

/* One row (n_in % 32 == 0) -> n_in/32 blocks of 34 bytes (f16 d, 32 i8). */
void ora_q8_0_quantize_act(const float* x, int n_in, uint8_t* out) {
  for (int b = 0; b < n_in / 32; ++b) {
    uint16_t dh;
    q8_0_quantize_block(x + 32 * b, &dh, (int8_t*)(out + (size_t)b * 34 + 2));
    memcpy(out + (size_t)b * 34, &dh, 2);
  }
}

static float vec_dot_q8_0_q8_0(const uint8_t* xb, const uint8_t* yb, int nb) {
  float sumf = 0.0f;
  for (int b = 0; b < nb; ++b) {
    const uint8_t* x = xb + (size_t)b * ORA_Q8_0_BYTES;
    const uint8_t* y = yb + (size_t)b * 34;
    int sumi = 0;
    for (int j = 0; j < 32; ++j) sumi += (int)(int8_t)x[2 + j] * (int)(int8_t)y[2 + j];
    sumf += (float)sumi * ora_f16_to_f32((uint16_t)(x[0] | (x[1] << 8))) * ora_f16_to_f32((uint16_t)(y[0] | (y[1] << 8)));
  }
  return sumf;
}

static float vec_dot_q5_0_q8_0(const uint8_t* xb, const uint8_t* yb, int nb) {
  float sumf = 0.0f;
  for (int b = 0; b < nb; ++b) {
    const uint8_t* x = xb + (size_t)b * ORA_Q5_0_BYTES;
    const uint8_t* y = yb + (size_t)b * 34;
    const uint32_t qh = (uint32_t)x[2] | ((uint32_t)x[3] << 8) | ((uint32_t)x[4] << 16) | ((uint32_t)x[5] << 24);
    int sumi = 0;
    for (int j = 0; j < 16; ++j) {
      const int x0 = (int)((x[6 + j] & 15u) | (((qh >> j) & 1u) << 4)) - 16;
      const int x1 = (int)((x[6 + j] >> 4) | (((qh >> (j + 16)) & 1u) << 4)) - 16;
      sumi += x0 * (int)(int8_t)y[2 + j] + x1 * (int)(int8_t)y[2 + j + 16];
    }
    sumf += (float)sumi * ora_f16_to_f32((uint16_t)(x[0] | (x[1] << 8))) * ora_f16_to_f32((uint16_t)(y[0] | (y[1] << 8)));
  }
  return sumf;
}

/* fmt 3 (Q8_0) / 4 (Q5_0): y[r] = vec_dot(row r's blocks, q8_0 activation blocks). */
void ora_q8_0_vec_dot(int fmt, const uint8_t* blocks, int rows, int n_in, const uint8_t* q8, float* y) {
  const int nb = n_in / 32;
  const size_t bb = fmt == 3 ? ORA_Q8_0_BYTES : ORA_Q5_0_BYTES;
  for (int r = 0; r < rows; ++r)
    y[r] = fmt == 3 ? vec_dot_q8_0_q8_0(blocks + (size_t)r * nb * bb, q8, nb)
                    : vec_dot_q5_0_q8_0(blocks + (size_t)r * nb * bb, q8, nb);
}

/* 0: f32 dequant-then-dot (the Metal/hybrid arithmetic, config 2's check);
 * 1: candle's CPU quantized matmul: Q4_K/Q6_K through Q8_K activations,
 *    Q8_0/Q5_0 through Q8_0 activations. */
static int g_kquant_mode = 0;

/* ------------------------------------------------------------------ */
/* quantized matrices                                                   */
/* ------------------------------------------------------------------ */
enum { FMT_A8 = 0, FMT_Q4K = 1, FMT_Q6K = 2, FMT_Q8_0 = 3, FMT_Q5_0 = 4 };

typedef struct {
  int fmt, n_out, n_in;
  uint32_t* packed; /* A8 */
  uint16_t* scales;
  uint16_t* biases;
  uint8_t* blocks; /* Q4K/Q6K */
} qmat;

/* Tensor keys of the synthetic generator: (layer << 8) | kind, layer 0xFFFF
 * for model-global tensors. Shared by the GPU generator. */
enum {
  K_EMBED = 1, K_HEAD = 2, K_FINAL_NORM = 3,
  K_IN_NORM = 10, K_POST_NORM = 11, K_GATE = 12, K_UP = 13, K_DOWN = 14,
  K_QKV = 20, K_Z = 21, K_A = 22, K_B = 23, K_OUT = 24, K_CONV = 25, K_ALOG = 26, K_DTB = 27,
  K_GNORM = 28,
  K_Q = 30, K_K = 31, K_V = 32, K_O = 33, K_QNORM = 34, K_KNORM = 35, K_QB = 36, K_KB = 37, K_VB = 38
};

static uint64_t tkey(int layer, int kind) {
  return ((uint64_t)(layer < 0 ? 0xFFFF : layer) << 8) | (uint64_t)kind;
}

static qmat qmat_synth(uint64_t seed, uint64_t key, int fmt, int n_out, int n_in) {
  qmat m;
  memset(&m, 0, sizeof m);
  m.fmt = fmt;
  m.n_out = n_out;
  m.n_in = n_in;
  float* w = (float*)malloc(sizeof(float) * (size_t)n_out * n_in);
  ora_synth_normal_fill(seed, key, 0.02f, w, (size_t)n_out * n_in);
  if (fmt == FMT_A8) {
    m.packed = (uint32_t*)malloc((size_t)n_out * n_in);
    m.scales = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n_out * (n_in / 64));
    m.biases = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n_out * (n_in / 64));
    ora_a8_quantize(w, n_out, n_in, m.packed, m.scales, m.biases);
  } else if (fmt == FMT_Q4K) {
    m.blocks = (uint8_t*)malloc((size_t)n_out * ora_kq_blocks(n_in) * ORA_Q4K_BYTES);
    ora_q4k_quantize(w, n_out, n_in, m.blocks);
  } else {
    m.blocks = (uint8_t*)malloc((size_t)n_out * ora_kq_blocks(n_in) * ORA_Q6K_BYTES);
    ora_q6k_quantize(w, n_out, n_in, m.blocks);
  }
  free(w);
  return m;
}

static void qmat_free(qmat* m) {
  free(m->packed);
  free(m->scales);
  free(m->biases);
  free(m->blocks);
}

static void qmat_dequant(const qmat* m, int row0, int rows, float* out) {
  if (m->fmt == FMT_A8) ora_a8_dequant(m->packed, m->scales, m->biases, row0, rows, m->n_in, out);
  else if (m->fmt == FMT_Q4K) ora_q4k_dequant(m->blocks, row0, rows, m->n_in, out);
  else if (m->fmt == FMT_Q6K) ora_q6k_dequant(m->blocks, row0, rows, m->n_in, out);
  else if (m->fmt == FMT_Q8_0) ora_q8_0_dequant(m->blocks, row0, rows, m->n_in, out);
  else ora_q5_0_dequant(m->blocks, row0, rows, m->n_in, out);
}

static const void* qmat_part(const qmat* m, int part) {
  if (m->fmt == FMT_A8) return part == 0 ? (const void*)m->packed : part == 1 ? (const void*)m->scales : (const void*)m->biases;
  return m->blocks;
}

/* y[seq, n_out] = x[seq, n_in] . W^T with W dequantized per row chunk and a
 * sequential f32 dot per output (pagoda-hf/src/qwen3_5.rs:1137-1161 logits
 * loop; linear() at 1163-1179 goes through a dequantized f32 matmul). */
static void qmat_linear(const qmat* m, const float* x, int seq, float* y) {
  const int chunk = 256;
  if (g_kquant_mode == 1 && (m->fmt == FMT_Q4K || m->fmt == FMT_Q6K)) {
    int nb = ora_kq_blocks(m->n_in);
    size_t bb = m->fmt == FMT_Q4K ? ORA_Q4K_BYTES : ORA_Q6K_BYTES;
    for (int t = 0; t < seq; ++t) {
      q8k_block* yb = (q8k_block*)malloc(sizeof(q8k_block) * (size_t)nb);
      const float* xv = x + (size_t)t * m->n_in;
      for (int b = 0; b < nb; ++b) {
        float tb[256];
        for (int i = 0; i < 256; ++i) tb[i] = b * 256 + i < m->n_in ? xv[b * 256 + i] : 0.0f;
        q8k_quantize_block(tb, &yb[b]);
      }
#pragma omp parallel for schedule(static)
      for (int r = 0; r < m->n_out; ++r)
        y[(size_t)t * m->n_out + r] = m->fmt == FMT_Q4K ? vec_dot_q4k_q8k(m->blocks + (size_t)r * nb * bb, yb, nb)
                                                        : vec_dot_q6k_q8k(m->blocks + (size_t)r * nb * bb, yb, nb);
      free(yb);
    }
    return;
  }
  if (g_kquant_mode == 1 && (m->fmt == FMT_Q8_0 || m->fmt == FMT_Q5_0)) {
    const int nb = m->n_in / 32;
    const size_t bb = m->fmt == FMT_Q8_0 ? ORA_Q8_0_BYTES : ORA_Q5_0_BYTES;
    uint8_t* q8 = (uint8_t*)malloc((size_t)nb * 34);
    for (int t = 0; t < seq; ++t) {
      ora_q8_0_quantize_act(x + (size_t)t * m->n_in, m->n_in, q8);
#pragma omp parallel for schedule(static)
      for (int r = 0; r < m->n_out; ++r)
        y[(size_t)t * m->n_out + r] = m->fmt == FMT_Q8_0 ? vec_dot_q8_0_q8_0(m->blocks + (size_t)r * nb * bb, q8, nb)
                                                         : vec_dot_q5_0_q8_0(m->blocks + (size_t)r * nb * bb, q8, nb);
    }
    free(q8);
    return;
  }
  int n_out = m->n_out, n_in = m->n_in;
  /* R output rows at a time: their dequantized weights transposed to
   * [n_in][R] so the R dot products advance together (one SIMD lane
   * each). Every output is still the sequential sum over i = 0..n_in-1 of
   * x[i]*w[i], rounded after each product and each add, in that order. */
  (void)chunk;
  /* 32 rows (16 for long rows, to stay in L2): several independent 8-wide
   * accumulator chains per i */
  const int R = n_in <= 8192 ? 32 : 16;
#pragma omp parallel
  {
    float* rows = (float*)malloc(sizeof(float) * (size_t)R * n_in);
    float* wt = (float*)malloc(sizeof(float) * (size_t)R * n_in);
#pragma omp for schedule(dynamic, 16)
    for (int c0 = 0; c0 < n_out; c0 += R) {
      int n = n_out - c0 < R ? n_out - c0 : R;
      qmat_dequant(m, c0, n, rows);
      for (int i = 0; i < n_in; ++i)
        for (int r = 0; r < R; ++r) wt[(size_t)i * R + r] = r < n ? rows[(size_t)r * n_in + i] : 0.0f;
      for (int t = 0; t < seq; ++t) {
        const float* xv = x + (size_t)t * n_in;
        float acc[32] = {0};
        if (R == 32) {
          for (int i = 0; i < n_in; ++i) {
            const float xi = xv[i];
            const float* w = wt + (size_t)i * 32;
            for (int r = 0; r < 32; ++r) acc[r] += xi * w[r];
          }
        } else {
          for (int i = 0; i < n_in; ++i) {
            const float xi = xv[i];
            const float* w = wt + (size_t)i * 16;
            for (int r = 0; r < 16; ++r) acc[r] += xi * w[r];
          }
        }
        for (int r = 0; r < n; ++r) y[(size_t)t * n_out + c0 + r] = acc[r];
      }
    }
    free(rows);
    free(wt);
  }
}

static float* vec_synth_normal(uint64_t seed, uint64_t key, float scale, size_t n) {
  float* v = (float*)malloc(sizeof(float) * n);
  ora_synth_normal_fill(seed, key, scale, v, n);
  return v;
}

static float* vec_const(float c, size_t n) {
  float* v = (float*)malloc(sizeof(float) * n);
  for (size_t i = 0; i < n; ++i) v[i] = c;
  return v;
}

/* ------------------------------------------------------------------ */
/* Qwen3.5 hybrid (pagoda-hf/src/qwen3_5.rs)                            */
/* ------------------------------------------------------------------ */
typedef struct {
  int full;
  float *in_norm, *post_norm;
  qmat gate, up, down;
  /* linear attention */
  qmat qkv, z, a, b, out;
  float *conv, *a_log, *dt_bias, *gnorm;
  /* full attention */
  qmat q, k, v, o;
  float *q_norm, *k_norm;
} q35_layer;

struct ora_qwen35 {
  ora_qwen35_config cfg;
  int conv_dim;
  qmat embed, head;
  float* final_norm;
  q35_layer* layers;
};

typedef struct {
  int full;
  float *k, *v; /* [cap, kv_heads, hd] */
  int cap;
  float* conv;  /* [conv_dim, kernel-1] */
  float* state; /* [v_heads, k_dim, v_dim] */
} q35_cache_layer;

struct ora_qwen35_cache {
  int n_layers, len, kv_width, kv_heads, head_dim, conv_n, state_n;
  q35_cache_layer* layers;
};

static int q35_is_full(const ora_qwen35_config* c, int i) { return i % c->full_every == c->full_every - 1; }

/* Synthetic init for the configs: N(0,0.02) matrices, unit norms,
 * A_log = ln(16)*U so A ~ exp(U(0, ln 16)) in [1,16), dt_bias 0.1*N, conv
 * 0.2*N. The tensor set and shapes follow Qwen35::load
 * (pagoda-hf/src/qwen3_5.rs:338-452). */
ora_qwen35* ora_qwen35_new(const ora_qwen35_config* cfg, uint64_t seed) {
  ora_qwen35* m = (ora_qwen35*)calloc(1, sizeof *m);
  m->cfg = *cfg;
  const ora_qwen35_config* c = cfg;
  int key_dim = c->k_heads * c->k_dim, value_dim = c->v_heads * c->v_dim;
  m->conv_dim = 2 * key_dim + value_dim;
  m->embed = qmat_synth(seed, tkey(-1, K_EMBED), FMT_A8, c->vocab, c->hidden);
  m->head = qmat_synth(seed, tkey(-1, K_HEAD), FMT_A8, c->vocab, c->hidden);
  m->final_norm = vec_const(1.0f, c->hidden);
  m->layers = (q35_layer*)calloc((size_t)c->n_layers, sizeof(q35_layer));
  for (int i = 0; i < c->n_layers; ++i) {
    q35_layer* L = &m->layers[i];
    L->full = q35_is_full(c, i);
    L->in_norm = vec_const(1.0f, c->hidden);
    L->post_norm = vec_const(1.0f, c->hidden);
    L->gate = qmat_synth(seed, tkey(i, K_GATE), FMT_A8, c->intermediate, c->hidden);
    L->up = qmat_synth(seed, tkey(i, K_UP), FMT_A8, c->intermediate, c->hidden);
    L->down = qmat_synth(seed, tkey(i, K_DOWN), FMT_A8, c->hidden, c->intermediate);
    if (!L->full) {
      L->qkv = qmat_synth(seed, tkey(i, K_QKV), FMT_A8, m->conv_dim, c->hidden);
      L->z = qmat_synth(seed, tkey(i, K_Z), FMT_A8, value_dim, c->hidden);
      L->a = qmat_synth(seed, tkey(i, K_A), FMT_A8, c->v_heads, c->hidden);
      L->b = qmat_synth(seed, tkey(i, K_B), FMT_A8, c->v_heads, c->hidden);
      L->out = qmat_synth(seed, tkey(i, K_OUT), FMT_A8, c->hidden, value_dim);
      L->conv = vec_synth_normal(seed, tkey(i, K_CONV), 0.2f, (size_t)m->conv_dim * c->conv_kernel);
      L->a_log = (float*)malloc(sizeof(float) * c->v_heads);
      for (int h = 0; h < c->v_heads; ++h)
        L->a_log[h] = 2.7725887f * ora_synth_uniform(seed, tkey(i, K_ALOG), (uint64_t)h);
      L->dt_bias = vec_synth_normal(seed, tkey(i, K_DTB), 0.1f, c->v_heads);
      L->gnorm = vec_const(1.0f, c->v_dim);
    } else {
      L->q = qmat_synth(seed, tkey(i, K_Q), FMT_A8, c->heads * c->head_dim * 2, c->hidden);
      L->k = qmat_synth(seed, tkey(i, K_K), FMT_A8, c->kv_heads * c->head_dim, c->hidden);
      L->v = qmat_synth(seed, tkey(i, K_V), FMT_A8, c->kv_heads * c->head_dim, c->hidden);
      L->o = qmat_synth(seed, tkey(i, K_O), FMT_A8, c->hidden, c->heads * c->head_dim);
      L->q_norm = vec_const(1.0f, c->head_dim);
      L->k_norm = vec_const(1.0f, c->head_dim);
    }
  }
  return m;
}

void ora_qwen35_free(ora_qwen35* m) {
  if (!m) return;
  qmat_free(&m->embed);
  qmat_free(&m->head);
  free(m->final_norm);
  for (int i = 0; i < m->cfg.n_layers; ++i) {
    q35_layer* L = &m->layers[i];
    free(L->in_norm);
    free(L->post_norm);
    qmat_free(&L->gate);
    qmat_free(&L->up);
    qmat_free(&L->down);
    qmat_free(&L->qkv);
    qmat_free(&L->z);
    qmat_free(&L->a);
    qmat_free(&L->b);
    qmat_free(&L->out);
    qmat_free(&L->q);
    qmat_free(&L->k);
    qmat_free(&L->v);
    qmat_free(&L->o);
    free(L->conv);
    free(L->a_log);
    free(L->dt_bias);
    free(L->gnorm);
    free(L->q_norm);
    free(L->k_norm);
  }
  free(m->layers);
  free(m);
}

const void* ora_qwen35_tensor(const ora_qwen35* m, int layer, int kind, int part) {
  if (layer < 0) {
    if (kind == K_EMBED) return qmat_part(&m->embed, part);
    if (kind == K_HEAD) return qmat_part(&m->head, part);
    if (kind == K_FINAL_NORM) return m->final_norm;
    return NULL;
  }
  const q35_layer* L = &m->layers[layer];
  switch (kind) {
    case K_IN_NORM: return L->in_norm;
    case K_POST_NORM: return L->post_norm;
    case K_GATE: return qmat_part(&L->gate, part);
    case K_UP: return qmat_part(&L->up, part);
    case K_DOWN: return qmat_part(&L->down, part);
    case K_QKV: return qmat_part(&L->qkv, part);
    case K_Z: return qmat_part(&L->z, part);
    case K_A: return qmat_part(&L->a, part);
    case K_B: return qmat_part(&L->b, part);
    case K_OUT: return qmat_part(&L->out, part);
    case K_CONV: return L->conv;
    case K_ALOG: return L->a_log;
    case K_DTB: return L->dt_bias;
    case K_GNORM: return L->gnorm;
    case K_Q: return qmat_part(&L->q, part);
    case K_K: return qmat_part(&L->k, part);
    case K_V: return qmat_part(&L->v, part);
    case K_O: return qmat_part(&L->o, part);
    case K_QNORM: return L->q_norm;
    case K_KNORM: return L->k_norm;
  }
  return NULL;
}

/* pagoda-hf/src/qwen3_5.rs:466-503 (new_cache). */
ora_qwen35_cache* ora_qwen35_cache_new(const ora_qwen35* m) {
  const ora_qwen35_config* c = &m->cfg;
  ora_qwen35_cache* cc = (ora_qwen35_cache*)calloc(1, sizeof *cc);
  cc->n_layers = c->n_layers;
  cc->kv_width = c->kv_heads * c->head_dim;
  cc->kv_heads = c->kv_heads;
  cc->head_dim = c->head_dim;
  cc->conv_n = m->conv_dim * (c->conv_kernel - 1);
  cc->state_n = c->v_heads * c->k_dim * c->v_dim;
  cc->layers = (q35_cache_layer*)calloc((size_t)c->n_layers, sizeof(q35_cache_layer));
  for (int i = 0; i < c->n_layers; ++i) {
    q35_cache_layer* L = &cc->layers[i];
    L->full = q35_is_full(c, i);
    if (!L->full) {
      L->conv = (float*)calloc((size_t)cc->conv_n, sizeof(float));
      L->state = (float*)calloc((size_t)cc->state_n, sizeof(float));
    }
  }
  return cc;
}

ora_qwen35_cache* ora_qwen35_cache_clone(const ora_qwen35_cache* s) {
  ora_qwen35_cache* cc = (ora_qwen35_cache*)calloc(1, sizeof *cc);
  *cc = *s;
  cc->layers = (q35_cache_layer*)calloc((size_t)s->n_layers, sizeof(q35_cache_layer));
  for (int i = 0; i < s->n_layers; ++i) {
    const q35_cache_layer* a = &s->layers[i];
    q35_cache_layer* L = &cc->layers[i];
    L->full = a->full;
    if (a->full) {
      L->cap = a->cap;
      if (a->cap) {
        L->k = (float*)malloc(sizeof(float) * (size_t)a->cap * s->kv_width);
        L->v = (float*)malloc(sizeof(float) * (size_t)a->cap * s->kv_width);
        memcpy(L->k, a->k, sizeof(float) * (size_t)s->len * s->kv_width);
        memcpy(L->v, a->v, sizeof(float) * (size_t)s->len * s->kv_width);
      }
    } else {
      L->conv = (float*)malloc(sizeof(float) * (size_t)s->conv_n);
      L->state = (float*)malloc(sizeof(float) * (size_t)s->state_n);
      memcpy(L->conv, a->conv, sizeof(float) * (size_t)s->conv_n);
      memcpy(L->state, a->state, sizeof(float) * (size_t)s->state_n);
    }
  }
  return cc;
}

void ora_qwen35_cache_free(ora_qwen35_cache* c) {
  if (!c) return;
  for (int i = 0; i < c->n_layers; ++i) {
    free(c->layers[i].k);
    free(c->layers[i].v);
    free(c->layers[i].conv);
    free(c->layers[i].state);
  }
  free(c->layers);
  free(c);
}

int ora_qwen35_cache_len(const ora_qwen35_cache* c) { return c->len; }

static void put_u32(uint8_t* b, size_t* at, size_t cap, uint32_t v) {
  if (b && *at + 4 <= cap) memcpy(b + *at, &v, 4);
  *at += 4;
}

static void put_f32s(uint8_t* b, size_t* at, size_t cap, const float* v, uint32_t n) {
  put_u32(b, at, cap, n);
  if (b && *at + (size_t)n * 4 <= cap && n) memcpy(b + *at, v, (size_t)n * 4);
  *at += (size_t)n * 4;
}

/* pagoda-hf/src/qwen3_5.rs:177-206 (Qwen35Cache::to_bytes, format v1). */
size_t ora_qwen35_cache_to_bytes(const ora_qwen35_cache* c, uint8_t* buf, size_t cap) {
  size_t at = 0;
  put_u32(buf, &at, cap, 1);
  uint64_t len = (uint64_t)c->len;
  if (buf && at + 8 <= cap) memcpy(buf + at, &len, 8);
  at += 8;
  put_u32(buf, &at, cap, (uint32_t)c->n_layers);
  for (int i = 0; i < c->n_layers; ++i) {
    const q35_cache_layer* L = &c->layers[i];
    if (L->full) {
      if (buf && at < cap) buf[at] = 2;
      at += 1;
      int kv_heads_hd = c->kv_width;
      put_u32(buf, &at, cap, (uint32_t)c->len);
      put_u32(buf, &at, cap, (uint32_t)c->kv_heads);
      put_u32(buf, &at, cap, (uint32_t)c->head_dim);
      put_f32s(buf, &at, cap, L->k, (uint32_t)(c->len * kv_heads_hd));
      put_f32s(buf, &at, cap, L->v, (uint32_t)(c->len * kv_heads_hd));
    } else {
      if (buf && at < cap) buf[at] = 1;
      at += 1;
      put_f32s(buf, &at, cap, L->conv, (uint32_t)c->conv_n);
      put_f32s(buf, &at, cap, L->state, (uint32_t)c->state_n);
    }
  }
  return at;
}

static int take_bytes(const uint8_t* b, size_t n, size_t* at, void* dst, size_t k) {
  if (*at + k > n) return -1;
  memcpy(dst, b + *at, k);
  *at += k;
  return 0;
}

/* take_f32 (counted f32 vector): u32 count, then count f32 LE. Returns a
 * malloc'd array (NULL for count 0) through *out, -1 when truncated. */
static int take_f32s(const uint8_t* b, size_t n, size_t* at, float** out, uint32_t* count) {
  uint32_t c;
  if (take_bytes(b, n, at, &c, 4)) return -1;
  if ((size_t)c * 4 > n - *at) return -1;
  *count = c;
  *out = NULL;
  if (c) {
    *out = (float*)malloc((size_t)c * 4);
    memcpy(*out, b + *at, (size_t)c * 4);
  }
  *at += (size_t)c * 4;
  return 0;
}

/* pagoda-hf/src/qwen3_5.rs:208-256 (Qwen35Cache::from_bytes): version 1,
 * tags 1 (linear: conv, state) and 2 (full: kv_len, kv_heads, head_dim, k,
 * v with |k| == |v| == kv_len*kv_heads*head_dim), no trailing bytes. This
 * cache keeps one conv/state/KV geometry for all layers, so it also rejects
 * layers of differing sizes and a kv_len other than the cache length, which
 * a model-written cache never has. Returns NULL on any error. */
ora_qwen35_cache* ora_qwen35_cache_from_bytes(const uint8_t* b, size_t n) {
  size_t at = 0;
  uint32_t version, n_layers;
  uint64_t len;
  if (take_bytes(b, n, &at, &version, 4) || version != 1) return NULL;
  if (take_bytes(b, n, &at, &len, 8) || take_bytes(b, n, &at, &n_layers, 4)) return NULL;
  if (len > (1u << 30) || n_layers > (1u << 16)) return NULL;
  ora_qwen35_cache* cc = (ora_qwen35_cache*)calloc(1, sizeof *cc);
  cc->n_layers = (int)n_layers;
  cc->len = (int)len;
  cc->conv_n = cc->state_n = cc->kv_heads = cc->head_dim = -1;
  cc->layers = (q35_cache_layer*)calloc(n_layers ? n_layers : 1, sizeof(q35_cache_layer));
  for (uint32_t i = 0; i < n_layers; ++i) {
    q35_cache_layer* L = &cc->layers[i];
    uint8_t tag;
    if (take_bytes(b, n, &at, &tag, 1)) goto bad;
    if (tag == 2) {
      uint32_t kv_len, kvh, hd, nk, nv;
      if (take_bytes(b, n, &at, &kv_len, 4) || take_bytes(b, n, &at, &kvh, 4) ||
          take_bytes(b, n, &at, &hd, 4))
        goto bad;
      L->full = 1;
      if (take_f32s(b, n, &at, &L->k, &nk) || take_f32s(b, n, &at, &L->v, &nv)) goto bad;
      if ((uint64_t)kv_len * kvh * hd != nk || nk != nv) goto bad;
      if (kv_len != len) goto bad;
      if (cc->kv_heads < 0) {
        cc->kv_heads = (int)kvh;
        cc->head_dim = (int)hd;
      } else if (cc->kv_heads != (int)kvh || cc->head_dim != (int)hd) {
        goto bad;
      }
      L->cap = (int)kv_len;
    } else if (tag == 1) {
      uint32_t nc, ns;
      if (take_f32s(b, n, &at, &L->conv, &nc) || take_f32s(b, n, &at, &L->state, &ns)) goto bad;
      if (cc->conv_n < 0) {
        cc->conv_n = (int)nc;
        cc->state_n = (int)ns;
      } else if (cc->conv_n != (int)nc || cc->state_n != (int)ns) {
        goto bad;
      }
    } else {
      goto bad;
    }
  }
  if (at != n) goto bad;
  if (cc->kv_heads < 0) cc->kv_heads = cc->head_dim = 0;
  if (cc->conv_n < 0) cc->conv_n = cc->state_n = 0;
  cc->kv_width = cc->kv_heads * cc->head_dim;
  return cc;
bad:
  ora_qwen35_cache_free(cc);
  return NULL;
}

/* pagoda-hf/src/qwen3_5.rs:1313-1385 (LinearAttn::forward). */
static void q35_linear_attn(const ora_qwen35* m, const q35_layer* L, const float* x, int seq,
                            q35_cache_layer* cl, float* y) {
  const ora_qwen35_config* c = &m->cfg;
  int value_dim = c->v_heads * c->v_dim;
  float* qkv = (float*)malloc(sizeof(float) * (size_t)seq * m->conv_dim);
  float* z = (float*)malloc(sizeof(float) * (size_t)seq * value_dim);
  float* a = (float*)malloc(sizeof(float) * (size_t)seq * c->v_heads);
  float* b = (float*)malloc(sizeof(float) * (size_t)seq * c->v_heads);
  qmat_linear(&L->qkv, x, seq, qkv);
  qmat_linear(&L->z, x, seq, z);
  qmat_linear(&L->b, x, seq, b);
  qmat_linear(&L->a, x, seq, a);
  float* conv_out = (float*)malloc(sizeof(float) * (size_t)seq * m->conv_dim);
  ora_causal_conv(qkv, seq, m->conv_dim, c->conv_kernel, L->conv, cl->conv, conv_out);
  float* outputs = (float*)calloc((size_t)seq * value_dim, sizeof(float));
  ora_gdn_step(conv_out, a, b, z, L->a_log, L->dt_bias, L->gnorm, seq, c->k_heads, c->v_heads, c->k_dim,
               c->v_dim, cl->state, outputs);
  qmat_linear(&L->out, outputs, seq, y);
  free(qkv);
  free(z);
  free(a);
  free(b);
  free(conv_out);
  free(outputs);
}

/* pagoda-hf/src/qwen3_5.rs:1389-1478 (FullAttn::forward). */
static void q35_full_attn(const ora_qwen35* m, const q35_layer* L, const float* x, int seq, int pos0,
                          q35_cache_layer* cl, int cache_len, float* y) {
  const ora_qwen35_config* c = &m->cfg;
  int hd = c->head_dim, H = c->heads, KVH = c->kv_heads;
  int qout = H * hd * 2, kvw = KVH * hd;
  float* q_all = (float*)malloc(sizeof(float) * (size_t)seq * qout);
  float* k_all = (float*)malloc(sizeof(float) * (size_t)seq * kvw);
  float* v_all = (float*)malloc(sizeof(float) * (size_t)seq * kvw);
  qmat_linear(&L->q, x, seq, q_all);
  qmat_linear(&L->k, x, seq, k_all);
  qmat_linear(&L->v, x, seq, v_all);
  float* attn_out = (float*)calloc((size_t)seq * H * hd, sizeof(float));
  float* q = (float*)malloc(sizeof(float) * (size_t)H * hd);
  float* gate = (float*)malloc(sizeof(float) * (size_t)H * hd);
  float cs[512], sn[512];
  int need = cache_len + seq;
  if (need > cl->cap) {
    int cap = cl->cap ? cl->cap : 16;
    while (cap < need) cap *= 2;
    cl->k = (float*)realloc(cl->k, sizeof(float) * (size_t)cap * kvw);
    cl->v = (float*)realloc(cl->v, sizeof(float) * (size_t)cap * kvw);
    cl->cap = cap;
  }
  for (int t = 0; t < seq; ++t) {
    const float* raw = q_all + (size_t)t * qout;
    for (int h = 0; h < H; ++h) {
      memcpy(q + (size_t)h * hd, raw + (size_t)h * 2 * hd, sizeof(float) * hd);
      memcpy(gate + (size_t)h * hd, raw + (size_t)h * 2 * hd + hd, sizeof(float) * hd);
      ora_rms_zero(q + (size_t)h * hd, L->q_norm, hd);
    }
    float* k = cl->k + (size_t)(cache_len + t) * kvw;
    float* v = cl->v + (size_t)(cache_len + t) * kvw;
    memcpy(k, k_all + (size_t)t * kvw, sizeof(float) * kvw);
    memcpy(v, v_all + (size_t)t * kvw, sizeof(float) * kvw);
    for (int h = 0; h < KVH; ++h) ora_rms_zero(k + (size_t)h * hd, L->k_norm, hd);
    ora_rope_cos_sin(pos0 + t, c->rotary_dim, c->rope_theta, cs, sn);
    for (int h = 0; h < H; ++h) ora_rope_inplace(q + (size_t)h * hd, cs, sn, c->rotary_dim);
    for (int h = 0; h < KVH; ++h) ora_rope_inplace(k + (size_t)h * hd, cs, sn, c->rotary_dim);
    ora_attn_decode(q, cl->k, cl->v, cache_len + t + 1, H, KVH, hd, gate, attn_out + (size_t)t * H * hd);
  }
  qmat_linear(&L->o, attn_out, seq, y);
  free(q_all);
  free(k_all);
  free(v_all);
  free(attn_out);
  free(q);
  free(gate);
}

static float silu_(float x) { return silu(x); }

/* pagoda-hf/src/qwen3_5.rs:1193-1250 (Layer::forward, CPU branch). */
static void q35_layer_forward(const ora_qwen35* m, int li, float* x, int seq, int pos0,
                              q35_cache_layer* cl, int cache_len) {
  const ora_qwen35_config* c = &m->cfg;
  const q35_layer* L = &m->layers[li];
  int H = c->hidden, I = c->intermediate;
  float* normed = (float*)malloc(sizeof(float) * (size_t)seq * H);
  memcpy(normed, x, sizeof(float) * (size_t)seq * H);
  for (int t = 0; t < seq; ++t) ora_rms_zero(normed + (size_t)t * H, L->in_norm, H);
  float* mixed = (float*)malloc(sizeof(float) * (size_t)seq * H);
  if (L->full) q35_full_attn(m, L, normed, seq, pos0, cl, cache_len, mixed);
  else q35_linear_attn(m, L, normed, seq, cl, mixed);
  for (size_t i = 0; i < (size_t)seq * H; ++i) x[i] += mixed[i];
  memcpy(normed, x, sizeof(float) * (size_t)seq * H);
  for (int t = 0; t < seq; ++t) ora_rms_zero(normed + (size_t)t * H, L->post_norm, H);
  float* g = (float*)malloc(sizeof(float) * (size_t)seq * I);
  float* u = (float*)malloc(sizeof(float) * (size_t)seq * I);
  qmat_linear(&L->gate, normed, seq, g);
  qmat_linear(&L->up, normed, seq, u);
  for (size_t i = 0; i < (size_t)seq * I; ++i) g[i] = silu_(g[i]) * u[i];
  qmat_linear(&L->down, g, seq, mixed);
  for (size_t i = 0; i < (size_t)seq * H; ++i) x[i] += mixed[i];
  free(normed);
  free(mixed);
  free(g);
  free(u);
}

/* pagoda-hf/src/qwen3_5.rs:847-893 (forward_hidden) + 1137-1161 (logits).
 * Returns logits of the last position. */
static int q35_forward_rows(ora_qwen35* m, const uint32_t* toks, int n, ora_qwen35_cache* cc,
                            float* logits) {
  const ora_qwen35_config* c = &m->cfg;
  int H = c->hidden;
  if (n <= 0) return -1;
  for (int i = 0; i < n; ++i)
    if ((int)toks[i] >= c->vocab) return -2;
  float* x = (float*)malloc(sizeof(float) * (size_t)n * H);
  for (int i = 0; i < n; ++i) qmat_dequant(&m->embed, (int)toks[i], 1, x + (size_t)i * H);
  int pos0 = cc->len;
  for (int li = 0; li < c->n_layers; ++li) q35_layer_forward(m, li, x, n, pos0, &cc->layers[li], cc->len);
  for (int t = 0; t < n; ++t) ora_rms_zero(x + (size_t)t * H, m->final_norm, H);
  qmat_linear(&m->head, x + (size_t)(n - 1) * H, 1, logits);
  cc->len += n;
  free(x);
  return 0;
}

int ora_qwen35_forward(ora_qwen35* m, const uint32_t* toks, int n, ora_qwen35_cache* c, float* logits) {
  return q35_forward_rows(m, toks, n, c, logits);
}

/* Teacher-forced logits at every fed position. Fed one token at a time,
 * which the reference's verify path must equal (pagoda-hf/examples/
 * qwen3_8.rs:219-247). */
int ora_qwen35_forward_all(ora_qwen35* m, const uint32_t* toks, int n, ora_qwen35_cache* c,
                           float* logits_all) {
  for (int i = 0; i < n; ++i) {
    int rc = q35_forward_rows(m, toks + i, 1, c, logits_all + (size_t)i * m->cfg.vocab);
    if (rc) return rc;
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* Qwen2 GGUF (pagoda-hf/src/qwen2_gguf.rs)                             */
/* ------------------------------------------------------------------ */
typedef struct {
  float *attn_norm, *ffn_norm, *qb, *kb, *vb;
  qmat q, k, v, o, gate, up, down;
} q2_layer;

struct ora_qwen2 {
  ora_qwen2_config cfg;
  int kquant_mode; /* qmat_linear arithmetic of this model's GGML matrices (see g_kquant_mode) */
  qmat embed; /* token_embd (Q6K), also the tied lm_head */
  float* final_norm;
  q2_layer* layers;
  float *cos_t, *sin_t; /* [max_pos, hd/2] */
};

struct ora_qwen2_cache {
  int n_layers, len, cap, kvw;
  float** k; /* per layer [cap, kv_heads, hd] */
  float** v;
};

/* Q4_K_M-style type choice of the configs: Q6_K for attn_v, ffn_down on even
 * layers and token_embd; Q4_K elsewhere. Norm weights 1, q/k/v biases
 * 0.02*N. Shapes follow Qwen2Gguf::load (pagoda-hf/src/qwen2_gguf.rs:65-140). */
ora_qwen2* ora_qwen2_new(const ora_qwen2_config* cfg, uint64_t seed) {
  ora_qwen2* m = (ora_qwen2*)calloc(1, sizeof *m);
  m->cfg = *cfg;
  const ora_qwen2_config* c = cfg;
  int hd = c->head_dim;
  m->embed = qmat_synth(seed, tkey(-1, K_EMBED), FMT_Q6K, c->vocab, c->hidden);
  m->final_norm = vec_const(1.0f, c->hidden);
  m->layers = (q2_layer*)calloc((size_t)c->n_layers, sizeof(q2_layer));
  for (int i = 0; i < c->n_layers; ++i) {
    q2_layer* L = &m->layers[i];
    L->attn_norm = vec_const(1.0f, c->hidden);
    L->ffn_norm = vec_const(1.0f, c->hidden);
    L->q = qmat_synth(seed, tkey(i, K_Q), FMT_Q4K, c->heads * hd, c->hidden);
    L->k = qmat_synth(seed, tkey(i, K_K), FMT_Q4K, c->kv_heads * hd, c->hidden);
    L->v = qmat_synth(seed, tkey(i, K_V), FMT_Q6K, c->kv_heads * hd, c->hidden);
    L->o = qmat_synth(seed, tkey(i, K_O), FMT_Q4K, c->hidden, c->heads * hd);
    L->gate = qmat_synth(seed, tkey(i, K_GATE), FMT_Q4K, c->intermediate, c->hidden);
    L->up = qmat_synth(seed, tkey(i, K_UP), FMT_Q4K, c->intermediate, c->hidden);
    L->down = qmat_synth(seed, tkey(i, K_DOWN), i % 2 == 0 ? FMT_Q6K : FMT_Q4K, c->hidden, c->intermediate);
    L->qb = vec_synth_normal(seed, tkey(i, K_QB), 0.02f, (size_t)c->heads * hd);
    L->kb = vec_synth_normal(seed, tkey(i, K_KB), 0.02f, (size_t)c->kv_heads * hd);
    L->vb = vec_synth_normal(seed, tkey(i, K_VB), 0.02f, (size_t)c->kv_heads * hd);
  }
  /* pagoda-hf/src/qwen2_gguf.rs:327-344 (rope_tables): theta_i =
   * 1/base^(i/hd) for even i; freqs = pos * theta in f32. */
  int half = hd / 2;
  m->cos_t = (float*)malloc(sizeof(float) * (size_t)c->max_pos * half);
  m->sin_t = (float*)malloc(sizeof(float) * (size_t)c->max_pos * half);
  for (int j = 0; j < half; ++j) {
    float theta = 1.0f / powf(c->rope_theta, (float)(2 * j) / (float)hd);
    for (int p = 0; p < c->max_pos; ++p) {
      float f = (float)p * theta;
      m->cos_t[(size_t)p * half + j] = cosf(f);
      m->sin_t[(size_t)p * half + j] = sinf(f);
    }
  }
  return m;
}

void ora_qwen2_free(ora_qwen2* m) {
  if (!m) return;
  qmat_free(&m->embed);
  free(m->final_norm);
  for (int i = 0; i < m->cfg.n_layers; ++i) {
    q2_layer* L = &m->layers[i];
    free(L->attn_norm);
    free(L->ffn_norm);
    free(L->qb);
    free(L->kb);
    free(L->vb);
    qmat_free(&L->q);
    qmat_free(&L->k);
    qmat_free(&L->v);
    qmat_free(&L->o);
    qmat_free(&L->gate);
    qmat_free(&L->up);
    qmat_free(&L->down);
  }
  free(m->layers);
  free(m->cos_t);
  free(m->sin_t);
  free(m);
}

const void* ora_qwen2_tensor(const ora_qwen2* m, int layer, int kind, int part) {
  if (layer < 0) {
    if (kind == K_EMBED) return qmat_part(&m->embed, part);
    if (kind == K_FINAL_NORM) return m->final_norm;
    return NULL;
  }
  const q2_layer* L = &m->layers[layer];
  switch (kind) {
    case K_IN_NORM: return L->attn_norm;
    case K_POST_NORM: return L->ffn_norm;
    case K_Q: return qmat_part(&L->q, part);
    case K_K: return qmat_part(&L->k, part);
    case K_V: return qmat_part(&L->v, part);
    case K_O: return qmat_part(&L->o, part);
    case K_GATE: return qmat_part(&L->gate, part);
    case K_UP: return qmat_part(&L->up, part);
    case K_DOWN: return qmat_part(&L->down, part);
    case K_QB: return L->qb;
    case K_KB: return L->kb;
    case K_VB: return L->vb;
  }
  return NULL;
}

int ora_qwen2_set_matrix(ora_qwen2* m, int layer, int kind, int fmt, const uint8_t* blocks) {
  qmat* q = NULL;
  if (layer < 0) {
    if (kind == K_EMBED) q = &m->embed;
  } else if (layer < m->cfg.n_layers) {
    q2_layer* L = &m->layers[layer];
    switch (kind) {
      case K_Q: q = &L->q; break;
      case K_K: q = &L->k; break;
      case K_V: q = &L->v; break;
      case K_O: q = &L->o; break;
      case K_GATE: q = &L->gate; break;
      case K_UP: q = &L->up; break;
      case K_DOWN: q = &L->down; break;
    }
  }
  if (!q || fmt < FMT_Q4K || fmt > FMT_Q5_0) return -1;
  if ((fmt == FMT_Q4K || fmt == FMT_Q6K) ? q->n_in % ORA_QK != 0 : q->n_in % 32 != 0) return -1;
  size_t bytes = fmt == FMT_Q4K   ? (size_t)q->n_out * (q->n_in / ORA_QK) * ORA_Q4K_BYTES
                 : fmt == FMT_Q6K ? (size_t)q->n_out * (q->n_in / ORA_QK) * ORA_Q6K_BYTES
                 : fmt == FMT_Q8_0 ? (size_t)q->n_out * (q->n_in / 32) * ORA_Q8_0_BYTES
                                   : (size_t)q->n_out * (q->n_in / 32) * ORA_Q5_0_BYTES;
  uint8_t* nb = (uint8_t*)malloc(bytes);
  memcpy(nb, blocks, bytes);
  free(q->blocks);
  q->blocks = nb;
  q->fmt = fmt;
  return 0;
}

ora_qwen2_cache* ora_qwen2_cache_new(const ora_qwen2* m) {
  ora_qwen2_cache* c = (ora_qwen2_cache*)calloc(1, sizeof *c);
  c->n_layers = m->cfg.n_layers;
  c->kvw = m->cfg.kv_heads * m->cfg.head_dim;
  c->k = (float**)calloc((size_t)c->n_layers, sizeof(float*));
  c->v = (float**)calloc((size_t)c->n_layers, sizeof(float*));
  return c;
}

void ora_qwen2_cache_free(ora_qwen2_cache* c) {
  if (!c) return;
  for (int i = 0; i < c->n_layers; ++i) {
    free(c->k[i]);
    free(c->v[i]);
  }
  free(c->k);
  free(c->v);
  free(c);
}

int ora_qwen2_cache_len(const ora_qwen2_cache* c) { return c->len; }

#define Q2_WIRE_MAGIC 0x50444B56u

/* pagoda-hf/src/llama.rs:215-266 (SessionKv::export_bytes): magic, version
 * 2, token count, layer count, logits (count + f32), then per layer a
 * present flag (0 before the first forward), kv_heads, head_dim, the wire
 * dtype (0 f32, 1 f16 with llama.rs:139-172's rounding) and K then V as
 * [kv_heads, len, head_dim] (candle's [1, kv_heads, seq, hd] flattened). */
size_t ora_qwen2_cache_export(const ora_qwen2* m, const ora_qwen2_cache* c, const float* logits, int n_logits,
                              int f16, uint8_t* buf, size_t cap) {
  size_t at = 0;
  const int kvh = m->cfg.kv_heads, hd = m->cfg.head_dim;
  put_u32(buf, &at, cap, Q2_WIRE_MAGIC);
  put_u32(buf, &at, cap, 2);
  put_u32(buf, &at, cap, (uint32_t)c->len);
  put_u32(buf, &at, cap, (uint32_t)c->n_layers);
  put_f32s(buf, &at, cap, logits, (uint32_t)(logits ? n_logits : 0));
  for (int l = 0; l < c->n_layers; ++l) {
    if (c->len == 0) {
      put_u32(buf, &at, cap, 0);
      continue;
    }
    put_u32(buf, &at, cap, 1);
    put_u32(buf, &at, cap, (uint32_t)kvh);
    put_u32(buf, &at, cap, (uint32_t)hd);
    put_u32(buf, &at, cap, f16 ? 1u : 0u);
    for (int which = 0; which < 2; ++which) {
      const float* src = which ? c->v[l] : c->k[l];
      for (int h = 0; h < kvh; ++h)
        for (int p = 0; p < c->len; ++p)
          for (int d = 0; d < hd; ++d) {
            float x = src[((size_t)p * kvh + h) * hd + d];
            if (f16) {
              uint16_t b = ora_f32_to_f16(x);
              if (buf && at + 2 <= cap) memcpy(buf + at, &b, 2);
              at += 2;
            } else {
              if (buf && at + 4 <= cap) memcpy(buf + at, &x, 4);
              at += 4;
            }
          }
    }
  }
  return at;
}

/* pagoda-hf/src/llama.rs:268-345 (SessionKv::import_bytes) into a cache of
 * model m: magic, version 1 (payload f32 whatever the dtype field says) or
 * 2 (dtype field 1 = f16 payload), logits handed back through logits_out
 * (capacity logits_cap, count in *n_logits). Also requires what this cache
 * can hold: every layer present (or none when len is 0) with the model's
 * kv_heads/head_dim. Trailing bytes are ignored, as the reference reader
 * does. Returns NULL on a malformed payload. */
ora_qwen2_cache* ora_qwen2_cache_import(const ora_qwen2* m, const uint8_t* b, size_t n, float* logits_out,
                                        int logits_cap, int* n_logits) {
  size_t at = 0;
  uint32_t magic, version, len, n_layers, nl;
  const int kvh = m->cfg.kv_heads, hd = m->cfg.head_dim;
  if (take_bytes(b, n, &at, &magic, 4) || magic != Q2_WIRE_MAGIC) return NULL;
  if (take_bytes(b, n, &at, &version, 4) || (version != 1 && version != 2)) return NULL;
  if (take_bytes(b, n, &at, &len, 4) || take_bytes(b, n, &at, &n_layers, 4)) return NULL;
  if (take_bytes(b, n, &at, &nl, 4) || (size_t)nl * 4 > n - at) return NULL;
  if ((int)n_layers != m->cfg.n_layers || len > (uint32_t)m->cfg.max_pos) return NULL;
  if (n_logits) *n_logits = (int)nl;
  if (logits_out) memcpy(logits_out, b + at, (size_t)(nl < (uint32_t)logits_cap ? nl : (uint32_t)logits_cap) * 4);
  at += (size_t)nl * 4;
  ora_qwen2_cache* c = ora_qwen2_cache_new(m);
  c->len = (int)len;
  c->cap = (int)len;
  for (uint32_t l = 0; l < n_layers; ++l) {
    uint32_t present, h, d, dt;
    if (take_bytes(b, n, &at, &present, 4)) goto bad;
    if (present == 0) {
      if (len) goto bad;
      continue;
    }
    if (take_bytes(b, n, &at, &h, 4) || take_bytes(b, n, &at, &d, 4) || take_bytes(b, n, &at, &dt, 4)) goto bad;
    if ((int)h != kvh || (int)d != hd) goto bad;
    int f16 = version >= 2 && dt == 1;
    size_t count = (size_t)kvh * len * hd, es = f16 ? 2 : 4;
    if (count * es * 2 > n - at) goto bad;
    for (int which = 0; which < 2; ++which) {
      float* dst = (float*)malloc(sizeof(float) * (count ? count : 1));
      if (which) c->v[l] = dst; else c->k[l] = dst;
      for (int hh = 0; hh < kvh; ++hh)
        for (uint32_t p = 0; p < len; ++p)
          for (int dd = 0; dd < hd; ++dd) {
            float x;
            if (f16) {
              uint16_t u;
              memcpy(&u, b + at, 2);
              x = ora_f16_to_f32(u);
            } else {
              memcpy(&x, b + at, 4);
            }
            at += es;
            dst[((size_t)p * kvh + hh) * hd + dd] = x;
          }
    }
  }
  return c;
bad:
  ora_qwen2_cache_free(c);
  return NULL;
}

/* candle_nn RmsNorm as used at pagoda-hf/src/qwen2_gguf.rs:92,109,117:
 * x / sqrt(mean(x^2) + eps) * w (candle-core's CPU rms_norm; the exact op
 * order inside candle is unpinned). */
static void q2_rmsnorm(float* x, const float* w, int n, float eps) {
  float ss = 0.0f;
  for (int i = 0; i < n; ++i) ss += x[i] * x[i];
  float mm = sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) x[i] = x[i] / mm * w[i];
}

/* candle_nn::rotary_emb::rope (non-interleaved) at one position. */
static void q2_rope(float* x, const float* cs, const float* sn, int hd) {
  int half = hd / 2;
  for (int i = 0; i < half; ++i) {
    float x1 = x[i], x2 = x[i + half];
    x[i] = x1 * cs[i] - x2 * sn[i];
    x[i + half] = x1 * sn[i] + x2 * cs[i];
  }
}

/* pagoda-hf/src/qwen2_gguf.rs:142-166 (forward_tokens) and 206-266
 * (Block::forward, project, attend); SessionKv::push_kv appends K/V
 * (pagoda-hf/src/llama.rs:65). Matmuls use f32 dequantized weights. */
void ora_qwen2_set_kquant_mode(ora_qwen2* m, int mode) { m->kquant_mode = mode; }

static int q2_forward(ora_qwen2* m, const uint32_t* toks, int n, ora_qwen2_cache* cc, float* logits);

int ora_qwen2_forward(ora_qwen2* m, const uint32_t* toks, int n, ora_qwen2_cache* cc, float* logits) {
  const int saved = g_kquant_mode;
  g_kquant_mode = m->kquant_mode;
  const int rc = q2_forward(m, toks, n, cc, logits);
  g_kquant_mode = saved;
  return rc;
}

static int q2_forward(ora_qwen2* m, const uint32_t* toks, int n, ora_qwen2_cache* cc, float* logits) {
  const ora_qwen2_config* c = &m->cfg;
  int H = c->hidden, hd = c->head_dim, NH = c->heads, KVH = c->kv_heads, I = c->intermediate;
  int kvw = KVH * hd, half = hd / 2;
  if (n <= 0) return -1;
  if (cc->len + n > c->max_pos) return -3;
  for (int i = 0; i < n; ++i)
    if ((int)toks[i] >= c->vocab) return -2;
  int need = cc->len + n;
  if (need > cc->cap) {
    int cap = cc->cap ? cc->cap : 64;
    while (cap < need) cap *= 2;
    for (int l = 0; l < c->n_layers; ++l) {
      cc->k[l] = (float*)realloc(cc->k[l], sizeof(float) * (size_t)cap * kvw);
      cc->v[l] = (float*)realloc(cc->v[l], sizeof(float) * (size_t)cap * kvw);
    }
    cc->cap = cap;
  }
  float* x = (float*)malloc(sizeof(float) * (size_t)n * H);
  for (int i = 0; i < n; ++i) qmat_dequant(&m->embed, (int)toks[i], 1, x + (size_t)i * H);
  float* xn = (float*)malloc(sizeof(float) * (size_t)n * H);
  float* q = (float*)malloc(sizeof(float) * (size_t)n * NH * hd);
  float* k = (float*)malloc(sizeof(float) * (size_t)n * kvw);
  float* v = (float*)malloc(sizeof(float) * (size_t)n * kvw);
  float* att = (float*)malloc(sizeof(float) * (size_t)n * NH * hd);
  float* y = (float*)malloc(sizeof(float) * (size_t)n * H);
  float* g = (float*)malloc(sizeof(float) * (size_t)n * I);
  float* u = (float*)malloc(sizeof(float) * (size_t)n * I);
  int pos0 = cc->len;
  for (int l = 0; l < c->n_layers; ++l) {
    const q2_layer* L = &m->layers[l];
    memcpy(xn, x, sizeof(float) * (size_t)n * H);
    for (int t = 0; t < n; ++t) q2_rmsnorm(xn + (size_t)t * H, L->attn_norm, H, c->eps);
    qmat_linear(&L->q, xn, n, q);
    qmat_linear(&L->k, xn, n, k);
    qmat_linear(&L->v, xn, n, v);
    for (int t = 0; t < n; ++t) {
      for (int i = 0; i < NH * hd; ++i) q[(size_t)t * NH * hd + i] += L->qb[i];
      for (int i = 0; i < kvw; ++i) {
        k[(size_t)t * kvw + i] += L->kb[i];
        v[(size_t)t * kvw + i] += L->vb[i];
      }
      const float* cs = m->cos_t + (size_t)(pos0 + t) * half;
      const float* sn = m->sin_t + (size_t)(pos0 + t) * half;
      for (int h = 0; h < NH; ++h) q2_rope(q + (size_t)t * NH * hd + (size_t)h * hd, cs, sn, hd);
      for (int h = 0; h < KVH; ++h) q2_rope(k + (size_t)t * kvw + (size_t)h * hd, cs, sn, hd);
      memcpy(cc->k[l] + (size_t)(pos0 + t) * kvw, k + (size_t)t * kvw, sizeof(float) * kvw);
      memcpy(cc->v[l] + (size_t)(pos0 + t) * kvw, v + (size_t)t * kvw, sizeof(float) * kvw);
    }
    /* causal: query t sees positions <= pos0 + t (causal_mask at
     * pagoda-hf/src/qwen2_gguf.rs:350-360). */
    for (int t = 0; t < n; ++t)
      ora_attn_decode(q + (size_t)t * NH * hd, cc->k[l], cc->v[l], pos0 + t + 1, NH, KVH, hd, NULL,
                      att + (size_t)t * NH * hd);
    qmat_linear(&L->o, att, n, y);
    for (size_t i = 0; i < (size_t)n * H; ++i) x[i] += y[i];
    memcpy(xn, x, sizeof(float) * (size_t)n * H);
    for (int t = 0; t < n; ++t) q2_rmsnorm(xn + (size_t)t * H, L->ffn_norm, H, c->eps);
    qmat_linear(&L->gate, xn, n, g);
    qmat_linear(&L->up, xn, n, u);
    for (size_t i = 0; i < (size_t)n * I; ++i) g[i] = silu(g[i]) * u[i];
    qmat_linear(&L->down, g, n, y);
    for (size_t i = 0; i < (size_t)n * H; ++i) x[i] += y[i];
  }
  float* last = x + (size_t)(n - 1) * H;
  q2_rmsnorm(last, m->final_norm, H, c->eps);
  qmat_linear(&m->embed, last, 1, logits);
  cc->len += n;
  free(x);
  free(xn);
  free(q);
  free(k);
  free(v);
  free(att);
  free(y);
  free(g);
  free(u);
  return 0;
}
