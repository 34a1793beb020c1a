// common.h — shared device helpers for the pagoda HIP backend (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace pgd {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// error plumbing: every C-ABI call returns 0 or a negative code and leaves a
// message readable through pgd_last_error().
// ---------------------------------------------------------------------------
enum Status : int {
  kOk = 0,
  kErrArg = -1,
  kErrDevice = -2,
  kErrHip = -3,
  kErrShape = -4,
  kErrState = -5,
  kErrAlloc = -6,
  kErrFormat = -7,
};

void set_error(const std::string& msg);
const std::string& last_error();

struct Error {
  int code;
  std::string msg;
};

#define PGD_HIP(expr)                                                                   \
  do {                                                                                  \
    hipError_t _e = (expr);                                                             \
    if (_e != hipSuccess)                                                               \
      throw ::pgd::Error{::pgd::kErrHip, std::string(#expr) + ": " + hipGetErrorString(_e)}; \
  } while (0)

#define PGD_CHECK(cond, code, msg)                   \
  do {                                               \
    if (!(cond)) throw ::pgd::Error{(code), (msg)};  \
  } while (0)

// ---------------------------------------------------------------------------
// exact conversions (bit level, identical on host and device)
// ---------------------------------------------------------------------------
__host__ __device__ inline float bf16_to_f32(uint32_t h) { return __builtin_bit_cast(float, h << 16); }

__host__ __device__ inline uint16_t f32_to_bf16(float x) {
  uint32_t bits = __builtin_bit_cast(uint32_t, x);
  uint32_t round = 0x7fffu + ((bits >> 16) & 1u);
  uint64_t s = (uint64_t)bits + round;
  if (s > 0xffffffffull) s = 0xffffffffull;
  return (uint16_t)(s >> 16);
}

__host__ __device__ inline float f16_to_f32(uint32_t h) {
  uint32_t sign = (h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int e = -1;
      do {
        e++;
        man <<= 1;
      } while (!(man & 0x400u));
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  return __builtin_bit_cast(float, bits);
}

__host__ __device__ inline uint16_t f32_to_f16(float x) {
  uint32_t b = __builtin_bit_cast(uint32_t, x);
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

// ---------------------------------------------------------------------------
// wave64 reductions (fixed butterfly order: results are deterministic)
// ---------------------------------------------------------------------------
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// sum over aligned groups of `width` lanes (width a power of two <= 64)
__device__ inline float group_sum(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// e^x correctly rounded to f32: the double-precision exponential (error well
// below one double ulp) rounded once, so the result is the f32 nearest to
// e^x except when e^x lies within ~2^-29 f32 ulp of a rounding midpoint. The
// CPU restatement evaluates it the same way, so both sides agree bit for bit.
__device__ inline float exp_cr(float x) { return (float)exp((double)x); }
__device__ inline float silu_f(float x) { return x / (1.0f + exp_cr(-x)); }
__device__ inline float sigmoid_f(float x) { return 1.0f / (1.0f + exp_cr(-x)); }

}  // namespace pgd
