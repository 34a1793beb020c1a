// a8_stage_reads.h — LDS reads of one ring stage of the A8 matrix-core GEMV.
//
// Each block issues every ds_read a group needs (weights, scale/bias,
// activation operands, per-row constants) and waits for them once. Outputs
// are early-clobber: a read may not land in a register that a later read of
// the same block still uses as its address. The reads live in inline asm so
// that the compiler does not see LDS accesses after the global->LDS loads and
// add waits of its own; the kernel places the vmcnt waits explicitly.
//
// Stage layout (bytes from the stage base): weights NS x 1 KiB at 0 (lane's
// own 16 B at 16 * lane), scale/bias u32 at SBOFF (subtile st, row j at
// 4 * (16 st + j)), activation operands at XOFF, per-row constants at COFF.
// MODE 0: <= 4 batch rows, operands of 4 rows staged as [i][q][row] 16 B
// MODE 1: <= 16 rows ([i][lane] 16 B), MODE 2: <= 32 rows (two such tiles;
// eight subtiles split into two blocks for the asm operand limit)
// MODE 3: one row (row 0 only, [i][q] 16 B)
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace pgd {
namespace gemv {

template <int MODE, int NS> struct StageReads;
template <> struct StageReads<0, 2> {
  static __device__ __forceinline__ void run(uint32_t wa, uint32_t sa, uint32_t xa, uint32_t ca, uint4 (&W)[2],
                                             uint32_t (&S)[2], uint4 (&X)[1][4], float4 (&CC)[1][4]) {
    asm volatile("ds_read_b128 %0, %[wa]\n\tds_read_b128 %1, %[wa] offset:1024\n\tds_read_b32 %2, %[sa]\n\tds_read_b32 %3, %[sa] offset:64\n\tds_read_b128 %4, %[xa]\n\tds_read_b128 %5, %[xa] offset:256\n\tds_read_b128 %6, %[xa] offset:512\n\tds_read_b128 %7, %[xa] offset:768\n\tds_read_b128 %8, %[ca]\n\tds_read_b128 %9, %[ca] offset:16\n\tds_read_b128 %10, %[ca] offset:32\n\tds_read_b128 %11, %[ca] offset:48\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(W[0]), "=&v"(W[1]), "=&v"(S[0]), "=&v"(S[1]), "=&v"(X[0][0]), "=&v"(X[0][1]), "=&v"(X[0][2]), "=&v"(X[0][3]), "=&v"(CC[0][0]), "=&v"(CC[0][1]), "=&v"(CC[0][2]), "=&v"(CC[0][3])
                 : [wa] "v"(wa), [sa] "v"(sa), [xa] "v"(xa), [ca] "v"(ca)
                 : "memory");
  }
};

template <> struct StageReads<0, 4> {
  static __device__ __forceinline__ void run(uint32_t wa, uint32_t sa, uint32_t xa, uint32_t ca, uint4 (&W)[4],
                                             uint32_t (&S)[4], uint4 (&X)[1][4], float4 (&CC)[1][4]) {
    asm volatile("ds_read_b128 %0, %[wa]\n\tds_read_b128 %1, %[wa] offset:1024\n\tds_read_b128 %2, %[wa] offset:2048\n\tds_read_b128 %3, %[wa] offset:3072\n\tds_read_b32 %4, %[sa]\n\tds_read_b32 %5, %[sa] offset:64\n\tds_read_b32 %6, %[sa] offset:128\n\tds_read_b32 %7, %[sa] offset:192\n\tds_read_b128 %8, %[xa]\n\tds_read_b128 %9, %[xa] offset:256\n\tds_read_b128 %10, %[xa] offset:512\n\tds_read_b128 %11, %[xa] offset:768\n\tds_read_b128 %12, %[ca]\n\tds_read_b128 %13, %[ca] offset:16\n\tds_read_b128 %14, %[ca] offset:32\n\tds_read_b128 %15, %[ca] offset:48\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(W[0]), "=&v"(W[1]), "=&v"(W[2]), "=&v"(W[3]), "=&v"(S[0]), "=&v"(S[1]), "=&v"(S[2]), "=&v"(S[3]), "=&v"(X[0][0]), "=&v"(X[0][1]), "=&v"(X[0][2]), "=&v"(X[0][3]), "=&v"(CC[0][0]), "=&v"(CC[0][1]), "=&v"(CC[0][2]), "=&v"(CC[0][3])
                 : [wa] "v"(wa), [sa] "v"(sa), [xa] "v"(xa), [ca] "v"(ca)
                 : "memory");
  }
};

template <> struct StageReads<1, 2> {
  static __device__ __forceinline__ void run(uint32_t wa, uint32_t sa, uint32_t xa, uint32_t ca, uint4 (&W)[2],
                                             uint32_t (&S)[2], uint4 (&X)[1][4], float4 (&CC)[1][4]) {
    asm volatile("ds_read_b128 %0, %[wa]\n\tds_read_b128 %1, %[wa] offset:1024\n\tds_read_b32 %2, %[sa]\n\tds_read_b32 %3, %[sa] offset:64\n\tds_read_b128 %4, %[xa]\n\tds_read_b128 %5, %[xa] offset:1024\n\tds_read_b128 %6, %[xa] offset:2048\n\tds_read_b128 %7, %[xa] offset:3072\n\tds_read_b128 %8, %[ca]\n\tds_read_b128 %9, %[ca] offset:64\n\tds_read_b128 %10, %[ca] offset:128\n\tds_read_b128 %11, %[ca] offset:192\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(W[0]), "=&v"(W[1]), "=&v"(S[0]), "=&v"(S[1]), "=&v"(X[0][0]), "=&v"(X[0][1]), "=&v"(X[0][2]), "=&v"(X[0][3]), "=&v"(CC[0][0]), "=&v"(CC[0][1]), "=&v"(CC[0][2]), "=&v"(CC[0][3])
                 : [wa] "v"(wa), [sa] "v"(sa), [xa] "v"(xa), [ca] "v"(ca)
                 : "memory");
  }
};

template <> struct StageReads<1, 4> {
  static __device__ __forceinline__ void run(uint32_t wa, uint32_t sa, uint32_t xa, uint32_t ca, uint4 (&W)[4],
                                             uint32_t (&S)[4], uint4 (&X)[1][4], float4 (&CC)[1][4]) {
    asm volatile("ds_read_b128 %0, %[wa]\n\tds_read_b128 %1, %[wa] offset:1024\n\tds_read_b128 %2, %[wa] offset:2048\n\tds_read_b128 %3, %[wa] offset:3072\n\tds_read_b32 %4, %[sa]\n\tds_read_b32 %5, %[sa] offset:64\n\tds_read_b32 %6, %[sa] offset:128\n\tds_read_b32 %7, %[sa] offset:192\n\tds_read_b128 %8, %[xa]\n\tds_read_b128 %9, %[xa] offset:1024\n\tds_read_b128 %10, %[xa] offset:2048\n\tds_read_b128 %11, %[xa] offset:3072\n\tds_read_b128 %12, %[ca]\n\tds_read_b128 %13, %[ca] offset:64\n\tds_read_b128 %14, %[ca] offset:128\n\tds_read_b128 %15, %[ca] offset:192\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(W[0]), "=&v"(W[1]), "=&v"(W[2]), "=&v"(W[3]), "=&v"(S[0]), "=&v"(S[1]), "=&v"(S[2]), "=&v"(S[3]), "=&v"(X[0][0]), "=&v"(X[0][1]), "=&v"(X[0][2]), "=&v"(X[0][3]), "=&v"(CC[0][0]), "=&v"(CC[0][1]), "=&v"(CC[0][2]), "=&v"(CC[0][3])
                 : [wa] "v"(wa), [sa] "v"(sa), [xa] "v"(xa), [ca] "v"(ca)
                 : "memory");
  }
};

template <> struct StageReads<2, 2> {
  static __device__ __forceinline__ void run(uint32_t wa, uint32_t sa, uint32_t xa, uint32_t ca, uint4 (&W)[2],
                                             uint32_t (&S)[2], uint4 (&X)[2][4], float4 (&CC)[2][4]) {
    asm volatile("ds_read_b128 %0, %[wa]\n\tds_read_b128 %1, %[wa] offset:1024\n\tds_read_b32 %2, %[sa]\n\tds_read_b32 %3, %[sa] offset:64\n\tds_read_b128 %4, %[xa]\n\tds_read_b128 %5, %[xa] offset:1024\n\tds_read_b128 %6, %[xa] offset:2048\n\tds_read_b128 %7, %[xa] offset:3072\n\tds_read_b128 %8, %[xa] offset:4096\n\tds_read_b128 %9, %[xa] offset:5120\n\tds_read_b128 %10, %[xa] offset:6144\n\tds_read_b128 %11, %[xa] offset:7168\n\tds_read_b128 %12, %[ca]\n\tds_read_b128 %13, %[ca] offset:64\n\tds_read_b128 %14, %[ca] offset:128\n\tds_read_b128 %15, %[ca] offset:192\n\tds_read_b128 %16, %[ca] offset:256\n\tds_read_b128 %17, %[ca] offset:320\n\tds_read_b128 %18, %[ca] offset:384\n\tds_read_b128 %19, %[ca] offset:448\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(W[0]), "=&v"(W[1]), "=&v"(S[0]), "=&v"(S[1]), "=&v"(X[0][0]), "=&v"(X[0][1]), "=&v"(X[0][2]), "=&v"(X[0][3]), "=&v"(X[1][0]), "=&v"(X[1][1]), "=&v"(X[1][2]), "=&v"(X[1][3]), "=&v"(CC[0][0]), "=&v"(CC[0][1]), "=&v"(CC[0][2]), "=&v"(CC[0][3]), "=&v"(CC[1][0]), "=&v"(CC[1][1]), "=&v"(CC[1][2]), "=&v"(CC[1][3])
                 : [wa] "v"(wa), [sa] "v"(sa), [xa] "v"(xa), [ca] "v"(ca)
                 : "memory");
  }
};

template <> struct StageReads<2, 4> {
  static __device__ __forceinline__ void run(uint32_t wa, uint32_t sa, uint32_t xa, uint32_t ca, uint4 (&W)[4],
                                             uint32_t (&S)[4], uint4 (&X)[2][4], float4 (&CC)[2][4]) {
    asm volatile("ds_read_b128 %0, %[wa]\n\tds_read_b128 %1, %[wa] offset:1024\n\tds_read_b128 %2, %[wa] offset:2048\n\tds_read_b128 %3, %[wa] offset:3072\n\tds_read_b32 %4, %[sa]\n\tds_read_b32 %5, %[sa] offset:64\n\tds_read_b32 %6, %[sa] offset:128\n\tds_read_b32 %7, %[sa] offset:192\n\tds_read_b128 %8, %[xa]\n\tds_read_b128 %9, %[xa] offset:1024\n\tds_read_b128 %10, %[xa] offset:2048\n\tds_read_b128 %11, %[xa] offset:3072\n\tds_read_b128 %12, %[xa] offset:4096\n\tds_read_b128 %13, %[xa] offset:5120\n\tds_read_b128 %14, %[xa] offset:6144\n\tds_read_b128 %15, %[xa] offset:7168\n\tds_read_b128 %16, %[ca]\n\tds_read_b128 %17, %[ca] offset:64\n\tds_read_b128 %18, %[ca] offset:128\n\tds_read_b128 %19, %[ca] offset:192\n\tds_read_b128 %20, %[ca] offset:256\n\tds_read_b128 %21, %[ca] offset:320\n\tds_read_b128 %22, %[ca] offset:384\n\tds_read_b128 %23, %[ca] offset:448\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(W[0]), "=&v"(W[1]), "=&v"(W[2]), "=&v"(W[3]), "=&v"(S[0]), "=&v"(S[1]), "=&v"(S[2]), "=&v"(S[3]), "=&v"(X[0][0]), "=&v"(X[0][1]), "=&v"(X[0][2]), "=&v"(X[0][3]), "=&v"(X[1][0]), "=&v"(X[1][1]), "=&v"(X[1][2]), "=&v"(X[1][3]), "=&v"(CC[0][0]), "=&v"(CC[0][1]), "=&v"(CC[0][2]), "=&v"(CC[0][3]), "=&v"(CC[1][0]), "=&v"(CC[1][1]), "=&v"(CC[1][2]), "=&v"(CC[1][3])
                 : [wa] "v"(wa), [sa] "v"(sa), [xa] "v"(xa), [ca] "v"(ca)
                 : "memory");
  }
};

template <> struct StageReads<2, 8> {
  static __device__ __forceinline__ void run(uint32_t wa, uint32_t sa, uint32_t xa, uint32_t ca, uint4 (&W)[8],
                                             uint32_t (&S)[8], uint4 (&X)[2][4], float4 (&CC)[2][4]) {
    asm volatile("ds_read_b128 %0, %[wa]\n\tds_read_b128 %1, %[wa] offset:1024\n\tds_read_b128 %2, %[wa] offset:2048\n\tds_read_b128 %3, %[wa] offset:3072\n\tds_read_b128 %4, %[wa] offset:4096\n\tds_read_b128 %5, %[wa] offset:5120\n\tds_read_b128 %6, %[wa] offset:6144\n\tds_read_b128 %7, %[wa] offset:7168\n\tds_read_b32 %8, %[sa]\n\tds_read_b32 %9, %[sa] offset:64\n\tds_read_b32 %10, %[sa] offset:128\n\tds_read_b32 %11, %[sa] offset:192\n\tds_read_b32 %12, %[sa] offset:256\n\tds_read_b32 %13, %[sa] offset:320\n\tds_read_b32 %14, %[sa] offset:384\n\tds_read_b32 %15, %[sa] offset:448\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(W[0]), "=&v"(W[1]), "=&v"(W[2]), "=&v"(W[3]), "=&v"(W[4]), "=&v"(W[5]), "=&v"(W[6]), "=&v"(W[7]), "=&v"(S[0]), "=&v"(S[1]), "=&v"(S[2]), "=&v"(S[3]), "=&v"(S[4]), "=&v"(S[5]), "=&v"(S[6]), "=&v"(S[7])
                 : [wa] "v"(wa), [sa] "v"(sa)
                 : "memory");
    asm volatile("ds_read_b128 %0, %[xa]\n\tds_read_b128 %1, %[xa] offset:1024\n\tds_read_b128 %2, %[xa] offset:2048\n\tds_read_b128 %3, %[xa] offset:3072\n\tds_read_b128 %4, %[xa] offset:4096\n\tds_read_b128 %5, %[xa] offset:5120\n\tds_read_b128 %6, %[xa] offset:6144\n\tds_read_b128 %7, %[xa] offset:7168\n\tds_read_b128 %8, %[ca]\n\tds_read_b128 %9, %[ca] offset:64\n\tds_read_b128 %10, %[ca] offset:128\n\tds_read_b128 %11, %[ca] offset:192\n\tds_read_b128 %12, %[ca] offset:256\n\tds_read_b128 %13, %[ca] offset:320\n\tds_read_b128 %14, %[ca] offset:384\n\tds_read_b128 %15, %[ca] offset:448\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(X[0][0]), "=&v"(X[0][1]), "=&v"(X[0][2]), "=&v"(X[0][3]), "=&v"(X[1][0]), "=&v"(X[1][1]), "=&v"(X[1][2]), "=&v"(X[1][3]), "=&v"(CC[0][0]), "=&v"(CC[0][1]), "=&v"(CC[0][2]), "=&v"(CC[0][3]), "=&v"(CC[1][0]), "=&v"(CC[1][1]), "=&v"(CC[1][2]), "=&v"(CC[1][3])
                 : [xa] "v"(xa), [ca] "v"(ca)
                 : "memory");
  }
};

template <> struct StageReads<3, 2> {
  static __device__ __forceinline__ void run(uint32_t wa, uint32_t sa, uint32_t xa, uint32_t ca, uint4 (&W)[2],
                                             uint32_t (&S)[2], uint4 (&X)[1][4], float4& C1) {
    asm volatile("ds_read_b128 %0, %[wa]\n\tds_read_b128 %1, %[wa] offset:1024\n\tds_read_b32 %2, %[sa]\n\tds_read_b32 %3, %[sa] offset:64\n\tds_read_b128 %4, %[xa]\n\tds_read_b128 %5, %[xa] offset:64\n\tds_read_b128 %6, %[xa] offset:128\n\tds_read_b128 %7, %[xa] offset:192\n\tds_read_b128 %8, %[ca]\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(W[0]), "=&v"(W[1]), "=&v"(S[0]), "=&v"(S[1]), "=&v"(X[0][0]), "=&v"(X[0][1]), "=&v"(X[0][2]), "=&v"(X[0][3]), "=&v"(C1)
                 : [wa] "v"(wa), [sa] "v"(sa), [xa] "v"(xa), [ca] "v"(ca)
                 : "memory");
  }
};

template <> struct StageReads<3, 4> {
  static __device__ __forceinline__ void run(uint32_t wa, uint32_t sa, uint32_t xa, uint32_t ca, uint4 (&W)[4],
                                             uint32_t (&S)[4], uint4 (&X)[1][4], float4& C1) {
    asm volatile("ds_read_b128 %0, %[wa]\n\tds_read_b128 %1, %[wa] offset:1024\n\tds_read_b128 %2, %[wa] offset:2048\n\tds_read_b128 %3, %[wa] offset:3072\n\tds_read_b32 %4, %[sa]\n\tds_read_b32 %5, %[sa] offset:64\n\tds_read_b32 %6, %[sa] offset:128\n\tds_read_b32 %7, %[sa] offset:192\n\tds_read_b128 %8, %[xa]\n\tds_read_b128 %9, %[xa] offset:64\n\tds_read_b128 %10, %[xa] offset:128\n\tds_read_b128 %11, %[xa] offset:192\n\tds_read_b128 %12, %[ca]\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(W[0]), "=&v"(W[1]), "=&v"(W[2]), "=&v"(W[3]), "=&v"(S[0]), "=&v"(S[1]), "=&v"(S[2]), "=&v"(S[3]), "=&v"(X[0][0]), "=&v"(X[0][1]), "=&v"(X[0][2]), "=&v"(X[0][3]), "=&v"(C1)
                 : [wa] "v"(wa), [sa] "v"(sa), [xa] "v"(xa), [ca] "v"(ca)
                 : "memory");
  }
};


}  // namespace gemv
}  // namespace pgd
