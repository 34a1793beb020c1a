// gemv_sk.hip — MLX affine-8 (group 64) skinny GEMM for 5..32 batch rows on
// the matrix cores: persistent stream-K over (tile block, group) units.
//
// Arithmetic (per 64-wide group, 16 weight rows x 16 batch rows):
//   P[b, n] = sum_k (1024 + c[n,k]) * (xh[b,k] + xl[b,k])    4 x v_mfma_f32_16x16x32_f16
//   Y[b, n] += s[n,g] * (P[b, n] - 1024 * XSP[b,g]) + bias[n,g] * XS[b,g]
// with xh = f16(x), xl = f16(x - xh) (x to ~22 bits), 1024 + c exact in f16
// (one byte permute per two codes), XS = sum x, XSP = sum (xh + xl) over the
// group (activation layout: a8_act.h). A lane owns one weight row and four
// batch rows; every batch row runs the same instructions over the same split
// of the groups for every row count in 5..32, so those launches are bitwise
// equal row for row (1..4-row launches use the split-K kernel of gemv_mma.hip).
//
// Work split. A block is 8 consecutive 32-row tiles (gate/up tile pairs for
// the fused SwiGLU), one per wave of an 8-wave workgroup. The units
// (block, group) are numbered block-major and cut into one contiguous run per
// workgroup, one workgroup per compute unit: every CU streams the same number
// of weight bytes and there is no tail round. A block whose groups all fall in
// one run is finished in place; a block cut between runs leaves one partial
// sum per run (slot 0: the run's first block, slot 1: its last), and a second
// kernel adds them in run order, i.e. in k order, and applies the epilogue.
// It runs once the stream is done, when memory latency is low again (a
// last-arriver reduction inside the streaming kernel waits behind every CU's
// queued weight loads). The cut depends on the matrix shape and the CU count.
//
// Streaming. Weights and scale/bias go straight into registers, D units ahead
// of the unit being computed (a ring unrolled D times, so registers never
// move and the compiler waits for exactly the load it needs). The group's
// activation operands (4 or 8 KiB + constants) ride in the same ring, one
// 16-byte slice per thread, and are published through a two-slot LDS ring one
// unit before use (one barrier per unit), so each workgroup reads them once
// for its 8 tiles. Every wave issues the same loads (no lane-dependent
// branches around them), which keeps the compiler's in-order load counts exact.
//
// Counterpart of affine_gemv / affine_gemm4 / gemv2_silu / gemv_res
// (pagoda-hf/src/qwen3_gemv.rs:54-306, 414-567).
#include <map>
#include <mutex>

#include "a8_act.h"
#include "common.h"
#include "gemv_impl.h"
#include "quant.h"

namespace pgd {
namespace gemv {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;  // waves (tiles) per workgroup / block

struct SkArgs {
  int G;        // groups of 64 along K
  int ntiles;   // 32-row tiles (of one matrix)
  int nblocks;  // ceil(ntiles / tiles per block)
  int nwg;      // workgroups (runs)
  long long U;  // nblocks * G
  f4* part;     // [nwg][2][kWaves][NF][64]: partial sums of a run's first / last block
};

// bytes [c, 0x64] of a permute form the f16 1024 + c
__device__ inline h8 codes8(uint32_t w0, uint32_t w1) {
  const uint32_t c0 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u);
  const uint32_t c1 = __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u);
  const uint32_t c2 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u);
  const uint32_t c3 = __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u);
  return __builtin_bit_cast(h8, (u4){c0, c1, c2, c3});
}

__device__ inline long long run_start(long long U, int nwg, int i) { return (long long)i * U / nwg; }
// run holding unit x
__device__ inline int run_of(long long U, int nwg, long long x) { return (int)(((x + 1) * nwg - 1) / U); }

// MODE 1: <= 16 rows (one batch tile), MODE 2: <= 32 rows (two), MODE 4:
// 37..64 rows as two 32-row activation chunks in one launch (four batch
// tiles), so the weights stream once for both
template <int MODE, bool DUAL>
struct Geo {
  // four 16-row weight subtiles per wave: SwiGLU gate halves 0-1 and up halves
  // 2-3 of one tile; plain matrices two consecutive tiles (0-1, 2-3), so that
  // every operand read from LDS feeds four subtiles
  static constexpr int NS = 4;
  static constexpr int TPW = DUAL ? 1 : 2;       // tiles per wave (per matrix)
  static constexpr int TPB = kWaves * TPW;       // tiles per block
  static constexpr int NBT = MODE;              // 16-row batch tiles
  static constexpr int NC = MODE == 4 ? 2 : 1;   // 32-row activation chunks
  static constexpr int ROWS = 16 * NBT;          // batch rows per launch at most
  static constexpr int NF = NS * NBT;            // f4 accumulators per lane
  static constexpr int XU4 = NBT * 256;          // u4 of operands per group ([bt][i][lane], a8_act.h)
  // constants per group in LDS: [bt][-1024 (XSP_A + XSP_B) | XS_A + XS_B][16],
  // the half-group sums added by the thread that stages them
  static constexpr int XCF = NBT * 32;
  static constexpr int SLOT = XU4 * 16 + XCF * 4;
  static constexpr int HBR = ROWS < 32 ? 32 : ROWS;             // rows of a wave's transpose buffer
  static constexpr int HB = DUAL ? kWaves * HBR * 33 * 4 : 0;  // SwiGLU transpose buffers
};

// Epilogue of one 32-row tile from accumulators V, subtiles s0, s0 + 1 (SwiGLU:
// gate 0-1, up 2-3); lane: weight row n of half h, batch rows 16 bt + 4 q + rr.
// hb: this wave's HBR x 33 float LDS buffer (SwiGLU).
template <int MODE, int EPI>
__device__ __attribute__((always_inline)) inline void tile_epilogue(
    const GemvArgs& a, int nb, int tile, const f4 (&V)[4][Geo<MODE, EPI == EPI_SWIGLU>::NBT], int s0, float* hb) {
  constexpr int NBT = Geo<MODE, EPI == EPI_SWIGLU>::NBT;
  if (tile >= (a.n_out + 31) / 32) return;
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  if constexpr (EPI == EPI_SWIGLU) {
    if (a.oact.XA) {
      // the tile's 32 products of a batch row are one half of group tile / 2 of
      // the down projection's input: transpose through LDS, then lane L
      // prepares 16 of them (row L % 32, quarter pair L / 32)
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int b = 16 * bt + 4 * q + rr;
            if (b < nb) hb[b * 33 + 16 * h + j] = silu_f(V[h][bt][rr]) * V[2 + h][bt][rr];
          }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int c = 0; c < (NBT + 1) / 2; ++c) {
        const int b = 32 * c + (lane & 31), h = lane >> 5;
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = b < nb ? hb[b * 33 + 16 * h + e] : 0.0f;
        a8act::emit_slice<32>(a.oact, a.row0 + b, tile >> 1, (tile & 1) * 2 + h, v, b < nb);
      }
      __builtin_amdgcn_wave_barrier();
      if (!a.y) return;
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int n = tile * 32 + 16 * h + j;
    if (n >= a.n_out) continue;
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int b = 16 * bt + 4 * q + rr;
        if (b >= nb) continue;
        const size_t o = (size_t)b * a.ldy + n;
        if constexpr (EPI == EPI_STORE) a.y[o] = V[s0 + h][bt][rr];
        if constexpr (EPI == EPI_RES) a.y[o] = a.res[(size_t)b * a.ldres + n] + V[s0 + h][bt][rr];
        if constexpr (EPI == EPI_SWIGLU) a.y[o] = silu_f(V[h][bt][rr]) * V[2 + h][bt][rr];
      }
  }
}

// Epilogue of wave `wave`'s tiles of block `blk`.
template <int MODE, int EPI>
__device__ __attribute__((always_inline)) inline void wave_epilogue(
    const GemvArgs& a, int nb, int blk, int wave, const f4 (&V)[4][Geo<MODE, EPI == EPI_SWIGLU>::NBT], float* hb) {
  using Gm = Geo<MODE, EPI == EPI_SWIGLU>;
  if constexpr (EPI == EPI_SWIGLU) {
    tile_epilogue<MODE, EPI>(a, nb, blk * Gm::TPB + wave, V, 0, hb);
  } else {
    tile_epilogue<MODE, EPI>(a, nb, (blk * kWaves + wave) * 2, V, 0, hb);
    tile_epilogue<MODE, EPI>(a, nb, (blk * kWaves + wave) * 2 + 1, V, 2, hb);
  }
}

// Deferred RMSNorm of the input: accumulators of batch row b times inv_rows[b].
template <int NS, int NBT>
__device__ __attribute__((always_inline)) inline void scale_rows(f4 (&Y)[NS][NBT], const float* inv_rows, int nb) {
  const int q = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int b = 16 * bt + 4 * q + rr;
      const float f = b < nb ? inv_rows[b] : 1.0f;
#pragma unroll
      for (int st = 0; st < NS; ++st) Y[st][bt][rr] *= f;
    }
}

// D: units of weights in flight per wave.
template <int MODE, int EPI, int D>
__global__ __launch_bounds__(64 * kWaves) void a8_sk_kernel(GemvArgs a, const uint4* __restrict__ XA,
                                                            const float* __restrict__ CA, int nb, SkArgs k) {
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  using Gm = Geo<MODE, DUAL>;
  constexpr int NS = Gm::NS, NBT = Gm::NBT, NF = Gm::NF;
  static_assert(D % 2 == 0, "LDS slot parity is fixed per unrolled step");
  __shared__ __attribute__((aligned(16))) char smem[2 * Gm::SLOT + Gm::HB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, q = lane >> 4;
  const int G = k.G;
  const long long U = k.U;
  const long long u0 = run_start(U, k.nwg, blockIdx.x), u1 = run_start(U, k.nwg, blockIdx.x + 1);
  if (u0 >= u1) return;
  float* hb = reinterpret_cast<float*>(smem + 2 * Gm::SLOT) + wave * Gm::HBR * 33;
  // deferred RMSNorm of the input: the rows' 1/rms, shared out over the waves;
  // workgroup 0 also leaves them for the fix-up kernel
  __shared__ float s_inv[Gm::ROWS];
  if (a.rss) {
    for (int b = wave; b < nb; b += kWaves) {
      const float v = rss_inv(a.rss + (size_t)b * a.rss_nh, a.rss_nh, a.rss_n, a.rss_eps);
      if (lane == 0) {
        s_inv[b] = v;
        if (blockIdx.x == 0) a.inv[b] = v;
      }
    }
    __syncthreads();
  }

  // ---- per-unit register payload: weights, scale/bias, one operand slice ----
  struct WR {
    u4 w[NS];
    uint32_t s[NS];
    u4 x[Gm::NC];  // thread t: u4 t % 512 of each chunk's operands of the group
    float c[2];    // thread t: the two half-group terms of constant t % XCF
  };
  // lane's byte offset in a 2 KiB [k half][row][32 codes] block (subtile half 0)
  const uint32_t woff0 = (q >> 1) * 1024 + j * 32 + (q & 1) * 16;
  // constant t (bt = t / 32, w = t % 32): w < 16 -1024 XSP of row w (halves at
  // +0, +16 of the item's 64 floats), else XS of row w - 16 (halves at +32, +48)
  // (MODE 4: constants 64.. are the second chunk's, G groups of 128 floats on)
  const uint32_t ct = tid % Gm::XCF, cw = ct % 32, cbt = ct / 32;
  const size_t coff = ((size_t)(cbt / 2) * G * 128 + (cbt % 2) * 64 + (cw < 16 ? cw : cw + 16)) * 4;
  const uint32_t xoff = (tid % (Gm::XU4 / Gm::NC)) * 16, soff = j * 4;
  auto load_unit = [&](int b, int g, WR& r) {
    // the operands first: they are published one unit before use, and the
    // loads retire in issue order, so waiting for them leaves the unit's
    // weights in flight
    // items 2g, 2g + 1 (both batch tiles) are contiguous: 512 u4 + 128 floats per
    // group; chunk c of a two-chunk launch starts c G groups on
#pragma unroll
    for (int c = 0; c < Gm::NC; ++c)
      r.x[c] = *reinterpret_cast<const u4*>(reinterpret_cast<const uint8_t*>(XA + ((size_t)c * G + g) * 512) + xoff);
    const float* cp = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(CA + (size_t)g * 128) + coff);
    r.c[0] = cp[0];
    r.c[1] = cp[16];
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      // missing tiles re-read the last one
      const int tile = min(DUAL ? b * Gm::TPB + wave : (b * kWaves + wave) * 2 + (st >> 1), k.ntiles - 1);
      const size_t base = (size_t)tile * G + g;
      const uint8_t* pc = ((DUAL && st >= 2) ? a.u0 : a.p0) + (base << 11) + (st & 1) * 512;
      const uint8_t* ps = ((DUAL && st >= 2) ? a.u1 : a.p1) + (base << 7) + (st & 1) * 64;
      r.w[st] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(pc + woff0));
      r.s[st] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(ps + soff));
    }
  };
  // operand ring: unit u in slot u & 1
  auto store_x = [&](int slot, const WR& r) {
    char* sb = smem + slot * Gm::SLOT;
#pragma unroll
    for (int c = 0; c < Gm::NC; ++c)
      if (tid < Gm::XU4 / Gm::NC) reinterpret_cast<u4*>(sb)[c * 512 + tid] = r.x[c];
    if (tid < Gm::XCF) reinterpret_cast<float*>(sb + Gm::XU4 * 16)[tid] = r.c[0] + r.c[1];
  };

  f4 Y[NS][NBT];
  auto zero_y = [&]() {
#pragma unroll
    for (int st = 0; st < NS; ++st)
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) Y[st][bt] = (f4){0.f, 0.f, 0.f, 0.f};
  };
  zero_y();

  // batch tile outer, subtile inner: one batch tile's operands are live at a
  // time (the byte permutes of the codes are redone per batch tile, cheaper
  // than the registers holding them)
  auto compute = [&](const WR& r, int slot) {
    const char* sb = smem + slot * Gm::SLOT;
    const u4* sx = reinterpret_cast<const u4*>(sb);
    const f4* sc = reinterpret_cast<const f4*>(sb + Gm::XU4 * 16);
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) {
      // operands [bt][i][lane]; constants [bt][-1024 XSP | XS][16]
      u4 X[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) X[i] = sx[bt * 256 + i * 64 + lane];
      const f4 cp = sc[bt * 8 + q], xs = sc[bt * 8 + 4 + q];
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        const h8 b0 = codes8(r.w[st].x, r.w[st].y);
        const h8 b1 = codes8(r.w[st].z, r.w[st].w);
        const float sc = bf16_to_f32(r.s[st] & 0xffffu);
        const float bi = bf16_to_f32(r.s[st] >> 16);
        // the MFMA adds the codes' dot product to -1024 XSP (the 1024 + c offset)
        f4 Pm = cp;
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[0]), b0, Pm, 0, 0, 0);
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[1]), b1, Pm, 0, 0, 0);
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[2]), b0, Pm, 0, 0, 0);
        Pm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, X[3]), b1, Pm, 0, 0, 0);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) Y[st][bt][rr] = fmaf(bi, xs[rr], fmaf(sc, Pm[rr], Y[st][bt][rr]));
      }
    }
  };

  auto store_part = [&](int slot) {
    f4* p = k.part + ((((size_t)blockIdx.x * 2 + slot) * kWaves + wave) * NF) * 64 + lane;
#pragma unroll
    for (int st = 0; st < NS; ++st)
#pragma unroll
      for (int bt = 0; bt < NBT; ++bt) p[(st * NBT + bt) * 64] = Y[st][bt];
  };

  // ---- the run ----
  const int first_blk = (int)(u0 / G), last_blk = (int)((u1 - 1) / G);
  const bool cut_head = (u0 % G) != 0, cut_tail = (u1 % G) != 0;
  int cb = first_blk, cg = (int)(u0 % G);  // compute cursor
  int ib = cb, ig = cg;                     // weight issue cursor (stops at the last unit)
  long long iu = u0;
  auto iadv = [&]() {
    if (iu + 1 < u1) {
      ++iu;
      if (++ig == G) {
        ig = 0;
        ++ib;
      }
    }
  };
  // after a unit: a block whose last group this was is finished in place,
  // unless the run started inside it (then its sums are the run's slot-0 partial)
  auto close = [&]() {
    if (++cg == G) {
      cg = 0;
      if (cb == first_blk && cut_head) store_part(0);
      else {
        if (a.rss) scale_rows(Y, s_inv, nb);
        wave_epilogue<MODE, EPI>(a, nb, cb, wave, Y, hb);
      }
      zero_y();
      ++cb;
    }
  };

  const long long n = u1 - u0;
  WR W[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load_unit(ib, ig, W[d]);
    iadv();
  }
  store_x(0, W[0]);
  __syncthreads();

  // step d of an unrolled round: compute unit i + d (operands in slot d & 1),
  // publish unit i + d + 1's operands, refill W[d] with unit i + d + D (past
  // the run's end the last unit is re-read, an L2 hit)
  for (long long i = 0; i < n; i += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (i + d < n) {
        compute(W[d], d & 1);
        close();
      }
      store_x((d + 1) & 1, W[(d + 1) % D]);
      load_unit(ib, ig, W[d]);
      iadv();
      __syncthreads();
    }
  }
  if (cut_tail) store_part(last_blk == first_blk ? 0 : 1);
}

// Cut blocks: add the runs' partial sums in run order, then the epilogue.
// One single-wave workgroup per (block, wave of the streaming kernel), so the
// few blocks of a matrix still spread over many compute units.
// MODE 4 (two 32-row chunks): grid y = chunk, each workgroup the 32-row
// fix-up of its chunk's batch tiles (half the accumulators, so five runs load
// together), with the rows, outputs and row scales offset by 32.
template <int MODE, int EPI>
__global__ __launch_bounds__(64) void a8_sk_fix_kernel(GemvArgs a, int nb, SkArgs k) {
  using Gs = Geo<MODE, EPI == EPI_SWIGLU>;  // the streaming kernel's (partial-sum layout)
  constexpr int CM = Gs::NC == 2 ? 2 : MODE;  // one chunk's mode
  using Gm = Geo<CM, EPI == EPI_SWIGLU>;
  constexpr int NS = Gm::NS, NBT = Gm::NBT, NF = Gm::NF;
  const int ch = Gs::NC == 2 ? blockIdx.y : 0;
  if (Gs::NC == 2) {
    if (ch == 1) {
      a.row0 += 32;
      if (a.y) a.y += (size_t)32 * a.ldy;
      if (a.res) a.res += (size_t)32 * a.ldres;
      if (a.inv) a.inv += 32;
    }
    nb = ch == 1 ? nb - 32 : min(nb, 32);
  }
  __shared__ __attribute__((aligned(16))) char smem[Gm::HB > 0 ? Gm::HB / kWaves : 16];
  const int blk = blockIdx.x / kWaves, wave = blockIdx.x % kWaves, lane = threadIdx.x;
  const long long b0 = (long long)blk * k.G;
  const int r0 = run_of(k.U, k.nwg, b0), r1 = run_of(k.U, k.nwg, b0 + k.G - 1);
  if (r0 == r1 || (blk * kWaves + wave) * Gm::TPW >= k.ntiles) return;  // whole in one run: done in place
  // every run but possibly the first starts inside the block (slot 0); the
  // first run holds the block in slot 1 when it started in an earlier block
  const int slot_r0 = run_start(k.U, k.nwg, r0) < b0 ? 1 : 0;
  auto at = [&](int r, int f) -> const f4* {
    const int slot = r == r0 ? slot_r0 : 0;
    return k.part + ((((size_t)r * 2 + slot) * kWaves + wave) * Gs::NF + f) * 64 + lane;
  };
  constexpr int RB = NF >= 16 ? 2 : NF >= 8 ? 5 : 8;  // runs loaded together
  f4 V[NS][NBT];
  for (int r = r0; r <= r1; r += RB) {
    f4 P[RB][NS][NBT];
#pragma unroll
    for (int t = 0; t < RB; ++t)
#pragma unroll
      for (int st = 0; st < NS; ++st)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) P[t][st][bt] = *at(min(r + t, r1), st * Gs::NBT + ch * NBT + bt);
#pragma unroll
    for (int t = 0; t < RB; ++t) {
      if (r + t > r1) break;
#pragma unroll
      for (int st = 0; st < NS; ++st)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) V[st][bt] = r + t == r0 ? P[t][st][bt] : V[st][bt] + P[t][st][bt];
    }
  }
  if (a.rss) scale_rows(V, a.inv, nb);
  wave_epilogue<CM, EPI>(a, nb, blk, wave, V, reinterpret_cast<float*>(smem));
}

// ---- host side ----
int cu_count() {
  static std::mutex mu;
  static std::map<int, int> m;
  int dev = 0;
  PGD_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  auto it = m.find(dev);
  if (it != m.end()) return it->second;
  int cus = 0;
  PGD_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  m[dev] = cus;
  return cus;
}

template <int MODE, int EPI, int D>
void launch_sk(const GemvArgs& a, const uint4* XA, const float* CA, int nb, hipStream_t s) {
  using Gm = Geo<MODE, EPI == EPI_SWIGLU>;
  SkArgs k;
  k.G = a.n_in / 64;
  k.ntiles = (a.n_out + 31) / 32;
  k.nblocks = (k.ntiles + Gm::TPB - 1) / Gm::TPB;
  k.U = (long long)k.nblocks * k.G;
  k.nwg = (int)std::min<long long>(cu_count(), k.U);
  k.part = static_cast<f4*>(gemv_scratch(s, (size_t)k.nwg * 2 * kWaves * Gm::NF * 64 * sizeof(f4), 3));
  hipLaunchKernelGGL((a8_sk_kernel<MODE, EPI, D>), dim3(k.nwg), dim3(64 * kWaves), 0, s, a, XA, CA, nb, k);
  hipLaunchKernelGGL((a8_sk_fix_kernel<MODE, EPI>), dim3(k.nblocks * kWaves, Gm::NC), dim3(64), 0, s, a, nb, k);
}

template <int EPI>
void launch_chunk_sk(const GemvArgs& a, const uint4* XA, const float* CA, int nb, hipStream_t s) {
  // units in flight per wave: as many as the registers hold (32 rows carry
  // twice the accumulators and operands)
  if (nb <= 16) return launch_sk<1, EPI, 4>(a, XA, CA, nb, s);
  if (nb <= 32) return launch_sk<2, EPI, 2>(a, XA, CA, nb, s);
  return launch_sk<4, EPI, 2>(a, XA, CA, nb, s);
}

}  // namespace

bool a8_sk_wanted(const GemvArgs& a, int epi) {
  // The streaming kernel pays a second launch and partial-sum traffic for the
  // cut blocks; it wins for the fused gate/up pair and for matrices tall
  // enough that each run spans several whole blocks (measured on MI355X).
  return epi == EPI_SWIGLU || (a.n_out + 31) / 32 >= 2048;
}

void sk_scratch_need(const GemvArgs& a, int nb, int epi, size_t* slot3, size_t* slot5) {
  static_assert(Geo<1, false>::NF == 4 && Geo<2, false>::NF == 8 && Geo<4, false>::NF == 16 &&
                    Geo<1, true>::NF == 4 && Geo<2, true>::NF == 8 && Geo<4, true>::NF == 16 &&
                    Geo<1, true>::TPB == kWaves && Geo<1, false>::TPB == 2 * kWaves,
                "scratch bound follows Geo");
  const bool dual = epi == EPI_SWIGLU;
  // launch_chunk_sk: MODE 1 up to 16 rows, MODE 2 up to 32, MODE 4 above
  const int TPB = kWaves * (dual ? 1 : 2), NF = 4 * (nb <= 16 ? 1 : nb <= 32 ? 2 : 4);
  const long long nblocks = ((a.n_out + 31) / 32 + TPB - 1) / TPB;
  const long long U = nblocks * (a.n_in / 64);
  const long long nwg = std::min<long long>(cu_count(), U);
  *slot3 = (size_t)nwg * 2 * kWaves * NF * 64 * sizeof(f4);
  *slot5 = a.rss ? 64 * sizeof(float) : 0;
}

void run_a8_sk_chunk(const GemvArgs& a_in, const uint4* XA, const float* CA, int nb, int epi, hipStream_t s) {
  // 37..64 rows: two chunks, the second of at least 5 rows (1..4-row launches
  // are another bitwise class, taken by the split-K kernels)
  PGD_CHECK(nb >= 5 && (nb <= 32 || (nb >= 37 && nb <= 64)), kErrArg,
            "stream-K A8 GEMV takes 5..32 or 37..64 rows per launch");
  GemvArgs a = a_in;
  if (a.rss) a.inv = static_cast<float*>(gemv_scratch(s, 64 * sizeof(float), 5));
  if (epi == EPI_SWIGLU) launch_chunk_sk<EPI_SWIGLU>(a, XA, CA, nb, s);
  else if (epi == EPI_RES) launch_chunk_sk<EPI_RES>(a, XA, CA, nb, s);
  else launch_chunk_sk<EPI_STORE>(a, XA, CA, nb, s);
}

}  // namespace gemv
}  // namespace pgd
