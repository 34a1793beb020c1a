// attn.hip — paged GQA decode attention on the matrix cores, by page chunks.
//
// Counterpart of FullAttn::forward's softmax attention (pagoda-hf/src/
// qwen3_5.rs:1433-1475), full_attn_heads (qwen3_fuse.rs:384-440) and the
// Qwen2 attention core (qwen2_gguf.rs:252-266): row r attends to positions
// [0, pos_of_row[r]] of its sequence, softmax(q k^T / sqrt(hd)) v per head,
// GQA group = heads / kv_heads query heads per KV head; the hybrid model then
// multiplies by sigmoid(gate).
//
// Work split (the plan, built on the host from the block tables). A row's
// context is cut into chunks of kChunkPages pages. Rows whose chunk holds the
// same physical pages — requests forked from one trunk, the rows of one
// sequence in a prefill or verify chunk — share one work item, so the chunk's
// K/V is read once for all of them (once per item of up to 16 query
// vectors = rows x group heads; more sharers make more items, which the
// chunk's K/V then feeds from L2).
//
// Item kernel, per page of the chunk (16 positions), per wave (the four waves
// of an item take every fourth page and are combined in LDS):
//   S[p][n] = sum_d K[p][d] Q[n][d]        64 x v_mfma_f32_16x16x4_f32 (hd 256)
//   block softmax update per query n (positions past the row's length masked)
//   O[n][d] += sum_p P[n][p] V[p][d]       64 x v_mfma_f32_16x16x4_f32
// in fp32 like the reference. The score registers of the first product are
// the A operand of the second as they stand: lane (n, kq) holds positions
// 4 kq + r, which is the k index the second product assigns to it. The
// item writes per query its running max m, sum l and unnormalized O.
// Merge kernel, per (row, kv head): the row's chunk partials in chunk order,
// O / l, then gate and output (or the o projection's prepared operands).
// When every row of a launch has a single chunk, the item kernel does this
// last step itself and the merge is skipped (one launch for short contexts).
// A row's result depends only on its own chunks, never on which rows shared
// an item, so batched rows equal single-row calls bit for bit.
#include <algorithm>
#include <unordered_map>
#include <vector>

#include "a8_act.h"
#include "common.h"
#include "gemv_impl.h"
#include "ops.h"

namespace pgd {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kItemFields = 6;  // page_off, npages, row_off, first query, queries, chunk index

// ---------------------------------------------------------------------------
// item kernel
// ---------------------------------------------------------------------------
// Workgroup (item, kv head), 4 waves. The item's query vectors (query
// qi = row k * G + head g) are taken 16 at a time (a tile); for each tile, wave
// w runs the chunk's pages w, w + 4, ... (a page subset fixed by the page's
// place in the chunk, whatever the item's rows) and the four subsets' states
// are combined in LDS in subset order. Lane (j, kq) = (lane % 16, lane / 16).
// DIRECT: every row of the launch has one chunk; the item normalizes and
// writes the final output (gate, out / prepared operands) itself.
constexpr int kSubsets = 4;
// 16-query tiles per item of attn_split_kernel. More tiles share each loaded
// K/V page, but their query and output slices cost registers: config 5's
// 64-row decode measured 96.5 us per layer with 1 (110 VGPRs, 4 waves per
// SIMD), 114.5 with 2 (150, 3 waves), 180 with 4 (226, 2 waves).
constexpr int kSplitTiles = 1;
constexpr int kXcds = 8;  // MI355X: accelerator complex dies, one L2 each

template <int HD>
struct ItemLds {
  float o[kSubsets][16][HD];  // subset states: unnormalized O per query
  float m[kSubsets][16], l[kSubsets][16];
};

template <int HD, bool DIRECT>
__global__ __launch_bounds__(256) void attn_item_kernel(const float* __restrict__ q, const float* __restrict__ gate,
                                                        float* __restrict__ out, AttnLayout L, RowMeta m,
                                                        AttnPlan plan, int G, float* __restrict__ part_o,
                                                        float* __restrict__ part_ml, a8act::Dst act) {
  constexpr int T = HD / 4;    // QK k-steps; lane (i, kq) holds d = T kq + t
  constexpr int NT = HD / 16;  // PV n-tiles; lane (j, kq) holds d = NT j + nt
  __shared__ __attribute__((aligned(16))) ItemLds<HD> sh;
  // workgroups are dispatched to the 8 XCDs round robin (linear id % 8), each
  // with its own L2: give XCD x a contiguous range of the (kv head, item)
  // work list, so the items of one chunk (adjacent in the plan) share an L2
  const int total = gridDim.x, lin = blockIdx.x;
  const int xcd = lin % kXcds, per = total / kXcds, rem = total % kXcds;
  const int w = xcd * per + min(xcd, rem) + lin / kXcds;
  const int item = w % plan.n_items, kvh = w / plan.n_items;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, kq = lane >> 4;
  const int* it = plan.items + (size_t)item * kItemFields;
  // queries q0 .. q0 + nq - 1 of the rows from slot row_off on (query = row * G + head)
  const int page_off = it[0], npages = it[1], row_off = it[2], q0 = it[3], nq = it[4], chunk = it[5];
  const int chunk_pos0 = chunk * kChunkPages * L.block;
  const float inv_scale = 1.0f / sqrtf((float)HD);
  // this wave's pages: w, w + 4, ... (none when the chunk has fewer pages)
  const int my_pages = npages > wave ? (npages - wave + kSubsets - 1) / kSubsets : 0;
  auto page_base = [&](int k) {  // k-th page of this wave, clamped to its last one
    const int pi = wave + kSubsets * min(k, max(my_pages - 1, 0));
    const int page = plan.pages[page_off + min(pi, npages - 1)];
    return ((size_t)page * L.kv_heads + kvh) * L.block * HD;
  };

  for (int t0 = 0; t0 < nq; t0 += 16) {
    // this lane's query vector n = j: Q[n][T kq + t] (zero past the item's queries)
    const int qi = t0 + j;
    const bool qlive = qi < nq;
    const int krow = qlive ? (q0 + qi) / G : 0, g = qlive ? (q0 + qi) % G : 0;
    const int row = plan.item_rows[row_off + krow];
    const int len = m.pos_of_row[row] + 1;  // positions [0, len) are visible
    // V rows at or past every live query's length are unwritten slots of the
    // last page (any bit pattern). P is 0 there, but 0 * NaN is not 0, so
    // those rows are zeroed before P V.
    int lmax = qlive ? len : 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) lmax = max(lmax, __shfl_xor(lmax, o, 64));
    float Q[T];
    {
      const float* qp = q + ((size_t)row * L.heads + kvh * G + g) * HD + T * kq;
#pragma unroll
      for (int t = 0; t < T; t += 4) {
        const float4 v = qlive ? *reinterpret_cast<const float4*>(qp + t) : make_float4(0.f, 0.f, 0.f, 0.f);
        Q[t] = v.x;
        Q[t + 1] = v.y;
        Q[t + 2] = v.z;
        Q[t + 3] = v.w;
      }
    }
    float mx = -INFINITY, lsum = 0.0f;  // of query j (replicated over kq)
    f4 O[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) O[nt] = (f4){0.f, 0.f, 0.f, 0.f};

    // K and V of a page in registers: lane (j, kq) holds K[p = j][T kq + t] and
    // V[4 kq + s][NT j + nt]. Software pipeline: the next page's K is issued
    // once this page's scores are done, its V once this page's P V is done
    // (the last page re-reads itself, an L2 hit): no load waits behind a branch.
    float Kr[T], Vr[4][NT];
    auto load_k = [&](size_t base) {
      const float* kp = L.k_pool + base + (size_t)j * HD + T * kq;
#pragma unroll
      for (int e = 0; e < T; e += 4) {
        const float4 v = *reinterpret_cast<const float4*>(kp + e);
        Kr[e] = v.x;
        Kr[e + 1] = v.y;
        Kr[e + 2] = v.z;
        Kr[e + 3] = v.w;
      }
    };
    auto load_v = [&](size_t base) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float* vp = L.v_pool + base + (size_t)(4 * kq + s) * HD + NT * j;
#pragma unroll
        for (int e = 0; e < NT; e += 4) {
          const float4 v = *reinterpret_cast<const float4*>(vp + e);
          Vr[s][e] = v.x;
          Vr[s][e + 1] = v.y;
          Vr[s][e + 2] = v.z;
          Vr[s][e + 3] = v.w;
        }
      }
    };
    load_k(page_base(0));
    load_v(page_base(0));
    for (int k = 0; k < my_pages; ++k) {
      // ---- S = K Q^T: A = K[p = j][T kq + t], B = Q[n = j][T kq + t]; four
      // independent accumulators (t mod 4), added pairwise ----
      f4 Sa[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int t = 0; t < T; ++t) Sa[t & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(Kr[t], Q[t], Sa[t & 3], 0, 0, 0);
      const f4 S = (Sa[0] + Sa[1]) + (Sa[2] + Sa[3]);
      load_k(page_base(k + 1));
      // lane (j, kq) holds S[p = 4 kq + r][n = j]
      const int pos0 = chunk_pos0 + (wave + kSubsets * k) * L.block + 4 * kq;
      float sc[4];
      float pm = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[r] = pos0 + r < len ? S[r] * inv_scale : -INFINITY;
        pm = fmaxf(pm, sc[r]);
      }
      pm = fmaxf(pm, __shfl_xor(pm, 16, 64));
      pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
      // a page past a live query's length (its last page is w's, not this one)
      // leaves the state as it is
      const float mn = fmaxf(mx, pm);
      const float alpha = mn == -INFINITY ? 1.0f : expf(mx - mn);
      float ps = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[r] = (qlive && sc[r] != -INFINITY) ? expf(sc[r] - mn) : 0.0f;
        ps += sc[r];
      }
      ps += __shfl_xor(ps, 16, 64);
      ps += __shfl_xor(ps, 32, 64);
      lsum = lsum * alpha + ps;
      mx = mn;
      // O rows of this lane are queries 4 kq + r; their alphas live in lanes 4 kq + r
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float al = __shfl(alpha, 4 * kq + r, 64);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) O[nt][r] *= al;
      }
      if (pos0 - 4 * kq + L.block > lmax) {  // wave-uniform: a page with unwritten slots
#pragma unroll
        for (int s = 0; s < 4; ++s)
          if (pos0 + s >= lmax)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) Vr[s][nt] = 0.0f;
      }
      // ---- O += P V: A = P[n = j][p = 4 kq + s] (= sc[s]), B = V[4 kq + s][NT j + nt] ----
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) O[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(sc[s], Vr[s][nt], O[nt], 0, 0, 0);
      load_v(page_base(k + 1));
    }
    // ---- subset state to LDS: lane (j, kq) holds O[query 4 kq + r][NT j + nt] ----
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int e = 0; e < NT; e += 4)
        *reinterpret_cast<float4*>(&sh.o[wave][4 * kq + r][NT * j + e]) =
            make_float4(O[e][r], O[e + 1][r], O[e + 2][r], O[e + 3][r]);
    if (kq == 0) {
      sh.m[wave][j] = mx;
      sh.l[wave][j] = lsum;
    }
    __syncthreads();
    // ---- combine the subsets in order; thread = (query n, 16 dims) ----
    constexpr int SL = HD / 16;  // 16-dim slices per query
    for (int u = tid; u < 16 * SL; u += 256) {
      const int n = u / SL, d0 = (u % SL) * 16;
      const int qo = t0 + n;
      const bool live = qo < nq;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kSubsets; ++w) M = fmaxf(M, sh.m[w][n]);
      float lt = 0.0f, v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = 0.0f;
#pragma unroll
      for (int w = 0; w < kSubsets; ++w) {
        if (sh.m[w][n] == -INFINITY) continue;  // no visible position in this subset
        const float wt = expf(sh.m[w][n] - M);
        lt += sh.l[w][n] * wt;
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] += sh.o[w][n][d0 + e] * wt;
      }
      const int qa = q0 + (live ? qo : 0);
      const int orow = plan.item_rows[row_off + qa / G], head = kvh * G + qa % G;
      if constexpr (DIRECT) {
        const size_t oo = ((size_t)orow * L.heads + head) * HD + d0;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          v[e] = v[e] / lt;
          if (gate && live) v[e] *= 1.0f / (1.0f + expf(-gate[oo + e]));
        }
        if (out && live) {
#pragma unroll
          for (int e = 0; e < 16; e += 4)
            *reinterpret_cast<float4*>(out + oo + e) = make_float4(v[e], v[e + 1], v[e + 2], v[e + 3]);
        }
        if (act.XA) {
          // one 16-dim slice of the o projection's input; thread u ^ 1 holds the
          // neighbouring slice of the same 64-wide group (HD >= 64, SL even)
          const int col = head * HD + d0;
          a8act::emit_slice(act, orow, col >> 6, (col >> 4) & 3, v, live);
        }
      } else if (live) {
        const int slot = row_off + qa / G, go = qa % G;
        float* po = part_o + (((size_t)slot * L.kv_heads + kvh) * G + go) * HD + d0;
#pragma unroll
        for (int e = 0; e < 16; e += 4) *reinterpret_cast<float4*>(po + e) = make_float4(v[e], v[e + 1], v[e + 2], v[e + 3]);
        if (d0 == 0) {
          float* pml = part_ml + (((size_t)slot * L.kv_heads + kvh) * G + go) * 2;
          pml[0] = M;
          pml[1] = lt;
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// head-dim split item kernel (head_dim 256)
// ---------------------------------------------------------------------------
// Workgroup (item, kv head), 4 waves; an item is up to kSplitTiles 16-query
// tiles over the same chunk pages. Wave w owns head dims [64 w, 64 w + 64):
// per page it loads that slice of K and V once for every tile, computes each
// tile's partial scores over its dims (16 x v_mfma_f32_16x16x4_f32), and the
// four partials meet in LDS, added in wave order, so every wave holds the
// same scores; then each wave runs the same online-softmax update and
// O += P V for its dims (16 MFMAs per tile). Every wave walks all pages of
// the chunk in page order: a query's result depends only on its own row's
// pages, never on the item it shares (batched rows equal single-row calls).
// Registers hold a tile's query slice and output slice (16 + 16 per lane),
// so one K/V page can feed several tiles (kSplitTiles).
template <bool DIRECT>
__global__ __launch_bounds__(256) void attn_split_kernel(const float* __restrict__ q, const float* __restrict__ gate,
                                                         float* __restrict__ out, AttnLayout L, RowMeta m,
                                                         AttnPlan plan, int G, float* __restrict__ part_o,
                                                         float* __restrict__ part_ml, a8act::Dst act) {
  constexpr int HD = 256, TQ = kSplitTiles;
  constexpr int T = 16;  // QK k-steps per wave: lane (i, kq) holds d = 64 w + 16 kq + t
  // PV n-tiles: lane (j, kq) holds d = 64 w + 4 j + nt, nt = 0..3
  __shared__ __attribute__((aligned(16))) f4 xs[2][TQ][kSubsets][64];  // partial scores, by page parity
  __shared__ __attribute__((aligned(16))) float tb[16][HD + 4];         // a tile's normalized outputs
  const int total = gridDim.x, lin = blockIdx.x;
  const int xcd = lin % kXcds, per = total / kXcds, rem = total % kXcds;
  const int wi = xcd * per + min(xcd, rem) + lin / kXcds;
  const int item = wi % plan.n_items, kvh = wi / plan.n_items;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, kq = lane >> 4;
  const int* it = plan.items + (size_t)item * kItemFields;
  const int page_off = it[0], npages = it[1], row_off = it[2], q0 = it[3], nq = it[4], chunk = it[5];
  const int chunk_pos0 = chunk * kChunkPages * L.block;
  const float inv_scale = 1.0f / sqrtf((float)HD);
  const int d0 = 64 * wave;

  float Q[TQ][T];
  f4 O[TQ][4];
  float mx[TQ], lsum[TQ];
  int len[TQ];
  bool qlive[TQ];
  int lmax = 0;  // longest context of the item's live queries
#pragma unroll
  for (int t = 0; t < TQ; ++t) {
    const int qi = 16 * t + j;
    qlive[t] = qi < nq;
    const int krow = qlive[t] ? (q0 + qi) / G : 0, g = qlive[t] ? (q0 + qi) % G : 0;
    const int row = plan.item_rows[row_off + krow];
    len[t] = qlive[t] ? m.pos_of_row[row] + 1 : 0;
    lmax = max(lmax, len[t]);
    const float* qp = q + ((size_t)row * L.heads + kvh * G + g) * HD + d0 + 16 * kq;
#pragma unroll
    for (int e = 0; e < T; e += 4) {
      const float4 v = (16 * t < nq && qlive[t]) ? *reinterpret_cast<const float4*>(qp + e)
                                                   : make_float4(0.f, 0.f, 0.f, 0.f);
      Q[t][e] = v.x;
      Q[t][e + 1] = v.y;
      Q[t][e + 2] = v.z;
      Q[t][e + 3] = v.w;
    }
    mx[t] = -INFINITY;
    lsum[t] = 0.0f;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) O[t][nt] = (f4){0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) lmax = max(lmax, __shfl_xor(lmax, o, 64));
  lmax = max(lmax, 0);

  float Kr[T], Vr[4][4];
  auto page_base = [&](int k) {
    const int page = plan.pages[page_off + min(k, npages - 1)];
    return ((size_t)page * L.kv_heads + kvh) * L.block * HD;
  };
  auto load_k = [&](size_t base) {
    const float* kp = L.k_pool + base + (size_t)j * HD + d0 + 16 * kq;
#pragma unroll
    for (int e = 0; e < T; e += 4) {
      const float4 v = *reinterpret_cast<const float4*>(kp + e);
      Kr[e] = v.x;
      Kr[e + 1] = v.y;
      Kr[e + 2] = v.z;
      Kr[e + 3] = v.w;
    }
  };
  auto load_v = [&](size_t base) {
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
      const float4 v = *reinterpret_cast<const float4*>(L.v_pool + base + (size_t)(4 * kq + s2) * HD + d0 + 4 * j);
      Vr[s2][0] = v.x;
      Vr[s2][1] = v.y;
      Vr[s2][2] = v.z;
      Vr[s2][3] = v.w;
    }
  };
  load_k(page_base(0));
  load_v(page_base(0));
  for (int k = 0; k < npages; ++k) {
    const int par = k & 1;
    // ---- partial scores over this wave's dims, every tile ----
#pragma unroll
    for (int t = 0; t < TQ; ++t) {
      if (16 * t >= nq) break;
      f4 Sa[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int e = 0; e < T; ++e) Sa[e & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(Kr[e], Q[t][e], Sa[e & 3], 0, 0, 0);
      xs[par][t][wave][lane] = (Sa[0] + Sa[1]) + (Sa[2] + Sa[3]);
    }
    load_k(page_base(k + 1));
    __syncthreads();
    const int pos0 = chunk_pos0 + k * L.block + 4 * kq;  // lane (j, kq) holds positions 4 kq + r
    if (pos0 - 4 * kq + L.block > lmax) {  // a page with unwritten slots: 0 * NaN is not 0
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2)
        if (pos0 + s2 >= lmax)
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) Vr[s2][nt] = 0.0f;
    }
#pragma unroll
    for (int t = 0; t < TQ; ++t) {
      if (16 * t >= nq) break;
      const f4 S = ((xs[par][t][0][lane] + xs[par][t][1][lane]) + xs[par][t][2][lane]) + xs[par][t][3][lane];
      float sc[4];
      float pm = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[r] = pos0 + r < len[t] ? S[r] * inv_scale : -INFINITY;
        pm = fmaxf(pm, sc[r]);
      }
      pm = fmaxf(pm, __shfl_xor(pm, 16, 64));
      pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
      const float mn = fmaxf(mx[t], pm);
      const float alpha = mn == -INFINITY ? 1.0f : expf(mx[t] - mn);
      float ps = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[r] = (qlive[t] && sc[r] != -INFINITY) ? expf(sc[r] - mn) : 0.0f;
        ps += sc[r];
      }
      ps += __shfl_xor(ps, 16, 64);
      ps += __shfl_xor(ps, 32, 64);
      lsum[t] = lsum[t] * alpha + ps;
      mx[t] = mn;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float al = __shfl(alpha, 4 * kq + r, 64);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) O[t][nt][r] *= al;
      }
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          O[t][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(sc[s2], Vr[s2][nt], O[t][nt], 0, 0, 0);
    }
    load_v(page_base(k + 1));
  }
  // ---- outputs: lane (j, kq) holds O[query 4 kq + r][64 w + 4 j + nt] ----
#pragma unroll
  for (int t = 0; t < TQ; ++t) {
    if (16 * t >= nq) break;
    if constexpr (DIRECT) {
      // normalize into LDS, then thread u = (query n, 16-dim slice) writes
      __syncthreads();
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float lt = __shfl(lsum[t], 4 * kq + r, 64);
        *reinterpret_cast<float4*>(&tb[4 * kq + r][d0 + 4 * j]) =
            make_float4(O[t][0][r] / lt, O[t][1][r] / lt, O[t][2][r] / lt, O[t][3][r] / lt);
      }
      __syncthreads();
      const int n = tid >> 4, s16 = (tid & 15) * 16;
      const int qo = 16 * t + n;
      const bool live = qo < nq;
      const int qa = q0 + (live ? qo : 0);
      const int orow = plan.item_rows[row_off + qa / G], head = kvh * G + qa % G;
      const size_t oo = ((size_t)orow * L.heads + head) * HD + s16;
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        v[e] = tb[n][s16 + e];
        if (gate && live) v[e] *= 1.0f / (1.0f + expf(-gate[oo + e]));
      }
      if (out && live) {
#pragma unroll
        for (int e = 0; e < 16; e += 4)
          *reinterpret_cast<float4*>(out + oo + e) = make_float4(v[e], v[e + 1], v[e + 2], v[e + 3]);
      }
      if (act.XA) {
        const int col = head * HD + s16;
        a8act::emit_slice(act, orow, col >> 6, (col >> 4) & 3, v, live);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qo = 16 * t + 4 * kq + r;
        if (qo >= nq) continue;
        const int qa = q0 + qo;
        const int slot = row_off + qa / G, go = qa % G;
        float* po = part_o + (((size_t)slot * L.kv_heads + kvh) * G + go) * HD + d0 + 4 * j;
        *reinterpret_cast<float4*>(po) = make_float4(O[t][0][r], O[t][1][r], O[t][2][r], O[t][3][r]);
      }
      if (wave == 0 && kq == 0 && 16 * t + j < nq) {
        const int qa = q0 + 16 * t + j;
        float* pml = part_ml + (((size_t)(row_off + qa / G) * L.kv_heads + kvh) * G + qa % G) * 2;
        pml[0] = mx[t];
        pml[1] = lsum[t];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// merge kernel: workgroup (row, kv head), 256 threads over the G x HD outputs
// ---------------------------------------------------------------------------
constexpr int kMergeMax = 1024;  // chunk slots per row, staged in LDS

// Workgroup (row, kv head, group head g), thread = one of the head's HD dims.
template <int HD>
__global__ __launch_bounds__(HD) void attn_merge_kernel(const float* __restrict__ gate, float* __restrict__ out,
                                                        AttnLayout L, AttnPlan plan, int G,
                                                        const float* __restrict__ part_o,
                                                        const float* __restrict__ part_ml, a8act::Dst act) {
  __shared__ float s_w[kMergeMax];  // per slot: m, then exp(m - M)
  __shared__ float s_l[kMergeMax];
  __shared__ int s_slot[kMergeMax];
  __shared__ float s_lt;
  __shared__ __attribute__((aligned(16))) float obuf[HD];
  const int r = blockIdx.x, kvh = blockIdx.y, g = blockIdx.z, d = threadIdx.x;
  const int s0 = plan.row_slot_off[r], ns = plan.row_slot_off[r + 1] - s0;
  // every slot's (m, l) in one round of loads
  for (int i = d; i < ns; i += HD) {
    const int slot = plan.row_slots[s0 + i];
    s_slot[i] = slot;
    const float* ml = part_ml + (((size_t)slot * L.kv_heads + kvh) * G + g) * 2;
    s_w[i] = ml[0];
    s_l[i] = ml[1];
  }
  __syncthreads();
  // in chunk order: M = max m, weights exp(m - M), l = sum l * weight
  if (d == 0) {
    float M = -INFINITY;
    for (int i = 0; i < ns; ++i) M = fmaxf(M, s_w[i]);
    float lt = 0.0f;
    for (int i = 0; i < ns; ++i) {
      const float w = expf(s_w[i] - M);
      s_w[i] = w;
      lt += s_l[i] * w;
    }
    s_lt = lt;
  }
  __syncthreads();
  float o = 0.0f;
#pragma unroll 8
  for (int i = 0; i < ns; ++i) o += part_o[(((size_t)s_slot[i] * L.kv_heads + kvh) * G + g) * HD + d] * s_w[i];
  float res = o / s_lt;
  const size_t oo = ((size_t)r * L.heads + kvh * G + g) * HD + d;
  if (gate) res *= 1.0f / (1.0f + expf(-gate[oo]));
  if (out) out[oo] = res;
  if (act.XA) {
    // the head's HD dims are whole 64-wide groups of the o projection's input
    obuf[d] = res;
    __syncthreads();
    if (d < HD / 16) {
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = obuf[16 * d + e];
      const int col = (kvh * G + g) * HD + 16 * d;
      a8act::emit_slice(act, r, col >> 6, (col >> 4) & 3, v, true);
    }
  }
}

template <int HD>
void attn_hd(const float* q, const float* gate, float* out, const AttnLayout& L, const RowMeta& m,
             const AttnPlan& plan, int rows, hipStream_t s, const a8act::Dst& act) {
  const int G = L.heads / L.kv_heads;
  const size_t o_floats = (size_t)plan.n_slots * L.kv_heads * G * HD;
  const size_t ml_floats = (size_t)plan.n_slots * L.kv_heads * G * 2;
  // one chunk per row (n_slots == rows): the items finish the rows themselves
  if (plan.n_slots == rows) {
    if constexpr (HD == 256)
      hipLaunchKernelGGL((attn_split_kernel<true>), dim3(plan.n_items * L.kv_heads), dim3(256), 0, s, q, gate, out,
                         L, m, plan, G, nullptr, nullptr, act);
    else
      hipLaunchKernelGGL((attn_item_kernel<HD, true>), dim3(plan.n_items * L.kv_heads), dim3(256), 0, s, q, gate,
                         out, L, m, plan, G, nullptr, nullptr, act);
    return;
  }
  PGD_CHECK(plan.max_row_slots <= kMergeMax, kErrShape, "attention context too long for the merge");
  float* ws = static_cast<float*>(gemv::gemv_scratch(s, (o_floats + ml_floats) * sizeof(float), 4));
  if constexpr (HD == 256)
    hipLaunchKernelGGL((attn_split_kernel<false>), dim3(plan.n_items * L.kv_heads), dim3(256), 0, s, q, gate, out,
                       L, m, plan, G, ws, ws + o_floats, act);
  else
    hipLaunchKernelGGL((attn_item_kernel<HD, false>), dim3(plan.n_items * L.kv_heads), dim3(256), 0, s, q, gate,
                       out, L, m, plan, G, ws, ws + o_floats, act);
  hipLaunchKernelGGL(attn_merge_kernel<HD>, dim3(rows, L.kv_heads, G), dim3(HD), 0, s,
                     gate, out, L, plan, G, ws, ws + o_floats, act);
}

}  // namespace

// ---------------------------------------------------------------------------
// host: plan
// ---------------------------------------------------------------------------
void build_attn_plan(const int* seq_of_row, const int* pos_of_row, int rows, const int* block_tables,
                     int max_blocks, int block, int group, int head_dim, std::vector<int>& out) {
  // queries per work item: one 16-query tile (head_dim 64, 128) or up to
  // kSplitTiles tiles over the same pages (head_dim 256, attn_split_kernel)
  const int qpi = head_dim == 256 ? 16 * kSplitTiles : 16;
  PGD_CHECK(group > 0 && group <= 64 && block == 16, kErrShape, "attention plan: group <= 64 heads, pages of 16");
  struct Key {
    int chunk;
    std::vector<int> pages;
    bool operator==(const Key& o) const { return chunk == o.chunk && pages == o.pages; }
  };
  struct KeyHash {
    size_t operator()(const Key& k) const {
      size_t h = std::hash<int>()(k.chunk) * 0x9e3779b97f4a7c15ull;
      for (int p : k.pages) h = (h ^ (size_t)(unsigned)p) * 0x100000001b3ull;
      return h;
    }
  };
  std::unordered_map<Key, int, KeyHash> index;  // key -> group id
  std::vector<Key> keys;
  std::vector<std::vector<int>> members;        // rows of each group, in row order
  std::vector<std::vector<int>> row_chunk_group(rows);
  for (int r = 0; r < rows; ++r) {
    const int npages = pos_of_row[r] / block + 1;
    PGD_CHECK(npages <= max_blocks, kErrShape, "attention plan: position past the block table");
    const int* bt = block_tables + (size_t)seq_of_row[r] * max_blocks;
    const int nch = (npages + kChunkPages - 1) / kChunkPages;
    for (int c = 0; c < nch; ++c) {
      Key k{c, std::vector<int>(bt + c * kChunkPages, bt + std::min(npages, (c + 1) * kChunkPages))};
      auto f = index.find(k);
      int gid;
      if (f == index.end()) {
        gid = (int)keys.size();
        index.emplace(k, gid);
        keys.push_back(std::move(k));
        members.emplace_back();
      } else {
        gid = f->second;
      }
      members[gid].push_back(r);
      row_chunk_group[r].push_back(gid);
    }
  }
  // items: each group's queries (row-major over its rows, G heads per row) in
  // runs of 16, one matrix-core tile; a query's result does not depend on the
  // other queries of its tile, so tiles may cut between a row's heads
  std::vector<int> items, pages, item_rows;
  std::vector<std::vector<int>> group_slot0(keys.size());  // slot of each member
  for (size_t gi = 0; gi < keys.size(); ++gi) {
    const int page_off = (int)pages.size();
    pages.insert(pages.end(), keys[gi].pages.begin(), keys[gi].pages.end());
    const auto& mem = members[gi];
    const int base = (int)item_rows.size();
    for (size_t k = 0; k < mem.size(); ++k) {
      group_slot0[gi].push_back(base + (int)k);
      item_rows.push_back(mem[k]);
    }
    const int nqs = (int)mem.size() * group;
    for (int qs = 0; qs < nqs; qs += qpi)
      items.insert(items.end(), {page_off, (int)keys[gi].pages.size(), base + qs / group, qs % group,
                                 std::min(qpi, nqs - qs), keys[gi].chunk});
  }
  // row -> slots in chunk order
  std::vector<int> row_slot_off(rows + 1), row_slots;
  std::vector<size_t> cursor(keys.size(), 0);
  for (int r = 0; r < rows; ++r) {
    row_slot_off[r] = (int)row_slots.size();
    for (int gid : row_chunk_group[r]) row_slots.push_back(group_slot0[gid][cursor[gid]++]);
  }
  row_slot_off[rows] = (int)row_slots.size();
  // layout: header {n_items, n_slots, off_items, off_pages, off_item_rows, off_row_slot_off, off_row_slots}
  const int hdr = 8;
  out.assign(hdr, 0);
  out[0] = (int)(items.size() / kItemFields);
  out[1] = (int)item_rows.size();
  int max_slots = 0;
  for (int r = 0; r < rows; ++r) max_slots = std::max(max_slots, row_slot_off[r + 1] - row_slot_off[r]);
  out[7] = max_slots;
  auto put = [&](int field, const std::vector<int>& v) {
    out[field] = (int)out.size();
    out.insert(out.end(), v.begin(), v.end());
  };
  // the page list last: a decode step's other sections keep their offsets
  // while its rows' contexts grow within a chunk (stable launch arguments for
  // a captured step)
  put(2, items);
  put(4, item_rows);
  put(5, row_slot_off);
  put(6, row_slots);
  put(3, pages);
}

AttnPlan attn_plan_view(const int* host, const int* dev) {
  AttnPlan p;
  p.n_items = host[0];
  p.n_slots = host[1];
  p.items = dev + host[2];
  p.pages = dev + host[3];
  p.item_rows = dev + host[4];
  p.row_slot_off = dev + host[5];
  p.row_slots = dev + host[6];
  p.max_row_slots = host[7];
  return p;
}

// Attention in the CPU path's exact operation order, one 256-thread
// workgroup per (row, head): score_p = (sum_i q_i k_pi, i in order) / sqrt(hd)
// (one thread per position); the max; e_p = exp(score_p - max);
// sum = e_0 + e_1 + ... in position order; w_p = e_p / sum;
// out_i = sum_p w_p v_pi in position order, one thread per dimension over V
// rows staged in LDS a chunk at a time (FullAttn::forward / Qwen2 attend:
// pagoda-hf/src/qwen3_5.rs:1433-1475, qwen2_gguf.rs:252-266). Bit-equal to
// that order; used by the Qwen2 arithmetic that reproduces the reference CPU
// path (candle's quantized matmul). Scores live in LDS: the context is at
// most kExactMax positions.
constexpr int kExactMax = 30720;
constexpr int kExactThreads = 256;
constexpr int kExactChunkFloats = 8192;  // V rows staged per round: 32 KiB
template <int HD>
__global__ __launch_bounds__(kExactThreads) void attn_exact_kernel(const float* __restrict__ q,
                                                                   float* __restrict__ out, AttnLayout L, RowMeta m) {
  extern __shared__ __attribute__((aligned(16))) float sc[];  // [len] scores, then weights | V chunk [kExactChunkFloats / HD][HD] | page ids
  __shared__ __attribute__((aligned(16))) float qs[HD];
  __shared__ float red[kExactThreads / 64];
  __shared__ float s_sum;
  const int r = blockIdx.y, h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int kvh = h / (L.heads / L.kv_heads);
  const int seq = m.seq_of_row[r], len = m.pos_of_row[r] + 1;
  float* vs = sc + m.max_blocks * L.block;
  const float* qh = q + ((size_t)r * L.heads + h) * HD;
  // the sequence's page ids go to LDS first, so every K / V row address after
  // them is one LDS read away rather than a dependent global load
  const int nblk = (len + L.block - 1) / L.block;
  int* bt = reinterpret_cast<int*>(vs + kExactChunkFloats);
  {
    const int* src = m.block_tables + (size_t)seq * m.max_blocks;
    for (int i = tid; i < nblk; i += kExactThreads) bt[i] = src[i];
  }
  for (int i = tid; i < HD; i += kExactThreads) qs[i] = qh[i];
  constexpr int chunk = kExactChunkFloats / HD;
  constexpr int KV = kExactChunkFloats / (kExactThreads * 4);
  // V rows p0 .. p0 + n - 1: the thread's loads into registers (eight named
  // float4, so they stay in registers), then (after other work if any) its
  // stores into LDS. Every load is issued (past the end it re-reads row p0).
  static_assert(KV == 8, "eight V loads per thread and chunk");
  auto ldv = [&](int p0, int n, int k) -> float4 {
    const int e = tid * 4 + k * kExactThreads * 4, ec = e < n * HD ? e : 0;
    const int p = p0 + ec / HD, i = ec % HD;
    const float* vr = L.v_pool + (((size_t)bt[p / L.block] * L.kv_heads + kvh) * L.block + (p % L.block)) * HD;
    return *reinterpret_cast<const float4*>(vr + i);
  };
  auto stv = [&](int n, int k, const float4& v) {
    const int e = tid * 4 + k * kExactThreads * 4;
    if (e < n * HD) *reinterpret_cast<float4*>(vs + e) = v;
  };
  float4 v0, v1, v2, v3, v4, v5, v6, v7;
  auto load_v = [&](int p0, int n) {
    v0 = ldv(p0, n, 0);
    v1 = ldv(p0, n, 1);
    v2 = ldv(p0, n, 2);
    v3 = ldv(p0, n, 3);
    v4 = ldv(p0, n, 4);
    v5 = ldv(p0, n, 5);
    v6 = ldv(p0, n, 6);
    v7 = ldv(p0, n, 7);
  };
  auto store_v = [&](int n) {
    stv(n, 0, v0);
    stv(n, 1, v1);
    stv(n, 2, v2);
    stv(n, 3, v3);
    stv(n, 4, v4);
    stv(n, 5, v5);
    stv(n, 6, v6);
    stv(n, 7, v7);
  };
  __syncthreads();
  // the first V chunk is in flight while the scores are computed
  const int n0 = min(chunk, len);
  load_v(0, n0);
  const float scale = sqrtf((float)HD);
  float mx = -INFINITY;
  for (int p = tid; p < len; p += kExactThreads) {
    const float* kr = L.k_pool + (((size_t)bt[p / L.block] * L.kv_heads + kvh) * L.block + (p % L.block)) * HD;
    float dot = 0.0f;
    // the K row 64 values at a time, all of a part's loads in flight together
#pragma unroll
    for (int c = 0; c < HD; c += 64) {
      float4 k4[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) k4[i] = *reinterpret_cast<const float4*>(kr + c + 4 * i);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float4 q4 = *reinterpret_cast<const float4*>(qs + c + 4 * i);
        dot += q4.x * k4[i].x;
        dot += q4.y * k4[i].y;
        dot += q4.z * k4[i].z;
        dot += q4.w * k4[i].w;
      }
    }
    const float s = dot / scale;
    sc[p] = s;
    mx = fmaxf(mx, s);
  }
  store_v(n0);
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) red[wv] = mx;
  __syncthreads();
  mx = red[0];
  for (int w = 1; w < kExactThreads / 64; ++w) mx = fmaxf(mx, red[w]);
  for (int p = tid; p < len; p += kExactThreads) sc[p] = exp_cr(sc[p] - mx);
  __syncthreads();
  if (tid == 0) {
    // in position order; 16 at a time from LDS so the loads run ahead of
    // the dependent additions
    float sum = 0.0f;
    int p = 0;
    for (; p + 16 <= len; p += 16) {
      float4 e[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) e[u] = *reinterpret_cast<const float4*>(sc + p + 4 * u);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        sum += e[u].x;
        sum += e[u].y;
        sum += e[u].z;
        sum += e[u].w;
      }
    }
    for (; p < len; ++p) sum += sc[p];
    s_sum = sum;
  }
  __syncthreads();
  const float sum = s_sum;
  for (int p = tid; p < len; p += kExactThreads) sc[p] = sc[p] / sum;
  float acc = 0.0f;
  for (int p0 = 0; p0 < len; p0 += chunk) {
    const int n = min(chunk, len - p0);
    if (p0 > 0) {
      load_v(p0, n);
      __syncthreads();  // the previous chunk is consumed
      store_v(n);
    }
    __syncthreads();  // the weights are written, the chunk is staged
    if (tid < HD) {
      // 16 positions per round: all their LDS reads issued before the
      // dependent additions (position order within and across rounds)
      int t = 0;
      for (; t + 16 <= n; t += 16) {
        float4 w4[4];
        float vv[16];
#pragma unroll
        for (int u = 0; u < 4; ++u) w4[u] = *reinterpret_cast<const float4*>(sc + p0 + t + 4 * u);
#pragma unroll
        for (int u = 0; u < 16; ++u) vv[u] = vs[(t + u) * HD + tid];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          acc += w4[u].x * vv[4 * u];
          acc += w4[u].y * vv[4 * u + 1];
          acc += w4[u].z * vv[4 * u + 2];
          acc += w4[u].w * vv[4 * u + 3];
        }
      }
      for (; t < n; ++t) acc += sc[p0 + t] * vs[t * HD + tid];
    }
  }
  if (tid < HD) out[((size_t)r * L.heads + h) * HD + tid] = acc;
}

template <int HD>
void launch_exact(const float* q, float* out, const AttnLayout& L, const RowMeta& m, int rows, int max_len,
                  hipStream_t s) {
  // scores | V chunk | page ids
  const size_t lds = ((size_t)max_len + kExactChunkFloats + m.max_blocks) * sizeof(float);
  if (lds > 64 * 1024) {
    static bool set = false;
    if (!set) {
      PGD_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_exact_kernel<HD>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  160 * 1024));
      set = true;
    }
  }
  hipLaunchKernelGGL(attn_exact_kernel<HD>, dim3(L.heads, rows), dim3(kExactThreads), lds, s, q, out, L, m);
}

void attn_exact(const float* q, float* out, const AttnLayout& L, const RowMeta& m, int rows, int max_len,
                hipStream_t s) {
  PGD_CHECK(L.kv_heads > 0 && L.heads % L.kv_heads == 0, kErrShape, "heads must be a multiple of kv_heads");
  PGD_CHECK(L.head_dim == 64 || L.head_dim == 128 || L.head_dim == 256, kErrShape,
            "exact-order attention: head_dim 64, 128 or 256");
  PGD_CHECK(max_len <= kExactMax && max_len == m.max_blocks * L.block &&
                (size_t)(max_len + kExactChunkFloats + m.max_blocks) * sizeof(float) <= 160 * 1024,
            kErrShape, "exact-order attention holds at most " + std::to_string(kExactMax) + " positions");
  if (rows <= 0) return;
  if (L.head_dim == 64) launch_exact<64>(q, out, L, m, rows, max_len, s);
  else if (L.head_dim == 128) launch_exact<128>(q, out, L, m, rows, max_len, s);
  else launch_exact<256>(q, out, L, m, rows, max_len, s);
  PGD_HIP(hipGetLastError());
}

void attn_decode(const float* q, const float* gate, float* out, const AttnLayout& L, const RowMeta& m,
                 const AttnPlan& plan, int rows, hipStream_t s, const a8act::Dst* act) {
  PGD_CHECK(L.kv_heads > 0 && L.heads % L.kv_heads == 0, kErrShape, "heads must be a multiple of kv_heads");
  PGD_CHECK(L.heads / L.kv_heads <= 64, kErrShape, "GQA group of at most 64 heads");
  PGD_CHECK(L.block == 16, kErrShape, "attention pages hold 16 positions");
  PGD_CHECK(out || act, kErrArg, "attention needs an output");
  if (rows <= 0) return;
  const a8act::Dst d = act ? *act : a8act::Dst{nullptr, nullptr, 0, 0};
  if (act) PGD_CHECK(act->G * 64 == L.heads * L.head_dim && act->rows == rows, kErrShape, "prepared attention output");
  switch (L.head_dim) {
    case 64: attn_hd<64>(q, gate, out, L, m, plan, rows, s, d); break;
    case 128: attn_hd<128>(q, gate, out, L, m, plan, rows, s, d); break;
    case 256: attn_hd<256>(q, gate, out, L, m, plan, rows, s, d); break;
    default: throw Error{kErrShape, "attention head_dim must be 64, 128 or 256"};
  }
  PGD_HIP(hipGetLastError());
}

}  // namespace pgd
