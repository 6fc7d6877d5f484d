// HIP kernels of the MoE layer forward and backward (gfx950 / CDNA4).
//
// Semantics restate oxidizr's MoE layer (reference src/model.rs:1385-1958,
// arithmetic of boostr::nn::moe with explicit constants):
//   logits = x Wr^T (+ b);  probs = softmax(logits / tau);  top-k on logits,
//   lowest expert index first on ties;  w = probs[top-k] (optionally renormalised);
//   per expert: G = X Wg^T, U = X Wu^T, A = silu(G) * U, Y = A Wd^T;
//   out_t = sum_j w_tj Y[pos(t, j)] + s * shared(x_t);
//   aux = E (c_sw sum_e f_e P_e + c_sq sum_e P_e^2), z = mean_t lse_t^2.
// No floating-point atomics anywhere; integer LDS atomics only in the
// expert histogram, whose result is order-independent.
#pragma once
#include <climits>
#include <cmath>
#include <type_traits>
#include "gemm.hpp"

namespace moe {

// ------------------------------------------------------------------ tilings
// One tiling per GEMM role.  bf16 tiles are 256 x 256 outputs per workgroup
// (the gate/up forward's two B operands and the paired wgrad's two A
// operands each halve one side), one workgroup per CU.  The expert GEMMs run
// eight waves per workgroup, two per SIMD, each with a 64 x 128 (or 64 x 64
// per operand pair) block in 128 accumulation registers: while one wave of a
// SIMD waits on the k-tile's DMA or barrier the other issues MFMAs, and eight
// waves keep more direct-to-LDS loads in flight (a microbenchmark of the
// k-tile pattern: 1.92 -> 1.59 us per k-tile against four waves).  Measured
// against four waves with 128 x 128 blocks: config 5 step 30.2 -> 29.2 ms,
// config 2 2.13 -> 2.02 ms, config 3 8.33 -> 7.94 ms (same bits: each output
// keeps its k order).  The paired weight gradient's waves are stacked 4 x 2
// (32 x 128 blocks per operand): config 5's gate/up weight gradient 6.79 ->
// 6.61 ms against 2 x 4; a 2 x 4 grid for the 256 x 256 tiles made the down
// weight gradient 14 % slower.  Router-sized GEMMs (one side = E) keep
// 128 x 128 and four waves.  fp32 keeps four waves.
template <typename T> struct Tilings;
// RouterNarrow: 64-row router tiles with four stages, for launches whose
// 128-row grid would leave CUs idle (config 5: 128 -> 256 workgroups, router
// GEMM 120.7 -> 105 us; two stages 107.5 us).
// RouterDx: the input gradient dx (k_router_dgrad): 64-row tiles give its
// gather-sum twice the workgroups (config 2 43 -> 38 us, config 3 184 -> 176
// us, config 5 unchanged), where the router GEMM itself is faster on 128 rows.
template <> struct Tilings<bf16_t> {
  using Router = Tiling<bf16_t, 128, 128, 64>;
  using RouterDx = Tiling<bf16_t, 64, 128, 64>;
  using RouterNarrow = Tiling<bf16_t, 64, 128, 64, 4, 4>;
  using GateUp = Tiling<bf16_t, 256, 128, 64, 2, 2, 8>;
  using Big = Tiling<bf16_t, 256, 256, 64, 2, 2, 8>;
  using WgradPair = Tiling<bf16_t, 128, 256, 64, 2, 2, 8>;
};
// fp32 (config 1: T = 1024, H = 384, I = 1024): 64-column tiles give the
// N = H GEMMs 96 workgroups instead of the 48 that 128-column tiles leave for
// 256 CUs (config 1 step 0.48 -> 0.37 ms, same bits); for the router and the
// weight-gradient pair they measured no faster.  64-row tiles for the
// row-grouped GEMMs double the workgroups again (~256 rows per expert: gate/up
// input gradient 86 -> 55 us, down forward 40 -> 27 us, step 0.321 -> 0.297
// ms); the weight-gradient pair on 64 x 128 tiles as well (gate/up weight
// gradient 55 -> 48 us, step 0.300 -> 0.292 ms), and the router GEMMs and the
// input gradient dx (dx 16.8 -> 11.8 us, step 0.292 -> 0.288 ms).
constexpr int kF32RowTile = 64;
template <> struct Tilings<float> {
  using Router = Tiling<float, 64, 128, 32>;
  using RouterDx = Router;
  using RouterNarrow = Router;
  using GateUp = Tiling<float, kF32RowTile, 64, 32>;
  using Big = Tiling<float, kF32RowTile, 64, 32>;
  using WgradPair = Tiling<float, 64, 128, 32>;
};

// Row-grouped problems: groups split the M dimension (permuted token rows).
// offsets == nullptr means one dense group of M rows.
// A group of c rows has c / BM full row tiles and, when r = c % BM is not 0, a
// last tile of r rows.  That tile counts among the "big" tiles when r > BM / 2
// and is a "half" tile otherwise.  With tall > 0, a tail of 0 < r <= tall rows
// behind at least one full tile has no tile of its own: the group's last full
// tile covers BM + r rows.  Tiles run group by group (a group's tiles share
// its weight panels in L2), or, with half_last, every half tile after every
// big tile: the half-height tiles then fill the last round of the launch
// instead of adding a round among the big tiles, at the cost of reading their
// group's weights once more.
struct RowGroups {
  const int* offsets;      // [G + 1] row offsets
  const int* tile_prefix;  // [G + 1] prefix of the row tiles: ceil(c / BM) - merged
  const int* big_prefix;   // [G + 1] prefix of the big row tiles: c / BM + (r > BM / 2)
  const int* half_prefix;  // [G + 1] prefix of the half row tiles: 0 < r <= BM / 2, not merged
  int G;
  int M;                   // rows in all groups (the extent of row-major operands)
  int half_last;
  int tall;                // tail rows the last full tile takes (0 or BM / 4)
};

// Tile coordinates are workgroup-uniform, but integer division by a runtime
// value is expanded on the vector ALU; readfirstlane moves the results back to
// scalar registers so that the address arithmetic built on them stays scalar.
MOE_DEV int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Waves of the router kernels that split the hidden dimension (k_router_small,
// k_router_route).
constexpr int kRouterWaves = 16;

// 16 x 16 x 32 bf16 MFMA: acc[r] of lane l = sum_k a[row 4 (l / 16) + r][k] * b[row l % 16][k]
// with lane l supplying k-vector 8 (l / 16) (+ 32 q per step) of a-row and b-row l % 16.
MOE_DEV void mfma16(f32x4& acc, u32x4 a, u32x4 b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
}
MOE_DEV void mfma16(f32x4& acc, u32x4 a, u32x4 b, bf16_t) { mfma16(acc, a, b); }
// fp32 operands, four 16 x 16 x 4 MFMAs: lane l supplies the four consecutive k
// 4 (l / 16) + c (+ 16 q per load) of a-row and b-row l % 16, component c to
// step c, so the four lane groups cover 16 k per load; same output layout.
MOE_DEV void mfma16(f32x4& acc, u32x4 a, u32x4 b, float) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
}

// Output-tile order.  Workgroup ids are first made contiguous per XCD
// (xcd_slot); consecutive ids then walk GM row-tiles down a tile column
// before moving one column right, so the ~32 workgroups resident on one XCD
// cover about GM A panels and 32 / GM B panels, which its L2 holds, instead of
// one A panel and 32 B panels.  Returns false for ids past the nM x nN tiles.
// GM = 2 measured against 1, 3, 4 and 8: configs 3 and 5 0.6-0.9 % faster
// than with 4 (their experts hold few row tiles, so pairs stay inside an
// expert more often), config 2 unchanged; 1 was 1 % slower on configs 2 and 3,
// 8 1.5 % slower on config 5, 3 within 0.3 % (run-to-run noise).
template <int GM = 2>
MOE_DEV bool tile_order(int id, int nM, int nN, int& mt, int& nt) {
  const int g = uni(id / (GM * nN));
  const int r = id - g * (GM * nN);
  const int gm = min(GM, nM - g * GM);
  if (gm <= 0) return false;
  mt = uni(g * GM + r % gm);
  nt = uni(r / gm);
  return nt < nN;
}

// Row tiles of one group that walk down a tile column together.  A group's
// tiles are numbered group by group (a group of R row tiles owns R x nN
// consecutive ids) and, inside the group, bands of up to kRowWalk row tiles
// walk down each column before moving right: the workgroups that run
// together on an XCD then share the group's weight panel of each column
// (every row tile of an expert multiplies the same weights) and its token-row
// panels, instead of pairing row tiles across expert boundaries.
constexpr int kRowWalk = 8;
MOE_DEV void group_tile(const int* prefix, int G, int nN, int id, int& grp, int& local, int& nt) {
  grp = uni(find_group(prefix, G, id / nN));
  const int p0 = prefix[grp];
  int lr;
  tile_order<kRowWalk>(id - p0 * nN, prefix[grp + 1] - p0, nN, lr, nt);
  local = lr;
}

// Row-grouped launches need a grid of at least 8 * ceil(tiles / 8) blocks
// (xcd_slot2); dense ones at least the tile count.
MOE_DEV bool resolve_rows(const RowGroups& g, int N, int BM, int BN, int& grp, int& row0,
                          int& mv, int& n0) {
  const int nN = (N + BN - 1) / BN;
  int id, mt, nt;
  if (g.offsets == nullptr) {
    const int nM = (g.M + BM - 1) / BM;
    if (!xcd_slot(blockIdx.x, nM * nN, id) || !tile_order(id, nM, nN, mt, nt)) return false;
    n0 = nt * BN;
    grp = 0;
    row0 = mt * BM;
    mv = min(BM, g.M - row0);
    return mv > 0;
  }
  int local;
  if (g.half_last) {
    const int nB = g.big_prefix[g.G], nH = g.half_prefix[g.G];
    int cls;
    if (!xcd_slot2(blockIdx.x, nB * nN, nH * nN, cls, id)) return false;
    if (cls) {  // one half tile per group at most: pairs down a column
      if (!tile_order(id, nH, nN, mt, nt)) return false;
      grp = uni(find_group(g.half_prefix, g.G, mt));
      local = -1;
    } else {
      group_tile(g.big_prefix, g.G, nN, id, grp, local, nt);
    }
  } else {  // group by group
    const int nM = g.tile_prefix[g.G];
    if (!xcd_slot(blockIdx.x, nM * nN, id)) return false;
    group_tile(g.tile_prefix, g.G, nN, id, grp, local, nt);
  }
  n0 = nt * BN;
  const int rows = g.offsets[grp + 1] - g.offsets[grp];
  if (g.tall > 0 && !g.half_last) {
    // a tail of tall < r <= BM / 2 rows and the full tile before it run as two
    // 3BM/4-row tiles (3BM/4 and BM/4 + r rows): tiles of equal speed stay
    // together on their XCD and read the group's weight panels from its L2
    // once (config 5: step -0.25 %)
    const int nfull = rows / BM, r = rows - nfull * BM;
    if (nfull >= 1 && r > g.tall && r <= BM / 2 && local >= nfull - 1) {
      const int off = (nfull - 1) * BM + (local == nfull ? 3 * BM / 4 : 0);
      row0 = uni(g.offsets[grp] + off);
      mv = uni(local == nfull ? rows - off : 3 * BM / 4);
      return true;
    }
  }
  local = local < 0 ? (rows / BM) * BM : local * BM;  // -1: the group's half tile
  row0 = uni(g.offsets[grp] + local);
  // more than BM rows only for the last full tile with its merged tail
  const int left = rows - local;
  mv = uni(left > BM + g.tall ? BM : left);
  return mv > 0;
}

// K-grouped problems (weight gradients): groups split the reduction over
// token rows.  offsets == nullptr means one group with K rows, which may be
// split into nsplit fixed chunks of kchunk rows (a multiple of the k-tile):
// each chunk then produces an fp32 partial tile and k_splitk_reduce adds the
// chunks in ascending order, so the result does not depend on scheduling.
// col_walk: an XCD's tiles of a group run in tile_order (GM row tiles down a
// column, then right) instead of row by row.  Measured on the weight
// gradients: faster for the dense ones (shared expert: 1-3 %), for groups of
// >= 512 rows (configs 2 and 3: step -1.1 % / -0.4 %) and for the down
// projection's at every size (config 5: 3.52 -> 3.42 ms); slower for the
// gate/up pair's whole experts of ~256 rows (config 5: 5.94 -> 6.06 ms).
// xcd_order (grouped, G a multiple of 8): when not null and its flag
// xcd_order[G] is set, XCD x runs the whole groups xcd_order[x * G / 8 + j],
// j < G / 8 (k_xcd_order), one after another, instead of 1/8 of every group.
struct KGroups {
  const int* offsets;
  int G;
  int K;
  int nsplit;
  int kchunk;
  int col_walk;
  const int* xcd_order;
};

MOE_DEV bool resolve_k(const KGroups& g, int blk, int M, int N, int BM, int BN, int& grp,
                       int& split, int& krow0, int& K, int& m0, int& n0) {
  const int nM = (M + BM - 1) / BM, nN = (N + BN - 1) / BN;
  // Each group (or split chunk) owns 8 * ceil(per / 8) consecutive blocks and
  // its per tiles are dealt over the 8 XCDs in contiguous ranges, so every XCD
  // takes 1/8 of every group: the groups' token counts (the K of their tiles)
  // differ widely, and whole groups per XCD would leave the XCD that holds the
  // busiest expert running long after the others.
  const int per = nM * nN;
  int gs, r;  // group (grouped) or split chunk (dense); tile of it
  if (g.xcd_order && g.xcd_order[g.G]) {
    // whole groups per XCD: block b runs on XCD b % 8 and is that XCD's
    // (b / 8)-th block; the grid of 8 * ceil(per / 8) blocks per group covers
    // G / 8 groups of per tiles on every XCD
    const int epx = g.G >> 3, local = (blk >> 3);
    const int j = uni(local / per);
    if (j >= epx) return false;
    r = uni(local - j * per);
    gs = uni(g.xcd_order[(blk & 7) * epx + j]);
  } else {
    const int span = 8 * ((per + 7) >> 3);
    gs = uni(blk / span);
    if (!xcd_slot(blk - gs * span, per, r)) return false;
  }
  if (g.col_walk) {
    int mt, nt;
    if (!tile_order(r, nM, nN, mt, nt)) return false;
    m0 = mt * BM;
    n0 = nt * BN;
  } else {
    m0 = uni(r / nN) * BM;
    n0 = uni(r % nN) * BN;
  }
  if (g.offsets) {
    grp = gs;
    split = 0;
    if (grp >= g.G) return false;
    krow0 = uni(g.offsets[grp]);
    K = uni(g.offsets[grp + 1] - krow0);
  } else {
    grp = 0;
    split = gs;
    if (split >= g.nsplit) return false;
    krow0 = split * g.kchunk;
    K = min(g.kchunk, g.K - krow0);
  }
  return K > 0;
}

// Expert order of a grouped weight gradient over the 8 XCDs (E a multiple of
// 8, one block of 1024 threads): the experts ranked by token count (most
// first, ties by index) are dealt in a snake, rank r to XCD r % 8 in even
// rounds r / 8 and to 7 - r % 8 in odd ones, so every XCD holds E / 8 whole
// experts: each XCD's L2 then reads an expert's operand panels once instead of
// all eight reading every expert (config 5 gate/up weight gradient: 7.7 ->
// 6.7 ms; for the down projection's weight gradient, whose larger operand is
// already split over the XCDs, it measured slower).  order[E] = 1 when the
// busiest XCD holds at most 8 % more rows than the mean, else 0 (the kernels
// then deal every expert's tiles over all XCDs).  Integer arithmetic only.
__global__ __launch_bounds__(1024) void k_xcd_order(const int* __restrict__ counts, int E,
                                                    int* __restrict__ order) {
  __shared__ int cnt[1024];
  __shared__ int load[8];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) cnt[e] = counts[e];
  if (tid < 8) load[tid] = 0;
  __syncthreads();
  for (int e = tid; e < E; e += 1024) {
    const int c = cnt[e];
    int rank = 0;
    for (int f = 0; f < E; ++f) {
      const int d = cnt[f];
      rank += (d > c || (d == c && f < e)) ? 1 : 0;
    }
    const int round = rank >> 3, pos = rank & 7, x = (round & 1) ? 7 - pos : pos;
    order[x * (E >> 3) + round] = e;
    atomicAdd(&load[x], c);
  }
  __syncthreads();
  if (tid == 0) {
    int64_t total = 0;
    int mx = 0;
    for (int x = 0; x < 8; ++x) {
      total += load[x];
      mx = max(mx, load[x]);
    }
    order[E] = 100 * 8 * (int64_t)mx <= 108 * total ? 1 : 0;
  }
}

template <typename T>
MOE_DEV const T* pick(const T* const* tab, const T* single, int g) {
  return tab ? tab[g] : single;
}
template <typename T>
MOE_DEV T* pick(T* const* tab, T* single, int g) {
  return tab ? tab[g] : single;
}

// ------------------------------------------------------------------ router GEMM
// logits[t, e] = x[t] . Wr[e] (+ bias[e]), fp32 out.  C: Router or
// RouterNarrow (same per-element k order, same bits).
template <typename T, class C = typename Tilings<T>::Router>
__global__ __launch_bounds__(256) void k_router_logits(const T* __restrict__ x,
                                                       const T* __restrict__ wr,
                                                       const float* __restrict__ bias,
                                                       float* __restrict__ logits, int Tn, int H,
                                                       int E) {
  __shared__ __align__(16) T smem[kernel_smem_elems<C, T, 1, 1, 1>()];
  RowGroups g{nullptr, nullptr, nullptr, nullptr, 1, Tn, 0, 0};
  int grp, row0, mv, n0;
  if (!resolve_rows(g, E, C::BM, C::BN, grp, row0, mv, n0)) return;
  OpDesc<T> a[1] = {{x + (int64_t)row0 * H, H, mv, H}};
  OpDesc<T> b[1] = {{wr + (int64_t)n0 * H, H, E - n0, H}};
  f32x16 acc[1][C::TN][C::TM];
  zero_acc<C, 1>(acc);
  mainloop<C, T, false, false, 1, 1>(acc, a, b, H, smem);
  for_each_frag<C, 1>(acc, [&](int m, int n, auto& v) {
    if (m >= mv) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = n0 + n + i;
      if (e < E) logits[(int64_t)(row0 + m) * E + e] = v[0][i] + (bias ? bias[e] : 0.0f);
    }
  });
}

// Split-K router GEMM for wide H with too few output tiles to fill the CUs
// (T / 128 x E / 128 of them): partial[s][t][e] = x[t, ks) . Wr[e, ks) over
// the s-th kchunk-column chunk of H, ks = s * kchunk (a multiple of C::BK);
// k_router_reduce adds the chunks in order, then the bias.  The chunking
// depends on H only, so a token's logits are the same bits in any batch.
template <typename T, class C>
__global__ __launch_bounds__(C::THREADS) void k_router_logits_split(const T* __restrict__ x,
                                                                    const T* __restrict__ wr,
                                                                    float* __restrict__ partial,
                                                                    int Tn, int H, int E,
                                                                    int kchunk) {
  __shared__ __align__(16) T smem[kernel_smem_elems<C, T, 1, 1, 1>()];
  const int nN = (E + C::BN - 1) / C::BN;
  const int tiles = ((Tn + C::BM - 1) / C::BM) * nN;
  const int split = (int)blockIdx.x / tiles, id = (int)blockIdx.x - split * tiles;
  const int row0 = (id / nN) * C::BM, n0 = (id % nN) * C::BN;
  const int k0 = split * kchunk;
  const int kv = min(kchunk, H - k0);
  if (row0 >= Tn || kv <= 0) return;
  const int mv = min(C::BM, Tn - row0);
  OpDesc<T> a[1] = {{x + (int64_t)row0 * H + k0, H, mv, kv}};
  OpDesc<T> b[1] = {{wr + (int64_t)n0 * H + k0, H, E - n0, kv}};
  f32x16 acc[1][C::TN][C::TM];
  zero_acc<C, 1>(acc);
  mainloop<C, T, false, false, 1, 1>(acc, a, b, kv, smem);
  float* out = partial + (int64_t)split * Tn * E;
  for_each_frag<C, 1>(acc, [&](int m, int n, auto& v) {
    if (m >= mv) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = n0 + n + i;
      if (e < E) out[(int64_t)(row0 + m) * E + e] = v[0][i];
    }
  });
}

// logits[i] = ((partial[0][i] + partial[1][i]) + ...) + bias[i % E]
__global__ __launch_bounds__(256) void k_router_reduce(const float* __restrict__ partial,
                                                       int nsplit, int64_t TE, int E,
                                                       const float* __restrict__ bias,
                                                       float* __restrict__ logits) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= TE) return;
  float v = partial[i];
  for (int s = 1; s < nsplit; ++s) v += partial[(int64_t)s * TE + i];
  logits[i] = v + (bias ? bias[i % E] : 0.0f);
}

// ------------------------------------------------------------------ routing
// One wave routes token t: softmax(logits / tau), log-sum-exp, top-k on the
// raw logits (NaN selects as -inf; equal values -> lower expert index first).
// `row` holds the token's E logits (global memory, or a row staged in LDS by
// the fused router kernel): the same arithmetic either way, so the same bits.
// Also returns, in registers, the lane's probabilities pr[i] (expert
// lane + 64 i, 0 past E) and, in lane j < k, the j-th chosen expert (sel;
// -1 in lanes >= k).  Selection j is kept by lane j rather than in arrays
// indexed by the runtime k, which the compiler would keep in scratch or in
// 48 extra registers.
template <int EPL>
MOE_DEV void route_row(const float* row, int t, int E, int k, float tau,
                       int norm, float* __restrict__ probs, float* __restrict__ lse,
                       int* __restrict__ idx, float* __restrict__ w, float (&pr)[EPL],
                       int& sel) {
  const int lane = threadIdx.x & 63;
  float v[EPL], ex[EPL];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? row[e] : -INFINITY;
    if (e < E) mx = fmaxf(mx, v[i] / tau);
  }
  mx = wave_max(mx);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    ex[i] = e < E ? expf(v[i] / tau - mx) : 0.0f;
    s += ex[i];
  }
  s = wave_sum(s);
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    pr[i] = e < E ? ex[i] / s : 0.0f;
    if (e < E) probs[(int64_t)t * E + e] = pr[i];
  }
  if (lane == 0) lse[t] = mx + logf(s);

  uint32_t taken = 0;
  float wsel = 0.0f;
  sel = -1;
  float wsum = 0.0f;
  for (int j = 0; j < k; ++j) {
    float bv = -INFINITY;
    int be = INT_MAX;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      const float val = isnan(v[i]) ? -INFINITY : v[i];
      if (e < E && !((taken >> i) & 1u) && (be == INT_MAX || val > bv)) {
        bv = val;
        be = e;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oe = __shfl_xor(be, o, 64);
      const bool better = oe != INT_MAX && (be == INT_MAX || ov > bv || (ov == bv && oe < be));
      if (better) {
        bv = ov;
        be = oe;
      }
    }
    // every lane now holds the same winner; its owner marks it taken
    float mine = 0.0f;
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (lane + 64 * i == be) {
        taken |= 1u << i;
        mine = ex[i];
      }
    const float pj = __shfl(mine, be & 63, 64) / s;
    if (lane == j) {
      wsel = pj;
      sel = be;
    }
    wsum += pj;
  }
  if (lane < k) {
    idx[(int64_t)t * k + lane] = sel;
    w[(int64_t)t * k + lane] = norm ? wsel / wsum : wsel;
  }
}

// One wave per token.
template <int EPL>
__global__ __launch_bounds__(256) void k_route(const float* __restrict__ logits, int Tn, int E,
                                               int k, float tau, int norm,
                                               float* __restrict__ probs, float* __restrict__ lse,
                                               int* __restrict__ idx, float* __restrict__ w) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= Tn) return;
  float pr[EPL];
  int sel;
  route_row<EPL>(logits + (int64_t)t * E, t, E, k, tau, norm, probs, lse, idx, w, pr, sel);
}

// ------------------------------------------------------------------ fused router
// Router GEMM, softmax, log-sum-exp and top-k in one launch (bf16 or fp32, up
// to kFusedRouterMaxExperts experts).  A workgroup of kRouterWaves waves owns
// 16 tokens and every expert (NEB = ceil(E / 16) blocks of 16): each wave
// takes every kRouterWaves-th k-chunk of kFusedRouterChunkBytes per row of the
// hidden dimension and multiplies its 16 token rows with the NEB router-row
// blocks (v_mfma_f32_16x16x32_bf16, or four v_mfma_f32_16x16x4f32 per load
// for fp32), the partial sums are added through LDS in wave order, and each
// of the 16 waves then routes one token with route_row (the arithmetic of
// k_route) from the logits row staged in LDS.  256-byte chunks (128 bf16)
// give every wave a chunk at H = 2048 and keep the loads in flight within
// 64 VGPRs, so two workgroups share a CU (512-byte chunks: half the waves
// idle at H = 2048, 72 VGPRs, one workgroup per CU, two rounds of
// workgroups for 8192 tokens).
constexpr int kFusedRouterMaxExperts = 64;
constexpr int kFusedRouterChunkBytes = 256;
// The workgroup also writes what the dispatch and the losses need from its 16
// tokens: the expert histogram of their k choices (group_hist[b][e], an
// integer LDS histogram) and the column sums of their probabilities
// (prob_part[b][e], tokens added in order), so that k_scan over the 16-token
// groups and k_colsum_final finish the counts, offsets and P.
template <typename T, int NEB>
__global__ __launch_bounds__(64 * kRouterWaves) __attribute__((amdgpu_waves_per_eu(8))) void k_router_route(
    const T* __restrict__ x, const T* __restrict__ wr, const float* __restrict__ bias,
    int Tn, int H, int E, int k, float tau, int norm, float* __restrict__ logits,
    float* __restrict__ probs, float* __restrict__ lse, int* __restrict__ idx,
    float* __restrict__ w, int* __restrict__ group_hist, float* __restrict__ prob_part) {
  static_assert(16 * NEB <= kFusedRouterMaxExperts, "expert blocks");
  __shared__ f32x4 red[kRouterWaves][NEB][64];
  __shared__ float lg[16][16 * NEB + 4];
  __shared__ float pl[16][64];  // probabilities of the group's tokens
  __shared__ int hist[16 * NEB];
  const int t0 = blockIdx.x * 16;
  const int wave = uni(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int g = lane >> 4, rl = lane & 15;
  const int ntok = min(16, Tn - t0);
  constexpr int B = (int)sizeof(T);
  constexpr int V = 16 / B;                           // elements per 16-byte load
  constexpr int CH = kFusedRouterChunkBytes / B;      // chunk elements per row
  constexpr int NQ = CH / (4 * V);                    // loads per chunk: 4 lane groups x V
  const rsrc_t rx = make_rsrc(x + (int64_t)t0 * H, (uint32_t)((int64_t)ntok * H * B));
  const rsrc_t rw = make_rsrc(wr, (uint32_t)((int64_t)E * H * B));
  const uint32_t vx = (uint32_t)((rl * H + V * g) * B);
  f32x4 acc[NEB];
#pragma unroll
  for (int b = 0; b < NEB; ++b) acc[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int kc = wave; kc * CH < H; kc += kRouterWaves) {
    const uint32_t soff = (uint32_t)kc * kFusedRouterChunkBytes;
    u32x4 xa[NQ], wa[NEB][NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const bool kin = kc * CH + 4 * V * q + V * g < H;
      xa[q] = buf_ld16(rx, kin ? vx + 64 * q : kOobOffset, soff);
#pragma unroll
      for (int b = 0; b < NEB; ++b) {
        const uint32_t vw = (uint32_t)(((b * 16 + rl) * H + V * g) * B);
        wa[b][q] = buf_ld16(rw, kin && b * 16 + rl < E ? vw + 64 * q : kOobOffset, soff);
      }
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int b = 0; b < NEB; ++b) mfma16(acc[b], xa[q], wa[b][q], T());
  }
#pragma unroll
  for (int b = 0; b < NEB; ++b) red[wave][b][lane] = acc[b];
  __syncthreads();
  // wave b < NEB adds expert block b over the waves in order; lane holds
  // D[token 4 g + r][expert 16 b + rl]
  if (wave < NEB) {
    const int e = wave * 16 + rl;
    f32x4 v = red[0][wave][lane];
    // four LDS reads in flight (all fifteen hoisted ahead of the adds took 60
    // VGPRs); the adds stay in wave order
#pragma unroll 4
    for (int q = 1; q < kRouterWaves; ++q) v += red[q][wave][lane];
    const float bv = e < E && bias ? bias[e] : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) lg[4 * g + r][e] = v[r] + bv;
  }
  if (threadIdx.x < 16 * NEB) hist[threadIdx.x] = 0;
  __syncthreads();
  if (wave < ntok) {
    const int t = t0 + wave;
    for (int e = lane; e < E; e += 64) logits[(int64_t)t * E + e] = lg[wave][e];
    float pr[1];
    int sel;
    route_row<1>(&lg[wave][0], t, E, k, tau, norm, probs, lse, idx, w, pr, sel);
    pl[wave][lane] = pr[0];
    if (lane < k) atomicAdd(&hist[sel], 1);
  }
  __syncthreads();
  // the group's histogram and probability column sums (tokens in order)
  const int b = blockIdx.x;
  if (threadIdx.x < E) {
    const int e = threadIdx.x;
    group_hist[(int64_t)b * E + e] = hist[e];
    float sum = 0.0f;
    for (int i = 0; i < ntok; ++i) sum += pl[i][e];
    prob_part[(int64_t)b * E + e] = sum;
  }
}

// The split router GEMM's chunks added in order, then the bias (the
// arithmetic of k_router_reduce), and the routing of one 16-token group as in
// k_router_route: one wave per token (route_row from the logits row in LDS),
// the group's expert histogram and probability column sums for k_scan and the
// column-sum kernels (as k_router_route writes them).  E <= 64 EPL.
template <int EPL>
__global__ __launch_bounds__(1024) void k_reduce_route(
    const float* __restrict__ partial, int nsplit, int Tn, int E, int k, float tau, int norm,
    const float* __restrict__ bias, float* __restrict__ logits, float* __restrict__ probs,
    float* __restrict__ lse, int* __restrict__ idx, float* __restrict__ w,
    int* __restrict__ group_hist, float* __restrict__ prob_part) {
  __shared__ float lg[16][64 * EPL];
  __shared__ float pl[16][64 * EPL];
  __shared__ int hist[64 * EPL];
  const int t0 = blockIdx.x * 16;
  const int wave = uni(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int ntok = min(16, Tn - t0);
  const int64_t TE = (int64_t)Tn * E;
  if (threadIdx.x < 64 * EPL) hist[threadIdx.x] = 0;
  if (wave < ntok) {
    const int t = t0 + wave;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      if (e < E) {
        const int64_t o = (int64_t)t * E + e;
        float v = partial[o];
        for (int sp = 1; sp < nsplit; ++sp) v += partial[(int64_t)sp * TE + o];
        v = v + (bias ? bias[e] : 0.0f);
        lg[wave][e] = v;
        logits[o] = v;
      }
    }
  }
  __syncthreads();
  if (wave < ntok) {
    const int t = t0 + wave;
    float pr[EPL];
    int sel;
    route_row<EPL>(&lg[wave][0], t, E, k, tau, norm, probs, lse, idx, w, pr, sel);
#pragma unroll
    for (int i = 0; i < EPL; ++i) pl[wave][lane + 64 * i] = pr[i];
    if (lane < k) atomicAdd(&hist[sel], 1);
  }
  __syncthreads();
  const int b = blockIdx.x;
  for (int e = threadIdx.x; e < E; e += 1024) {
    group_hist[(int64_t)b * E + e] = hist[e];
    float sum = 0.0f;
    for (int i = 0; i < ntok; ++i) sum += pl[i][e];
    prob_part[(int64_t)b * E + e] = sum;
  }
}

// ------------------------------------------------------------------ column sums
// part[rb, e] = sum over rows [rb*64, rb*64+64) of a[t, e], fixed order.
__global__ __launch_bounds__(256) void k_colsum_partial(const float* __restrict__ a, int Tn, int E,
                                                        float* __restrict__ part) {
  __shared__ float red[4][64];
  const int c = threadIdx.x & 63, r = threadIdx.x >> 6;
  const int e = blockIdx.x * 64 + c;
  const int t0 = blockIdx.y * 64;
  float s = 0.0f;
  if (e < E)
    for (int t = t0 + r; t < min(t0 + 64, Tn); t += 4) s += a[(int64_t)t * E + e];
  red[r][c] = s;
  __syncthreads();
  if (r == 0 && e < E)
    part[(int64_t)blockIdx.y * E + e] = ((red[0][c] + red[1][c]) + red[2][c]) + red[3][c];
}

// out[e] = scale * sum_rb part[rb, e]: four running sums over rb = 4 i + j
// (independent loads stay in flight), added in the fixed order j = 0..3.
__global__ void k_colsum_final(const float* __restrict__ part, int nrb, int E, float scale,
                               float* __restrict__ out) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  int rb = 0;
  for (; rb + 4 <= nrb; rb += 4)
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] += part[(int64_t)(rb + j) * E + e];
  for (; rb < nrb; ++rb) s[rb & 3] += part[(int64_t)rb * E + e];
  out[e] = (((s[0] + s[1]) + s[2]) + s[3]) * scale;
}

// aux = E (c_sw sum_e f_e P_e + c_sq sum_e P_e^2), z = mean_t lse_t^2.
// counts == nullptr: the expert counts are built here from the top-k indices
// (integer LDS histogram, E <= 1024), so the kernel can run beside the
// dispatch instead of after it.
__global__ __launch_bounds__(256) void k_losses(const float* __restrict__ P,
                                                const int* __restrict__ counts,
                                                const int* __restrict__ idx,
                                                const float* __restrict__ lse, int Tn, int E,
                                                int k, float c_sw, float c_sq,
                                                float* __restrict__ aux, float* __restrict__ z) {
  __shared__ float r_sw[256], r_sq[256], r_z[256];
  __shared__ int hist[1024];
  const int tid = threadIdx.x;
  if (!counts) {
    for (int e = tid; e < E; e += 256) hist[e] = 0;
    __syncthreads();
    const int64_t n = (int64_t)Tn * k;
    for (int64_t i = tid; i < n; i += 256) {
      const int e = idx[i];
      if ((unsigned)e < (unsigned)E) atomicAdd(&hist[e], 1);
    }
    __syncthreads();
  }
  const float inv_tk = 1.0f / ((float)Tn * (float)k);
  float sw = 0.0f, sq = 0.0f, zz = 0.0f;
  for (int e = tid; e < E; e += 256) {
    const float p = P[e];
    sw += ((float)(counts ? counts[e] : hist[e]) * inv_tk) * p;
    sq += p * p;
  }
  {
    float zp[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // independent loads in flight
    int t = tid, j = 0;
    for (; t < Tn; t += 256, j = (j + 1) & 3) zp[j] += lse[t] * lse[t];
    zz = ((zp[0] + zp[1]) + zp[2]) + zp[3];
  }
  r_sw[tid] = sw; r_sq[tid] = sq; r_z[tid] = zz;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if (tid < o) {
      r_sw[tid] += r_sw[tid + o];
      r_sq[tid] += r_sq[tid + o];
      r_z[tid] += r_z[tid + o];
    }
    __syncthreads();
  }
  if (tid == 0) {
    if (aux) *aux = (float)E * (c_sw * r_sw[0] + c_sq * r_sq[0]);
    if (z) *z = r_z[0] / (float)Tn;
  }
}

// ------------------------------------------------------------------ dispatch
// Per-block expert histogram of 256 tokens' k assignments.
__global__ __launch_bounds__(256) void k_hist(const int* __restrict__ idx, int Tn, int k, int E,
                                              int* __restrict__ block_hist) {
  extern __shared__ int hist[];
  for (int e = threadIdx.x; e < E; e += 256) hist[e] = 0;
  __syncthreads();
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t < Tn)
    for (int j = 0; j < k; ++j) atomicAdd(&hist[idx[(int64_t)t * k + j]], 1);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256) block_hist[(int64_t)blockIdx.x * E + e] = hist[e];
}

// counts, exclusive offsets, per-block bases, and GEMM tile prefixes for the
// row-tile heights in kTileBM: per height, the prefixes of all, big and half
// row tiles (RowGroups), each [E + 1].
constexpr int kTilePrefixes = 3;
constexpr int kNumTileBM = 3;
__constant__ int kTileBM[kNumTileBM] = {kF32RowTile, 256, 384};
// Tail rows a group's last full row tile takes (RowGroups::tall) for row
// tiles of height bm: the bf16 256-row tilings run it as a tall tile; fp32's
// 128-row tiles take none.
constexpr int tall_rows_for(int bm) { return bm == 256 ? bm / 4 : 0; }

// Inclusive prefix sums across the 64 lanes of a wave of N values at once:
// each step issues the N shuffles before adding, so the N scans wait for one
// LDS round trip per step instead of N.
template <int N>
MOE_DEV void wave_incl_scans(int (&v)[N]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int t[N];
#pragma unroll
    for (int j = 0; j < N; ++j) t[j] = __shfl_up(v[j], o, 64);
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (lane >= o) v[j] += t[j];
  }
}

// With cnt[e] (LDS, e < E <= 1024) in place, a block of 1024 threads writes
// the exclusive offsets (also to offs, LDS) and the tile prefixes of every
// height in kTileBM, one expert per thread.  The kScanCount scans run
// together: a wave scan each, the wave totals to wsum[j][wave] (LDS,
// kScanCount x 16), one barrier, and each thread adds the totals of the
// waves below it with a fixed-trip predicated loop (its LDS reads all in
// flight).  Integer arithmetic only.
constexpr int kScanCount = 1 + kTilePrefixes * kNumTileBM;
MOE_DEV void scan_counts(const int* cnt, int E, int* __restrict__ offsets,
                         int* __restrict__ tile_prefix, int* offs, int* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = tid < E ? cnt[tid] : 0;
  int v[kScanCount], incl[kScanCount];
#pragma unroll
  for (int j = 0; j < kScanCount; ++j) {
    v[j] = c;
    if (j > 0) {
      const int bm = kTileBM[(j - 1) / kTilePrefixes], r = c % bm, kind = (j - 1) % kTilePrefixes;
      // a short tail behind a full tile joins that tile (tall tile)
      const int merged = c > bm && r > 0 && r <= tall_rows_for(bm) ? 1 : 0;
      const int tail = r > 0 && !merged ? 1 : 0;
      v[j] = kind == 0 ? c / bm + tail
           : kind == 1 ? c / bm + (r > bm / 2 ? 1 : 0)
                       : (tail && r <= bm / 2 ? 1 : 0);
    }
    incl[j] = v[j];
  }
  wave_incl_scans(incl);
#pragma unroll
  for (int j = 0; j < kScanCount; ++j)
    if (lane == 63) wsum[j * 16 + wave] = incl[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kScanCount; ++j) {
    int base = 0;
#pragma unroll
    for (int w = 0; w < 15; ++w) base += w < wave ? wsum[j * 16 + w] : 0;
    int* dst = j == 0 ? offsets : tile_prefix + (j - 1) * (E + 1);
    if (tid < E) {
      dst[tid] = base + incl[j] - v[j];
      if (j == 0) offs[tid] = base + incl[j] - v[j];
    }
    if (tid == 1023) dst[E] = base + incl[j];
  }
  __syncthreads();
}

// One block of 1024 threads (E <= 1024).  Thread (g, e) = (tid / E, tid % E)
// owns expert e's histogram entries of a contiguous chunk of blocks: the
// chunk sums and their exclusive prefix over g (a log-step scan in LDS) give
// the expert counts and the chunk bases; the expert counts are then scanned
// in parallel (one expert per thread) for the offsets and for the tile prefix
// of every height in kTileBM; a last pass writes every block's base.  Chunks
// of up to kScanRegChunk blocks stay in registers between the two passes (one
// round of loads, all in flight); longer ones are read twice, eight loads in
// flight.  Integer arithmetic only.
constexpr int kScanRegChunk = 64;
__global__ __launch_bounds__(1024) void k_scan(const int* __restrict__ block_hist, int nb, int E,
                                               int* __restrict__ block_base,
                                               int* __restrict__ counts,
                                               int* __restrict__ offsets,
                                               int* __restrict__ tile_prefix) {
  __shared__ int cnt[1024], offs[1024], part[1024];
  __shared__ int wsum[16 * kScanCount];
  const int tid = threadIdx.x;
  const int G = 1024 / E;            // threads per expert
  const int e = tid % E, g = tid / E;
  const bool act = g < G;
  const int chunk = (nb + G - 1) / G;
  const int b0 = act ? g * chunk : 0, b1 = act ? min(nb, b0 + chunk) : 0;
  const int n = b1 - b0;
  const bool in_regs = chunk <= kScanRegChunk;  // the same in every thread
  int c[kScanRegChunk];
  int sum = 0;
  constexpr int U = 8;
  if (in_regs) {
#pragma unroll
    for (int u = 0; u < kScanRegChunk; ++u) c[u] = u < n ? block_hist[(int64_t)(b0 + u) * E + e] : 0;
#pragma unroll
    for (int u = 0; u < kScanRegChunk; ++u) sum += c[u];
  } else {
    int b = b0;
    for (; b + U <= b1; b += U) {
      int cu[U];
#pragma unroll
      for (int u = 0; u < U; ++u) cu[u] = block_hist[(int64_t)(b + u) * E + e];
#pragma unroll
      for (int u = 0; u < U; ++u) sum += cu[u];
    }
    for (; b < b1; ++b) sum += block_hist[(int64_t)b * E + e];
  }
  // inclusive scan of the chunk sums over g, per expert
  part[tid] = act ? sum : 0;
  __syncthreads();
  for (int d = 1; d < G; d <<= 1) {
    const int v = act && g >= d ? part[tid - d * E] : 0;
    __syncthreads();
    if (act) part[tid] += v;
    __syncthreads();
  }
  if (tid < E) {
    const int total = part[(G - 1) * E + tid];
    cnt[tid] = total;
    counts[tid] = total;
  }
  __syncthreads();
  scan_counts(cnt, E, offsets, tile_prefix, offs, wsum);
  if (!act) return;
  int run = offs[e] + part[tid] - sum;
  if (in_regs) {
#pragma unroll
    for (int u = 0; u < kScanRegChunk; ++u)
      if (u < n) {
        block_base[(int64_t)(b0 + u) * E + e] = run;
        run += c[u];
      }
  } else {
    int b = b0;
    for (; b + U <= b1; b += U) {
      int cu[U];
#pragma unroll
      for (int u = 0; u < U; ++u) cu[u] = block_hist[(int64_t)(b + u) * E + e];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        block_base[(int64_t)(b + u) * E + e] = run;
        run += cu[u];
      }
    }
    for (; b < b1; ++b) {
      const int cv = block_hist[(int64_t)b * E + e];
      block_base[(int64_t)b * E + e] = run;
      run += cv;
    }
  }
}


// Stable scatter: position of assignment (t, j) = offset of its expert +
// number of earlier tokens (same expert) before it.  Inside a wave, the lanes
// that chose expert e are the bits of a 64-lane mask built with LDS atomic
// ORs (order-independent), so a lane's rank is a popcount of the mask below
// it; across the block's 4 waves the offsets come from per-wave counts.  A
// token picks distinct experts, so each lane is in a mask at most once.
__global__ __launch_bounds__(256) void k_scatter(const int* __restrict__ idx, int Tn, int k,
                                                 int E, const int* __restrict__ block_base,
                                                 int* __restrict__ perm,
                                                 int* __restrict__ inv_perm) {
  extern __shared__ int lds[];
  int* wcnt = lds;                                // [4][E]
  int* wbase = lds + 4 * E;                       // [4][E]
  unsigned* wmask = (unsigned*)(lds + 8 * E);     // [4][E][2] lane masks
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t = blockIdx.x * 256 + tid;
  const bool valid = t < Tn;
  for (int i = tid; i < 16 * E; i += 256) lds[i] = 0;
  __syncthreads();
  int keys[16];
  for (int j = 0; j < k; ++j) {
    keys[j] = valid ? idx[(int64_t)t * k + j] : 0;
    if (valid) {
      atomicAdd(&wcnt[wave * E + keys[j]], 1);
      atomicOr(&wmask[(wave * E + keys[j]) * 2 + (lane >> 5)], 1u << (lane & 31));
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += 256) {
    int s = 0;
    for (int w = 0; w < 4; ++w) {
      wbase[w * E + e] = s;
      s += wcnt[w * E + e];
    }
  }
  __syncthreads();
  if (!valid) return;
  const unsigned below = (1u << (lane & 31)) - 1u;
  for (int j = 0; j < k; ++j) {
    const int e = keys[j];
    const unsigned lo = wmask[(wave * E + e) * 2], hi = wmask[(wave * E + e) * 2 + 1];
    const int rank = lane < 32 ? __popc(lo & below) : __popc(lo) + __popc(hi & below);
    const int pos = block_base[(int64_t)blockIdx.x * E + e] + wbase[wave * E + e] + rank;
    perm[pos] = t * k + j;
    inv_perm[(int64_t)t * k + j] = pos;
  }
}

// Dispatch of a small batch (T <= kRouteSmallTokens, after k_route) in one
// workgroup of 1024 threads, with the bits of the multi-kernel path: P is
// summed in k_colsum_partial's order (four running sums over t mod 4, added
// in order, one lane each) and scaled as k_colsum_final does; counts,
// offsets and tile prefixes come from scan_counts; the rank of assignment
// (t, j) within its expert is the number of earlier tokens that chose the
// expert, read from a 64-bit token mask per expert (built with LDS atomic
// ORs, which do not depend on order).
constexpr int kRouteSmallTokens = 64;
__global__ __launch_bounds__(1024) void k_dispatch_small(const int* __restrict__ idx,
                                                         const float* __restrict__ probs, int Tn,
                                                         int E, int k, float scale,
                                                         float* __restrict__ P,
                                                         int* __restrict__ counts,
                                                         int* __restrict__ offsets,
                                                         int* __restrict__ tile_prefix,
                                                         int* __restrict__ perm,
                                                         int* __restrict__ inv_perm) {
  __shared__ int sidx[kRouteSmallTokens * 16];
  __shared__ unsigned tmask[1024][2];
  __shared__ int cnt[1024], offs[1024], wsum[16 * kScanCount];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) tmask[e][0] = tmask[e][1] = 0u;
  for (int i = tid; i < Tn * k; i += 1024) sidx[i] = idx[i];
  // P: lanes 4e + q hold the running sum over tokens t = q mod 4
  for (int e0 = 0; e0 < E; e0 += 256) {
    const int e = e0 + (tid >> 2), q = tid & 3;
    float r = 0.0f;
    if (e < E) {
      float v[kRouteSmallTokens / 4];
#pragma unroll
      for (int i = 0; i < kRouteSmallTokens / 4; ++i) {
        const int t = q + 4 * i;
        v[i] = t < Tn ? probs[(int64_t)t * E + e] : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < kRouteSmallTokens / 4; ++i)
        if (q + 4 * i < Tn) r += v[i];
    }
    const int base = threadIdx.x & 60;  // lanes 4e .. 4e + 3 of this wave
    const float r0 = __shfl(r, base, 64), r1 = __shfl(r, base + 1, 64);
    const float r2 = __shfl(r, base + 2, 64), r3 = __shfl(r, base + 3, 64);
    // k_colsum_final adds this single partial to three zeros: the same value
    if (e < E && q == 0) P[e] = (((r0 + r1) + r2) + r3) * scale;
  }
  __syncthreads();
  for (int i = tid; i < Tn * k; i += 1024) {
    const int t = i / k;
    atomicOr(&tmask[sidx[i]][t >> 5], 1u << (t & 31));
  }
  __syncthreads();
  if (tid < E) {
    const int c = __popc(tmask[tid][0]) + __popc(tmask[tid][1]);
    cnt[tid] = c;
    counts[tid] = c;
  }
  __syncthreads();
  scan_counts(cnt, E, offsets, tile_prefix, offs, wsum);
  for (int i = tid; i < Tn * k; i += 1024) {
    const int t = i / k, e = sidx[i];
    const unsigned lo = tmask[e][0], hi = tmask[e][1];
    const int rank = t < 32 ? __popc(lo & ((1u << t) - 1u))
                            : __popc(lo) + __popc(hi & ((1u << (t - 32)) - 1u));
    const int pos = offs[e] + rank;
    perm[pos] = i;
    inv_perm[i] = pos;
  }
}

// x_perm[inv_perm[t * k + j]] = x[t] for j < k: one wave per token reads its
// row once (16-byte vectors, up to eight per lane in flight) and writes it to
// the token's k slots of the permuted layout.  Reading each row once instead
// of k times (a wave per permuted row) keeps x out of the write stream's way
// in the caches.
template <typename T>
__global__ __launch_bounds__(256) void k_gather(const T* __restrict__ x,
                                                const int* __restrict__ inv_perm, int Tn, int k,
                                                int H, T* __restrict__ xp,
                                                const float* __restrict__ w = nullptr) {
  constexpr int V = Vec16<T>::N;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= Tn) return;
  const int lane = threadIdx.x & 63;
  const int64_t TK = (int64_t)Tn * k;
  const T* src = x + (int64_t)t * H;
  constexpr int U = 8;
  const int nv = H / V;
  for (int c0 = lane; c0 < nv; c0 += 64 * U) {
    u32x4 buf[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c0 + 64 * u < nv) buf[u] = ld16(src + (c0 + 64 * u) * V);
    for (int j = 0; j < k; ++j) {
      const int pos = inv_perm[(int64_t)t * k + j];
      if (pos < 0 || pos >= TK) continue;
      T* dst = xp + (int64_t)pos * H;
      if (w) {
        const float wj = w[(int64_t)t * k + j];
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (c0 + 64 * u < nv) {
            float f[V];
            unpack16(buf[u], f, T());
#pragma unroll
            for (int i = 0; i < V; ++i) f[i] *= wj;
            st16(dst + (c0 + 64 * u) * V, pack16(f, T()));
          }
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (c0 + 64 * u < nv) st16(dst + (c0 + 64 * u) * V, buf[u]);
      }
    }
  }
}

// The stable scatter of the fused router's 16-token groups (after the fused
// router and k_scan over its groups).  The wave of token t finds where each
// of its k choices goes: the base of its group and expert plus the number of
// earlier tokens of the group that chose the same expert, counted from the
// group's idx entries before t's (64 at a time, one ballot per choice; a
// token picks distinct experts, so each earlier token counts at most once):
// expert ascending, then token ascending.  Lane j < k writes perm and
// inv_perm for choice j.  A position outside [0, T k) (which valid routing
// never makes) is skipped.  No row is copied: the expert GEMMs read token
// rows through perm.
__global__ __launch_bounds__(256) void k_scatter_groups(const int* __restrict__ idx, int Tn,
                                                        int k, int E,
                                                        const int* __restrict__ group_base,
                                                        int* __restrict__ perm,
                                                        int* __restrict__ inv_perm) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= Tn) return;
  const int lane = threadIdx.x & 63;
  const int64_t TK = (int64_t)Tn * k;
  const int grp = t >> 4, t0 = grp << 4;
  const int mine = lane < k ? idx[(int64_t)t * k + lane] : -1;
  const int* prev = idx + (int64_t)t0 * k;
  const int nprev = (t - t0) * k;
  int rank = 0;
  for (int b = 0; b < nprev; b += 64) {
    const int v = b + lane < nprev ? prev[b + lane] : -1;
    for (int j = 0; j < k; ++j) {  // j is wave-uniform: read lane j directly
      const int ej = __builtin_amdgcn_readlane(mine, j);
      const int n = __popcll(__ballot(v == ej));
      if (lane == j) rank += n;
    }
  }
  if (lane < k && mine >= 0 && mine < E) {
    const int q = group_base[(int64_t)grp * E + mine] + rank;
    if (q >= 0 && q < TK) {
      perm[q] = t * k + lane;
      inv_perm[(int64_t)t * k + lane] = q;
    }
  }
}

// ------------------------------------------------------------------ expert GEMMs (forward)
// G = X Wg^T, U = X Wu^T, A = silu(G) * U for each row group (expert), or for
// all T rows (shared expert, groups.offsets == nullptr).  G and U are written
// only when G is not null (a forward that keeps state for a backward).
// GROUPED: expert row groups (offsets set); otherwise one dense group (a
// separate instantiation, so profiles tell the two launches apart).
// C: the tiling (Tilings<T>::GateUp, or 128-row tiles for experts with few
// rows, whose last row tile would otherwise be mostly padding).
// The last row tile of a group (an expert's rows past its last full tile, or
// the dense problem's last rows) runs as the shortest of three shorter
// tilings that covers its valid rows: BM/4 rows (QuarterRows, the four waves
// side by side along N), BM/2 rows (HalfRows, likewise) or 3BM/4 rows
// (ThreeQuarterRows, a 2 x 2 wave grid of 3BM/8-row blocks), so the MFMAs
// spend no more than BM/4 rows on padding.  Config 5's ~256-row experts run
// 79 % useful rows with BM/2 granularity and 94 % with BM/4.  Every output
// element keeps its k order (same bits).  bf16 256-row tiles only.  The BM/4-
// and BM/2-row tilings (40 and 48 KB per k-tile) run three LDS stages, within
// the LDS the full tile's epilogue already takes (config 5 gate/up forward
// 5.06 -> 4.87 ms; four stages for BM/4 were no faster).
template <class C>
using QuarterRows = Tiling<bf16_t, C::BM / 4, C::BN, C::BK, 4, 3, C::NW>;
template <class C>
using HalfRows = Tiling<bf16_t, C::BM / 2, C::BN, C::BK, 4, 3, C::NW>;
template <class C>
using ThreeQuarterRows = Tiling<bf16_t, 3 * C::BM / 4, C::BN, C::BK, C::NW / 2, C::NST, C::NW>;
template <typename T, class C>
constexpr bool has_half_rows() { return sizeof(T) == 2 && C::BM == 256; }
// A group's last full row tile also takes a tail of at most BM / 4 rows
// (TallRows: BM + BM / 4 rows, the tail's blocks shared out over the waves,
// which reuse their B fragments), instead of a BM / 4-row tile that streams
// the group's whole weight panel again.  Every bf16 256-row tiling of the
// row-grouped GEMMs has it (their tile prefixes count tiles that way).
template <class C>
using TallRows = Tiling<bf16_t, C::BM, C::BN, C::BK, C::WGN, C::NST, C::NW, C::BM / 4>;
// 384-row tiles for launches whose groups average at least three 256-row
// tiles: the BM rows of C and 128 more, one 32-row block per wave row at all
// of its columns (one fragment register set, 250-256 VGPRs).  A k-tile then
// brings 25 % more operand rows for 50 % more MFMA work.  Row tiles of at most
// BM + BM / 4 rows run as C's tilings (RowBase).
template <class C>
using Rows384 = Tiling<bf16_t, C::BM, C::BN, C::BK, C::WGN, C::NST, C::NW, C::BM / 2>;
template <class C>
using RowBase = Tiling<bf16_t, C::BM, C::BN, C::BK, C::WGN, C::NST, C::NW>;
// The 3BM/4-row tiling's wave blocks are 96 rows tall; with eight waves and
// two accumulator sets its epilogue stages them 32 rows at a time
// (epi_rows), within the LDS.
template <class C, int NACC>
constexpr bool has_three_quarter_rows() {
  return epi_lds_floats<ThreeQuarterRows<C>, NACC>() * 4 <= kLdsBytes;
}
template <typename T, class C, int NA, int NB, int NACC>
constexpr int rowgroup_smem_elems() {
  constexpr int a = kernel_smem_elems<C, T, NA, NB, NACC>();
  if constexpr (C::XR == 128) {
    constexpr int b = rowgroup_smem_elems<T, RowBase<C>, NA, NB, NACC>();
    return a > b ? a : b;
  } else if constexpr (has_half_rows<T, C>()) {
    constexpr int b = kernel_smem_elems<QuarterRows<C>, T, NA, NB, NACC>();
    constexpr int c = kernel_smem_elems<HalfRows<C>, T, NA, NB, NACC>();
    constexpr int d = has_three_quarter_rows<C, NACC>()
                          ? kernel_smem_elems<ThreeQuarterRows<C>, T, NA, NB, NACC>() : 0;
    constexpr int e = kernel_smem_elems<TallRows<C>, T, NA, NB, NACC>();
    constexpr int ab = a > b ? a : b, cd = c > d ? c : d, abcd = ab > cd ? ab : cd;
    return abcd > e ? abcd : e;
  } else {
    return a;
  }
}
// Runs body(tiling) for a resolved row tile with mv valid rows: the shortest
// row tiling that covers them (NACC: the kernel's accumulator sets); more than
// BM rows (a group's last full tile with its short tail) run as the tall tile.
template <typename T, class C, int NACC, class F>
MOE_DEV void with_tile_rows(int mv, F&& body) {
  if constexpr (C::XR == 128) {
    if (mv > C::BM + C::BM / 4) {
      body(C{});
      return;
    }
    with_tile_rows<T, RowBase<C>, NACC>(mv, body);
    return;
  }
  if constexpr (has_half_rows<T, C>()) {
    if (mv > C::BM) {
      body(TallRows<C>{});
      return;
    }
    if (mv <= C::BM / 4) {
      body(QuarterRows<C>{});
      return;
    }
    if (mv <= C::BM / 2) {
      body(HalfRows<C>{});
      return;
    }
    if constexpr (has_three_quarter_rows<C, NACC>()) {
      if (mv <= 3 * C::BM / 4) {
        body(ThreeQuarterRows<C>{});
        return;
      }
    }
  }
  body(C{});
}
// Likewise along N: a 256-column tile with at most 128 valid columns (the
// last tile column when N % 256 is in 1..128, e.g. I = 1408) runs as a
// 128-column tile with the waves stacked along M (HalfCols<C>, three LDS
// stages), with the same per-element k order (same bits).  bf16 256-column
// tiles only.
template <class C>
using HalfCols = Tiling<bf16_t, C::BM, C::BN / 2, C::BK, C::NW / 4, 3, C::NW>;
template <typename T, class C>
constexpr bool has_half_cols() { return sizeof(T) == 2 && C::BN == 256; }
template <typename T, class C, int NA, int NB, int NACC>
constexpr int rowcol_smem_elems() {
  constexpr int a = rowgroup_smem_elems<T, C, NA, NB, NACC>();
  if constexpr (C::XR == 128) {
    constexpr int b = rowcol_smem_elems<T, RowBase<C>, NA, NB, NACC>();
    return a > b ? a : b;
  } else if constexpr (has_half_cols<T, C>()) {
    constexpr int b = kernel_smem_elems<HalfCols<C>, T, NA, NB, NACC>();
    return a > b ? a : b;
  } else {
    return a;
  }
}
// body(tiling): the tall tiling for more than BM rows, a BM/4- or BM/2-row
// tiling when that covers the mv valid rows, else the half-width tiling when
// at most BN / 2 of the nv remaining columns are valid, else the 3BM/4-row
// tiling when that covers the rows, else C.
template <typename T, class C, class F>
MOE_DEV void with_tile_shape(int mv, int nv, F&& body) {
  if constexpr (C::XR == 128) {
    if (mv > C::BM + C::BM / 4) {  // full width, as the tall tiling
      body(C{});
      return;
    }
    with_tile_shape<T, RowBase<C>>(mv, nv, body);
    return;
  }
  if constexpr (has_half_rows<T, C>()) {
    if (mv > C::BM) {  // full width even when at most BN / 2 columns are valid
      body(TallRows<C>{});
      return;
    }
    if (mv <= C::BM / 4) {
      body(QuarterRows<C>{});
      return;
    }
    if (mv <= C::BM / 2) {
      body(HalfRows<C>{});
      return;
    }
  }
  if constexpr (has_half_cols<T, C>()) {
    if (nv <= C::BN / 2) {
      body(HalfCols<C>{});
      return;
    }
  }
  if constexpr (has_half_rows<T, C>()) {
    if constexpr (has_three_quarter_rows<C, 1>()) {
      if (mv <= 3 * C::BM / 4) {
        body(ThreeQuarterRows<C>{});
        return;
      }
    }
  }
  body(C{});
}

template <typename T, bool GROUPED, class C = typename Tilings<T>::GateUp>
__global__ __launch_bounds__(C::THREADS) void k_gateup_fwd(const T* __restrict__ X, RowGroups groups,
                                                    const T* const* wg_tab, const T* wg_one,
                                                    const T* const* wu_tab, const T* wu_one,
                                                    int H, int N, T* __restrict__ G,
                                                    T* __restrict__ U, T* __restrict__ A,
                                                    const int* __restrict__ perm, int Tn, int k) {
  __shared__ __align__(16) T smem[rowgroup_smem_elems<T, C, 1, 2, 2>()];
  int grp, row0, mv, n0;
  if (!resolve_rows(groups, N, C::AR, C::BN, grp, row0, mv, n0)) return;
  const T* wg = pick(wg_tab, wg_one, grp);
  const T* wu = pick(wu_tab, wu_one, grp);
  with_tile_rows<T, C, 2>(mv, [&](auto ct) {
    using CT = decltype(ct);
    // grouped: the token rows of x, gathered in expert order (row r is token
    // perm[r] / k); dense: X's rows
    OpDesc<T> a[1] = {{X + (int64_t)row0 * H, H, mv, H}};
    if constexpr (GROUPED) a[0] = {X, H, mv, H, perm + row0, Tn, k};
    OpDesc<T> b[2] = {{wg + (int64_t)n0 * H, H, N - n0, H}, {wu + (int64_t)n0 * H, H, N - n0, H}};
    f32x16 acc[2][CT::TN][CT::TM], xacc[2][CT::XTN];
    zero_acc<CT, 2>(acc, xacc);
    mainloop_x<CT, T, false, false, 1, 2, GROUPED>(acc, xacc, a, b, H, smem);
    static_assert(epi_lds_floats<CT, 2>() * 4 <= (int)sizeof(smem), "epilogue LDS");
    for_each_row8_x<CT, 2>(acc, xacc, reinterpret_cast<float*>(smem), [&](int m, int n, auto& v) {
      if (m >= mv || n0 + n >= N) return;
      float act[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) act[i] = silu_f(v[0][i]) * v[1][i];
      const int64_t o = (int64_t)(row0 + m) * N + n0 + n;
      if (G) {  // pre-activations are kept only for a backward
        store8(G + o, v[0]);
        store8(U + o, v[1]);
      }
      store8(A + o, act);
    });
  });
}

// Y = A Wd^T per row group (K = I) or for the dense shared expert.  orow
// (grouped, not null): output row r goes to row orow[r] (the permutation:
// slot t * k + j), so the combine reads a token's k rows as one contiguous
// block; the row indices of a pass are loaded one pass ahead.
template <typename T, bool GROUPED, class C = typename Tilings<T>::Big>
__global__ __launch_bounds__(C::THREADS) void k_down_fwd(const T* __restrict__ A, RowGroups groups,
                                                  const T* const* wd_tab, const T* wd_one, int I,
                                                  int H, T* __restrict__ Y,
                                                  const int* __restrict__ orow) {
  __shared__ __align__(16) T smem[rowgroup_smem_elems<T, C, 1, 1, 1>()];
  int grp, row0, mv, n0;
  if (!resolve_rows(groups, H, C::AR, C::BN, grp, row0, mv, n0)) return;
  const T* wd = pick(wd_tab, wd_one, grp);
  with_tile_rows<T, C, 1>(mv, [&](auto ct) {
    using CT = decltype(ct);
    OpDesc<T> a[1] = {{A + (int64_t)row0 * I, I, mv, I}};
    OpDesc<T> b[1] = {{wd + (int64_t)n0 * I, I, H - n0, I}};
    f32x16 acc[1][CT::TN][CT::TM], xacc[1][CT::XTN];
    zero_acc<CT, 1>(acc, xacc);
    mainloop_x<CT, T, false, false, 1, 1>(acc, xacc, a, b, I, smem);
    static_assert(epi_lds_floats<CT, 1>() * 4 <= (int)sizeof(smem), "epilogue LDS");
    if (GROUPED && orow) {
      struct Pre { int r; };
      const rsrc_t ro = make_rsrc(orow + row0, (uint32_t)mv * 4u);
      for_each_row8_xpre<CT, 1, Pre>(acc, xacc, reinterpret_cast<float*>(smem),
                                     [&](int m, int, Pre& q) {
        q.r = (int)__builtin_amdgcn_raw_buffer_load_b32(ro, m < mv ? (uint32_t)m * 4u : kOobOffset, 0, 0);
      }, [&](int m, int n, auto& v, const Pre& q) {
        if (m >= mv || n0 + n >= H) return;
        store8(Y + (int64_t)q.r * H + n0 + n, v[0]);
      });
    } else {
      for_each_row8_x<CT, 1>(acc, xacc, reinterpret_cast<float*>(smem), [&](int m, int n, auto& v) {
        if (m >= mv || n0 + n >= H) return;
        store8(Y + (int64_t)(row0 + m) * H + n0 + n, v[0]);
      });
    }
  });
}

// ------------------------------------------------------------------ combine
// out[t] = sum_j w[t, j] * Y[inv_perm[t, j]] (+ s * Ys[t]) (+ resid[t]), added in
// that order in fp32 and rounded once (inv_perm == nullptr: Y is token-major,
// row t * k + j, as the grouped down projection writes it).  One wave per (token, slice of 64
// 16-byte vectors of the row); the k expert rows of a slice are all requested
// before the first one is added.
constexpr int kCombineSlice = 64;  // 16-byte vectors per wave
template <typename T>
__global__ __launch_bounds__(256) void k_combine_fwd(const T* __restrict__ Y,
                                                     const int* __restrict__ inv_perm,
                                                     const float* __restrict__ w,
                                                     const T* __restrict__ Ys, float s, int Tn,
                                                     int k, int H, const T* __restrict__ resid,
                                                     T* __restrict__ out) {
  constexpr int V = Vec16<T>::N;
  const int nv = H / V;
  const int nsl = (nv + kCombineSlice - 1) / kCombineSlice;
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= (int64_t)Tn * nsl) return;
  const int t = (int)(wid / nsl), sl = (int)(wid % nsl);
  const int c = sl * kCombineSlice + (threadIdx.x & 63);
  if (c >= nv) return;
  const int64_t TK = (int64_t)Tn * k;
  u32x4 ya[16];
  float wj[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    if (j < k) {
      int64_t p = inv_perm ? inv_perm[(int64_t)t * k + j] : (int64_t)t * k + j;
      p = p < 0 ? 0 : (p >= TK ? TK - 1 : p);
      wj[j] = w[(int64_t)t * k + j];
      ya[j] = ld16(Y + p * H + c * V);
    }
  }
  u32x4 ys{}, rs{};
  if (Ys) ys = ld16(Ys + (int64_t)t * H + c * V);
  if (resid) rs = ld16(resid + (int64_t)t * H + c * V);
  float acc[V], y[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    if (j < k) {
      unpack16(ya[j], y, T());
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] += wj[j] * y[i];
    }
  }
  if (Ys) {
    unpack16(ys, y, T());
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] += s * y[i];
  }
  if (resid) {  // the block's residual add, fused
    unpack16(rs, y, T());
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] += y[i];
  }
  st16(out + (int64_t)t * H + c * V, pack16(acc, T()));
}

// dY[pos] = w[t, j] * dout[t] for the down projection's weight gradient (its
// input gradient reads d_out rows directly, and the combine weights' gradient
// comes from that kernel's epilogue).  One wave per token: it reads the row
// once, 8 vectors per lane at a time, and writes its k weighted copies.
template <typename T>
__global__ __launch_bounds__(256) void k_combine_bwd(const T* __restrict__ dout,
                                                     const int* __restrict__ inv_perm,
                                                     const float* __restrict__ w, int Tn, int k,
                                                     int H, T* __restrict__ dY) {
  constexpr int V = Vec16<T>::N;
  constexpr int U = 8;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= Tn) return;
  const int lane = threadIdx.x & 63;
  const int64_t TK = (int64_t)Tn * k;
  // lane j < k holds slot j's row and weight; read back wave-uniformly
  int64_t mypos = 0;
  float myw = 0.0f;
  if (lane < k) {
    const int64_t p = inv_perm[(int64_t)t * k + lane];
    mypos = p < 0 ? 0 : (p >= TK ? TK - 1 : p);
    myw = w[(int64_t)t * k + lane];
  }
  const int nv = H / V;
  const T* src = dout + (int64_t)t * H;
  for (int b0 = 0; b0 < nv; b0 += 64 * U) {
    float d[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (b0 + lane + 64 * u < nv) unpack16(ld16(src + (b0 + lane + 64 * u) * V), d[u], T());
    for (int j = 0; j < k; ++j) {
      const int64_t pj = __shfl(mypos, j, 64);
      const float wj = __shfl(myw, j, 64);
      T* dst = dY + pj * H;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = b0 + lane + 64 * u;
        if (c < nv) {
          float o[V];
#pragma unroll
          for (int i = 0; i < V; ++i) o[i] = wj * d[u][i];
          st16(dst + c * V, pack16(o, T()));
        }
      }
    }
  }
}

// v of lane l ^ X within each group of four lanes (DPP quad_perm, X = 1 or 2).
template <int X>
MOE_DEV float quad_xor(float v) {
  constexpr int ctrl = X == 1 ? 0xB1 : 0x4E;  // quad_perm [1,0,3,2] / [2,3,0,1]
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false));
}

// ------------------------------------------------------------------ expert GEMMs (backward)
// dA = alpha * dY Wd (NN, K = H), then the SwiGLU backward in the epilogue:
// dG = dA * U * silu'(G), dU = dA * silu(G).
// GROUPED (routed experts): the A operand is the token rows of d_out itself,
// gathered in expert order (permuted row r is token perm[r] / k), and the
// routing weight w_r is left out: dY[r] = w_r d_out[t_r], so dA = w_r dA_u with
// dA_u = d_out[t_r] Wd, and the epilogue writes the unweighted dG_u, dU_u
// (dG = w_r dG_u, dU = w_r dU_u).  The weight is applied where those are
// consumed: the gate/up weight gradient multiplies by w_r X[r] (its token rows
// are built weighted), and dx adds w_tj times each gathered row of the gate/up
// input gradient.  The epilogue also forms the combine weights' gradient from
// the unweighted product: dw_r = <d_out[t_r], Y[r]> = <dA_u[r], A[r]> with
// A = silu(G) U rebuilt from the G and U it loads anyway; each 32-column
// block's part (8 products per lane, in order, then the 4 lanes of the row
// as (l0 + l1) + (l2 + l3)) goes to dwp[block][r], and k_dw_sum adds the
// blocks in order.  Dense (shared expert): dY = dY_dense, weight alpha.
template <typename T, bool GROUPED, class C = typename Tilings<T>::Big>
__global__ __launch_bounds__(C::THREADS) void k_down_dgrad(const T* __restrict__ dY, RowGroups groups,
                                                    const T* const* wd_tab, const T* wd_one,
                                                    int H, int N, float alpha,
                                                    const T* __restrict__ G,
                                                    const T* __restrict__ U,
                                                    T* __restrict__ dG, T* __restrict__ dU,
                                                    const int* __restrict__ perm, int Tn, int k,
                                                    float* __restrict__ dwp) {
  __shared__ __align__(16) T smem[rowcol_smem_elems<T, C, 1, 1, 1>()];
  int grp, row0, mv, n0;
  if (!resolve_rows(groups, N, C::AR, C::BN, grp, row0, mv, n0)) return;
  const T* wd = pick(wd_tab, wd_one, grp);  // [H, N]: element (n, k=h) at wd + h*N + n
  // G and U of a whole 32-column block are requested before its rows are
  // visited; rows outside the tile read zeros (out-of-range offsets).  The
  // resources start at the tile's first row and cover its mv rows, so the
  // 32-bit offsets stay small whatever the number of routed rows.
  constexpr int NV = (int)sizeof(T) / 2;  // 16-byte vectors per 8 elements
  struct Pre {
    u32x4 gu[2 * NV];  // G, then U
  };
  const int64_t tile_base = (int64_t)row0 * N;
  const rsrc_t rg = make_rsrc(G + tile_base, (uint32_t)((int64_t)mv * N * sizeof(T)));
  const rsrc_t ru = make_rsrc(U + tile_base, (uint32_t)((int64_t)mv * N * sizeof(T)));
  auto pre = [&](int m, int n, Pre& q) {
    const bool in = m < mv && n0 + n < N;
    const uint32_t off = in ? (uint32_t)(((int64_t)m * N + n0 + n) * sizeof(T)) : kOobOffset;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      q.gu[j] = buf_ld16(rg, off + 16 * j, 0);
      q.gu[NV + j] = buf_ld16(ru, off + 16 * j, 0);
    }
  };
  with_tile_shape<T, C>(mv, N - n0, [&](auto ct) {
    using CT = decltype(ct);
    OpDesc<T> a[1] = {{dY + (int64_t)row0 * H, H, mv, H}};
    if constexpr (GROUPED) a[0] = {dY, H, mv, H, perm + row0, Tn, k};
    OpDesc<T> b[1] = {{wd + n0, N, N - n0, H}};
    f32x16 acc[1][CT::TN][CT::TM], xacc[1][CT::XTN];
    zero_acc<CT, 1>(acc, xacc);
    mainloop_x<CT, T, false, true, 1, 1, GROUPED>(acc, xacc, a, b, H, smem);
    static_assert(epi_lds_floats<CT, 1>() * 4 <= (int)sizeof(smem), "epilogue LDS");
    for_each_row8_xpre<CT, 1, Pre>(acc, xacc, reinterpret_cast<float*>(smem), pre,
                                   [&](int m, int n, auto& v, const Pre& q) {
      const bool ok = m < mv && n0 + n < N;
      float g[8], u[8], dg[8], du[8];
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        unpack16(q.gu[j], g + j * (8 / NV), T());
        unpack16(q.gu[NV + j], u + j * (8 / NV), T());
      }
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float da = alpha * v[0][i];  // grouped: unweighted, d_out Wd
        const float sg = sigmoid_f(g[i]);
        const float gs = g[i] * sg;
        if constexpr (GROUPED) part += ok ? da * (gs * u[i]) : 0.0f;
        dg[i] = da * u[i] * (sg * (1.0f + g[i] * (1.0f - sg)));
        du[i] = da * gs;
      }
      if constexpr (GROUPED) {
        // the row's 4 lanes (lane / 4 equal) hold its 32-column block; DPP
        // quad permutes (lanes xor 1, then xor 2) keep the sum off the LDS
        const float p1 = part + quad_xor<1>(part);
        const float p2 = quad_xor<2>(p1);
        const bool lo = (threadIdx.x & 2) == 0;
        const float blk = lo ? p1 + p2 : p2 + p1;
        if (m < mv && (threadIdx.x & 3) == 0 && n0 + n < N)
          dwp[(int64_t)((n0 + n) >> 5) * groups.M + row0 + m] = blk;
      }
      if (!ok) return;
      const int64_t o = (int64_t)(row0 + m) * N + n0 + n;
      store8(dG + o, dg);
      store8(dU + o, du);
    });
  });
}

// dw[perm[r]] = sum over the 32-column blocks c < nb of dwp[c][r] (c ascending):
// the combine weights' gradient in (token, slot) order.
__global__ __launch_bounds__(256) void k_dw_sum(const float* __restrict__ dwp, int nb, int TK,
                                                const int* __restrict__ perm,
                                                float* __restrict__ dw) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r >= TK) return;
  // 16 loads in flight per thread, then added in block order
  constexpr int U = 16;
  float s = 0.0f;
  for (int c0 = 0; c0 < nb; c0 += U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = c0 + u < nb ? dwp[(int64_t)(c0 + u) * TK + r] : 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c0 + u < nb) s += v[u];
  }
  const int p = perm[r];
  if ((unsigned)p < (unsigned)TK) dw[p] = s;
}

// dX = dG Wg + dU Wu (NN, K = I twice) per row group.  orow (grouped, not
// null): output row r goes to row orow[r] (the permutation: slot t * k + j),
// so dx reads a token's k rows as one contiguous block; the row indices of a
// pass are loaded one pass ahead with the epilogue's prefetch.
template <typename T, bool GROUPED, class C = typename Tilings<T>::Big>
__global__ __launch_bounds__(C::THREADS) void k_gateup_dgrad(const T* __restrict__ dG,
                                                      const T* __restrict__ dU, RowGroups groups,
                                                      const T* const* wg_tab, const T* wg_one,
                                                      const T* const* wu_tab, const T* wu_one,
                                                      int I, int H, T* __restrict__ dX,
                                                      const int* __restrict__ orow) {
  __shared__ __align__(16) T smem[rowgroup_smem_elems<T, C, 1, 1, 1>()];
  int grp, row0, mv, n0;
  if (!resolve_rows(groups, H, C::AR, C::BN, grp, row0, mv, n0)) return;
  const T* wg = pick(wg_tab, wg_one, grp);  // [I, H]: element (n=h, k=i) at wg + i*H + h
  const T* wu = pick(wu_tab, wu_one, grp);
  with_tile_rows<T, C, 1>(mv, [&](auto ct) {
    using CT = decltype(ct);
    f32x16 acc[1][CT::TN][CT::TM], xacc[1][CT::XTN];
    zero_acc<CT, 1>(acc, xacc);
    // one pipelined loop over K = 2I: the dG / Wg segment, then dU / Wu
    OpDesc<T> a[1] = {{dG + (int64_t)row0 * I, I, mv, I}};
    OpDesc<T> b[1] = {{wg + n0, H, H - n0, I}};
    OpDesc<T> a2[1] = {{dU + (int64_t)row0 * I, I, mv, I}};
    OpDesc<T> b2[1] = {{wu + n0, H, H - n0, I}};
    mainloop_x<CT, T, false, true, 1, 1>(acc, xacc, a, b, I, smem, a2, b2, I);
    static_assert(epi_lds_floats<CT, 1>() * 4 <= (int)sizeof(smem), "epilogue LDS");
    if (GROUPED && orow) {
      struct Pre { int r; };
      const rsrc_t ro = make_rsrc(orow + row0, (uint32_t)mv * 4u);
      for_each_row8_xpre<CT, 1, Pre>(acc, xacc, reinterpret_cast<float*>(smem),
                                     [&](int m, int, Pre& q) {
        q.r = (int)__builtin_amdgcn_raw_buffer_load_b32(ro, m < mv ? (uint32_t)m * 4u : kOobOffset, 0, 0);
      }, [&](int m, int n, auto& v, const Pre& q) {
        if (m >= mv || n0 + n >= H) return;
        store8(dX + (int64_t)q.r * H + n0 + n, v[0]);
      });
    } else {
      for_each_row8_x<CT, 1>(acc, xacc, reinterpret_cast<float*>(smem), [&](int m, int n, auto& v) {
        if (m >= mv || n0 + n >= H) return;
        store8(dX + (int64_t)(row0 + m) * H + n0 + n, v[0]);
      });
    }
  });
}

// Weight gradients, K-grouped over token rows (TN):
//   W_a[g][m, n] = alpha * sum_r P_a[r, m] * Q[r, n],  r over the group's rows,
// with NA = 1 (single) or 2 (two P operands sharing Q).  P is [rows, M]
// (ld = ldp), Q is [rows, N] (ld = ldq), outputs [M, N].
template <typename T, int NA>
using WgradTiling = typename std::conditional<NA == 2, typename Tilings<T>::WgradPair,
                                              typename Tilings<T>::Big>::type;
template <typename T, int NA, bool GROUPED>
MOE_DEV void wgrad_tile(T* smem, int blk, const T* __restrict__ P0, const T* __restrict__ P1,
                        int64_t ldp, const T* __restrict__ Q, int64_t ldq, const KGroups& groups,
                        int M, int N, float alpha, T* const* out0_tab, T* out0_one,
                        T* const* out1_tab, T* out1_one, float* __restrict__ partial) {
  using C = WgradTiling<T, NA>;
  int grp, split, krow0, K, m0, n0;
  if (!resolve_k(groups, blk, M, N, C::BM, C::BN, grp, split, krow0, K, m0, n0)) return;
  OpDesc<T> a[NA];
  a[0] = {P0 + krow0 * ldp + m0, ldp, M - m0, K};
  if constexpr (NA == 2) a[1] = {P1 + krow0 * ldp + m0, ldp, M - m0, K};
  OpDesc<T> b[1] = {{Q + krow0 * ldq + n0, ldq, N - n0, K}};
  f32x16 acc[NA][C::TN][C::TM];
  zero_acc<C, NA>(acc);
  mainloop<C, T, true, true, NA, 1>(acc, a, b, K, smem);
  T* o0 = pick(out0_tab, out0_one, grp);
  T* o1 = NA == 2 ? pick(out1_tab, out1_one, grp) : nullptr;
  const int mv = min(C::BM, M - m0);
  if constexpr (GROUPED && sizeof(T) == 2) {
    // groups never split: alpha * acc rounded once, as store8 of the scaled
    // value; the bf16 staging halves the epilogue's LDS traffic.  The packing
    // copies the accumulators into VGPRs, which spilled while the split
    // branch below shared the kernel; here that branch is compiled out.
    static_assert(epi_lds_bf16_elems<C, NA>() * 2 <= kernel_smem_elems<C, T, NA, 1, NA>() * (int)sizeof(T), "epilogue LDS");
    for_each_row8_bf16<C, NA>(acc, reinterpret_cast<bf16_t*>(smem), alpha,
                              [&](int m, int n, const u32x4 (&p)[NA]) {
      if (m >= mv || n0 + n >= N) return;
      const int64_t o = (int64_t)(m0 + m) * N + n0 + n;
      *gptr(reinterpret_cast<u32x4*>(o0 + o)) = p[0];
      if constexpr (NA == 2) *gptr(reinterpret_cast<u32x4*>(o1 + o)) = p[NA - 1];
    });
    return;
  }
  static_assert(epi_lds_floats<C, NA>() * 4 <= kernel_smem_elems<C, T, NA, 1, NA>() * (int)sizeof(T), "epilogue LDS");
  if (groups.nsplit > 1) {  // fp32 partial tile of this chunk, [NA][nsplit][M][N]
    const int64_t MN = (int64_t)M * N;
    for_each_row8<C, NA>(acc, reinterpret_cast<float*>(smem), [&](int m, int n, auto& v) {
      if (m >= mv || n0 + n >= N) return;
      const int64_t o = (int64_t)(m0 + m) * N + n0 + n;
#pragma unroll
      for (int x = 0; x < NA; ++x) store8(partial + ((int64_t)x * groups.nsplit + split) * MN + o, v[x]);
    });
    return;
  }
  for_each_row8<C, NA>(acc, reinterpret_cast<float*>(smem), [&](int m, int n, auto& v) {
    if (m >= mv || n0 + n >= N) return;
    const int64_t o = (int64_t)(m0 + m) * N + n0 + n;
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = alpha * v[0][i];
    store8(o0 + o, r);
    if constexpr (NA == 2) {
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = alpha * v[1][i];
      store8(o1 + o, r);
    }
  });
}

// One tile per block (block b is virtual block b), except when `slots` > 0
// and either the groups run whole per XCD (xcd_order flag set, as the device
// decided from the expert counts) or the grid holds only `slots` blocks (the
// host's expectation of that flag): then the first `slots` blocks (a
// multiple of 8, at most one per CU) are persistent and block b runs the
// virtual blocks b, b + slots, ... below vblocks, each keeping the XCD of the
// block it stands for; the other blocks of a full grid leave at once.  Every
// virtual block is computed once by one workgroup either way, so the results
// are the same bits.  A persistent workgroup issues its next tile's first
// loads while the previous tile's output stores drain, where a new workgroup
// could only start after them (a wave ends by waiting for its stores):
// config 5 gate/up pair 6.57 -> 5.86 ms alone.  With every expert's tiles
// dealt over all XCDs instead (skewed counts), tiles of very different K
// would land unevenly on a static schedule, and the hardware's dispatch
// balances them better.
template <typename T, int NA, bool GROUPED>
__global__ __launch_bounds__((WgradTiling<T, NA>::THREADS)) void k_wgrad(const T* __restrict__ P0, const T* __restrict__ P1,
                                               int64_t ldp, const T* __restrict__ Q, int64_t ldq,
                                               KGroups groups, int M, int N, float alpha,
                                               T* const* out0_tab, T* out0_one,
                                               T* const* out1_tab, T* out1_one,
                                               float* __restrict__ partial, int vblocks,
                                               int slots) {
  using C = WgradTiling<T, NA>;
  __shared__ __align__(16) T smem[kernel_smem_elems<C, T, NA, 1, NA>()];
  // a grid of `slots` blocks (the host expected whole experts per XCD) runs
  // persistent whatever the flag says; a full grid only when the flag is set
  const bool reduced = (int)gridDim.x < vblocks;
  const bool persist =
      slots > 0 && (reduced || (groups.xcd_order && groups.xcd_order[groups.G]));
  if (!persist) {
    wgrad_tile<T, NA, GROUPED>(smem, (int)blockIdx.x, P0, P1, ldp, Q, ldq, groups, M, N, alpha,
                               out0_tab, out0_one, out1_tab, out1_one, partial);
    return;
  }
  for (int vb = (int)blockIdx.x; blockIdx.x < (unsigned)slots && vb < vblocks; vb += slots) {
    wgrad_tile<T, NA, GROUPED>(smem, vb, P0, P1, ldp, Q, ldq, groups, M, N, alpha, out0_tab,
                               out0_one, out1_tab, out1_one, partial);
    __syncthreads();  // the next tile's loads overwrite the epilogue's LDS
  }
}

// out_x[i] = alpha * sum_s partial[x][s][i], s ascending; 8 elements per thread.
template <typename T>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ partial,
                                                       int nsplit, int64_t MN, float alpha,
                                                       T* __restrict__ out0, T* __restrict__ out1) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i >= MN) return;
  const int x = blockIdx.y;
  T* out = x == 0 ? out0 : out1;
  float acc[8], v[8];
  load8(partial + (int64_t)x * nsplit * MN + i, acc);
  for (int s = 1; s < nsplit; ++s) {
    load8(partial + ((int64_t)x * nsplit + s) * MN + i, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += v[e];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] *= alpha;
  store8(out + i, acc);
}

// ------------------------------------------------------------------ router backward
// d logits from the routing-weight gradients dw, the aux loss (through P_e)
// and the z loss, through the softmax Jacobian; one wave per token.
template <typename T, int EPL>
__global__ __launch_bounds__(256) void k_router_bwd(
    const float* __restrict__ probs, const float* __restrict__ lse, const int* __restrict__ idx,
    const float* __restrict__ w, const float* __restrict__ dw, const float* __restrict__ P,
    const int* __restrict__ counts, const float* __restrict__ d_aux,
    const float* __restrict__ d_z, int Tn, int E, int Epad, int k, float tau, int norm,
    float c_sw, float c_sq, float* __restrict__ dlogits, T* __restrict__ dlogits_t) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= Tn) return;
  const float daux = d_aux ? *d_aux : 0.0f;
  const float dz = d_z ? *d_z : 0.0f;
  const float inv_tk = 1.0f / ((float)Tn * (float)k);
  float p[EPL], dp[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    p[i] = e < E ? probs[(int64_t)t * E + e] : 0.0f;
    dp[i] = e < E ? daux * (float)E *
                        (c_sw * ((float)counts[e] * inv_tk) + 2.0f * c_sq * P[e]) / (float)Tn
                  : 0.0f;
  }
  float psum = 0.0f, wdot = 0.0f;
  if (norm) {
    for (int j = 0; j < k; ++j) {
      psum += probs[(int64_t)t * E + idx[(int64_t)t * k + j]];
      wdot += dw[(int64_t)t * k + j] * w[(int64_t)t * k + j];
    }
  }
  for (int j = 0; j < k; ++j) {
    const int e = idx[(int64_t)t * k + j];
    const float g = norm ? (dw[(int64_t)t * k + j] - wdot) / psum : dw[(int64_t)t * k + j];
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (lane + 64 * i == e) dp[i] += g;
  }
  float dot = 0.0f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) dot += p[i] * dp[i];
  dot = wave_sum(dot);
  const float zc = dz * 2.0f / (float)Tn * lse[t];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    if (e < E) {
      const float ds = p[i] * (dp[i] - dot) + zc * p[i];
      const float dl = ds / tau;
      dlogits[(int64_t)t * E + e] = dl;
      dlogits_t[(int64_t)t * Epad + e] = from_f<T>(dl);
    } else if (e < Epad) {
      dlogits_t[(int64_t)t * Epad + e] = from_f<T>(0.0f);
    }
  }
}

// dx = dlogits Wr (NN, K = E) + sum_j w[t, j] dXp[inv_perm[t, j]] + dxs[t]
// (the rows of the gate/up input gradient are unweighted: w[t, j] multiplies
// them here, one product per gathered element).  inv_perm == nullptr: dXp is
// token-major (row t * k + j), as the grouped gate/up input gradient writes it.
// The whole fp32 accumulator tile is staged in LDS (rows of BN + 4 floats)
// and read back by units of 8 outputs: 16 consecutive lanes cover 128
// consecutive columns of one row, so every gathered dXp row segment is read
// as whole 128-byte lines by one instruction.  (Visiting one 32-column block
// at a time read half lines, whose other half came back from memory a block
// later.)  KMAX >= k, a power of two, sizes the units each thread keeps in
// flight.  Per output: the
// accumulator, then the k weighted gathered rows in slot order, then dxs.
template <typename T>
constexpr int dgrad_smem_elems() {
  using C = typename Tilings<T>::RouterDx;
  constexpr int a = kernel_smem_elems<C, T, 1, 1, 1>();
  constexpr int b = C::BM * (C::BN + 4) * 4 / (int)sizeof(T);
  return a > b ? a : b;
}
template <typename T, int KMAX>
__global__ __launch_bounds__(256) void k_router_dgrad(const T* __restrict__ dl, int Epad, int E,
                                                      const T* __restrict__ wr, int Tn, int H,
                                                      const T* __restrict__ dXp,
                                                      const int* __restrict__ inv_perm, int k,
                                                      const float* __restrict__ topw,
                                                      const T* __restrict__ dxs,
                                                      T* __restrict__ dx) {
  using C = typename Tilings<T>::RouterDx;
  static_assert(C::THREADS == 256 && C::BN == 128, "16 units of 8 columns per row, 16 rows per pass");
  __shared__ __align__(16) T smem[dgrad_smem_elems<T>()];
  // row-major tile order: the column tiles of one row block run together, so
  // the pieces of every gathered dXp row are read at about the same time
  const int ntn = (H + C::BN - 1) / C::BN;
  const int row0 = (int)(blockIdx.x / ntn) * C::BM, n0 = (int)(blockIdx.x % ntn) * C::BN;
  if (row0 >= Tn) return;
  const int mv = min(C::BM, Tn - row0);
  OpDesc<T> a[1] = {{dl + (int64_t)row0 * Epad, Epad, mv, Epad}};
  OpDesc<T> b[1] = {{wr + n0, H, H - n0, E}};
  f32x16 acc[1][C::TN][C::TM];
  zero_acc<C, 1>(acc);
  mainloop<C, T, false, true, 1, 1>(acc, a, b, Epad, smem);
  // the main loop ends with a barrier: its stages are free
  constexpr int P = C::BN + 4;
  float* tile = reinterpret_cast<float*>(smem);
  {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / C::WGN, wn = wave % C::WGN;
#pragma unroll
    for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int row = wm * C::WM + tm * 32 + (lane & 31);
          const int col = wn * C::WN + tn * 32 + 8 * qq + 4 * (lane >> 5);
          *reinterpret_cast<f32x4*>(tile + row * P + col) =
              f32x4{acc[0][tn][tm][4 * qq], acc[0][tn][tm][4 * qq + 1],
                    acc[0][tn][tm][4 * qq + 2], acc[0][tn][tm][4 * qq + 3]};
        }
  }
  __syncthreads();
  const int64_t TK = (int64_t)Tn * k;
  constexpr int NV = (int)sizeof(T) / 2;  // 16-byte vectors per 8 elements
  const int cu = threadIdx.x & 15;        // unit (8 columns) of the row
  const int n = n0 + cu * 8;
  const bool nin = n < H;
  // U units per step, rows r0, r0 + 16, ..., sized so that U * KMAX * NV
  // gathered 16-byte vectors (32 for bf16, 16 for fp32) are in flight per
  // thread
  constexpr int UW = NV == 1 ? 32 / KMAX : 8 / KMAX;
  constexpr int U = UW < 1 ? 1 : UW > C::BM / 16 ? C::BM / 16 : UW;
  static_assert(U >= 1 && (C::BM / 16) % U == 0, "units per step");
  for (int r0 = threadIdx.x >> 4; r0 < C::BM; r0 += 16 * U) {
    u32x4 raw[U][KMAX][NV], rs[U][NV];
    float wt[U][KMAX];
    bool ok[U];
#pragma unroll
    for (int h2 = 0; h2 < U; ++h2) {
      const int r = r0 + 16 * h2;
      ok[h2] = nin && r < mv;
      const int t = row0 + r;
#pragma unroll
      for (int j = 0; j < KMAX; ++j) {
        if (j < k && ok[h2]) {
          // token-major rows (inv_perm null) or expert-major ones
          int64_t p = inv_perm ? inv_perm[(int64_t)t * k + j] : (int64_t)t * k + j;
          p = p < 0 ? 0 : (p >= TK ? TK - 1 : p);
          wt[h2][j] = topw[(int64_t)t * k + j];
#pragma unroll
          for (int h = 0; h < NV; ++h)
            raw[h2][j][h] = *gptr(reinterpret_cast<const u32x4*>(dXp + p * H + n + h * (8 / NV)));
        }
      }
      if (dxs && ok[h2]) {
#pragma unroll
        for (int h = 0; h < NV; ++h)
          rs[h2][h] = *gptr(reinterpret_cast<const u32x4*>(dxs + (int64_t)t * H + n + h * (8 / NV)));
      }
    }
#pragma unroll
    for (int h2 = 0; h2 < U; ++h2) {
      if (!ok[h2]) continue;
      const int r = r0 + 16 * h2;
      float v[8], q[8];
      const f32x4 lo = *reinterpret_cast<const f32x4*>(tile + r * P + cu * 8);
      const f32x4 hi = *reinterpret_cast<const f32x4*>(tile + r * P + cu * 8 + 4);
      v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
      v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
#pragma unroll
      for (int j = 0; j < KMAX; ++j) {
        if (j < k) {
#pragma unroll
          for (int h = 0; h < NV; ++h) unpack16(raw[h2][j][h], q + h * (8 / NV), T());
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] += wt[h2][j] * q[i];
        }
      }
      if (dxs) {
#pragma unroll
        for (int h = 0; h < NV; ++h) unpack16(rs[h2][h], q + h * (8 / NV), T());
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] += q[i];
      }
      store8(dx + (int64_t)(row0 + r) * H + n, v);
    }
  }
}

__global__ void k_has_grad(const int* __restrict__ counts, int E, uint8_t* __restrict__ has_grad) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e < E) has_grad[e] = counts[e] > 0 ? 1 : 0;
}

// Sets n bytes at p to zero: 16-byte stores where p + i is 16-byte aligned
// and whole, single bytes otherwise.  A kernel rather than hipMemsetAsync, so
// a caller may capture the call in a HIP graph.
__global__ __launch_bounds__(256) void k_zero(uint8_t* __restrict__ p, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16;
  if (i >= n) return;
  if ((((uintptr_t)(p + i)) & 15u) == 0 && i + 16 <= n) {
    *reinterpret_cast<u32x4*>(p + i) = u32x4{0u, 0u, 0u, 0u};
    return;
  }
  const int64_t end = i + 16 < n ? i + 16 : n;
  for (int64_t j = i; j < end; ++j) p[j] = 0;
}

// ------------------------------------------------------------------ fused RMSNorm (block path)
// The MoE sub-block of a decoder block (src/model.rs:2792-2800):
//   x = RMSNorm(h) = h * rstd * w,  rstd = 1 / sqrt(mean_i h_i^2 + eps),
//   out = MoE(x) + h  (the residual add is fused into k_combine_fwd).
// Statistics and products in fp32, one rounding of x to the dtype; one wave
// per token row, lanes over 16-byte vectors.
template <typename T>
__global__ __launch_bounds__(256) void k_rmsnorm_fwd(const T* __restrict__ h,
                                                     const T* __restrict__ w, float eps, int Tn,
                                                     int H, T* __restrict__ x,
                                                     float* __restrict__ rstd) {
  constexpr int V = Vec16<T>::N;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= Tn) return;
  const int lane = threadIdx.x & 63;
  const T* row = h + (int64_t)t * H;
  float ss = 0.0f;
  for (int c = lane; c < H / V; c += 64) {
    float v[V];
    unpack16(ld16(row + c * V), v, T());
#pragma unroll
    for (int i = 0; i < V; ++i) ss += v[i] * v[i];
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)H + eps);
  if (lane == 0) rstd[t] = r;
  for (int c = lane; c < H / V; c += 64) {
    float v[V], g[V];
    unpack16(ld16(row + c * V), v, T());
    unpack16(ld16(w + c * V), g, T());
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = v[i] * r * g[i];
    st16(x + (int64_t)t * H + c * V, pack16(v, T()));
  }
}

// RMSNorm backward with the residual's gradient:
//   dh = d_out + rstd * (w * dx - xhat * mean_i(xhat_i * w_i * dx_i)),  xhat = h * rstd,
// and per-block partial rows of the weight gradient,
//   part[b][i] = sum over the block's rows (ascending) of dx_i * xhat_i.
// One block of 256 threads per kRmsRows consecutive rows; thread j owns the
// 8-column chunks j, j + 256, ... (NCH of them, H <= 2048 * NCH).
constexpr int kRmsRows = 8;
template <typename T, int NCH>
__global__ __launch_bounds__(256) void k_rmsnorm_bwd(const T* __restrict__ dx,
                                                     const T* __restrict__ h,
                                                     const T* __restrict__ w,
                                                     const float* __restrict__ rstd,
                                                     const T* __restrict__ dout, int Tn, int H,
                                                     T* __restrict__ dh, float* __restrict__ part) {
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nch = H / 8;
  float wv[NCH][8], acc[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int ch = tid + c * 256;
#pragma unroll
    for (int i = 0; i < 8; ++i) wv[c][i] = acc[c][i] = 0.0f;
    if (ch < nch) load8(w + ch * 8, wv[c]);
  }
  const int t0 = blockIdx.x * kRmsRows, t1 = min(Tn, t0 + kRmsRows);
  // dx and h of the next row are requested before this row's reduction
  float dn[NCH][8], hn[NCH][8];
  auto load_row = [&](int t) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int ch = tid + c * 256;
      if (ch < nch) {
        load8(dx + (int64_t)t * H + ch * 8, dn[c]);
        load8(h + (int64_t)t * H + ch * 8, hn[c]);
      }
    }
  };
  if (t0 < t1) load_row(t0);
  for (int t = t0; t < t1; ++t) {
    const float r = rstd[t];
    float d[NCH][8], xh[NCH][8];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        d[c][i] = dn[c][i];
        xh[c][i] = hn[c][i];
      }
    if (t + 1 < t1) load_row(t + 1);
    float dot = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int ch = tid + c * 256;
      if (ch < nch) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          xh[c][i] *= r;
          dot += xh[c][i] * wv[c][i] * d[c][i];
        }
      }
    }
    dot = wave_sum(dot);
    if (lane == 0) red[wave] = dot;
    __syncthreads();
    const float mean = ((red[0] + red[1]) + (red[2] + red[3])) / (float)H;
    __syncthreads();  // red is rewritten by the next row
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int ch = tid + c * 256;
      if (ch < nch) {
        float g[8], o[8];
        load8(dout + (int64_t)t * H + ch * 8, g);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          o[i] = g[i] + r * (wv[c][i] * d[c][i] - xh[c][i] * mean);
          acc[c][i] += d[c][i] * xh[c][i];
        }
        store8(dh + (int64_t)t * H + ch * 8, o);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int ch = tid + c * 256;
    if (ch < nch) store8(part + (int64_t)blockIdx.x * H + ch * 8, acc[c]);
  }
}

// out[g][i] = sum of in[r][i] over the rows r of group g (rpg rows, ascending);
// 8 columns per thread.  Applied level by level, it reduces partial rows in a
// fixed tree, independent of scheduling.
template <typename OUT>
__global__ __launch_bounds__(256) void k_rowsum(const float* __restrict__ in, int R, int H,
                                                int rpg, OUT* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i >= H) return;
  const int g = blockIdx.y, r0 = g * rpg, r1 = min(R, r0 + rpg);
  float acc[8], v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  for (int r = r0; r < r1; ++r) {
    load8(in + (int64_t)r * H + i, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += v[e];
  }
  store8(out + (int64_t)g * H + i, acc);
}

// ------------------------------------------------------------------ small-token forward
// With T <= kSkinnyMaxTokens no expert holds more than that many rows, and the
// forward is a stream of the touched experts' weights.  One wave owns 16 weight
// rows and multiplies them with every token row of the expert (up to four
// chunks of 16) using v_mfma_f32_16x16x32_bf16, A = token rows, B = weight
// rows.  In a 256-wide k-chunk, MFMA step q covers k = 256 kc + 32 q + [0, 32):
// lane l (row l % 16, group g = l / 16) supplies k-vector 32 q + 8 g of its
// weight row and of its token row, so the four lanes of a row read 64
// contiguous bytes per load instruction.  Experts without tokens read
// no weights.  GATEUP: out0 = G, out1 = U, out2 = silu(G) * U from W0 = W_g,
// W1 = W_u (out0 and out1 skipped when out0 is null); otherwise out0 = X W0^T
// (down projection).
constexpr int kSkinnyMaxTokens = 64;
constexpr int kSkinnyRows = 64;  // weight rows (output columns) per workgroup
// Dynamic LDS every launch of the narrow (<= 16 tokens per expert) kernels
// reserves, unused by the kernel: half of a CU's 160 KB, so a CU holds two
// workgroups (two waves per SIMD) instead of the five its registers allow.
// Fewer concurrent weight streams read HBM faster: config 4's gate/up stream
// 69.8-70.2 % -> 71.4-72.0 % of 8 TB/s over four runs each (one workgroup per
// CU: 70.6 %; prefetching the next k-chunk at two: 68.1-68.4 %).
constexpr int kSkinnyLdsReserve = 80 * 1024;


// A pointer every lane holds, moved to scalar registers: buffer resources
// built from it then stay scalar (a resource the compiler cannot prove uniform
// costs a readfirstlane loop around every load).
template <typename T>
MOE_DEV const T* uni_ptr(const T* p) {
  const uint64_t a = (uint64_t)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  return (const T*)(((uint64_t)hi << 32) | lo);
}

// The expert holding the j-th (from 0) group of more than 16 rows, or -1:
// each wave counts the wide groups 64 at a time with a ballot.  Uniform.
MOE_DEV int nth_wide_group(const int* offsets, int G, int j) {
  const int lane = threadIdx.x & 63;
  int seen = 0;
  for (int base = 0; base < G; base += 64) {
    const int e = base + lane;
    const bool wide = e < G && offsets[e + 1] - offsets[e] > 16;
    uint64_t m = __ballot(wide);
    const int n = __popcll(m);
    if (j < seen + n) {
      for (int i = seen; i < j; ++i) m &= m - 1;  // drop the lower wide groups
      return uni(base + __ffsll((unsigned long long)m) - 1);
    }
    seen += n;
  }
  return -1;
}
// Routed launches of the WIDE kernel need blocks for at most this many groups.
inline int max_wide_groups(int64_t rows, int G) {
  const int64_t w = rows / 17;
  return (int)(w < G ? w : G);
}

// WIDE = false handles the experts with at most 16 tokens (one chunk of token
// rows), WIDE = true those with 17..64; both are launched and each skips the
// other's experts.  The WIDE launch of a grouped problem is sized for the
// most groups that can hold 17 rows (rows / 17) and its block j / nNb takes
// the (j / nNb)-th such group.  A workgroup owns 64 consecutive weight rows (16 per wave)
// of one expert.  GATEUP: each wave streams its 16 gate rows over all of K,
// then the same 16 up rows, and applies SwiGLU in registers (a lane holds the
// gate and up values of the same outputs), so at any time a workgroup reads
// one contiguous 64-row block of one matrix: measured on the config-4 shape,
// that streams at 6.1 TB/s where reading 32 gate and 32 up rows at once
// reached 5.2.  The token loads of a k-chunk are issued as one group before
// its MFMAs, so they overlap each other instead of one L2 latency per MFMA.
template <bool GATEUP, bool WIDE>
__global__ __launch_bounds__(256) void k_skinny_fwd(const bf16_t* __restrict__ X,
                                                    const int* __restrict__ xrow, int kdiv,
                                                    int xrows,
                                                    const int* __restrict__ offsets, int ngroups,
                                                    int Mdense,
                                                    const bf16_t* const* w0_tab, const bf16_t* w0_one,
                                                    const bf16_t* const* w1_tab, const bf16_t* w1_one,
                                                    int K, int N, bf16_t* __restrict__ out0,
                                                    bf16_t* __restrict__ out1,
                                                    bf16_t* __restrict__ out2) {
  constexpr int ROWS_PER_WG = kSkinnyRows;
  constexpr int NC = WIDE ? 4 : 1;
  constexpr int NM = GATEUP ? 2 : 1;  // weight matrices streamed in turn
  const int nNb = (N + ROWS_PER_WG - 1) / ROWS_PER_WG;
  const int slot = uni(blockIdx.x / nNb), nb = uni(blockIdx.x % nNb);
  const int e = WIDE && offsets ? nth_wide_group(offsets, ngroups, slot) : slot;
  if (e < 0) return;
  const int r0 = offsets ? offsets[e] : 0;
  const int M = offsets ? offsets[e + 1] - r0 : Mdense;
  if (M <= 0 || (WIDE ? M <= 16 : M > 16)) return;
  const int wave = uni(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n0 = nb * ROWS_PER_WG + wave * 16;
  const int nrows = uni(min(16, N - n0));
  if (nrows <= 0) return;  // wave-uniform; no barrier follows
  const int g = lane >> 4, rl = lane & 15;
  // token row i of the group: row r0 + i of X, or (xrow != null) row
  // xrow[r0 + i] / kdiv of X (the assignment's token: no gathered copy)
  const rsrc_t rx = xrow ? make_rsrc(uni_ptr(X), (uint32_t)uni(xrows * K * 2))
                         : make_rsrc(uni_ptr(X + (int64_t)r0 * K), (uint32_t)uni(M * K * 2));
  const int nch = (M + 15) / 16;
  const uint32_t vw = (uint32_t)((rl * K + 8 * g) * 2);
  uint32_t vxc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int i = c * 16 + rl;
    const int row = i >= M ? -1 : xrow ? xrow[r0 + i] / kdiv : i;
    vxc[c] = row < 0 ? kOobOffset : (uint32_t)((row * K + 8 * g) * 2);
  }
  f32x4 acc[NM][NC];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[m][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const bf16_t* wsrc = m ? pick(w1_tab, w1_one, e) : pick(w0_tab, w0_one, e);
    const rsrc_t rw = make_rsrc(uni_ptr(wsrc + (int64_t)n0 * K), (uint32_t)uni(nrows * K * 2));
    for (int kc = 0; kc * 256 < K; ++kc) {
      const uint32_t soff = (uint32_t)kc * 512;
      u32x4 wa[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const bool kin = kc * 256 + 32 * q + 8 * g < K;
        wa[q] = buf_ld16(rw, kin ? vw + 64 * q : kOobOffset, soff);
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (c >= nch) break;
        u32x4 xa[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const bool kin = kc * 256 + 32 * q + 8 * g < K;
          xa[q] = buf_ld16(rx, kin ? vxc[c] + 64 * q : kOobOffset, soff);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 8; ++q) mfma16(acc[m][c], xa[q], wa[q]);
      }
    }
  }
  // lane holds D[token = 16 c + 4 g + r][row = rl]
  if (rl >= nrows) return;
  const int n = n0 + rl;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c >= nch) break;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = c * 16 + 4 * g + r;
      if (t >= M) continue;
      const int64_t o = (int64_t)(r0 + t) * N + n;
      if constexpr (GATEUP) {
        const float gv = acc[0][c][r], uv = acc[NM - 1][c][r];
        if (out0) {  // pre-activations are kept only for a backward
          out0[o] = f2bf(gv);
          out1[o] = f2bf(uv);
        }
        out2[o] = f2bf(silu_f(gv) * uv);
      } else {
        out0[o] = f2bf(acc[0][c][r]);
      }
    }
  }
}

// Router logits with few experts or few tokens (bf16): a workgroup owns 16
// experts and 16 tokens; its kRouterWaves waves take every kRouterWaves-th
// 256-wide k-chunk of the hidden dimension (same lane layout as k_skinny_fwd)
// and the partial sums are added through LDS in wave order.  With few experts
// the launch is small, so the work is cut finely (H = 4096: one chunk per
// wave, 16 token rows per workgroup): one CU cannot pull the whole token
// matrix quickly.
__global__ __launch_bounds__(64 * kRouterWaves) void k_router_small(const bf16_t* __restrict__ x,
                                                      const bf16_t* __restrict__ wr,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ logits, int Tn, int H,
                                                      int E) {
  __shared__ f32x4 red[kRouterWaves][64];
  const int neb = (E + 15) / 16;
  const int e0 = uni(blockIdx.x % neb) * 16, t0 = uni(blockIdx.x / neb) * 16;
  const int wave = uni(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int g = lane >> 4, rl = lane & 15;
  const int nrows = min(16, E - e0), ntok = min(16, Tn - t0);
  const rsrc_t rw = make_rsrc(wr + (int64_t)e0 * H, (uint32_t)((int64_t)nrows * H * 2));
  const rsrc_t rx = make_rsrc(x + (int64_t)t0 * H, (uint32_t)((int64_t)ntok * H * 2));
  const uint32_t vw = (uint32_t)((rl * H + 8 * g) * 2);
  f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int kc = wave; kc * 256 < H; kc += kRouterWaves) {
    const uint32_t soff = (uint32_t)kc * 512;
    u32x4 wa[8], xa[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const bool kin = kc * 256 + 32 * q + 8 * g < H;
      wa[q] = buf_ld16(rw, kin ? vw + 64 * q : kOobOffset, soff);
      xa[q] = buf_ld16(rx, kin ? vw + 64 * q : kOobOffset, soff);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) mfma16(acc, xa[q], wa[q]);
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0 || rl >= nrows) return;
  const int e = e0 + rl;
  const float b = bias ? bias[e] : 0.0f;
  f32x4 v = red[0][lane];
#pragma unroll
  for (int w = 1; w < kRouterWaves; ++w) v += red[w][lane];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = 4 * g + r;  // lane holds D[token t0 + 4 g + r][expert e0 + rl]
    if (t < ntok) logits[(int64_t)(t0 + t) * E + e] = v[r] + b;
  }
}

}  // namespace moe
