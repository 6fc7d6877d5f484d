// Tiled MFMA GEMM main loop for the MoE layer (gfx950 / CDNA4).
//
// One workgroup = 256 threads = 4 wave64s in a 2 x 2 arrangement computes a
// BM x BN output tile of  C[m, n] = sum_k A(m, k) * B(n, k).
// Operands are staged through LDS as K-contiguous rows ([row][k], padded by
// one 16-byte vector per row against bank conflicts). An operand whose memory
// layout is K-major ("transposed": element (r, k) at base + k * ld + r) is
// turned into that LDS layout with an in-register V x V transpose, so the
// MFMA fragment reads are always one ds_read_b128 per lane.
//
// The MFMA "row" input is fed from the B tile and the "column" input from the
// A tile, so the accumulator D[i][j] holds C[m = j][n = i]: each lane then
// owns 4 consecutive n of one output row, which makes the epilogue stores
// 4-element contiguous instead of scattered.
//
// bf16: v_mfma_f32_32x32x16_bf16, fp32: v_mfma_f32_32x32x2f32 (fp32 inputs,
// fp32 accumulate). Both read 16 bytes per lane per operand per step; the k
// slot a lane supplies is the same function of (lane / 32, element) for both
// operands, so the contraction covers every k exactly once.
#pragma once
#include "common.hpp"

namespace moe {

template <typename T, int BM_, int BN_, int BK_>
struct Tiling {
  static constexpr int BM = BM_, BN = BN_, BK = BK_;
  static constexpr int V = Vec16<T>::N;   // elements per 16-byte vector
  static constexpr int LDK = BK + V;      // padded LDS row pitch (elements)
  static constexpr int THREADS = 256;
  static constexpr int WM = BM / 2, WN = BN / 2;  // per-wave tile
  static constexpr int TM = WM / 32, TN = WN / 32;  // 32x32 MFMA blocks per wave
  static_assert(BM % 64 == 0 && BN % 64 == 0, "tile must be a multiple of 64");
  static_assert(BK % (2 * V) == 0, "BK must cover whole MFMA k-steps");
};

// Source of one operand tile.  K-contiguous: element (r, k) at base + r*ld + k;
// transposed: at base + k*ld + r.  Rows at or beyond rows_valid are clamped
// (K-contiguous) or read as zero (transposed); k at or beyond k_valid reads
// as zero.  For K-contiguous operands k_valid must be a multiple of V; for
// transposed operands ld must be at least rows_valid rounded up to V.
template <typename T>
struct OpDesc {
  const T* base;
  int64_t ld;
  int rows_valid;
  int k_valid;
};

MOE_DEV void mfma_frag(f32x16& acc, u32x4 bt, u32x4 at, bf16_t) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, bt),
                                                __builtin_bit_cast(bf16x8_t, at), acc, 0, 0, 0);
}
MOE_DEV void mfma_frag(f32x16& acc, u32x4 bt, u32x4 at, float) {
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(bt.x), __uint_as_float(at.x), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(bt.y), __uint_as_float(at.y), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(bt.z), __uint_as_float(at.z), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(bt.w), __uint_as_float(at.w), acc, 0, 0, 0);
}

// V x V transpose of 16-byte row vectors: out[c] element i = in[i] element c.
MOE_DEV void transpose_vv(const u32x4 (&in)[8], u32x4 (&out)[8], bf16_t) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {      // source word q holds elements 2q (low) and 2q+1 (high)
#pragma unroll
    for (int w = 0; w < 4; ++w) {    // destination word w holds rows 2w (low) and 2w+1 (high)
      uint32_t a = in[2 * w][q], b = in[2 * w + 1][q];
      out[2 * q][w] = (a & 0xffffu) | (b << 16);
      out[2 * q + 1][w] = (a >> 16) | (b & 0xffff0000u);
    }
  }
}
MOE_DEV void transpose_vv(const u32x4 (&in)[4], u32x4 (&out)[4], float) {
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) out[c][i] = in[i][c];
}

// Per-thread staging of one operand tile of R rows between global memory and LDS.
template <class C, typename T, int R, bool TRANS>
struct Stager;

template <class C, typename T, int R>
struct Stager<C, T, R, false> {
  static constexpr int KV = C::BK / C::V;              // vectors per row
  static constexpr int TOTAL = R * KV;
  static constexpr int PER = (TOTAL + C::THREADS - 1) / C::THREADS;
  u32x4 r[PER];
  MOE_DEV void load(const OpDesc<T>& d, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int c = tid + i * C::THREADS;
      int row = c / KV, kv = c % KV;
      int rr = row < d.rows_valid ? row : d.rows_valid - 1;
      int k = k0 + kv * C::V;
      if ((TOTAL % C::THREADS == 0 || c < TOTAL) && k < d.k_valid)
        r[i] = ld16(d.base + (int64_t)rr * d.ld + k);
      else
        r[i] = u32x4{0, 0, 0, 0};
    }
  }
  MOE_DEV void store(T* s, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int c = tid + i * C::THREADS;
      if (TOTAL % C::THREADS == 0 || c < TOTAL) {
        int row = c / KV, kv = c % KV;
        st16(s + row * C::LDK + kv * C::V, r[i]);
      }
    }
  }
};

template <class C, typename T, int R>
struct Stager<C, T, R, true> {
  static constexpr int V = C::V;
  static constexpr int RB = R / V, KB = C::BK / V;     // V x V blocks
  static constexpr int TOTAL = RB * KB;
  static constexpr int PER = (TOTAL + C::THREADS - 1) / C::THREADS;
  u32x4 r[PER][V];
  MOE_DEV void load(const OpDesc<T>& d, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int b = tid + i * C::THREADS;
      int rb = b % RB, kb = b / RB;                    // adjacent threads: adjacent rows
      bool ok = (TOTAL % C::THREADS == 0 || b < TOTAL) && rb * V < d.rows_valid;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        int k = k0 + kb * V + j;
        if (ok && k < d.k_valid)
          r[i][j] = ld16(d.base + (int64_t)k * d.ld + rb * V);
        else
          r[i][j] = u32x4{0, 0, 0, 0};
      }
    }
  }
  MOE_DEV void store(T* s, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int b = tid + i * C::THREADS;
      if (TOTAL % C::THREADS == 0 || b < TOTAL) {
        int rb = b % RB, kb = b / RB;
        u32x4 t[V];
        transpose_vv(r[i], t, T());
#pragma unroll
        for (int c = 0; c < V; ++c) st16(s + (rb * V + c) * C::LDK + kb * C::V, t[c]);
      }
    }
  }
};

// LDS elements needed by a main loop with NA A operands and NB B operands.
template <class C, int NA, int NB>
constexpr int smem_elems() { return (NA * C::BM + NB * C::BN) * C::LDK; }

// acc[a * NB + b][tn][tm] += B_b-tile x A_a-tile over k in [0, K).
// Register-prefetch pipeline: the next k-tile is fetched from global memory
// while the current one is multiplied out of LDS.
template <class C, typename T, bool A_T, bool B_T, int NA, int NB>
MOE_DEV void mainloop(f32x16 (&acc)[NA * NB][C::TN][C::TM], const OpDesc<T> (&a)[NA],
                      const OpDesc<T> (&b)[NB], int K, T* smem) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  T* sA = smem;
  T* sB = smem + NA * C::BM * C::LDK;
  Stager<C, T, C::BM, A_T> sa[NA];
  Stager<C, T, C::BN, B_T> sb[NB];
  const int nk = (K + C::BK - 1) / C::BK;
  if (nk == 0) return;

#pragma unroll
  for (int i = 0; i < NA; ++i) sa[i].load(a[i], 0, tid);
#pragma unroll
  for (int i = 0; i < NB; ++i) sb[i].load(b[i], 0, tid);
#pragma unroll
  for (int i = 0; i < NA; ++i) sa[i].store(sA + i * C::BM * C::LDK, tid);
#pragma unroll
  for (int i = 0; i < NB; ++i) sb[i].store(sB + i * C::BN * C::LDK, tid);
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * C::V;
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) {
#pragma unroll
      for (int i = 0; i < NA; ++i) sa[i].load(a[i], (kt + 1) * C::BK, tid);
#pragma unroll
      for (int i = 0; i < NB; ++i) sb[i].load(b[i], (kt + 1) * C::BK, tid);
    }
#pragma unroll
    for (int kk = 0; kk < C::BK; kk += 2 * C::V) {
      u32x4 af[NA][C::TM], bfr[NB][C::TN];
#pragma unroll
      for (int i = 0; i < NA; ++i)
#pragma unroll
        for (int tm = 0; tm < C::TM; ++tm)
          af[i][tm] = *reinterpret_cast<const u32x4*>(
              sA + i * C::BM * C::LDK + (wm * C::WM + tm * 32 + frag_row) * C::LDK + kk + frag_k);
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int tn = 0; tn < C::TN; ++tn)
          bfr[i][tn] = *reinterpret_cast<const u32x4*>(
              sB + i * C::BN * C::LDK + (wn * C::WN + tn * 32 + frag_row) * C::LDK + kk + frag_k);
#pragma unroll
      for (int ia = 0; ia < NA; ++ia)
#pragma unroll
        for (int ib = 0; ib < NB; ++ib)
#pragma unroll
          for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
            for (int tm = 0; tm < C::TM; ++tm)
              mfma_frag(acc[ia * NB + ib][tn][tm], bfr[ib][tn], af[ia][tm], T());
    }
    __syncthreads();
    if (more) {
#pragma unroll
      for (int i = 0; i < NA; ++i) sa[i].store(sA + i * C::BM * C::LDK, tid);
#pragma unroll
      for (int i = 0; i < NB; ++i) sb[i].store(sB + i * C::BN * C::LDK, tid);
      __syncthreads();
    }
  }
}

template <class C, int NACC>
MOE_DEV void zero_acc(f32x16 (&acc)[NACC][C::TN][C::TM]) {
#pragma unroll
  for (int x = 0; x < NACC; ++x)
#pragma unroll
    for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[x][tn][tm][r] = 0.0f;
}

// Calls f(m_local, n_local, v) for every 4-wide output fragment of the tile,
// where v[x][i] = acc[x] at (m_local, n_local + i).
template <class C, int NACC, class F>
MOE_DEV void for_each_frag(const f32x16 (&acc)[NACC][C::TN][C::TM], F&& f) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
    for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = wm * C::WM + tm * 32 + (lane & 31);
        const int n = wn * C::WN + tn * 32 + 8 * q + 4 * (lane >> 5);
        float v[NACC][4];
#pragma unroll
        for (int x = 0; x < NACC; ++x)
#pragma unroll
          for (int i = 0; i < 4; ++i) v[x][i] = acc[x][tn][tm][4 * q + i];
        f(m, n, v);
      }
}

// Find the group g with prefix[g] <= t < prefix[g + 1] (prefix[0] = 0).
MOE_DEV int find_group(const int* prefix, int G, int t) {
  int lo = 0, hi = G;
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (prefix[mid] <= t) lo = mid; else hi = mid;
  }
  return lo;
}

// Store 4 consecutive elements (4-element aligned) of one output row.
MOE_DEV void store4(bf16_t* p, const float* v) {
  uint2 w;
  w.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
  w.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
  *reinterpret_cast<uint2*>(p) = w;
}
MOE_DEV void store4(float* p, const float* v) {
  *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
}
MOE_DEV void load4(const bf16_t* p, float* v) {
  uint2 w = *reinterpret_cast<const uint2*>(p);
  v[0] = __uint_as_float(w.x << 16); v[1] = __uint_as_float(w.x & 0xffff0000u);
  v[2] = __uint_as_float(w.y << 16); v[3] = __uint_as_float(w.y & 0xffff0000u);
}
MOE_DEV void load4(const float* p, float* v) {
  f32x4 w = *reinterpret_cast<const f32x4*>(p);
  v[0] = w[0]; v[1] = w[1]; v[2] = w[2]; v[3] = w[3];
}

}  // namespace moe
