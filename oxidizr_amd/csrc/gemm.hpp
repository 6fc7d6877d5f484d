// Tiled MFMA GEMM main loop for the MoE layer (gfx950 / CDNA4).
//
// One workgroup of 4 or 8 wave64s (Tiling::NW) in a WGM x WGN arrangement
// computes a BM x BN output tile of  C[m, n] = sum_k A(m, k) * B(n, k).
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
#include <type_traits>
#include "common.hpp"

namespace moe {

// BM x BN output tile per workgroup of NW waves arranged WGM x WGN (wave w
// owns block (w / WGN, w % WGN)), BK-deep k-tiles.
//
// XR > 0 ("tall" tile, direct-to-LDS loop only): the tile has XR more rows
// below its BM rows, shared out over the four wave rows.  XR = 64: wave
// (wm, wn) also owns extra row block wm & 1 (rows BM + 32 (wm & 1) ..) at the
// XTN = WN / 64 column blocks of half wm >> 1 of its own WN columns.  XR = 128:
// wave (wm, wn) also owns extra row block wm (rows BM + 32 wm ..) at all TN
// column blocks of its WN columns.  Either way the extra blocks use B
// fragments the wave already reads for its main blocks.  XR = 128 keeps one
// register set of fragments (FB1) to fit its 192 accumulators.
template <typename T, int BM_, int BN_, int BK_, int WGN_ = 2, int NST_ = 2, int NW_ = 4,
          int XR_ = 0>
struct Tiling {
  static constexpr int BM = BM_, BN = BN_, BK = BK_;
  static constexpr int NST = NST_;        // LDS pipeline stages (direct-to-LDS loop)
  static constexpr int V = Vec16<T>::N;   // elements per 16-byte vector
  static constexpr int LDK = BK + V;      // padded LDS row pitch (elements)
  static constexpr int NW = NW_;          // waves per workgroup
  static constexpr int THREADS = 64 * NW;
  static constexpr int WGN = WGN_, WGM = NW_ / WGN_;  // wave grid
  static constexpr int WM = BM / WGM, WN = BN / WGN;  // per-wave tile
  static constexpr int TM = WM / 32, TN = WN / 32;  // 32x32 MFMA blocks per wave
  static constexpr int XR = XR_;                    // extra rows of a tall tile
  static constexpr int XTN = XR == 128 ? TN : XR > 0 ? WN / 64 : 1;  // extra column blocks per wave
  static constexpr int AR = BM + XR;                // A-operand rows per k-tile
  static constexpr bool FB1 = XR == 128;            // one register set of fragments
  static_assert(WGM * WGN == NW && (NW == 4 || NW == 8), "four or eight waves");
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tiles of whole 32 x 32 blocks");
  static_assert(BM % 64 == 0 && BN % 64 == 0, "tile must be a multiple of 64");
  static_assert(BK % (2 * V) == 0, "BK must cover whole MFMA k-steps");
  static_assert(NST >= 2 && NST <= 6, "2 to 6 pipeline stages");
  static_assert(XR == 0 || (((XR == 64 && WN % 64 == 0) || XR == 128) && WGM == 4 && sizeof(T) == 2),
                "tall tiles: 64 or 128 extra rows over a four-row wave grid, bf16");
};

// Source of one operand tile.  K-contiguous: element (r, k) at base + r*ld + k;
// transposed: at base + k*ld + r.  Rows at or beyond rows_valid and k at or
// beyond k_valid read as zero (rows beyond rows_valid of a transposed operand
// may also read neighbouring columns of the same matrix: their products only
// reach output rows the epilogue drops).  For K-contiguous operands k_valid and
// ld must be multiples of V; for transposed operands ld must be a multiple of V
// and at least rows_valid rounded up to V.  Every byte the tile can reach must
// lie within 2^31 bytes of base: buffer offsets are 32-bit and kOobOffset
// (2^31) must fall outside every resource.  Bases are the tile's own rows or
// columns, so the extent is at most (rows or k of one group) x ld; the entry
// points refuse token counts whose largest such extent (T x max(H, I, S, E)
// elements, a group holding at most T rows) reaches 2^31 bytes
// (moe_check_tokens), and plans whose weight matrices do.
//
// Gathered K-contiguous operand (the main loop's AG flag): tile row r < rows_valid
// is row rows[r] / rdiv of the src_rows x ld matrix at base, so a tile reads
// token rows of an unpermuted matrix in expert order (rows: the permutation,
// entries t * k + j; rdiv = k) without a permuted copy.  Each lane reads its
// rows' indices once, before the k-loop; an index outside [0, src_rows * rdiv)
// reads zeros.
template <typename T>
struct OpDesc {
  const T* base;
  int64_t ld;
  int rows_valid;
  int k_valid;
  const int* rows = nullptr;
  int src_rows = 0;
  int rdiv = 1;
};
// Byte offset of gathered row r's k-column kcol, or kOobOffset.
template <typename T>
MOE_DEV uint32_t gathered_row_offset(const OpDesc<T>& d, int r, int kcol) {
  if (r >= d.rows_valid) return kOobOffset;
  const int p = d.rows[r];
  if ((unsigned)p >= (unsigned)d.src_rows * (unsigned)d.rdiv) return kOobOffset;
  return (uint32_t)(((int64_t)(p / d.rdiv) * d.ld + kcol) * (int64_t)sizeof(T));
}

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

// Per-thread staging of one operand tile of R rows between global memory and
// LDS.  Loads are raw buffer loads: the resource covers exactly the operand's
// readable extent, so out-of-range rows and the K tail come back as zero from
// the hardware (no per-load branches), the tile base sits in scalar registers
// and each load needs one 32-bit offset register.
template <class C, typename T, int R, bool TRANS, bool G = false>
struct Stager;

template <class C, typename T, int R, bool G>
struct Stager<C, T, R, false, G> {
  static constexpr int KV = C::BK / C::V;              // vectors per row
  static constexpr int TOTAL = R * KV;
  static_assert(TOTAL % C::THREADS == 0, "tile rows must cover the workgroup");
  static constexpr int PER = TOTAL / C::THREADS;
  static constexpr int ROWS_STEP = C::THREADS / KV;    // rows between a thread's loads
  u32x4 r[PER];
  rsrc_t rs[2];                                        // one per K segment
  int k_valid[2];
  uint32_t voff, step;
  uint32_t vrow[G ? PER : 1];                          // gathered: each load's row offset
  int kcol;
  MOE_DEV static rsrc_t rsrc_of(const OpDesc<T>& d) {
    const int64_t limit = G ? (int64_t)d.src_rows * d.ld
                            : (int64_t)(d.rows_valid - 1) * d.ld + d.k_valid;
    return make_rsrc(d.base, (uint32_t)(limit * (int64_t)sizeof(T)));
  }
  MOE_DEV void init(const OpDesc<T>& d, int tid) {
    rs[0] = rs[1] = rsrc_of(d);
    k_valid[0] = k_valid[1] = d.k_valid;
    kcol = (tid % KV) * C::V;
    voff = (uint32_t)(((tid / KV) * d.ld + kcol) * (int64_t)sizeof(T));
    step = (uint32_t)(ROWS_STEP * d.ld * (int64_t)sizeof(T));
    if constexpr (G) {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        vrow[i] = gathered_row_offset(d, tid / KV + i * ROWS_STEP, kcol);
      }
    }
  }
  // Second K segment: same ld and rows as the first.
  MOE_DEV void init_second(const OpDesc<T>& d) {
    rs[1] = rsrc_of(d);
    k_valid[1] = d.k_valid;
  }
  MOE_DEV void load(int k0, int seg) {
    const uint32_t soff = (uint32_t)k0 * sizeof(T);
    const bool kin = k0 + kcol < k_valid[seg];
#pragma unroll
    for (int i = 0; i < PER; ++i)
      r[i] = buf_ld16(rs[seg], kin ? (G ? vrow[i] : voff + i * step) : kOobOffset, soff);
  }
  MOE_DEV void store(T* s, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * C::THREADS;
      const int row = c / KV, kv = c % KV;
      st16(s + row * C::LDK + kv * C::V, r[i]);
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
  rsrc_t rs[2];                                        // one per K segment
  uint32_t voff, ldb;
  MOE_DEV static rsrc_t rsrc_of(const OpDesc<T>& d) {
    const int rv = (d.rows_valid + V - 1) / V * V;
    const int64_t limit = (int64_t)(d.k_valid - 1) * d.ld + rv;
    return make_rsrc(d.base, d.k_valid > 0 ? (uint32_t)(limit * (int64_t)sizeof(T)) : 0u);
  }
  MOE_DEV void init(const OpDesc<T>& d, int tid) {
    rs[0] = rs[1] = rsrc_of(d);
    const int rb = tid % RB, kb = tid / RB;            // adjacent threads: adjacent rows
    voff = (uint32_t)(((int64_t)kb * V * d.ld + rb * V) * (int64_t)sizeof(T));
    ldb = (uint32_t)(d.ld * (int64_t)sizeof(T));
  }
  // Second K segment: same ld and rows as the first.
  MOE_DEV void init_second(const OpDesc<T>& d) { rs[1] = rsrc_of(d); }
  MOE_DEV void load(int k0, int seg) {
    const uint32_t soff = (uint32_t)k0 * ldb;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (TOTAL % C::THREADS == 0 || (int)threadIdx.x + i * C::THREADS < TOTAL) {
        const uint32_t vi = voff + (uint32_t)(i * (C::THREADS / RB) * V) * ldb;
#pragma unroll
        for (int j = 0; j < V; ++j) r[i][j] = buf_ld16(rs[seg], vi + j * ldb, soff);
      }
    }
  }
  MOE_DEV void store(T* s, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int b = tid + i * C::THREADS;
      if (TOTAL % C::THREADS == 0 || b < TOTAL) {
        const int rb = b % RB, kb = b / RB;
        u32x4 t[V];
        transpose_vv(r[i], t, T());
#pragma unroll
        for (int c = 0; c < V; ++c) st16(s + (rb * V + c) * C::LDK + kb * C::V, t[c]);
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Direct-to-LDS path.  Buffer loads with the LDS modifier stream 16-byte
// vectors from global memory straight into LDS (no staging registers, no
// ds_write); one instruction writes 64 lanes x 16 B = 1 KB of LDS.
//
// K-contiguous operand tile: R rows of BK k, unpadded 128-byte rows; the
// 16-byte slot of k-vector kv in row r sits at kv ^ nt_swz(r).  A fragment
// read serves 16 consecutive rows per LDS cycle (256 bytes, 64 banks): rows r
// and r + 8 share a bank window, so the swizzle also depends on bit 3 of r and
// the 16 rows land on 16 different 16-byte bank groups (the first 8 on 8
// different ones as well).  The lane that fills slot s of row r therefore
// loads k-vector s ^ nt_swz(r).
//
// K-major operand tile (bf16 only; element (r, k) at base + k*ld + r): BK
// k-rows of R contiguous columns; the 16-byte slot p of k-row k sits at
// p ^ tr_swz(k).  Fragments come from ds_read_b64_tr_b16: within each group of
// 16 lanes, lane 4i + j receives in slot q element j of the 8-byte chunk
// addressed by lane 4q + i.  When lane 4q + i of group b addresses k-row
// kk + 8 (b >> 1) + q at column c0 + 16 (b & 1) + 4i, lane L receives the four
// k = kk + 8 (b >> 1) + [0, 4) of column c0 + (L % 32); a second read at k + 4
// completes the 8 consecutive k an MFMA lane supplies.
typedef __attribute__((address_space(3))) void lds_void_t;
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

// 16-byte slot swizzles.  K-contiguous tiles: see above.  K-major tiles: the 32
// lanes one transposing read serves per cycle cover slots 0..3 of four
// consecutive k-rows; XOR-ing by 4 (k & 3) gives them 16 different slots.
MOE_DEV int nt_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }
MOE_DEV int tr_swz(int k) { return (k & 3) << 2; }

template <class C, typename T, int R, bool G = false>
struct DmaStager {
  static constexpr int KV = C::BK / C::V;    // 16-byte slots per row
  static_assert(KV == 8 || KV == 4, "rows of 8 or 4 slots");
  static constexpr int RPI = 64 / KV;        // rows per wave per 1 KB instruction
  static_assert(R % (C::NW * RPI) == 0, "NW waves x RPI rows per instruction");
  static constexpr int PER = R / (C::NW * RPI);  // instructions per wave per k-tile
  // slot swizzle: the 16 lanes of a ds_read_b128 phase read 16 rows at one kv
  // and must hit 16 distinct 16-byte bank groups of a 256-byte window
  MOE_DEV static int swz(int r) { return KV == 8 ? nt_swz(r) : ((r >> 2) & 3); }
  rsrc_t rs[2];                              // one per K segment
  int k_valid[2];
  uint32_t voff, step;
  uint32_t vrow[G ? PER : 1];                // gathered: each instruction's row offset
  int kcol;
  MOE_DEV static rsrc_t rsrc_of(const OpDesc<T>& d) {
    const int64_t limit = G ? (int64_t)d.src_rows * d.ld
                            : (int64_t)(d.rows_valid - 1) * d.ld + d.k_valid;
    return make_rsrc(d.base, (uint32_t)(limit * (int64_t)sizeof(T)));
  }
  MOE_DEV void init(const OpDesc<T>& d, int tid) {
    rs[0] = rs[1] = rsrc_of(d);
    k_valid[0] = k_valid[1] = d.k_valid;
    const int lane = tid & 63, wave = tid >> 6;
    const int row = wave * RPI + lane / KV;   // the swizzle bits are the same for every chunk i
    kcol = ((lane % KV) ^ swz(row)) * C::V;
    voff = (uint32_t)((row * d.ld + kcol) * (int64_t)sizeof(T));
    step = (uint32_t)(C::NW * RPI * d.ld * (int64_t)sizeof(T));
    if constexpr (G) {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        vrow[i] = gathered_row_offset(d, row + i * C::NW * RPI, kcol);
      }
    }
  }
  MOE_DEV void init_second(const OpDesc<T>& d) {  // same ld and rows as the first
    rs[1] = rsrc_of(d);
    k_valid[1] = d.k_valid;
  }
  MOE_DEV void issue(T* tile, int k0, int seg) const {
    // wave-uniform: the LDS destination (M0) is then scalar arithmetic
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t soff = (uint32_t)k0 * sizeof(T);
    const bool kin = k0 + kcol < k_valid[seg];
#pragma unroll
    for (int i = 0; i < PER; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs[seg], (lds_void_t*)(tile + (i * C::NW * RPI + wave * RPI) * C::BK), 16,
          kin ? (G ? vrow[i] : voff + i * step) : kOobOffset, soff, 0, 0);
  }
  MOE_DEV static u32x4 frag(const T* tile, int row, int kv) {
    return *reinterpret_cast<const u32x4*>(tile + row * C::BK + ((kv ^ swz(row)) * C::V));
  }
};

template <class C, typename T, int R>
struct DmaStagerT {
  static_assert(sizeof(T) == 2, "transposing LDS reads are 16-bit");
  static constexpr int SPR = R / 8;              // 16-byte slots per k-row
  // tr_swz XORs slot indices with 4 (k & 3): a k-row needs at least 16 slots
  static_assert(SPR >= 16 && SPR <= 64, "K-major tiles of 128 to 512 columns");
  static constexpr int RPI = 64 / SPR;           // k-rows per 1 KB instruction
  static constexpr int PER = C::BK / (C::NW * RPI);  // instructions per wave per k-tile
  static_assert(PER >= 1 && C::BK % (C::NW * RPI) == 0, "k-rows must cover the waves");
  rsrc_t rs[2];
  uint32_t voff, ldb;
  MOE_DEV static rsrc_t rsrc_of(const OpDesc<T>& d) {
    const int rv = (d.rows_valid + 7) / 8 * 8;
    const int64_t limit = (int64_t)(d.k_valid - 1) * d.ld + rv;
    return make_rsrc(d.base, d.k_valid > 0 ? (uint32_t)(limit * (int64_t)sizeof(T)) : 0u);
  }
  MOE_DEV void init(const OpDesc<T>& d, int tid) {
    rs[0] = rs[1] = rsrc_of(d);
    const int lane = tid & 63, wave = tid >> 6;
    const int krow = wave * RPI + lane / SPR;
    const int src = (lane % SPR) ^ tr_swz(krow);
    voff = (uint32_t)(((int64_t)krow * d.ld + src * 8) * (int64_t)sizeof(T));
    ldb = (uint32_t)(d.ld * (int64_t)sizeof(T));
  }
  MOE_DEV void init_second(const OpDesc<T>& d) { rs[1] = rsrc_of(d); }
  MOE_DEV void issue(T* tile, int k0, int seg) const {
    // wave-uniform: the LDS destination (M0) is then scalar arithmetic
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < PER; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs[seg], (lds_void_t*)(tile + (i * C::NW * RPI + wave * RPI) * R), 16,
          voff + (uint32_t)(i * C::NW * RPI) * ldb, (uint32_t)k0 * ldb, 0, 0);
  }
  // operand of the fragment whose first column is col0, k-step starting at kk
  MOE_DEV static u32x4 frag(const T* tile, int col0, int kk) {
    const int lane = threadIdx.x & 63;
    const int s = lane & 15, b = lane >> 4;
    const int q = s >> 2, i = s & 3;
    const int col = col0 + 16 * (b & 1) + 4 * i;
    const int k1 = kk + 8 * (b >> 1) + q, k2 = k1 + 4;
    const T* a1 = tile + k1 * R + (((col >> 3) ^ tr_swz(k1)) << 3) + (col & 7);
    const T* a2 = tile + k2 * R + (((col >> 3) ^ tr_swz(k2)) << 3) + (col & 7);
    const i16x4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)a1);
    const i16x4_t v2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)a2);
    const u32x2 w1 = __builtin_bit_cast(u32x2, v1), w2 = __builtin_bit_cast(u32x2, v2);
    return u32x4{w1.x, w1.y, w2.x, w2.y};
  }
};

// acc += B x A over K with both operands fed by DMA into C::NST unpadded LDS
// stages (k-tile kt in stage kt % NST).  While k-tile kt is multiplied out,
// the DMA of the next NST - 1 k-tiles is in flight.  Before k-tile kt + 1 is
// read each wave waits until its own DMA instructions for that tile have
// landed (vmcnt counts vector memory instructions in issue order, so "at most
// the later tiles' instructions outstanding" means this tile's are done),
// then a barrier makes every wave's part visible.  The barrier for tile kt + 1
// sits inside the last k-step of tile kt: once every wave is past it, no wave
// reads the stage of tile kt again, so the first fragments of tile kt + 1 are
// read while the last MFMAs of tile kt issue, and the DMA of tile kt + NST
// refills that stage.  An optional second K segment (a2, b2, K2: same ld and
// rows) continues the pipeline.
//
// The refill is interleaved with the MFMAs of that last k-step, one DMA
// instruction after each MFMA.  Issued back to back, the DMA instructions of
// all four waves fill the CU's vector memory queue and a wave stalls, in
// order, on its next DMA instruction while its MFMAs wait behind it (config-5
// gate/up forward alone: 5.15 -> 4.61 ms, dense 65536 x 4096 x 7168: 1132 ->
// 1318 TFLOP/s; the transposed-operand input gradients measured unchanged).  The
// interleaving needs the DMA and the MFMAs in one basic block, so the loop
// runs in three phases without a data-dependent branch around the DMA:
// k-tiles that refill a stage (kt + NST < nk), then the k-tiles whose DMA is
// all in flight, then the last one.
//
// Tall tiles (C::XR > 0, K-contiguous A): the A tile holds C::AR rows and each
// wave also multiplies its extra A fragment (row block wm & 1 of the XR extra
// rows) with the B fragments of half wm >> 1 of its columns into xacc, which
// are picked out of the registers it already holds (a wave-uniform select).
// Workgroup barrier of the direct-to-LDS pipeline: this wave's LDS reads are
// done (s_waitcnt lgkmcnt(0)) and every wave has passed its own explicit
// vmcnt wait for the k-tile it needs next.  __syncthreads() compiles to
// s_waitcnt vmcnt(0) lgkmcnt(0) before s_barrier: it would also wait for the
// DMA of every later k-tile already in flight, which drains a pipeline of more
// than two stages at each k-tile.
MOE_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <class C, typename T, bool A_T, bool B_T, int NA, int NB, bool AG = false>
MOE_DEV void mainloop_dma(f32x16 (&acc)[NA * NB][C::TN][C::TM],
                          f32x16 (&xacc)[NA * NB][C::XTN], const OpDesc<T> (&a)[NA],
                          const OpDesc<T> (&b)[NB], int K, T* smem, const OpDesc<T>* a2,
                          const OpDesc<T>* b2, int K2) {
  constexpr int TILE_A = C::AR * C::BK, TILE_B = C::BN * C::BK;
  constexpr int STAGE = NA * TILE_A + NB * TILE_B;
  constexpr int NST = C::NST;
  constexpr bool TALL = C::XR > 0;
  static_assert(!TALL || !A_T, "tall tiles take a K-contiguous A operand");
  static_assert(!AG || !A_T, "gathered rows: K-contiguous A");
  using SA = typename std::conditional<A_T, DmaStagerT<C, T, C::AR>, DmaStager<C, T, C::AR, AG>>::type;
  using SB = typename std::conditional<B_T, DmaStagerT<C, T, C::BN>, DmaStager<C, T, C::BN>>::type;
  // DMA instructions one wave issues per k-tile
  constexpr int IPT = NA * SA::PER + NB * SB::PER;
  static_assert((NST - 2) * IPT <= 63, "vmcnt range");
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  SA sa[NA];
  SB sb[NB];
  const int nk1 = (K + C::BK - 1) / C::BK;
  const int nk = nk1 + (K2 > 0 ? (K2 + C::BK - 1) / C::BK : 0);
  if (nk <= 0) return;
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    sa[i].init(a[i], tid);
    if (K2 > 0) sa[i].init_second(a2[i]);
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    sb[i].init(b[i], tid);
    if (K2 > 0) sb[i].init_second(b2[i]);
  }
  auto stage_of = [](int kt) { return NST == 2 ? (kt & 1) : kt % NST; };
  auto issue = [&](int kt) {
    const int seg = kt >= nk1 ? 1 : 0;
    const int k0 = (kt - seg * nk1) * C::BK;
    T* st = smem + stage_of(kt) * STAGE;
#pragma unroll
    for (int i = 0; i < NA; ++i) sa[i].issue(st + i * TILE_A, k0, seg);
#pragma unroll
    for (int i = 0; i < NB; ++i) sb[i].issue(st + NA * TILE_A + i * TILE_B, k0, seg);
  };
  const int pro = min(NST - 1, nk);
  for (int kt = 0; kt < pro; ++kt) issue(kt);
  const int frag_row = lane & 31;
  const int frag_kv = lane >> 5;
  constexpr int KSTEPS = C::BK / (2 * C::V);
  static_assert(KSTEPS % 2 == 0, "the next tile's first fragments go to register set 0");
  constexpr int NSET = C::FB1 ? 1 : 2;
  u32x4 af[NSET][NA][C::TM], bfr[NSET][NB][C::TN], afx[NSET][NA];
  // tall tiles: the wave's extra row block and column half (wave-uniform)
  const int xrow = C::BM + 32 * (C::XR == 128 ? wm : (wm & 1)) + frag_row;
  const bool xhi = __builtin_amdgcn_readfirstlane(wm >> 1) != 0;
  auto read_frags = [&](const T* sA, const T* sB, int ks, int set) {
    const int kv = ks * 2 + frag_kv;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
#pragma unroll
      for (int tm = 0; tm < C::TM; ++tm) {
        if constexpr (A_T) af[set][i][tm] = SA::frag(sA + i * TILE_A, wm * C::WM + tm * 32, ks * 16);
        else af[set][i][tm] = SA::frag(sA + i * TILE_A, wm * C::WM + tm * 32 + frag_row, kv);
      }
      if constexpr (TALL) afx[set][i] = SA::frag(sA + i * TILE_A, xrow, kv);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int tn = 0; tn < C::TN; ++tn) {
        if constexpr (B_T) bfr[set][i][tn] = SB::frag(sB + i * TILE_B, wn * C::WN + tn * 32, ks * 16);
        else bfr[set][i][tn] = SB::frag(sB + i * TILE_B, wn * C::WN + tn * 32 + frag_row, kv);
      }
  };
  // wait until k-tile kt has landed when k-tiles up to `last` were issued
  auto wait_tile = [&](int kt, int last) {
    const int later = last - kt;
    if constexpr (NST > 4) {
      if (later >= 3) { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(3 * IPT) : "memory"); return; }
    }
    if constexpr (NST > 3) {
      if (later >= 2) { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * IPT) : "memory"); return; }
    }
    if constexpr (NST > 2) {
      if (later >= 1) { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(IPT) : "memory"); return; }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };
  static_assert(NST <= 5, "wait_tile covers up to three later tiles");
  wait_tile(0, pro - 1);
  lds_barrier();
  int issued = pro - 1;
  if (NST - 1 < nk) {
    issue(NST - 1);
    issued = NST - 1;
  }
  if constexpr (!C::FB1) read_frags(smem, smem + NA * TILE_A, 0, 0);
  // One k-tile.  Phase 0: k-tiles up to kt + NST - 1 are issued and the last
  // k-step refills the stage of kt with k-tile kt + NST; phase 1: every
  // k-tile is issued, the last k-step only moves on to kt + 1; phase 2: the
  // last k-tile.
  // Weight gradients (both operands K-major; K = a group's tokens, ragged):
  // the last k-tile runs only the k-steps that reach a valid k.  The others
  // would multiply the zeros the buffer loads return past K, and nothing
  // overlaps the last k-tile's MFMAs.  (The other GEMMs keep the full k-tile:
  // their K is a model dimension, and the branch costs their registers.)
  constexpr bool SKIPK = A_T && B_T;
  const int klast = K2 > 0 ? K2 - (nk - nk1 - 1) * C::BK : K - (nk1 - 1) * C::BK;
  const int kslast = SKIPK ? __builtin_amdgcn_readfirstlane((klast + 2 * C::V - 1) / (2 * C::V))
                           : KSTEPS;
  auto body = [&](int kt, auto phase_c) {
    constexpr int phase = decltype(phase_c)::value;
    const T* sA = smem + stage_of(kt) * STAGE;
    const T* sB = sA + NA * TILE_A;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      if constexpr (phase == 2 && SKIPK) {
        if (ks >= kslast) break;
      }
      const int cur = C::FB1 ? 0 : ks & 1;
      if constexpr (C::FB1) {
        // one register set: this k-step's fragments, then (last k-step) the
        // barrier for the next k-tile and the refill of this stage
        read_frags(sA, sB, ks, 0);
        if constexpr (phase < 2) {
          if (ks + 1 == KSTEPS) {
            if constexpr (phase == 0) {
              asm volatile("s_waitcnt vmcnt(%0)" :: "n"((NST - 2) * IPT) : "memory");
            } else {
              wait_tile(kt + 1, issued);
            }
            lds_barrier();
            if constexpr (phase == 0) issue(kt + NST);
          }
        }
      } else if (ks + 1 < KSTEPS) {
        if (phase < 2 || !SKIPK || ks + 1 < kslast) read_frags(sA, sB, ks + 1, cur ^ 1);
      } else if constexpr (phase < 2) {
        if constexpr (phase == 0) {
          asm volatile("s_waitcnt vmcnt(%0)" :: "n"((NST - 2) * IPT) : "memory");
        } else {
          wait_tile(kt + 1, issued);
        }
        lds_barrier();
        const T* nA = smem + stage_of(kt + 1) * STAGE;
        read_frags(nA, nA + NA * TILE_A, 0, cur ^ 1);
        if constexpr (phase == 0) issue(kt + NST);
      }
#pragma unroll
      for (int ia = 0; ia < NA; ++ia)
#pragma unroll
        for (int ib = 0; ib < NB; ++ib) {
#pragma unroll
          for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
            for (int tm = 0; tm < C::TM; ++tm)
              mfma_frag(acc[ia * NB + ib][tn][tm], bfr[cur][ib][tn], af[cur][ia][tm], T());
          if constexpr (C::XR == 128) {
#pragma unroll
            for (int j = 0; j < C::XTN; ++j)
              mfma_frag(xacc[ia * NB + ib][j], bfr[cur][ib][j], afx[cur][ia], T());
          } else if constexpr (TALL) {
#pragma unroll
            for (int j = 0; j < C::XTN; ++j) {
              const u32x4 bx = xhi ? bfr[cur][ib][C::XTN + j] : bfr[cur][ib][j];
              mfma_frag(xacc[ia * NB + ib][j], bx, afx[cur][ia], T());
            }
          }
        }
      if constexpr (phase == 0) {
        if (ks + 1 == KSTEPS) {
          constexpr int NM = NA * NB * (C::TN * C::TM + (TALL ? C::XTN : 0));
          // scheduling groups (masks: 0x100 LDS reads, 0x008 MFMA, 0x020
          // vector memory reads): the next tile's first fragment reads (two
          // per fragment of a transposed operand), then one DMA instruction
          // after each MFMA while they last
          if constexpr (!C::FB1)
            __builtin_amdgcn_sched_group_barrier(0x100, (NA * (C::TM + (TALL ? 1 : 0)) * (A_T ? 2 : 1)) + (NB * C::TN * (B_T ? 2 : 1)), 0);
#pragma unroll
          for (int i = 0; i < NM; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i < IPT) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int kt = 0;
  for (; kt + NST < nk; ++kt) body(kt, std::integral_constant<int, 0>{});
  issued = nk - 1;
  for (; kt + 1 < nk; ++kt) body(kt, std::integral_constant<int, 1>{});
  body(kt, std::integral_constant<int, 2>{});
  __syncthreads();  // the caller's epilogue reuses the LDS
}

// LDS elements of one pipeline stage and of the whole (double-buffered)
// main loop with NA A operands and NB B operands.
template <class C, int NA, int NB>
constexpr int stage_elems() { return (NA * C::BM + NB * C::BN) * C::LDK; }
// 16-bit operands always take the direct-to-LDS loop, whose tiles are
// unpadded; fp32 keeps the padded pitch of the register-staged loop.
template <class C, int NA, int NB>
constexpr int smem_elems() {
  return C::V == 8 ? C::NST * (NA * C::AR + NB * C::BN) * C::BK : 2 * stage_elems<C, NA, NB>();
}

// acc[a * NB + b][tn][tm] += B_b-tile x A_a-tile over k in [0, K).
// Two LDS stages: while the waves multiply out of stage kt & 1, the k-tile
// kt + 1 (fetched into registers one iteration earlier) is written to the
// other stage and k-tile kt + 2 is fetched from global memory, so each global
// load has a whole iteration of MFMA work to land and every iteration needs a
// single barrier.
//
// An optional second K segment (a2, b2, K2: same ld and rows as a and b)
// continues the same pipeline, so sum_k A1 B1 + sum_k A2 B2 runs as one loop.
template <class C, typename T, bool A_T, bool B_T, int NA, int NB, bool AG = false>
MOE_DEV void mainloop(f32x16 (&acc)[NA * NB][C::TN][C::TM], const OpDesc<T> (&a)[NA],
                      const OpDesc<T> (&b)[NB], int K, T* smem, const OpDesc<T>* a2 = nullptr,
                      const OpDesc<T>* b2 = nullptr, int K2 = 0) {
  // DMA for every bf16 operand layout; fp32 K-major operands keep the
  // register-staged transpose below (the transposing LDS read is 16-bit)
  static_assert(C::XR == 0, "tall tiles run mainloop_x");
  if constexpr (sizeof(T) == 2 || (!A_T && !B_T)) {
    static_assert(C::NST * (NA * C::BM + NB * C::BN) * C::BK <= smem_elems<C, NA, NB>(), "LDS");
    f32x16 unused[NA * NB][C::XTN];
    mainloop_dma<C, T, A_T, B_T, NA, NB, AG>(acc, unused, a, b, K, smem, a2, b2, K2);
    return;
  }
  constexpr int STAGE = stage_elems<C, NA, NB>();
  constexpr int B_OFF = NA * C::BM * C::LDK;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  static_assert(!AG || !A_T, "gathered rows: K-contiguous A");
  Stager<C, T, C::BM, A_T, AG> sa[NA];
  Stager<C, T, C::BN, B_T> sb[NB];
  const int nk1 = (K + C::BK - 1) / C::BK;
  const int nk = nk1 + (K2 > 0 ? (K2 + C::BK - 1) / C::BK : 0);
  if (nk <= 0) return;

#pragma unroll
  for (int i = 0; i < NA; ++i) {
    sa[i].init(a[i], tid);
    if (K2 > 0) sa[i].init_second(a2[i]);
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    sb[i].init(b[i], tid);
    if (K2 > 0) sb[i].init_second(b2[i]);
  }
  auto fetch = [&](int kt) {
    const int seg = kt >= nk1 ? 1 : 0;
    const int k0 = (kt - seg * nk1) * C::BK;
#pragma unroll
    for (int i = 0; i < NA; ++i) sa[i].load(k0, seg);
#pragma unroll
    for (int i = 0; i < NB; ++i) sb[i].load(k0, seg);
  };
  auto put = [&](T* stage) {
#pragma unroll
    for (int i = 0; i < NA; ++i) sa[i].store(stage + i * C::BM * C::LDK, tid);
#pragma unroll
    for (int i = 0; i < NB; ++i) sb[i].store(stage + B_OFF + i * C::BN * C::LDK, tid);
  };

  fetch(0);
  put(smem);
  if (nk > 1) fetch(1);
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * C::V;
  constexpr int KSTEPS = C::BK / (2 * C::V);
  // Fragments of one k-step; two register sets so the LDS reads of step
  // kk + 1 are in flight while the MFMAs of step kk issue.
  u32x4 af[2][NA][C::TM], bfr[2][NB][C::TN];
  auto read_frags = [&](const T* sA, const T* sB, int kk, int set) {
#pragma unroll
    for (int i = 0; i < NA; ++i)
#pragma unroll
      for (int tm = 0; tm < C::TM; ++tm)
        af[set][i][tm] = *reinterpret_cast<const u32x4*>(
            sA + i * C::BM * C::LDK + (wm * C::WM + tm * 32 + frag_row) * C::LDK + kk + frag_k);
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int tn = 0; tn < C::TN; ++tn)
        bfr[set][i][tn] = *reinterpret_cast<const u32x4*>(
            sB + i * C::BN * C::LDK + (wn * C::WN + tn * 32 + frag_row) * C::LDK + kk + frag_k);
  };
  for (int kt = 0; kt < nk; ++kt) {
    const T* sA = smem + (kt & 1) * STAGE;
    const T* sB = sA + B_OFF;
    read_frags(sA, sB, 0, 0);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < KSTEPS) read_frags(sA, sB, (ks + 1) * 2 * C::V, cur ^ 1);
#pragma unroll
      for (int ia = 0; ia < NA; ++ia)
#pragma unroll
        for (int ib = 0; ib < NB; ++ib)
#pragma unroll
          for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
            for (int tm = 0; tm < C::TM; ++tm)
              mfma_frag(acc[ia * NB + ib][tn][tm], bfr[cur][ib][tn], af[cur][ia][tm], T());
      __builtin_amdgcn_sched_barrier(0);
    }
    if (kt + 1 < nk) {
      // stage (kt + 1) & 1 was last read in iteration kt - 1, which every
      // wave finished before the barrier that closed that iteration
      put(smem + ((kt + 1) & 1) * STAGE);
      // keep the next fetch below the stores: hoisting it would need a
      // second set of staging registers
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 2 < nk) fetch(kt + 2);
    }
    __syncthreads();
  }
}

// mainloop for a row tile that may be tall (C::XR > 0, bf16): xacc holds the
// wave's extra blocks (unused when C::XR == 0).
template <class C, typename T, bool A_T, bool B_T, int NA, int NB, bool AG = false>
MOE_DEV void mainloop_x(f32x16 (&acc)[NA * NB][C::TN][C::TM], f32x16 (&xacc)[NA * NB][C::XTN],
                        const OpDesc<T> (&a)[NA], const OpDesc<T> (&b)[NB], int K, T* smem,
                        const OpDesc<T>* a2 = nullptr, const OpDesc<T>* b2 = nullptr,
                        int K2 = 0) {
  if constexpr (C::XR > 0)
    mainloop_dma<C, T, A_T, B_T, NA, NB, AG>(acc, xacc, a, b, K, smem, a2, b2, K2);
  else
    mainloop<C, T, A_T, B_T, NA, NB, AG>(acc, a, b, K, smem, a2, b2, K2);
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
template <class C, int NACC>
MOE_DEV void zero_acc(f32x16 (&acc)[NACC][C::TN][C::TM], f32x16 (&xacc)[NACC][C::XTN]) {
  zero_acc<C, NACC>(acc);
#pragma unroll
  for (int x = 0; x < NACC; ++x)
#pragma unroll
    for (int j = 0; j < C::XTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) xacc[x][j][r] = 0.0f;
}

// Calls f(m_local, n_local, v) for every 4-wide output fragment of the tile,
// where v[x][i] = acc[x] at (m_local, n_local + i).
template <class C, int NACC, class F>
MOE_DEV void for_each_frag(const f32x16 (&acc)[NACC][C::TN][C::TM], F&& f) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
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
        // one 32 x 32 block at a time: keeps the scheduler from moving every
        // accumulator into VGPRs at once
        if (q == 3) __builtin_amdgcn_sched_barrier(0);
      }
}

constexpr int kLdsBytes = 160 * 1024;  // LDS one workgroup may hold on gfx950
// Rows of a wave's block the row epilogue stages at once: all WM rows, or one
// 32-row MFMA block at a time when the whole blocks of every wave would
// outgrow the LDS (the 96-row wave blocks of a 192-row tile with two
// accumulator sets).
template <class C, int NACC>
constexpr int epi_rows() { return C::NW * NACC * C::WM * 36 * 4 <= kLdsBytes ? C::WM : 32; }
// LDS floats the row epilogue needs: every wave stages NACC blocks of
// epi_rows x 32 accumulators, rows padded to 36 floats.
template <class C, int NACC>
constexpr int epi_lds_floats() { return C::NW * NACC * epi_rows<C, NACC>() * 36; }

// LDS elements of a kernel whose main loop (NA A / NB B operands) is followed
// by the row epilogue over NACC accumulator sets in the same buffer.
template <class C, typename T, int NA, int NB, int NACC>
constexpr int kernel_smem_elems() {
  constexpr int a = smem_elems<C, NA, NB>();
  constexpr int b = (epi_lds_floats<C, NACC>() * 4 + (int)sizeof(T) - 1) / (int)sizeof(T);
  return a > b ? a : b;
}

// Row epilogue: calls f(m_local, n_local, v, q) with v[x][i] = acc[x] at
// (m_local, n_local + i) for i < 8, n_local a multiple of 8.  The accumulators
// of one 32-column block (epi_rows rows of it at a time) are first written to
// a wave-private LDS region and read back as rows, so the caller's element-wise work runs on 8 consecutive
// outputs per lane (16-byte bf16 stores) and only one block's accumulators is
// in VGPRs at a time.  The LDS must no longer be in use by the main loop (it
// ends with a barrier); regions are wave-private, so no barrier is needed.
// With a prefetch type QT other than NoPre, pre(m_local, n_local, q) is called
// for every row of a block before any row of it is visited: it issues the
// loads the visit needs into q (a QT), so a block's loads are all in flight
// together instead of being waited for row group by row group, and the next
// block's loads are issued before this block's rows are visited.
struct NoPre {};
template <class C, int NACC, class QT, class PRE, class F>
MOE_DEV void for_each_row8_pre(const f32x16 (&acc)[NACC][C::TN][C::TM], float* lds, PRE&& pre,
                               F&& f) {
  static_assert(C::WM % 16 == 0, "rows are visited 16 at a time");
  constexpr int P = 36;  // padded row pitch (floats)
  constexpr bool HAS_PRE = !std::is_same<QT, NoPre>::value;
  constexpr int SR = epi_rows<C, NACC>();  // rows staged per pass
  constexpr int NSP = C::WM / SR;          // passes per 32-column block
  constexpr int RG = SR / 16;              // row groups of a pass
  constexpr int NPASS = C::TN * NSP;       // passes of the wave's block
  static_assert(C::WM % SR == 0 && SR % 32 == 0, "whole MFMA blocks per pass");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  float* reg = lds + wave * NACC * SR * P;
  // the loads of pass b + 1 are issued before the rows of pass b are visited
  // (two register sets), so their latency overlaps one pass of work
  QT q[2][RG];
  auto prefetch = [&](int b, int set) {
    const int r0 = wm * C::WM + (b % NSP) * SR;
#pragma unroll
    for (int g = 0; g < RG; ++g)
      pre(r0 + g * 16 + (lane >> 2), wn * C::WN + (b / NSP) * 32 + (lane & 3) * 8, q[set][g]);
  };
  if constexpr (HAS_PRE) prefetch(0, 0);
#pragma unroll
  for (int b = 0; b < NPASS; ++b) {  // unrolled: acc is indexed by constants only
    const int tn = b / NSP, sp = b % NSP, set = b & 1;
    const int r0 = wm * C::WM + sp * SR;  // first row of this pass
    if constexpr (HAS_PRE) {
      if (b + 1 < NPASS) prefetch(b + 1, set ^ 1);
    }
#pragma unroll
    for (int x = 0; x < NACC; ++x)
#pragma unroll
      for (int tl = 0; tl < SR / 32; ++tl)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int tm = sp * (SR / 32) + tl;
          const int row = tl * 32 + (lane & 31);
          const int col = 8 * qq + 4 * (lane >> 5);
          *reinterpret_cast<f32x4*>(reg + (x * SR + row) * P + col) =
              f32x4{acc[x][tn][tm][4 * qq], acc[x][tn][tm][4 * qq + 1],
                    acc[x][tn][tm][4 * qq + 2], acc[x][tn][tm][4 * qq + 3]};
        }
    __builtin_amdgcn_sched_barrier(0);
    auto visit = [&](int g) {
      const int row = g * 16 + (lane >> 2);
      const int col = (lane & 3) * 8;
      float v[NACC][8];
#pragma unroll
      for (int x = 0; x < NACC; ++x) {
        const f32x4 lo = *reinterpret_cast<const f32x4*>(reg + (x * SR + row) * P + col);
        const f32x4 hi = *reinterpret_cast<const f32x4*>(reg + (x * SR + row) * P + col + 4);
        v[x][0] = lo[0]; v[x][1] = lo[1]; v[x][2] = lo[2]; v[x][3] = lo[3];
        v[x][4] = hi[0]; v[x][5] = hi[1]; v[x][6] = hi[2]; v[x][7] = hi[3];
      }
      f(r0 + row, wn * C::WN + tn * 32 + col, v, q[set][g]);
    };
    if constexpr (HAS_PRE) {
#pragma unroll
      for (int g = 0; g < RG; ++g) visit(g);  // q[set][g] needs constant indices
    } else {
#pragma unroll 2
      for (int g = 0; g < RG; ++g) visit(g);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <class C, int NACC, class F>
MOE_DEV void for_each_row8(const f32x16 (&acc)[NACC][C::TN][C::TM], float* lds, F&& f) {
  for_each_row8_pre<C, NACC, NoPre>(acc, lds, [](int, int, NoPre&) {},
                                    [&](int m, int n, auto& v, const NoPre&) { f(m, n, v); });
}

// for_each_row8_pre over a tile that may be tall: the main blocks, then the
// wave's extra blocks (C::XR > 0: rows BM + 32 (wm & 1) .., columns of half
// wm >> 1 of its WN), staged the same way, 32 rows at a time.
template <class C, int NACC, class QT, class PRE, class F>
MOE_DEV void for_each_row8_xpre(const f32x16 (&acc)[NACC][C::TN][C::TM],
                                const f32x16 (&xacc)[NACC][C::XTN], float* lds, PRE&& pre,
                                F&& f) {
  auto extra = [&]() {
    constexpr int P = 36;
    constexpr int SR = epi_rows<C, NACC>();
    static_assert(SR >= 32, "one 32-row block per pass");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / C::WGN, wn = wave % C::WGN;
    float* reg = lds + wave * NACC * SR * P;
    const int r0 = C::BM + 32 * (C::XR == 128 ? wm : (wm & 1));
    const int c0 = wn * C::WN + (C::XR == 128 ? 0 : (wm >> 1) * (C::WN / 2));
#pragma unroll
    for (int j = 0; j < C::XTN; ++j) {
      QT q[2];
      if constexpr (!std::is_same<QT, NoPre>::value) {
#pragma unroll
        for (int g = 0; g < 2; ++g) pre(r0 + g * 16 + (lane >> 2), c0 + j * 32 + (lane & 3) * 8, q[g]);
      }
#pragma unroll
      for (int x = 0; x < NACC; ++x)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int row = lane & 31;
          const int col = 8 * qq + 4 * (lane >> 5);
          *reinterpret_cast<f32x4*>(reg + (x * SR + row) * P + col) =
              f32x4{xacc[x][j][4 * qq], xacc[x][j][4 * qq + 1], xacc[x][j][4 * qq + 2],
                    xacc[x][j][4 * qq + 3]};
        }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int row = g * 16 + (lane >> 2);
        const int col = (lane & 3) * 8;
        float v[NACC][8];
#pragma unroll
        for (int x = 0; x < NACC; ++x) {
          const f32x4 lo = *reinterpret_cast<const f32x4*>(reg + (x * SR + row) * P + col);
          const f32x4 hi = *reinterpret_cast<const f32x4*>(reg + (x * SR + row) * P + col + 4);
          v[x][0] = lo[0]; v[x][1] = lo[1]; v[x][2] = lo[2]; v[x][3] = lo[3];
          v[x][4] = hi[0]; v[x][5] = hi[1]; v[x][6] = hi[2]; v[x][7] = hi[3];
        }
        f(r0 + row, c0 + j * 32 + col, v, q[g]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if constexpr (C::XR == 128) {
    // the extra blocks first: their 64 accumulators are then dead during the
    // main passes (config 3 gate/up input gradient 1.20 -> 1.19 ms)
    extra();
    for_each_row8_pre<C, NACC, QT>(acc, lds, pre, f);
  } else {
    for_each_row8_pre<C, NACC, QT>(acc, lds, pre, f);
    if constexpr (C::XR > 0) extra();
  }
}
template <class C, int NACC, class F>
MOE_DEV void for_each_row8_x(const f32x16 (&acc)[NACC][C::TN][C::TM],
                             const f32x16 (&xacc)[NACC][C::XTN], float* lds, F&& f) {
  for_each_row8_xpre<C, NACC, NoPre>(acc, xacc, lds, [](int, int, NoPre&) {},
                                     [&](int m, int n, auto& v, const NoPre&) { f(m, n, v); });
}

// Row epilogue for bf16 outputs that need no element-wise work beyond a scale:
// the accumulators of one 32-column block are scaled in fp32, rounded to bf16
// (v_cvt_pk_bf16_f32, as store8 rounds) and staged through a wave-private LDS
// region as packed pairs, half the LDS traffic of the fp32 staging above, then
// read back as rows of 8 outputs: f(m_local, n_local, p) with p[x] the 16-byte
// packed row of accumulator set x.  Row pitch 40 elements: the 8-byte writes
// of 32 rows and the 16-byte reads of 4 rows per phase spread over the banks
// (pitches 36 and 34 measured slower).  Same LDS preconditions as
// for_each_row8.
constexpr int kRowPitchBf16 = 40;
template <class C, int NACC>
constexpr int epi_lds_bf16_elems() { return C::NW * NACC * C::WM * kRowPitchBf16; }
template <class C, int NACC, class F>
MOE_DEV void for_each_row8_bf16(const f32x16 (&acc)[NACC][C::TN][C::TM], bf16_t* lds, float scale,
                                F&& f) {
  static_assert(C::WM % 16 == 0, "rows are visited 16 at a time");
  constexpr int P = kRowPitchBf16;
  constexpr int RG = C::WM / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  bf16_t* reg = lds + wave * NACC * C::WM * P;
#pragma unroll
  for (int tn = 0; tn < C::TN; ++tn) {  // unrolled: acc is indexed by constants only
#pragma unroll
    for (int x = 0; x < NACC; ++x)
#pragma unroll
      for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int row = tm * 32 + (lane & 31);
          const int col = 8 * qq + 4 * (lane >> 5);
          const f32x16& a = acc[x][tn][tm];
          *reinterpret_cast<u32x2*>(reg + (x * C::WM + row) * P + col) =
              u32x2{pack_bf16x2(scale * a[4 * qq], scale * a[4 * qq + 1]),
                    pack_bf16x2(scale * a[4 * qq + 2], scale * a[4 * qq + 3])};
        }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll 2
    for (int g = 0; g < RG; ++g) {
      const int row = g * 16 + (lane >> 2);
      const int col = (lane & 3) * 8;
      u32x4 pk[NACC];
#pragma unroll
      for (int x = 0; x < NACC; ++x)
        pk[x] = *reinterpret_cast<const u32x4*>(reg + (x * C::WM + row) * P + col);
      f(wm * C::WM + row, wn * C::WN + tn * 32 + col, pk);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Store / load 8 consecutive elements (8-element aligned) of one row in global
// memory.
MOE_DEV void store8(bf16_t* p, const float* v) {
  *gptr(reinterpret_cast<u32x4*>(p)) = u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                             pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
}
MOE_DEV void store8(float* p, const float* v) {
  *gptr(reinterpret_cast<f32x4*>(p)) = f32x4{v[0], v[1], v[2], v[3]};
  *gptr(reinterpret_cast<f32x4*>(p + 4)) = f32x4{v[4], v[5], v[6], v[7]};
}
MOE_DEV void load8(const bf16_t* p, float* v) {
  const u32x4 w = *gptr(reinterpret_cast<const u32x4*>(p));
  unpack16(w, v, bf16_t());
}
MOE_DEV void load8(const float* p, float* v) {
  const f32x4 a = *gptr(reinterpret_cast<const f32x4*>(p));
  const f32x4 b = *gptr(reinterpret_cast<const f32x4*>(p + 4));
  v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
  v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
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

// Store / load 4 consecutive elements (4-element aligned) of one row in global
// memory.
MOE_DEV void store4(bf16_t* p, const float* v) {
  *gptr(reinterpret_cast<u32x2*>(p)) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
}
MOE_DEV void store4(float* p, const float* v) {
  *gptr(reinterpret_cast<f32x4*>(p)) = f32x4{v[0], v[1], v[2], v[3]};
}
MOE_DEV void load4(const bf16_t* p, float* v) {
  const u32x2 w = *gptr(reinterpret_cast<const u32x2*>(p));
  v[0] = __uint_as_float(w.x << 16); v[1] = __uint_as_float(w.x & 0xffff0000u);
  v[2] = __uint_as_float(w.y << 16); v[3] = __uint_as_float(w.y & 0xffff0000u);
}
MOE_DEV void load4(const float* p, float* v) {
  f32x4 w = *gptr(reinterpret_cast<const f32x4*>(p));
  v[0] = w[0]; v[1] = w[1]; v[2] = w[2]; v[3] = w[3];
}

}  // namespace moe
