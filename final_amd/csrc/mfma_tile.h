// MFMA tile of the grouped and dense GEMMs: C = A . B^T on
// v_mfma_f32_32x32x2_f32, LDS double-buffered slabs with global loads three
// slabs ahead.
#pragma once

#include "gpu_common.h"

namespace moe {

// ---------------------------------------------------------------------------
// MFMA grouped GEMM tile
// ---------------------------------------------------------------------------

template <int BM> struct TileCfg;
// 4 waves as WAVES_M x WAVES_N; a wave owns WM 32-row blocks x WN 32-column
// blocks.  B rows come in groups of 64 (gate/up phase: 32 rows of W1, then
// the same 32 columns' rows of W3), and the epilogue pairs them through LDS.
template <> struct TileCfg<128> {
  static constexpr int WAVES_M = 2, WM = 2, WAVES_N = 2, WN = 2, BK = 32, NS = 2;
};
// 64x128 tiles (49-831 tokens): 64x256 tiles left 1.4 tiles per block at
// T=256 (637 us per step, 527 with 64x128); 64x64 tiles balance the blocks
// better but lose more per tile (537 us at T=256, 1208 vs 1115 at T=1024)
template <> struct TileCfg<64> {
  static constexpr int WAVES_M = 2, WM = 1, WAVES_N = 2, WN = 2, BK = 32, NS = 3;
};
template <> struct TileCfg<32> {
  static constexpr int WAVES_M = 1, WM = 1, WAVES_N = 4, WN = 2, BK = 16, NS = 3;
};

// Half-width down tiles for the last units of a launch (same rows, half the
// columns), so the last round of tiles is half as long.
template <int BM> struct TileHalfCfg;
template <> struct TileHalfCfg<128> {
  static constexpr int WAVES_M = 4, WM = 1, WAVES_N = 1, WN = 2, BK = 32, NS = 3;
};
template <> struct TileHalfCfg<64> {
  static constexpr int WAVES_M = 2, WM = 1, WAVES_N = 2, WN = 1, BK = 32, NS = 3;
};
template <> struct TileHalfCfg<32> {
  static constexpr int WAVES_M = 1, WM = 1, WAVES_N = 4, WN = 1, BK = 16, NS = 3;
};

template <int BM_, typename C> struct TileT {
  static constexpr int BM = BM_;
  static constexpr int WAVES_M = C::WAVES_M, WM = C::WM, WAVES_N = C::WAVES_N, WN = C::WN;
  static constexpr int BK = C::BK;
  static constexpr int NS = C::NS;             // slabs of global loads in flight
  static constexpr int BN = WAVES_N * WN * 32;
  static constexpr int PITCH = BK + 4;           // floats per LDS row
  static constexpr int KV = BK / 4;              // float4 per row per slab
  static constexpr int A_F4 = BM * KV;           // float4 per A slab
  static constexpr int B_F4 = BN * KV;
  static constexpr int A_PER = (A_F4 + kThreads - 1) / kThreads;
  static constexpr int B_PER = (B_F4 + kThreads - 1) / kThreads;
  static constexpr int CPITCH = BN + 8;          // epilogue tile row pitch
  static constexpr int SLAB_FLOATS = 2 * (BM + BN) * PITCH;
  static constexpr int EPI_FLOATS = BM * CPITCH;
  static constexpr int LDS_FLOATS = SLAB_FLOATS > EPI_FLOATS ? SLAB_FLOATS : EPI_FLOATS;
  static_assert(BM == WAVES_M * WM * 32, "tile rows");
  static_assert(WAVES_M * WAVES_N == kThreads / 64, "four waves");
  static_assert(BN % 64 == 0, "whole W1/W3 row groups");
  static_assert(BK % 8 == 0, "k groups of 8");
};
template <int BM> using Tile = TileT<BM, TileCfg<BM>>;
template <int BM> using TileHalf = TileT<BM, TileHalfCfg<BM>>;

// Slab staging of the MFMA tile: buffer float4 loads into registers (A rows
// gathered; an empty row's offset lies past the buffer, so its loads return
// zeros without a branch; B rows contiguous with stride K), then LDS stores.
// Every load is unconditional, so the compiler's count of loads in flight
// stays exact and a slab's LDS stores wait only for that slab.  Fully
// unrolled with compile-time indices so the arrays stay in registers while
// the loads are in flight.
constexpr uint32_t kTileOOB = 0xFF000000u;  // past every A buffer (moe_create bounds them)

template <int A_PER, int B_PER, int RPP>
__device__ __forceinline__ void slab_load(f32x4 (&ra)[A_PER], f32x4 (&rb)[B_PER],
                                          const uint32_t (&a_off)[A_PER],
                                          __amdgpu_buffer_rsrc_t ar, uint32_t b_off,
                                          __amdgpu_buffer_rsrc_t br, int K, int k0) {
  // per-thread offsets are the same for every slab; the slab's k offset is
  // the instruction's scalar offset, so no VGPR is rewritten per slab (a
  // rewritten address register made the compiler wait for loads in flight)
  const int ks = k0 * 4;
#pragma unroll
  for (int i = 0; i < A_PER; ++i)
    ra[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ar, a_off[i], ks, 0));
#pragma unroll
  for (int i = 0; i < B_PER; ++i)
    rb[i] = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(br, b_off + (uint32_t)(i * RPP * K) * 4u, ks, 0));
}

template <int BM, int A_PER, int B_PER, int RPP, int PITCH>
__device__ __forceinline__ void slab_store(const f32x4 (&ra)[A_PER], const f32x4 (&rb)[B_PER],
                                           float *As, float *Bs, int lds_st, int lrow) {
#pragma unroll
  for (int i = 0; i < A_PER; ++i)
    if (A_PER * RPP <= BM || lrow + i * RPP < BM)  // rows past BM: threads of a partial pass
      st4(As + lds_st + i * RPP * PITCH, ra[i]);
#pragma unroll
  for (int i = 0; i < B_PER; ++i) st4(Bs + lds_st + i * RPP * PITCH, rb[i]);
}


// A-operand readiness of a tile's slabs.  NoWait: A is complete before the
// tile starts.  SlabReady: A is the intermediate rows of one unit, whose
// gate/up tiles each set one bit of a mask when their stores have completed
// (tile n wrote columns [n w, n w + w)); wave 0 waits for the bits a slab's
// columns need before the barrier that precedes the slab's loads, and keeps
// the bits it has seen (wave-uniform, so the state stays in scalar
// registers).  The rows are written once with agent-scope
// stores and read by no one before their bit is set, so the loads after the
// wait need no fence (the caches start the kernel invalidated).
struct NoWait {
  static constexpr bool kActive = false;
  __device__ void wait(int) {}
};
// Slow path of SlabReady: polls mask word w until it holds bit mask m (or
// the wait gives up and reports a timeout); returns the word.  Out of line
// and with scalar arguments, so the slab loop keeps its registers and its
// state stays out of memory.
__device__ __attribute__((noinline)) unsigned slab_poll(const int *w, unsigned m, int limit,
                                                         int *err) {
  unsigned seen = 0;
  for (int spins = 0;; ++spins) {
    seen = (unsigned)__builtin_amdgcn_readfirstlane(load_relaxed(w));
    if ((seen & m) == m) return seen;
    if (spins >= limit) {
      if ((threadIdx.x & 63) == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return seen | m;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

struct SlabReady {
  static constexpr bool kActive = true;
  const int *bits;   // mask words of the unit (bit n: word n / 32)
  int shift;         // log2 of the slabs one gate/up tile's columns span
  int nslab;
  int limit;         // polls before the wait gives up and reports a timeout
  int *err;
  int word = -1;     // the mask word last read (slabs come in order)
  unsigned seen = 0;
  // wave 0: wait until the gate/up tile behind the slab's columns is done
  __device__ __forceinline__ void wait(int slab) {
    if (slab >= nslab) return;
    const int b = slab >> shift;
    const unsigned m = 1u << (b & 31);
    if (b >> 5 != word) {
      word = b >> 5;
      seen = 0;
    }
    if (!(seen & m)) seen = slab_poll(bits + word, m, limit, err);
  }
};

// Wave layouts of the slab loop, chosen once per tile (each is its own
// instantiation, so the inner loops have no runtime branches on the layout).
//   kWide: the config's WAVES_M x WAVES_N grid of 32x32 blocks.
//   kFull: kWide for a tile whose rows are all valid, with no row checks in
//     its inner loop (straight-line MFMA code).
//   kNarrow (64-row tiles whose valid rows fit the first 32-row block, and
//     128-row tiles with 81-96 valid rows): instead of the waves of the
//     empty row blocks idling on their SIMDs, each of the 4 waves takes one
//     32-column block and every row block that holds rows (a 128-row tile
//     with 3 of its 4 row blocks then costs 3/4 of a full one).
//   kSkinny1 / kSkinny2 / kSkinny3 (64-row tiles with 1-16, 17-32 or 33-48
//     valid rows, which 32-row blocks pad to twice or 4/3 the rows):
//     v_mfma_f32_16x16x4_f32 over 1, 2 or 3 16-row blocks, each wave taking
//     a quarter of the columns as 16-column blocks (the 2-block form serves
//     the half-width tiles, which the narrow layout cannot split in four).
//     kSkinny5 / kSkinny7: the same over 5 or 7 16-row blocks, for 128-row
//     tiles with 65-80 or 97-112 valid rows (5/8 and 7/8 of a full tile's
//     MFMAs, where 32-row blocks take 3/4 and all of it).
// Same tile, LDS layout and products in every layout.
enum TileLayout {
  kWide = 0, kNarrow = 1, kSkinny1 = 2, kSkinny3 = 3, kFull = 4, kSkinny2 = 5, kSkinny5 = 6,
  kSkinny7 = 7
};

// 64x128 tiles (the 2 x 2 grid of 32x64 wave tiles) and 128x128 tiles (2 x 2
// of 64x64): four 32-column blocks, one per wave.  (A 128-row tile with at
// most 64 valid rows runs as a 64-row tile; its caller decides.)
template <typename TL>
constexpr bool tile_narrowable() {
  return TL::WAVES_M == 2 && TL::WAVES_N == 2 && TL::WN == 2 && TL::BN == 128;
}
// 64- and 128-row tiles of 4 waves whose columns split into 16-column blocks
// per wave (64x128, the half-width 64x64, 128x128): the 16-row layouts.
template <typename TL>
constexpr bool tile_skinnyable() {
  return (TL::BM == 64 || TL::BM == 128) && TL::WAVES_M * TL::WAVES_N == 4 && TL::BN % 64 == 0;
}

// The block's next task, claimed by thread 0 at the end of a tile's MFMAs:
// from a queue head (null: none, 0 returned) or by a callable.
__device__ __forceinline__ int claim_next(int *head) { return head ? claim(head) : 0; }
__device__ __forceinline__ int claim_next(decltype(nullptr)) { return 0; }
template <typename F>
__device__ __forceinline__ int claim_next(F &next_task) {
  return next_task();
}

// Slab loop of one tile: global loads NS slabs ahead in registers, LDS
// double-buffered, one barrier per slab; then the block's next task is
// claimed (thread 0; returned) and the products are written to the LDS
// epilogue tile Cs [BM][CPITCH] in B-row order.
template <typename TL, TileLayout LAYOUT, typename Ready, typename Claim>
__device__ __forceinline__ int tile_slabs(float *lds, const uint32_t (&a_src)[TL::A_PER],
                                          __amdgpu_buffer_rsrc_t abase_r,
                                          __amdgpu_buffer_rsrc_t bsrc_r,
                                          __amdgpu_buffer_rsrc_t none_r, uint32_t bsrc, int lds_st,
                                          int lrow, int K, int rows_valid, Claim &head, Ready &ready) {
  constexpr int BM = TL::BM, BN = TL::BN;
  constexpr int WM = TL::WM, WN = TL::WN, BK = TL::BK, PITCH = TL::PITCH;
  constexpr int A_PER = TL::A_PER, B_PER = TL::B_PER;
  constexpr int ROWS_PER_PASS = kThreads / TL::KV;
  constexpr bool SKINNY = LAYOUT == kSkinny1 || LAYOUT == kSkinny2 || LAYOUT == kSkinny3 ||
                          LAYOUT == kSkinny5 || LAYOUT == kSkinny7;
  constexpr bool NARROW = LAYOUT == kNarrow;
  static_assert(!NARROW || tile_narrowable<TL>(), "narrow layout of 64x128 tiles");
  static_assert(!SKINNY || tile_skinnyable<TL>(), "16-row layouts of 64-row tiles");
  float *As = lds;                      // [2][BM][PITCH]
  float *Bs = lds + 2 * BM * PITCH;     // [2][BN][PITCH]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform branches

  // 32x32 layouts: this wave's row blocks (AM from wrow0) and column blocks
  // (AN from cb0), and rows that hold data (0 = skip the MFMAs; a row block
  // starting at or past wrows is skipped; wave-uniform branches)
  constexpr int AM = NARROW ? TL::WAVES_M * WM : WM;
  constexpr int AN = NARROW ? 1 : WN;
  const int wm = NARROW ? 0 : wave % TL::WAVES_M;
  const int cb0 = NARROW ? wave : (wave / TL::WAVES_M) * WN;
  const int wrow0 = wm * WM * 32;
  const int wrows = LAYOUT == kFull ? AM * 32 : min(max(rows_valid - wrow0, 0), AM * 32);
  const int lr = lane & 31, lh = (lane >> 5) * 4;
  const float *a_rd = As + (wrow0 + lr) * PITCH + lh;
  const float *b_rd = Bs + (cb0 * 32 + lr) * PITCH + lh;
  // skinny layout: lane l supplies row l % 16 at k offset 4 * (l / 16) of each
  // 16-wide k group, as a float4 whose component q feeds the q-th MFMA (the
  // same k permutation in A and B)
  constexpr int SRB = LAYOUT == kSkinny7 ? 7 : LAYOUT == kSkinny5 ? 5 : LAYOUT == kSkinny3 ? 3
                      : LAYOUT == kSkinny2 ? 2 : 1;
  static_assert(SRB * 16 <= BM, "16-row blocks of the tile");
  constexpr int SKC = BN / 64;  // 16-column blocks per wave
  const int l16 = lane & 15, k16 = (lane >> 4) * 4;
  const float *a16 = As + l16 * PITCH + k16;
  const float *b16 = Bs + (wave * 16 * SKC + l16) * PITCH + k16;

  floatx16 acc[SKINNY ? 1 : AM][SKINNY ? 1 : AN];
  f32x4 acc16[SRB][SKINNY ? SKC : 1];
  if constexpr (SKINNY) {
#pragma unroll
    for (int i = 0; i < SRB; ++i)
#pragma unroll
      for (int c = 0; c < SKC; ++c) acc16[i][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  } else {
#pragma unroll
    for (int i = 0; i < AM; ++i)
#pragma unroll
      for (int c = 0; c < AN; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][c][r] = 0.0f;
  }

  const int nslab = K / BK;
  // Global loads run NS slabs ahead in NS register sets: slab t + NS is
  // loaded while slab t's MFMAs run, and slab t + 1 (loaded NS - 1 slabs
  // earlier) is written to LDS after them.
  constexpr int NS = TL::NS;
  constexpr int L = NS % 2 == 0 ? NS : 2 * NS;  // steps per unrolled round
  f32x4 sa[NS][A_PER], sb[NS][B_PER];
  if constexpr (Ready::kActive) {
    // the A columns of the slabs loaded before the loop (0 .. NS - 1) and in
    // its first step (NS); each later step waits for the one after it
    if (wave == 0)
      for (int j = 0; j <= NS; ++j) ready.wait(j);
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const bool in = j < nslab;
    slab_load<A_PER, B_PER, ROWS_PER_PASS>(sa[j], sb[j], a_src, in ? abase_r : none_r, bsrc,
                                           in ? bsrc_r : none_r, K, in ? j * BK : 0);
  }
  slab_store<BM, A_PER, B_PER, ROWS_PER_PASS, PITCH>(sa[0], sb[0], As, Bs, lds_st, lrow);
  __syncthreads();
  for (int s = 0; s < nslab; s += L) {
#pragma unroll
    for (int u = 0; u < L; ++u) {
      const int t = s + u;
      if (t >= nslab) break;
      // the set of slab t is free (written to LDS a step ago): slab t + NS.
      // The scheduling barrier keeps these loads ahead of the step's MFMAs:
      // sunk below them, their destinations took the MFMA operands'
      // registers, and the next step's first LDS reads then waited for them.
      {
        const bool in = t + NS < nslab;
        slab_load<A_PER, B_PER, ROWS_PER_PASS>(sa[u % NS], sb[u % NS], a_src, in ? abase_r : none_r,
                                               bsrc, in ? bsrc_r : none_r, K, in ? (t + NS) * BK : 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (SKINNY) {
        const float *A16 = a16 + (u & 1) * BM * PITCH;
        const float *B16 = b16 + (u & 1) * BN * PITCH;
#pragma unroll
        for (int g16 = 0; g16 < BK / 16; ++g16) {
          f32x4 af[SRB], bf[SKC];
#pragma unroll
          for (int i = 0; i < SRB; ++i) af[i] = ld4(A16 + i * 16 * PITCH + g16 * 16);
#pragma unroll
          for (int c = 0; c < SKC; ++c) bf[c] = ld4(B16 + c * 16 * PITCH + g16 * 16);
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int i = 0; i < SRB; ++i)
#pragma unroll
              for (int c = 0; c < SKC; ++c)
                acc16[i][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][q], bf[c][q], acc16[i][c], 0, 0, 0);
        }
      } else if (wrows > 0) {
        const float *Ac = a_rd + (u & 1) * BM * PITCH;
        const float *Bc = b_rd + (u & 1) * BN * PITCH;
#pragma unroll
        for (int g8 = 0; g8 < BK / 8; ++g8) {
          f32x4 af[AM], bf[AN];
#pragma unroll
          for (int i = 0; i < AM; ++i)
            if (i == 0 || wrows > i * 32) af[i] = ld4(Ac + i * 32 * PITCH + g8 * 8);
#pragma unroll
          for (int c = 0; c < AN; ++c) bf[c] = ld4(Bc + c * 32 * PITCH + g8 * 8);
#pragma unroll
          for (int i = 0; i < AM; ++i) {
            if (i > 0 && wrows <= i * 32) break;
#pragma unroll
            for (int c = 0; c < AN; ++c) {
#pragma unroll
              for (int q = 0; q < 4; ++q)
                acc[i][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][q], bf[c][q], acc[i][c], 0, 0, 0);
            }
          }
        }
      }
      // slab t + 1 (past the end: zeros into a buffer nobody reads again)
      slab_store<BM, A_PER, B_PER, ROWS_PER_PASS, PITCH>(
          sa[(u + 1) % NS], sb[(u + 1) % NS], As + ((u + 1) & 1) * BM * PITCH,
          Bs + ((u + 1) & 1) * BN * PITCH, lds_st, lrow);
      // the next step loads slab t + 1 + NS: its A columns before the barrier
      if constexpr (Ready::kActive)
        if (wave == 0) ready.wait(t + 1 + NS);
      __syncthreads();
    }
  }

  const int next = threadIdx.x == 0 ? claim_next(head) : 0;

  // Products into the epilogue tile (the slab buffers are free after the
  // last barrier).
  constexpr int CP = TL::CPITCH;
  float *Cs = lds;
  if constexpr (SKINNY) {
    // 16x16 f32 MFMA result layout: lane l holds column l % 16 and rows
    // 4 * (l / 16) + r for r = 0..3
#pragma unroll
    for (int i = 0; i < SRB; ++i)
#pragma unroll
      for (int c = 0; c < SKC; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          Cs[(i * 16 + k16 + r) * CP + wave * 16 * SKC + c * 16 + l16] = acc16[i][c][r];
  } else if (wrows > 0) {
    // 32x32 f32 MFMA result layout: lane l holds column l % 32 and rows
    // 8*(r/4) + 4*(l/32) + r%4 for r = 0..15
#pragma unroll
    for (int i = 0; i < AM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wrow0 + i * 32 + 8 * (r >> 2) + (lane >> 5) * 4 + (r & 3);
#pragma unroll
        for (int c = 0; c < AN; ++c) Cs[row * CP + (cb0 + c) * 32 + lr] = acc[i][c][r];
      }
    }
  }
  return next;
}

// One output tile of C[rows][cols] = A[rows][K] . B[cols][K]^T.
// A rows are gathered: row r starts at abase + aoff[r] (aoff in LDS; rows at
// or past rows_valid are zero; abytes = bytes readable from abase).  B rows
// are contiguous with stride K from brow0.  GATED: per wave the B tile holds
// 32 rows of W1 then the same 32 of W3 and the epilogue writes
// silu(W1 x) * (W3 x); otherwise the product.
//
// Slab pipeline: global loads of slab s+1 are in flight while the MFMAs of
// slab s run from LDS; one barrier per slab (double-buffered LDS).
// Thread 0 claims the block's next task with `head` (a queue head, or a
// callable that claims) once the MFMAs are done (returned; other threads
// return 0): the epilogue hides the claim's round trip, and a block commits
// to its next task only near the end of this one.  head == nullptr: no claim
// (grids of one tile per block).  `out` stores the
// epilogue's float4s: out.store(byte offset into [rows][ldo], value).
template <typename TL, bool GATED, typename Out = AgentOut, typename Ready = NoWait,
          typename Claim = int *>
__device__ __forceinline__ int mfma_tile(float *lds, const float *abase, uint32_t abytes,
                                         const int *aoff, int rows_valid,
                                         const float *brow0, int K, const Out &out,
                                         int row0, int ldo, int col0, Claim head,
                                         Ready ready = Ready{}) {
  constexpr int BM = TL::BM;
  constexpr int KV = TL::KV, A_PER = TL::A_PER;
  constexpr int ROWS_PER_PASS = kThreads / KV;  // rows one pass of loads covers
  static_assert(TL::B_F4 % kThreads == 0, "B slab splits evenly");
  const int tid = threadIdx.x;
  const int lrow = tid / KV, lc4 = (tid % KV) * 4;

  uint32_t a_src[A_PER];  // byte offset of this thread's A float4 (kTileOOB: zero row)
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int r = lrow + i * ROWS_PER_PASS;
    a_src[i] = (r < BM && r < rows_valid) ? (uint32_t)(aoff[r] + lc4) * 4u : kTileOOB;
  }
  const __amdgpu_buffer_rsrc_t abase_r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(abase), 0, (int)abytes, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t bsrc_r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(brow0), 0, (int)((uint32_t)TL::BN * K * 4u), kBufferRsrcWord3);
  // loads past the last slab use descriptors of size 0 (zeros, no traffic):
  // every load and LDS store of the loop is unconditional, which keeps the
  // compiler's count of loads in flight exact across the loop
  const __amdgpu_buffer_rsrc_t none_r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(brow0), 0, 0, kBufferRsrcWord3);
  const uint32_t bsrc = (uint32_t)(lrow * K + lc4) * 4u;
  const int lds_st = lrow * TL::PITCH + lc4;

  constexpr bool kNa = tile_narrowable<TL>(), kSk = tile_skinnyable<TL>() && BM == 64;
  constexpr bool kSkL = tile_skinnyable<TL>() && BM == 128;
  constexpr TileLayout kS1 = kSk ? kSkinny1 : kWide, kS2 = kSk ? kSkinny2 : kWide;
  constexpr TileLayout kS3 = kSk ? kSkinny3 : kWide, kNw = kNa ? kNarrow : kWide;
  constexpr TileLayout kS5 = kSkL ? kSkinny5 : kWide, kS7 = kSkL ? kSkinny7 : kWide;
  int next;
  if (kSkL && rows_valid > 64 && rows_valid <= 80)
    next = tile_slabs<TL, kS5, Ready, Claim>(lds, a_src, abase_r, bsrc_r, none_r, bsrc, lds_st, lrow, K,
                               rows_valid, head, ready);
  else if (kSkL && rows_valid > 96 && rows_valid <= 112)
    next = tile_slabs<TL, kS7, Ready, Claim>(lds, a_src, abase_r, bsrc_r, none_r, bsrc, lds_st, lrow, K,
                               rows_valid, head, ready);
  else if (kSk && rows_valid <= 16)
    next = tile_slabs<TL, kS1, Ready, Claim>(lds, a_src, abase_r, bsrc_r, none_r, bsrc, lds_st, lrow, K,
                               rows_valid, head, ready);
  else if (kSk && rows_valid > 32 && rows_valid <= 48)
    next = tile_slabs<TL, kS3, Ready, Claim>(lds, a_src, abase_r, bsrc_r, none_r, bsrc, lds_st, lrow, K,
                               rows_valid, head, ready);
  else if (kNa && (BM == 64 ? rows_valid <= 32 : rows_valid > 80 && rows_valid <= 96))
    next = tile_slabs<TL, kNw, Ready, Claim>(lds, a_src, abase_r, bsrc_r, none_r, bsrc, lds_st, lrow, K,
                               rows_valid, head, ready);
  else if (kSk && rows_valid <= 32)
    next = tile_slabs<TL, kS2, Ready, Claim>(lds, a_src, abase_r, bsrc_r, none_r, bsrc, lds_st, lrow, K,
                               rows_valid, head, ready);
  else if (rows_valid >= BM)
    next = tile_slabs<TL, kFull, Ready, Claim>(lds, a_src, abase_r, bsrc_r, none_r, bsrc, lds_st, lrow, K,
                                 rows_valid, head, ready);
  else
    next = tile_slabs<TL, kWide, Ready, Claim>(lds, a_src, abase_r, bsrc_r, none_r, bsrc, lds_st, lrow, K,
                                 rows_valid, head, ready);

  // Epilogue: the [BM][BN] tile in LDS is stored as whole-row float4s;
  // gate/up tiles store silu(W1 x) * (W3 x) of each 64-row group's two halves.
  constexpr int NC = GATED ? TL::BN / 2 : TL::BN;  // output columns of the tile
  constexpr int CP = TL::CPITCH;
  const float *Cs = lds;
  __syncthreads();
  constexpr int NC4 = NC / 4;
  for (int f = tid; f < BM * NC4; f += kThreads) {
    const int row = f / NC4, c4 = (f % NC4) * 4;
    if (row < rows_valid) {
      f32x4 v;
      if (GATED) {
        const float *g = Cs + row * CP + (c4 >> 5) * 64 + (c4 & 31);
        const f32x4 w1 = ld4(g), w3 = ld4(g + 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = silu(w1[j]) * w3[j];
      } else {
        v = ld4(Cs + row * CP + c4);
      }
      out.store((uint32_t)(((size_t)(row0 + row) * ldo + col0 + c4) * sizeof(float)), v);
    }
  }
  __syncthreads();  // Cs aliases the slab buffers of the next tile
  return next;
}

}  // namespace moe
