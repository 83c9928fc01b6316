// HIP kernels of the MI355X (gfx950) sparse-MoE block.
//
// Two launches per forward:
//   1. router -- gate GEMM as fp32 FMA chains (bit-exact with the reference's
//      attn_matmul_tiled_kernel, layer.cu:9-141), sigmoid with a double exp,
//      top-4 (layer.cu:439-499), per-token-block expert histogram and in-block
//      ranks; the last token block scans the histograms and writes the expert
//      kernel's task plan.  router_decode_kernel serves T <= 256 (expert-split
//      blocks, whole rows staged in LDS), router_kernel larger T (64-token
//      blocks) and routing from given logits.
//   2. expert kernel -- persistent, gate/up projection with the SwiGLU
//      epilogue (layer.cu:773-972), down projection (layer.cu:974-1126) and
//      the weighted top-4 combine with the residual add (layer.cu:695-721,
//      1860-1880).  T > 48: expert_mfma_kernel, MFMA 32x32x2 f32 tiles with
//      slots assigned by the router up to 1024 tokens, by a dispatch phase
//      above (both replace moe_scatter_kernel, layer.cu:501-542, without
//      copying x), one dynamic task queue, the combine inside the down
//      tiles; 64-row tiles up to 831 tokens, 128-row tiles above.  T <= 48:
//      expert_ring_kernel, weight streaming through MFMA 16x16x4 f32 with
//      round-robin tasks and slots assigned by the router -- or, for a fused
//      forward of at most 8 tokens, planned by each of its own blocks from
//      bounds of the scores that the router writes instead of the logits (a
//      slot for every expert the bounds leave possible: a token's exact
//      top-4, and one or two more when two scores nearly tie at the 4th
//      place), while 8 of its blocks compute the logits as chain jobs for
//      the weights, the rank order and the published routing.
//
// Phase dependencies are counters in the control block.  A task only waits
// on tasks with a smaller index and every block runs its tasks in increasing
// order, so the smallest unfinished task is always running and every wait
// ends; each wait is still bounded and reports MOE_ERR_DEVICE_TIMEOUT instead
// of spinning forever.
#include <type_traits>

#include "gpu_common.h"
#include "mfma_tile.h"

namespace moe {

// ---------------------------------------------------------------------------
// Router
// ---------------------------------------------------------------------------

// Weight-streaming plan: the expert kernel's intermediate rows and expert
// outputs start every launch as this value, and their readers reload a value
// until it has been replaced, so a value is its own completion signal.  It is
// a signalling NaN: arithmetic never produces one (an operation on a NaN
// returns a quiet NaN), and every value of those rows is computed.
constexpr uint32_t kUnwritten = 0x7FBADA55u;
// idx / pos of a token whose routing the streaming kernel has not published yet
constexpr int kRouteUnset = -2;

// Fill the slot rows of the intermediate and expert-output buffers (4T, or
// kSpecSlots * T for a deferred routing) with kUnwritten, shared by nthr
// threads in each of nblk blocks (this thread: thread thr of block blk).  The
// kernel boundary orders these stores before every store and load of the
// expert kernel.
__device__ void fill_unwritten(const RouterArgs &a, int blk, int nblk, int thr, int nthr) {
  if (a.tile_rows != 0) return;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const f32x4 v = __builtin_bit_cast(f32x4, u32x4{kUnwritten, kUnwritten, kUnwritten, kUnwritten});
  // a deferred routing plans up to kSpecSlots slots per token
  const size_t rows = (size_t)a.T * (a.defer == 2 ? kSpecSlots : kTopK);
  const size_t ni = rows * (size_t)a.inter / 4, ns = rows * (size_t)a.H / 4;
  const size_t stride = (size_t)nblk * nthr;
  for (size_t i = (size_t)blk * nthr + thr; i < ni + ns; i += stride) {
    if (i < ni) st4(a.s.inter + 4 * i, v);
    else st4(a.s.sout + 4 * (i - ni), v);
  }
}

// Exactly layer.cu:434: exp in double, add and IEEE divide in float.
__device__ __forceinline__ float ref_sigmoid(float x) {
#pragma clang fp contract(off)
  const float e = (float)exp(-(double)x);
  return 1.0f / (1.0f + e);
}


// Four rows per block (their loads in flight together): out = rmsnorm(h)
// (large batches; small ones normalise inside router_decode_kernel).
constexpr int kNormRowsPerBlock = 4;

__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float *h, const float *w,
                                                               float *out, int T, int H) {
  constexpr int NR = kNormRowsPerBlock;
  __shared__ float s_grp[NR * kNormGroups], s_tot[NR];
  const int r0 = blockIdx.x * NR;
  const float *src[NR];
  float *dst[NR];
#pragma unroll
  for (int m = 0; m < NR; ++m) {
    src[m] = h + (size_t)min(r0 + m, T - 1) * H;
    dst[m] = out + (size_t)min(r0 + m, T - 1) * H;
  }
  norm_rows<NR>(src, dst, min(NR, T - r0), w, H, s_grp, s_tot);
}


// acc = FMA chain over k = 0 .. K-1 of x[k] * g[k] (LDS rows xp, gp), k
// ascending (layer.cu:109-127).  The chain is latency-bound, so the operands
// of the next 16 k are read while this 16 k's FMAs run; the loop body has no
// branch so both operand sets stay in fixed registers.  K % 32 == 0.
__device__ __forceinline__ float chain_dot(const float *gp, const float *xp, int K) {
#pragma clang fp contract(off)
  constexpr int U = 4;  // float4 per half step: 16 k
  f32x4 ga[U], xa[U], gb[U], xb[U];
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    ga[u] = ld4(gp + 4 * u);
    xa[u] = ld4(xp + 4 * u);
  }
  int k = 0;
  for (; k < K - 8 * U; k += 8 * U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      gb[u] = ld4(gp + k + 4 * (U + u));
      xb[u] = ld4(xp + k + 4 * (U + u));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc = __builtin_fmaf(xa[u].x, ga[u].x, acc);
      acc = __builtin_fmaf(xa[u].y, ga[u].y, acc);
      acc = __builtin_fmaf(xa[u].z, ga[u].z, acc);
      acc = __builtin_fmaf(xa[u].w, ga[u].w, acc);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ga[u] = ld4(gp + k + 8 * U + 4 * u);
      xa[u] = ld4(xp + k + 8 * U + 4 * u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc = __builtin_fmaf(xb[u].x, gb[u].x, acc);
      acc = __builtin_fmaf(xb[u].y, gb[u].y, acc);
      acc = __builtin_fmaf(xb[u].z, gb[u].z, acc);
      acc = __builtin_fmaf(xb[u].w, gb[u].w, acc);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    gb[u] = ld4(gp + k + 4 * (U + u));
    xb[u] = ld4(xp + k + 4 * (U + u));
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    acc = __builtin_fmaf(xa[u].x, ga[u].x, acc);
    acc = __builtin_fmaf(xa[u].y, ga[u].y, acc);
    acc = __builtin_fmaf(xa[u].z, ga[u].z, acc);
    acc = __builtin_fmaf(xa[u].w, ga[u].w, acc);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    acc = __builtin_fmaf(xb[u].x, gb[u].x, acc);
    acc = __builtin_fmaf(xb[u].y, gb[u].y, acc);
    acc = __builtin_fmaf(xb[u].z, gb[u].z, acc);
    acc = __builtin_fmaf(xb[u].w, gb[u].w, acc);
  }
  return acc;
}

// Planning, by the last token block of the router (256 threads): expert
// counts and offsets (the exclusive scan of layer.cu:737-760), each token
// block's base within every expert, the units (tiles, or one per active
// expert for the streaming plan), the expert kernel's task plan, and for the
// streaming plan each slot's token (slot = block base + in-block rank).
// The planning block reads each thread's token-block counts in batches of
// kPlanRegBlocks (every load of a batch in flight at once); up to one batch
// per thread they stay in registers, and up to kPlanLdsBlocks token blocks the
// block bases are also kept in LDS for the slot assignment.
constexpr int kPlanRegBlocks = 8;
constexpr int kPlanLdsBlocks = 32;
constexpr int kPlanSlotsPerThread = kRouterSlotTokens * kTopK / kThreads;

struct PlanShared {
  int part[8][kExperts];
  int off[kExperts + 1];
  int cnt[kExperts];
  int units;
  int base[kPlanLdsBlocks][kExperts];
};

// A planning block that routed the only token block itself passes its
// routing from LDS instead of reading it back from memory.
struct PlanLocal {
  const int *cnt;              // [nb][kExperts] tokens (or possible pairs) per block and expert
  const int (*ids)[kTopK];     // [token][k] expert ids (-1: none)
  const int (*rank)[kTopK];    // [token][k] in-block ranks
};

// Exclusive prefix sum over lanes 0..31 of a wave (lanes >= 32 idle).
__device__ __forceinline__ int lane_scan32(int v, int lane, int *total) {
  int inc = v;
#pragma unroll
  for (int d = 1; d < 32; d <<= 1) {
    const int u = __shfl_up(inc, d, 32);
    if (lane >= d) inc += u;
  }
  *total = __shfl(inc, 31, 32);
  return inc - v;
}

// Units whose gate/up tiles run as two half-width tiles (the launch's last
// units, so its last gate/up tiles end sooner and the down tiles after them
// wait less): in the 64-row plan up to kGateUpTailTokens tokens
// kGateUpTailUnits of them, every unit at 37-52 tokens (against 8 of them,
// two boxes: T=40 265.9 -> 260.7 and 264.5 -> 261.0 us, T=48 264.3 -> 261.1
// and 262.9 -> 261.2; T=33 1.6 us and T=56 1 us slower); in the 128-row
// plan up to kGateUpTailTokens128 tokens kGateUpTailUnits of them.
__device__ __forceinline__ int gate_up_tail(int tile_rows, int T, int units) {
  if (tile_rows == 64 && T <= kGateUpTailTokens)
    return min(units, T > 36 && T <= 52 ? kExperts : kGateUpTailUnits);
  if (tile_rows == 128 && T <= kGateUpTailTokens128) return min(units, kGateUpTailUnits);
  return 0;
}

template <int RT>
__device__ void router_plan(const RouterArgs &a, int nb, int T, PlanShared &ps,
                            PlanLocal loc = PlanLocal{nullptr, nullptr, nullptr}) {
  Ctrl *ctrl = a.s.ctrl;
  const int tid = threadIdx.x;
  const int e = tid & (kExperts - 1);
  const int part = tid >> 5;  // 8 parts x 32 experts
  const int per = (nb + 7) / 8;
  const int lo = part * per;
  const int hi = min(nb, lo + per);
  // one batch per thread: the counts stay in registers for the block bases
  const bool in_regs = per <= kPlanRegBlocks;
  const bool bases_lds = nb <= kPlanLdsBlocks;
  int bv[kPlanRegBlocks];
  {
    int sum = 0;
    for (int b0 = lo; b0 < hi; b0 += kPlanRegBlocks) {
#pragma unroll
      for (int i = 0; i < kPlanRegBlocks; ++i)
        bv[i] = b0 + i < hi ? (loc.cnt ? loc.cnt[(b0 + i) * kExperts + e]
                                       : a.s.blk[(b0 + i) * kExperts + e])
                            : 0;
#pragma unroll
      for (int i = 0; i < kPlanRegBlocks; ++i) sum += bv[i];
    }
    ps.part[part][e] = sum;
  }
  __syncthreads();
  if (tid < kExperts) {
    const int lane = tid;
    int run = 0;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int v = ps.part[p][lane];
      ps.part[p][lane] = run;
      run += v;
    }
    const int cnt = run;
    int maxcnt = cnt;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) maxcnt = max(maxcnt, __shfl_xor(maxcnt, o, 32));
    int total = 0, utotal = 0;
    const int off = lane_scan32(cnt, lane, &total);
    const int tr = a.tile_rows;
    const int units_e = tr > 0 ? (cnt + tr - 1) / tr : (cnt > 0 ? 1 : 0);
    const int uoff = lane_scan32(units_e, lane, &utotal);
    const unsigned long long act = __ballot(cnt > 0);
    const int nact = __popcll(act);
    const int aidx = __popcll(act & ((1ull << lane) - 1ull));
    ps.cnt[lane] = cnt;
    ps.off[lane] = off;
    ctrl->counts[lane] = cnt;
    ctrl->offsets[lane] = off;
    ctrl->unit_off[lane] = uoff;
    if (cnt > 0) ctrl->active[aidx] = lane;
    if (lane >= nact) ctrl->active[lane] = -1;
    if (lane == 0) {
      ps.off[kExperts] = total;
      ctrl->offsets[kExperts] = total;
      ctrl->unit_off[kExperts] = utotal;
      ctrl->n_active = nact;
      const int units = utotal;
      // a.bn: columns of an MFMA tile, or weight rows of a streaming task.
      // A streaming plan whose largest expert needs more than the two token
      // passes of a 64-row task takes 32-row tasks with four passes, so
      // experts of up to 64 tokens read each weight row once.
      int rows = a.bn;
      if (tr == 0 && rows == kStreamRows * kRingWideGroups && maxcnt > kRingMaxPasses * kRingTokens)
        rows = kStreamRows * kRingDenseGroups;
      const int p1u = a.inter / (rows / 2);
      const int p2u = a.H / rows;
      ctrl->stream_rows = tr > 0 ? 0 : rows;
      ctrl->max_count = maxcnt;
      ctrl->p1_per_unit = p1u;
      ctrl->p2_per_unit = p2u;
      // The streaming plan (small T) gets its slots from this block below, so
      // its expert kernel has no dispatch tasks to wait for.
      const int ndisp = tr > 0 ? nb : 0;
      ctrl->n_rblocks = ndisp;
      ctrl->rtokens = RT;
      // MFMA plans: the last tail units split each down tile in two halves;
      // streaming plan with 64-row tasks of up to 16 tokens: the last units'
      // down rows run as 16-row tasks (4 per 64-row task)
      const int tail = tr > 0 ? min(units, a.tail_units)
                       : (rows == kStreamRows * kRingWideGroups && maxcnt <= kRingTokens
                              ? min(units, kRingTailUnits) : 0);
      const int tail_mult = tr > 0 ? 2 : kRingWideGroups;
      ctrl->tail_units = tail;
      // small batches (the 64-row plan's units of few rows, memory-bound
      // tiles; the 128-row plan's long tiles up to 1024 tokens): the last
      // units' gate/up tiles run at half width too, so the last gate/up tiles
      // end sooner and the down tiles after them wait less
      const int gtail = gate_up_tail(tr, T, units);
      ctrl->gu_tail = gtail;
      ctrl->n_p1 = (units + gtail) * p1u;
      ctrl->n_p2 = (units - tail + tail * tail_mult) * p2u;
      // the MFMA plans combine inside their down tiles; the streaming kernel
      // runs one combine task per token
      ctrl->n_comb = tr > 0 ? 0 : T;
      ctrl->n_total = ndisp + ctrl->n_p1 + ctrl->n_p2 + ctrl->n_comb;
      ctrl->num_tokens = T;
      ctrl->tile_rows = tr;
      ctrl->head = 0;
      ctrl->assign_done = 0;
      ctrl->deferred = 0;
      ps.units = units;
    }
  }
  __syncthreads();
  {
    // block bases: offsets[e] + tokens of e in earlier token blocks
    int base = ps.off[e] + ps.part[part][e];
    for (int b0 = lo; b0 < hi; b0 += kPlanRegBlocks) {
      if (!in_regs) {  // several batches: read this one's counts again
#pragma unroll
        for (int i = 0; i < kPlanRegBlocks; ++i)
          bv[i] = b0 + i < hi ? a.s.blk[(b0 + i) * kExperts + e] : 0;
      }
#pragma unroll
      for (int i = 0; i < kPlanRegBlocks; ++i) {
        if (b0 + i < hi) {
          a.s.blk[(b0 + i) * kExperts + e] = base;
          if (bases_lds) ps.base[b0 + i][e] = base;
          base += bv[i];
        }
      }
    }
  }
  const int units = min(ps.units, a.max_units);
  for (int i = tid; i < dep_words(a.inter) * units; i += kThreads) a.s.dep[i] = 0;
  // The streaming plan takes its slots from here, and so do the MFMA plans of
  // small batches (a few slots per thread): their gate/up tiles then start
  // without waiting for the expert kernel's dispatch tasks (T=256: ~7 us).
  const bool router_slots = a.tile_rows == 0 || T <= kRouterSlotTokens;
  if (router_slots) {
    __syncthreads();  // the block bases above are read back below
    // slot = token block base + in-block rank (stable by token), as the
    // dispatch tasks of the tiled plans compute it
    const int n = T * kTopK;
    if (bases_lds && n <= kThreads * kPlanSlotsPerThread) {
      // every thread's (expert, rank) pairs loaded at once, bases from LDS
      int id[kPlanSlotsPerThread], rk[kPlanSlotsPerThread];
#pragma unroll
      for (int i = 0; i < kPlanSlotsPerThread; ++i) {
        const int f = tid + i * kThreads;
        if (loc.ids) {
          id[i] = f < n ? loc.ids[f / kTopK][f % kTopK] : -1;
          rk[i] = f < n ? loc.rank[f / kTopK][f % kTopK] : 0;
        } else {
          id[i] = f < n ? a.s.idx[f] : -1;
          rk[i] = f < n ? a.s.pos[f] : 0;
        }
      }
#pragma unroll
      for (int i = 0; i < kPlanSlotsPerThread; ++i) {
        const int f = tid + i * kThreads;
        if (f < n) {
          const int t = f / kTopK, ee = id[i];
          int slot = -1;
          if (ee >= 0 && ee < kExperts) {
            slot = ps.base[t / RT][ee] + rk[i];
            if (slot >= 0 && slot < n) {
              a.s.slot_token[slot] = t;
            } else {  // inconsistent plan: flag it, never write out of range
              slot = -1;
              __hip_atomic_store(&ctrl->err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
          }
          a.s.pos[f] = slot;
        }
      }
    } else {
      for (int f = tid; f < n; f += kThreads) {
        const int t = f / kTopK;
        const int ee = a.s.idx[f];
        int slot = -1;
        if (ee >= 0 && ee < kExperts) {
          slot = a.s.blk[(t / RT) * kExperts + ee] + a.s.pos[f];
          if (slot >= 0 && slot < n) {
            a.s.slot_token[slot] = t;
          } else {  // inconsistent plan: flag it, never write out of range
            slot = -1;
            __hip_atomic_store(&ctrl->err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
        a.s.pos[f] = slot;
      }
    }
  }
  if (tid == 0) {
    ctrl->router_done = 0;  // every token block has counted in
    ctrl->slots_assigned = router_slots ? 1 : 0;
  }
}

// Router.  A block computes the gate logits of RT tokens x (32/ES) experts as
// fp32 FMA chains over k ascending (the reference's per-output order,
// layer.cu:109-127), staging x and gate through LDS in KC-wide k chunks with
// the next chunk's global loads in flight during the current chunk's FMAs.
// ES > 1 splits the experts over ES blocks so small T (decode) spreads the
// gate over more CUs; the last of a token block's ES blocks then finishes it.
// Finishing a token block: sigmoid with a double exp, score = p + bias,
// top-4 insertion (layer.cu:439-499), weights, in-block ranks by 64-lane
// ballots and per-block expert counts.  The last token block to finish scans
// the counts and writes the expert kernel's plan.
template <int RT, int ES, int KC> struct RouterCfg {
  static constexpr int EPB = kExperts / ES;          // experts per block
  static constexpr int NGRP = kThreads / EPB;        // lane groups
  static constexpr int TPL = RT >= NGRP ? RT / NGRP : 1;  // tokens per lane
  static constexpr int PITCH = KC + 4;
  static constexpr int X_F4 = RT * KC / 4, G_F4 = EPB * KC / 4;
  static constexpr int X_PER = (X_F4 + kThreads - 1) / kThreads;
  static constexpr int G_PER = (G_F4 + kThreads - 1) / kThreads;
  static_assert(RT <= 64, "ballot ranks need <= 64 tokens per block");
  static_assert(KC % 4 == 0 && kThreads % (KC / 4) == 0, "chunk split");
};

// One LDS chunk of TPL interleaved FMA chains (tokens j of rows xp + j *
// PITCH against the gate row gp), k ascending, as chain_dot: the operands of
// the next 8 k are read while this 8 k's FMAs run.  KC % 16 == 0.
template <int TPL, int KC, int PITCH>
__device__ __forceinline__ void chain_chunk(const float *gp, const float *xp, float (&acc)[TPL]) {
#pragma clang fp contract(off)
  static_assert(KC % 16 == 0 && KC >= 16, "chunk of whole 16-k steps");
  constexpr int U = 2;  // float4 per half step: 8 k
  f32x4 ga[U], gb[U], xa[TPL][U], xb[TPL][U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    ga[u] = ld4(gp + 4 * u);
#pragma unroll
    for (int j = 0; j < TPL; ++j) xa[j][u] = ld4(xp + j * PITCH + 4 * u);
  }
#define MOE_CHUNK_FMAS(G, X)                                   \
  _Pragma("unroll") for (int u = 0; u < U; ++u)                \
  _Pragma("unroll") for (int j = 0; j < TPL; ++j) {            \
      acc[j] = __builtin_fmaf(X[j][u].x, G[u].x, acc[j]);      \
      acc[j] = __builtin_fmaf(X[j][u].y, G[u].y, acc[j]);      \
      acc[j] = __builtin_fmaf(X[j][u].z, G[u].z, acc[j]);      \
      acc[j] = __builtin_fmaf(X[j][u].w, G[u].w, acc[j]);      \
    }
#pragma unroll
  for (int k = 0; k < KC - 16; k += 16) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      gb[u] = ld4(gp + k + 8 + 4 * u);
#pragma unroll
      for (int j = 0; j < TPL; ++j) xb[j][u] = ld4(xp + j * PITCH + k + 8 + 4 * u);
    }
    MOE_CHUNK_FMAS(ga, xa)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ga[u] = ld4(gp + k + 16 + 4 * u);
#pragma unroll
      for (int j = 0; j < TPL; ++j) xa[j][u] = ld4(xp + j * PITCH + k + 16 + 4 * u);
    }
    MOE_CHUNK_FMAS(gb, xb)
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    gb[u] = ld4(gp + KC - 8 + 4 * u);
#pragma unroll
    for (int j = 0; j < TPL; ++j) xb[j][u] = ld4(xp + j * PITCH + KC - 8 + 4 * u);
  }
  MOE_CHUNK_FMAS(ga, xa)
  MOE_CHUNK_FMAS(gb, xb)
#undef MOE_CHUNK_FMAS
}

// At most a few blocks per CU run (T/64 blocks), so the kernel is compiled for
// instruction-level parallelism (all of a chunk's LDS reads in flight), not
// occupancy.
template <bool FROM_LOGITS, int RT, int ES, int KC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
void router_kernel(RouterArgs a) {
#pragma clang fp contract(off)
  using C = RouterCfg<RT, ES, KC>;
  constexpr int EPB = C::EPB, TPL = C::TPL, PITCH = C::PITCH;
  __shared__ float xs[RT * PITCH];
  __shared__ float gs[EPB * PITCH];
  __shared__ float s_score[RT][kExperts + 1];
  __shared__ float s_prob[RT][kExperts + 1];
  __shared__ int s_cnt[kExperts];
  __shared__ float s_bias[kExperts];
  __shared__ PlanShared ps;
  __shared__ int s_flag;

  const int tid = threadIdx.x;
  const int tb = blockIdx.x / ES, es = blockIdx.x % ES;
  const int t0 = tb * RT, e0 = es * EPB;
  const int T = a.T, H = a.H;
  const int el = tid % EPB, grp = tid / EPB;
  const bool chain_lane = grp * TPL < RT;
  Ctrl *ctrl = a.s.ctrl;
  if (tid < kExperts) s_bias[tid] = a.w.bias ? a.w.bias[tid] : 0.0f;  // the score bias
  fill_unwritten(a, blockIdx.x, gridDim.x, tid, kThreads);

  if (!FROM_LOGITS) {
    // staging map: thread -> (row, float4 column) of a KC-wide chunk; the
    // X_PER (G_PER) passes cover the RT (EPB) rows exactly
    constexpr int KV = KC / 4, RPP = kThreads / KV;
    static_assert(C::X_PER * RPP == RT && C::G_PER * RPP == EPB, "exact staging passes");
    const int srow = tid / KV, sc4 = (tid % KV) * 4;
    const float *xrow[C::X_PER];
#pragma unroll
    for (int i = 0; i < C::X_PER; ++i) {
      int tok = t0 + srow + i * RPP;
      tok = tok < T ? tok : T - 1;  // rows past T: a copy, never stored
      xrow[i] = a.x + (size_t)tok * H + sc4;
    }
    const float *grow = a.w.gate + (size_t)(e0 + srow) * H + sc4;
    f32x4 px[C::X_PER], pg[C::G_PER];
    float acc[TPL];
#pragma unroll
    for (int j = 0; j < TPL; ++j) acc[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < C::X_PER; ++i) px[i] = ld4(xrow[i]);
#pragma unroll
    for (int i = 0; i < C::G_PER; ++i)
      pg[i] = ld4(grow + (size_t)i * RPP * H);
    for (int k0 = 0; k0 < H; k0 += KC) {
      __syncthreads();  // the previous chunk's readers are done
#pragma unroll
      for (int i = 0; i < C::X_PER; ++i)
        st4(xs + (srow + i * RPP) * PITCH + sc4, px[i]);
#pragma unroll
      for (int i = 0; i < C::G_PER; ++i)
        st4(gs + (srow + i * RPP) * PITCH + sc4, pg[i]);
      __syncthreads();
      if (k0 + KC < H) {  // next chunk in flight during this chunk's FMAs
#pragma unroll
        for (int i = 0; i < C::X_PER; ++i)
          px[i] = ld4(xrow[i] + k0 + KC);
#pragma unroll
        for (int i = 0; i < C::G_PER; ++i)
          pg[i] = ld4(grow + (size_t)i * RPP * H + k0 + KC);
      }
      if (chain_lane) chain_chunk<TPL, KC, PITCH>(gs + el * PITCH, xs + grp * TPL * PITCH, acc);
    }
    if (chain_lane) {
#pragma unroll
      for (int j = 0; j < TPL; ++j) {
        const int tl = grp * TPL + j;
        if (t0 + tl < T) st_agent(&a.s.logits[(size_t)(t0 + tl) * kExperts + e0 + el], acc[j]);
        if (ES == 1) s_prob[tl][el] = acc[j];  // the block has every expert: logits stay in LDS
      }
    }
  }

  // ---- the last of the token block's ES blocks finishes it ---------------
  if (ES > 1 && !FROM_LOGITS) {
    __builtin_amdgcn_s_waitcnt(0);  // this block's logits are stored
    __syncthreads();
    if (tid == 0) {
      s_flag = fetch_add(&a.s.tb_done[tb], 1) == ES - 1;
      if (s_flag) {
        a.s.tb_done[tb] = 0;  // all ES blocks counted in: reset
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      }
    }
    __syncthreads();
    if (!s_flag) return;
  } else if (!FROM_LOGITS) {
    __syncthreads();  // logits written by this block are read back below
  }
  if (FROM_LOGITS) __syncthreads();  // s_bias written
  const float *lsrc = FROM_LOGITS ? a.logits_in : a.s.logits;
  // every logit of the thread is loaded before any is used (a loop that
  // waited for each load made the finishing ~8 global round trips long)
  constexpr int LPT = RT * kExperts / kThreads;  // logits per thread
  static_assert(RT * kExperts % kThreads == 0, "whole logit passes");
  float lv[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int f = tid + i * kThreads;
    const int tl = f / kExperts, e = f % kExperts;
    const int tok = t0 + tl;
    float l = 0.0f;
    if (tok < T) l = (!FROM_LOGITS && ES == 1) ? s_prob[tl][e] : lsrc[(size_t)tok * kExperts + e];
    lv[i] = l;
  }
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int f = tid + i * kThreads;
    const int tl = f / kExperts, e = f % kExperts;
    const int tok = t0 + tl;
    if (FROM_LOGITS && tok < T) a.s.logits[(size_t)tok * kExperts + e] = lv[i];
    const float p = ref_sigmoid(lv[i]);
    s_prob[tl][e] = p;
    s_score[tl][e] = p + s_bias[e];  // layer.cu:462
  }
  __syncthreads();

  if (tid < 64) {  // wave 0: lane = token of the block
    const int tl = tid;
    const int tok = t0 + tl;
    const bool valid = tl < RT && tok < T;
    float ms[kTopK], mp[kTopK];
    int mi[kTopK];
#pragma unroll
    for (int i = 0; i < kTopK; ++i) {
      ms[i] = -1e30f;
      mp[i] = 0.0f;
      mi[i] = -1;
    }
    if (valid) {
      // Insertion with strict '>' (layer.cu:465-476): rank order is score
      // descending, lower expert index first among equal scores.  The list
      // stays sorted (ms[0] >= ... >= ms[3], never NaN), so score > ms[i]
      // implies score > ms[i+1], and the nested insertion is the selects
      // below; all 32 scores and probabilities are read first, so no LDS
      // read waits on a branch.
      float sv[kExperts], pv[kExperts];
#pragma unroll
      for (int ee = 0; ee < kExperts; ++ee) {
        sv[ee] = s_score[tl][ee];
        pv[ee] = s_prob[tl][ee];
      }
#pragma unroll
      for (int ee = 0; ee < kExperts; ++ee) {
        const float score = sv[ee], prob = pv[ee];
        const bool c0 = score > ms[0], c1 = score > ms[1], c2 = score > ms[2], c3 = score > ms[3];
        ms[3] = c2 ? ms[2] : (c3 ? score : ms[3]);
        mp[3] = c2 ? mp[2] : (c3 ? prob : mp[3]);
        mi[3] = c2 ? mi[2] : (c3 ? ee : mi[3]);
        ms[2] = c1 ? ms[1] : (c2 ? score : ms[2]);
        mp[2] = c1 ? mp[1] : (c2 ? prob : mp[2]);
        mi[2] = c1 ? mi[1] : (c2 ? ee : mi[2]);
        ms[1] = c0 ? ms[0] : (c1 ? score : ms[1]);
        mp[1] = c0 ? mp[0] : (c1 ? prob : mp[1]);
        mi[1] = c0 ? mi[0] : (c1 ? ee : mi[1]);
        ms[0] = c0 ? score : ms[0];
        mp[0] = c0 ? prob : mp[0];
        mi[0] = c0 ? ee : mi[0];
      }
      float sum = 0.0f;  // layer.cu:480-482, rank order
#pragma unroll
      for (int i = 0; i < kTopK; ++i) sum += mp[i];
      const float scale = (sum > 1e-6f) ? (1.0f / sum) : 1.0f;  // layer.cu:484
#pragma unroll
      for (int i = 0; i < kTopK; ++i) {
        st_agent(&a.s.idx[(size_t)tok * kTopK + i], mi[i]);  // read by the planning block
        a.s.wts[(size_t)tok * kTopK + i] = mp[i] * scale * 1.0f;  // :489
      }
    }
    // In-block rank of this token among the block's tokens that chose ee:
    // a 64-lane ballot per expert (deterministic, no atomics).
    int rank[kTopK] = {-1, -1, -1, -1};
    const unsigned long long below = (1ull << tl) - 1ull;
    for (int ee = 0; ee < kExperts; ++ee) {
      const bool sel = valid & ((mi[0] == ee) | (mi[1] == ee) | (mi[2] == ee) | (mi[3] == ee));
      const unsigned long long m = __ballot(sel);
      const int r = __popcll(m & below);
#pragma unroll
      for (int i = 0; i < kTopK; ++i) rank[i] = mi[i] == ee ? r : rank[i];
      if (tl == 0) s_cnt[ee] = __popcll(m);
    }
    if (valid) {
#pragma unroll
      for (int i = 0; i < kTopK; ++i) st_agent(&a.s.pos[(size_t)tok * kTopK + i], rank[i]);
    }
  }
  __syncthreads();
  if (tid < kExperts) st_agent(&a.s.blk[tb * kExperts + tid], s_cnt[tid]);

  // ---- last-block election: the token block that finishes last plans -----
  const int nb = gridDim.x / ES;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    // a single token block is the last one by construction
    s_flag = nb == 1 || (fetch_add(&ctrl->router_done, 1) == nb - 1);
    if (s_flag) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (!s_flag) return;

  router_plan<RT>(a, nb, T, ps);
}

// Decode router shape: 8-token blocks, 4 experts per block, 8 blocks per token block.
constexpr int kDecRT = 8, kDecEPB = 4, kDecES = kExperts / kDecEPB;
static_assert(kDecRT == kDeferTokens && kDecES == kChainJobs, "a chain job is one router block's chains");
// Blocks of a deferred decode routing's router that only fill the streaming
// kernel's rows (kSpecSlots * T rows of I + H floats: 983 KB at T=8).
constexpr int kDeferFillBlocks = 56;
// Tokens per router block of a deferred decode routing (more blocks, each
// staging fewer token rows, 64 threads per pair in its bound sums; from 8
// per block, 4 took T=8 183.2 -> 182.0 us, 2 then T=4 117.1 -> 116.4, T=6
// 159.6 -> 158.7, T=8 182.4 -> 181.6, and 1 a further 0.3-0.4 us at T=2-8).
constexpr int kDeferBlockTokens = 1;
// Tokens per block of a routing from score bounds for the MFMA plans: up to
// 32 tokens four blocks per token block of 8 and expert slice, up to 64 two
// (the last of a token block's blocks plans it).  Same box against one:
// T=11 231.4 -> 229.1 us, T=21 245.2 -> 243.7, T=64 264.7 -> 263.9 with two;
// four then T=11 228.7 -> 227.7, T=16 235.2 -> 234.0 (another box: T=11
// 229.3 -> 228.7, T=16 234.7 -> 234.1, T=24-48 equal; 1 us slower at 64,
// and eight 6 us slower there); at 128 and 256 two were about 1 us slower,
// so larger batches keep one.
constexpr int kBoundSplitTokens = 64, kBoundSplit4Tokens = 32;
__host__ __device__ inline int router_block_tokens(int defer, int T) {
  if (defer == 2) return T > kDeferBlockTokens ? kDeferBlockTokens : kDecRT;
  if (defer == 3) {
    if (T > 2 && T <= kBoundSplit4Tokens) return 2;
    if (T > 4 && T <= kBoundSplitTokens) return 4;
  }
  return kDecRT;
}
constexpr int kChainClaimBlocks = 16;  // streaming-kernel blocks that try for a chain job as they start

// Bounds of the score fl(ref_sigmoid(l) + bias) of the float logit l that an
// FMA chain over H products computes, from s and m, float sums of the
// products and of their magnitudes with at most n roundings on any path.
// Each of the chain's H roundings perturbs by at most u = 2^-24 relatively,
// so |l - sum| <= gamma_H * M with gamma_k = k u / (1 - k u) and M the exact
// sum of magnitudes (Higham, Accuracy and Stability of Numerical Algorithms,
// 3.1; plus 2^-150 per rounding below the normal range); likewise |s - sum| <=
// gamma_n * M, and M <= m / (1 - gamma_n).  ref_sigmoid is within 3
// roundings (exp to float, the add, the divide) of the real sigmoid, which is
// monotone: its value lies within a relative 2^-20 of the sigmoid's at the
// interval's ends.  fl(p + bias) is monotone in p.  False (bounds infinite)
// where this does not hold: non-finite sums or bias, sums large enough for a
// partial sum to overflow, and logits below -80, whose probability may be
// subnormal.
__device__ __forceinline__ bool score_bounds(float s, float m, int H, int n, float bias, float *lo,
                                             float *hi) {
#pragma clang fp contract(off)
  const double u = 0x1p-24, gh = H * u / (1.0 - H * u), gn = n * u / (1.0 - n * u);
  const double r = (gh + gn) / (1.0 - gn) * 1.0001 * (double)m + 1e-37;
  const double sd = s;
  const bool ok = __builtin_isfinite(s) && __builtin_isfinite(m) && m < 1e37f &&
                  __builtin_isfinite(bias) && sd - r > -80.0;
  if (!ok) {
    *lo = -__builtin_inff();
    *hi = __builtin_inff();
    return false;
  }
  const double pl = 1.0 / (1.0 + exp(-(sd - r))), ph = 1.0 / (1.0 + exp(-(sd + r)));
  *lo = __double2float_rd(pl * (1.0 - 0x1p-20)) + bias;
  *hi = __double2float_ru(ph * (1.0 + 0x1p-20)) + bias;
  return true;
}

// One token block's routing (up to kDecRT tokens x 32 experts) in LDS.
struct RouteShared {
  float score[kDecRT][kExperts + 1];
  float prob[kDecRT][kExperts + 1];
  int sel[kDecRT][kExperts];   // rank in the token's top-4, or -1
  int ti[kDecRT][kTopK];       // expert ids in rank order (-1: rank left empty)
  float tp[kDecRT][kTopK];     // their probabilities
  float tw[kDecRT][kTopK];     // routing weights
  int rank[kDecRT][kTopK];     // in-block rank among the block's tokens choosing ti
  int cnt[kExperts];           // the block's tokens per expert
};

// Routing of nt <= kDecRT tokens from their logits, threads 0..255 as
// (token tid / 32, expert tid % 32), each passing the logit of its pair (l,
// read by the caller, which can issue that load early; ignored for tokens
// past nt); every thread of the block calls it (it holds barriers) and finds
// rs complete on return.
//  - probability 1/(1+(float)exp(-(double)l)) (layer.cu:434), score = p + bias
//    (bias in LDS, layer.cu:462);
//  - top-4 as a rank: e is kept iff fewer than 4 selectable experts have a
//    higher score or an equal score and a lower index, which is what the
//    strict-'>' insertion of layer.cu:465-476 keeps; the insertion only takes
//    a score above its -1e30 sentinel (layer.cu:452, 465), so NaN and scores
//    <= -1e30 are never selected and never outrank another expert; all 32
//    scores are read first and combined without branches (short-circuit
//    tests made each LDS read wait for the previous one);
//  - weights p * (1 / sum) * 1.0f, the sum in rank order (layer.cu:480-489);
//  - in-block ranks (tokens of the block before this one that chose the
//    same expert) and per-expert counts.
__device__ __forceinline__ void route_token_block(RouteShared &rs, int nt, const float *bias,
                                                  float logit) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x;
  const bool act = tid < kDecRT * kExperts;
  const int tl = (tid >> 5) & (kDecRT - 1), e = tid & (kExperts - 1);
  const bool tvalid = act && tl < nt;
  if (act) {
    const float l = tvalid ? logit : 0.0f;
    const float p = ref_sigmoid(l);
    rs.prob[tl][e] = p;
    rs.score[tl][e] = p + bias[e];
    if (e < kTopK) {  // rank slots no expert fills keep the reference's -1 / 0
      rs.ti[tl][e] = -1;
      rs.tp[tl][e] = 0.0f;
    }
  }
  __syncthreads();
  int sel = -1;
  if (act) {
    const float sc = rs.score[tl][e];
    int r = 0;
#pragma unroll
    for (int j0 = 0; j0 < kExperts; j0 += 8) {  // 8 scores in flight at a time
      float sv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) sv[j] = rs.score[tl][j0 + j];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sj = sv[j];
        r += (int)((sj > -1e30f) & ((sj > sc) | ((sj == sc) & (j0 + j < e))));
      }
    }
    if (tvalid && sc > -1e30f && r < kTopK) sel = r;
    rs.sel[tl][e] = sel;
    if (sel >= 0) {
      rs.ti[tl][sel] = e;
      rs.tp[tl][sel] = rs.prob[tl][e];
    }
  }
  __syncthreads();
  if (tid < nt) {
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kTopK; ++i) sum += rs.tp[tid][i];
    const float scale = (sum > 1e-6f) ? (1.0f / sum) : 1.0f;
#pragma unroll
    for (int i = 0; i < kTopK; ++i) rs.tw[tid][i] = rs.tp[tid][i] * scale * 1.0f;
  }
  if (act) {  // rows of tokens past nt hold -1
    int before = 0, all = 0;
#pragma unroll
    for (int t2 = 0; t2 < kDecRT; ++t2) {
      const int chose = rs.sel[t2][e] >= 0;
      before += chose & (t2 < tl);
      all += chose;
    }
    if (sel >= 0) rs.rank[tl][sel] = before;
    if (tl == 0) rs.cnt[e] = all;
  }
  __syncthreads();
}

// Expert-split router (T <= 256).  A token block is 8 tokens; its 32 experts are
// split over 8 blocks of 4, so 8x more CUs share the gate.  Each block copies
// its 4 gate rows and the token rows whole into LDS with direct-to-LDS loads
// (no chunk loop) and runs one FMA chain per (token, expert) lane (the
// reference's order, layer.cu:109-127).  The last of a token block's blocks
// finishes it (route_token_block) and the last token block plans.  With
// defer 2 (one token block, weight-streaming plan) the blocks write score
// bounds in place of the chains and the expert kernel routes and plans in
// its own blocks; with defer 3 (MFMA plans of up to kBoundTokens tokens)
// they write the bounds, and every block of the expert kernel plans from
// them (bounds_local_plan) and its dispatch tasks compute the logits and
// route.
__host__ __device__ constexpr size_t router_decode_lds(int H) {
  return (size_t)(kDecEPB + kDecRT) * (size_t)(H + 4) * sizeof(float);
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
void router_decode_kernel(RouterArgs a) {
#pragma clang fp contract(off)
  extern __shared__ float lds[];  // gate rows [4][H + 4], then token rows [8][H + 4]
  __shared__ RouteShared rs;
  __shared__ PlanShared ps;
  __shared__ int s_flag;
  __shared__ float s_ngrp[kDecRT][kNormGroups], s_ntot[kDecRT];
  __shared__ float s_bias[kExperts];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, H = a.H, P = H + 4;
  // tokens per block: a deferred routing of more than kDeferBlockTokens
  // tokens runs blocks of kDeferBlockTokens per expert slice (fewer rows to
  // stage, and more threads per pair in its bound sums)
  const int rtb = router_block_tokens(a.defer, T);
  if (a.defer == 2) {
    // blocks past the token block's 8: the streaming kernel's rows to
    // kUnwritten (its readers reload a value until it is written), and the
    // token routing it publishes to "not yet" (kRouteUnset), apart from the
    // blocks that stage rows, whose loads those stores would hold up
    const int ncomp = kDecES * ((T + rtb - 1) / rtb);
    if ((int)blockIdx.x >= ncomp) {
      const int fb = (int)blockIdx.x - ncomp, nfb = (int)gridDim.x - ncomp;
      fill_unwritten(a, fb, nfb, tid, kThreads);
      if (fb == 0 && tid < T * kTopK) {
        a.s.idx[tid] = kRouteUnset;
        a.s.pos[tid] = kRouteUnset;
        a.s.wts[tid] = __builtin_bit_cast(float, kUnwritten);
      }
      return;
    }
  }
  const int tb = blockIdx.x / kDecES, es = blockIdx.x % kDecES;
  const int t0 = tb * rtb, e0 = es * kDecEPB;
  const int nt = min(rtb, T - t0);
  float *gs = lds, *xs = lds + kDecEPB * P;
  // the score bias, read now so the finishing block finds it in LDS
  if (tid < kExperts) s_bias[tid] = a.w.bias ? a.w.bias[tid] : 0.0f;
  if (a.defer == 3) {
    // the expert kernel's blocks plan the launch from the bounds: its queue
    // and dispatch counter start at 0, the gate/up tiles' masks at 0
    if (blockIdx.x == 0 && tid == 0) {
      Ctrl *ctrl = a.s.ctrl;
      ctrl->head = 0;
      ctrl->assign_done = 0;
      ctrl->deferred = 3;
      ctrl->num_tokens = T;
      ctrl->tile_rows = a.tile_rows;
      ctrl->n_rblocks = (T + kDecRT - 1) / kDecRT;
      ctrl->rtokens = kDecRT;
      ctrl->slots_assigned = 1;
      ctrl->router_done = 0;
    }
    if (blockIdx.x == 0 && tid < kClaimGroups) a.s.ctrl->gclaim[tid][0] = 0;
    const int ndep = dep_words(a.inter) * a.max_units;
    for (int i = blockIdx.x * kThreads + tid; i < ndep; i += gridDim.x * kThreads) a.s.dep[i] = 0;
  }
  if (a.defer == 2 && blockIdx.x == 0 && tid == 0) {
    // the streaming kernel routes and plans: its queues start at 0
    Ctrl *ctrl = a.s.ctrl;
    ctrl->head = 0;
    ctrl->deferred = a.defer;
    ctrl->num_tokens = T;
    ctrl->tile_rows = 0;
    ctrl->n_rblocks = 0;
    ctrl->stream_rows = a.bn;
    ctrl->chain_head = 0;
    ctrl->chain_done = 0;
    ctrl->chain_lazy = a.lazy_chains;
  }

  // 1. gate rows e0..e0+3 and token rows t0..t0+nt-1, 1 KiB per load
  {
    const int nch = H >> 8;
    const int items = (kDecEPB + nt) * nch;
    for (int i = wave; i < items; i += kThreads / 64) {
      const int r = i / nch, c = i % nch;
      const float *src = (r < kDecEPB ? a.w.gate + (size_t)(e0 + r) * H
                                      : a.x + (size_t)(t0 + r - kDecEPB) * H) +
                         c * 256 + lane * 4;
      float *dst = (r < kDecEPB ? gs + r * P : xs + (r - kDecEPB) * P) + c * 256;
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // 1b. fused post-attention RMSNorm: the staged rows are h; normalise them in
  // place, and the first of the token block's blocks stores them for the
  // expert kernel
  if (a.norm_w) {
    static_assert(kThreads == kNormThreads, "one reference row-block per router block");
    float part[kDecRT];
#pragma unroll
    for (int m = 0; m < kDecRT; ++m) {
      float sq = 0.0f;
      if (m < nt)
        for (int i = tid; i < H; i += kNormThreads) sq = __builtin_fmaf(xs[m * P + i], xs[m * P + i], sq);
      part[m] = sq;
    }
    norm_totals<kDecRT>(part, &s_ngrp[0][0], s_ntot);
    for (int m = 0; m < nt; ++m) {
      const float rms = norm_rms(s_ntot[m], H);
      for (int i = tid; i < H; i += kNormThreads) {
        const float v = (xs[m * P + i] * rms) * a.norm_w[i];
        xs[m * P + i] = v;
        if (es == 0) a.xn[(size_t)(t0 + m) * H + i] = v;
      }
    }
    __syncthreads();
  }
  if (a.defer >= 2) {
    // 2'. score bounds in place of the chains (score_bounds): tpp threads
    // per (token, expert) pair (all 256 threads on the block's nt tokens: 64
    // at one token, 8 at 5-8), k interleaved in float4s, four float sums of
    // products and four of magnitudes each (H / (4 tpp) FMAs per sum, then
    // 2 adds and log2(tpp) shuffle levels).  A pair's threads are
    // consecutive lanes.  Each thread's chains were the sums' critical path:
    // at one token 32 threads ran 64 steps each.
    const int tpp = nt == 1 ? 64 : nt == 2 ? 32 : nt <= 4 ? 16 : 8;
    const int lg = tpp == 64 ? 6 : tpp == 32 ? 5 : tpp == 16 ? 4 : 3;
    const int pr = tid >> lg, part = tid & (tpp - 1);
    const int tl = pr / kDecEPB, el = pr % kDecEPB;
    if (tl < nt) {
      const float *gp = gs + el * P, *xp = xs + tl * P;
      float sq[4] = {0.0f, 0.0f, 0.0f, 0.0f}, mq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
      for (int k = part * 4; k < H; k += 4 * tpp) {
        const f32x4 g = ld4(gp + k), xv = ld4(xp + k);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          sq[q] = __builtin_fmaf(g[q], xv[q], sq[q]);
          mq[q] = __builtin_fmaf(__builtin_fabsf(g[q]), __builtin_fabsf(xv[q]), mq[q]);
        }
      }
      float sum = (sq[0] + sq[1]) + (sq[2] + sq[3]), mag = (mq[0] + mq[1]) + (mq[2] + mq[3]);
      for (int o = 1; o < tpp; o <<= 1) {
        sum += __shfl_xor(sum, o, tpp);
        mag += __shfl_xor(mag, o, tpp);
      }
      if (part == 0) {
        float lo, hi;
        score_bounds(sum, mag, H, H / (4 * tpp) + 2 + lg, s_bias[e0 + el], &lo, &hi);
        if (a.defer == 2) {
          a.s.ctrl->sbound[0][t0 + tl][e0 + el] = lo;
          a.s.ctrl->sbound[1][t0 + tl][e0 + el] = hi;
        } else {  // read by the token block's finishing block
          float *b = a.s.bounds + (size_t)(t0 + tl) * 2 * kExperts + e0 + el;
          st_agent(b, lo);
          st_agent(b + kExperts, hi);
        }
      }
    }
    if (a.defer == 2) return;
    // 3'. the last of the token block's 8 blocks turns its tokens' bounds
    // into their possible sets: expert e stays possible unless four experts'
    // lower bounds exceed e's upper bound (then four experts beat e strictly
    // whatever the logits' rounding, and the strict-'>' insertion of
    // layer.cu:465-476 cannot keep it), so a set holds the token's exact
    // top-4, usually just those, a 5th or 6th on a near-tie at the 4th
    // place, all 32 where the bounds are infinite (non-finite inputs).  It
    // writes each token's mask and the block's count per expert (a copy per
    // die); every block of the expert kernel plans from them
    // (bounds_local_plan).
    // the token block of 8 this block's tokens belong to, and its blocks
    // (kDecES per rtb tokens)
    const int tb8 = t0 / kDecRT, t08 = tb8 * kDecRT, nt8 = min(kDecRT, T - t08);
    const int nblk8 = kDecES * ((nt8 + rtb - 1) / rtb);
    __builtin_amdgcn_s_waitcnt(0);  // this block's bounds are stored
    __syncthreads();
    if (tid == 0) {
      s_flag = fetch_add(&a.s.tb_done[tb8], 1) == nblk8 - 1;
      if (s_flag) {
        a.s.tb_done[tb8] = 0;  // all blocks counted in: reset
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      }
    }
    __syncthreads();
    if (!s_flag) return;
    {
      const int tl = tid >> 5, e = tid & (kExperts - 1);
      const bool tv = tl < nt8;
      const float *b = a.s.bounds + (size_t)(t08 + min(tl, nt8 - 1)) * 2 * kExperts + e;
      const float hi = b[kExperts];
      rs.prob[tl][e] = b[0];
      __syncthreads();
      int beat = 0;
#pragma unroll
      for (int j0 = 0; j0 < kExperts; j0 += 8) {
        float lv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) lv[j] = rs.prob[tl][j0 + j];
#pragma unroll
        for (int j = 0; j < 8; ++j) beat += (int)(lv[j] > hi);
      }
      const bool poss = tv && beat < kTopK;
      const uint32_t m = (uint32_t)(__ballot(poss) >> (32 * ((tid & 63) >> 5)));
      rs.sel[tl][e] = poss ? 1 : 0;
      // one copy per die (kPlanCopies): lane e < 8 of each token's row
      if (tv && e < kPlanCopies) a.s.bplan[(size_t)e * kPlanCopyInts + t08 + tl] = m;
      __syncthreads();
      {
        int cnt = 0;
#pragma unroll
        for (int t2 = 0; t2 < kDecRT; ++t2) cnt += rs.sel[t2][e];
        // thread (copy tl, expert e)
        static_assert(kPlanCopies == kDecRT, "a copy per token row of the block");
        a.s.bplan[(size_t)tl * kPlanCopyInts + kBoundTokens + tb8 * kExperts + e] = (uint32_t)cnt;
      }
    }
    return;
  } else if (wave == 0) {
    // 2. chains: wave 0, lane = (token l / 4, expert l % 4)
    const int tl = lane >> 2, el = lane & 3;
    const float *gp = gs + el * P;
    const float *xp = xs + min(tl, nt - 1) * P;
    const float acc = chain_dot(gp, xp, H);
    if (tl < nt) st_agent(&a.s.logits[(size_t)(t0 + tl) * kExperts + e0 + el], acc);
  } else {
    // waves 1-3, idle during the chains, prepare the expert kernel's rows
    fill_unwritten(a, blockIdx.x, gridDim.x, tid - 64, kThreads - 64);
  }
  const int nb = gridDim.x / kDecES;
  // the plan's input from LDS (one token block)
  PlanLocal loc{nullptr, nullptr, nullptr};
  {
    // 3. the last of the token block's 8 blocks finishes it
    __builtin_amdgcn_s_waitcnt(0);  // this block's logits are stored
    __syncthreads();
    if (tid == 0) {
      s_flag = fetch_add(&a.s.tb_done[tb], 1) == kDecES - 1;
      if (s_flag) {
        a.s.tb_done[tb] = 0;  // all blocks counted in: reset
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      }
    }
    __syncthreads();
    if (!s_flag) return;
    // 4-7. probabilities, top-4, weights, in-block ranks and counts
    {
      const int tl = tid >> 5;  // thread = (token tl, expert tid % 32)
      const float l = tl < nt ? a.s.logits[(size_t)(t0 + tl) * kExperts + (tid & (kExperts - 1))] : 0.0f;
      route_token_block(rs, nt, s_bias, l);
    }
    if (tid < nt) {
#pragma unroll
      for (int i = 0; i < kTopK; ++i) {
        st_agent(&a.s.idx[(size_t)(t0 + tid) * kTopK + i], rs.ti[tid][i]);
        a.s.wts[(size_t)(t0 + tid) * kTopK + i] = rs.tw[tid][i];
      }
    }
    if (nb == 1) {
      // a single token block plans from LDS (its plan writes pos and blk)
      static_assert(kDecRT <= kRouterSlotTokens, "one token block: the plan assigns every slot");
      loc = PlanLocal{rs.cnt, rs.ti, rs.rank};
    } else {
      {
        const int tl = tid >> 5, e = tid & (kExperts - 1);
        const int sel = rs.sel[tl][e];
        if (sel >= 0) st_agent(&a.s.pos[(size_t)(t0 + tl) * kTopK + sel], rs.rank[tl][sel]);
        if (tl == 0) st_agent(&a.s.blk[tb * kExperts + e], rs.cnt[e]);
      }
      // 8. the token block that finishes last plans
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0) {
        s_flag = fetch_add(&a.s.ctrl->router_done, 1) == nb - 1;
        if (s_flag) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      }
      __syncthreads();
      if (!s_flag) return;
    }
  }
  router_plan<kDecRT>(a, nb, T, ps, loc);
}

// Dense SwiGLU FFN (MLP::forward_gpu, layer.cu:1231-1269) as the block with
// its intermediate dimension cut into kDenseChunks "experts": every token
// goes to all of them with weight 1, so the combine adds the chunks' partial
// down-projections (W2 x = sum over chunks of W2[:, chunk] x[chunk]).  This
// router writes that fixed routing the way the routers write theirs (ids in
// rank order, in-block ranks, per-block counts) and plans with router_plan.
template <int RT>
__global__ __launch_bounds__(kThreads) void router_dense_kernel(RouterArgs a) {
  __shared__ PlanShared ps;
  __shared__ int s_flag;
  const int tid = threadIdx.x;
  const int T = a.T, t0 = blockIdx.x * RT;
  // blocks past the token blocks only prepare the expert kernel's rows
  const int nb = (T + RT - 1) / RT;
  if ((int)gridDim.x > nb) {
    if ((int)blockIdx.x >= nb)
      fill_unwritten(a, blockIdx.x - nb, gridDim.x - nb, tid, kThreads);
  } else {
    fill_unwritten(a, blockIdx.x, gridDim.x, tid, kThreads);
  }
  if ((int)blockIdx.x >= nb) return;
  const int nt = min(RT, T - t0);
  for (int f = tid; f < nt * kTopK; f += kThreads) {
    const size_t g = (size_t)t0 * kTopK + f;
    const int k = f % kTopK;
    st_agent(&a.s.idx[g], k < kDenseChunks ? k : -1);
    a.s.wts[g] = k < kDenseChunks ? 1.0f : 0.0f;
    st_agent(&a.s.pos[g], f / kTopK);  // every token of the block chose chunk k
  }
  if (tid < kExperts) st_agent(&a.s.blk[(size_t)blockIdx.x * kExperts + tid], tid < kDenseChunks ? nt : 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    s_flag = nb == 1 || (fetch_add(&a.s.ctrl->router_done, 1) == nb - 1);
    if (s_flag) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (!s_flag) return;
  router_plan<RT>(a, nb, T, ps);
}

// ---------------------------------------------------------------------------
// Expert kernel building blocks
// ---------------------------------------------------------------------------

// Dispatch task q: slots of the 64 tokens of router block q (replaces
// moe_scatter_kernel layer.cu:501-542: slot = block base + in-block rank, so
// slots are stable by token; x itself is not copied, the GEMM gathers rows).
__device__ __forceinline__ void assign_task(const ExpertArgs &a, int q, int rt, bool slots_ready) {
  const int tl = threadIdx.x >> 2, k = threadIdx.x & 3;
  const int tok = q * rt + tl;
  if (tl < rt && tok < a.T) {
    const int ee = a.s.idx[(size_t)tok * kTopK + k];
    if (slots_ready) {
      // the router assigned the slots (pos holds them already)
    } else if (ee >= 0 && ee < kExperts) {
      const int slot = a.s.blk[q * kExperts + ee] + a.s.pos[(size_t)tok * kTopK + k];
      if (slot >= 0 && slot < a.T * kTopK) {
        st_agent(&a.s.pos[(size_t)tok * kTopK + k], slot);
        st_agent(&a.s.slot_token[slot], tok);
      } else {  // inconsistent plan: flag it, never write out of range
        st_agent(&a.s.pos[(size_t)tok * kTopK + k], -1);
        __hip_atomic_store(&a.s.ctrl->err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    } else {
      st_agent(&a.s.pos[(size_t)tok * kTopK + k], -1);
    }
    // A token none of whose scores is selectable (all NaN or <= -1e30) has no
    // expert output, so no down tile completes it: its row is written here,
    // y = residual + 0.0f (the empty sum of layer.cu:708-720, then :1866).
    bool none = true;
#pragma unroll
    for (int kk = 0; kk < kTopK; ++kk) {
      const int ek = a.s.idx[(size_t)tok * kTopK + kk];
      none = none && (ek < 0 || ek >= kExperts);
    }
    if (none) {
      const int H4 = a.H >> 2;
      const float4 *r4 = reinterpret_cast<const float4 *>(a.residual);
      float4 *y4 = reinterpret_cast<float4 *>(a.y);
      for (int c4 = k; c4 < H4; c4 += kTopK) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r4) {
          const float4 rv = r4[(size_t)tok * H4 + c4];
          v = make_float4(rv.x + 0.0f, rv.y + 0.0f, rv.z + 0.0f, rv.w + 0.0f);
        }
        y4[(size_t)tok * H4 + c4] = v;
      }
    }
  }
}

// Token of a slot, clamped into [0, T) so a bad plan can never address
// outside x (the dispatch guards flag such plans in ctrl->err).
__device__ __forceinline__ int slot_tok(const ExpertArgs &a, int slot) {
  const int t = a.s.slot_token[slot];
  return t < 0 ? 0 : (t >= a.T ? a.T - 1 : t);
}

// Combine inside the down tiles (MFMA plans).  A down tile counts, for each
// of its rows and each kCombineCols-wide column range it covers, one more
// expert output of that row's token; the block whose count completes a
// token's expert outputs computes y for those columns with the reference's order: sum from 0.0f,
// fma over k ascending (layer.cu:708-720), then the residual add
// (layer.cu:1866-1871).  The arithmetic is the same whichever block does it.
// The tile's stores have completed before it counts (agent-scope stores), and
// the completing block acquires before it reads the other tiles' outputs.
// y may alias the residual: a thread reads its columns before it writes them.
// row_tok / mask (routing from score bounds, Ctrl::deferred == 3): the tile
// rows' tokens and each token's mask of possible experts, in LDS; the plan
// has a slot for every possible expert, so a token's outputs are complete
// once all of its slots have landed, and the sum takes its exact top-4 (pos,
// wts), which the dispatch tasks published before any down tile started.
template <int BN>
__device__ __forceinline__ void tile_combine(const ExpertArgs &a, int slot0, int rows, int col0,
                                             int *s_list, int *s_n, const int *row_tok = nullptr,
                                             const uint32_t *mask = nullptr) {
#pragma clang fp contract(off)
  constexpr int NJ = BN / kCombineCols;  // counters the tile's columns cover
  const int tid = threadIdx.x;
  const int ncc = a.H / kCombineCols, j0 = col0 / kCombineCols;
  __builtin_amdgcn_s_waitcnt(0);  // this block's expert-output stores have completed
  if (tid == 0) *s_n = 0;
  __syncthreads();
  if (tid < rows) {
    const int t = row_tok ? row_tok[tid] : slot_tok(a, slot0 + tid);
    int nvalid = 0;
    if (mask) {
      nvalid = __popc(mask[t]);
    } else {
#pragma unroll
      for (int k = 0; k < kTopK; ++k) nvalid += a.s.pos[(size_t)t * kTopK + k] >= 0;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (fetch_add(&a.s.ccount[(size_t)t * ncc + j0 + j], 1) == nvalid - 1)
        s_list[atomicAdd(s_n, 1)] = t * ncc + j0 + j;
  }
  __syncthreads();
  const int n = *s_n;
  if (n == 0) return;
  if (tid == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  __syncthreads();
  constexpr int NC4 = kCombineCols / 4;
  const int H4 = a.H >> 2;
  const float4 *so = reinterpret_cast<const float4 *>(a.s.sout);
  const float4 *r4 = reinterpret_cast<const float4 *>(a.residual);
  float4 *y4 = reinterpret_cast<float4 *>(a.y);
  for (int f = tid; f < n * NC4; f += kThreads) {
    const int item = s_list[f / NC4];
    const int t = item / ncc, c4 = (item % ncc) * NC4 + f % NC4;
    float4 v[kTopK];
    float w[kTopK];
    bool ok[kTopK];
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
      const int slot = a.s.pos[(size_t)t * kTopK + k];
      ok[k] = slot >= 0 && slot < a.s.slot_cap;
      w[k] = a.s.wts[(size_t)t * kTopK + k];
      v[k] = so[(size_t)(ok[k] ? slot : 0) * H4 + c4];
    }
    const float4 rv = r4 ? r4[(size_t)t * H4 + c4] : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
      if (!ok[k]) continue;
      acc.x = __builtin_fmaf(v[k].x, w[k], acc.x);
      acc.y = __builtin_fmaf(v[k].y, w[k], acc.y);
      acc.z = __builtin_fmaf(v[k].z, w[k], acc.z);
      acc.w = __builtin_fmaf(v[k].w, w[k], acc.w);
    }
    if (r4) {
      acc.x = rv.x + acc.x;
      acc.y = rv.y + acc.y;
      acc.z = rv.z + acc.z;
      acc.w = rv.w + acc.w;
    }
    y4[(size_t)t * H4 + c4] = acc;
  }
}



// Gate logits of TB token blocks (nt <= TB * kDecRT tokens from row t0) in
// the MFMA kernel: thread (token tid / 32, expert tid % 32) runs the FMA
// chains of that token of each of the TB blocks, each over k ascending,
// chain_dot's order (layer.cu:109-127), on operands staged through LDS in
// KC-wide chunks (the 32 gate rows, then the token rows), double-buffered,
// with the global loads of the next NR chunks in flight in registers (the
// weight tiles keep HBM busy meanwhile, so a load waits several
// microseconds).  acc[j]: the logit of token block j's token (tokens past nt:
// a copy of the last token's).  Ends with a barrier, after which lds is free.
template <int KC, int TB> constexpr int bc_floats() {
  return 2 * (kExperts + kDecRT * TB) * (KC + 4);
}

template <int KC, int NR, int TB>
__device__ void block_chains(const float *x, const float *gate, int t0, int nt, int H,
                             float *lds, float (&acc)[TB]) {
#pragma clang fp contract(off)
  constexpr int ROWS = kExperts + kDecRT * TB, P = KC + 4, F4 = ROWS * KC / 4;
  constexpr int PERT = (F4 + kThreads - 1) / kThreads;
  const int tid = threadIdx.x, tl = tid >> 5, e = tid & (kExperts - 1);
  const int nc = H / KC;
  f32x4 v[NR][PERT];
  auto load = [&](int c, f32x4 (&d)[PERT]) {
    if (c >= nc) return;
#pragma unroll
    for (int i = 0; i < PERT; ++i) {
      const int f = tid + i * kThreads;
      if (f < F4) {
        const int r = f / (KC / 4), c4 = f % (KC / 4);
        const float *row = r < kExperts ? gate + (size_t)r * H
                                        : x + (size_t)(t0 + min(r - kExperts, nt - 1)) * H;
        d[i] = ld4(row + c * KC + 4 * c4);
      }
    }
  };
  auto store = [&](const f32x4 (&d)[PERT], float *b) {
#pragma unroll
    for (int i = 0; i < PERT; ++i) {
      const int f = tid + i * kThreads;
      if (f < F4) st4(b + (f / (KC / 4)) * P + 4 * (f % (KC / 4)), d[i]);
    }
  };
  // chunk 0 in LDS, chunks 1 .. NR - 1 in registers v[1 ..]
  load(0, v[0]);
  store(v[0], lds);
#pragma unroll
  for (int j = 1; j < NR; ++j) load(j, v[j]);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < TB; ++j) acc[j] = 0.0f;
  for (int c0 = 0; c0 < nc; c0 += NR) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int c = c0 + r;
      if (c >= nc) break;
      // v[r] held chunk c (in LDS since the last step): chunk c + NR
      load(c + NR, v[r]);
      const float *b = lds + (c & 1) * ROWS * P;
      const float *gp = b + e * P, *xp = b + (kExperts + tl) * P;
#pragma unroll 4
      for (int k = 0; k < KC; k += 4) {
        const f32x4 g = ld4(gp + k);
#pragma unroll
        for (int j = 0; j < TB; ++j) {
          const f32x4 xv = ld4(xp + j * kDecRT * P + k);
          acc[j] = __builtin_fmaf(xv.x, g.x, acc[j]);
          acc[j] = __builtin_fmaf(xv.y, g.y, acc[j]);
          acc[j] = __builtin_fmaf(xv.z, g.z, acc[j]);
          acc[j] = __builtin_fmaf(xv.w, g.w, acc[j]);
        }
      }
      // chunk c + 1 to the other buffer (last read in chunk c - 1)
      if (c + 1 < nc) store(v[(r + 1) % NR], lds + ((c + 1) & 1) * ROWS * P);
      __syncthreads();
    }
  }
}

// Routing from score bounds under the MFMA plans (Ctrl::deferred == 3, up to
// kBoundTokens tokens, 32- and 64-row tiles): every block of the expert
// kernel plans the launch itself, in LDS, from the router's bounds.
struct BoundPlan {
  uint32_t mask[kBoundTokens];                    // possible experts of each token
  int base[kBoundTokens / kDecRT][kExperts];      // slot of token block b's first pair of expert e
  int tok[64];                                    // the current down tile's row tokens
  int wcnt[kThreads / 64];                        // per-wave counts (unit_tokens)
  int plan[8];                                    // nb, n1, n2, ntot, p1u, p2u, gtail, tail
};

// The plan of a routing from bounds, by every block (all threads), from the
// router's possible sets (each token's mask, each token block's count per
// expert: router_decode_kernel, defer 3):
//  - the exclusive prefix of the counts over token blocks, the counts,
//    offsets and units per expert, and the task plan router_plan writes for
//    the MFMA plans (its arithmetic, for BM-row tiles);
//  - base[b][e] = offsets[e] + expert e's pairs in token blocks before b, so
//    pair (t, e)'s slot is base[t / 8][e] + the block's earlier tokens with
//    e possible: the slots routing computes for the top-4 (layer.cu:494-542,
//    stable by token), over the possible pairs.
// Block 0 also publishes the counts (moe_last_plan_counts).
template <int BM>
__device__ __forceinline__ void bounds_local_plan(const ExpertArgs &a, Ctrl *c, BoundPlan &bp,
                                                  int *s_counts, int *s_offsets, int *s_unit_off) {
  constexpr int NBMAX = kBoundTokens / kDecRT;
  static_assert(kBoundTokens <= 4 * 64 && kThreads >= 128 + 64, "masks in wave 0, counts in wave 1");
  const int tid = threadIdx.x;
  const int T = a.T, nb = (T + kDecRT - 1) / kDecRT;
  // this die's copy of the router's masks and counts (blocks are dealt to
  // the dies in turn); wave 0 loads the masks (4 tokens a thread), wave 1
  // the counts (lane e: expert e's), each wave's loads in flight at once;
  // wave 3 has claimed the block's first task, whose return would hold up a
  // wave's later loads
  const uint32_t *cp = a.s.bplan + (size_t)(blockIdx.x % kPlanCopies) * kPlanCopyInts;
  if (4 * tid < T) {
    const int t0 = 4 * tid;
    if (t0 + 4 <= T) {
      const uint4 m4 = *reinterpret_cast<const uint4 *>(cp + t0);
      bp.mask[t0] = m4.x;
      bp.mask[t0 + 1] = m4.y;
      bp.mask[t0 + 2] = m4.z;
      bp.mask[t0 + 3] = m4.w;
    } else {
      for (int t = t0; t < T; ++t) bp.mask[t] = cp[t];
    }
  }
  const int e = tid - 64;
  if (e >= 0 && e < kExperts) {
    int v[NBMAX];
#pragma unroll
    for (int b = 0; b < NBMAX; ++b) v[b] = b < nb ? (int)cp[kBoundTokens + b * kExperts + e] : 0;
    int run = 0;
#pragma unroll
    for (int b = 0; b < NBMAX; ++b) {
      if (b < nb) bp.base[b][e] = run;
      run += v[b];
    }
    const int cnt = run;
    int total = 0, utotal = 0;
    const int off = lane_scan32(cnt, e, &total);
    const int uoff = lane_scan32((cnt + BM - 1) / BM, e, &utotal);
    s_counts[e] = cnt;
    s_offsets[e] = off;
    s_unit_off[e] = uoff;
    if (blockIdx.x == 0) c->counts[e] = cnt;
    if (e == 0) {
      s_offsets[kExperts] = total;
      s_unit_off[kExperts] = utotal;
      const int units = utotal;
      const int p1u = a.I / (Tile<BM>::BN / 2), p2u = a.H / Tile<BM>::BN;
      const int tail = min(units, a.tail_units);
      const int gtail = BM == 64 ? gate_up_tail(BM, T, units) : 0;
      const int n1 = (units + gtail) * p1u, n2 = (units - tail + 2 * tail) * p2u;
      bp.plan[0] = nb;
      bp.plan[1] = n1;
      bp.plan[2] = n2;
      bp.plan[3] = nb + n1 + n2;
      bp.plan[4] = p1u;
      bp.plan[5] = p2u;
      bp.plan[6] = gtail;
      bp.plan[7] = tail;
    }
  }
  __syncthreads();
  for (int i = tid; i < nb * kExperts; i += kThreads) bp.base[i / kExperts][i % kExperts] += s_offsets[i % kExperts];
  __syncthreads();
}

// The tokens of rows m0 .. m0 + rows - 1 of expert e's slots (its possible
// tokens in token order): out[r] = f(token of row r).  All threads; ends
// before the caller's barrier that publishes out.
template <typename F>
__device__ __forceinline__ void unit_tokens(BoundPlan &bp, int T, int e, int m0, int rows, F f) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool has = tid < T && ((bp.mask[tid] >> e) & 1u);
  const unsigned long long b = __ballot(has);
  if (lane == 0) bp.wcnt[wave] = __popcll(b);
  __syncthreads();
  int r = __popcll(b & ((1ull << lane) - 1ull));
  for (int w = 0; w < wave; ++w) r += bp.wcnt[w];
  if (has && r >= m0 && r < m0 + rows) f(r - m0, tid);
}

// Routing job q of a routing from score bounds (Ctrl::deferred == 3), run by
// the dispatch task of token block q * TB: the logits of token blocks q * TB
// .. q * TB + TB - 1 (block_chains), each block's exact routing
// (route_token_block: the reference's sigmoid, strict-'>' top-4 and
// weights), and for each (token, rank) the slot the plan gave that expert
// (the possible set holds the exact top-4: a miss, which the token's mask
// shows, is an inconsistent plan, flagged); bp: the block's plan.  Down
// tiles, whose combines read idx / wts / pos, start only after every
// dispatch task has signalled.
template <int KC, int NR, int TB>
__device__ __forceinline__ void route_task(const ExpertArgs &a, int q, float *lds, const BoundPlan &bp) {
  const int tid = threadIdx.x, tl = tid >> 5, e = tid & (kExperts - 1);
  const int t0 = q * TB * kDecRT, nt = min(TB * kDecRT, a.T - t0);
  float l[TB];
  block_chains<KC, NR, TB>(a.x, a.w.gate, t0, nt, a.H, lds, l);
  RouteShared &rs = *reinterpret_cast<RouteShared *>(lds);
  float *bias = lds + (sizeof(RouteShared) + sizeof(float) - 1) / sizeof(float);
  if (tid < kExperts) bias[tid] = a.w.bias ? a.w.bias[tid] : 0.0f;
#pragma unroll
  for (int j = 0; j < TB; ++j)
    if (j * kDecRT + tl < nt) a.s.logits[(size_t)(t0 + j * kDecRT + tl) * kExperts + e] = l[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < TB; ++j) {
    const int tb0 = t0 + j * kDecRT, ntj = min(kDecRT, a.T - tb0);
    if (ntj <= 0) break;
    route_token_block(rs, ntj, bias, l[j]);
    if (tid < ntj * kTopK) {
      const int tt = tid / kTopK, k = tid % kTopK, t = tb0 + tt;
      const int ee = rs.ti[tt][k];
      int slot = -1;
      if (ee >= 0 && ee < kExperts) {
        // the plan's slot: token block base + the block's earlier tokens
        // with ee possible
        if ((bp.mask[t] >> ee) & 1u) {
          slot = bp.base[t / kDecRT][ee];
          for (int t2 = t - t % kDecRT; t2 < t; ++t2) slot += (int)((bp.mask[t2] >> ee) & 1u);
        }
        if (slot < 0 || slot >= a.s.slot_cap) {
          slot = -1;
          __hip_atomic_store(&a.s.ctrl->err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      st_agent(&a.s.idx[(size_t)t * kTopK + k], ee);
      st_agent(&a.s.wts[(size_t)t * kTopK + k], rs.tw[tt][k]);
      st_agent(&a.s.pos[(size_t)t * kTopK + k], slot);
    }
    __syncthreads();  // rs is rewritten by the next block's routing
  }
}

// Expert owning unit u: the largest e with unit_off[e] <= u (skips experts
// without units, whose unit_off equals the next one's).
__device__ __forceinline__ int unit_expert(const int *unit_off, int u) {
  int lo = 0, hi = kExperts;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (unit_off[mid] <= u) lo = mid; else hi = mid;
  }
  return lo;
}

// Unit order of the MFMA plans' tile phases (the task indices and dep
// counters of both phases use it).  When most experts hold a single partial
// unit (64-row plan, twice the full units at most the partial ones: T <= ~400
// tokens), units go longest first: every expert's full BM-row units (expert
// order; full_off = their exclusive scan over experts), then each expert's
// partial last unit by its rows descending (pexp, ties by expert index), so
// the queue ends with the cheapest tiles and the last round of tasks is short
// (expert launch 372 -> 343 us at T=256; whole step 395 -> 345 us at T=160).
// Otherwise units keep expert order (unit_off): experts holding several
// units then read the same weights in tiles close together in time, and
// longest first cost 3.5% at T=640 and 1.5-4% with 128-row tiles.
// Unit v: expert e, rows m0 .. m0 + rows - 1 of the expert's slots.
struct UnitOrder {
  const int *unit_off, *full_off, *pexp, *counts;
  int nfull;
  bool lpt;
};

template <int BM>
__device__ __forceinline__ void unit_rows(int v, const UnitOrder &o, int &e, int &m0, int &rows) {
  if (BM <= 64 && o.lpt) {
    if (v < o.nfull) {
      e = unit_expert(o.full_off, v);
      m0 = (v - o.full_off[e]) * BM;
      rows = BM;
    } else {
      e = o.pexp[v - o.nfull];
      rows = o.counts[e] % BM;
      m0 = o.counts[e] - rows;
    }
  } else {
    e = unit_expert(o.unit_off, v);
    m0 = (v - o.unit_off[e]) * BM;
    rows = min(BM, o.counts[e] - m0);
  }
}

// The first round of claims of a routing from bounds: tasks [0, f), group
// g's k-th claim (Ctrl::gclaim) task k * kClaimGroups + g.  Thread 0, before
// the block's first claim from the queue head: a first-round task that no
// block has claimed yet, claimed now, or -1 once all of them are claimed
// (the counters only grow, so a count at its quota is final).
__device__ __forceinline__ int first_round_left(Ctrl *c, int f) {
  int v[kClaimGroups];
#pragma unroll
  for (int g = 0; g < kClaimGroups; ++g) v[g] = load_relaxed(&c->gclaim[g][0]);
#pragma unroll
  for (int g = 0; g < kClaimGroups; ++g) {
    const int quota = f > g ? (f - 1 - g) / kClaimGroups + 1 : 0;
    if (v[g] < quota) {
      const int t = claim(&c->gclaim[g][0]) * kClaimGroups + g;
      if (t < f) return t;
    }
  }
  return -1;
}

template <int BM>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void expert_mfma_kernel(ExpertArgs a) {
  using TL = Tile<BM>;
  extern __shared__ float lds[];
  __shared__ int s_task;
  __shared__ int s_unit_off[kExperts + 1];
  __shared__ int s_full_off[kExperts + 1];  // unit order (unit_rows)
  __shared__ int s_pexp[kExperts];
  __shared__ int s_nfull, s_lpt;
  __shared__ int s_offsets[kExperts + 1];
  __shared__ int s_counts[kExperts];
  __shared__ int s_aoff[BM];
  __shared__ int s_comb[BM * (Tile<BM>::BN / kCombineCols)];
  __shared__ int s_ncomb;
  // routing from score bounds (Ctrl::deferred == 3): 32- and 64-row plans
  // of up to kBoundTokens tokens, planned by every block (bounds_local_plan)
  constexpr bool kBounds = BM <= 64;
  struct NoPlan {};
  __shared__ typename std::conditional<kBounds, BoundPlan, NoPlan>::type s_bp;
  Ctrl *c = a.s.ctrl;
  const int tid = threadIdx.x;
  const bool bounds = kBounds && a.bounds != 0;
  // the last wave claims: the plan's loads are in the other waves.  A
  // routing from bounds draws the blocks' first tasks from kClaimGroups
  // counters (Ctrl::gclaim): the first round of claims, in a grid of more
  // blocks than dispatch tasks (a block that runs one late ends after it)
  const bool groups = bounds && (int)gridDim.x > (a.T + kDecRT - 1) / kDecRT;
  if (tid == kThreads - 1) {
    const int g = (int)(blockIdx.x % kClaimGroups);
    s_task = groups ? claim(&c->gclaim[g][0]) * kClaimGroups + g : claim(&c->head);
  }
  int pv[8];  // nb, n1, n2, ntot, p1u, p2u, gtail, tail
  const int *row_tok = nullptr;
  const uint32_t *pmask = nullptr;
  if constexpr (kBounds) {
    if (bounds) {
      bounds_local_plan<BM>(a, c, s_bp, s_counts, s_offsets, s_unit_off);
#pragma unroll
      for (int i = 0; i < 8; ++i) pv[i] = s_bp.plan[i];
      row_tok = s_bp.tok;
      pmask = s_bp.mask;
    }
  }
  if (!bounds) {
    if (tid <= kExperts) {
      s_unit_off[tid] = c->unit_off[tid];
      s_offsets[tid] = c->offsets[tid];
    }
    if (tid < kExperts) s_counts[tid] = c->counts[tid];
    pv[0] = c->n_rblocks;
    pv[1] = c->n_p1;
    pv[2] = c->n_p2;
    pv[3] = c->n_total;
    pv[4] = c->p1_per_unit;
    pv[5] = c->p2_per_unit;
    pv[6] = BM >= 64 ? c->gu_tail : 0;
    pv[7] = c->tail_units;
  }
  const int nb = pv[0], n1 = pv[1], n2 = pv[2], ntot = pv[3], p1u = pv[4], p2u = pv[5];
  const int gtail = pv[6];
  const int nunits = n1 / p1u - gtail, tail = pv[7];
  const int H = a.H, I = a.I;
  const AgentOut inter_out(a.s.inter, a.s.inter_bytes), sout_out(a.s.sout, a.s.sout_bytes);
  __syncthreads();
  if (BM <= 64 && tid < kExperts) {  // the unit order, from the counts (lanes 0-31 of wave 0)
    const int cnt = s_counts[tid];
    const int part = cnt % BM;
    int nfull;
    s_full_off[tid] = lane_scan32(cnt / BM, tid, &nfull);
    const int npart = __popcll(__ballot(part > 0));
    if (tid == 0) {
      s_full_off[kExperts] = nfull;
      s_nfull = nfull;
      s_lpt = 2 * nfull <= npart;
    }
    // the rank from the other lanes' values, read from their registers
    // (a loop of LDS reads, each waiting for the last: same box, T=256
    // 307.2 -> 305.4 us, T=64-192 ~0.9 us)
    int r = 0;
#pragma unroll
    for (int j = 0; j < kExperts; ++j) {
      const int pj = __builtin_amdgcn_readlane(part, j);
      r += pj > part || (pj == part && j < tid);
    }
    if (part > 0) s_pexp[r] = tid;
  }
  __syncthreads();
  const UnitOrder uo{s_unit_off, s_full_off, s_pexp, s_counts, BM <= 64 ? s_nfull : 0,
                     BM <= 64 && s_lpt != 0};
  // slots written by the router: gate/up tiles need not wait for the dispatch
  // tasks, which then only clear the combine counters (down tiles wait for
  // them) and write the rows of tokens without an expert
  // (routing from bounds: the blocks' own plan, no control field to read)
  const bool slots_ready = bounds || c->slots_assigned != 0;
  // routing jobs (routing from bounds): one token block each, 128-wide k
  // chunks where the tiles' LDS holds two of them (else 64), six chunks of
  // loads in flight
  constexpr int kBcTB = 1, kBcNR = 6;
  constexpr int kBcKC = bc_floats<128, kBcTB>() <= TL::LDS_FLOATS ? 128 : 64;
  static_assert(bc_floats<kBcKC, kBcTB>() <= TL::LDS_FLOATS &&
                    sizeof(RouteShared) + kExperts * sizeof(float) <= TL::LDS_FLOATS * sizeof(float),
                "a routing job's chains and routing fit the kernel's LDS");
  // Claims.  The queue head hands out tasks nfirst + 0, 1, 2, ...  A routing
  // from bounds hands out the first nfirst tasks (at most one per block, the
  // dispatch and gate/up tasks, none of which waits for another task) from
  // the group counters.  A block claims from the head only once every
  // first-round task is claimed (first_round_left: it claims any left
  // itself), so a block that has not started (another kernel holds its CU)
  // holds no task that a running block's down tile waits for: claims then
  // follow the task order, as with the head alone.
  const int nfirst = groups ? min((int)gridDim.x, nb + n1) : 0;
  int first_left = groups ? 1 : 0;  // thread 0: first-round tasks may be unclaimed
  auto next_task = [&]() -> int {
    if (first_left) {
      const int t = first_round_left(c, nfirst);
      if (t >= 0) return t;
      first_left = 0;
    }
    return nfirst + claim(&c->head);
  };
  int task = s_task;
  if (groups && task >= nfirst) {  // a group's claim past the first round
    __syncthreads();
    if (tid == 0) s_task = next_task();
    __syncthreads();
    task = s_task;
  }
  // A dispatch task: the routing of its token block (a routing from bounds)
  // or its slots, and its tokens' combine counters cleared.
  auto run_dispatch = [&](int task) {
    const int rt = bounds ? kDecRT : c->rtokens;
    if (!bounds) {
      assign_task(a, task, rt, slots_ready);
    } else if (task % kBcTB == 0) {
      if constexpr (kBounds) route_task<kBcKC, kBcNR, kBcTB>(a, task / kBcTB, lds, s_bp);
    }
    // this router block's tokens start with no expert outputs counted
    const int ncc = H / kCombineCols;
    for (int i = tid; i < rt * ncc; i += kThreads) {
      const int tok = task * rt + i / ncc;
      if (tok < a.T) st_agent(&a.s.ccount[(size_t)tok * ncc + i % ncc], 0);
    }
    block_signal(&c->assign_done);
  };
  // Dispatch tasks lead the queue, so a block runs its dispatch tasks before
  // its first tile (a loop of their own: the tiles' registers are allocated
  // apart from the routing's).
  while (task < nb && task < ntot) {
    run_dispatch(task);
    if (tid == 0) s_task = next_task();
    __syncthreads();
    task = s_task;
    __syncthreads();
  }
  while (task >= nb && task < ntot) {
    int next = 0;  // the block's next task (thread 0), claimed near this one's end
    if (task < nb + n1) {
      // gate/up tiles: full width for the first units, two half-width tiles
      // per column range for the last gtail units (small batches of either plan)
      const int q = task - nb;
      const int gfull = (nunits - gtail) * p1u;
      const bool ghalf = q >= gfull;
      const int u = ghalf ? nunits - gtail + (q - gfull) / (2 * p1u) : q / p1u;
      const int nt = ghalf ? (q - gfull) % (2 * p1u) : q % p1u;
      int e, m0, rows;
      unit_rows<BM>(u, uo, e, m0, rows);
      const int slot0 = s_offsets[e] + m0;
      if (!slots_ready) block_wait(&c->assign_done, nb, a.wait_limit, &c->err);
      if (!bounds) {
        if (tid < BM) s_aoff[tid] = tid < rows ? slot_tok(a, slot0 + tid) * H : -1;
      } else {
        if constexpr (kBounds) {
          if (tid >= rows && tid < BM) s_aoff[tid] = -1;
          unit_tokens(s_bp, a.T, e, m0, rows, [&](int r, int t) { s_aoff[r] = t * H; });
        }
      }
      __syncthreads();
      const float *brow0 = a.w.w13 + ((size_t)e * 2 * I + (size_t)nt * TL::BN) * H;
      const uint32_t xbytes = (uint32_t)((size_t)a.T * H * sizeof(float));
      // a 128-row unit holding at most 64 rows runs as a 64x128 tile (same
      // columns and outputs, half the padding MFMAs)
      static_assert(Tile<64>::BN == Tile<128>::BN, "a 64-row tile covers a 128-row unit's columns");
      if constexpr (BM == 64) {
        if (ghalf) {  // one W1/W3 row group: 32 intermediate columns
          using TH = TileHalf<64>;
          const float *hrow0 = a.w.w13 + ((size_t)e * 2 * I + (size_t)nt * TH::BN) * H;
          next = mfma_tile<TH, true>(lds, a.x, xbytes, s_aoff, rows, hrow0, H, inter_out, slot0,
                                     I, nt * (TH::BN / 2), next_task);
        } else {
          next = mfma_tile<TL, true>(lds, a.x, xbytes, s_aoff, rows, brow0, H, inter_out, slot0,
                                     I, nt * (TL::BN / 2), next_task);
        }
      } else if (BM == 128 && ghalf) {  // one W1/W3 row group: 32 intermediate columns
        static_assert(TileHalf<64>::BN == TileHalf<128>::BN, "a half tile's columns");
        using TH = TileHalf<128>;
        const float *hrow0 = a.w.w13 + ((size_t)e * 2 * I + (size_t)nt * TH::BN) * H;
        if (rows <= 64)
          next = mfma_tile<TileHalf<64>, true>(lds, a.x, xbytes, s_aoff, rows, hrow0, H, inter_out,
                                               slot0, I, nt * (TH::BN / 2), next_task);
        else
          next = mfma_tile<TH, true>(lds, a.x, xbytes, s_aoff, rows, hrow0, H, inter_out, slot0, I,
                                     nt * (TH::BN / 2), next_task);
      } else if (BM == 128 && rows <= 64) {
        next = mfma_tile<Tile<64>, true>(lds, a.x, xbytes, s_aoff, rows, brow0, H, inter_out, slot0,
                                         I, nt * (TL::BN / 2), next_task);
      } else {
        next = mfma_tile<Tile<BM>, true>(lds, a.x, xbytes, s_aoff, rows, brow0, H, inter_out, slot0,
                                         I, nt * (TL::BN / 2), next_task);
      }
      // this tile's intermediate columns are stored: its bit of the unit's mask
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0)
        __hip_atomic_fetch_or(&a.s.dep[(size_t)dep_words(I) * u + (nt >> 5)], (int)(1u << (nt & 31)),
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (task < nb + n1 + n2) {
      // down tiles: full width for the first units, two half-width tiles per
      // column range for the last tail units
      const int q = task - nb - n1;
      const int nfull = (nunits - tail) * p2u;
      const bool half = q >= nfull;
      const int u = half ? nunits - tail + (q - nfull) / (2 * p2u) : q / p2u;
      const int ht = half ? (q - nfull) % (2 * p2u) : q % p2u;
      int e, m0, rows;
      unit_rows<BM>(u, uo, e, m0, rows);
      const int slot0 = s_offsets[e] + m0;
      block_wait(&c->assign_done, nb, a.wait_limit, &c->err);  // combine counters cleared
      if (tid < BM) s_aoff[tid] = tid < rows ? tid * I : -1;
      if constexpr (kBounds) {  // the rows' tokens, for the combine
        if (bounds) unit_tokens(s_bp, a.T, e, m0, rows, [&](int r, int t) { s_bp.tok[r] = t; });
      }
      __syncthreads();
      // 32- and 64-row plans above 128 tokens: each slab of the tile waits
      // for the gate/up tile that wrote its intermediate columns (half-width
      // ones for the last gtail units), so the tile starts once its unit's
      // first gate/up tiles have landed (T=256 320.7 -> 316.2 us, T=512
      // 514.4 -> 507.4).  At 64-128 tokens, whose down tiles seldom wait (the
      // per-slab form was 0.5 % slower there), and in the 128-row plan, whose
      // slab loop has no registers to spare, the tile waits for all of them
      // first.
      static_assert(TL::BK == TileHalf<BM>::BK && (BM != 128 || Tile<64>::BK == TL::BK),
                    "one slab width");
      using Ready = typename std::conditional<BM == 128, NoWait, SlabReady>::type;
      Ready ready{};
      const bool whole = BM == 128 || a.T <= kSlabWaitMinTokens;
      if (whole) {
        if (tid == 0) {
          const int *bits = a.s.dep + (size_t)dep_words(I) * u;
          const int gbits = u >= nunits - gtail ? 2 * p1u : p1u;
          for (int b = 0; b < gbits; b += 32) {
            const unsigned m = gbits - b >= 32 ? ~0u : (1u << (gbits - b)) - 1u;
            int spins = 0;
            while (((unsigned)load_relaxed(bits + b / 32) & m) != m) {
              __builtin_amdgcn_s_sleep(8);
              if (++spins > a.wait_limit) {
                st_agent(&c->err, 1);
                break;
              }
            }
          }
        }
        __syncthreads();
      }
      if constexpr (BM != 128) if (!whole) {
        // a gate/up tile writes BN / 2 intermediate columns (a power of two,
        // at least a slab's BK): slab s needs tile s >> shift
        constexpr int kFullShift = __builtin_ctz(TL::BN / 2 / TL::BK);
        constexpr int kHalfShift = __builtin_ctz(TileHalf<BM>::BN / 2 / TL::BK);
        static_assert((TL::BN / 2) % TL::BK == 0 && (TileHalf<BM>::BN / 2) % TL::BK == 0 &&
                          (1 << kFullShift) * TL::BK == TL::BN / 2 &&
                          (1 << kHalfShift) * TL::BK == TileHalf<BM>::BN / 2,
                      "gate/up tiles cover whole slabs");
        ready = Ready{a.s.dep + (size_t)dep_words(I) * u, u >= nunits - gtail ? kHalfShift : kFullShift,
                      I / TL::BK, a.wait_limit, &c->err};
      }
      const float *abase = a.s.inter + (size_t)slot0 * I;
      const uint32_t abytes = a.s.inter_bytes - (uint32_t)((size_t)slot0 * I * sizeof(float));
      if (half) {
        using TH = TileHalf<BM>;
        const float *brow0 = a.w.w2 + ((size_t)e * H + (size_t)ht * TH::BN) * I;
        next = mfma_tile<TH, false>(lds, abase, abytes, s_aoff, rows, brow0, I, sout_out, slot0,
                                    H, ht * TH::BN, next_task, ready);
        tile_combine<TH::BN>(a, slot0, rows, ht * TH::BN, s_comb, &s_ncomb, row_tok, pmask);
      } else {
        const float *brow0 = a.w.w2 + ((size_t)e * H + (size_t)ht * TL::BN) * I;
        if (BM == 128 && rows <= 64)
          next = mfma_tile<Tile<64>, false>(lds, abase, abytes, s_aoff, rows, brow0, I, sout_out,
                                            slot0, H, ht * TL::BN, next_task, ready);
        else
          next = mfma_tile<TL, false>(lds, abase, abytes, s_aoff, rows, brow0, I, sout_out, slot0,
                                      H, ht * TL::BN, next_task, ready);
        tile_combine<TL::BN>(a, slot0, rows, ht * TL::BN, s_comb, &s_ncomb, row_tok, pmask);
      }
    }
    __syncthreads();
    if (tid == 0) s_task = next;
    __syncthreads();
    task = s_task;
  }
  // A first-round dispatch task that no block had claimed when this block's
  // tile claimed (its group's blocks had not started: first_round_left)
  // runs here, and the block ends: the blocks that claim on finish the
  // queue (the grid holds more blocks than dispatch tasks).
  if (task < nb) run_dispatch(task);
}

// ---------------------------------------------------------------------------
// Weight-streaming kernel for small T (expert_ring_kernel).
//
// HBM saturates with ~32 KiB of loads in flight per CU, and every round trip
// a CU makes queues behind whatever it already has in flight, so this kernel
// keeps each wave only a few KiB ahead and never puts a control round trip
// between a wave and its weights.  Each block has eight streaming waves and
// one control wave.  Streaming wave w owns the k slice [256w, 256w + 256) of
// a task's 16 weight rows and walks it in 16 steps of 16 floats; a step loads
// one f32x4 of weights per lane (lane l: row l%16, k offset 4*(l/16)) and one
// f32x4 of token rows per pass of 16 tokens in the same shape, and feeds both
// to v_mfma_f32_16x16x4f32 (16 rows x 16 tokens, k permuted consistently in
// the A and B operands).  Loads run kRingDepth steps ahead in a register ring
// that crosses task boundaries.  The control wave sums the eight k-slice
// partials a task leaves in LDS and stores the results (SwiGLU applied for
// gate/up) with agent-coherent stores; nothing signals that they are done.
// The router fills the intermediate and expert-output rows with kUnwritten,
// and their readers load them coherently (sc1) and reload any value that is
// still kUnwritten, so a consumer starts as soon as the values it needs have
// landed, with no store-completion wait, counter or poll in between.
//
// Row tasks follow the plan's order: gate/up row blocks expert by expert,
// then down row blocks.  Every task comes from a queue counter: a block's
// first one is claimed as it starts, each later one by streaming wave 0 at
// the first step of the block's current task, so a block that draws cheap
// tasks takes more of them, and a block that is not resident (another
// kernel holds its CU) owns no task that a running block waits for.  The ring issues a down
// task's loads while the task before it still runs; a down task waits, at
// the step that consumes them, for intermediate values still unwritten.
// Only down tasks wait and gate/up tasks never do, and a block claims a down
// task only after every gate/up task has been claimed (claims follow the
// order), by a block that runs it to the end: a block's earlier tasks are
// finished before its streaming waves reach its next task's first step.  So
// every gate/up task finishes, and then every down task.  The combine tasks
// (one per token), which wait for their token's expert outputs, are dealt
// round-robin (block b runs tokens b, b + G, ...) after the row tasks.
// ---------------------------------------------------------------------------

constexpr int kRingWaves = 8;                       // k-slice streaming waves
constexpr int kRingThreads = (kRingWaves + 1) * 64; // + the control wave
constexpr int kRingSteps = 16;                      // 16-float k steps per wave per task
constexpr int kRingDepth = 4;                       // steps in flight ahead of the MFMAs
constexpr int kRingSlice = kRingSteps * 16;         // floats of k per wave (256)
constexpr int kRingMaxSlots = 4096;                 // slot -> token map kept in LDS
static_assert(kRingWaves * kRingSlice == 2048, "k slices cover rows of <= 2048 floats");
static_assert(kRingSteps % kRingDepth == 0, "ring rotation realigns at task boundaries");
// Token passes per ring step: 1 or 2, the fewest that cover the largest
// expert's tokens (larger experts run in several groups).  A pass that holds
// no tokens would still move 1 KiB per wave per step through the CU's
// load-return path, so the kernel picks the count from the plan at run time.
// (kRingMaxPasses, moe_internal.h)
// 64-row tasks (batches from 32 tokens) share each token-row load across
// their 4 row groups.  Up to 16 tokens per expert, a wave streams the groups
// one after another and keeps its token slice in registers: a CU then reads
// one 16-row block at a time, which streams at ~6.3 TB/s where reading 2 or 4
// row blocks at once reaches 5.0-5.9 TB/s (measured with a bare load probe).
// With two token passes the four groups are read at once.
// (kRingWideGroups, moe_internal.h)
// 32-row tasks with 4 passes: batches whose largest expert holds 33-64
// tokens (the router picks them from the counts; the dense FFN's chunks hold
// all tokens), so each weight row is read once; 64-row tasks with 4 passes
// would need twice the LDS for their partials.
// (kRingDenseGroups, kRingDensePasses, moe_internal.h)

// 64-row tasks read at once load 4 weight rows per step; with two token
// passes half the depth keeps the ring within the register budget of 3 waves
// per SIMD.
constexpr int ring_depth(int rg, int p) { return rg == 1 || p == 1 ? kRingDepth : kRingDepth / 2; }

struct RingShared {
  int active[kExperts], counts[kExperts], offsets[kExperts];
  int tok[kRingMaxSlots];  // slot -> token
  int flushed;             // items whose partials the control wave has consumed
  int done[2];             // streaming waves that wrote item i's partials into buffer i & 1
  int abort;
  int seq[8];              // the block's j-th row task id at seq[j & 7]
  int nseq;                // row task ids published so far
  int local;               // 1: routing computed by this block; 2: planned from the score bounds
  int rpos[kDecRT][kTopK]; // local routing: slot of each (token, rank), -1: none
  float rw[kDecRT][kTopK]; // local routing: weights
  int slotmap[kDecRT][kExperts];  // plan from the bounds: slot of each (token, expert), -1: none
  float bias[kExperts];    // score bias (deferred routing)
};

__device__ __forceinline__ int lds_load(const int *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_store(int *p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Orderings of LDS accesses between waves of the block; they wait only for
// LDS operations (lgkmcnt), never for the wave's outstanding global loads.
__device__ __forceinline__ void release_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
}
__device__ __forceinline__ void acquire_lds() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 100 MHz constant clock: waits are bounded in time, not in polls.
__device__ __forceinline__ long long ring_now() { return __builtin_amdgcn_s_memrealtime(); }
constexpr long long kRingTicksPerLimit = 20;  // wait_limit x 200 ns

// Streaming side: wait until cond(*p) holds.  False if the block aborts; a
// wait longer than `ticks` reports a device timeout and aborts the block.
template <typename Cond>
__device__ __forceinline__ bool ring_wait(const int *p, Cond cond, int *abort_flag, int *err,
                                          long long ticks) {
  if (cond(__builtin_amdgcn_readfirstlane(lds_load(p)))) {
    acquire_lds();
    return true;
  }
  const long long t0 = ring_now();
  while (!cond(__builtin_amdgcn_readfirstlane(lds_load(p)))) {
    if (__builtin_amdgcn_readfirstlane(lds_load(abort_flag))) return false;
    if (ring_now() - t0 > ticks) {
      if ((threadIdx.x & 63) == 0) {
        st_agent(err, 1);
        lds_store(abort_flag, 1);
      }
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  acquire_lds();
  return true;
}

struct RingPlan {
  int n1, n2, ncomb, p1u, p2u, grid, rows;
  int sub;                // row sub-groups streamed one after another per task
  int tail_q, tail_u0;    // down tasks from tail_q: 16-row tasks of units tail_u0..
};

// A row task, wave-uniform.  kind: 1 gate/up rows, 2 down rows, 4 none (the
// queue ran out).  A row task runs in groups of up to 16 * P tokens (one
// pass of the ring per group).
struct RingTask {
  int kind, q, u, e, cnt, slot0, col, ngroups, nsub;
};

template <int P>
__device__ __forceinline__ RingTask ring_task(const RingShared &sh, const RingPlan &pl, int task) {
  task = __builtin_amdgcn_readfirstlane(task);
  RingTask t{4, 0, 0, 0, 0, 0, 0, 1, 1};
  if (task < 0 || task >= pl.n1 + pl.n2) return t;
  t.nsub = pl.sub;
  if (task < pl.n1) {
    t.kind = 1;
    t.q = task;
    t.u = task / pl.p1u;
    t.col = (task % pl.p1u) * (pl.rows / 2);
  } else {
    t.kind = 2;
    t.q = task - pl.n1;
    if (t.q < pl.tail_q) {
      t.u = t.q / pl.p2u;
      t.col = (t.q % pl.p2u) * pl.rows;
    } else {  // the last units' down rows in single 16-row sub-groups
      const int qq = t.q - pl.tail_q, per = pl.p2u * pl.sub;
      t.u = pl.tail_u0 + qq / per;
      t.col = (qq % per) * (pl.rows / pl.sub);
      t.nsub = 1;
    }
  }
  t.e = __builtin_amdgcn_readfirstlane(sh.active[t.u]);
  t.cnt = __builtin_amdgcn_readfirstlane(sh.counts[t.e]);
  t.slot0 = __builtin_amdgcn_readfirstlane(sh.offsets[t.e]);
  t.ngroups = t.cnt > 0 ? (t.cnt + kRingTokens * P - 1) / (kRingTokens * P) : 1;
  return t;
}

// The block's j-th row task; its id is published before any wave reads it.
template <int P>
__device__ __forceinline__ RingTask ring_seq_task(const RingShared &sh, const RingPlan &pl, int j) {
  return ring_task<P>(sh, pl, lds_load(&sh.seq[j & 7]));
}

// Buffer descriptors: weights, token rows, intermediate rows, and an empty
// one whose loads return zeros without touching memory.
struct RingRsrc {
  __amdgpu_buffer_rsrc_t w13, w2, x, inter, none;
};

__device__ __forceinline__ RingRsrc ring_rsrc(const ExpertArgs &a) {
  RingRsrc r;
  const size_t b13 = (size_t)kExperts * 2 * a.I * a.H * sizeof(float);
  const size_t b2 = (size_t)kExperts * a.H * a.I * sizeof(float);
  const size_t bx = (size_t)a.T * a.H * sizeof(float);
  r.w13 = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(a.w.w13), 0, (int)b13, kBufferRsrcWord3);
  r.w2 = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(a.w.w2), 0, (int)b2, kBufferRsrcWord3);
  r.x = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(a.x), 0, (int)bx, kBufferRsrcWord3);
  r.inter = __builtin_amdgcn_make_buffer_rsrc(a.s.inter, 0, (int)a.s.inter_bytes, kBufferRsrcWord3);
  r.none = __builtin_amdgcn_make_buffer_rsrc(a.s.inter, 0, 0, kBufferRsrcWord3);
  return r;
}

constexpr uint32_t kRingOff = 0xFFFF0000u;  // lane offset past any buffer: loads read 0

// What one streaming lane loads for a group of a task: a weight row byte
// offset per 16-row group (with this wave's k slice) and a token-row byte
// offset per pass (token rows for gate/up, intermediate rows for down).
template <int RG, int P>
struct RingWork {
  __amdgpu_buffer_rsrc_t wr, xr;
  uint32_t woff[RG];
  uint32_t xoff[P];
  int npass;
};

// Item g of a task: token group g / SUB and, for tasks streamed as SUB
// sequential row sub-groups, sub-group g % SUB.  Only sub-group 0 loads the
// token rows; the later ones reuse the wave's copy of them.
template <int RG, int P, int SUB>
__device__ __forceinline__ RingWork<RG, P> ring_work(const ExpertArgs &a, const RingShared &sh,
                                                     const RingRsrc &rr, const RingTask &t, int g,
                                                     int w) {
  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  RingWork<RG, P> r;
  r.wr = rr.none;
  r.xr = rr.none;
  r.npass = 0;
#pragma unroll
  for (int gg = 0; gg < RG; ++gg) r.woff[gg] = kRingOff;
#pragma unroll
  for (int p = 0; p < P; ++p) r.xoff[p] = kRingOff;
  if (t.kind != 1 && t.kind != 2) return r;
  const int u = g % t.nsub;
  const int m0 = (g / t.nsub) * kRingTokens * P;
  // every wave writes partials for every pass of the group (zeros from a
  // slice past the end of the rows), so the control wave sums all eight
  r.npass = min(P, (t.cnt - m0 + kRingTokens - 1) / kRingTokens);
  const int K = t.kind == 1 ? a.H : a.I;
  const int k0 = w * kRingSlice;
  if (k0 >= K) return r;  // this wave's slice is past the end of the rows
  const int kl = k0 + 4 * lg;
  if (t.kind == 1) {
    // MFMA row li of group gg: W1 row col + 8gg + li (li < 8) or the W3 row
    // of the same column, packed [I/32][2][32][H] so the two are 32 rows apart
#pragma unroll
    for (int gg = 0; gg < RG; ++gg) {
      const int n = t.col + 8 * (u * RG + gg) + (li & 7);
      const uint32_t prow = (uint32_t)(n >> 5) * 64 + (li >= 8 ? 32 : 0) + (n & 31);
      r.woff[gg] = (((uint32_t)t.e * 2 * a.I + prow) * (uint32_t)a.H + kl) * 4u;
    }
    r.wr = rr.w13;
    r.xr = rr.x;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int m = m0 + p * kRingTokens + li;
      if (m < t.cnt) {
        const int s = min(t.slot0 + m, kRingMaxSlots - 1);  // plans here have T * 4 <= kRingMaxSlots
        int tk = sh.tok[s];
        tk = tk < 0 ? 0 : (tk >= a.T ? a.T - 1 : tk);
        r.xoff[p] = ((uint32_t)tk * a.H + kl) * 4u;
      }
    }
  } else {
#pragma unroll
    for (int gg = 0; gg < RG; ++gg)
      r.woff[gg] = (((uint32_t)t.e * a.H + t.col + 16 * (u * RG + gg) + li) * (uint32_t)a.I + kl) * 4u;
    r.wr = rr.w2;
    r.xr = rr.inter;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int m = m0 + p * kRingTokens + li;
      if (m < t.cnt) r.xoff[p] = ((uint32_t)(t.slot0 + m) * a.I + kl) * 4u;
    }
  }
  if (u != 0) {
    r.xr = rr.none;
#pragma unroll
    for (int p = 0; p < P; ++p) r.xoff[p] = kRingOff;
  }
  return r;
}

// One ring step's loads (each row group's weights + every pass's token or
// intermediate rows) into one slot.  Both row kinds use the default cache
// policy, so rows that many tasks share (an expert's tokens or intermediate
// values) come from the XCD's L2 after the first read.  Intermediate rows are
// written by other blocks during the kernel, but each of their values is only
// ever kUnwritten (the router's fill) or final, and caches start the kernel
// invalidated: a load returns either the final value or kUnwritten, possibly
// a stale cached kUnwritten, and ring_await then reloads coherently (sc1).
// Token and intermediate loads are one instruction, so the compiler's wait
// counts stay exact whichever kind a task is.
template <int RG, int P>
__device__ __forceinline__ void ring_issue(const RingWork<RG, P> &r, int s, f32x4 (&wt)[RG],
                                           f32x4 (&xv)[P]) {
#pragma unroll
  for (int gg = 0; gg < RG; ++gg)
    wt[gg] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r.wr, r.woff[gg] + s * 64, 0, 0));
#pragma unroll
  for (int p = 0; p < P; ++p)
    xv[p] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r.xr, r.xoff[p] + s * 64, 0, 0));
}

template <int N>
__device__ __forceinline__ bool any_unwritten(const f32x4 (&v)[N]) {
  bool bad = false;
#pragma unroll
  for (int n = 0; n < N; ++n)
#pragma unroll
    for (int i = 0; i < 4; ++i) bad |= __builtin_bit_cast(uint32_t, v[n][i]) == kUnwritten;
  return __builtin_amdgcn_ballot_w64(bad) != 0;  // wave-uniform
}

// Step s of a down task read intermediate values not yet written: reload
// the step's rows (coherently) until every value has landed, then load the
// rows of the steps already in flight again, since they were issued no later
// and are likely stale too (their weights are not reloaded).  False if the
// block aborts; a wait longer than `ticks` reports a device timeout and
// aborts the block.
template <int RG, int P, int D>
__device__ __forceinline__ bool ring_await(const RingWork<RG, P> &r, int s, f32x4 (&wt)[D][RG],
                                           f32x4 (&xv)[D][P], int *abort_flag, int *err,
                                           long long ticks) {
  const long long t0 = ring_now();
  const int sl = s % D;
  do {
    if (__builtin_amdgcn_readfirstlane(lds_load(abort_flag))) return false;
    if (ring_now() - t0 > ticks) {
      if ((threadIdx.x & 63) == 0) {
        st_agent(err, 1);
        lds_store(abort_flag, 1);
      }
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int p = 0; p < P; ++p)
      xv[sl][p] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(r.xr, r.xoff[p] + s * 64, 0, kCachePolicySc1));
  } while (any_unwritten<P>(xv[sl]));
#pragma unroll
  for (int d = 1; d < D; ++d)
    if (s + d < kRingSteps) {
#pragma unroll
      for (int p = 0; p < P; ++p)
        xv[(s + d) % D][p] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(r.xr, r.xoff[p] + (s + d) * 64, 0, kCachePolicySc1));
    }
  return true;
}

// A token's routing: slots of its four expert rows (-1: no expert in that
// rank, which a token whose scores are NaN or <= -1e30 leaves empty) and
// their weights.
struct RingRoute {
  int slot[kTopK];
  float w[kTopK];
};

__device__ __forceinline__ RingRoute ring_route(const ExpertArgs &a, const RingShared &sh, int tok) {
  RingRoute r;
  const bool local = sh.local != 0;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    int slot = local ? sh.rpos[tok][k] : a.s.pos[(size_t)tok * kTopK + k];
    float w = local ? sh.rw[tok][k] : a.s.wts[(size_t)tok * kTopK + k];
    if (slot < 0 || slot >= a.T * kTopK) {
      slot = -1;
      w = 0.0f;
    }
    r.slot[k] = slot;
    r.w[k] = w;
  }
  return r;
}

// Chain jobs of a certified decode routing (Ctrl::deferred == 2): job j
// stores the gate logits of experts 4j..4j+3 for the batch's <= 8 tokens,
// with chain_dot's arithmetic (the reference's FMA order), and counts itself
// in chain_done once its stores are complete.  Blocks claim jobs as they
// start; a job never waits, so every claimed job ends.
//
// Block form: every thread of the block calls it; the operands are staged in
// the block's partial buffers (free until it streams) with direct-to-LDS
// loads and wave 0 runs one chain per (token, expert) lane.  The block that
// completes the last job routes every token from the logits at once
// (route_token_block) and publishes idx and w, so the combine finds them
// (each block maps an expert to its slot with its own plan); rsh serves as
// scratch (sh.bias must be loaded).
__device__ __forceinline__ void ring_chain_job(const ExpertArgs &a, RingShared &sh,
                                               RouteShared &rsh, int *s_flag, int j,
                                               float *lds) {
  const int T = a.T, H = a.H, P = H + 4, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  float *gs = lds, *xs = lds + kDecEPB * P;
  const int e0 = j * kDecEPB, nch = H >> 8, items = (kDecEPB + T) * nch;
  for (int i = wave; i < items; i += kRingThreads / 64) {
    const int r = i / nch, ch = i % nch;
    const float *src = (r < kDecEPB ? a.w.gate + (size_t)(e0 + r) * H
                                    : a.x + (size_t)(r - kDecEPB) * H) + ch * 256 + lane * 4;
    float *dst = (r < kDecEPB ? gs + r * P : xs + (r - kDecEPB) * P) + ch * 256;
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (wave == 0) {
    const int tl = lane >> 2, el = lane & 3;
    const float acc = chain_dot(gs + el * P, xs + min(tl, T - 1) * P, H);
    if (tl < T) st_agent(&a.s.logits[(size_t)tl * kExperts + e0 + el], acc);
    __builtin_amdgcn_s_waitcnt(0);  // the logits are stored
    if (lane == 0) *s_flag = fetch_add(&a.s.ctrl->chain_done, 1) == kChainJobs - 1;
  }
  __syncthreads();  // the staging buffers are free again
  if (*s_flag) {
    // the other jobs' logits: stored before they counted in, read with
    // agent-scope loads
    const int tl = (tid >> 5) & (kDecRT - 1);
    const float l = tid < kDecRT * kExperts && tl < T
                        ? __hip_atomic_load(&a.s.logits[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                        : 0.0f;
    route_token_block(rsh, T, sh.bias, l);
    if (tid < T * kTopK) {
      const int t = tid / kTopK, k = tid % kTopK;
      st_agent(&a.s.idx[tid], rsh.ti[t][k]);
      st_agent(&a.s.wts[tid], rsh.tw[t][k]);
    }
    __syncthreads();
  }
}

// Wave form, for a wave that waits for the logits while a job is still
// unclaimed: the same chains with their operands read from global memory
// (slow, but it lets a wait finish when blocks that have not started hold
// the job).
__device__ __forceinline__ void ring_chain_job_wave(const ExpertArgs &a, int j) {
  const int T = a.T, H = a.H, lane = threadIdx.x & 63;
  const int tl = lane >> 2, el = lane & 3, e = j * kDecEPB + el;
  const float acc = chain_dot(a.w.gate + (size_t)e * H, a.x + (size_t)min(tl, T - 1) * H, H);
  if (tl < T) st_agent(&a.s.logits[(size_t)tl * kExperts + e], acc);
  __builtin_amdgcn_s_waitcnt(0);
  if (lane == 0) fetch_add(&a.s.ctrl->chain_done, 1);
}

// A token's routing once its logits are stored (certified decode routing):
// the calling wave waits for every chain job (running unclaimed ones
// itself), then computes the token's top-4 in rank order and weights with
// route_token_block's arithmetic (lane e: expert e; lanes 32-63 repeat
// lanes 0-31).  The slots come from the block's plan of the experts the
// score bounds left possible, which must hold every expert of the exact
// top-4 (else the status word reads 2 and the block aborts).  Wave 0
// publishes the token's idx and weights.  False if the block aborts or the
// wait times out.
__device__ __forceinline__ bool ring_route_exact(const ExpertArgs &a, RingShared &sh, int tok,
                                                 RingRoute *out, int *abort_flag, int *err,
                                                 long long ticks) {
#pragma clang fp contract(off)
  Ctrl *ctrl = a.s.ctrl;
  const int lane = threadIdx.x & 63, e = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (__builtin_amdgcn_readfirstlane(load_relaxed(&ctrl->chain_done)) < kChainJobs) {
    const long long t0 = ring_now();
    while (__builtin_amdgcn_readfirstlane(load_relaxed(&ctrl->chain_done)) < kChainJobs) {
      if (__builtin_amdgcn_readfirstlane(lds_load(abort_flag))) return false;
      if (ring_now() - t0 > ticks) {
        if (lane == 0) {
          st_agent(err, 1);
          lds_store(abort_flag, 1);
        }
        return false;
      }
      int j = kChainJobs;
      if (__builtin_amdgcn_readfirstlane(load_relaxed(&ctrl->chain_head)) < kChainJobs) {
        j = lane == 0 ? claim(&ctrl->chain_head) : 0;
        j = __builtin_amdgcn_readfirstlane(j);
      }
      if (j < kChainJobs) ring_chain_job_wave(a, j);
      else __builtin_amdgcn_s_sleep(1);
    }
  }
  // agent-scope loads of logits whose stores completed before their jobs
  // counted in (no acquire fence needed)
  const float l = __hip_atomic_load(&a.s.logits[(size_t)tok * kExperts + e], __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
  const float p = ref_sigmoid(l);
  const float sc = p + sh.bias[e];
  int r = 0;
#pragma unroll
  for (int jx = 0; jx < kExperts; ++jx) {
    const float sj = __shfl(sc, jx, 32);
    r += (int)((sj > -1e30f) & ((sj > sc) | ((sj == sc) & (jx < e))));
  }
  const int sel = (sc > -1e30f && r < kTopK) ? r : -1;
  int ek[kTopK];
  float pk[kTopK];
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    const uint32_t m = (uint32_t)__ballot(sel == k);  // lanes 0-31
    ek[k] = m ? __builtin_ctz(m) : -1;
    pk[k] = m ? __shfl(p, ek[k], 64) : 0.0f;
  }
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) sum += pk[k];
  const float scale = (sum > 1e-6f) ? (1.0f / sum) : 1.0f;
  bool same = true;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    out->w[k] = pk[k] * scale * 1.0f;
    out->slot[k] = ek[k] >= 0 ? sh.slotmap[tok][ek[k]] : -1;
    same = same && (ek[k] < 0 || out->slot[k] >= 0);  // every expert has a planned slot
  }
  if (!same) {
    if (lane == 0) {
      st_agent(err, 2);
      lds_store(abort_flag, 1);
    }
    return false;
  }
  if (w == 0 && lane < kTopK) {
    int ev = ek[0];
    float wv = out->w[0];
#pragma unroll
    for (int k = 1; k < kTopK; ++k)
      if (lane == k) {
        ev = ek[k];
        wv = out->w[k];
      }
    st_agent(&a.s.idx[(size_t)tok * kTopK + lane], ev);
    a.s.wts[(size_t)tok * kTopK + lane] = wv;
  }
  return true;
}

// The token's routing as the block that finished the chain jobs published
// it (coherent loads; one round trip), each expert's slot from this block's
// plan, which must hold it (else the status word reads 2 and the block
// aborts); if it is not there yet, ring_route_exact.
__device__ __forceinline__ bool ring_route_planned(const ExpertArgs &a, RingShared &sh, int tok,
                                                   RingRoute *out, int *abort_flag, int *err,
                                                   long long ticks) {
  int ex[kTopK], sl[kTopK];
  float wv[kTopK];
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    const size_t i = (size_t)tok * kTopK + k;
    ex[k] = __hip_atomic_load(&a.s.idx[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wv[k] = __hip_atomic_load(&a.s.wts[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  bool there = true, same = true;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    there = there && ex[k] != kRouteUnset && __builtin_bit_cast(uint32_t, wv[k]) != kUnwritten;
    sl[k] = ex[k] >= 0 && ex[k] < kExperts ? sh.slotmap[tok][ex[k]] : -1;
    same = same && ex[k] < kExperts && (ex[k] < 0 || sl[k] >= 0);
  }
  if (!__builtin_amdgcn_readfirstlane((int)there))
    return ring_route_exact(a, sh, tok, out, abort_flag, err, ticks);
  if (!same) {
    if ((threadIdx.x & 63) == 0) {
      st_agent(err, 2);
      lds_store(abort_flag, 1);
    }
    return false;
  }
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    out->slot[k] = sl[k];
    out->w[k] = wv[k];
  }
  return true;
}

// Combine of token tok by the 512 threads of the streaming waves (thread ts:
// float4 columns ts, ts + 512, ...), with the arithmetic of tile_combine:
// FMA chain over k ascending, then the residual.  The expert outputs are
// loaded coherently and reloaded while any is still kUnwritten.  y may alias
// the residual: each thread reads its columns before it writes them.  False
// if the block aborts or the wait times out.
__device__ bool ring_combine(const ExpertArgs &a, int tok, const RingRoute &r, int ts,
                             int *abort_flag, int *err, long long ticks) {
#pragma clang fp contract(off)
  const int H4 = a.H >> 2;
  const __amdgpu_buffer_rsrc_t so =
      __builtin_amdgcn_make_buffer_rsrc(a.s.sout, 0, (int)a.s.sout_bytes, kBufferRsrcWord3);
  const float4 *r4 = reinterpret_cast<const float4 *>(a.residual);
  float4 *y4 = reinterpret_cast<float4 *>(a.y);
  for (int c4 = ts; c4 < H4; c4 += kRingWaves * 64) {
    f32x4 v[kTopK];
    uint32_t off[kTopK];
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
      // an empty rank reads past the buffer: zeros, never kUnwritten
      off[k] = r.slot[k] >= 0 ? ((uint32_t)r.slot[k] * (uint32_t)H4 + (uint32_t)c4) * 16u : kRingOff;
      v[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(so, off[k], 0, kCachePolicySc1));
    }
    const float4 rv = r4 ? r4[(size_t)tok * H4 + c4] : make_float4(0.f, 0.f, 0.f, 0.f);
    if (any_unwritten<kTopK>(v)) {
      const long long t0 = ring_now();
      do {
        if (__builtin_amdgcn_readfirstlane(lds_load(abort_flag))) return false;
        if (ring_now() - t0 > ticks) {
          if ((threadIdx.x & 63) == 0) {
            st_agent(err, 1);
            lds_store(abort_flag, 1);
          }
          return false;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < kTopK; ++k)
          v[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(so, off[k], 0, kCachePolicySc1));
      } while (any_unwritten<kTopK>(v));
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
      if (r.slot[k] < 0) continue;  // layer.cu:708-720 sums the selected experts only
      acc.x = __builtin_fmaf(v[k].x, r.w[k], acc.x);
      acc.y = __builtin_fmaf(v[k].y, r.w[k], acc.y);
      acc.z = __builtin_fmaf(v[k].z, r.w[k], acc.z);
      acc.w = __builtin_fmaf(v[k].w, r.w[k], acc.w);
    }
    if (r4) {
      acc.x = rv.x + acc.x;
      acc.y = rv.y + acc.y;
      acc.z = rv.z + acc.z;
      acc.w = rv.w + acc.w;
    }
    y4[(size_t)tok * H4 + c4] = acc;
  }
  return true;
}

// Partials of item i: res[i & 1][wave][row group][pass][row][token], 16 x 16.
template <int RG, int P>
__device__ __forceinline__ float *ring_res(float *res, int b, int w, int gg, int p) {
  return res + (((((size_t)b * kRingWaves + w) * RG + gg) * P + p) * kRingTokens * kRingTokens);
}

// Streaming side: RG row groups of 16 rows share every token-row load; with
// one group two accumulators per pass break the MFMA dependency chain.  With
// SUB > 1 a task's SUB * RG row groups are streamed as SUB items one after
// another (the access pattern of a 16-row task, which streams faster than
// several row groups read at once), and each wave keeps the token slice that
// sub-group 0 loaded in registers (xt) for the later sub-groups.
template <int RG, int P, int SUB>
__device__ void ring_streamer(const ExpertArgs &a, RingShared &sh, float *res, const RingPlan &pl,
                              long long ticks) {
  constexpr int NA = RG == 1 ? 2 : 1;
  constexpr int D = ring_depth(RG, P);
  static_assert(kRingSteps % D == 0, "ring rotation realigns at task boundaries");
  static_assert(D < kRingSteps - D - 1, "the next task is published before it is read");
  int *err = &a.s.ctrl->err;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const RingRsrc rr = ring_rsrc(a);
  const RingTask none{4, 0, 0, 0, 0, 0, 0, 1, 1};
  f32x4 wt[D][RG];
  f32x4 xv[D][P];
  f32x4 xt[SUB > 1 ? kRingSteps : 1][P];  // token slice of the task's current group
  int j = 0, g = 0, it = 0;  // task, item within it, item counter
  RingTask t = ring_seq_task<P>(sh, pl, 0);
  RingWork<RG, P> cur = ring_work<RG, P, SUB>(a, sh, rr, t, 0, w);
  bool ok = true;
  // in step order: the first step's MFMAs then wait only for the first
  // step's loads (the scheduler would otherwise issue them last)
#pragma unroll
  for (int s = 0; s < D; ++s) {
    ring_issue<RG, P>(cur, s, wt[s], xv[s]);
    __builtin_amdgcn_sched_barrier(0);
  }
  // the queue counter, claimed by lane 0 only (other lanes' offsets are out
  // of range: no-ops that return 0) without a divergent branch
  const __amdgpu_buffer_rsrc_t cr =
      __builtin_amdgcn_make_buffer_rsrc(a.s.ctrl, 0, (int)sizeof(Ctrl), kBufferRsrcWord3);
  const uint32_t claim_off = lane == 0 ? (uint32_t)offsetof(Ctrl, head) : kRingOff;
  int claimed = 0;
  while (ok && t.kind != 4) {
    // Issue priority: the control wave's flushes are on every reader's path
    // (highest, set in ring_role); a gate/up task produces what down tasks
    // read; and of the two streaming waves that share a SIMD's MFMA unit the
    // younger would otherwise trail the older by up to a whole task.
    if (t.kind == 1) {
      if (w >= kRingWaves / 2) __builtin_amdgcn_s_setprio(2);
      else __builtin_amdgcn_s_setprio(1);
    } else {
      if (w >= kRingWaves / 2) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    // Wave 0 claims the block's next task as this one starts.  Loads
    // complete in issue order, so the reply has arrived by the time step D's
    // weights have, and the id is published then, well before the waves
    // need it to issue the next task's loads.
    const bool claim_now = w == 0 && g == 0;
    if (claim_now) claimed = __builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(1, cr, claim_off, 0, 0);
    int jn = j, gn = g + 1;
    const bool fresh = g % t.nsub == 0;  // this item loads the token rows
    RingTask tn = t;
    RingWork<RG, P> nxt;
    f32x4 acc[RG][P][NA];
#pragma unroll
    for (int gg = 0; gg < RG; ++gg)
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int n = 0; n < NA; ++n) acc[gg][p][n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kRingSteps; ++s) {
      const int sl = s % D;
      // a down task's intermediate values were loaded up to D steps earlier,
      // possibly before they had landed
      if (t.kind == 2 && any_unwritten<P>(xv[sl]) && ok)
        ok = ring_await<RG, P, D>(cur, s, wt, xv, &sh.abort, err, ticks);
#pragma unroll
      for (int p = 0; p < P; ++p) {
        if (p < cur.npass) {
          f32x4 xo = xv[sl][p];
          if constexpr (SUB > 1) {
            xo = fresh ? xo : xt[s][p];
            xt[s][p] = xo;
          }
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int gg = 0; gg < RG; ++gg)
              acc[gg][p][q % NA] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                  wt[sl][gg][q], xo[q], acc[gg][p][q % NA], 0, 0, 0);
        }
      }
      if (s == D && claim_now) {
        if (lane == 0) lds_store(&sh.seq[(j + 1) & 7], claimed);
        release_lds();
        if (lane == 0) lds_store(&sh.nseq, j + 2);
      }
      if (s == kRingSteps - D - 1) {
        // the next group's rows are about to be issued
        if (gn >= t.ngroups * t.nsub) {
          jn = j + 1;
          gn = 0;
          if (ok) ok = ring_wait(&sh.nseq, [&](int v) { return v >= j + 2; }, &sh.abort, err, ticks);
          tn = ok ? ring_seq_task<P>(sh, pl, jn) : none;
        }
        nxt = ring_work<RG, P, SUB>(a, sh, rr, ok ? tn : none, gn, w);
      }
      if (s + D < kRingSteps) ring_issue<RG, P>(cur, s + D, wt[sl], xv[sl]);
      else ring_issue<RG, P>(nxt, s + D - kRingSteps, wt[sl], xv[sl]);
    }
    if (ok) {
      // partials of item it into buffer it & 1, once item it - 2 is consumed
      ok = ring_wait(&sh.flushed, [&](int v) { return v >= it - 1; }, &sh.abort, err, ticks);
      if (ok) {
        const int b = it & 1;
#pragma unroll
        for (int gg = 0; gg < RG; ++gg) {
#pragma unroll
          for (int p = 0; p < P; ++p) {
            if (p < cur.npass) {
              float *r = ring_res<RG, P>(res, b, w, gg, p);
              f32x4 v = acc[gg][p][0];
              if (NA == 2) v += acc[gg][p][NA - 1];
#pragma unroll
              for (int i = 0; i < 4; ++i) r[(4 * lg + i) * kRingTokens + li] = v[i];
            }
          }
        }
        release_lds();
        if (lane == 0) __hip_atomic_fetch_add(&sh.done[b], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      ++it;
    }
    j = jn;
    g = gn;
    t = tn;
    cur = nxt;
  }
  // combine tasks (one token each), after every row task, with the ring's
  // registers free
  for (int tok = blockIdx.x; ok && tok < pl.ncomb; tok += pl.grid) {
    RingRoute r;
    if (sh.local == 2) ok = ring_route_planned(a, sh, tok, &r, &sh.abort, err, ticks);
    else r = ring_route(a, sh, tok);
    if (ok) ok = ring_combine(a, tok, r, (int)threadIdx.x, &sh.abort, err, ticks);
  }
}

// Control side: sums the 8 k-slice partials of item (t, g) and stores the
// outputs with 16-byte agent-scope stores (gate/up: silu(W1 x) * (W3 x) for
// 8 columns per row group; down: 16 columns per row group).
template <int RG, int P, int SUB>
__device__ __forceinline__ void ring_flush(const ExpertArgs &a, const RingTask &t, int g,
                                           const float *res, int b, const AgentOut &inter_out,
                                           const AgentOut &sout_out) {
  const int lane = threadIdx.x & 63;
  const int u = g % t.nsub;  // row sub-group of the item
  const int m0 = (g / t.nsub) * kRingTokens * P;
  const int nt = min(kRingTokens * P, t.cnt - m0);
  // gate/up: lane -> (token, 4 columns): 2 lanes per token and row group;
  // down: 4 lanes
  const int per = t.kind == 1 ? 2 : 4;
  for (int f = lane; f < nt * per * RG; f += 64) {
    const int gg = f / (nt * per), fr = f % (nt * per);
    const int m = fr / per, q = fr % per;
    const int p = m / kRingTokens, mt = m % kRingTokens;
    f32x4 o;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int c = q * 4 + jj;
      if (t.kind == 1) {
        float gs = 0.f, us = 0.f;
#pragma unroll
        for (int w = 0; w < kRingWaves; ++w) {
          const float *r = ring_res<RG, P>(const_cast<float *>(res), b, w, gg, p);
          gs += r[c * kRingTokens + mt];
          us += r[(8 + c) * kRingTokens + mt];
        }
        o[jj] = silu(gs) * us;
      } else {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < kRingWaves; ++w)
          s += ring_res<RG, P>(const_cast<float *>(res), b, w, gg, p)[c * kRingTokens + mt];
        o[jj] = s;
      }
    }
    const int slot = t.slot0 + m0 + m;
    if (t.kind == 1)
      inter_out.store((uint32_t)(((size_t)slot * a.I + t.col + 8 * (u * RG + gg) + q * 4) * sizeof(float)), o);
    else
      sout_out.store((uint32_t)(((size_t)slot * a.H + t.col + 16 * (u * RG + gg) + q * 4) * sizeof(float)), o);
  }
}

// Control side: flushes every item whose eight partials are complete, in
// order, and ends once the block's last row task is flushed.  It never waits
// for its stores: their readers wait for the values themselves.
template <int RG, int P, int SUB>
__device__ void ring_control(const ExpertArgs &a, RingShared &sh, const float *res,
                             const RingPlan &pl) {
  Ctrl *c = a.s.ctrl;
  const int lane = threadIdx.x & 63;
  const AgentOut inter_out(a.s.inter, a.s.inter_bytes), sout_out(a.s.sout, a.s.sout_bytes);
  const long long ticks = (long long)a.wait_limit * kRingTicksPerLimit;
  int j = 0, g = 0, it = 0;  // next item to flush
  RingTask t = ring_seq_task<P>(sh, pl, 0);
  long long last = ring_now();
  while (t.kind != 4) {
    int flushed_now = 0;
    while (t.kind != 4) {
      const int b = it & 1;
      if (__builtin_amdgcn_readfirstlane(lds_load(&sh.done[b])) != kRingWaves) break;
      acquire_lds();
      ring_flush<RG, P, SUB>(a, t, g, res, b, inter_out, sout_out);
      lds_store(&sh.done[b], 0);
      ++it;
      ++flushed_now;
      if (++g >= t.ngroups * t.nsub) {
        g = 0;
        ++j;
        t = ring_seq_task<P>(sh, pl, j);  // published before task j - 1's partials
      }
      if (flushed_now == 2) break;
    }
    if (flushed_now) {
      // partials are read: the streaming waves may reuse the buffers
      release_lds();
      if (lane == 0) lds_store(&sh.flushed, it);
      last = ring_now();
    } else {
      if (__builtin_amdgcn_readfirstlane(lds_load(&sh.abort))) break;
      if (ring_now() - last > ticks) {
        if (lane == 0) {
          st_agent(&c->err, 1);
          lds_store(&sh.abort, 1);
        }
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
}

// LDS of the partials: [2][kRingWaves][row groups][passes][16][16]
constexpr size_t ring_res_bytes(int rg, int p) {
  return (size_t)2 * kRingWaves * rg * p * kRingTokens * kRingTokens * sizeof(float);
}

template <int RG, int P, int SUB = 1>
__device__ __forceinline__ void ring_role(const ExpertArgs &a, RingShared &sh, float *res,
                                          const RingPlan &pl, long long ticks) {
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) == kRingWaves) {  // uniform branch per wave
    __builtin_amdgcn_s_setprio(3);  // above every streaming wave
    ring_control<RG, P, SUB>(a, sh, res, pl);
  } else {
    ring_streamer<RG, P, SUB>(a, sh, res, pl, 2 * ticks);
  }
}

// Counts of a decode token block (rsh.cnt) -> the block's expert table (sh),
// its active-expert count and largest count; block 0 also publishes them
// for moe_last_routing.  Lanes 0-31 of wave 0.
__device__ __forceinline__ void ring_expert_table(const ExpertArgs &a, RingShared &sh,
                                                  const RouteShared &rsh, bool pub, int *s_nact,
                                                  int *s_maxcnt) {
  const int tid = threadIdx.x;
  if (tid >= kExperts) return;
  const int cnt = rsh.cnt[tid];
  int total = 0;
  const int off = lane_scan32(cnt, tid, &total);
  int mc = cnt;
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) mc = max(mc, __shfl_xor(mc, o, 32));
  const unsigned long long act = __ballot(cnt > 0);
  const int nact = __popcll(act);
  const int aidx = __popcll(act & ((1ull << tid) - 1ull));
  sh.counts[tid] = cnt;
  sh.offsets[tid] = off;
  if (cnt > 0) sh.active[aidx] = tid;
  if (tid >= nact) sh.active[tid] = -1;
  if (tid == 0) {
    *s_nact = nact;
    *s_maxcnt = mc;
  }
  if (pub) {
    Ctrl *cw = a.s.ctrl;
    cw->counts[tid] = cnt;
    cw->offsets[tid] = off;
    if (cnt > 0) cw->active[aidx] = tid;
    if (tid >= nact) cw->active[tid] = -1;
    if (tid == 0) {
      cw->offsets[kExperts] = total;
      cw->n_active = nact;
      cw->max_count = mc;
    }
  }
}

template <int KCH1, int KCH2>
__global__ __launch_bounds__(kRingThreads) void expert_ring_kernel(ExpertArgs a) {
  static_assert(KCH1 * 256 <= kRingWaves * kRingSlice && KCH2 * 256 <= kRingWaves * kRingSlice,
                "row length");
  static_assert((size_t)(kDecEPB + kDecRT) * (KCH1 * 256 + 4) * sizeof(float) <=
                    ring_res_bytes(kRingWideGroups, kRingMaxPasses),
                "a chain job's operands fit the partial buffers");
  // partials, ring_res_bytes(row groups, passes); 16-byte aligned for the
  // chain jobs' float4 reads
  extern __shared__ __align__(16) float res[];
  __shared__ RingShared sh;
  __shared__ RouteShared rsh;  // deferred routing only
  __shared__ int s_nact, s_maxcnt, s_job, s_fin, s_notok;
  const Ctrl *c = a.s.ctrl;
  const int tid = threadIdx.x;
  // 2: the router wrote score bounds, and the logits are this kernel's chain
  // jobs (0: the router routed and planned)
  const int mode = c->deferred;
  const bool local = mode == 2;
  if (tid < 2) sh.done[tid] = 0;
  // Chain jobs (mode 2) go to the first of blocks 0..kChainClaimBlocks-1 to
  // start, which claim their first row task after the job (a row task held
  // through a job would hold up its expert's down tasks); the other blocks
  // claim a row task at once and leave the chain-job counter alone (claims
  // on one cache line serialise).  Jobs that blocks 0..15 leave unclaimed are
  // run by the waits that need them.
  const bool chain_try = mode == 2 && !c->chain_lazy && blockIdx.x < kChainClaimBlocks;
  if (tid == 0) {
    sh.flushed = 0;
    sh.abort = 0;
    sh.local = local ? 1 : 0;
    s_notok = 0;
    const int job = chain_try ? claim(&a.s.ctrl->chain_head) : kChainJobs;
    s_job = job;
    // every task, the first included, is claimed from the queue, so only a
    // block that is running owns one (blocks not yet resident own nothing
    // another block waits for)
    if (chain_try && job >= kChainJobs) sh.seq[0] = claim(&a.s.ctrl->head);
    sh.nseq = 1;
  }
  // Other blocks claim their first row task now and store it only after the
  // plan: 256 blocks' first claims on one counter serialise (a reply came
  // back up to ~4 us after the block started), and the plan's barriers
  // order LDS only (lds_barrier), so the claim's round trip overlaps it.
  // Wave 4, which loads nothing for the plan (a wait for a later load would
  // wait for the claim too: loads complete in issue order), issues it with
  // its first lane's offset the only one in range (the other lanes' are
  // no-ops), so nothing waits for it before its use.
  constexpr int kClaimWave0 = kDecRT * kExperts;  // the first thread past the plan's pairs
  static_assert(kClaimWave0 % 64 == 0 && kClaimWave0 + 64 <= kRingThreads, "a wave of its own");
  int first_task = 0;
  if (!chain_try && tid >= kClaimWave0 && tid < kClaimWave0 + 64) {
    const __amdgpu_buffer_rsrc_t cr0 =
        __builtin_amdgcn_make_buffer_rsrc(a.s.ctrl, 0, (int)sizeof(Ctrl), kBufferRsrcWord3);
    first_task = __builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(
        1, cr0, tid == kClaimWave0 ? (uint32_t)offsetof(Ctrl, head) : kRingOff, 0, 0);
  }
  bool claim_late = false;  // the first row task is claimed after a chain job
  RingPlan pl;
  pl.ncomb = a.T;  // combine tasks: one per token
  pl.grid = gridDim.x;
  int maxcnt;
  if (local && (a.T < 1 || a.T > kDecRT)) {  // a deferred route covers one token block
    if (tid == 0) st_agent(&a.s.ctrl->err, 2);
    return;
  }
  if (local) {
    // One token block (T <= 8), 16-row tasks: every block plans the launch
    // itself, as the router's last block would (same functions, same order).
    // Slot = offsets[e] + in-block rank.
    const long long ticks = (long long)a.wait_limit * kRingTicksPerLimit;
    const int tl = (tid >> 5) & (kDecRT - 1), e = tid & (kExperts - 1);
    const bool pair = tid < kDecRT * kExperts;
    bool planned = false, chosen = false;
    float l = 0.0f;
    {
      // Expert e stays possible for a token unless four experts' lower
      // bounds exceed e's upper bound: then four experts beat e strictly,
      // whatever the logits' rounding, and the strict-'>' insertion of
      // layer.cu:465-476 cannot keep it.  So the possible set holds the
      // token's exact top-4; it is usually exactly the top-4, sometimes one
      // or two experts more (a 4th/5th score gap inside the bounds).  Every
      // possible expert gets a slot, and the combine, which needs the logits
      // (chain jobs) for the weights and the rank order anyway, uses the
      // exact top-4's.  The slots depend on the sets only, so the block
      // streams at once.
      float lo = 0.0f, hi = 0.0f;
      if (pair && tl < a.T) {
        lo = c->sbound[0][tl][e];
        hi = c->sbound[1][tl][e];
      }
      if (tid < kExperts) sh.bias[tid] = a.w.bias ? a.w.bias[tid] : 0.0f;
      lds_barrier();
      claim_late = s_job < kChainJobs;
      if (claim_late) ring_chain_job(a, sh, rsh, &s_fin, s_job, res);
      if (pair) rsh.prob[tl][e] = lo;
      lds_barrier();
      if (pair && tl < a.T) {
        int beat = 0;
#pragma unroll
        for (int j0 = 0; j0 < kExperts; j0 += 8) {
          float lv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) lv[j] = rsh.prob[tl][j0 + j];
#pragma unroll
          for (int j = 0; j < 8; ++j) beat += (int)(lv[j] > hi);
        }
        chosen = beat < kTopK;
      }
      const int half = (tid & 63) >> 5;
      const uint32_t gin = (uint32_t)(__ballot(chosen) >> (32 * half));
      const bool tok_ok = !pair || tl >= a.T || __popc(gin) <= kSpecSlots;
      if (!tok_ok) s_notok = 1;
      lds_barrier();
      planned = s_notok == 0;
      if (!planned) {
        // a token with more than kSpecSlots possible experts (non-finite
        // inputs or bias): run the chain jobs nobody has claimed, wait for
        // the others (all claimed by running blocks, and a job never
        // waits), then route from the logits
        for (;;) {
          // a read first: most blocks find every job claimed and take no
          // atomic on the counter
          if (tid == 0)
            s_job = load_relaxed(&a.s.ctrl->chain_head) < kChainJobs ? claim(&a.s.ctrl->chain_head)
                                                                      : kChainJobs;
          __syncthreads();
          const int j = s_job;
          __syncthreads();
          if (j >= kChainJobs) break;
          ring_chain_job(a, sh, rsh, &s_fin, j, res);
        }
        if (tid == 0) {
          const long long t0 = ring_now();
          while (load_relaxed(&a.s.ctrl->chain_done) < kChainJobs) {
            if (ring_now() - t0 > ticks) {
              st_agent(&a.s.ctrl->err, 1);
              sh.abort = 1;
              break;
            }
            __builtin_amdgcn_s_sleep(8);
          }
        }
        __syncthreads();
        if (sh.abort) return;
        // the logits' stores completed before their jobs counted in, and
        // agent-scope loads read them from the coherent level: no acquire
        // fence (each one invalidates the XCD's L2, 256 of them cost ~15 us)
        if (pair && tl < a.T)
          l = __hip_atomic_load(&a.s.logits[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (planned) {
      // per-expert counts and each possible pair's rank among the block's
      // tokens
      if (pair) rsh.sel[tl][e] = chosen ? 1 : 0;
      lds_barrier();
      int before = 0;
      if (pair && tl < a.T) {
        int all = 0;
#pragma unroll
        for (int t2 = 0; t2 < kDecRT; ++t2) {
          const int ch = rsh.sel[t2][e];
          before += ch & (t2 < tl);
          all += ch;
        }
        if (tl == 0) rsh.cnt[e] = all;
      }
      lds_barrier();
      ring_expert_table(a, sh, rsh, blockIdx.x == 0, &s_nact, &s_maxcnt);
      lds_barrier();
      if (pair) {
        const int slot = chosen ? sh.offsets[e] + before : -1;
        sh.slotmap[tl][e] = slot;
        if (slot >= 0) {
          sh.tok[slot] = tl;
          if (blockIdx.x == 0) st_agent(&a.s.slot_token[slot], tl);
        }
      }
      if (tid == 0) sh.local = 2;  // the combine routes each token from its logits
    } else {
      route_token_block(rsh, a.T, sh.bias, l);
      ring_expert_table(a, sh, rsh, blockIdx.x == 0, &s_nact, &s_maxcnt);
      __syncthreads();
      if (tid < a.T * kTopK) {
        const int t = tid / kTopK, k = tid % kTopK;
        const int ex = rsh.ti[t][k];
        const int slot = ex >= 0 ? sh.offsets[ex] + rsh.rank[t][k] : -1;
        if (slot >= 0) sh.tok[slot] = t;
        sh.rpos[t][k] = slot;
        sh.rw[t][k] = rsh.tw[t][k];
        if (blockIdx.x == 0) {
          st_agent(&a.s.idx[tid], ex);
          a.s.wts[tid] = rsh.tw[t][k];
          st_agent(&a.s.pos[tid], slot);
          if (slot >= 0) st_agent(&a.s.slot_token[slot], t);
        }
      }
    }
    lds_barrier();
    const int units = s_nact;  // read after the barrier above
    pl.rows = kStreamRows;
    pl.p1u = a.I / (kStreamRows / 2);
    pl.p2u = a.H / kStreamRows;
    pl.n1 = units * pl.p1u;
    pl.n2 = units * pl.p2u;
    pl.sub = 1;
    pl.tail_u0 = units;
    pl.tail_q = units * pl.p2u;
    maxcnt = __builtin_amdgcn_readfirstlane(s_maxcnt);
  } else {
    if (tid < kExperts) {
      sh.active[tid] = c->active[tid];
      sh.counts[tid] = c->counts[tid];
      sh.offsets[tid] = c->offsets[tid];
    }
    const int nslots = min(a.T * kTopK, kRingMaxSlots);
    for (int i = tid; i < nslots; i += kRingThreads) sh.tok[i] = a.s.slot_token[i];
    pl.n1 = c->n_p1;
    pl.n2 = c->n_p2;
    pl.p1u = c->p1_per_unit;
    pl.p2u = c->p2_per_unit;
    pl.rows = __builtin_amdgcn_readfirstlane(c->stream_rows);
    maxcnt = __builtin_amdgcn_readfirstlane(c->max_count);
    // 64-row tasks of experts holding at most 16 tokens are streamed as four
    // 16-row sub-groups; the router then plans the last units' down rows as
    // 16-row tasks (tail_units), so the last round of tasks is short
    const bool seq = pl.rows == kStreamRows * kRingWideGroups && maxcnt <= kRingTokens;
    pl.sub = seq ? kRingWideGroups : 1;
    {
      const int units = pl.n1 / max(pl.p1u, 1);
      const int tail = seq ? __builtin_amdgcn_readfirstlane(c->tail_units) : 0;
      pl.tail_u0 = units - tail;
      pl.tail_q = (units - tail) * pl.p2u;
    }
    // plans for this kernel take their slots from the router, and a task
    // covers 16, 32 or 64 rows
    if (c->n_rblocks != 0 ||
        (pl.rows != kStreamRows && pl.rows != kStreamRows * kRingWideGroups &&
         pl.rows != kStreamRows * kRingDenseGroups)) {
      if (tid == 0) st_agent(&a.s.ctrl->err, 2);
      return;
    }
  }
  if (claim_late && tid == 0) sh.seq[0] = claim(&a.s.ctrl->head);
  if (!chain_try && tid == kClaimWave0) sh.seq[0] = first_task;
  __syncthreads();
  const long long ticks = (long long)a.wait_limit * kRingTicksPerLimit;
  if (pl.rows == kStreamRows) {
    if (maxcnt <= kRingTokens) ring_role<1, 1>(a, sh, res, pl, ticks);
    else ring_role<1, kRingMaxPasses>(a, sh, res, pl, ticks);
  } else if (pl.rows == kStreamRows * kRingWideGroups) {
    if (maxcnt <= kRingTokens) ring_role<1, 1, kRingWideGroups>(a, sh, res, pl, ticks);
    else ring_role<kRingWideGroups, kRingMaxPasses>(a, sh, res, pl, ticks);
  } else {
    ring_role<kRingDenseGroups, kRingDensePasses>(a, sh, res, pl, ticks);
  }
}

// Streaming-kernel instantiations: (H/256, I/256) pairs it is compiled for.
#define MOE_STREAM_SHAPES(X) X(8, 7)

// ---------------------------------------------------------------------------
// Weight packing (once per set_weights)
// ---------------------------------------------------------------------------

// dst [I/32][2][32][H] from w1, w3 [I][H] of one expert.
__global__ void pack_w13_kernel(float4 *dst, const float4 *w1, const float4 *w3,
                                int H4, int I) {
  const size_t n = (size_t)2 * I * H4;
  for (size_t f = blockIdx.x * (size_t)blockDim.x + threadIdx.x; f < n;
       f += (size_t)gridDim.x * blockDim.x) {
    const size_t prow = f / H4, c4 = f % H4;
    const size_t g = prow / 64, w = (prow % 64) / 32, j = prow % 32;
    const size_t srow = g * 32 + j;
    dst[f] = (w == 0 ? w1 : w3)[srow * H4 + c4];
  }
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

// Router shapes: small T uses 8-token blocks with all 32 experts, so each of
// the 256 lanes runs one chain and a token block needs no hand-off between
// blocks; larger T uses 64-token blocks and 8 chains per lane.  The
// expert-split router (8 blocks per 8 tokens, one block per CU for its LDS)
// serves batches up to kSplitRouterTokens.
constexpr int kSmallRT = kDecRT, kSmallKC = 256;
constexpr int kLargeRT = 64, kLargeKC = 64;
// Larger T: the experts of a 64-token block are split over ES blocks while
// that keeps the grid within about one block per CU (T=4096: 64 token blocks
// x 4, router 90 -> 51 us; at T=16384 the unsplit 256 blocks are fastest).
constexpr int kSplitRouterTokens = 256;  // 505 vs 527 us per step at 256 tokens, 563 vs 545 at 384
static_assert(kBoundTokens <= kSplitRouterTokens && kBoundTokens / kDecRT <= kPlanLdsBlocks,
              "routing from bounds runs in the decode router, its bases in LDS");

int router_tokens_per_block(int T) { return T <= kSplitRouterTokens ? kSmallRT : kLargeRT; }

bool router_fuses_norm(int T) { return T <= kSplitRouterTokens; }

hipError_t launch_router_dense(const RouterArgs &a, hipStream_t st) {
  if (a.T <= 64) {
    // the weight-streaming plan adds blocks that prepare its rows
    const int nb = (a.T + kSmallRT - 1) / kSmallRT;
    const int grid = a.tile_rows == 0 ? nb * (1 + kDecES) : nb;
    hipLaunchKernelGGL(router_dense_kernel<kSmallRT>, dim3(grid), dim3(kThreads), 0, st, a);
  } else {
    const int nb = (a.T + kLargeRT - 1) / kLargeRT;
    hipLaunchKernelGGL(router_dense_kernel<kLargeRT>, dim3(nb), dim3(kThreads), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *h, const float *w, float *out, int T, int H, hipStream_t st) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((T + kNormRowsPerBlock - 1) / kNormRowsPerBlock),
                     dim3(kNormThreads), 0, st, h, w, out, T, H);
  return hipGetLastError();
}

hipError_t launch_router(const RouterArgs &a, bool from_logits, hipStream_t st) {
  const bool small = a.T <= 64;
  if (a.T <= kSplitRouterTokens && !from_logits) {
    const size_t lds = router_decode_lds(a.H);
    if (lds > 65536) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&router_decode_kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    // a deferred routing: blocks of up to kDeferBlockTokens tokens per
    // expert slice (router_decode_kernel's rtb), and kDeferFillBlocks more
    // blocks prepare the streaming kernel's rows
    const int rtb = router_block_tokens(a.defer, a.T);
    const int nb = (a.T + rtb - 1) / rtb;
    const int fill = a.defer == 2 ? kDeferFillBlocks : 0;
    hipLaunchKernelGGL(router_decode_kernel, dim3(nb * kDecES + fill), dim3(kThreads), lds, st, a);
    return hipGetLastError();
  }
  const int rt = small ? kSmallRT : kLargeRT;
  const int nb = (a.T + rt - 1) / rt;
  if (from_logits) {
    // no gate GEMM: one block per token block finishes routing directly
    if (small)
      hipLaunchKernelGGL((router_kernel<true, kSmallRT, 1, kSmallKC>), dim3(nb), dim3(kThreads), 0, st, a);
    else
      hipLaunchKernelGGL((router_kernel<true, kLargeRT, 1, kLargeKC>), dim3(nb), dim3(kThreads), 0, st, a);
  } else {
    if (nb <= 64)
      hipLaunchKernelGGL((router_kernel<false, kLargeRT, 4, 2 * kLargeKC>), dim3(nb * 4),
                         dim3(kThreads), 0, st, a);
    else if (nb <= 128)
      hipLaunchKernelGGL((router_kernel<false, kLargeRT, 2, kLargeKC>), dim3(nb * 2),
                         dim3(kThreads), 0, st, a);
    else
      hipLaunchKernelGGL((router_kernel<false, kLargeRT, 1, kLargeKC>), dim3(nb), dim3(kThreads),
                         0, st, a);
  }
  return hipGetLastError();
}

static size_t stream_lds_bytes() {
  const size_t a = ring_res_bytes(kRingWideGroups, kRingMaxPasses),
               b = ring_res_bytes(kRingDenseGroups, kRingDensePasses);
  return a > b ? a : b;
}

static const void *stream_fn(int H, int I) {
#define MOE_STREAM_CASE(K1, K2) \
  if (H == (K1)*256 && I == (K2)*256) return reinterpret_cast<const void *>(&expert_ring_kernel<K1, K2>);
  MOE_STREAM_SHAPES(MOE_STREAM_CASE)
#undef MOE_STREAM_CASE
  return nullptr;
}

bool stream_supported(int H, int I) { return stream_fn(H, I) != nullptr; }

int stream_max_tokens() { return kRingMaxSlots / kTopK; }

template <int BM> static void *mfma_fn() {
  return reinterpret_cast<void *>(&expert_mfma_kernel<BM>);
}

static hipError_t ensure_lds_attr(const void *fn, size_t bytes) {
  if (bytes <= 65536) return hipSuccess;
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)bytes);
}

hipError_t launch_experts(const ExpertArgs &a, int tile_rows, int grid,
                          hipStream_t st) {
  hipError_t err = hipSuccess;
  switch (tile_rows) {
    case 0: {
      const size_t lds = stream_lds_bytes();
      const void *fn = stream_fn(a.H, a.I);
      if (!fn) return hipErrorInvalidValue;
      err = ensure_lds_attr(fn, lds);
      if (err != hipSuccess) return err;
      void *args[] = {const_cast<ExpertArgs *>(&a)};
      err = hipLaunchKernel(fn, dim3(grid), dim3(kRingThreads), args, lds, st);
      if (err != hipSuccess) return err;
      break;
    }
    case 32: {
      const size_t lds = Tile<32>::LDS_FLOATS * sizeof(float);
      err = ensure_lds_attr(mfma_fn<32>(), lds);
      if (err != hipSuccess) return err;
      hipLaunchKernelGGL(expert_mfma_kernel<32>, dim3(grid), dim3(kThreads), lds, st, a);
      break;
    }
    case 64: {
      const size_t lds = Tile<64>::LDS_FLOATS * sizeof(float);
      err = ensure_lds_attr(mfma_fn<64>(), lds);
      if (err != hipSuccess) return err;
      hipLaunchKernelGGL(expert_mfma_kernel<64>, dim3(grid), dim3(kThreads), lds, st, a);
      break;
    }
    case 128: {
      const size_t lds = Tile<128>::LDS_FLOATS * sizeof(float);
      err = ensure_lds_attr(mfma_fn<128>(), lds);
      if (err != hipSuccess) return err;
      hipLaunchKernelGGL(expert_mfma_kernel<128>, dim3(grid), dim3(kThreads), lds, st, a);
      break;
    }
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

int stream_rows_dense(int T) {
  return T > 2 * kRingTokens ? kStreamRows * kRingDenseGroups : expert_bn(0, T);
}

bool router_can_bound(int T, int tile_rows, int H) {
  return T >= 1 && T <= kBoundTokens && (tile_rows == 32 || tile_rows == 64) && H % 256 == 0;
}

bool router_can_defer(int T, int tile_rows, int bn) {
  return T >= 1 && T <= kDecRT && T <= kSplitRouterTokens && tile_rows == 0 && bn == kStreamRows;
}

int expert_bn(int tile_rows, int T) {
  switch (tile_rows) {
    case 32: return Tile<32>::BN;
    case 64: return Tile<64>::BN;
    case 128: return Tile<128>::BN;
    // streaming: 64-row tasks once a batch has enough tokens per expert that
    // sharing each token-row load across 4 row groups pays
    default: return T >= kStreamWideTokens ? kStreamRows * kRingWideGroups : kStreamRows;
  }
}

int expert_blocks_per_cu(int tile_rows) {
  int n = 0;
  hipError_t e = hipSuccess;
  switch (tile_rows) {
    case 0: {
      const void *fn = stream_fn(2048, 1792);
      if (!fn) return 1;
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kRingThreads, stream_lds_bytes());
      break;
    }
    case 32:
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &n, mfma_fn<32>(), kThreads, Tile<32>::LDS_FLOATS * sizeof(float));
      break;
    case 64:
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &n, mfma_fn<64>(), kThreads, Tile<64>::LDS_FLOATS * sizeof(float));
      break;
    case 128:
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &n, mfma_fn<128>(), kThreads, Tile<128>::LDS_FLOATS * sizeof(float));
      break;
    default:
      return 1;
  }
  if (e != hipSuccess || n < 1) return 1;
  return n;
}

hipError_t launch_pack_w13(float *dst, const float *w1, const float *w3, int H,
                           int I, hipStream_t st) {
  hipLaunchKernelGGL(pack_w13_kernel, dim3(1024), dim3(256), 0, st,
                     reinterpret_cast<float4 *>(dst), reinterpret_cast<const float4 *>(w1),
                     reinterpret_cast<const float4 *>(w3), H / 4, I);
  return hipGetLastError();
}

}  // namespace moe
