// Internal layout shared by the HIP kernels (moe_kernels.hip) and the C-ABI
// host code (moe_capi.hip).  Not installed; the public boundary is
// include/moe_capi.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

constexpr int kExperts = 32;     // NUM_EXPERTS, reference include/config.h:14
constexpr int kDenseChunks = 4;  // dense FFN: intermediate cut into 4 chunk "experts"
constexpr int kTopK = 4;         // NUM_EXPERTS_PER_TOK, config.h:15
constexpr int kMinRouterTokens = 8;  // smallest token block of the router
constexpr int kThreads = 256;    // every kernel runs 4 waves of 64
constexpr int kCombineCols = 64;  // columns per combine counter (MFMA plans)
constexpr int kRouterSlotTokens = 1024;  // MFMA plans up to this many tokens: the router assigns slots
// 64-row plan up to this many tokens: the last kGateUpTailUnits units run
// half-width gate/up tiles (T=56-128: 1.2-2 % faster; 160 equal; 192-256: 1 % slower)
constexpr int kGateUpTailTokens = 128;
// 32/64-row plans: batches above this many tokens run their down tiles'
// per-slab waits (below it a down tile waits for its whole unit first)
constexpr int kSlabWaitMinTokens = 128;
constexpr int kGateUpTailUnits = 8;
// 128-row plan up to this many tokens: the same for its last kGateUpTailUnits
// units (a unit's 128-row gate/up tiles are long there, and its down tiles
// wait for the last of them: T=832 755 -> 732 us, T=1024 868 -> 862; at
// 2048 and 4096 tokens, where the down phase is long, 0.4-0.7 % slower)
constexpr int kGateUpTailTokens128 = 1024;
constexpr int kStreamRows = 16;  // weight rows per streaming-plan task (small batches)
constexpr int kStreamWideTokens = 32;  // batches from this size use 64-row tasks
// Streaming kernel shapes: tokens per MFMA pass; token passes of 16- and
// 64-row tasks; row groups of 16 in a 64-row task; row groups and passes of a
// 32-row task (experts of up to 64 tokens).
constexpr int kRingTokens = 16;
constexpr int kRingMaxPasses = 2;
constexpr int kRingWideGroups = 4;
constexpr int kRingDenseGroups = 2, kRingDensePasses = 4;
// Units (experts) whose down rows the streaming plan splits into 16-row tasks
// at the end of the queue when its 64-row tasks are streamed in sub-groups
// (T=64: 277 us with none, 275.7 with 2, 274.4 with 6, 277.4 with 12).
constexpr int kRingTailUnits = 6;
// Tokens of one decode token block: the batches whose routing the streaming
// kernel may finish itself (Ctrl::deferred).
constexpr int kDeferTokens = 8;
// Gate-logit chain jobs of a certified decode routing: 4 experts each.
constexpr int kChainJobs = kExperts / 4;
// A deferred decode routing gives each token a slot for every expert its
// score bounds leave possible (usually exactly its top-4, sometimes 5 or 6),
// at most kSpecSlots; a batch with a token past that waits for its logits.
constexpr int kSpecSlots = 8;
// 32- and 64-row MFMA plans: moe_forward of up to this many tokens routes
// from score bounds (Ctrl::deferred == 3): every block of the expert kernel
// plans a slot for every expert a token's bounds leave possible, and its
// dispatch tasks compute the logits and each token's exact top-4 while the
// gate/up tiles run.
constexpr int kBoundTokens = 256;
constexpr int kPlanCopies = 8;
constexpr int kPlanCopyInts = kBoundTokens + kBoundTokens / kDeferTokens * kExperts;
// Counters the blocks of a routing from bounds claim their first tasks from
// (Ctrl::gclaim): one counter serialises 512 claims at ~11 ns each, so the
// last block of a launch had its first task ~6 us after the first block;
// over 8 counters every block has its first task within ~1.3 us of starting.
constexpr int kClaimGroups = 8;

// Device control block.  Filled by the last router block of a forward and
// consumed by the expert kernel of the same forward.  All counters are reset
// by that router block, so a forward needs no memset (and no host round trip).
struct Ctrl {
  int router_done;  // router blocks finished (last-block election)
  int assign_done;  // dispatch (slot assignment) tasks finished
  int err;          // sticky: 1 = a bounded wait expired
  int num_tokens;
  int tile_rows;    // 0 = streaming kernel, else MFMA rows per tile
  int n_rblocks;    // router blocks = dispatch tasks
  int n_p1;         // gate/up (W1,W3) tasks
  int n_p2;         // down (W2) tasks
  int n_comb;       // combine tasks (streaming plan; MFMA plans combine in their down tiles)
  int n_total;      // sum of the four
  int p1_per_unit;  // W1W3 tasks per m-tile (MFMA) or per expert (streaming)
  int p2_per_unit;
  int n_active;     // experts with count > 0
  int rtokens;      // tokens per router block (dispatch task size)
  int stream_rows;  // streaming plan: weight rows per task (16, 32 or 64)
  int max_count;    // tokens of the largest expert
  int slots_assigned;  // MFMA plans: the router wrote every slot (pos = slot, slot_token)
  // 0: the router routed and planned; 2: it wrote score bounds (sbound), the
  // streaming kernel plans a slot for every expert they leave possible, and
  // computes the logits (chain jobs) and each token's exact top-4
  int deferred;
  int chain_lazy;   // test hook: blocks leave the chain jobs to the waits that need them
  int tail_units;   // last units whose down tiles run as two half-width tiles
  int gu_tail;      // 64-row plan: of those, the units whose gate/up tiles also run at half width
  int counts[kExperts];
  int offsets[kExperts + 1];
  int unit_off[kExperts + 1];  // prefix of units (m-tiles or 1 per active expert)
  int active[kExperts];
  // 3: the router wrote score bounds (MFMA plans); every block of the expert
  // kernel plans from them, and its dispatch tasks compute the logits and
  // each token's exact top-4
  // deferred == 2: lower and upper bound of each (token, expert) score
  // sigmoid(logit) + bias, whatever order the logit's FMA chain ran in
  float sbound[2][kDeferTokens][kExperts];
  // chain jobs claimed and stored (deferred == 2), on a cache line of their
  // own: atomics on one line serialise, and head takes one per block
  alignas(128) int chain_head;
  int chain_done;
  // expert-kernel task queue head, on a cache line of its own: every block
  // claims its first task at once as it starts, and loads of the plan's
  // fields on the same line waited behind those atomics (~5 us at 512 blocks)
  alignas(128) int head;
  // routing from bounds (deferred == 3): the first round of claims, one
  // counter per group of blocks (block b: group b % kClaimGroups), each on
  // a 128-byte line of its own; group g's k-th claim is task
  // k * kClaimGroups + g (expert_mfma_kernel, first_round_left)
  alignas(128) int gclaim[kClaimGroups][32];
  // followed in memory by int dep[max_units][dep_words(I)]: bit n of a
  // unit's mask is set once its W1W3 (gate/up) tile n has stored its
  // intermediate columns
};

// Mask words per unit of Scratch::dep: one bit per gate/up tile, at most
// 2 I / 64 of them (half-width tiles of 32 intermediate columns).
__host__ __device__ constexpr int dep_words(int inter) { return (inter + 1023) / 1024; }

struct Weights {
  const float *gate;     // [E][H]
  const float *bias;     // [E] (may be null)
  const float *w13;      // [E][I/32][2][32][H]: 32 rows of W1 then 32 of W3
  const float *w2;       // [E][H][I]
};

struct Scratch {
  float *logits;         // [Tmax][E]
  int *idx;              // [Tmax][4]
  float *wts;            // [Tmax][4]
  int *pos;              // [Tmax][4]: local rank, then slot
  int *blk;              // [Tmax/8][E]: block counts, then block bases
  int *tb_done;          // [Tmax/8]: expert-split blocks finished per token block
  int *slot_token;       // [slot_cap]: token of each slot
  float *inter;          // [slot_cap][I]
  float *sout;           // [slot_cap][H]
  uint32_t inter_bytes;  // allocation sizes (< 4 GiB: 32-bit buffer offsets)
  uint32_t sout_bytes;
  int slot_cap;          // slot rows of slot_token, inter and sout
  Ctrl *ctrl;
  int *dep;              // [max_units][dep_words(I)]: gate/up tiles done per unit (bit masks)
  int *ccount;           // [Tmax][H/64]: expert outputs landed per (token, column tile)
  // routing from score bounds (Ctrl::deferred == 3), min(Tmax, kBoundTokens)
  // tokens; null where a context has no room for it
  float *bounds;         // [T][2][E]: lower, then upper bound of each score
  // [kPlanCopies][kPlanCopyInts]: copies of each token's possible-expert mask
  // ([kBoundTokens]) and each token block's possible pairs per expert
  // ([kBoundTokens / 8][E]), one per die: every block of the expert kernel
  // reads them as it starts, and one copy read by all 512 blocks at once
  // came back ~5 us late
  uint32_t *bplan;
};

struct RouterArgs {
  const float *x;        // [T][H] (null when routing from logits)
  const float *logits_in;  // [T][E] or null
  Weights w;
  Scratch s;
  int T, H;
  int tile_rows;         // plan: 0 streaming, else MFMA tile rows
  int inter;             // I (for task counts)
  int bn;                // MFMA n-tile width (columns of the B tile)
  int tail_units;        // MFMA plans: last units whose down tiles run at half width
  int max_units;
  int defer;             // 2: score bounds instead of the logits (router_can_defer); 3: the
                         // same for an MFMA plan (router_can_bound); else 0
  int lazy_chains;       // defer == 2: Ctrl::chain_lazy
  const float *norm_w;   // post-attention RMSNorm weight [H]: x is h, normalise it (decode router only)
  float *xn;             // [T][H]: the normalised rows, for the expert kernel
};

struct ExpertArgs {
  const float *x;        // [T][H]
  float *y;              // [T][H]
  const float *residual; // [T][H] or null
  Weights w;
  Scratch s;
  int T, H, I;
  int wait_limit;        // bounded-wait iterations before giving up
  // routing from score bounds (RouterArgs::defer 3, MFMA plans): the blocks
  // plan from the router's masks and counts, with this many tail units (the
  // routing's own values, so a block reads no control field before its plan)
  int bounds;
  int tail_units;
};

// Launchers (moe_kernels.hip).  Return hipSuccess or the launch error.
hipError_t launch_router(const RouterArgs &a, bool from_logits, hipStream_t st);
hipError_t launch_experts(const ExpertArgs &a, int tile_rows, int grid,
                          hipStream_t st);
hipError_t launch_pack_w13(float *dst, const float *w1, const float *w3, int H,
                           int I, hipStream_t st);
// Tokens per router block for a forward of T tokens.
int router_tokens_per_block(int T);
// Whether the router normalises h itself (RouterArgs::norm_w) for T tokens;
// otherwise launch_rmsnorm writes the normalised rows first.
bool router_fuses_norm(int T);
hipError_t launch_rmsnorm(const float *h, const float *w, float *out, int T, int H,
                          hipStream_t st);
// Fixed routing of the dense FFN (every token to chunks 0..kDenseChunks-1,
// weight 1) and the plan for it; a.tile_rows/bn/inter as for launch_router.
hipError_t launch_router_dense(const RouterArgs &a, hipStream_t st);
// Whether the weight-streaming kernel is compiled for (H, I).
bool stream_supported(int H, int I);
// Largest batch the streaming plan handles (its slot -> token map is in LDS).
int stream_max_tokens();
// Max resident blocks per CU of the expert kernel for a plan.
int expert_blocks_per_cu(int tile_rows);
// Columns of the B tile of the MFMA kernel, or weight rows per task of the
// streaming kernel, for a plan and batch size.
int expert_bn(int tile_rows, int T);
// Whether a forward may leave routing and planning to the expert kernel: one
// decode-router token block under the weight-streaming plan with 16-row tasks.
bool router_can_defer(int T, int tile_rows, int bn);
// Whether a forward under an MFMA plan may route from score bounds (the
// context's Scratch must also hold bounds and smap, and T * kExperts slots).
bool router_can_bound(int T, int tile_rows, int H);
// Weight rows per streaming task for the dense FFN, whose chunks all hold T
// tokens: 32-row tasks with 4 token passes above 32 tokens.
int stream_rows_dense(int T);

}  // namespace moe
