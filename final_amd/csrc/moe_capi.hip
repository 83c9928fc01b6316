// C-ABI of the MI355X sparse-MoE block (include/moe_capi.h).
//
// Host orchestration of SparseMoeBlock (reference src/layer.cu:1274-1503):
// owns the repacked weights and the scratch, plans the expert kernel from the
// token count and launches router + expert kernels on the caller's stream
// with no host synchronisation.
#include "moe_capi.h"

#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <new>
#include <vector>

#include "moe_internal.h"

using namespace moe;

namespace {

constexpr int kDefaultWaitLimit = 1 << 20;
constexpr int kMaxTokensLimit = 1 << 20;

// Switches to the context's device for the duration of a call.
struct DeviceGuard {
  int prev = -1;
  bool ok = true;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) {
      ok = false;
      return;
    }
    if (prev != dev && hipSetDevice(dev) != hipSuccess) ok = false;
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev)
      (void)hipSetDevice(prev);
  }
};

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

// ---------------------------------------------------------------------------
// Scratch of moe_forward_noalloc: one file-scope device array per GPU, for
// callers that cannot allocate (code under HIP graph capture, serving loops).
// Layout: a fixed header whose counters must start at zero (Ctrl + dep, then
// the router's per-token-block counters), cleared once per device at set-up
// and returned to zero by every forward that completes (the router resets the
// counters it and the expert kernel use; it never waits, so it always ends);
// then the data regions of one call, laid out for that call's token count.
// In host code `scratch` names a host-side stand-in: kernels and copies use
// the device address hipGetSymbolAddress returned for the current device.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kNoAllocBytes = (size_t)8 << 20;  // 8 MiB per GPU
constexpr int kNoAllocMaxTokens = 128;
constexpr size_t kNoAllocHeader = 12288;  // Ctrl + dep[], then tb_done[]
constexpr size_t kNoAllocTbDone = 8192;   // offset of tb_done in the header
constexpr int kNoAllocMaxUnits = kNoAllocMaxTokens * kTopK / 32 + kExperts + 1;
constexpr int kMaxDevices = 64;
static_assert(sizeof(Ctrl) + 2 * sizeof(int) * kNoAllocMaxUnits <= kNoAllocTbDone,
              "ctrl + dep fit for intermediates up to 2048 (noalloc_layout checks larger ones)");
static_assert(kNoAllocTbDone + sizeof(int) * (kNoAllocMaxTokens / kMinRouterTokens) <=
                  kNoAllocHeader, "tb_done fits");

std::mutex g_noalloc_mu;
char *g_noalloc_ptr[kMaxDevices] = {};  // device address of `scratch` per device
// set by moe_forward_noalloc, cleared by the moe_device_status that reads the
// array's status word: status checks read it only after a no-alloc call
std::atomic<bool> g_noalloc_used[kMaxDevices] = {};

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

// Once per device, with that device current (from moe_create): the device
// address of `scratch` and a cleared header.  MOE_OK or MOE_ERR_HIP.
static int noalloc_setup(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return MOE_OK;  // moe_forward_noalloc then reports not ready
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (g_noalloc_ptr[dev]) return MOE_OK;
  void *p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
    (void)hipGetLastError();
    return MOE_ERR_HIP;
  }
  if (hipMemset(p, 0, kNoAllocHeader) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
    return MOE_ERR_HIP;
  g_noalloc_ptr[dev] = static_cast<char *>(p);
  return MOE_OK;
}

static char *noalloc_ptr(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  return g_noalloc_ptr[dev];
}

// The call's Scratch inside the device array at `base`, for T tokens of a
// context with hidden H and intermediate I.  False if it does not fit.
static bool noalloc_layout(char *base, int T, int H, int I, Scratch *s, int *max_units) {
  const size_t S = (size_t)T * kTopK, E = kExperts;
  const size_t nb = (T + kMinRouterTokens - 1) / kMinRouterTokens;
  size_t off = kNoAllocHeader;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = align256(off + bytes);
    return base + o;
  };
  s->ctrl = reinterpret_cast<Ctrl *>(base);
  s->dep = reinterpret_cast<int *>(base + sizeof(Ctrl));
  s->tb_done = reinterpret_cast<int *>(base + kNoAllocTbDone);
  s->logits = reinterpret_cast<float *>(take(T * E * sizeof(float)));
  s->idx = reinterpret_cast<int *>(take(S * sizeof(int)));
  s->wts = reinterpret_cast<float *>(take(S * sizeof(float)));
  s->pos = reinterpret_cast<int *>(take(S * sizeof(int)));
  s->blk = reinterpret_cast<int *>(take(nb * E * sizeof(int)));
  s->slot_token = reinterpret_cast<int *>(take(S * sizeof(int)));
  s->ccount = reinterpret_cast<int *>(take((size_t)T * (H / kCombineCols) * sizeof(int)));
  s->inter = reinterpret_cast<float *>(take(S * I * sizeof(float)));
  s->sout = reinterpret_cast<float *>(take(S * H * sizeof(float)));
  s->inter_bytes = (uint32_t)(S * I * sizeof(float));
  s->sout_bytes = (uint32_t)(S * H * sizeof(float));
  s->slot_cap = (int)S;
  *max_units = (int)(S / 32 + E + 1);
  return off <= kNoAllocBytes &&
         sizeof(Ctrl) + sizeof(int) * (size_t)dep_words(I) * (size_t)*max_units <= kNoAllocTbDone;
}

struct moe_ctx {
  moe_dims d{};
  int device = 0;
  int cus = 1;
  int tile_override = -1;
  int wait_div = 1;
  bool lazy_chains = false;  // test hook (moe_set_lazy_chains)
  bool weights_set = false;
  bool has_bias = false;
  bool dense = false;      // dense FFN context (moe_dense_create): kDenseChunks chunk experts
  int dense_inter = 0;     // its full intermediate size
  bool stream_ok = false;  // streaming kernel compiled for (H, I)
  int max_units = 0;
  int grid[4] = {1, 1, 1, 1};  // plans 0, 32, 64, 128
  // last routing state
  int routed_T = -1;
  bool route_pending = false;  // a routing not yet consumed by moe_experts
  int routed_plan = -1;
  bool routed_bounds = false;  // the routing wrote score bounds (RouterArgs::defer 3)
  int routed_tail = 0;         // its tail units
  // device memory
  float *gate = nullptr;
  float *bias = nullptr;
  float *w13 = nullptr;
  float *w2 = nullptr;
  // post-attention RMSNorm (moe_forward_norm)
  float *norm_w = nullptr;  // [H]
  float *xn = nullptr;      // [max_tokens][H]: normalised rows
  int normed_T = -1;
  Scratch s{};
  moe_ctx *donor = nullptr;  // context whose scratch this one uses (moe_create_shared)
  std::vector<void *> allocs;
};

static int plan_index(int rows) {
  switch (rows) {
    case 0: return 0;
    case 32: return 1;
    case 64: return 2;
    case 128: return 3;
    default: return -1;
  }
}

// Crossovers measured on MI355X with the seed-0 workload (moe_forward
// whole-step times, four weight copies cycled, clocks settled; streaming vs
// 64-row tiles): weight streaming is fastest up to 10 tokens (183.3 vs 198.5
// us at 8, 207.9 vs 211.5 at 9, 223.4 vs 225.1 at 10), 64-row MFMA tiles,
// whose routing from score bounds planned in every block takes the router's
// chains and planning off the critical path and whose down tiles all run at
// half width up to 128 tokens, from 11 to 1024 tokens (231.1 vs 228.9 at
// 11, 233.1 vs 230.2 at 12, 245.6 vs 235.1 at 16, 258.2 vs 243.5 at 20;
// before the half-width down tiles streaming led up to 20; 283.3 vs 269.8
// and 282.0 vs 276.3 at 48, two boxes;
// equal at 640-768; 720 vs 726 at 832, 846 vs 854 at 1024), 128-row tiles
// from 1025 (990 vs 1023 us at 1280, 1478 vs 1540 at 2048).  moe_route +
// moe_experts, which keep the full router, take the same plans (with it,
// streaming led up to 48).
constexpr int kStreamMaxTokens = 10;
// The dense FFN's 4 chunk experts each hold every token, so its MFMA plans
// have few tiles at small T: streaming stays fastest up to 192 tokens (214
// vs 217 us at 128, 280 vs 283 at 192), 64-row tiles at 256 (290 vs 349 us),
// 128-row tiles from 384 (433 vs 495 us at 512).
static int auto_plan(int T, bool stream_ok, bool dense) {
  if (T <= (dense ? 192 : kStreamMaxTokens) && stream_ok) return 0;
  if (T < (dense ? 384 : 1025)) return 64;
  return 128;
}

static int ctx_plan(const moe_ctx *ctx, int T) {
  const int p = ctx->tile_override >= 0 ? ctx->tile_override : auto_plan(T, ctx->stream_ok, ctx->dense);
  // the streaming plan keeps the batch's slot -> token map in LDS
  return p == 0 && T > stream_max_tokens() ? 64 : p;
}

// MFMA plans: the last units' down tiles run as two half-width tiles, so the
// last round of tiles is about half as long.  128-row plan: about one
// block's worth of half tiles (T=4096: 3.01 -> 2.95 ms).  64-row plan: half
// that many units above 64 tokens (its units are few; with every expert in
// one unit, the longest-first order puts the smallest experts last): T=256
// expert launch 329 -> 311 us; one block's worth, 16 units at T=256, took as
// much there and lost 2 % at T=128.  Up to 128 tokens, where every unit
// is one small expert, two blocks' worth (32 units: every unit of such a
// batch).  One block's worth up to 64 tokens had taken T=21 256.0 -> 251.6
// us, T=32 262.5 -> 258.2, T=48 269.9 -> 266.7, T=64 268.5 -> 267.1 from
// half of one; two, same box: T=21 252.6 -> 247.3 us, T=64 269.1 -> 266.5,
// T=48 equal; then at 65-128 tokens (another box): T=80 271.6 -> 270.6,
// T=128 273.4 -> 270.2, while T=192 lost 7 us and one block's worth lost 3
// at T=128.  At 129-192 tokens one block's worth (same box, 2 rounds:
// T=160 278.9 -> 273.4 us, T=192 282.9 -> 280.9; at 256 it lost 4.8, a
// quarter of one lost 1.5-3 % at 160-1024).  Twice as many in the 128-row
// plan: equal at T=2048-4096.
static int tail_units(const moe_ctx *ctx, int tile_rows, int bn, int T) {
  const int pi = plan_index(tile_rows);
  if ((tile_rows != 128 && tile_rows != 64) || pi < 0) return 0;
  const int half_tiles_per_unit = 2 * (ctx->d.hidden / bn);
  const int block = ctx->grid[pi] / half_tiles_per_unit;  // one block's worth of units
  const int k = tile_rows == 128 ? block : T <= 128 ? 2 * block : T <= 192 ? block : block / 2;
  return k > 0 ? k : 1;
}

template <typename T>
static int dev_alloc(moe_ctx *ctx, T **p, size_t count) {
  void *v = nullptr;
  if (hipMalloc(&v, count * sizeof(T) + 16) != hipSuccess) {
    (void)hipGetLastError();
    return MOE_ERR_OUT_OF_MEMORY;
  }
  ctx->allocs.push_back(v);
  *p = static_cast<T *>(v);
  return MOE_OK;
}

static void free_all(moe_ctx *ctx) {
  for (void *p : ctx->allocs) (void)hipFree(p);
  ctx->allocs.clear();
}

extern "C" {

const char *moe_strerror(int status) {
  switch (status) {
    case MOE_OK: return "ok";
    case MOE_ERR_INVALID_ARG: return "invalid argument";
    case MOE_ERR_UNSUPPORTED: return "unsupported dimensions";
    case MOE_ERR_HIP: return "HIP runtime error";
    case MOE_ERR_OUT_OF_MEMORY: return "device out of memory";
    case MOE_ERR_NOT_READY: return "weights not set";
    case MOE_ERR_TOO_MANY_TOKENS: return "num_tokens exceeds max_tokens";
    case MOE_ERR_DEVICE_TIMEOUT: return "device-side dependency wait expired";
    case MOE_ERR_INTERNAL: return "inconsistent device dispatch plan";
    default: return "unknown status";
  }
}

const char *moe_version(void) { return "final_amd-moe 0.1.0 gfx950"; }

// A context with expert weights for e_alloc experts (all kExperts for the
// MoE block, kDenseChunks for the dense FFN, which has no gate).  With a
// donor the context allocates only its weights and runs on the donor's
// scratch (same hidden and per-expert inter, max_tokens <= the donor's).
static int create_ctx(const moe_dims &d, size_t e_alloc, bool dense, moe_ctx **out,
                      moe_ctx *donor = nullptr) {
  moe_ctx *ctx = new (std::nothrow) moe_ctx();
  if (!ctx) return MOE_ERR_OUT_OF_MEMORY;
  ctx->d = d;
  if (hipGetDevice(&ctx->device) != hipSuccess) {
    delete ctx;
    return MOE_ERR_HIP;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, ctx->device) != hipSuccess) {
    delete ctx;
    return MOE_ERR_HIP;
  }
  ctx->cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 1;
  ctx->stream_ok = stream_supported(d.hidden, d.inter);
  ctx->dense = dense;
  const size_t H = d.hidden, I = d.inter, E = kExperts;
  const size_t Tm = d.max_tokens;
  // slot rows: the top-4 of every token, the slots of every possible expert
  // of a deferred decode routing (moe_forward up to kDeferTokens tokens), or
  // of a routing from bounds under an MFMA plan (moe_forward up to
  // kBoundTokens tokens; all 32 experts for a token whose bounds are
  // infinite), whichever is most
  const size_t Ts = Tm < (size_t)kDeferTokens ? Tm : (size_t)kDeferTokens;
  const size_t Tb = Tm < (size_t)kBoundTokens ? Tm : (size_t)kBoundTokens;
  size_t S = Tm * kTopK > Ts * kSpecSlots ? Tm * kTopK : Ts * kSpecSlots;
  if (!dense && S < Tb * kExperts) S = Tb * kExperts;
  const size_t nb = (Tm + kMinRouterTokens - 1) / kMinRouterTokens;
  ctx->max_units = (int)(S / 32 + E + 1);
  // inter and sout are addressed with 32-bit byte offsets, and the MFMA
  // tiles use offsets from 0xFF000000 up as out-of-range (zero) loads
  if (S * (H > I ? H : I) * sizeof(float) >= 0xFF000000ull) {
    delete ctx;
    return MOE_ERR_UNSUPPORTED;
  }
  int rc = MOE_OK;
  if (donor) {
    while (donor->donor) donor = donor->donor;
    if (donor->d.hidden != d.hidden || donor->d.inter != d.inter ||
        donor->d.max_tokens < d.max_tokens || donor->device != ctx->device) {
      delete ctx;
      return MOE_ERR_INVALID_ARG;
    }
    if ((!dense && (rc = dev_alloc(ctx, &ctx->gate, E * H))) ||
        (!dense && (rc = dev_alloc(ctx, &ctx->bias, E))) ||
        (rc = dev_alloc(ctx, &ctx->w13, e_alloc * 2 * I * H)) ||
        (rc = dev_alloc(ctx, &ctx->w2, e_alloc * H * I))) {
      free_all(ctx);
      delete ctx;
      return rc;
    }
    ctx->donor = donor;
    ctx->s = donor->s;
    ctx->max_units = donor->max_units;
    for (int p = 0; p < 4; ++p) ctx->grid[p] = donor->grid[p];
    *out = ctx;
    return MOE_OK;
  }
  if ((!dense && (rc = dev_alloc(ctx, &ctx->gate, E * H))) ||
      (!dense && (rc = dev_alloc(ctx, &ctx->bias, E))) ||
      (rc = dev_alloc(ctx, &ctx->w13, e_alloc * 2 * I * H)) ||
      (rc = dev_alloc(ctx, &ctx->w2, e_alloc * H * I)) ||
      (rc = dev_alloc(ctx, &ctx->s.logits, Tm * E)) ||
      (rc = dev_alloc(ctx, &ctx->s.idx, S)) ||
      (rc = dev_alloc(ctx, &ctx->s.wts, S)) ||
      (rc = dev_alloc(ctx, &ctx->s.pos, S)) ||
      (rc = dev_alloc(ctx, &ctx->s.blk, nb * E)) ||
      (rc = dev_alloc(ctx, &ctx->s.tb_done, nb)) ||
      (rc = dev_alloc(ctx, &ctx->s.slot_token, S)) ||
      (rc = dev_alloc(ctx, &ctx->s.inter, S * I)) ||
      (rc = dev_alloc(ctx, &ctx->s.sout, S * H)) ||
      (rc = dev_alloc(ctx, &ctx->s.ccount, Tm * (H / 64))) ||
      (!dense && (rc = dev_alloc(ctx, &ctx->s.bounds, Tb * 2 * E))) ||
      (!dense && (rc = dev_alloc(ctx, &ctx->s.bplan, (size_t)kPlanCopies * kPlanCopyInts)))) {
    free_all(ctx);
    delete ctx;
    return rc;
  }
  ctx->s.inter_bytes = (uint32_t)(S * I * sizeof(float));
  ctx->s.sout_bytes = (uint32_t)(S * H * sizeof(float));
  ctx->s.slot_cap = (int)S;
  char *ctrl_mem = nullptr;
  // Ctrl, then dep[max_units][dep_words(I)]
  const size_t ctrl_bytes = sizeof(Ctrl) + sizeof(int) * (size_t)dep_words((int)I) * ctx->max_units;
  if ((rc = dev_alloc(ctx, &ctrl_mem, ctrl_bytes))) {
    free_all(ctx);
    delete ctx;
    return rc;
  }
  ctx->s.ctrl = reinterpret_cast<Ctrl *>(ctrl_mem);
  ctx->s.dep = reinterpret_cast<int *>(ctrl_mem + sizeof(Ctrl));
  if (hipMemset(ctrl_mem, 0, ctrl_bytes) != hipSuccess ||
      hipMemset(ctx->s.tb_done, 0, nb * sizeof(int)) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess) {
    free_all(ctx);
    delete ctx;
    return MOE_ERR_HIP;
  }
  for (int p = 0; p < 4; ++p) {
    static const int rows[4] = {0, 32, 64, 128};
    ctx->grid[p] = ctx->cus * expert_blocks_per_cu(rows[p]);
  }
  if ((rc = noalloc_setup(ctx->device))) {
    free_all(ctx);
    delete ctx;
    return rc;
  }
  *out = ctx;
  return MOE_OK;
}

int moe_create(const moe_dims *dims, moe_ctx **out) {
  if (!dims || !out) return MOE_ERR_INVALID_ARG;
  *out = nullptr;
  const moe_dims d = *dims;
  if (d.hidden <= 0 || d.inter <= 0 || d.max_tokens <= 0 ||
      d.max_tokens > kMaxTokensLimit)
    return MOE_ERR_INVALID_ARG;
  if (d.num_experts != kExperts || d.top_k != kTopK || d.hidden % 256 != 0 ||
      d.inter % 256 != 0)
    return MOE_ERR_UNSUPPORTED;
  return create_ctx(d, kExperts, false, out);
}

int moe_create_shared(const moe_dims *dims, moe_ctx *donor, moe_ctx **out) {
  if (!dims || !donor || !out) return MOE_ERR_INVALID_ARG;
  *out = nullptr;
  const moe_dims d = *dims;
  if (d.hidden <= 0 || d.inter <= 0 || d.max_tokens <= 0 || d.max_tokens > kMaxTokensLimit)
    return MOE_ERR_INVALID_ARG;
  if (d.num_experts != kExperts || d.top_k != kTopK || d.hidden % 256 != 0 || d.inter % 256 != 0)
    return MOE_ERR_UNSUPPORTED;
  DeviceGuard g(donor->device);
  if (!g.ok) return MOE_ERR_HIP;
  return create_ctx(d, kExperts, false, out, donor);
}

int moe_dense_create(int hidden, int inter, int max_tokens, moe_ctx **out) {
  return moe_dense_create_shared(hidden, inter, max_tokens, nullptr, out);
}

int moe_dense_create_shared(int hidden, int inter, int max_tokens, moe_ctx *donor,
                            moe_ctx **out) {
  if (!out) return MOE_ERR_INVALID_ARG;
  *out = nullptr;
  if (hidden <= 0 || inter <= 0 || max_tokens <= 0 || max_tokens > kMaxTokensLimit)
    return MOE_ERR_INVALID_ARG;
  if (hidden % 256 != 0 || inter % (kDenseChunks * 256) != 0) return MOE_ERR_UNSUPPORTED;
  moe_dims d{};
  d.hidden = hidden;
  d.inter = inter / kDenseChunks;  // each chunk is one "expert"
  d.num_experts = kExperts;
  d.top_k = kTopK;
  d.max_tokens = max_tokens;
  int rc;
  if (donor) {
    DeviceGuard g(donor->device);
    if (!g.ok) return MOE_ERR_HIP;
    rc = create_ctx(d, kDenseChunks, true, out, donor);
  } else {
    rc = create_ctx(d, kDenseChunks, true, out);
  }
  if (rc == MOE_OK) (*out)->dense_inter = inter;
  return rc;
}

int moe_destroy(moe_ctx *ctx) {
  if (!ctx) return MOE_OK;
  DeviceGuard g(ctx->device);
  free_all(ctx);
  delete ctx;
  return MOE_OK;
}

int moe_set_weights(moe_ctx *ctx, const float *gate, const float *bias,
                    const float *const *w1, const float *const *w3,
                    const float *const *w2, int src_on_device,
                    moe_stream_t stream) {
  if (!ctx || !gate || !w1 || !w3 || !w2 || ctx->dense) return MOE_ERR_INVALID_ARG;
  for (int e = 0; e < kExperts; ++e)
    if (!w1[e] || !w3[e] || !w2[e]) return MOE_ERR_INVALID_ARG;
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t H = ctx->d.hidden, I = ctx->d.inter, E = kExperts;
  const hipMemcpyKind kind =
      src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
  float *stage = nullptr;  // [2][I][H] (or E*H for the gate) staging on device
  const size_t stage_n = 2 * I * H > E * H ? 2 * I * H : E * H;
  if (!src_on_device) {
    if (hipMalloc(&stage, stage_n * sizeof(float)) != hipSuccess) {
      (void)hipGetLastError();
      return MOE_ERR_OUT_OF_MEMORY;
    }
  }
  int rc = MOE_OK;
  auto fail = [&](int code) {
    rc = code;
    return code;
  };
  do {
    if (hipMemcpyAsync(ctx->gate, gate, E * H * sizeof(float), kind, st) != hipSuccess) {
      fail(MOE_ERR_HIP);
      break;
    }
    ctx->has_bias = bias != nullptr;
    if (bias && hipMemcpyAsync(ctx->bias, bias, E * sizeof(float), kind, st) != hipSuccess) {
      fail(MOE_ERR_HIP);
      break;
    }
    for (size_t e = 0; e < E && rc == MOE_OK; ++e) {
      const float *s1 = w1[e], *s3 = w3[e];
      if (!src_on_device) {
        if (hipMemcpyAsync(stage, w1[e], I * H * sizeof(float), kind, st) != hipSuccess ||
            hipMemcpyAsync(stage + I * H, w3[e], I * H * sizeof(float), kind, st) != hipSuccess) {
          fail(MOE_ERR_HIP);
          break;
        }
        s1 = stage;
        s3 = stage + I * H;
      }
      if (launch_pack_w13(ctx->w13 + e * 2 * I * H, s1, s3, (int)H, (int)I, st) !=
          hipSuccess) {
        fail(MOE_ERR_HIP);
        break;
      }
      if (hipMemcpyAsync(ctx->w2 + e * H * I, w2[e], H * I * sizeof(float), kind, st) !=
          hipSuccess) {
        fail(MOE_ERR_HIP);
        break;
      }
      // the staging buffer is reused by the next expert
      if (!src_on_device && hipStreamSynchronize(st) != hipSuccess) {
        fail(MOE_ERR_HIP);
        break;
      }
    }
    if (rc == MOE_OK && hipStreamSynchronize(st) != hipSuccess) fail(MOE_ERR_HIP);
  } while (0);
  if (stage) (void)hipFree(stage);
  if (rc == MOE_OK) ctx->weights_set = true;
  return rc;
}

static int check_tokens(const moe_ctx *ctx, int T) {
  if (T < 0) return MOE_ERR_INVALID_ARG;
  if (T > ctx->d.max_tokens) return MOE_ERR_TOO_MANY_TOKENS;
  return MOE_OK;
}

// defer: the caller launches the experts right after (moe_forward,
// moe_forward_norm) with arguments already checked, so a single decode token
// block under the streaming plan may leave its routing to the expert kernel.
static int do_route(moe_ctx *ctx, const float *x, const float *logits, int T,
                    moe_stream_t stream, const float *norm_w = nullptr,
                    float *xn = nullptr, bool defer = false) {
  if (!ctx || ctx->dense) return MOE_ERR_INVALID_ARG;
  int rc = check_tokens(ctx, T);
  if (rc) return rc;
  if (!ctx->weights_set) return MOE_ERR_NOT_READY;
  if (T == 0) {
    ctx->routed_T = 0;
    return MOE_OK;
  }
  if (logits ? !aligned16(logits) : (!x || !aligned16(x))) return MOE_ERR_INVALID_ARG;
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  RouterArgs a{};
  a.x = x;
  a.logits_in = logits;
  a.w.gate = ctx->gate;
  a.w.bias = ctx->has_bias ? ctx->bias : nullptr;
  a.w.w13 = ctx->w13;
  a.w.w2 = ctx->w2;
  a.s = ctx->s;
  a.T = T;
  a.H = ctx->d.hidden;
  a.inter = ctx->d.inter;
  a.tile_rows = ctx_plan(ctx, T);
  a.bn = expert_bn(a.tile_rows, T);
  a.tail_units = tail_units(ctx, a.tile_rows, a.bn, T);
  a.max_units = ctx->max_units;
  // deferred decode routing: the router writes score bounds, the streaming
  // kernel computes the logits and routes
  // 32- and 64-row MFMA plans of up to kBoundTokens tokens: the router writes
  // score bounds, every block of the expert kernel plans a slot for every
  // expert they leave possible, and its dispatch tasks compute the logits
  // and the exact top-4
  const bool bound_room =
      ctx->s.bounds && ctx->s.bplan && (size_t)T * kExperts <= (size_t)ctx->s.slot_cap;
  a.defer = !defer || logits ? 0
            : router_can_defer(T, a.tile_rows, a.bn) ? 2
            : bound_room && router_can_bound(T, a.tile_rows, a.H) ? 3 : 0;
  a.lazy_chains = ctx->lazy_chains ? 1 : 0;
  a.norm_w = norm_w;
  a.xn = xn;
  if (launch_router(a, logits != nullptr, static_cast<hipStream_t>(stream)) != hipSuccess)
    return MOE_ERR_HIP;
  ctx->routed_T = T;
  ctx->route_pending = true;
  ctx->routed_plan = a.tile_rows;
  ctx->routed_bounds = a.defer == 3;
  ctx->routed_tail = a.tail_units;
  return MOE_OK;
}

int moe_route(moe_ctx *ctx, const float *x, int num_tokens, moe_stream_t stream) {
  return do_route(ctx, x, nullptr, num_tokens, stream);
}

int moe_route_forward(moe_ctx *ctx, const float *x, int num_tokens, moe_stream_t stream) {
  return do_route(ctx, x, nullptr, num_tokens, stream, nullptr, nullptr, true);
}

int moe_route_logits(moe_ctx *ctx, const float *logits, int num_tokens,
                     moe_stream_t stream) {
  if (num_tokens > 0 && !logits) return MOE_ERR_INVALID_ARG;
  return do_route(ctx, nullptr, logits, num_tokens, stream);
}

int moe_experts(moe_ctx *ctx, const float *x, float *y, const float *residual,
                int num_tokens, moe_stream_t stream) {
  if (!ctx) return MOE_ERR_INVALID_ARG;
  int rc = check_tokens(ctx, num_tokens);
  if (rc) return rc;
  if (!ctx->weights_set) return MOE_ERR_NOT_READY;
  if (num_tokens == 0) return MOE_OK;
  if (ctx->routed_T != num_tokens || !ctx->route_pending) return MOE_ERR_INVALID_ARG;
  if (!x || !y || !aligned16(x) || !aligned16(y) || (residual && !aligned16(residual)))
    return MOE_ERR_INVALID_ARG;
  if (x == y) return MOE_ERR_INVALID_ARG;
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  ExpertArgs a{};
  a.x = x;
  a.y = y;
  a.residual = residual;
  a.w.gate = ctx->gate;
  a.w.bias = ctx->has_bias ? ctx->bias : nullptr;
  a.w.w13 = ctx->w13;
  a.w.w2 = ctx->w2;
  a.s = ctx->s;
  a.T = num_tokens;
  a.H = ctx->d.hidden;
  a.I = ctx->d.inter;
  a.wait_limit = kDefaultWaitLimit / (ctx->wait_div > 0 ? ctx->wait_div : 1);
  if (a.wait_limit < 1) a.wait_limit = 1;
  const int plan = ctx->routed_plan;
  a.bounds = ctx->routed_bounds ? 1 : 0;
  a.tail_units = ctx->routed_tail;
  const int pi = plan_index(plan);
  if (pi < 0) return MOE_ERR_INVALID_ARG;
  // the routing (and, for the streaming plan, the rows the router prepared)
  // serve this one launch
  ctx->route_pending = false;
  if (launch_experts(a, plan, ctx->grid[pi], static_cast<hipStream_t>(stream)) != hipSuccess)
    return MOE_ERR_HIP;
  return MOE_OK;
}

// The experts' pointer checks (moe_experts), so a forward can tell before
// routing whether its experts launch will be accepted.
static bool experts_args_ok(const float *x, const float *y, const float *residual) {
  return x && y && aligned16(x) && aligned16(y) && (!residual || aligned16(residual)) && x != y;
}

int moe_forward(moe_ctx *ctx, const float *x, float *y, const float *residual,
                int num_tokens, moe_stream_t stream) {
  // routing is left to the expert kernel only when its launch follows
  int rc = do_route(ctx, x, nullptr, num_tokens, stream, nullptr, nullptr,
                    experts_args_ok(x, y, residual));
  if (rc) return rc;
  return moe_experts(ctx, x, y, residual, num_tokens, stream);
}

int moe_forward_noalloc(moe_ctx *ctx, const float *x, float *y, const float *residual,
                        int num_tokens, moe_stream_t stream) {
  if (!ctx || ctx->dense) return MOE_ERR_INVALID_ARG;
  const int T = num_tokens;
  if (T < 0) return MOE_ERR_INVALID_ARG;
  if (T > kNoAllocMaxTokens) return MOE_ERR_TOO_MANY_TOKENS;
  if (!ctx->weights_set) return MOE_ERR_NOT_READY;
  if (T == 0) return MOE_OK;
  if (!x || !y || !aligned16(x) || !aligned16(y) || (residual && !aligned16(residual)) || x == y)
    return MOE_ERR_INVALID_ARG;
  char *base = noalloc_ptr(ctx->device);
  if (!base) return MOE_ERR_NOT_READY;
  Scratch s{};
  int max_units = 0;
  if (!noalloc_layout(base, T, ctx->d.hidden, ctx->d.inter, &s, &max_units))
    return MOE_ERR_TOO_MANY_TOKENS;
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // same plan, kernels and arithmetic as moe_forward, on the device array
  RouterArgs ra{};
  ra.x = x;
  ra.w.gate = ctx->gate;
  ra.w.bias = ctx->has_bias ? ctx->bias : nullptr;
  ra.w.w13 = ctx->w13;
  ra.w.w2 = ctx->w2;
  ra.s = s;
  ra.T = T;
  ra.H = ctx->d.hidden;
  ra.inter = ctx->d.inter;
  ra.tile_rows = ctx_plan(ctx, T);
  ra.bn = expert_bn(ra.tile_rows, T);
  ra.tail_units = tail_units(ctx, ra.tile_rows, ra.bn, T);
  ra.max_units = max_units;
  const int pi = plan_index(ra.tile_rows);
  if (pi < 0) return MOE_ERR_INVALID_ARG;
  if (launch_router(ra, false, st) != hipSuccess) return MOE_ERR_HIP;
  ExpertArgs ea{};
  ea.x = x;
  ea.y = y;
  ea.residual = residual;
  ea.w = ra.w;
  ea.s = s;
  ea.T = T;
  ea.H = ctx->d.hidden;
  ea.I = ctx->d.inter;
  ea.wait_limit = kDefaultWaitLimit / (ctx->wait_div > 0 ? ctx->wait_div : 1);
  if (ea.wait_limit < 1) ea.wait_limit = 1;
  g_noalloc_used[ctx->device].store(true, std::memory_order_relaxed);
  if (launch_experts(ea, ra.tile_rows, ctx->grid[pi], st) != hipSuccess) return MOE_ERR_HIP;
  return MOE_OK;
}

int moe_dense_set_weights(moe_ctx *ctx, const float *w1, const float *w3, const float *w2,
                          int src_on_device, moe_stream_t stream) {
  if (!ctx || !ctx->dense || !w1 || !w3 || !w2) return MOE_ERR_INVALID_ARG;
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t H = ctx->d.hidden, Ic = ctx->d.inter, I = (size_t)ctx->dense_inter;
  const hipMemcpyKind kind = src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
  float *stage = nullptr;  // [2][Ic][H] staging of a host chunk
  if (!src_on_device) {
    if (hipMalloc(&stage, 2 * Ic * H * sizeof(float)) != hipSuccess) {
      (void)hipGetLastError();
      return MOE_ERR_OUT_OF_MEMORY;
    }
  }
  int rc = MOE_OK;
  for (size_t c = 0; c < (size_t)kDenseChunks && rc == MOE_OK; ++c) {
    // chunk c: W1/W3 rows [c Ic, (c+1) Ic), W2 columns [c Ic, (c+1) Ic)
    const float *s1 = w1 + c * Ic * H, *s3 = w3 + c * Ic * H;
    if (!src_on_device) {
      if (hipMemcpyAsync(stage, s1, Ic * H * sizeof(float), kind, st) != hipSuccess ||
          hipMemcpyAsync(stage + Ic * H, s3, Ic * H * sizeof(float), kind, st) != hipSuccess) {
        rc = MOE_ERR_HIP;
        break;
      }
      s1 = stage;
      s3 = stage + Ic * H;
    }
    if (launch_pack_w13(ctx->w13 + c * 2 * Ic * H, s1, s3, (int)H, (int)Ic, st) != hipSuccess ||
        hipMemcpy2DAsync(ctx->w2 + c * H * Ic, Ic * sizeof(float), w2 + c * Ic, I * sizeof(float),
                         Ic * sizeof(float), H, kind, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
      rc = MOE_ERR_HIP;
      break;
    }
  }
  if (stage) (void)hipFree(stage);
  if (rc == MOE_OK) ctx->weights_set = true;
  return rc;
}

int moe_dense_forward(moe_ctx *ctx, const float *x, float *y, const float *residual,
                      int num_tokens, moe_stream_t stream) {
  if (!ctx || !ctx->dense) return MOE_ERR_INVALID_ARG;
  int rc = check_tokens(ctx, num_tokens);
  if (rc) return rc;
  if (!ctx->weights_set) return MOE_ERR_NOT_READY;
  if (num_tokens == 0) {
    ctx->routed_T = 0;
    return MOE_OK;
  }
  if (!x || !aligned16(x)) return MOE_ERR_INVALID_ARG;
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  RouterArgs a{};
  a.x = x;
  a.w.w13 = ctx->w13;
  a.w.w2 = ctx->w2;
  a.s = ctx->s;
  a.T = num_tokens;
  a.H = ctx->d.hidden;
  a.inter = ctx->d.inter;
  a.tile_rows = ctx_plan(ctx, num_tokens);
  a.bn = a.tile_rows == 0 ? stream_rows_dense(num_tokens) : expert_bn(a.tile_rows, num_tokens);
  a.tail_units = tail_units(ctx, a.tile_rows, a.bn, num_tokens);
  a.max_units = ctx->max_units;
  if (launch_router_dense(a, static_cast<hipStream_t>(stream)) != hipSuccess) return MOE_ERR_HIP;
  ctx->routed_T = num_tokens;
  ctx->route_pending = true;
  ctx->routed_plan = a.tile_rows;
  ctx->routed_bounds = false;
  return moe_experts(ctx, x, y, residual, num_tokens, stream);
}

int moe_set_norm_weight(moe_ctx *ctx, const float *weight, int src_on_device,
                        moe_stream_t stream) {
  if (!ctx || !weight) return MOE_ERR_INVALID_ARG;
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t H = ctx->d.hidden;
  if (!ctx->norm_w) {
    float *nw = nullptr, *xn = nullptr;
    int rc = dev_alloc(ctx, &nw, H);
    if (rc) return rc;
    if (ctx->donor) {
      // the normalised rows are scratch too: the donor's serve every sharer
      if (!ctx->donor->xn) {
        rc = dev_alloc(ctx->donor, &ctx->donor->xn, (size_t)ctx->donor->d.max_tokens * H);
        if (rc) return rc;
      }
      xn = ctx->donor->xn;
    } else if (ctx->xn) {
      xn = ctx->xn;  // allocated for the context's sharers already
    } else {
      rc = dev_alloc(ctx, &xn, (size_t)ctx->d.max_tokens * H);
      if (rc) return rc;
    }
    ctx->norm_w = nw;
    ctx->xn = xn;
  }
  const hipMemcpyKind kind = src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
  if (hipMemcpyAsync(ctx->norm_w, weight, H * sizeof(float), kind, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return MOE_ERR_HIP;
  return MOE_OK;
}

int moe_forward_norm(moe_ctx *ctx, const float *h, float *out, int num_tokens,
                     moe_stream_t stream) {
  if (!ctx) return MOE_ERR_INVALID_ARG;
  int rc = check_tokens(ctx, num_tokens);
  if (rc) return rc;
  if (!ctx->weights_set || !ctx->norm_w) return MOE_ERR_NOT_READY;
  if (!h || !out || !aligned16(h) || !aligned16(out)) return MOE_ERR_INVALID_ARG;
  if (num_tokens == 0) {
    ctx->normed_T = 0;
    return do_route(ctx, h, nullptr, 0, stream);
  }
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (router_fuses_norm(num_tokens)) {
    // the router normalises the rows it stages and stores them for the experts
    rc = do_route(ctx, h, nullptr, num_tokens, stream, ctx->norm_w, ctx->xn,
                  experts_args_ok(ctx->xn, out, h));
  } else {
    if (launch_rmsnorm(h, ctx->norm_w, ctx->xn, num_tokens, ctx->d.hidden, st) != hipSuccess)
      return MOE_ERR_HIP;
    rc = do_route(ctx, ctx->xn, nullptr, num_tokens, stream);
  }
  if (rc) return rc;
  ctx->normed_T = num_tokens;
  // the residual is h itself; out may alias it (the experts read the
  // normalised rows, and the combine reads each residual element before it
  // writes the same element of out)
  return moe_experts(ctx, ctx->xn, out, h, num_tokens, stream);
}

int moe_last_normed(moe_ctx *ctx, float *xn, int num_tokens, moe_stream_t stream) {
  if (!ctx || !xn) return MOE_ERR_INVALID_ARG;
  if (ctx->normed_T < 0 || !ctx->xn) return MOE_ERR_NOT_READY;
  if (num_tokens != ctx->normed_T) return MOE_ERR_INVALID_ARG;  // xn holds another count
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t n = (size_t)ctx->normed_T * ctx->d.hidden;
  if (n && hipMemcpyAsync(xn, ctx->xn, n * sizeof(float), hipMemcpyDeviceToHost, st) != hipSuccess)
    return MOE_ERR_HIP;
  if (hipStreamSynchronize(st) != hipSuccess) return MOE_ERR_HIP;
  return MOE_OK;
}

int moe_last_routing(moe_ctx *ctx, int *idx, float *w, int *counts, float *logits,
                     int num_tokens, moe_stream_t stream) {
  if (!ctx) return MOE_ERR_INVALID_ARG;
  if (ctx->routed_T < 0) return MOE_ERR_NOT_READY;
  if (num_tokens != ctx->routed_T) return MOE_ERR_INVALID_ARG;  // buffers sized for another T
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t T = (size_t)ctx->routed_T;
  if (T == 0) {
    if (counts) memset(counts, 0, sizeof(int) * kExperts);
    return MOE_OK;
  }
  if (idx && hipMemcpyAsync(idx, ctx->s.idx, T * kTopK * sizeof(int),
                            hipMemcpyDeviceToHost, st) != hipSuccess)
    return MOE_ERR_HIP;
  if (w && hipMemcpyAsync(w, ctx->s.wts, T * kTopK * sizeof(float),
                          hipMemcpyDeviceToHost, st) != hipSuccess)
    return MOE_ERR_HIP;
  // counts: tokens per expert of the routing, the histogram of idx
  // (layer.cu:494-497 counts every (token, rank) selection); the plan's own
  // counts are per slot, and a deferred decode routing plans a slot for
  // every expert a token's score bounds leave possible
  std::vector<int> idx_own;
  int *idx_h = idx;
  if (counts && !idx_h) {
    idx_own.resize(T * kTopK);
    idx_h = idx_own.data();
    if (hipMemcpyAsync(idx_h, ctx->s.idx, T * kTopK * sizeof(int), hipMemcpyDeviceToHost, st) !=
        hipSuccess)
      return MOE_ERR_HIP;
  }
  if (logits && hipMemcpyAsync(logits, ctx->s.logits, T * kExperts * sizeof(float),
                               hipMemcpyDeviceToHost, st) != hipSuccess)
    return MOE_ERR_HIP;
  if (hipStreamSynchronize(st) != hipSuccess) return MOE_ERR_HIP;
  if (counts) {
    for (int e = 0; e < kExperts; ++e) counts[e] = 0;
    for (size_t i = 0; i < T * kTopK; ++i)
      if (idx_h[i] >= 0 && idx_h[i] < kExperts) ++counts[idx_h[i]];
  }
  return MOE_OK;
}

int moe_last_plan_counts(moe_ctx *ctx, int *counts, moe_stream_t stream) {
  if (!ctx || !counts) return MOE_ERR_INVALID_ARG;
  if (ctx->routed_T < 0) return MOE_ERR_NOT_READY;
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (ctx->routed_T == 0) {
    memset(counts, 0, sizeof(int) * kExperts);
    return MOE_OK;
  }
  if (hipMemcpyAsync(counts, ctx->s.ctrl->counts, kExperts * sizeof(int), hipMemcpyDeviceToHost,
                     st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return MOE_ERR_HIP;
  return MOE_OK;
}

// Reads and clears one status word (device int) on `st`; 0 when clear.
static int take_status(int *word, hipStream_t st, int *err) {
  *err = 0;
  if (hipMemcpyAsync(err, word, sizeof(int), hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return MOE_ERR_HIP;
  if (*err) {
    const int zero = 0;
    if (hipMemcpyAsync(word, &zero, sizeof(int), hipMemcpyHostToDevice, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
      return MOE_ERR_HIP;
  }
  return MOE_OK;
}

int moe_device_status(moe_ctx *ctx, moe_stream_t stream) {
  if (!ctx) return MOE_ERR_INVALID_ARG;
  DeviceGuard g(ctx->device);
  if (!g.ok) return MOE_ERR_HIP;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int err = 0, err_na = 0;
  if (take_status(&ctx->s.ctrl->err, st, &err)) return MOE_ERR_HIP;
  // the status word of the device's moe_forward_noalloc scratch, after a
  // no-alloc call on this device since the last check
  const int dev = ctx->device;
  if (dev >= 0 && dev < kMaxDevices && g_noalloc_used[dev].exchange(false))
    if (char *base = noalloc_ptr(dev))
      if (take_status(&reinterpret_cast<Ctrl *>(base)->err, st, &err_na)) return MOE_ERR_HIP;
  const int e = err ? err : err_na;
  if (e) return e == 1 ? MOE_ERR_DEVICE_TIMEOUT : MOE_ERR_INTERNAL;
  return MOE_OK;
}

int moe_plan_tile_rows(const moe_ctx *ctx, int num_tokens) {
  if (!ctx) return -1;
  return ctx_plan(ctx, num_tokens);
}

int moe_force_tile_rows(moe_ctx *ctx, int rows) {
  if (!ctx) return MOE_ERR_INVALID_ARG;
  if (rows != -1 && plan_index(rows) < 0) return MOE_ERR_INVALID_ARG;
  if (rows == 0 && !ctx->stream_ok) return MOE_ERR_UNSUPPORTED;
  ctx->tile_override = rows;
  return MOE_OK;
}

int moe_set_wait_divisor(moe_ctx *ctx, int divisor) {
  if (!ctx || divisor < 1) return MOE_ERR_INVALID_ARG;
  ctx->wait_div = divisor;
  return MOE_OK;
}

int moe_set_lazy_chains(moe_ctx *ctx, int on) {
  if (!ctx || ctx->dense) return MOE_ERR_INVALID_ARG;
  ctx->lazy_chains = on != 0;
  return MOE_OK;
}

}  // extern "C"
