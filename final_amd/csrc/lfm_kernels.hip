// HIP kernels of the decoder model around the MoE block (gfx950): the dense
// projections, embedding, q/k RMSNorm + rotary embedding, causal GQA
// attention, the short-conv mix, row RMSNorm and the device-side synthetic
// weight generator.
//
//   gemm_nt_kernel      attn_matmul_tiled_kernel (layer.cu:9-141) and
//                       lm_head_gemm_kernel (model.cu:42-116) as one MFMA GEMM,
//                       with the decoder's residual add_kernel (layer.cu:1860-
//                       1880 at 1912-1913) fused into its epilogue
//   embed_kernel        embedding_lookup_kernel (model.cu:18-32)
//   rmsnorm_rows_kernel rms_norm_kernel (layer.cu:144-193) on strided rows
//   qk_norm_rope_kernel the q/k RMSNorm of Attention::forward_gpu
//                       (layer.cu:1638-1642) + rope_transpose_kernel
//                       (layer.cu:195-231), in place, no transpose
//   attention_kernel    fused_attn_gqa_kernel (layer.cu:262-354) for any
//                       sequence length (the reference's holds 16 positions)
//   shortconv_kernel    conv_transpose_split_kernel + causal_conv1d_kernel +
//                       conv_gating_transpose_kernel (layer.cu:360-429) in one
//                       token-major pass
#include "lfm_internal.h"

#include "gpu_common.h"
#include "mfma_tile.h"

namespace lfm {

using moe::f32x4;
using moe::kThreads;

// ---------------------------------------------------------------------------
// Dense GEMM: C = A . B^T (+ R)
// ---------------------------------------------------------------------------

// Epilogue stores of the dense GEMM: plain 16-byte buffer stores (the output
// is consumed by the next kernel, not by other blocks of this one).
struct PlainOut {
  __amdgpu_buffer_rsrc_t rsrc;
  __device__ PlainOut(float *base, uint32_t bytes)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(base, 0, (int)bytes, moe::kBufferRsrcWord3)) {}
  __device__ void store(uint32_t off, f32x4 v) const {
    __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, off, 0, 0);
  }
};

// out = residual + product: add_kernel's float adds (layer.cu:1870-1874) done
// as the tile is stored; residual may alias the output (each element is read
// and then written by the same thread).
struct ResidualOut {
  __amdgpu_buffer_rsrc_t rsrc;
  const float *res;
  __device__ ResidualOut(float *base, uint32_t bytes, const float *r)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(base, 0, (int)bytes, moe::kBufferRsrcWord3)),
        res(r) {}
  __device__ void store(uint32_t off, f32x4 v) const {
    const f32x4 r = moe::ld4(res + off / 4);
    f32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = r[j] + v[j];
    __builtin_amdgcn_raw_buffer_store_b128(o, rsrc, off, 0, 0);
  }
};

struct GemmArgs {
  const float *A;  // [M][K]
  const float *B;  // [N][K]
  float *C;        // [M][N]
  const float *R;  // [M][N] or null
  int M, N, K;
};

constexpr int kGroupM = 8;  // M tiles walked together (their B tiles are shared)

// One 128x128 (or 64x128) tile per block.  Tile order: the dispatcher sends
// block b to XCD b % 8, so consecutive tile indices are given to the blocks
// of one XCD (its L2 then holds the A and B slabs its blocks share), and
// within that range tiles run in groups of kGroupM M-tiles column by column,
// so the blocks running together share B tiles and A tiles.
template <int BM, bool RES>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_nt_kernel(GemmArgs g) {
  using TL = moe::Tile<BM>;
  extern __shared__ float lds[];
  __shared__ int s_aoff[BM];
  const int ntm = (g.M + BM - 1) / BM, ntn = g.N / TL::BN;
  const int ntiles = ntm * ntn;
  int t = blockIdx.x;
  if (ntiles % 8 == 0) t = (t % 8) * (ntiles / 8) + t / 8;
  const int per_group = kGroupM * ntn;
  const int grp = t / per_group, first_m = grp * kGroupM;
  const int gsz = min(ntm - first_m, kGroupM);
  const int r = t - grp * per_group;
  const int m0 = (first_m + r % gsz) * BM, n0 = (r / gsz) * TL::BN;
  const int rows = min(BM, g.M - m0);
  if (threadIdx.x < BM) s_aoff[threadIdx.x] = threadIdx.x < rows ? (m0 + threadIdx.x) * g.K : 0;
  __syncthreads();
  const uint32_t abytes = (uint32_t)((size_t)g.M * g.K * sizeof(float));
  const uint32_t cbytes = (uint32_t)((size_t)g.M * g.N * sizeof(float));
  const float *brow0 = g.B + (size_t)n0 * g.K;
  if (RES)
    moe::mfma_tile<TL, false, ResidualOut>(lds, g.A, abytes, s_aoff, rows, brow0, g.K,
                                           ResidualOut(g.C, cbytes, g.R), m0, g.N, n0, nullptr);
  else
    moe::mfma_tile<TL, false, PlainOut>(lds, g.A, abytes, s_aoff, rows, brow0, g.K,
                                        PlainOut(g.C, cbytes), m0, g.N, n0, nullptr);
}

// ---------------------------------------------------------------------------
// Embedding
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void embed_kernel(const int *ids, const float *table, float *h,
                                                    int H4, int V, int *bad) {
  const int t = blockIdx.x;
  const int id = ids[t];
  const bool ok = id >= 0 && id < V;
  if (!ok && threadIdx.x == 0 && bad) __hip_atomic_store(bad, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const f32x4 *src = reinterpret_cast<const f32x4 *>(table) + (size_t)(ok ? id : 0) * H4;
  f32x4 *dst = reinterpret_cast<f32x4 *>(h) + (size_t)t * H4;
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int i = threadIdx.x; i < H4; i += 256) dst[i] = ok ? src[i] : zero;
}

// ---------------------------------------------------------------------------
// RMSNorm of strided rows (rms_norm_kernel, layer.cu:144-193, bit for bit:
// the reduction order is moe::norm_totals')
// ---------------------------------------------------------------------------

constexpr int kNormRows = 4;  // rows per block (their loads in flight together)

__global__ __launch_bounds__(moe::kNormThreads) void rmsnorm_rows_kernel(
    const float *x, long long xs, const float *w, float *y, long long ys, int rows, int dim) {
  __shared__ float s_grp[kNormRows * moe::kNormGroups], s_tot[kNormRows];
  const int r0 = blockIdx.x * kNormRows;
  const float *src[kNormRows];
  float *dst[kNormRows];
#pragma unroll
  for (int m = 0; m < kNormRows; ++m) {
    const long long r = min(r0 + m, rows - 1);
    src[m] = x + r * xs;
    dst[m] = y + r * ys;
  }
  moe::norm_rows<kNormRows>(src, dst, min(kNormRows, rows - r0), w, dim, s_grp, s_tot);
}

// ---------------------------------------------------------------------------
// q/k RMSNorm + rotary embedding, in place
// ---------------------------------------------------------------------------

constexpr int kHeadDim = 64;

// One wave per token: its heads + kv_heads rows of 64 (q heads at columns
// h*64, k heads at k_col + h*64), four rows per float4 load (16 lanes per
// row, lane l holding elements 4(l%16)..4(l%16)+3), with the cos/sin row of
// the token's position and both norm weights held in registers.  The norm is
// rms_norm_kernel on a 64-wide row launched with 256 threads (layer.cu:1146):
// threads 0..63 hold one square each (fmaf(x, x, 0) = x*x), warps 0 and 1
// fold elements 0..31 and 32..63 with shuffle-down at 16..1, and the 8-warp
// fold adds warps 2..7's zeros, which leaves warp0 + warp1.  The same binary
// tree runs here over the float4 layout (16 -> 4 lanes down, 8 -> 2 lanes,
// 4 -> 1 lane, then 2 and 1 across a lane's components), so every addition is
// the reference's.  Then rope_transpose_kernel's rotation (layer.cu:217-228)
// for position s = t % seq: out[d] = q1*c1 - q2*s1, out[d+32] = q2*c2 + q1*s2
// with q1 = x[d], q2 = x[d+32] (element d + 32 is 8 lanes up); nvcc's
// contraction of each line is restated as fmaf(first product, -/+ second
// product).
constexpr int kRopeTokens = 4;   // tokens per block, one per wave
constexpr int kRopeGroups = 16;  // groups of 4 rows a wave holds: heads + kv_heads <= 64

__global__ __launch_bounds__(256) void qk_norm_rope_kernel(float *qkv, int ld, const float *qw,
                                                           const float *kw, const float *cos_t,
                                                           const float *sin_t, int ntok, int seq,
                                                           int heads, int per_tok, int k_col) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63, r = lane >> 4, c4 = (lane & 15) * 4;
  const int t = blockIdx.x * kRopeTokens + (threadIdx.x >> 6);
  if (t >= ntok) return;  // whole waves; the kernel has no block barrier
  const int ng = (per_tok + 3) >> 2;
  const int pos = t % seq;
  const f32x4 cs = moe::ld4(cos_t + (size_t)pos * kHeadDim + c4);
  const f32x4 sn = moe::ld4(sin_t + (size_t)pos * kHeadDim + c4);
  const f32x4 wq = moe::ld4(qw + c4), wk = moe::ld4(kw + c4);
  float *row0 = qkv + (size_t)t * ld;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(row0, 0, ld * (int)sizeof(float), moe::kBufferRsrcWord3);
  // every load is unconditional (rows past per_tok read past the token's row:
  // zeros), so all of a token's loads are in flight together
  f32x4 x[kRopeGroups];
  uint32_t off[kRopeGroups];
#pragma unroll
  for (int j = 0; j < kRopeGroups; ++j) {
    const int row = 4 * j + r;
    off[j] = row < per_tok ? (uint32_t)((row < heads ? row * kHeadDim : k_col + (row - heads) * kHeadDim) + c4) * 4u
                           : 0x7FFFFFF0u;
    x[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off[j], 0, 0));
  }
#pragma unroll
  for (int j = 0; j < kRopeGroups; ++j) {
    if (j >= ng) continue;  // wave-uniform
    const int row = 4 * j + r;
    f32x4 sq;
#pragma unroll
    for (int i = 0; i < 4; ++i) sq[i] = x[j][i] * x[j][i];
    f32x4 a, b, cc;
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = sq[i] + __shfl_down(sq[i], 4, 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = a[i] + __shfl_down(a[i], 2, 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) cc[i] = b[i] + __shfl_down(b[i], 1, 16);
    const float f = (cc[0] + cc[2]) + (cc[1] + cc[3]);
    const float total = __shfl(f, 16 * r) + __shfl(f, 16 * r + 8);
    const float rms = 1.0f / sqrtf(total / (float)kHeadDim + moe::kNormEps);
    const f32x4 w = row < heads ? wq : wk;
    f32x4 y, other, o;
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = (x[j][i] * rms) * w[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) other[i] = __shfl_xor(y[i], 8);
    const bool lo = (lane & 15) < 8;  // elements d < 32
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = lo ? __builtin_fmaf(y[i], cs[i], -(other[i] * sn[i])) : __builtin_fmaf(y[i], cs[i], other[i] * sn[i]);
    if (row < per_tok) __builtin_amdgcn_raw_buffer_store_b128(o, rs, off[j], 0, 0);
  }
}

// ---------------------------------------------------------------------------
// Causal GQA attention, head_dim 64
// ---------------------------------------------------------------------------
//
// Block = (sequence b, kv head g, 32 consecutive queries), 8 waves: wave w
// serves q head g*4 + (w & 3) for the 16 queries q0 + 16*(w >> 2), so the
// eight waves share every 64-key K/V tile staged in LDS (the four heads of a
// group and both query halves).  Both products run on
// v_mfma_f32_16x16x4_f32 in transposed form, S^T = K Q^T and O^T = V^T P^T,
// so that a lane's query is always l % 16: the softmax statistics of a query
// live in its four lanes (l % 16 equal), P goes from the S^T result registers
// straight into the B operand of O^T (the reduction index k of both MFMAs is
// permuted the same way in A and B), and nothing is transposed.  Online
// softmax in fp32 with base-2 exponentials: q is scaled by log2(e)/8, so a
// score is log2 of the unnormalised weight and v_exp_f32 gives it directly
// (the 1/8 is exact, log2(e) adds one rounding per q element).  Masked
// scores are -1e30 as in the reference (layer.cu:316-318), so exp2 gives 0.
constexpr int kAttnQW = 16;             // queries per wave
constexpr int kAttnQB = 2 * kAttnQW;    // queries per block
constexpr int kAttnThreads = 512;
constexpr int kAttnKT = 64;             // keys per tile
constexpr int kAttnPitch = 68;          // floats per LDS row of the K and V tiles [key][d]
constexpr float kLog2e = 1.44269504088896340736f;

__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(4)))
void attention_kernel(const float *qkv, int ld, float *out, int ldo, int seq, int kv_heads,
                      int group, int qblocks, int k_col, int v_col) {
  __shared__ float Ks[kAttnKT * kAttnPitch];
  __shared__ float Vs[kAttnKT * kAttnPitch];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bid = blockIdx.x;
  const int qb = qblocks - 1 - bid % qblocks;  // the longer rows of a sequence first
  const int rest = bid / qblocks;
  const int g = rest % kv_heads, b = rest / kv_heads;
  const int h = g * group + (wave & 3);
  const int q0b = qb * kAttnQB;
  const int q0 = q0b + kAttnQW * (wave >> 2);
  const size_t tok0 = (size_t)b * seq;
  const int ql = lane & 15, kq = lane >> 4;
  const int q = q0 + ql;
  const bool qvalid = q < seq;
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};

  // B operand of S^T: lane (ql, kq) holds q[16a + 4kq + j] * log2(e) / 8
  f32x4 qv[4];
  const float qscale = 0.125f * kLog2e;
#pragma unroll
  for (int a = 0; a < 4; ++a)
    qv[a] = qvalid ? moe::ld4(qkv + (tok0 + q) * ld + h * kHeadDim + 16 * a + 4 * kq) * qscale : zero;

  // keys [0, kend) serve the block; the last tile starts at or before q0b,
  // so no valid query sees a tile with every key masked
  const int kend = min(seq, q0b + kAttnQB);
  const int ntiles = (kend + kAttnKT - 1) / kAttnKT;
  float m = -1e30f, l = 0.0f;
  f32x4 o[4] = {zero, zero, zero, zero};

  // staging: thread tid moves rows tid/16 and tid/16 + 32 of K and V, float4
  // column (tid%16)*4
  const int srow = tid >> 4, scol = (tid & 15) * 4;
  f32x4 kreg[2], vreg[2];
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int kr = kt * kAttnKT + srow + 32 * i;
      const bool ok = kr < kend;
      const float *rowp = qkv + (tok0 + (ok ? kr : 0)) * ld;
      kreg[i] = ok ? moe::ld4(rowp + k_col + g * kHeadDim + scol) : zero;
      vreg[i] = ok ? moe::ld4(rowp + v_col + g * kHeadDim + scol) : zero;
    }
  };
  gload(0);
  for (int kt = 0; kt < ntiles; ++kt) {
    __syncthreads();  // the previous tile's readers are done
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = srow + 32 * i;
      moe::st4(Ks + r * kAttnPitch + scol, kreg[i]);
      moe::st4(Vs + r * kAttnPitch + scol, vreg[i]);
    }
    __syncthreads();
    if (kt + 1 < ntiles) gload(kt + 1);

    // S^T blocks: s[kb] holds S^T[key = 64kt + 16kb + 4kq + i][q]
    f32x4 s[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      s[kb] = zero;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const f32x4 kf = moe::ld4(Ks + (kb * 16 + ql) * kAttnPitch + 16 * a + 4 * kq);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          s[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j], qv[a][j], s[kb], 0, 0, 0);
      }
    }
    // causal mask (keys past q; this also covers keys past the sequence)
    const int kbase = kt * kAttnKT + 4 * kq;
    if (kt * kAttnKT + kAttnKT - 1 > q0) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kbase + 16 * kb + i > q) s[kb][i] = -1e30f;
    }
    float mt = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) mt = fmaxf(mt, s[kb][i]);
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float mn = fmaxf(m, mt);
    const float alpha = __builtin_amdgcn_exp2f(m - mn);
    m = mn;
    float ps = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[kb][i] = __builtin_amdgcn_exp2f(s[kb][i] - mn);
        ps += s[kb][i];
      }
    l = l * alpha + ps;
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] *= alpha;
    // O^T[d = 16db + 4kq + j][q] += sum over keys of V^T[d][key] P[q][key]:
    // the A operand of step (kb, i) is V[16kb + 4kq + i][16db + ql]
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      f32x4 acc = o[db];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const float *vp = Vs + (kb * 16 + 4 * kq) * kAttnPitch + db * 16 + ql;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(vp[i * kAttnPitch], s[kb][i], acc, 0, 0, 0);
      }
      o[db] = acc;
    }
  }
  float lt = l + __shfl_xor(l, 16);
  lt += __shfl_xor(lt, 32);
  const float inv = 1.0f / lt;
  if (qvalid) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
      moe::st4(out + (tok0 + q) * ldo + h * kHeadDim + db * 16 + 4 * kq, o[db] * inv);
  }
}

// ---------------------------------------------------------------------------
// Short-conv mix
// ---------------------------------------------------------------------------

// One thread per (4 consecutive tokens, 4 channels): Bx = B * gate
// (conv_transpose_split_kernel, layer.cu:377-378) of the window's rows, each
// computed once, then per token the causal conv as the FMA chain of
// causal_conv1d_kernel (layer.cu:397-403: sum from 0, taps k ascending, only
// positions of the token's own sequence), times C
// (conv_gating_transpose_kernel, layer.cu:420).  Threads next to each other
// take neighbouring channels of the same tokens (coalesced rows); the window's
// first L-1 rows are re-read by the thread of the previous tokens.
constexpr int kConvTok = 4;   // tokens per thread
constexpr int kConvMaxL = 4;  // taps the window holds

__global__ __launch_bounds__(256) void shortconv_kernel(const float *bcg, const float *w, float *y,
                                                        long long T, int seq, int H, int L) {
#pragma clang fp contract(off)
  const int H4 = H / 4;
  const long long groups = (T + kConvTok - 1) / kConvTok;
  for (long long f = blockIdx.x * 256LL + threadIdx.x; f < groups * H4;
       f += (long long)gridDim.x * 256) {
    const long long tg = f / H4;
    const int c = (int)(f - tg * H4) * 4;
    const long long t0 = tg * kConvTok;
    // taps of the 4 channels: w[c + j][k] = w[c*L + j*L + k], 4L floats from c*L
    float wk[4][kConvMaxL];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int k = 0; k < kConvMaxL; ++k) wk[j][k] = k < L ? w[(c + j) * L + k] : 0.0f;
    // Bx of tokens t0 - (L-1) .. t0 + kConvTok - 1 (zero where outside the tensor)
    f32x4 bx[kConvTok + kConvMaxL - 1];
#pragma unroll
    for (int r = 0; r < kConvTok + kConvMaxL - 1; ++r) {
      const long long t = t0 - (kConvMaxL - 1) + r;
      if (t >= 0 && t < T && r >= kConvMaxL - L) {
        const float *row = bcg + t * 3 * H;
        bx[r] = moe::ld4(row + c) * moe::ld4(row + 2 * H + c);
      } else {
        bx[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
#pragma unroll
    for (int u = 0; u < kConvTok; ++u) {
      const long long t = t0 + u;
      if (t >= T) break;
      const int s = (int)(t % seq);
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k = 0; k < kConvMaxL; ++k) {
        if (k >= L || s - (L - 1) + k < 0) continue;
        const f32x4 v = bx[u + (kConvMaxL - L) + k];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_fmaf(v[j], wk[j][k], acc[j]);
      }
      moe::st4(y + t * H + c, moe::ld4(bcg + t * 3 * H + H + c) * acc);
    }
  }
}

// ---------------------------------------------------------------------------
// Synthetic weights on the device (the generator of include/moe_synth.h)
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void synth_normal_kernel(float *dst, size_t n, uint64_t key,
                                                           float sd, uint64_t first) {
  for (size_t i = blockIdx.x * 256ULL + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const uint64_t gi = first + i, p = gi >> 1;
    const uint64_t h1 = mix64(key + 2 * p + 0x632be59bd9b4e019ULL);
    const uint64_t h2 = mix64(key + 2 * p + 1 + 0x632be59bd9b4e019ULL);
    const double u1 = (double)((h1 >> 11) + 1) * 0x1.0p-53;
    const double u2 = (double)(h2 >> 11) * 0x1.0p-53;
    const double r = sqrt(-2.0 * log(u1));
    const double a = 6.283185307179586476925286766559 * u2;
    dst[i] = (float)((double)sd * ((gi & 1) ? r * sin(a) : r * cos(a)));
  }
}

__global__ __launch_bounds__(256) void fill_kernel(float *dst, size_t n, float v) {
  for (size_t i = blockIdx.x * 256ULL + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = v;
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

static hipError_t lds_attr(const void *fn, size_t bytes) {
  if (bytes <= 65536) return hipSuccess;
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

template <int BM, bool RES>
static hipError_t gemm_launch(const GemmArgs &g, hipStream_t st) {
  using TL = moe::Tile<BM>;
  const size_t lds = TL::LDS_FLOATS * sizeof(float);
  const void *fn = reinterpret_cast<const void *>(&gemm_nt_kernel<BM, RES>);
  const hipError_t e = lds_attr(fn, lds);
  if (e != hipSuccess) return e;
  const int tiles = ((g.M + BM - 1) / BM) * (g.N / TL::BN);
  hipLaunchKernelGGL((gemm_nt_kernel<BM, RES>), dim3(tiles), dim3(kThreads), lds, st, g);
  return hipGetLastError();
}

// 64-row tiles for small M (the LM head's batch of last tokens), 128 above.
constexpr int kGemmSmallM = 1024;

hipError_t launch_gemm_nt(const float *A, const float *B, float *C, const float *R, int M, int N,
                          int K, hipStream_t st) {
  if (M <= 0) return hipSuccess;
  if (N <= 0 || K <= 0 || N % 128 != 0 || K % 32 != 0) return hipErrorInvalidValue;
  if ((size_t)M * K * sizeof(float) >= moe::kTileOOB || (size_t)M * N * sizeof(float) >= moe::kTileOOB)
    return hipErrorInvalidValue;
  const GemmArgs g{A, B, C, R, M, N, K};
  if (M <= kGemmSmallM) return R ? gemm_launch<64, true>(g, st) : gemm_launch<64, false>(g, st);
  return R ? gemm_launch<128, true>(g, st) : gemm_launch<128, false>(g, st);
}

hipError_t launch_embed(const int *ids, const float *table, float *h, int T, int H, int V, int *bad,
                        hipStream_t st) {
  if (T <= 0) return hipSuccess;
  if (H % 4 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(embed_kernel, dim3(T), dim3(256), 0, st, ids, table, h, H / 4, V, bad);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(const float *x, long long x_stride, const float *w, float *y,
                               long long y_stride, int rows, int dim, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3((rows + kNormRows - 1) / kNormRows),
                     dim3(moe::kNormThreads), 0, st, x, x_stride, w, y, y_stride, rows, dim);
  return hipGetLastError();
}

hipError_t launch_qk_norm_rope(float *qkv, int ld, const float *qw, const float *kw,
                               const float *cos_t, const float *sin_t, int batch, int seq,
                               int heads, int kv_heads, int k_col, hipStream_t st) {
  const long long ntok = (long long)batch * seq;
  if (ntok <= 0) return hipSuccess;
  const long long grid = (ntok + kRopeTokens - 1) / kRopeTokens;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)grid), dim3(256), 0, st, qkv, ld, qw, kw,
                     cos_t, sin_t, (int)ntok, seq, heads, heads + kv_heads, k_col);
  return hipGetLastError();
}

hipError_t launch_attention(const float *qkv, int ld, float *out, int batch, int seq, int heads,
                            int kv_heads, int k_col, int v_col, hipStream_t st) {
  if (batch <= 0 || seq <= 0) return hipSuccess;
  if (kv_heads <= 0 || heads != 4 * kv_heads) return hipErrorInvalidValue;
  const int qblocks = (seq + kAttnQB - 1) / kAttnQB;
  const long long grid = (long long)batch * kv_heads * qblocks;
  hipLaunchKernelGGL(attention_kernel, dim3((unsigned)grid), dim3(kAttnThreads), 0, st, qkv, ld,
                     out, heads * kHeadDim, seq, kv_heads, heads / kv_heads, qblocks, k_col, v_col);
  return hipGetLastError();
}

hipError_t launch_shortconv(const float *bcg, const float *w, float *y, int batch, int seq, int H,
                            int L, hipStream_t st) {
  const long long T = (long long)batch * seq;
  if (T <= 0) return hipSuccess;
  if (H % 4 != 0 || L <= 0 || L > kConvMaxL) return hipErrorInvalidValue;
  const long long n = (T + kConvTok - 1) / kConvTok * (H / 4);
  const long long grid = std::min<long long>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(shortconv_kernel, dim3((unsigned)grid), dim3(256), 0, st, bcg, w, y, T, seq,
                     H, L);
  return hipGetLastError();
}

static uint64_t host_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

hipError_t launch_synth_normal(float *dst, size_t n, uint64_t seed, uint64_t stream, float sd,
                               uint64_t first, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const uint64_t key = host_mix64(host_mix64(seed) ^ (stream * 0x9E3779B97F4A7C15ULL));
  const size_t grid = std::min<size_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(synth_normal_kernel, dim3((unsigned)grid), dim3(256), 0, st, dst, n, key, sd,
                     first);
  return hipGetLastError();
}

hipError_t launch_fill(float *dst, size_t n, float v, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const size_t grid = std::min<size_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)grid), dim3(256), 0, st, dst, n, v);
  return hipGetLastError();
}

}  // namespace lfm
