// Device helpers shared by the HIP kernels of this library: vector types,
// buffer-resource constants, agent-scope atomics and cross-block hand-off,
// and the bit-exact RMSNorm reduction of the reference's rms_norm_kernel.
#pragma once

#include "moe_internal.h"

namespace moe {

typedef float floatx16 __attribute__((ext_vector_type(16)));
// Native 4-wide vector for values held in registers across loop iterations
// (HIP's float4 is a union-based struct that the optimiser may leave in
// scratch memory when it is carried around a loop).
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 ld4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }
__device__ __forceinline__ void st4(float *p, f32x4 v) { *reinterpret_cast<f32x4 *>(p) = v; }

// Buffer-resource word 3 for raw (untyped) buffer access on CDNA, and the
// cache-policy bit that makes a store agent-coherent (written through L2).
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr int kCachePolicySc1 = 16;

// ---------------------------------------------------------------------------
// Cross-block synchronisation (agent scope: coherent across the 8 XCD L2s)
// ---------------------------------------------------------------------------

// Coherent read without ordering: polling with acquire loads would invalidate
// the L2 on every poll; the wait does one acquire fence after it succeeds.
__device__ __forceinline__ int load_relaxed(const int *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int fetch_add(int *p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block barrier that orders LDS only: each wave waits for its own LDS
// operations, not for its outstanding global loads and atomics, whose
// results are waited for where they are used (a full __syncthreads waits for
// those too).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Task-queue claim: the index publishes no data, so no fence is needed.
__device__ __forceinline__ int claim(int *p) {
  return __hip_atomic_fetch_add(p, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-block hand-off inside one kernel.  Data another block reads before the
// kernel ends is written with agent-scope stores (write-through to the
// device-coherent level, sc1), so publishing it needs no L2 writeback: a
// release fence here would write back the whole XCD L2 per task, which costs
// ~10x the HBM time of a weight-streaming task.  The signal waits for the
// block's stores to complete and then counts; the consumer's single acquire
// fence drops stale L2/L1 lines before it reads.
__device__ __forceinline__ void st_agent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(int *p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte agent-scope stores through a buffer resource: one sc1 store per
// float4 (a dword-wide atomic store per element would send 4 write
// transactions per 16 bytes), and the descriptor's byte range drops any store
// past the end of the buffer.
struct AgentOut {
  __amdgpu_buffer_rsrc_t rsrc;
  __device__ AgentOut(float *base, uint32_t bytes)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(base, 0, (int)bytes, kBufferRsrcWord3)) {}
  __device__ void store(uint32_t byte_off, f32x4 v) const {
    __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, byte_off, 0, kCachePolicySc1);
  }
};

// Block-wide: wait until *p >= target (thread 0 polls), then acquire.
__device__ inline void block_wait(const int *p, int target, int limit, int *err) {
  if (threadIdx.x == 0) {
    int spins = 0;
    while (load_relaxed(p) < target) {
      __builtin_amdgcn_s_sleep(8);
      if (++spins > limit) {
        __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
}

// Block-wide: once every thread's agent-scope stores have completed, count one.
__device__ inline void block_signal(int *p) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(p, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Post-attention RMSNorm (rms_norm_kernel, layer.cu:144-193), bit for bit:
// 256 threads per row; thread t accumulates h[i]^2 for i = t, t+256, ... with
// FMA (nvcc contracts "sum_sq += src[i] * src[i]"); each group of 32 threads
// (a CUDA warp) folds its sums with shuffle-down at 16, 8, 4, 2, 1, where a
// lane whose source lies outside its 32 keeps its own value; the first group
// folds the 8 group sums (the rest 0) at 4, 2, 1; rms = 1 / sqrt(sum / H +
// 1e-5) with IEEE division and square root; x = (h * rms) * weight.
// ---------------------------------------------------------------------------
constexpr int kNormThreads = 256;
constexpr int kNormGroups = kNormThreads / 32;
constexpr float kNormEps = 1e-5f;  // layer.cu:189 (RMS_NORM_EPS, config.h)

// Sum of the 256 threads' partials of NR rows at once; every thread gets the
// totals in tot[].  s_grp: [NR][kNormGroups] LDS scratch.  Block of 256.
template <int NR>
__device__ __forceinline__ void norm_totals(float (&part)[NR], float *s_grp, float *s_tot) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int m = 0; m < NR; ++m) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) part[m] += __shfl_down(part[m], off, 32);
    if ((tid & 31) == 0) s_grp[m * kNormGroups + (tid >> 5)] = part[m];
  }
  __syncthreads();
  if (tid < 32) {
#pragma unroll
    for (int m = 0; m < NR; ++m) {
      float v = tid < kNormGroups ? s_grp[m * kNormGroups + tid] : 0.0f;
#pragma unroll
      for (int off = kNormGroups / 2; off > 0; off >>= 1) v += __shfl_down(v, off, 32);
      if (tid == 0) s_tot[m] = v;
    }
  }
  __syncthreads();
}

__device__ __forceinline__ float norm_rms(float total, int H) {
#pragma clang fp contract(off)
  return 1.0f / sqrtf(total / (float)H + kNormEps);
}

// dst_m = rmsnorm(src_m) * w for NR rows of dim floats (row m valid when
// m < nrows), 256 threads.  Thread t holds row elements t, t+256, ... in
// registers (up to kNormRegs per row, so every load is in flight before the
// first FMA) and sums their squares in that order; rows longer than
// 256 * kNormRegs are read in a loop instead.  s_grp [NR][kNormGroups],
// s_tot [NR]: LDS scratch.  dst may alias src.
constexpr int kNormRegs = 8;

template <int NR>
__device__ __forceinline__ void norm_rows(const float *const (&src)[NR], float *const (&dst)[NR],
                                          int nrows, const float *w, int dim, float *s_grp,
                                          float *s_tot) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x;
  float part[NR];
  if (dim <= kNormThreads * kNormRegs) {
    float v[NR][kNormRegs];
#pragma unroll
    for (int m = 0; m < NR; ++m)
#pragma unroll
      for (int j = 0; j < kNormRegs; ++j) {
        const int i = tid + j * kNormThreads;
        v[m][j] = (m < nrows && i < dim) ? src[m][i] : 0.0f;
      }
#pragma unroll
    for (int m = 0; m < NR; ++m) {
      part[m] = 0.0f;
#pragma unroll
      for (int j = 0; j < kNormRegs; ++j)
        if (tid + j * kNormThreads < dim) part[m] = __builtin_fmaf(v[m][j], v[m][j], part[m]);
    }
    norm_totals<NR>(part, s_grp, s_tot);
#pragma unroll
    for (int m = 0; m < NR; ++m) {
      if (m >= nrows) break;
      const float rms = norm_rms(s_tot[m], dim);
#pragma unroll
      for (int j = 0; j < kNormRegs; ++j) {
        const int i = tid + j * kNormThreads;
        if (i < dim) dst[m][i] = (v[m][j] * rms) * w[i];
      }
    }
    return;
  }
#pragma unroll
  for (int m = 0; m < NR; ++m) {
    part[m] = 0.0f;
    if (m < nrows)
      for (int i = tid; i < dim; i += kNormThreads) part[m] = __builtin_fmaf(src[m][i], src[m][i], part[m]);
  }
  norm_totals<NR>(part, s_grp, s_tot);
#pragma unroll
  for (int m = 0; m < NR; ++m) {
    if (m >= nrows) break;
    const float rms = norm_rms(s_tot[m], dim);
    for (int i = tid; i < dim; i += kNormThreads) dst[m][i] = (src[m][i] * rms) * w[i];
  }
}

// layer.cu:728 d_silu_opt.
__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

}  // namespace moe
