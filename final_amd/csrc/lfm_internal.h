// Launchers of the decoder-model kernels around the MoE block (lfm_kernels.hip),
// shared with the C-ABI host code (lfm_capi.hip).  Not installed; the public
// boundary is include/lfm_capi.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lfm {

// C[M][N] = A[M][K] . B[N][K]^T (+ R[M][N] when R != null; R may alias C).
// N % 128 == 0, K % 32 == 0, M*K*4 and M*N*4 below 0xFF000000.
hipError_t launch_gemm_nt(const float *A, const float *B, float *C, const float *R, int M,
                          int N, int K, hipStream_t st);

// h[t][:] = table[ids[t]][:]; ids outside [0, V) give a zero row and set
// *bad = 1 (bad may be null).  H % 4 == 0.
hipError_t launch_embed(const int *ids, const float *table, float *h, int T, int H, int V,
                        int *bad, hipStream_t st);

// y[r][:] = rmsnorm(x[r][:]) * w for rows r < rows, row r of x at x + r*x_stride,
// of y at y + r*y_stride (floats); dim elements per row.
hipError_t launch_rmsnorm_rows(const float *x, long long x_stride, const float *w, float *y,
                               long long y_stride, int rows, int dim, hipStream_t st);

// In place on qkv [T][ld]: the heads of q (columns [0, heads*64)) and of k
// (columns [k_col, k_col + kv_heads*64)) are RMS-normalised with qw / kw [64]
// and rotated by the position s = t % seq (cos/sin [max_pos][64]).
hipError_t launch_qk_norm_rope(float *qkv, int ld, const float *qw, const float *kw,
                               const float *cos_t, const float *sin_t, int batch, int seq,
                               int heads, int kv_heads, int k_col, hipStream_t st);

// out[t][h*64 + d] = causal softmax(q_h k_g^T / 8) v_g for the kv head g = h /
// (heads / kv_heads), over the keys of t's own sequence; q, k, v read from qkv
// [T][ld] at columns h*64, k_col + g*64, v_col + g*64.  head_dim 64.
hipError_t launch_attention(const float *qkv, int ld, float *out, int batch, int seq, int heads,
                            int kv_heads, int k_col, int v_col, hipStream_t st);

// Short-conv mix: with B, C, g the three column blocks of bcg [T][3H],
// y[t][h] = C[t][h] * sum_{k<L, s-L+1+k >= 0} (B*g)[t-L+1+k][h] * w[h][k]
// (s = t % seq, FMA chain over k ascending from 0).  H % 4 == 0.
hipError_t launch_shortconv(const float *bcg, const float *w, float *y, int batch, int seq,
                            int H, int L, hipStream_t st);

// dst[i] = sd * N(0,1) sample (first + i) of (seed, stream), the generator of
// include/moe_synth.h evaluated on the device.
hipError_t launch_synth_normal(float *dst, size_t n, uint64_t seed, uint64_t stream, float sd,
                               uint64_t first, hipStream_t st);
hipError_t launch_fill(float *dst, size_t n, float v, hipStream_t st);

}  // namespace lfm
