// C-ABI of the decoder-model kernels (include/lfm_capi.h): argument checks
// and launches on the caller's stream, no host synchronisation.  Host-only
// helpers (rotary tables, synthetic tensor names) are in lfm_host.cpp; the
// model handle (lfm_model_*) wraps LFM2Model in model.cpp.
#include "lfm_capi.h"

#include <stdint.h>

#include "lfm_internal.h"

namespace {

bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

int launch_status(hipError_t e) {
  if (e == hipSuccess) return MOE_OK;
  (void)hipGetLastError();
  return e == hipErrorInvalidValue ? MOE_ERR_UNSUPPORTED : MOE_ERR_HIP;
}

hipStream_t S(moe_stream_t s) { return static_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

int lfm_gemm_nt(const float *A, const float *B, float *C, const float *R, int M, int N, int K,
                moe_stream_t stream) {
  if (M < 0 || N <= 0 || K <= 0) return MOE_ERR_INVALID_ARG;
  if (M == 0) return MOE_OK;
  if (!A || !B || !C || !al16(A) || !al16(B) || !al16(C) || (R && !al16(R)))
    return MOE_ERR_INVALID_ARG;
  if (C == A || C == B) return MOE_ERR_INVALID_ARG;  // tiles read A/B while others write C
  if (N % 128 != 0 || K % 32 != 0) return MOE_ERR_UNSUPPORTED;
  if ((size_t)M * K >= ((size_t)1 << 30) || (size_t)M * N >= ((size_t)1 << 30))
    return MOE_ERR_UNSUPPORTED;
  return launch_status(lfm::launch_gemm_nt(A, B, C, R, M, N, K, S(stream)));
}

int lfm_embed(const int *ids, const float *table, float *h, int num_tokens, int hidden, int vocab,
              int *bad_flag, moe_stream_t stream) {
  if (num_tokens < 0 || hidden <= 0 || vocab <= 0) return MOE_ERR_INVALID_ARG;
  if (num_tokens == 0) return MOE_OK;
  if (!ids || !table || !h || !al16(table) || !al16(h)) return MOE_ERR_INVALID_ARG;
  if (hidden % 4 != 0) return MOE_ERR_UNSUPPORTED;
  return launch_status(lfm::launch_embed(ids, table, h, num_tokens, hidden, vocab, bad_flag,
                                         S(stream)));
}

int lfm_rmsnorm(const float *x, long long x_stride, const float *weight, float *y,
                long long y_stride, int rows, int dim, moe_stream_t stream) {
  if (rows < 0 || dim <= 0 || x_stride < dim || y_stride < dim) return MOE_ERR_INVALID_ARG;
  if (rows == 0) return MOE_OK;
  if (!x || !weight || !y) return MOE_ERR_INVALID_ARG;
  return launch_status(
      lfm::launch_rmsnorm_rows(x, x_stride, weight, y, y_stride, rows, dim, S(stream)));
}

int lfm_qk_norm_rope(float *qkv, int ld, const float *q_weight, const float *k_weight,
                     const float *cos_table, const float *sin_table, int batch, int seq,
                     int heads, int kv_heads, int k_col, moe_stream_t stream) {
  if (batch < 0 || seq < 0 || heads <= 0 || kv_heads <= 0) return MOE_ERR_INVALID_ARG;
  if (batch == 0 || seq == 0) return MOE_OK;
  if (!qkv || !q_weight || !k_weight || !cos_table || !sin_table) return MOE_ERR_INVALID_ARG;
  if (!al16(qkv) || !al16(q_weight) || !al16(k_weight) || !al16(cos_table) || !al16(sin_table) ||
      ld % 4 != 0 || k_col % 4 != 0)
    return MOE_ERR_INVALID_ARG;
  if (k_col < heads * 64 || ld < k_col + kv_heads * 64) return MOE_ERR_INVALID_ARG;
  if (heads + kv_heads > 64) return MOE_ERR_UNSUPPORTED;
  return launch_status(lfm::launch_qk_norm_rope(qkv, ld, q_weight, k_weight, cos_table, sin_table,
                                                batch, seq, heads, kv_heads, k_col, S(stream)));
}

int lfm_attention(const float *qkv, int ld, float *out, int batch, int seq, int heads,
                  int kv_heads, int k_col, int v_col, moe_stream_t stream) {
  if (batch < 0 || seq < 0 || heads <= 0 || kv_heads <= 0) return MOE_ERR_INVALID_ARG;
  if (batch == 0 || seq == 0) return MOE_OK;
  if (!qkv || !out || !al16(qkv) || !al16(out) || ld % 4 != 0) return MOE_ERR_INVALID_ARG;
  if (k_col < heads * 64 || v_col < k_col + kv_heads * 64 || ld < v_col + kv_heads * 64 ||
      k_col % 4 != 0 || v_col % 4 != 0)
    return MOE_ERR_INVALID_ARG;
  if (heads != 4 * kv_heads) return MOE_ERR_UNSUPPORTED;
  if ((const void *)out == (const void *)qkv) return MOE_ERR_INVALID_ARG;
  return launch_status(
      lfm::launch_attention(qkv, ld, out, batch, seq, heads, kv_heads, k_col, v_col, S(stream)));
}

int lfm_shortconv(const float *bcg, const float *conv_weight, float *y, int batch, int seq,
                  int hidden, int kernel, moe_stream_t stream) {
  if (batch < 0 || seq < 0 || hidden <= 0 || kernel <= 0) return MOE_ERR_INVALID_ARG;
  if (batch == 0 || seq == 0) return MOE_OK;
  if (!bcg || !conv_weight || !y || !al16(bcg) || !al16(y)) return MOE_ERR_INVALID_ARG;
  if ((const void *)y == (const void *)bcg) return MOE_ERR_INVALID_ARG;
  if (hidden % 4 != 0) return MOE_ERR_UNSUPPORTED;
  return launch_status(
      lfm::launch_shortconv(bcg, conv_weight, y, batch, seq, hidden, kernel, S(stream)));
}

int lfm_synth_normal(float *dst, size_t n, uint64_t seed, uint64_t stream_id, float std_dev,
                     uint64_t first, moe_stream_t stream) {
  if (n == 0) return MOE_OK;
  if (!dst) return MOE_ERR_INVALID_ARG;
  return launch_status(lfm::launch_synth_normal(dst, n, seed, stream_id, std_dev, first, S(stream)));
}

int lfm_fill(float *dst, size_t n, float value, moe_stream_t stream) {
  if (n == 0) return MOE_OK;
  if (!dst) return MOE_ERR_INVALID_ARG;
  return launch_status(lfm::launch_fill(dst, n, value, S(stream)));
}

}  // extern "C"
