// Host-side helpers of the decoder-model C-ABI (include/lfm_capi.h): the
// rotary tables (computed with the host's float libm, as the reference does)
// and the synthetic-weight naming rules.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstring>

#include "lfm_capi.h"

extern "C" {

// RotaryEmbedding::init_gpu, layer.cu:1167-1178: for position i and column
// j < head_dim/2, theta = powf(ROPE_THETA, -2.0f * j / head_dim) with j and
// head_dim converted to float, angle = (float)i * theta, and the float
// overloads cos/sin of the float angle (libm cosf/sinf), stored in columns j
// and j + head_dim/2.
int lfm_rope_tables(float *cos_out, float *sin_out, int max_pos, int head_dim, float theta) {
  if (!cos_out || !sin_out || max_pos < 0 || head_dim <= 0 || head_dim % 2 != 0)
    return MOE_ERR_INVALID_ARG;
  const int half = head_dim / 2;
  for (int j = 0; j < half; ++j) {
    const float th = powf(theta, -2.0f * (float)j / (float)head_dim);
    for (int i = 0; i < max_pos; ++i) {
      const float angle = (float)i * th;
      const float c = cosf(angle), s = sinf(angle);
      cos_out[(size_t)i * head_dim + j] = c;
      cos_out[(size_t)i * head_dim + j + half] = c;
      sin_out[(size_t)i * head_dim + j] = s;
      sin_out[(size_t)i * head_dim + j + half] = s;
    }
  }
  return MOE_OK;
}

uint64_t lfm_synth_stream_of(const char *name) {
  uint64_t h = 0xcbf29ce484222325ULL;  // FNV-1a 64
  for (const char *p = name ? name : ""; *p; ++p) {
    h ^= (unsigned char)*p;
    h *= 0x100000001b3ULL;
  }
  return h;
}

int lfm_synth_is_norm(const char *name) {
  static const char kSuffix[] = "norm.weight";
  if (!name) return 0;
  const size_t n = strlen(name), m = sizeof(kSuffix) - 1;
  return n >= m && strcmp(name + n - m, kSuffix) == 0;
}

int lfm_synth_tensor(uint64_t seed, const char *name, float std_dev, float *host_out, size_t n) {
  if (!name || (n && !host_out)) return MOE_ERR_INVALID_ARG;
  if (n == 0) return MOE_OK;
  float *d = nullptr;
  if (hipMalloc(&d, n * sizeof(float)) != hipSuccess) {
    (void)hipGetLastError();
    return MOE_ERR_OUT_OF_MEMORY;
  }
  int rc = lfm_synth_is_norm(name)
               ? lfm_fill(d, n, 1.0f, nullptr)
               : lfm_synth_normal(d, n, seed, lfm_synth_stream_of(name), std_dev, 0, nullptr);
  if (rc == MOE_OK && hipMemcpy(host_out, d, n * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess)
    rc = MOE_ERR_HIP;
  (void)hipFree(d);
  return rc;
}

}  // extern "C"
