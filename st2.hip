#include <hip/hip_runtime.h>
typedef float f4 __attribute__((ext_vector_type(4)));
__global__ void e(float* p, f4 v) {
  __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(p, 0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, threadIdx.x * 16, 0, 16);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, threadIdx.x * 16 + 4096, 0, 1);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, threadIdx.x * 16 + 8192, 0, 2);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, threadIdx.x * 16 + 12288, 0, 17);
}
