#include <hip/hip_runtime.h>
typedef float f4 __attribute__((ext_vector_type(4)));
__global__ void a(f4* p, f4 v) { __builtin_nontemporal_store(v, p + threadIdx.x); }
__global__ void b(float4* p, float4 v) {
  __hip_atomic_store((long long*)(p + threadIdx.x), 5ll, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__global__ void c(f4* p, f4 v) {
  f4* q = p + threadIdx.x;
  asm volatile("global_store_dwordx4 %0, %1, off sc1" :: "v"(q), "v"(v) : "memory");
}
__global__ void d(f4* p, f4 v) { f4 x = __builtin_nontemporal_load(p + threadIdx.x); p[threadIdx.x + 64] = x; }
