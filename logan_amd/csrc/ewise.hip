// Element-wise SwiGLU between a dense gate/up pair and the down projection:
//   g[i] = silu(g[i]) * u[i],  silu(v) = v / (1 + exp(-v))
// (logan-metal/metal/backend_metal.mm:698-699 moe_silu, reached through
// coli_metal_silu_mul :2187-2203; silu as logan-qwen4/src/lib.rs:4516-4518).
// f32 arithmetic; bf16 operands are widened exactly and the result rounded
// to bf16 (RNE). Each thread handles 8 consecutive elements with 128-bit
// loads; the tail is handled element-wise by the same threads.
#include "affine_dev.hpp"
#include "lh_internal.hpp"

namespace lh {

constexpr int kEwThreads = 256;

__global__ __launch_bounds__(kEwThreads) void silu_mul_f32_kernel(float *g, const float *u, long long n) {
  const long long i0 = ((long long)blockIdx.x * kEwThreads + threadIdx.x) * 8;
  if (i0 + 8 <= n) {
    float4 a0 = *reinterpret_cast<const float4 *>(g + i0), a1 = *reinterpret_cast<const float4 *>(g + i0 + 4);
    const float4 b0 = *reinterpret_cast<const float4 *>(u + i0), b1 = *reinterpret_cast<const float4 *>(u + i0 + 4);
    a0.x = silu(a0.x) * b0.x; a0.y = silu(a0.y) * b0.y; a0.z = silu(a0.z) * b0.z; a0.w = silu(a0.w) * b0.w;
    a1.x = silu(a1.x) * b1.x; a1.y = silu(a1.y) * b1.y; a1.z = silu(a1.z) * b1.z; a1.w = silu(a1.w) * b1.w;
    *reinterpret_cast<float4 *>(g + i0) = a0;
    *reinterpret_cast<float4 *>(g + i0 + 4) = a1;
  } else {
    for (long long i = i0; i < n; ++i) g[i] = silu(g[i]) * u[i];
  }
}

__device__ __forceinline__ uint32_t silu_mul_bf16x2(uint32_t gw, uint32_t uw) {
  const float lo = silu(bf16_to_f32(gw & 0xffffu)) * bf16_to_f32(uw & 0xffffu);
  const float hi = silu(bf16_to_f32(gw >> 16)) * bf16_to_f32(uw >> 16);
  return f32_to_bf16_rne(lo) | (f32_to_bf16_rne(hi) << 16);
}

__global__ __launch_bounds__(kEwThreads) void silu_mul_bf16_kernel(uint16_t *g, const uint16_t *u,
                                                                   long long n) {
  const long long i0 = ((long long)blockIdx.x * kEwThreads + threadIdx.x) * 8;
  if (i0 + 8 <= n) {
    uint4 a = *reinterpret_cast<const uint4 *>(g + i0);
    const uint4 b = *reinterpret_cast<const uint4 *>(u + i0);
    a.x = silu_mul_bf16x2(a.x, b.x);
    a.y = silu_mul_bf16x2(a.y, b.y);
    a.z = silu_mul_bf16x2(a.z, b.z);
    a.w = silu_mul_bf16x2(a.w, b.w);
    *reinterpret_cast<uint4 *>(g + i0) = a;
  } else {
    for (long long i = i0; i < n; ++i)
      g[i] = (uint16_t)f32_to_bf16_rne(silu(bf16_to_f32(g[i])) * bf16_to_f32(u[i]));
  }
}

hipError_t launch_silu_mul(void *g, const void *u, long long n, bool bf16, hipStream_t st) {
  if (n <= 0) return hipErrorInvalidValue;
  // the 8-wide path needs 16-byte (bf16) / 32-byte (f32) aligned operands
  const uintptr_t need = 15;
  if (((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(u)) & need) != 0)
    return hipErrorInvalidValue;
  const long long threads = (n + 7) / 8;
  const long long blocks = (threads + kEwThreads - 1) / kEwThreads;
  if (blocks > 0x7fffffffll) return hipErrorInvalidValue;
  if (bf16)
    hipLaunchKernelGGL(silu_mul_bf16_kernel, dim3((unsigned)blocks), dim3(kEwThreads), 0, st,
                       reinterpret_cast<uint16_t *>(g), reinterpret_cast<const uint16_t *>(u), n);
  else
    hipLaunchKernelGGL(silu_mul_f32_kernel, dim3((unsigned)blocks), dim3(kEwThreads), 0, st,
                       reinterpret_cast<float *>(g), reinterpret_cast<const float *>(u), n);
  return hipGetLastError();
}

}  // namespace lh
