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

// In-place RMSNorm of each row of x [nrows][n]:
//   x[r][i] = x[r][i] * (1 / sqrt(sum_i x[r][i]^2 / n + eps)) * w[i]
// (logan-metal/metal/backend_metal.mm:705-714 a_rmsnorm, reached through
// coli_metal_rmsnorm :2147-2166). One 256-thread block per row; the sum of
// squares is a wave DPP/shuffle reduction plus one LDS step.
__global__ __launch_bounds__(kEwThreads) void rmsnorm_f32_kernel(float *x, const float *w, int n,
                                                                 float eps) {
  float *xr = x + (size_t)blockIdx.x * n;
  float s = 0.f;
  for (int i = threadIdx.x; i < n; i += kEwThreads) s = fmaf(xr[i], xr[i], s);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  __shared__ float red[kEwThreads / 64];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kEwThreads / 64; ++i) tot += red[i];
  const float r = 1.0f / sqrtf(tot / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += kEwThreads) xr[i] = xr[i] * r * w[i];
}

// y[i] += a[i] (backend_metal.mm:782-783 a_add, via coli_metal_add :2168-2185)
__global__ __launch_bounds__(kEwThreads) void add_f32_kernel(float *y, const float *a, long long n) {
  const long long i = (long long)blockIdx.x * kEwThreads + threadIdx.x;
  if (i < n) y[i] += a[i];
}

// ---- f32 activations on the bf16 GEMV kernels (hi/lo row pairs) ----------

__global__ __launch_bounds__(kEwThreads) void hilo_split_kernel(HiloBatch b) {
  const HiloJob j = b.j[blockIdx.y];
  const long long i = (long long)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= (long long)j.rows * j.n) return;
  const long long r = i / j.n, c = i % j.n;
  const float v = j.src[i];
  const uint32_t hi = f32_to_bf16_rne(v);
  uint16_t *d = reinterpret_cast<uint16_t *>(j.dst);
  d[(2 * r) * j.n + c] = (uint16_t)hi;
  d[(2 * r + 1) * j.n + c] = (uint16_t)f32_to_bf16_rne(v - bf16_to_f32(hi));  // v - hi is exact
}

__global__ __launch_bounds__(kEwThreads) void hilo_join_kernel(HiloBatch b) {
  const HiloJob j = b.j[blockIdx.y];
  const long long i = (long long)blockIdx.x * kEwThreads + threadIdx.x;
  if (i >= (long long)j.rows * j.n) return;
  const long long r = i / j.n, c = i % j.n;
  reinterpret_cast<float *>(j.dst)[i] = j.src[(2 * r) * j.n + c] + j.src[(2 * r + 1) * j.n + c];
}

static hipError_t hilo_launch(bool split, const HiloBatch &b, hipStream_t st) {
  if (b.n <= 0 || b.n > kHiloMaxJobs) return hipErrorInvalidValue;
  long long most = 0;
  for (int i = 0; i < b.n; ++i) {
    if (b.j[i].rows <= 0 || b.j[i].n <= 0 || !b.j[i].src || !b.j[i].dst) return hipErrorInvalidValue;
    most = max(most, (long long)b.j[i].rows * b.j[i].n);
  }
  const long long blocks = (most + kEwThreads - 1) / kEwThreads;
  if (blocks > 0x7fffffffll) return hipErrorInvalidValue;
  if (split)
    hipLaunchKernelGGL(hilo_split_kernel, dim3((unsigned)blocks, b.n), dim3(kEwThreads), 0, st, b);
  else
    hipLaunchKernelGGL(hilo_join_kernel, dim3((unsigned)blocks, b.n), dim3(kEwThreads), 0, st, b);
  return hipGetLastError();
}

hipError_t launch_hilo_split(const HiloBatch &b, hipStream_t st) { return hilo_launch(true, b, st); }
hipError_t launch_hilo_join(const HiloBatch &b, hipStream_t st) { return hilo_launch(false, b, st); }

hipError_t launch_rmsnorm(float *x, const float *w, int n, int nrows, float eps, hipStream_t st) {
  if (n <= 0 || nrows <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rmsnorm_f32_kernel, dim3((unsigned)nrows), dim3(kEwThreads), 0, st, x, w, n, eps);
  return hipGetLastError();
}

hipError_t launch_add(float *y, const float *a, long long n, hipStream_t st) {
  if (n <= 0) return hipErrorInvalidValue;
  const long long blocks = (n + kEwThreads - 1) / kEwThreads;
  if (blocks > 0x7fffffffll) return hipErrorInvalidValue;
  hipLaunchKernelGGL(add_f32_kernel, dim3((unsigned)blocks), dim3(kEwThreads), 0, st, y, a, n);
  return hipGetLastError();
}

}  // namespace lh
