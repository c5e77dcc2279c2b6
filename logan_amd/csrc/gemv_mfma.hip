// Small-batch MLX-affine product on MFMA (gfx950): y[m] = W x[m] for
// 3 <= M <= 32 activation rows, each weight byte read from HBM once.
//
// Same numerics as the dot2 GEMV (exact codes, f32 accumulation, per-group
// scale and bias factored out: sum_k w_k x_k = s * sum_k c_k x_k + b * sum_k x_k
// over each quantisation group, logan-qwen4/src/lib.rs:3723-3724), with the
// code x activation products on v_mfma_f32_16x16x32_bf16:
//   * the B operand (32 k x 16 weight rows) holds codes as exact bf16 values:
//     8-bit codes through v_cvt_f32_ubyteN (<= 8 significant bits), 4-bit
//     codes as the pattern 0x3F80 | code << 3 = 1 + code/16 (so the product
//     sum is X + sum c x / 16, with X = sum x);
//   * the A operand (16 tokens x 32 k) is the bf16 activations (4-bit: pairs
//     permuted to the code order with one v_perm_b32 per dword);
//   * X = sum x over the same k comes from one more MFMA against a B of ones,
//     already in the accumulator layout, so the per-group fold is two FMAs
//     per output element: y += s' * D + b' * X.
// A wave owns 16 weight rows and a contiguous range of 64-code steps; the
// waves of a block split K and their partial sums are added in wave order
// through LDS (deterministic). Lane l: weight row / token l % 16, k slice
// 16 * (l / 16) + [0, 16) of each 64-code step (two MFMAs of 8 codes each).
// Accumulator element i of lane l is token 4 * (l / 16) + i, row l % 16.
// Tokens past M read the last valid row and are never stored.
#include "lh_internal.hpp"
#include "mfma_dev.hpp"

namespace lh {

struct SkinnyParams {
  const uint8_t *w;
  const uint16_t *sc;
  const uint16_t *bi;
  const uint16_t *x;
  void *y;
  long long row_bytes;
  int N, K, ng, gsteps;  // gsteps = 64-code steps per group
  int fp16, x_stride, M, y_stride, y_bf16;
};

// One batch of kU 64-code steps for R row tiles and MT token tiles: the raw
// loads of a lane.
template <int BITS, int MT, int R, int U>
struct SkBatch {
  SkRaw<BITS> w[U][R];
  uint4 x[U][MT][2];
  uint32_t s[U][R], b[U][R];
};

// MT token tiles of 16 (M <= 16 * MT), R row tiles of 16 per wave, W waves
// per block splitting K, batches of U steps double-buffered in registers.
template <int BITS, int MT, int R, int U, int W>
__global__ __launch_bounds__(W * 64) void affine_skinny_kernel(SkinnyParams p) {
  static_assert(BITS == 4 || BITS == 8, "skinny MFMA path: 4- and 8-bit codes");
  __shared__ __align__(16) float s_part[W > 1 ? (W - 1) * R * MT * 64 * 4 : 1];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * R;
  const uint8_t *wrow[R];
  const uint16_t *srow[R], *brow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(n0 + 16 * r + r16, p.N - 1);
    wrow[r] = p.w + (size_t)row * p.row_bytes;
    srow[r] = p.sc + (size_t)row * p.ng;
    brow[r] = p.bi + (size_t)row * p.ng;
  }
  const uint16_t *xrow[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) xrow[t] = p.x + (size_t)min(16 * t + r16, p.M - 1) * p.x_stride;

  // this wave's 64-code steps [s0, s1), in batches of U
  const int steps = p.K >> 6;
  const int s0 = (int)(((long long)steps * wave) / W), s1 = (int)(((long long)steps * (wave + 1)) / W);
  const int nb = (s1 - s0 + U - 1) / U;
  UnpackConsts kc;
  kc.init();
  const bf16x8_t ones = as_bf16x8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  f32x4_t acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[r][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // loads of batch bi (steps clamped into [s0, s1), x rows of tokens past M
  // clamped to the last row: those accumulator rows are never stored). The
  // loads are unconditional so that the in-order vmcnt stays exact across the
  // pipeline (a conditional issue makes the compiler drain every load).
  auto issue = [&](int bi, SkBatch<BITS, MT, R, U> &B) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = min(s0 + bi * U + u, s1 - 1);
      const int k = st * 64 + 16 * g;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if constexpr (BITS == 4)
          B.w[u][r].v = *reinterpret_cast<const uint2 *>(wrow[r] + (k >> 1));
        else
          B.w[u][r].v = *reinterpret_cast<const uint4 *>(wrow[r] + k);
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        B.x[u][t][0] = *reinterpret_cast<const uint4 *>(xrow[t] + k);
        B.x[u][t][1] = *reinterpret_cast<const uint4 *>(xrow[t] + k + 8);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = min(s0 + bi * U + u, s1 - 1);
      const int gi = st / p.gsteps;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        B.s[u][r] = srow[r][gi];
        B.b[u][r] = brow[r][gi];
      }
    }
  };
  auto step = [&](int bi, const SkBatch<BITS, MT, R, U> &B) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = s0 + bi * U + u < s1;
      bf16x8_t a0[MT], a1[MT];
      f32x4_t xs[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        if constexpr (BITS == 4) {
          a0[t] = a_nibble_order(B.x[u][t][0]);
          a1[t] = a_nibble_order(B.x[u][t][1]);
        } else {
          a0[t] = __builtin_bit_cast(bf16x8_t, B.x[u][t][0]);
          a1[t] = __builtin_bit_cast(bf16x8_t, B.x[u][t][1]);
        }
        const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
        xs[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0[t], ones, z, 0, 0, 0);
        xs[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[t], ones, xs[t], 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        bf16x8_t b0, b1;
        if constexpr (BITS == 4) {
          b0 = b_from_nibbles(B.w[u][r].v.x, kc);
          b1 = b_from_nibbles(B.w[u][r].v.y, kc);
        } else {
          b0 = b_from_bytes(B.w[u][r].v.x, B.w[u][r].v.y);
          b1 = b_from_bytes(B.w[u][r].v.z, B.w[u][r].v.w);
        }
        const float s = live ? aux_to_f32_sel(B.s[u][r], p.fp16) : 0.f;
        const float b = live ? aux_to_f32_sel(B.b[u][r], p.fp16) : 0.f;
        // y += s' D + b' X: 4-bit D = X + sum(c x)/16, 8-bit D = sum(c x)
        const float s2 = BITS == 4 ? 16.f * s : s;
        const float b2 = BITS == 4 ? b - 16.f * s : b;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
          f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0[t], b0, z, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[t], b1, d, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[r][t][i] = fmaf(b2, xs[t][i], fmaf(s2, d[i], acc[r][t][i]));
        }
      }
    }
  };

  if (nb > 0) {
    // batches past the end reload the last step (weights zeroed in the fold)
    SkBatch<BITS, MT, R, U> B0, B1;
    issue(0, B0);
    for (int bi = 0; bi < nb; bi += 2) {
      issue(bi + 1, B1);
      __builtin_amdgcn_sched_barrier(0);
      step(bi, B0);
      issue(bi + 2, B0);
      __builtin_amdgcn_sched_barrier(0);
      step(bi + 1, B1);
    }
  }

  // partial sums of waves 1.. into LDS, wave 0 adds them in wave order
  if constexpr (W > 1) {
    if (wave > 0) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t)
          *reinterpret_cast<float4 *>(&s_part[((((wave - 1) * R + r) * MT + t) * 64 + lane) * 4]) =
              make_float4(acc[r][t][0], acc[r][t][1], acc[r][t][2], acc[r][t][3]);
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 1; w < W; ++w)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const float4 v =
              *reinterpret_cast<const float4 *>(&s_part[((((w - 1) * R + r) * MT + t) * 64 + lane) * 4]);
          acc[r][t][0] += v.x;
          acc[r][t][1] += v.y;
          acc[r][t][2] += v.z;
          acc[r][t][3] += v.w;
        }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = n0 + 16 * r + r16;
    if (n >= p.N) continue;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 16 * t + 4 * g + i;
        if (m < p.M) {
          if (p.y_bf16)
            reinterpret_cast<uint16_t *>(p.y)[(size_t)m * p.y_stride + n] =
                (uint16_t)f32_to_bf16_rne(acc[r][t][i]);
          else
            reinterpret_cast<float *>(p.y)[(size_t)m * p.y_stride + n] = acc[r][t][i];
        }
      }
  }
}

bool affine_skinny_supported(const DevMat &m) {
  if (m.bits != 4 && m.bits != 8) return false;
  if (m.gs <= 0 || m.gs % 64 != 0 || m.I % m.gs != 0) return false;
  if (m.row_bytes != (long long)m.I * m.bits / 8) return false;
  // per-lane loads of 8 (4-bit) / 16 (8-bit) bytes
  const uintptr_t need = m.bits == 4 ? 7 : 15;
  if ((reinterpret_cast<uintptr_t>(m.w) & need) != 0 || (m.row_bytes & (long long)need) != 0) return false;
  return true;
}

#ifndef SKINNY_R
#define SKINNY_R 1
#endif
#ifndef SKINNY_U
#define SKINNY_U 1
#endif

#ifndef SKINNY_WBIG
#define SKINNY_WBIG 8
#endif

template <int BITS, int MT>
static hipError_t skinny_launch(const SkinnyParams &p, hipStream_t st) {
  constexpr int R = SKINNY_R, U = SKINNY_U, WB = SKINNY_WBIG;
  const dim3 grid((p.N + 16 * R - 1) / (16 * R));
  if ((p.K >> 6) >= 4 * WB)
    hipLaunchKernelGGL((affine_skinny_kernel<BITS, MT, R, U, WB>), grid, dim3(64 * WB), 0, st, p);
  else if ((p.K >> 6) >= 32)
    hipLaunchKernelGGL((affine_skinny_kernel<BITS, MT, R, U, 8>), grid, dim3(512), 0, st, p);
  else
    hipLaunchKernelGGL((affine_skinny_kernel<BITS, MT, R, U, 4>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

// M in [1, 32] per launch; x 16-byte aligned rows.
hipError_t launch_affine_skinny(const DevMat &m, const uint16_t *x, int x_stride, int M, void *y,
                                int y_stride, int y_bf16, hipStream_t st) {
  if (!affine_skinny_supported(m) || M <= 0 || M > 32) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return hipErrorInvalidValue;
  SkinnyParams p;
  p.w = m.w;
  p.sc = m.sc;
  p.bi = m.bi;
  p.x = x;
  p.y = y;
  p.row_bytes = m.row_bytes;
  p.N = m.O;
  p.K = m.I;
  p.ng = m.ng;
  p.gsteps = m.gs / 64;
  p.fp16 = m.fp16;
  p.x_stride = x_stride;
  p.M = M;
  p.y_stride = y_stride;
  p.y_bf16 = y_bf16;
  if (m.bits == 4) return M <= 16 ? skinny_launch<4, 1>(p, st) : skinny_launch<4, 2>(p, st);
  return M <= 16 ? skinny_launch<8, 1>(p, st) : skinny_launch<8, 2>(p, st);
}

}  // namespace lh
