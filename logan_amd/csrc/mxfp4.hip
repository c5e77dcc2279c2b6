// MXFP4 (OCP microscaling FP4) GEMV for gfx950: logan-metal's fmt 7, and the
// two- and three-plane residual forms fmt 9 / 10 (y = sum over planes of
// W_p . x). Weights: per plane [O][I/2] bytes, element 2j in the low nibble
// of byte j, an E2M1 code each (sign, two exponent bits, one mantissa bit);
// scales: per plane [O][I/32] E8M0 bytes, scale = the f32 with bits
// byte << 23 (logan-qwen4/src/lib.rs:2932-3038, matmul_mxfp4_bytes /
// matmul_mxfp4_storage; logan-metal/metal/backend_metal.mm:438-459).
//
// One 32-column group is one 16-byte load of codes and one scale byte. The
// codes are turned into exact bf16 pairs by v_cvt_scalef32_pk_bf16_fp4
// (E2M1 values are exact in bf16; scale 1), dotted with x pairs by
// v_dot2_f32_bf16, and the group's sum is scaled by its power of two (exact)
// before it joins the row's f32 sum. f32 activations are split in registers
// into bf16 hi + lo halves (|x - hi - lo| <= 2^-18 |x|) whose products are
// summed. A team of LANES lanes owns U rows at a time; lane l takes the
// groups l, l + LANES, ..., the next group's loads in flight while the
// current one is used. Up to kMx4MaxDescs matrices (each with its own x and
// y) share one launch.
//
// The group-scaled sums equal the reference's per-element sum
// (acc += x * MX4[code] * scale in column order, lib.rs:2948-2961; planes
// added in order, :2985-3038) up to f32 rounding order only while no term or
// partial sum can reach the overflow range and scale and x are finite. A row
// with a group that breaks this (scale byte 255, i.e. scale = +inf, where a
// zero code or zero x gives NaN and terms of both signs give NaN; terms or
// sums that may overflow, whose inf/NaN outcome depends on the summation
// order; inf/NaN activations) is recomputed by one lane in the reference's
// own order, bit for bit. The test uses the group's largest activation
// exponent e (bf16 field, |x| < 2^(e - 126)) and scale byte s: each term is
// below 2^(e + s - 250), a 32-term group below 2^(e + s - 245), the row's
// C groups and at most 3 planes below 2^(e + s - 243 + ceil(log2 C)), so
// e + s <= 370 - ceil(log2 C) keeps every partial sum, in any order, under
// 2^127.
#include "affine_dev.hpp"
#include "lh_internal.hpp"

namespace lh {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

constexpr int kMx4U = 4;  // rows per team

// the 32 codes of one 16-byte group as 16 bf16 pairs, element order
__device__ __forceinline__ void mx4_pairs(const uint4 q, uint32_t (&pr)[16]) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    pr[4 * d + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 0));
    pr[4 * d + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 1));
    pr[4 * d + 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 2));
    pr[4 * d + 3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 3));
  }
}

__device__ __forceinline__ float e8m0(uint32_t b) { return __uint_as_float(b << 23); }

// one group's activation operands: bf16 pairs (and the lo halves for f32 x)
template <bool XF>
struct Mx4X {
  uint32_t hi[16];
  uint32_t lo[XF ? 16 : 1];
  uint32_t xe;  // largest bf16 exponent field among the group's hi halves
};

// largest exponent field of 32 bf16 values held as 16 pairs (an upper bound
// for f32 activations: RNE to bf16 never lowers the exponent)
__device__ __forceinline__ uint32_t mx4_max_exp(const uint32_t (&h)[16]) {
  uint32_t m = h[0] & 0x7fff7fffu;
#pragma unroll
  for (int k = 1; k < 16; ++k)
    m = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(
                                         __builtin_bit_cast(u16x2_t, m),
                                         __builtin_bit_cast(u16x2_t, h[k] & 0x7fff7fffu)));
  return max(m & 0xffffu, m >> 16) >> 7;
}

// one row the reference's way (flagged rows only): each term
// fl(fl(x * MX4) * scale) added in column order, plane results added in
// plane order; x re-read from memory (the f32 original, not its bf16 halves)
template <bool XF>
__device__ __noinline__ float mx4_row_exact(const Mx4Desc d, int row) {
  // no FMA contraction: a product must round (to inf when it overflows)
  // before it is added, as the reference's separate multiply and add do
#pragma clang fp contract(off)
  const int rb = d.I >> 1, ng = d.I >> 5;
  float tot = 0.f;
  for (int p = 0; p < d.planes; ++p) {
    const uint8_t *wr = d.w + (size_t)p * d.wplane + (size_t)row * rb;
    const uint8_t *sr = d.sc + (size_t)p * d.splane + (size_t)row * ng;
    float acc = 0.f;
    for (int j = 0; j < rb; ++j) {
      const f32x2_t v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((uint32_t)wr[j], 1.0f, 0);
      const float scale = e8m0(sr[j >> 4]);
      float x0, x1;
      if constexpr (XF) {
        x0 = reinterpret_cast<const float *>(d.x)[2 * j];
        x1 = reinterpret_cast<const float *>(d.x)[2 * j + 1];
      } else {
        x0 = bf16_to_f32(reinterpret_cast<const uint16_t *>(d.x)[2 * j]);
        x1 = bf16_to_f32(reinterpret_cast<const uint16_t *>(d.x)[2 * j + 1]);
      }
      acc = acc + (x0 * v[0]) * scale;
      acc = acc + (x1 * v[1]) * scale;
    }
    tot = p == 0 ? acc : tot + acc;
  }
  return tot;
}

// one group's activation words as loaded: 32 f32 (8 x 16 bytes) or 32 bf16
template <bool XF>
struct Mx4XRaw {
  uint4 v[XF ? 8 : 4];
};

template <bool XF>
__device__ __forceinline__ void mx4_load_x_raw(const void *x, int c, Mx4XRaw<XF> &r) {
  const uint4 *src = XF ? reinterpret_cast<const uint4 *>(reinterpret_cast<const float *>(x) + 32 * c)
                        : reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(x) + 32 * c);
#pragma unroll
  for (int v = 0; v < (XF ? 8 : 4); ++v) r.v[v] = src[v];
}

template <bool XF>
__device__ __forceinline__ void mx4_x_from_raw(const Mx4XRaw<XF> &r, Mx4X<XF> &o) {
  if constexpr (XF) {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float4 f = __builtin_bit_cast(float4, r.v[v]);
      const float e[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
      for (int q = 0; q < 4; q += 2) {
        const uint32_t h0 = f32_to_bf16_rne(e[q]), h1 = f32_to_bf16_rne(e[q + 1]);
        const uint32_t l0 = f32_to_bf16_rne(e[q] - bf16_to_f32(h0));
        const uint32_t l1 = f32_to_bf16_rne(e[q + 1] - bf16_to_f32(h1));
        o.hi[2 * v + q / 2] = h0 | (h1 << 16);
        o.lo[2 * v + q / 2] = l0 | (l1 << 16);
      }
    }
  } else {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      o.hi[4 * v] = r.v[v].x;
      o.hi[4 * v + 1] = r.v[v].y;
      o.hi[4 * v + 2] = r.v[v].z;
      o.hi[4 * v + 3] = r.v[v].w;
    }
  }
  o.xe = mx4_max_exp(o.hi);
}

template <bool XF>
__device__ __forceinline__ void mx4_load_x(const void *x, int c, Mx4X<XF> &o) {
  Mx4XRaw<XF> r;
  mx4_load_x_raw<XF>(x, c, r);
  mx4_x_from_raw<XF>(r, o);
}

template <int LANES, bool XF>
__global__ __launch_bounds__(256) void mxfp4_gemv_kernel(Mx4Batch b) {
  int di = 0;
  while (di + 1 < b.n && (int)blockIdx.x >= b.block_start[di + 1]) ++di;
  const Mx4Desc d = b.d[di];
  constexpr int TEAMS = 256 / LANES;
  const int lane = threadIdx.x & (LANES - 1), team = threadIdx.x / LANES;
  const int r0 = ((int)blockIdx.x - b.block_start[di]) * TEAMS * kMx4U + team * kMx4U;
  const int C = d.I >> 5;
  const long long rb = d.I >> 1;
  float acc[kMx4U];
#pragma unroll
  for (int u = 0; u < kMx4U; ++u) acc[u] = 0.f;
  float tot[kMx4U];
#pragma unroll
  for (int u = 0; u < kMx4U; ++u) tot[u] = 0.f;
  // rows the group-scaled sums may not serve (see the file comment)
  bool risky[kMx4U];
#pragma unroll
  for (int u = 0; u < kMx4U; ++u) risky[u] = false;
  const uint32_t lim = 370u - (C > 1 ? 32u - (uint32_t)__clz(C - 1) : 0u);
  auto use = [&](int cg, const uint4 (&q)[kMx4U], const uint32_t (&s)[kMx4U], const Mx4X<XF> &xv) {
    if (cg >= C) return;
#pragma unroll
    for (int u = 0; u < kMx4U; ++u) {
      uint32_t pr[16];
      mx4_pairs(q[u], pr);
      float g = 0.f;
#pragma unroll
      for (int k = 0; k < 16; ++k) g = dot2(pr[k], xv.hi[k], g);
      if constexpr (XF) {
#pragma unroll
        for (int k = 0; k < 16; ++k) g = dot2(pr[k], xv.lo[k], g);
      }
      acc[u] = fmaf(g, e8m0(s[u]), acc[u]);  // g * 2^(s - 127) is exact
      risky[u] = risky[u] || s[u] == 255u || xv.xe == 255u || s[u] + xv.xe > lim;
    }
  };
  if (C <= LANES) {
    // One group per lane (rows of up to 32 LANES codes): x first, then the
    // plane's scale bytes and codes of the team's rows, all in flight at
    // once; the weights with non-temporal loads (read once per launch, they
    // leave x and the kernel's code in L2). Loads complete in issue order, so
    // the x conversion waits for x alone.
    const int cc = lane < C ? lane : C - 1;
    Mx4XRaw<XF> xr;
    mx4_load_x_raw<XF>(d.x, cc, xr);
    for (int p = 0; p < d.planes; ++p) {
      const uint8_t *wp = d.w + (size_t)p * d.wplane;
      const uint8_t *sp = d.sc + (size_t)p * d.splane;
      uint4 q[kMx4U];
      uint32_t sb[kMx4U];
#pragma unroll
      for (int u = 0; u < kMx4U; ++u) sb[u] = ld_stream<uint8_t, true>(sp + (size_t)min(r0 + u, d.O - 1) * C + cc);
#pragma unroll
      for (int u = 0; u < kMx4U; ++u)
        q[u] = ld_stream<uint4, true>(reinterpret_cast<const uint4 *>(wp + (size_t)min(r0 + u, d.O - 1) * rb +
                                                                      16 * (size_t)cc));
      __builtin_amdgcn_sched_barrier(0);
      Mx4X<XF> xv;
      mx4_x_from_raw<XF>(xr, xv);
      use(lane, q, sb, xv);
#pragma unroll
      for (int u = 0; u < kMx4U; ++u) {
        tot[u] += team_sum<LANES>(acc[u]);
        acc[u] = 0.f;
      }
    }
  } else
  for (int p = 0; p < d.planes; ++p) {
    const uint8_t *wp = d.w + (size_t)p * d.wplane;
    const uint8_t *sp = d.sc + (size_t)p * d.splane;
    // groups of this lane, one ahead: codes and scale bytes of U rows, then x
    auto load = [&](int c, uint4 (&q)[kMx4U], uint32_t (&s)[kMx4U]) {
      const int cc = c < C ? c : C - 1;
#pragma unroll
      for (int u = 0; u < kMx4U; ++u) {
        const int row = min(r0 + u, d.O - 1);
        s[u] = sp[(size_t)row * C + cc];
        q[u] = *reinterpret_cast<const uint4 *>(wp + (size_t)row * rb + 16 * (size_t)cc);
      }
    };
    uint4 q0[kMx4U], q1[kMx4U];
    uint32_t s0[kMx4U], s1[kMx4U];
    Mx4X<XF> x0, x1;
    int c = lane;
    load(c, q0, s0);
    mx4_load_x<XF>(d.x, c < C ? c : C - 1, x0);
    for (; c < C; c += 2 * LANES) {
      load(c + LANES, q1, s1);
      mx4_load_x<XF>(d.x, c + LANES < C ? c + LANES : C - 1, x1);
      use(c, q0, s0, x0);
      load(c + 2 * LANES, q0, s0);
      mx4_load_x<XF>(d.x, c + 2 * LANES < C ? c + 2 * LANES : C - 1, x0);
      use(c + LANES, q1, s1, x1);
    }
    // plane p's product joins the rows' totals (planes 2, 3 are residual
    // corrections added in order, as the reference adds them)
#pragma unroll
    for (int u = 0; u < kMx4U; ++u) {
      tot[u] += team_sum<LANES>(acc[u]);
      acc[u] = 0.f;
    }
  }
  const uint64_t team_mask = (LANES == 64 ? ~0ull : ((1ull << LANES) - 1)) << ((threadIdx.x & 63) & ~(LANES - 1));
#pragma unroll
  for (int u = 0; u < kMx4U; ++u) {
    const bool redo = (__ballot(risky[u]) & team_mask) != 0ull;
    if (redo && lane == 0 && r0 + u < d.O) tot[u] = mx4_row_exact<XF>(d, r0 + u);
  }
  if (lane == 0) {
#pragma unroll
    for (int u = 0; u < kMx4U; ++u) {
      const int row = r0 + u;
      if (row < d.O) {
        if (b.y_bf16)
          reinterpret_cast<uint16_t *>(d.y)[row] = (uint16_t)f32_to_bf16_rne(tot[u]);
        else
          reinterpret_cast<float *>(d.y)[row] = tot[u];
      }
    }
  }
}

// out[r][c] = MX4[code] * scale for rows [row0, row0 + nrows) of plane 0,
// through the same conversion instruction (then the exact scale multiply)
__global__ __launch_bounds__(256) void mxfp4_dequant_kernel(const uint8_t *w, const uint8_t *sc, int I,
                                                            int row0, int nrows, float *out) {
  const long long n = (long long)nrows * (I >> 1);  // bytes = code pairs
  for (long long t = (long long)blockIdx.x * 256 + threadIdx.x; t < n; t += (long long)gridDim.x * 256) {
    const long long r = t / (I >> 1), j = t % (I >> 1);
    const uint8_t byte = w[(size_t)(row0 + r) * (I >> 1) + j];
    const float s = e8m0(sc[(size_t)(row0 + r) * (I >> 5) + (2 * j) / 32]);
    const f32x2_t v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((uint32_t)byte, 1.0f, 0);
    out[r * I + 2 * j] = v[0] * s;
    out[r * I + 2 * j + 1] = v[1] * s;
  }
}

bool mxfp4_supported(int O, int I, const void *w) {
  return O > 0 && I > 0 && I % 32 == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
}

hipError_t launch_mxfp4_gemv(Mx4Batch &b, bool x_f32, hipStream_t st) {
  if (b.n <= 0 || b.n > kMx4MaxDescs) return hipErrorInvalidValue;
  int cmax = 0;
  for (int i = 0; i < b.n; ++i) {
    const Mx4Desc &d = b.d[i];
    if (!mxfp4_supported(d.O, d.I, d.w) || !d.x || !d.y || d.planes < 1 || d.planes > 3)
      return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(d.x) & 15) != 0) return hipErrorInvalidValue;
    cmax = max(cmax, d.I >> 5);
  }
  const int lanes = cmax <= 16 ? 16 : 64;
  const int rows_per_block = (256 / lanes) * kMx4U;
  b.block_start[0] = 0;
  for (int i = 0; i < b.n; ++i)
    b.block_start[i + 1] = b.block_start[i] + (b.d[i].O + rows_per_block - 1) / rows_per_block;
  const dim3 grid(b.block_start[b.n]);
  if (lanes == 16) {
    if (x_f32) hipLaunchKernelGGL((mxfp4_gemv_kernel<16, true>), grid, dim3(256), 0, st, b);
    else hipLaunchKernelGGL((mxfp4_gemv_kernel<16, false>), grid, dim3(256), 0, st, b);
  } else {
    if (x_f32) hipLaunchKernelGGL((mxfp4_gemv_kernel<64, true>), grid, dim3(256), 0, st, b);
    else hipLaunchKernelGGL((mxfp4_gemv_kernel<64, false>), grid, dim3(256), 0, st, b);
  }
  return hipGetLastError();
}

hipError_t launch_mxfp4_dequant(const uint8_t *w, const uint8_t *sc, int O, int I, int row0,
                                int nrows, float *out, hipStream_t st) {
  if (!mxfp4_supported(O, I, w) || row0 < 0 || nrows <= 0 || row0 + nrows > O) return hipErrorInvalidValue;
  const long long n = (long long)nrows * (I >> 1);
  const int blocks = (int)std::min<long long>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(mxfp4_dequant_kernel, dim3(blocks), dim3(256), 0, st, w, sc, I, row0, nrows, out);
  return hipGetLastError();
}

}  // namespace lh
