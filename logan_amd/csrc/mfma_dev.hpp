// MFMA operand builders for MLX-affine codes on gfx950
// (v_mfma_f32_16x16x32_bf16: lane l holds row / column l % 16 and 8
// consecutive k of slice l / 16; the accumulator element i of lane l is row
// 4 * (l / 16) + i, column l % 16). Any permutation of k inside a lane's 8 is
// allowed as long as both operands use it.
//   * 8-bit codes: exact bf16 values through v_cvt_f32_ubyteN, natural order;
//   * 4-bit codes: 0x3F80 | code << 3 = 1 + code/16, pairs (nibble p, p+4) of
//     a dword; the activation operand is permuted to match (a_nibble_order)
//     and the sum of the activations (an MFMA against ones) removes the 1s.
#pragma once

#include "affine_dev.hpp"

namespace lh {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  u32x4_t v = {a, b, c, d};
  return __builtin_bit_cast(bf16x8_t, v);
}

// B operand of one MFMA from one dword of 8 nibbles: pair p = nibbles (p, p+4)
// at mantissa bits 3..6 of both halves.
__device__ __forceinline__ bf16x8_t b_from_nibbles(uint32_t w, const UnpackConsts &kc) {
  return as_bf16x8(((w << 3) & kc.m4) | kc.magic, ((w >> 1) & kc.m4) | kc.magic,
                   ((w >> 5) & kc.m4) | kc.magic, ((w >> 9) & kc.m4) | kc.magic);
}

// A operand matching b_from_nibbles: from 8 consecutive bf16 x (4 dwords),
// pairs (x_p, x_{p+4}).
__device__ __forceinline__ bf16x8_t a_nibble_order(uint4 d) {
  return as_bf16x8(__builtin_amdgcn_perm(d.z, d.x, 0x05040100u),
                   __builtin_amdgcn_perm(d.z, d.x, 0x07060302u),
                   __builtin_amdgcn_perm(d.w, d.y, 0x05040100u),
                   __builtin_amdgcn_perm(d.w, d.y, 0x07060302u));
}

// B operand from two dwords of 8-bit codes (codes in natural order).
__device__ __forceinline__ bf16x8_t b_from_bytes(uint32_t w0, uint32_t w1) {
  uint32_t q[4];
  const uint32_t ws[2] = {w0, w1};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const uint32_t f0 = __float_as_uint((float)(ws[t] & 255u));
    const uint32_t f1 = __float_as_uint((float)((ws[t] >> 8) & 255u));
    const uint32_t f2 = __float_as_uint((float)((ws[t] >> 16) & 255u));
    const uint32_t f3 = __float_as_uint((float)(ws[t] >> 24));
    q[2 * t + 0] = __builtin_amdgcn_perm(f1, f0, 0x07060302u);
    q[2 * t + 1] = __builtin_amdgcn_perm(f3, f2, 0x07060302u);
  }
  return as_bf16x8(q[0], q[1], q[2], q[3]);
}

template <int BITS>
struct SkRaw;
template <>
struct SkRaw<4> {
  uint2 v;  // 16 codes
};
template <>
struct SkRaw<8> {
  uint4 v;  // 16 codes
};
template <>
struct SkRaw<5> {
  uint32_t w[3];  // 96 bits holding 16 codes from bit 0 or 16 (lane group parity)
};
template <>
struct SkRaw<6> {
  uint32_t w[3];  // 16 codes, 96 bits
};

// B operand pairs (codes 2p, 2p + 1, natural order) of 5/6-bit codes as
// 0x3F80 | code << S (S = 2: 1 + code/32; S = 1: 1 + code/64) from a 96-bit
// window whose first code starts at bit `sh`.
template <int BITS>
__device__ __forceinline__ void b_from_window(const uint32_t (&w)[3], int sh, bf16x8_t &b0, bf16x8_t &b1) {
  constexpr int S = BITS == 5 ? 2 : 1;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  // shift the window so code 0 sits at bit 0 (sh is 0 or 16)
  const uint32_t v0 = __builtin_amdgcn_alignbit(w[1], w[0], sh);
  const uint32_t v1 = __builtin_amdgcn_alignbit(w[2], w[1], sh);
  const uint32_t v2 = w[2] >> sh;
  const uint32_t win[3] = {v0, v1, v2};
  uint32_t q[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    uint32_t c[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int bit = (2 * p + t) * BITS, i = bit >> 5, o = bit & 31;
      uint32_t v = win[i] >> o;
      if (o + BITS > 32) v |= win[i + 1] << (32 - o);
      c[t] = v & mask;
    }
    q[p] = 0x3F803F80u | (c[0] << S) | (c[1] << (16 + S));
  }
  b0 = as_bf16x8(q[0], q[1], q[2], q[3]);
  b1 = as_bf16x8(q[4], q[5], q[6], q[7]);
}

// ---------------------------------------------------------------- LDS tiles and steps

// LDS tile of 16 rows of bf16 in 16-byte granules; granule q of row m sits at
// q ^ m inside its aligned run of 16 granules, so the 16 rows of one MFMA
// operand read hit 16 different bank groups.
__device__ __forceinline__ int swz(int m, int q) { return q ^ (m & 15); }

// Direct global -> LDS copy (global_load_lds_dwordx4): lane l of the wave
// writes the 16 bytes at src into lds_wave + 16 l, without passing through
// VGPRs. lds_wave must be wave-uniform; completion is counted by vmcnt, so a
// reader waits with lds_dma_wait() and a barrier.
__device__ __forceinline__ void lds_dma16(const void *src, uint16_t *lds_wave) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_wave, 16, 0, 0);
}
__device__ __forceinline__ void lds_dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Wait for the copies while the N vector-memory instructions issued after the
// last of them may still be in flight (loads complete in issue order). N must
// not exceed the number actually issued after the copies.
template <int N>
__device__ __forceinline__ void lds_dma_wait_behind() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int BITS>
struct MfmaStep {
  // activation operand of one 64-code step (two 8-k slices per lane) from an
  // LDS tile already in the operand order of BITS-bit codes
  static __device__ __forceinline__ void a_ops(const uint16_t *rowp, int q0, int m, bf16x8_t &a0,
                                               bf16x8_t &a1) {
    a0 = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(rowp + 8 * swz(m, q0)));
    a1 = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(rowp + 8 * swz(m, q0 + 1)));
  }
  // position of activation k inside its run of 8 in the operand order
  static __device__ __forceinline__ int op_pos(int k) {
    if constexpr (BITS == 4) {
      const int i = k & 7;
      return (k & ~7) | (i < 4 ? 2 * i : 2 * (i - 4) + 1);
    } else {
      return k;
    }
  }
  static __device__ __forceinline__ void b_ops(const SkRaw<BITS> &r, const UnpackConsts &kc,
                                               bf16x8_t &b0, bf16x8_t &b1) {
    if constexpr (BITS == 4) {
      b0 = b_from_nibbles(r.v.x, kc);
      b1 = b_from_nibbles(r.v.y, kc);
    } else if constexpr (BITS == 8) {
      b0 = b_from_bytes(r.v.x, r.v.y);
      b1 = b_from_bytes(r.v.z, r.v.w);
    } else {
      // 5-bit runs of 16 codes start at bit 0 or 16 of their first dword
      b_from_window<BITS>(r.w, BITS == 5 ? 16 * ((threadIdx.x >> 4) & 1) : 0, b0, b1);
    }
  }
  // the lane's 16 codes [k, k + 16) of a row (k a multiple of 16)
  // (NT: non-temporal loads, for weights read once per launch)
  template <bool NT = false>
  static __device__ __forceinline__ void load_raw(SkRaw<BITS> &r, const uint8_t *row, int k) {
    if constexpr (BITS == 4) {
      r.v = ld_stream<uint2, NT>(reinterpret_cast<const uint2 *>(row + (k >> 1)));
    } else if constexpr (BITS == 8) {
      r.v = ld_stream<uint4, NT>(reinterpret_cast<const uint4 *>(row + k));
    } else {
      // dword holding the first code: 5-bit (k * 5) / 32, 6-bit (k * 6) / 32
      const uint32_t *p = reinterpret_cast<const uint32_t *>(row) + ((k * BITS) >> 5);
      r.w[0] = ld_stream<uint32_t, NT>(p);
      r.w[1] = ld_stream<uint32_t, NT>(p + 1);
      r.w[2] = ld_stream<uint32_t, NT>(p + 2);
    }
  }
  // y += s' D + b' X: D = X + 2^(s-7) sum(c x) for codes at mantissa bit s
  // (4-bit s = 3, 5-bit 2, 6-bit 1), D = sum(c x) for 8-bit
  static __device__ __forceinline__ void fold(f32x4_t &acc, const f32x4_t &d, const f32x4_t &xs,
                                              float s, float b) {
    constexpr float F = BITS == 4 ? 16.f : BITS == 5 ? 32.f : BITS == 6 ? 64.f : 1.f;
    const float s2 = BITS == 8 ? s : F * s;
    const float b2 = BITS == 8 ? b : b - F * s;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = fmaf(b2, xs[i], fmaf(s2, d[i], acc[i]));
  }
};

template <bool FP16>
__device__ __forceinline__ float aux_f32(uint32_t b) {
  if constexpr (FP16) return f16_to_f32(b);
  else return bf16_to_f32(b);
}

__device__ __forceinline__ const bf16x8_t mfma_ones() {
  return as_bf16x8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
}

}  // namespace lh
