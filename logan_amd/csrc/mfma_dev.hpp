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

}  // namespace lh
