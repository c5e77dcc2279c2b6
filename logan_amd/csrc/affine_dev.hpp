// Device-side building blocks for MLX-affine packed rows on gfx950 (CDNA4).
//
// Packed format (logan-qwen4/src/lib.rs:3688-3701, colisource.rs:719-722): a
// row of I codes is I*bits/32 little-endian u32 words holding one LSB-first
// bitstream. A "chunk" here is 32 consecutive codes = exactly `bits` words
// (16/20/24/32 bytes for 4/5/6/8-bit), which always lies inside one
// quantisation group because group sizes are multiples of 32.
//
// Dequantised weight (lib.rs:3723-3724): w = code * scale + bias, f32.
// The chunk dot product is evaluated in the factored form
//     sum_k w_k x_k = scale * sum_k code_k x_k + bias * sum_k x_k
// with the code*x products done by v_dot2c_f32_bf16 on bf16 pairs:
//   * 4/5/6-bit: each half of a pair is the bf16 pattern 0x3F80 | code << s,
//     i.e. exactly 1 + code * 2^(s-7) (code << s stays inside the 7 mantissa
//     bits: s = 3 for 4-bit, 2/1 for 5-bit, 1 for 6-bit). The x operand of
//     that half carries x' = x * 2^(7-s) (exact), so
//         sum (1 + code 2^(s-7)) x' = sum x' + sum code x,
//     and the chunk sum xsp = sum x' (of the values the products actually
//     used) is subtracted once per chunk. Placing the code high in the
//     mantissa keeps that offset small (16x for 4-bit) relative to code*x.
//   * 8-bit: v_cvt_f32_ubyteN gives code exactly in f32; its top 16 bits are
//     the exact bf16 of the code (<= 8 significant bits); no offset.
// All products are exact in f32; sums are f32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lh {

typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a),
                                         __builtin_bit_cast(bf16x2_v, b), c,
                                         false);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

__device__ __forceinline__ float f16_to_f32(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

__device__ __forceinline__ float aux_to_f32(uint32_t b, bool fp16) {
  return fp16 ? f16_to_f32(b) : bf16_to_f32(b);
}

// Same value, both conversions computed and one selected (no branch).
__device__ __forceinline__ float aux_to_f32_sel(uint32_t b, bool fp16) {
  const float h = f16_to_f32(b), f = bf16_to_f32(b);
  return fp16 ? h : f;
}

// Round-to-nearest-even f32 -> bf16 bits (logan-core/src/math.rs:279-283).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Exact bf16 bits of a float that is known to be representable (power-of-two
// scaled bf16 value).
__device__ __forceinline__ uint32_t f32_hi16(float f) {
  return __float_as_uint(f) >> 16;
}

// Which two codes of a 32-code chunk form bf16 pair p (0..15), and the
// mantissa bit s at which each code sits inside its pair half.
template <int BITS>
struct PairMap;

template <>
struct PairMap<4> {
  // word t = p/4 holds codes 8t..8t+7; pair (t,j) = nibbles j and j+4,
  // both placed at mantissa bits 3..6.
  static __device__ __forceinline__ int lo(int p) { return 8 * (p >> 2) + (p & 3); }
  static __device__ __forceinline__ int hi(int p) { return lo(p) + 4; }
  static __device__ __forceinline__ int slo(int) { return 3; }
  static __device__ __forceinline__ int shi(int) { return 3; }
};

template <>
struct PairMap<5> {
  // groups q of 6 codes (30 bits); pair (q,i) = codes 6q+i (mantissa bits
  // 2..6) and 6q+i+3 (bits 1..5, 15 bits later in the stream); pair 15 =
  // codes 30, 31, both at bits 2..6.
  static __device__ __forceinline__ int lo(int p) {
    return p == 15 ? 30 : 6 * (p / 3) + (p % 3);
  }
  static __device__ __forceinline__ int hi(int p) { return p == 15 ? 31 : lo(p) + 3; }
  static __device__ __forceinline__ int slo(int) { return 2; }
  static __device__ __forceinline__ int shi(int p) { return p == 15 ? 2 : 1; }
};

template <>
struct PairMap<6> {
  static __device__ __forceinline__ int lo(int p) { return 2 * p; }
  static __device__ __forceinline__ int hi(int p) { return 2 * p + 1; }
  static __device__ __forceinline__ int slo(int) { return 1; }
  static __device__ __forceinline__ int shi(int) { return 1; }
};

template <>
struct PairMap<8> {
  // exact codes, no offset: x' = x
  static __device__ __forceinline__ int lo(int p) { return 2 * p; }
  static __device__ __forceinline__ int hi(int p) { return 2 * p + 1; }
  static __device__ __forceinline__ int slo(int) { return 7; }
  static __device__ __forceinline__ int shi(int) { return 7; }
};

// x' = x * 2^(7-s): the x-operand scale that pairs with a code at mantissa
// bit s.
__device__ __forceinline__ float xscale(int s) { return (float)(1 << (7 - s)); }

// x operand of one chunk for one activation row: 16 bf16 pairs plus the two
// chunk sums (xs = sum x, xsp = sum x') used by the scale/bias fold.
struct XChunk {
  uint32_t p[16];
  float xs;
  float xsp;
};

// Build the x operand from 32 bf16 activations (raw bits, xb[k] = x[k]).
template <int BITS>
__device__ __forceinline__ void make_xchunk_bf16(XChunk &xc, const uint32_t (&xb)[32]) {
  float s = 0.f, sp = 0.f;
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    const int kl = PairMap<BITS>::lo(p), kh = PairMap<BITS>::hi(p);
    const float vl = bf16_to_f32(xb[kl]), vh = bf16_to_f32(xb[kh]);
    const float xl = vl * xscale(PairMap<BITS>::slo(p));
    const float xh = vh * xscale(PairMap<BITS>::shi(p));
    xc.p[p] = f32_hi16(xl) | (f32_hi16(xh) << 16);
    s += vl + vh;
    sp += xl + xh;
  }
  xc.xs = s;
  xc.xsp = sp;
}

// One pair word of make_xchunk_bf16 (pair p), with its two terms of xs and
// xsp, for callers that split a chunk's conversion across lanes or waves.
template <int BITS>
__device__ __forceinline__ void xpair_bf16(const uint32_t (&xb)[32], int p, uint32_t &word,
                                           float &s, float &sp) {
  const int kl = PairMap<BITS>::lo(p), kh = PairMap<BITS>::hi(p);
  const float vl = bf16_to_f32(xb[kl]), vh = bf16_to_f32(xb[kh]);
  const float xl = vl * xscale(PairMap<BITS>::slo(p));
  const float xh = vh * xscale(PairMap<BITS>::shi(p));
  word = f32_hi16(xl) | (f32_hi16(xh) << 16);
  s = vl + vh;
  sp = xl + xh;
}

// Constants kept in registers so the unpack uses v_and_or_b32 (VOP3 on gfx9
// takes no literal operands).
struct UnpackConsts {
  uint32_t m4;     // 0x00780078: nibble at mantissa bits 3..6 of both halves (SGPR)
  uint32_t m5;     // 0x003E007C: 5-bit code at bits 2..6 (lo) and 1..5 (hi) (SGPR)
  uint32_t magic;  // 0x3F803F80: 1.0 in both halves (VGPR)
  __device__ __forceinline__ void init() {
    m4 = 0x00780078u;
    m5 = 0x003E007Cu;
    magic = 0x3F803F80u;
    asm volatile("" : "+s"(m4));
    asm volatile("" : "+s"(m5));
    asm volatile("" : "+v"(magic));
  }
};

// Unpack one chunk (BITS words) into 16 bf16 pairs in PairMap order.
template <int BITS>
__device__ __forceinline__ void unpack_chunk(uint32_t (&q)[16], const uint32_t (&w)[BITS],
                                             const UnpackConsts &k);

template <>
__device__ __forceinline__ void unpack_chunk<4>(uint32_t (&q)[16], const uint32_t (&w)[4],
                                                const UnpackConsts &k) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    q[4 * t + 0] = ((w[t] << 3) & k.m4) | k.magic;
    q[4 * t + 1] = ((w[t] >> 1) & k.m4) | k.magic;
    q[4 * t + 2] = ((w[t] >> 5) & k.m4) | k.magic;
    q[4 * t + 3] = ((w[t] >> 9) & k.m4) | k.magic;
  }
}

template <>
__device__ __forceinline__ void unpack_chunk<5>(uint32_t (&q)[16], const uint32_t (&w)[5],
                                                const UnpackConsts &k) {
  // window q holds stream bits [30q-2, 30q+30): code 6q+i at bit 2+5i, and
  // code 6q+i+3 15 bits later at 17+5i (bit 1+5i of the high half).
  uint32_t win[5];
  win[0] = w[0] << 2;
  win[1] = __builtin_amdgcn_alignbit(w[1], w[0], 28);
  win[2] = __builtin_amdgcn_alignbit(w[2], w[1], 26);
  win[3] = __builtin_amdgcn_alignbit(w[3], w[2], 24);
  win[4] = __builtin_amdgcn_alignbit(w[4], w[3], 22);
#pragma unroll
  for (int g = 0; g < 5; ++g) {
    q[3 * g + 0] = (win[g] & k.m5) | k.magic;
    q[3 * g + 1] = ((win[g] >> 5) & k.m5) | k.magic;
    q[3 * g + 2] = ((win[g] >> 10) & k.m5) | k.magic;
  }
  // codes 30, 31 live in w[4] bits 22..31; both placed at bits 2..6
  q[15] = ((w[4] >> 20) & 0x7Cu) | ((w[4] >> 9) & 0x7C0000u) | k.magic;
}

template <int BITS, int K>
__device__ __forceinline__ uint32_t code_at(const uint32_t (&w)[BITS]) {
  constexpr int bit = K * BITS, wi = bit / 32, sh = bit % 32;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  if constexpr (sh + BITS <= 32) {
    return (w[wi] >> sh) & mask;
  } else {
    return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & mask;
  }
}

template <int P>
__device__ __forceinline__ void unpack6_pair(uint32_t (&q)[16], const uint32_t (&w)[6],
                                             const UnpackConsts &k) {
  q[P] = (code_at<6, 2 * P>(w) << 1) | (code_at<6, 2 * P + 1>(w) << 17) | k.magic;
  if constexpr (P + 1 < 16) unpack6_pair<P + 1>(q, w, k);
}

template <>
__device__ __forceinline__ void unpack_chunk<6>(uint32_t (&q)[16], const uint32_t (&w)[6],
                                                const UnpackConsts &k) {
  unpack6_pair<0>(q, w, k);
}

template <>
__device__ __forceinline__ void unpack_chunk<8>(uint32_t (&q)[16], const uint32_t (&w)[8],
                                                const UnpackConsts &) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const uint32_t f0 = __float_as_uint((float)(w[t] & 255u));
    const uint32_t f1 = __float_as_uint((float)((w[t] >> 8) & 255u));
    const uint32_t f2 = __float_as_uint((float)((w[t] >> 16) & 255u));
    const uint32_t f3 = __float_as_uint((float)(w[t] >> 24));
    q[2 * t + 0] = (f1 & 0xffff0000u) | (f0 >> 16);
    q[2 * t + 1] = (f3 & 0xffff0000u) | (f2 >> 16);
  }
}

// sum over the chunk of pair(q) . pair(x) with two independent accumulators.
__device__ __forceinline__ float pairs_dot(const uint32_t (&q)[16], const uint32_t (&x)[16]) {
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int p = 0; p < 16; p += 2) {
    a0 = dot2(q[p], x[p], a0);
    a1 = dot2(q[p + 1], x[p + 1], a1);
  }
  return a0 + a1;
}

// Contribution of one chunk: scale * (acc - xsp) + bias * xs.
template <int BITS>
__device__ __forceinline__ float chunk_fold(float acc, float sc, float bi, float xs,
                                            float xsp) {
  if constexpr (BITS == 8) {
    return fmaf(bi, xs, sc * acc);
  } else {
    return fmaf(bi, xs, sc * (acc - xsp));
  }
}

// Load one chunk (BITS dwords) starting at a byte address aligned to 4*BITS
// bytes modulo 16 (4-bit: 16 B, 5-bit: 4 B, 6-bit: 8 B, 8-bit: 32 B).
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x4_a16 __attribute__((ext_vector_type(4)));

// NT: non-temporal loads (the nt cache policy), for weight streams that are
// read once per launch: they then do not displace from L2 what the launch
// reads again (activations, routing inputs, hand-off data, its own code).
// (the builtin takes scalars and clang vectors: HIP's uint2 / uint4 structs
// are loaded as the native vector of the same size)
template <typename T>
struct NtNative {
  using type = T;
};
template <>
struct NtNative<uint2> {
  typedef uint32_t type __attribute__((ext_vector_type(2)));
};
template <>
struct NtNative<uint4> {
  typedef uint32_t type __attribute__((ext_vector_type(4)));
};
template <typename T, bool NT>
__device__ __forceinline__ T ld_stream(const T *p) {
  if constexpr (NT) {
    using V = typename NtNative<T>::type;
    return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const V *>(p)));
  } else {
    return *p;
  }
}

template <int BITS, bool NT = false>
__device__ __forceinline__ void load_chunk(uint32_t (&w)[BITS], const uint8_t *p) {
  if constexpr (BITS == 4) {
    const u32x4_a16 v = ld_stream<u32x4_a16, NT>(reinterpret_cast<const u32x4_a16 *>(p));
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
  } else if constexpr (BITS == 8) {
    const u32x4_a16 v0 = ld_stream<u32x4_a16, NT>(reinterpret_cast<const u32x4_a16 *>(p));
    const u32x4_a16 v1 = ld_stream<u32x4_a16, NT>(reinterpret_cast<const u32x4_a16 *>(p + 16));
    w[0] = v0[0]; w[1] = v0[1]; w[2] = v0[2]; w[3] = v0[3];
    w[4] = v1[0]; w[5] = v1[1]; w[6] = v1[2]; w[7] = v1[3];
  } else if constexpr (BITS == 6) {
    // (the under-aligned vector types go to the builtin directly: as a
    // template argument their alignment attribute would be dropped)
    const u32x2_a4 *q = reinterpret_cast<const u32x2_a4 *>(p);
    u32x2_a4 a, b, c;
    if constexpr (NT) {
      a = __builtin_nontemporal_load(q);
      b = __builtin_nontemporal_load(q + 1);
      c = __builtin_nontemporal_load(q + 2);
    } else {
      a = q[0]; b = q[1]; c = q[2];
    }
    w[0] = a[0]; w[1] = a[1]; w[2] = b[0]; w[3] = b[1]; w[4] = c[0]; w[5] = c[1];
  } else {
    const u32x4_a4 *q = reinterpret_cast<const u32x4_a4 *>(p);
    u32x4_a4 a;
    if constexpr (NT)
      a = __builtin_nontemporal_load(q);
    else
      a = *q;
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
    w[4] = ld_stream<uint32_t, NT>(reinterpret_cast<const uint32_t *>(p + 16));
  }
}

// Sum over `WIDTH` consecutive lanes (WIDTH a power of two <= 64).
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_src_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWMASK, 0xF, false));
}

// Sum over each aligned group of WIDTH lanes (16, 32 or 64), returned in
// every lane of the group. DPP within 16-lane rows (quad xor 1, xor 2, row
// rotate 4, 8), then row broadcasts across rows and readlane, instead of
// LDS-routed shuffles. Callers keep every lane of the wave active.
template <int WIDTH>
__device__ __forceinline__ float team_sum(float v) {
  static_assert(WIDTH == 16 || WIDTH == 32 || WIDTH == 64, "team width");
  v += dpp_src_f32<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v += dpp_src_f32<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v += dpp_src_f32<0x124, 0xF>(v);  // row_ror 4
  v += dpp_src_f32<0x128, 0xF>(v);  // row_ror 8: every lane holds its row's sum
  if constexpr (WIDTH == 16) return v;
  v += dpp_src_f32<0x142, 0xA>(v);  // row_bcast 15: rows 1, 3 += rows 0, 2
  if constexpr (WIDTH == 32) {
    const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    return (threadIdx.x & 32) ? hi : lo;
  }
  v += dpp_src_f32<0x143, 0xC>(v);  // row_bcast 31: row 3 += rows 0 + 1
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sums four values over all 64 lanes of a wave at once. On return every
// lane of 16-lane row r (r = lane / 16) holds the wave total of the r-th
// argument. permlane32_swap exchanges the wave halves (a with c, b with d),
// permlane16_swap the odd and even rows, then four DPP steps finish each row.
__device__ __forceinline__ float wave_reduce4(float a, float b, float c, float d) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(c), false, false);
  const float s1 = __uint_as_float(p[0]) + __uint_as_float(p[1]);  // rows 0-1: a, rows 2-3: c
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(b), __float_as_uint(d), false, false);
  const float s2 = __uint_as_float(q[0]) + __uint_as_float(q[1]);  // rows 0-1: b, rows 2-3: d
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(s1), __float_as_uint(s2), false, false);
  float t = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // row 0: a, 1: b, 2: c, 3: d
  t += dpp_src_f32<0xB1, 0xF>(t);
  t += dpp_src_f32<0x4E, 0xF>(t);
  t += dpp_src_f32<0x124, 0xF>(t);
  t += dpp_src_f32<0x128, 0xF>(t);
  return t;
}

// One 32-code chunk (LSB-first BITS-bit codes) as 16 f16 pairs (code 2i in
// the low half, code 2i+1 in the high half). Every code (< 256) is an exact
// f16: the pair is formed as f16 (1024 + code) by or-ing the code into the
// mantissa of 1024 (0x6400), then 1024 is subtracted with one packed f16
// add, which is exact since both operands and the result are integers
// below 2048.
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f16_pair_from_bias1024(uint32_t p) {
  const half2v v = __builtin_bit_cast(half2v, p | 0x64006400u);
  return __builtin_bit_cast(uint32_t, v - (half2v){(_Float16)1024.f, (_Float16)1024.f});
}
template <int BITS>
__device__ __forceinline__ void codes_to_f16(const uint32_t (&w)[BITS], uint32_t (&cp)[16]) {
  if constexpr (BITS == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // even codes in the bytes of lo, odd codes in the bytes of hi; v_perm
      // picks byte j of each into the two halves (selector 0x0C = zero byte)
      const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t sel = (uint32_t)j | 0x0C00u | ((uint32_t)(4 + j) << 16) | 0x0C000000u;
        cp[4 * i + j] = f16_pair_from_bias1024(__builtin_amdgcn_perm(hi, lo, sel));
      }
    }
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      cp[2 * i] = f16_pair_from_bias1024(__builtin_amdgcn_perm(0u, w[i], 0x0C010C00u));
      cp[2 * i + 1] = f16_pair_from_bias1024(__builtin_amdgcn_perm(0u, w[i], 0x0C030C02u));
    }
  } else {
    constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
    for (int k = 0; k < 32; k += 2) {
      uint32_t c[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int bit = (k + q) * BITS, i = bit >> 5, sh = bit & 31;
        uint32_t v = w[i] >> sh;
        if (sh + BITS > 32) v |= w[i + 1] << (32 - sh);
        c[q] = v & mask;
      }
      cp[k >> 1] = f16_pair_from_bias1024(c[0] | (c[1] << 16));
    }
  }
}

// sum_k code_k * h_k over one 32-code chunk (LSB-first BITS-bit codes)
template <int BITS>
__device__ __forceinline__ float codes_dot(const uint32_t (&w)[BITS], const float (&h)[32]) {
  float a0 = 0.f, a1 = 0.f;
  if constexpr (BITS == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // nibbles to bytes, then one v_cvt_f32_ubyteN per code (the empty asm
      // keeps the compiler from folding the masks into per-code bfe's)
      uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
      asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        a0 = fmaf((float)((lo >> (8 * b)) & 0xffu), h[8 * i + 2 * b], a0);
        a1 = fmaf((float)((hi >> (8 * b)) & 0xffu), h[8 * i + 2 * b + 1], a1);
      }
    }
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a0 = fmaf((float)(w[i] & 0xffu), h[4 * i], a0);
      a1 = fmaf((float)((w[i] >> 8) & 0xffu), h[4 * i + 1], a1);
      a0 = fmaf((float)((w[i] >> 16) & 0xffu), h[4 * i + 2], a0);
      a1 = fmaf((float)(w[i] >> 24), h[4 * i + 3], a1);
    }
  } else {
    constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      const int bit = k * BITS, i = bit >> 5, sh = bit & 31;
      uint32_t c = w[i] >> sh;
      if (sh + BITS > 32) c |= w[i + 1] << (32 - sh);
      if (k & 1)
        a1 = fmaf((float)(c & mask), h[k], a1);
      else
        a0 = fmaf((float)(c & mask), h[k], a0);
    }
  }
  return a0 + a1;
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

}  // namespace lh
