// Wave-level routing primitives for gfx950 (DPP reductions, top-k by key).
//
// Top-k with the reference's tie rule (logan-qwen4/src/lib.rs:8031-8040:
// larger value first, equal values -> lower expert index) is a selection on
// unique keys (ordered value, inverted index): each lane keeps its keys
// sorted, and each round takes the wave maximum of the lanes' best keys.
#pragma once
#include <cstdint>

#include "affine_dev.hpp"

namespace lh {

// ---------------------------------------------------------------- DPP helpers

template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWMASK, 0xF, false);
}

template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWMASK, 0xF, false));
}

// max over all 64 lanes, returned uniformly
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1, 0xF>(v));   // quad_perm [1,0,3,2]
  v = max(v, dpp_u32<0x4E, 0xF>(v));   // quad_perm [2,3,0,1]
  v = max(v, dpp_u32<0x124, 0xF>(v));  // row_ror 4
  v = max(v, dpp_u32<0x128, 0xF>(v));  // row_ror 8
  v = max(v, dpp_u32<0x142, 0xA>(v));  // row_bcast 15 -> rows 1, 3
  v = max(v, dpp_u32<0x143, 0xC>(v));  // row_bcast 31 -> rows 2, 3
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// sum over all 64 lanes, returned uniformly
__device__ __forceinline__ float wave_sum_f32(float v) {
  v += dpp_f32<0xB1, 0xF>(v);
  v += dpp_f32<0x4E, 0xF>(v);
  v += dpp_f32<0x124, 0xF>(v);
  v += dpp_f32<0x128, 0xF>(v);
  v += dpp_f32<0x142, 0xA>(v);
  v += dpp_f32<0x143, 0xC>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// sum over each aligned group of W lanes (W = 16, 32 or 64); every lane of
// the group gets the group sum
template <int W>
__device__ __forceinline__ float group_sum_f32(float v) {
  v += dpp_f32<0xB1, 0xF>(v);
  v += dpp_f32<0x4E, 0xF>(v);
  v += dpp_f32<0x124, 0xF>(v);
  v += dpp_f32<0x128, 0xF>(v);
  if constexpr (W >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (W >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// ---------------------------------------------------------------- routing

__device__ __forceinline__ uint32_t ord16(uint32_t b) {
  if (b == 0x8000u) b = 0;  // -0 == +0
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}

__device__ __forceinline__ float unord16(uint32_t o) {
  const uint32_t b = (o & 0x8000u) ? (o & 0x7fffu) : (~o & 0xffffu);
  return bf16_to_f32(b);
}

template <int N>
__device__ __forceinline__ void sort_desc(uint32_t (&v)[N]) {
  // bitonic network, descending
#pragma unroll
  for (int k = 2; k <= N; k <<= 1)
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int l = i ^ j;
        if (l > i) {
          const bool desc = (i & k) == 0;
          const uint32_t a = v[i], b = v[l];
          const uint32_t hi = max(a, b), lo = min(a, b);
          v[i] = desc ? hi : lo;
          v[l] = desc ? lo : hi;
        }
      }
}

// Routing by one wave, in two steps so the caller can put other loads in
// flight between them: route_keys issues the logit loads (lane l holds
// experts l + 64 i); route_select sorts each lane's keys and runs `rounds`
// rounds of a wave max. sel[r] = 32-bit key of rank r: high half = ordered
// logit, low half = 0xffff - expert.
template <int KPL>
__device__ __forceinline__ void route_keys(const uint16_t *logits, int E, uint32_t (&key)[KPL]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int e = i * 64 + lane;
    key[i] = logits[e < E ? e : 0];
  }
}

template <int KPL, int NSEL>
__device__ __forceinline__ void route_select(uint32_t (&key)[KPL], int E, int rounds,
                                             uint32_t (&sel)[NSEL]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int e = i * 64 + lane;
    key[i] = e < E ? ((ord16(key[i]) << 16) | (0xffffu - (uint32_t)e)) : 0u;
  }
  sort_desc<KPL>(key);
#pragma unroll
  for (int r = 0; r < NSEL; ++r) {
    sel[r] = 0;
    if (r < rounds) {
      const uint32_t m = wave_max_u32(key[0]);
      sel[r] = m;
      const bool mine = key[0] == m;  // keys are unique
#pragma unroll
      for (int i = 0; i < KPL - 1; ++i) key[i] = mine ? key[i + 1] : key[i];
      key[KPL - 1] = mine ? 0u : key[KPL - 1];
    }
  }
}

__device__ __forceinline__ int sel_expert(uint32_t key) { return (int)(0xffffu - (key & 0xffffu)); }
__device__ __forceinline__ float sel_logit(uint32_t key) { return unord16(key >> 16); }


// ---- f32 logits: 64-bit keys (ordered f32 << 32 | ~index) -----------------

__device__ __forceinline__ uint32_t ord32f(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0;  // -0 == +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float unord32f(uint32_t o) {
  const uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(u);
}

template <int CTRL, int ROWMASK>
__device__ __forceinline__ void dpp_max_u64_step(uint32_t &hi, uint32_t &lo) {
  const uint32_t ohi = dpp_u32<CTRL, ROWMASK>(hi), olo = dpp_u32<CTRL, ROWMASK>(lo);
  const bool take = ohi > hi || (ohi == hi && olo > lo);
  hi = take ? ohi : hi;
  lo = take ? olo : lo;
}

// max over all 64 lanes of (hi, lo) compared as one 64-bit value, uniform
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  uint32_t hi = (uint32_t)(v >> 32), lo = (uint32_t)v;
  dpp_max_u64_step<0xB1, 0xF>(hi, lo);
  dpp_max_u64_step<0x4E, 0xF>(hi, lo);
  dpp_max_u64_step<0x124, 0xF>(hi, lo);
  dpp_max_u64_step<0x128, 0xF>(hi, lo);
  dpp_max_u64_step<0x142, 0xA>(hi, lo);
  dpp_max_u64_step<0x143, 0xC>(hi, lo);
  hi = (uint32_t)__builtin_amdgcn_readlane((int)hi, 63);
  lo = (uint32_t)__builtin_amdgcn_readlane((int)lo, 63);
  return ((uint64_t)hi << 32) | lo;
}

template <int N>
__device__ __forceinline__ void sort_desc_u64(uint64_t (&v)[N]) {
#pragma unroll
  for (int k = 2; k <= N; k <<= 1)
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int l = i ^ j;
        if (l > i) {
          const bool desc = (i & k) == 0;
          const uint64_t a = v[i], b = v[l];
          const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
          v[i] = desc ? hi : lo;
          v[l] = desc ? lo : hi;
        }
      }
}

// One wave: top-k of E logits (bf16 or f32) of one token. On return lane r
// (r < k) holds rank r's expert in *idx and its weight
// w_r = exp(l_r - l_0) / sum_{j<k} exp(l_j - l_0) (= val_r / wsum of
// logan-qwen4/src/lib.rs:8043, :8694) in *w; other lanes get idx -1, w 0.
// KPL = keys per lane (E <= 64 * KPL).
template <int KPL, bool F32>
__device__ __forceinline__ void wave_topk_lanes(const void *logits, size_t row_off, int E, int k,
                                                int &idx, float &w) {
  const int lane = threadIdx.x & 63;
  float lmine = 0.f;
  uint32_t emine = 0xffffffffu;
  if constexpr (!F32) {
    uint32_t key[KPL];
    const uint16_t *lg = reinterpret_cast<const uint16_t *>(logits) + row_off;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int e = i * 64 + lane;
      key[i] = lg[e < E ? e : 0];
    }
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int e = i * 64 + lane;
      key[i] = e < E ? ((ord16(key[i]) << 16) | (0xffffu - (uint32_t)e)) : 0u;
    }
    sort_desc<KPL>(key);
    uint32_t kmine = 0;
#pragma unroll 1
    for (int r = 0; r < k; ++r) {
      const uint32_t m = wave_max_u32(key[0]);
      kmine = lane == r ? m : kmine;
      const bool mine = key[0] == m;
#pragma unroll
      for (int i = 0; i < KPL - 1; ++i) key[i] = mine ? key[i + 1] : key[i];
      key[KPL - 1] = mine ? 0u : key[KPL - 1];
    }
    lmine = unord16(kmine >> 16);
    emine = 0xffffu - (kmine & 0xffffu);
  } else {
    uint64_t key[KPL];
    const float *lg = reinterpret_cast<const float *>(logits) + row_off;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int e = i * 64 + lane;
      const float l = lg[e < E ? e : 0];
      key[i] = e < E ? (((uint64_t)ord32f(l) << 32) | (0xffffffffu - (uint32_t)e)) : 0ull;
    }
    sort_desc_u64<KPL>(key);
    uint64_t kmine = 0;
#pragma unroll 1
    for (int r = 0; r < k; ++r) {
      const uint64_t m = wave_max_u64(key[0]);
      kmine = lane == r ? m : kmine;
      const bool mine = key[0] == m;
#pragma unroll
      for (int i = 0; i < KPL - 1; ++i) key[i] = mine ? key[i + 1] : key[i];
      key[KPL - 1] = mine ? 0ull : key[KPL - 1];
    }
    lmine = unord32f((uint32_t)(kmine >> 32));
    emine = 0xffffffffu - (uint32_t)kmine;
  }
  const float l0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lmine), 0));
  const float ev = lane < k ? __expf(lmine - l0) : 0.f;
  const float ws = wave_sum_f32(ev);
  idx = lane < k ? (int)emine : -1;
  w = lane < k ? ev / ws : 0.f;
}

}  // namespace lh
