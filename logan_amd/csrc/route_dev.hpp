// Wave-level routing primitives for gfx950 (DPP reductions, top-k by key).
//
// Top-k with the reference's tie rule (logan-qwen4/src/lib.rs:8031-8040:
// larger value first, equal values -> lower expert index) is a selection on
// unique keys (ordered value, inverted index): each lane keeps its keys
// sorted, and each round takes the wave maximum of the lanes' best keys.
//
// The reference selects on softmax probabilities, p_i = fl(exp(fl(l_i - m))
// / s) (lib.rs:4558-4574), which are only non-decreasing in the logit: two
// different logits can share a probability (an exp argument rounded to the
// same value, an exp that underflows, two exps one ulp apart that divide to
// the same quotient), and the reference then takes the lower index. The
// fast selection runs on the logits and checks afterwards whether any pair
// that matters could tie that way; when one could, the wave recomputes the
// reference's probabilities (same max, exp, sequential sum, division) and
// selects on them (route_exact).
#pragma once
#include <cstdint>
#include <type_traits>

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

// Order-preserving 16-bit key of a bf16 value. Every NaN, either sign, maps
// to the top key: rank 0 is then NaN, its maximum fails tie_global's
// finiteness test and the token takes route_exact, which reproduces the
// reference's NaN sum (ranks 0..k-1 = experts 0..k-1, NaN weights). A NaN
// left below the selected ranks would skip that path on the bf16 shortcut.
__device__ __forceinline__ uint32_t ord16(uint32_t b) {
  if ((b & 0x7fffu) > 0x7f80u) return 0xffffu;  // NaN
  if (b == 0x8000u) b = 0;                     // -0 == +0
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

__device__ __forceinline__ int sel_expert(uint32_t key) { return (int)(0xffffu - (key & 0xffffu)); }


// ---- f32 logits: 64-bit keys (ordered f32 << 32 | ~index) -----------------

// f32 counterpart of ord16, NaN (either sign) first as there
__device__ __forceinline__ uint32_t ord32f(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // NaN
  if (u == 0x80000000u) u = 0;                            // -0 == +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float unord32f(uint32_t o) {
  const uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(u);
}

// max over all 64 lanes of (hi, lo) compared as one 64-bit value, uniform:
// the 32-bit max of the high halves, then the low half of the one lane that
// holds it; only when several lanes hold it (equal logits) a second 32-bit
// max over their low halves. (A 64-bit compare in each DPP step, two moves
// and a chained compare/select per step, made each of the ten selection
// rounds about three times as long: 0.6 against 0.2 us per round.)
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  const uint32_t hi = (uint32_t)(v >> 32), lo = (uint32_t)v;
  const uint32_t mh = wave_max_u32(hi);
  const uint64_t tied = __ballot(hi == mh);
  uint32_t ml;
  if (__popcll(tied) == 1)
    ml = (uint32_t)__builtin_amdgcn_readlane((int)lo, __ffsll((unsigned long long)tied) - 1);
  else
    ml = wave_max_u32(hi == mh ? lo : 0u);
  return ((uint64_t)mh << 32) | ml;
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

// ---- probability ties the logit order cannot see ---------------------------
//
// With a faithful exp (< 1 ulp), |fl(l_a - m) - fl(l_b - m)| > kTieGap makes
// the two exps differ by several ulps, so their quotients by the same sum
// differ too: only logits whose exp arguments are within kTieGap, exps in
// the underflow range, or non-finite values can tie in probability while
// differing in logit. A tie run (equal probabilities) is contiguous in
// logit order and every member is within kTieGap of every other, so for the
// ranks [0, R] it suffices to check consecutive selected ranks and the
// unselected logits against rank R's.
constexpr float kTieGap = 0x1p-19f;
constexpr float kTieFloor = -80.0f;  // exp(-80) ~ 1.8e-35: still normal

// rank pair (a above b in logit order) that may share a probability
__device__ __forceinline__ bool tie_pair(float la, float lb, float m) {
  return la != lb && (la - m) - (lb - m) <= kTieGap;
}
// an unselected logit lu that may share rank R's probability (or is NaN)
__device__ __forceinline__ bool tie_other(float lu, float lr, float m) {
  return (lu != lu) || (lu != lr && fabsf((lu - m) - (lr - m)) <= kTieGap);
}
// the reference's max (lib.rs:4560-4565: fold from -1e30, NaN ignored) may
// differ from rank 0's logit, or rank R's exp may underflow
__device__ __forceinline__ bool tie_global(float m, float lr) {
  return !(fabsf(m) <= 3.0e38f) || m < -1e30f || (lr - m) < kTieFloor;
}

// bf16 logits: two different bf16 values of magnitude >= 2^-9 are at least
// 2^-17 apart, and with |max| < 64 their exp arguments fl(l - m) are exact
// (at most 23 significant bits), so such a logit shares its probability with
// no different logit unless its exp underflows. These uniform tests let the
// bf16 paths skip the per-lane checks above in all but rare cases:
// rank r alone (logit lr) ...
__device__ __forceinline__ bool bf16_rank_tie_free(float m, float lr) {
  return fabsf(m) < 64.f && fabsf(lr) >= 0x1p-9f && (lr - m) >= kTieFloor;
}
// ... or every rank down to the one with logit llast (all logits in
// [llast, m], none of them in (-2^-9, 2^-9))
__device__ __forceinline__ bool bf16_ranks_tie_free(float m, float llast) {
  return fabsf(m) < 64.f && (llast >= 0x1p-9f || m <= -0x1p-9f) && (llast - m) >= kTieFloor;
}

// Logit keys of one wave, for routing split into a load step and a select
// step (other loads can be issued between them). bf16 logits give 32-bit
// keys (ordered bf16 << 16 | 0xffff - expert), f32 logits 64-bit keys
// (ordered f32 << 32 | 0xffffffff - expert); lane l holds experts
// l + 64 i. After select, key[] holds this lane's unselected keys (0 =
// none) and sel[r] the key of rank r.
template <int KPL, bool LF>
struct WaveKeys {
  using K = typename std::conditional<LF, uint64_t, uint32_t>::type;
  K key[KPL];
  __device__ __forceinline__ void load(const void *logits, int E) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int e = i * 64 + lane, ee = e < E ? e : 0;
      if constexpr (LF)
        key[i] = __float_as_uint(reinterpret_cast<const float *>(logits)[ee]);
      else
        key[i] = reinterpret_cast<const uint16_t *>(logits)[ee];
    }
  }
  template <int NSEL>
  __device__ __forceinline__ void select(int E, int rounds, K (&sel)[NSEL]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int e = i * 64 + lane;
      if constexpr (LF)
        key[i] = e < E ? (((uint64_t)ord32f(__uint_as_float((uint32_t)key[i])) << 32) |
                          (0xffffffffu - (uint32_t)e))
                       : 0ull;
      else
        key[i] = e < E ? ((ord16(key[i]) << 16) | (0xffffu - (uint32_t)e)) : 0u;
    }
    if constexpr (LF)
      sort_desc_u64<KPL>(key);
    else
      sort_desc<KPL>(key);
#pragma unroll
    for (int r = 0; r < NSEL; ++r) {
      sel[r] = 0;
      if (r < rounds) {
        K m;
        if constexpr (LF)
          m = wave_max_u64(key[0]);
        else
          m = wave_max_u32(key[0]);
        sel[r] = m;
        const bool mine = key[0] == m;  // keys are unique
#pragma unroll
        for (int i = 0; i < KPL - 1; ++i) key[i] = mine ? key[i + 1] : key[i];
        key[KPL - 1] = mine ? K(0) : key[KPL - 1];
      }
    }
  }
  __device__ static __forceinline__ int expert(K k) {
    if constexpr (LF) return (int)(0xffffffffu - (uint32_t)k);
    else return (int)(0xffffu - (k & 0xffffu));
  }

  // ---- f32 logits on 32-bit keys (LF only; before select) ----------------
  // Key = the upper 32 - IB bits of the ordered f32 (its prefix) above an
  // IB-bit inverted expert index. Distinct prefixes order as the values do,
  // so where the keys that decide the ranks have pairwise distinct prefixes
  // the 32-bit selection equals the selection on (value desc, index asc),
  // with each round a 32-bit wave max like the bf16 keys'. fast_ok says when
  // that holds and no probability tie can reach the ranks; otherwise the
  // caller selects on the 64-bit keys (select) instead. The raw logits stay
  // in key[] until select converts them.
  static constexpr int IB = KPL <= 8 ? 9 : 10;
  static constexpr uint32_t IM = (1u << IB) - 1u;
  __device__ static __forceinline__ int expert32(uint32_t k) { return (int)(IM - (k & IM)); }
  // exact logit of expert e (lane-varying): lane e % 64 holds it in key[e / 64]
  __device__ __forceinline__ float value_lane(int e) const {
    float out = 0.f;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const float t = __shfl(__uint_as_float((uint32_t)key[i]), e & 63, 64);
      out = (e >> 6) == i ? t : out;
    }
    return out;
  }
  // sel[r] for r <= rounds: the keys of ranks 0 .. rounds (0 past E)
  template <int NSEL>
  __device__ __forceinline__ void select_fast(int E, int rounds, uint32_t (&sel)[NSEL]) const {
    static_assert(LF, "f32 keys");
    const int lane = threadIdx.x & 63;
    uint32_t k32[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int e = i * 64 + lane;
      k32[i] = e < E ? ((ord32f(__uint_as_float((uint32_t)key[i])) & ~IM) | (IM - (uint32_t)e)) : 0u;
    }
    sort_desc<KPL>(k32);
#pragma unroll
    for (int r = 0; r < NSEL; ++r) {
      sel[r] = 0u;
      if (r <= rounds) {
        const uint32_t m = wave_max_u32(k32[0]);
        sel[r] = m;
        const bool mine = k32[0] == m;  // keys are unique
#pragma unroll
        for (int i = 0; i < KPL - 1; ++i) k32[i] = mine ? k32[i + 1] : k32[i];
        k32[KPL - 1] = mine ? 0u : k32[KPL - 1];
      }
    }
  }
  // True when ranks 0 .. R of select_fast's keys (sel[0 .. R + 1] filled)
  // are the reference's: no two of the keys of ranks 0 .. R + 1 share a
  // prefix, no probability tie joins consecutive ranks up to R, no logit of
  // the best unselected prefix can tie with rank R, and rank 0 / rank R pass
  // tie_global (route_dev.hpp's tie rules, on exact values). Lane r <= R
  // gets rank r's exact logit in v, every lane the maximum in m.
  template <int NSEL>
  __device__ __forceinline__ bool fast_ok(const uint32_t (&sel)[NSEL], int R, float &v, float &m) const {
    const int lane = threadIdx.x & 63;
    uint32_t kr = 0u;
#pragma unroll
    for (int r = 0; r < NSEL; ++r) kr = lane == r ? sel[r] : kr;
    const uint32_t knext = __shfl(kr, (lane + 1) & 63, 64);
    // every lane runs the cross-lane reads (a lane outside a branch would
    // not supply its registers to them)
    const float vall = value_lane(expert32(kr));
    v = lane <= R ? vall : 0.f;
    m = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
    const float vR = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), R));
    const float vnext = __shfl(v, (lane + 1) & 63, 64);
    bool bad = lane <= R && knext != 0u && (kr >> IB) == (knext >> IB);
    bad = bad || (lane < R && tie_pair(v, vnext, m));
    if (lane == R + 1 && kr != 0u) {
      const float bhi = unord32f(kr | IM);  // largest logit with this prefix
      bad = bad || fabsf((bhi - m) - (vR - m)) <= kTieGap;
    }
    return !__any(bad) && !tie_global(m, vR);
  }
  __device__ static __forceinline__ float logit(K k) {
    if constexpr (LF) return unord32f((uint32_t)(k >> 32));
    else return unord16(k >> 16);
  }
};

struct RouteLane {
  int idx;  // rank (lane) < k: expert; else -1
  float w;  // rank (lane) < k: val_r / wsum; else 0
};

// The reference's routing of one token, recomputed by one wave
// (logan-qwen4/src/lib.rs:4558-4574 softmax_row, :8031-8043 selection and
// wsum, :8694 weight): m = max(-1e30, l) ignoring NaN; e_i = exp(fl(l_i - m))
// rounded to f32 from a double-precision exp; s = e_0 + e_1 + ... in index
// order (f32, sequential); p_i = e_i / s; top-k on (p desc, index asc);
// wsum = sum of the k selected p in rank order; w_r = p_r / wsum. A NaN sum
// leaves every comparison false, so the reference keeps ranks 0..k-1 as
// experts 0..k-1 with NaN weights; so does this. Taken only when the
// logit-keyed selection could differ (see the checks above), so it is
// written for clarity, not speed.
template <int KPL, bool F32>
__device__ __noinline__ RouteLane route_exact(const void *logits, size_t row_off, int E, int k) {
  const int lane = threadIdx.x & 63;
  float l[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int e = i * 64 + lane;
    const int ee = e < E ? e : 0;
    if constexpr (F32)
      l[i] = reinterpret_cast<const float *>(logits)[row_off + ee];
    else
      l[i] = bf16_to_f32(reinterpret_cast<const uint16_t *>(logits)[row_off + ee]);
  }
  float mm = -1e30f;
#pragma unroll
  for (int i = 0; i < KPL; ++i)
    if (i * 64 + lane < E && l[i] > mm) mm = l[i];
  const float m = unord32f(wave_max_u32(ord32f(mm)));
  float ev[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const float d = __fsub_rn(l[i], m);
    ev[i] = i * 64 + lane < E ? (float)exp((double)d) : 0.f;
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < KPL; ++i)
    for (int j = 0; j < 64 && i * 64 + j < E; ++j)
      s = __fadd_rn(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev[i]), j)));
  RouteLane out;
  if (!(s == s)) {
    out.idx = lane < k ? lane : -1;
    out.w = lane < k ? __int_as_float(0x7fc00000) : 0.f;
    return out;
  }
  uint64_t key[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int e = i * 64 + lane;
    const float p = __fdiv_rn(ev[i], s);  // >= +0: its bits order as the value
    key[i] = e < E ? (((uint64_t)__float_as_uint(p) << 32) | (0xffffffffu - (uint32_t)e)) : 0ull;
  }
  sort_desc_u64<KPL>(key);
  uint64_t kmine = 0;
  for (int r = 0; r < k; ++r) {
    const uint64_t mx = wave_max_u64(key[0]);
    kmine = lane == r ? mx : kmine;
    const bool mine = key[0] == mx;
#pragma unroll
    for (int i = 0; i < KPL - 1; ++i) key[i] = mine ? key[i + 1] : key[i];
    key[KPL - 1] = mine ? 0ull : key[KPL - 1];
  }
  const float val = __uint_as_float((uint32_t)(kmine >> 32));
  float wsum = 0.f;
  for (int r = 0; r < k; ++r)
    wsum = __fadd_rn(wsum, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(val), r)));
  out.idx = lane < k ? (int)(0xffffffffu - (uint32_t)kmine) : -1;
  out.w = lane < k ? __fdiv_rn(val, wsum) : 0.f;
  return out;
}

// One wave: top-k of E logits (bf16 or f32) of one token. On return lane r
// (r < k) holds rank r's expert in *idx and its weight
// w_r = exp(l_r - l_0) / sum_{j<k} exp(l_j - l_0) (= val_r / wsum of
// logan-qwen4/src/lib.rs:8043, :8694) in *w; other lanes get idx -1, w 0.
// When a probability tie could reorder the selection, the result is
// route_exact's instead. KPL = keys per lane (E <= 64 * KPL).
template <int KPL, bool F32>
__device__ __forceinline__ void wave_topk_lanes(const void *logits, size_t row_off, int E, int k,
                                                int &idx, float &w) {
  const int lane = threadIdx.x & 63;
  float lmine = 0.f;
  uint32_t emine = 0xffffffffu;
  bool cand = false;  // a logit of this lane may share a probability with another
  float m = 0.f, llast = 0.f;
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
      const uint32_t mx = wave_max_u32(key[0]);
      kmine = lane == r ? mx : kmine;
      const bool mine = key[0] == mx;
#pragma unroll
      for (int i = 0; i < KPL - 1; ++i) key[i] = mine ? key[i + 1] : key[i];
      key[KPL - 1] = mine ? 0u : key[KPL - 1];
    }
    lmine = unord16(kmine >> 16);
    emine = 0xffffu - (kmine & 0xffffu);
    m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lmine), 0));
    llast = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lmine), k - 1));
    if (!bf16_ranks_tie_free(m, llast)) {  // rare: the full checks
#pragma unroll
      for (int i = 0; i < KPL; ++i)
        cand = cand || (key[i] != 0u && tie_other(unord16(key[i] >> 16), llast, m));
      const float lnext = __shfl(lmine, (lane + 1) & 63, 64);
      cand = cand || (lane + 1 < k && tie_pair(lmine, lnext, m));
      if (__any(cand) || tie_global(m, llast)) {
        const RouteLane rl = route_exact<KPL, F32>(logits, row_off, E, k);
        idx = rl.idx;
        w = rl.w;
        return;
      }
    }
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
      const uint64_t mx = wave_max_u64(key[0]);
      kmine = lane == r ? mx : kmine;
      const bool mine = key[0] == mx;
#pragma unroll
      for (int i = 0; i < KPL - 1; ++i) key[i] = mine ? key[i + 1] : key[i];
      key[KPL - 1] = mine ? 0ull : key[KPL - 1];
    }
    lmine = unord32f((uint32_t)(kmine >> 32));
    emine = 0xffffffffu - (uint32_t)kmine;
    m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lmine), 0));
    llast = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lmine), k - 1));
#pragma unroll
    for (int i = 0; i < KPL; ++i)
      cand = cand || (key[i] != 0ull && tie_other(unord32f((uint32_t)(key[i] >> 32)), llast, m));
    // consecutive selected ranks (lane r: ranks r, r + 1)
    const float lnext = __shfl(lmine, (lane + 1) & 63, 64);
    cand = cand || (lane + 1 < k && tie_pair(lmine, lnext, m));
    if (__any(cand) || tie_global(m, llast)) {
      const RouteLane rl = route_exact<KPL, F32>(logits, row_off, E, k);
      idx = rl.idx;
      w = rl.w;
      return;
    }
  }
  const float ev = lane < k ? __expf(lmine - m) : 0.f;
  const float ws = wave_sum_f32(ev);
  idx = lane < k ? (int)emine : -1;
  w = lane < k ? ev / ws : 0.f;
}

}  // namespace lh
