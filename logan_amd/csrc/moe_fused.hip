// Single-launch routed-MoE block for one token (B = 1), gfx950.
//
// One kernel, two kinds of blocks, one hand-off:
//
//   A blocks (first in the grid): each wave owns UA rows j of one expert slot
//   (rank r < k of the route, or the shared expert) and computes
//   h[slot][j] = silu(gate_j . x) * (up_j . x) for them, then publishes with an
//   agent-scope release and one atomic arrival.
//
//   B blocks: each wave owns ROWS_B output rows d for all k+1 slots. It
//   issues the loads of its down-projection weights for every slot right
//   after routing (so they stream from HBM while A runs), computes the
//   shared-expert scalar gate sigmoid(se_g . x), then waits for all A
//   arrivals, stages every h (as bf16 hi/lo x-operands) in LDS, and forms
//   out[d] = sum_{r<k} w_r * (down_r . h_r)[d]  (rank order)
//            + gs * (down_shared . h_shared)[d]
//   (logan-qwen4/src/lib.rs:8692-8711, :7597-7759).
//
// Every wave computes the route itself from the bf16 logits (top-k with the
// key (logit desc, index asc): per-lane sorted keys, k rounds of a DPP wave
// max), so no block waits for another before streaming weights.
//
// Progress: A waves never wait. Workgroups are dispatched in ID order on each
// XCD, and every A block precedes every B block, so a B block can only be
// resident after all A blocks of its XCD were dispatched: the waits always
// end. They are also bounded: after kSpinLimit polls a B block stops waiting,
// raises the sticky error word and finishes (its output is then garbage; the
// host can read the word with logan_hip_moe_sync_errors()).
//
// The arrival counters live in module-scope device memory (zero when the code
// object loads) and the last B block to finish puts them back to zero, so each
// launch starts from zero without a memset. Launches of this kernel on one
// device must therefore not overlap (one stream, or serialised streams).
#include "affine_dev.hpp"
#include "lh_internal.hpp"

namespace lh {

struct FusedSync {
  uint32_t a_done;
  uint32_t b_done;
  uint32_t error;
  uint32_t launches;
};
__device__ FusedSync g_fused_sync;

constexpr int kFusedMaxSlots = 12;  // k + 1 (routed + shared)
constexpr uint32_t kSpinLimit = 1u << 22;

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

// Top-`rounds` of E bf16 logits by one wave. sel[r] = 32-bit key of rank r:
// high half = ordered logit, low half = 0xffff - expert.
template <int KPL>
__device__ __forceinline__ void wave_route_bf16(const uint16_t *logits, int E, int rounds,
                                                uint32_t (&sel)[kFusedMaxSlots]) {
  const int lane = threadIdx.x & 63;
  uint32_t key[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int e = i * 64 + lane;
    const bool ok = e < E;
    const uint32_t b = logits[ok ? e : 0];
    key[i] = ok ? ((ord16(b) << 16) | (0xffffu - (uint32_t)e)) : 0u;
  }
  sort_desc<KPL>(key);
#pragma unroll
  for (int r = 0; r < kFusedMaxSlots; ++r) {
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

// ---------------------------------------------------------------- kernel

struct FusedGeom {
  int k;           // routed experts
  int slots;       // k + (shared ? 1 : 0)
  int wpr;         // A waves per routed slot
  int wps;         // A waves for the shared slot
  int nA_waves;
  int nA_blocks;
  int nB_blocks;
};

template <int BITS, int CPLA, int LANESB, int KPL>
__global__ __launch_bounds__(256) void moe_fused_b1_kernel(MoeArgs a, FusedGeom g) {
  constexpr int UA = BITS == 8 ? 2 : 4;      // rows of gate (and of up) per A wave
  constexpr int ROWS_B = 64 / LANESB;        // output rows per B wave
  constexpr int XDW = 36;                    // LDS dwords per (slot, chunk): 16 hi, 16 lo, xs, xsp
  __shared__ __align__(16) uint32_t s_h[kFusedMaxSlots * LANESB * XDW];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint16_t *logits = reinterpret_cast<const uint16_t *>(a.logits);
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  UnpackConsts kc;
  kc.init();

  if ((int)blockIdx.x < g.nA_blocks) {
    // ------------------------------------------------------------ phase A
    const int item = blockIdx.x * 4 + wave;
    if (item >= g.nA_waves) return;
    const bool shared = item >= g.k * g.wpr;
    const int slot = shared ? g.k : item / g.wpr;
    const int jb = shared ? item - g.k * g.wpr : item % g.wpr;
    const int rows = shared ? a.sinter : a.inter;
    int e = 0;
    if (!shared) {
      uint32_t sel[kFusedMaxSlots];
      wave_route_bf16<KPL>(logits, a.E, slot + 1, sel);
      uint32_t mine = sel[0];
#pragma unroll
      for (int r = 1; r < kFusedMaxSlots; ++r) mine = r == slot ? sel[r] : mine;
      e = sel_expert(mine);
    }
    const DevBank &bgk = shared ? a.sgate : a.gate;
    const DevBank &buk = shared ? a.sup : a.up;
    const uint8_t *gw = bgk.m.w + (size_t)e * bgk.w_stride;
    const uint8_t *uw = buk.m.w + (size_t)e * buk.w_stride;
    const uint16_t *gsc = bgk.m.sc + (size_t)e * bgk.p_stride;
    const uint16_t *gbi = bgk.m.bi + (size_t)e * bgk.p_stride;
    const uint16_t *usc = buk.m.sc + (size_t)e * buk.p_stride;
    const uint16_t *ubi = buk.m.bi + (size_t)e * buk.p_stride;
    const int j0 = jb * UA;
    const int C = a.D >> 5;
    const int gsc_chunks = bgk.m.gs >> 5;

    uint32_t wg[UA][CPLA][BITS], wu[UA][CPLA][BITS];
#pragma unroll
    for (int u = 0; u < UA; ++u)
#pragma unroll
      for (int i = 0; i < CPLA; ++i) {
        const int j = j0 + u, c = lane + 64 * i;
        if (j < rows && c < C) {
          load_chunk<BITS>(wg[u][i], gw + (size_t)j * bgk.m.row_bytes + (size_t)c * (4 * BITS));
          load_chunk<BITS>(wu[u][i], uw + (size_t)j * buk.m.row_bytes + (size_t)c * (4 * BITS));
        } else {
#pragma unroll
          for (int t = 0; t < BITS; ++t) wg[u][i][t] = wu[u][i][t] = 0;
        }
      }
    float sg[UA][CPLA], bg[UA][CPLA], su[UA][CPLA], bu[UA][CPLA];
#pragma unroll
    for (int u = 0; u < UA; ++u)
#pragma unroll
      for (int i = 0; i < CPLA; ++i) {
        const int j = j0 + u, c = lane + 64 * i;
        if (j < rows && c < C) {
          const size_t p = (size_t)j * bgk.m.ng + c / gsc_chunks;
          sg[u][i] = aux_to_f32(gsc[p], bgk.m.fp16);
          bg[u][i] = aux_to_f32(gbi[p], bgk.m.fp16);
          su[u][i] = aux_to_f32(usc[p], buk.m.fp16);
          bu[u][i] = aux_to_f32(ubi[p], buk.m.fp16);
        } else {
          sg[u][i] = bg[u][i] = su[u][i] = bu[u][i] = 0.f;
        }
      }
    float pg[UA], pu[UA];
#pragma unroll
    for (int u = 0; u < UA; ++u) pg[u] = pu[u] = 0.f;
#pragma unroll
    for (int i = 0; i < CPLA; ++i) {
      const int c = lane + 64 * i;
      uint32_t xb[32];
      if (c < C) {
        const uint4 *src = reinterpret_cast<const uint4 *>(a.x + 32 * c);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const uint4 q = src[v];
          xb[8 * v + 0] = q.x & 0xffffu; xb[8 * v + 1] = q.x >> 16;
          xb[8 * v + 2] = q.y & 0xffffu; xb[8 * v + 3] = q.y >> 16;
          xb[8 * v + 4] = q.z & 0xffffu; xb[8 * v + 5] = q.z >> 16;
          xb[8 * v + 6] = q.w & 0xffffu; xb[8 * v + 7] = q.w >> 16;
        }
      } else {
#pragma unroll
        for (int v = 0; v < 32; ++v) xb[v] = 0;
      }
      XChunk xc;
      make_xchunk_bf16<BITS>(xc, xb);
#pragma unroll
      for (int u = 0; u < UA; ++u) {
        uint32_t q[16];
        unpack_chunk<BITS>(q, wg[u][i], kc);
        pg[u] += chunk_fold<BITS>(pairs_dot(q, xc.p), sg[u][i], bg[u][i], xc.xs, xc.xsp);
        unpack_chunk<BITS>(q, wu[u][i], kc);
        pu[u] += chunk_fold<BITS>(pairs_dot(q, xc.p), su[u][i], bu[u][i], xc.xs, xc.xsp);
      }
    }
    float hv[UA];
#pragma unroll
    for (int u = 0; u < UA; ++u) {
      const float gv = wave_sum_f32(pg[u]);
      const float uv = wave_sum_f32(pu[u]);
      hv[u] = silu(gv) * uv;  // logan-qwen4/src/lib.rs:8807-8809
    }
    float *hrow = reinterpret_cast<float *>(a.ws) + (size_t)slot * hmax;
    if (lane < UA && j0 + lane < rows) {
      float v = hv[0];
#pragma unroll
      for (int u = 1; u < UA; ++u) v = lane == u ? hv[u] : v;
      hrow[j0 + lane] = v;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    if (lane == 0) __hip_atomic_fetch_add(&g_fused_sync.a_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  // -------------------------------------------------------------- phase B
  const int bb = blockIdx.x - g.nA_blocks;
  const int lb = lane % LANESB;           // chunk of a down row
  const int rsub = lane / LANESB;
  const int d = (bb * 4 + wave) * ROWS_B + rsub;
  const bool drow = d < a.D;
  const bool has_shared = a.sdown.m.w != nullptr;

  uint32_t sel[kFusedMaxSlots];
  wave_route_bf16<KPL>(logits, a.E, g.k, sel);
  float wr[kFusedMaxSlots];
  {
    const float l0 = sel_logit(sel[0]);
    float ws = 0.f;
#pragma unroll
    for (int r = 0; r < kFusedMaxSlots; ++r) {
      wr[r] = 0.f;
      if (r < g.k) {
        wr[r] = __expf(sel_logit(sel[r]) - l0);
        ws += wr[r];
      }
    }
#pragma unroll
    for (int r = 0; r < kFusedMaxSlots; ++r) wr[r] = wr[r] / ws;
  }
  if (bb == 0 && threadIdx.x == 0) {
    for (int r = 0; r < g.k; ++r) {
      if (a.idx_out) a.idx_out[r] = sel_expert(sel[r]);
      if (a.w_out) a.w_out[r] = wr[r];
    }
  }

  // issue every slot's down-row loads now
  uint32_t wv[kFusedMaxSlots][BITS];
  float sc[kFusedMaxSlots], bi[kFusedMaxSlots];
#pragma unroll
  for (int s = 0; s < kFusedMaxSlots; ++s) {
    const bool sh = s == g.k;
    const bool live = s < g.slots;
    const DevBank &bd = sh ? a.sdown : a.down;
    const int e = sh ? 0 : sel_expert(sel[s < g.k ? s : 0]);
    const int K = sh ? a.sinter : a.inter;
    if (live && drow && lb < (K >> 5)) {
      load_chunk<BITS>(wv[s], bd.m.w + (size_t)e * bd.w_stride + (size_t)d * bd.m.row_bytes +
                                  (size_t)lb * (4 * BITS));
    } else {
#pragma unroll
      for (int t = 0; t < BITS; ++t) wv[s][t] = 0;
    }
  }
#pragma unroll
  for (int s = 0; s < kFusedMaxSlots; ++s) {
    const bool sh = s == g.k;
    const bool live = s < g.slots;
    const DevBank &bd = sh ? a.sdown : a.down;
    const int e = sh ? 0 : sel_expert(sel[s < g.k ? s : 0]);
    const int K = sh ? a.sinter : a.inter;
    if (live && drow && lb < (K >> 5)) {
      const size_t p = (size_t)e * bd.p_stride + (size_t)d * bd.m.ng + lb / (bd.m.gs >> 5);
      sc[s] = aux_to_f32(bd.m.sc[p], bd.m.fp16);
      bi[s] = aux_to_f32(bd.m.bi[p], bd.m.fp16);
    } else {
      sc[s] = bi[s] = 0.f;
    }
  }
  // shared-expert scalar gate (logan-qwen4/src/lib.rs:7602-7604)
  float gsig = 1.0f;
  if (has_shared && a.se_gate_vec) {
    float acc = 0.f;
    for (int j = lane; j < a.D; j += 64)
      acc = fmaf(bf16_to_f32(a.se_gate_vec[j]), bf16_to_f32(a.x[j]), acc);
    acc = wave_sum_f32(acc);
    gsig = 1.0f / (1.0f + __expf(-acc));
  }

  // wait for every A wave
  __shared__ uint32_t s_timeout;
  if (threadIdx.x == 0) {
    uint32_t spins = 0, to = 0;
    while (__hip_atomic_load(&g_fused_sync.a_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
           (uint32_t)g.nA_waves) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > kSpinLimit) {
        to = 1;
        __hip_atomic_fetch_or(&g_fused_sync.error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    s_timeout = to;
  }
  __syncthreads();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

  // stage h of every slot as x-operands in LDS
  {
    const int CI = hmax >> 5;
    const int items = g.slots * LANESB;
    for (int it = threadIdx.x; it < items; it += 256) {
      const int s = it / LANESB, c = it % LANESB;
      const int K = (has_shared && s == g.k) ? a.sinter : a.inter;
      float xf[32];
      if (c < (K >> 5) && c < CI) {
        const float4 *src = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(a.ws) +
                                                             (size_t)s * hmax + 32 * c);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const float4 t = src[v];
          xf[4 * v + 0] = t.x; xf[4 * v + 1] = t.y; xf[4 * v + 2] = t.z; xf[4 * v + 3] = t.w;
        }
      } else {
#pragma unroll
        for (int v = 0; v < 32; ++v) xf[v] = 0.f;
      }
      XChunk xh, xl;
      make_xchunk_f32<BITS>(xh, xl, xf);
      uint32_t *dst = s_h + (size_t)it * XDW;
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        dst[p] = xh.p[p];
        dst[16 + p] = xl.p[p];
      }
      dst[32] = __float_as_uint(xh.xs);
      dst[33] = __float_as_uint(xh.xsp);
    }
  }
  __syncthreads();

  float acc_out = 0.f, y_sh = 0.f;
#pragma unroll
  for (int s = 0; s < kFusedMaxSlots; ++s) {
    if (s < g.slots) {
      const uint32_t *src = s_h + (size_t)(s * LANESB + lb) * XDW;
      uint32_t hp[16], lp[16];
#pragma unroll
      for (int p = 0; p < 16; p += 4) {
        const uint4 t0 = *reinterpret_cast<const uint4 *>(src + p);
        const uint4 t1 = *reinterpret_cast<const uint4 *>(src + 16 + p);
        hp[p] = t0.x; hp[p + 1] = t0.y; hp[p + 2] = t0.z; hp[p + 3] = t0.w;
        lp[p] = t1.x; lp[p + 1] = t1.y; lp[p + 2] = t1.z; lp[p + 3] = t1.w;
      }
      const float xs = __uint_as_float(src[32]), xsp = __uint_as_float(src[33]);
      uint32_t q[16];
      unpack_chunk<BITS>(q, wv[s], kc);
      const float acc = pairs_dot(q, hp) + pairs_dot(q, lp);
      float v = chunk_fold<BITS>(acc, sc[s], bi[s], xs, xsp);
      v = group_sum_f32<LANESB>(v);
      if (s < g.k)
        acc_out = fmaf(v, wr[s], acc_out);  // rank order, as lib.rs:8692-8698
      else
        y_sh = v;
    }
  }
  const float o = has_shared ? fmaf(y_sh, gsig, acc_out) : acc_out;
  if (lb == 0 && drow && !s_timeout) {
    if (a.out_f32)
      reinterpret_cast<float *>(a.out)[d] = o;
    else
      reinterpret_cast<uint16_t *>(a.out)[d] = (uint16_t)f32_to_bf16_rne(o);
  }

  // last B block resets the arrival counters for the next launch
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(&g_fused_sync.b_done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (uint32_t)g.nB_blocks - 1) {
      __hip_atomic_store(&g_fused_sync.a_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&g_fused_sync.b_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(&g_fused_sync.launches, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------- launch

size_t moe_fused_workspace_bytes(int slots, int inter, int sinter) {
  const size_t hmax = (size_t)(inter > sinter ? inter : sinter);
  return (size_t)slots * hmax * sizeof(float);
}

template <int BITS, int CPLA, int LANESB, int KPL>
static int fused_launch(const MoeArgs &a, const FusedGeom &g, hipStream_t st) {
  auto kern = moe_fused_b1_kernel<BITS, CPLA, LANESB, KPL>;
  hipLaunchKernelGGL(kern, dim3(g.nA_blocks + g.nB_blocks), dim3(256), 0, st, a, g);
  return hipGetLastError() == hipSuccess ? 1 : -1;
}

template <int BITS, int CPLA, int LANESB>
static int fused_kpl(const MoeArgs &a, const FusedGeom &g, hipStream_t st) {
  if (a.E <= 512) return fused_launch<BITS, CPLA, LANESB, 8>(a, g, st);
  if (a.E <= 1024) return fused_launch<BITS, CPLA, LANESB, 16>(a, g, st);
  return 0;
}

template <int BITS>
static int fused_bits(const MoeArgs &a, const FusedGeom &g, hipStream_t st) {
  const int Cd = a.D >> 5;
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  const int Ci = hmax >> 5;
  if (Cd > 128 || Ci > 32) return 0;
  if (Cd <= 64) return Ci <= 16 ? fused_kpl<BITS, 1, 16>(a, g, st) : fused_kpl<BITS, 1, 32>(a, g, st);
  return Ci <= 16 ? fused_kpl<BITS, 2, 16>(a, g, st) : fused_kpl<BITS, 2, 32>(a, g, st);
}

// 1 launched, 0 not applicable (caller uses the multi-launch path), -1 error
int launch_moe_fused_b1(const MoeArgs &a, hipStream_t st) {
  if (a.B != 1 || a.logits_f32) return 0;
  const int slots = a.k + (a.sdown.m.w ? 1 : 0);
  if (slots > kFusedMaxSlots || a.E > 1024) return 0;
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  if (a.ws_bytes < moe_fused_workspace_bytes(slots, a.inter, a.sinter)) return 0;
  if ((reinterpret_cast<uintptr_t>(a.ws) & 15) != 0 || (hmax & 3) != 0) return 0;
  const int UA = a.gate.m.bits == 8 ? 2 : 4;
  FusedGeom g;
  g.k = a.k;
  g.slots = slots;
  g.wpr = (a.inter + UA - 1) / UA;
  g.wps = a.sdown.m.w ? (a.sinter + UA - 1) / UA : 0;
  g.nA_waves = g.k * g.wpr + g.wps;
  g.nA_blocks = (g.nA_waves + 3) / 4;
  const int Ci = hmax >> 5;
  const int lanesb = Ci <= 16 ? 16 : 32;
  const int rows_per_block = 4 * (64 / lanesb);
  g.nB_blocks = (a.D + rows_per_block - 1) / rows_per_block;
  switch (a.gate.m.bits) {
    case 4: return fused_bits<4>(a, g, st);
    case 5: return fused_bits<5>(a, g, st);
    case 6: return fused_bits<6>(a, g, st);
    case 8: return fused_bits<8>(a, g, st);
  }
  return 0;
}

uint32_t moe_fused_sync_errors() {
  FusedSync s{};
  if (hipMemcpyFromSymbol(&s, HIP_SYMBOL(g_fused_sync), sizeof(s), 0, hipMemcpyDeviceToHost) !=
      hipSuccess)
    return 0xffffffffu;
  return s.error | (s.a_done ? 2u : 0u) | (s.b_done ? 4u : 0u);
}

}  // namespace lh
