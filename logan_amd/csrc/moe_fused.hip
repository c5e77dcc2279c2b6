// Single-launch routed-MoE block for one token (B = 1), gfx950.
//
// One kernel, two kinds of blocks, one hand-off:
//
//   A blocks (first in the grid): each wave owns UA rows j of one expert slot
//   (rank r < k of the route, or the shared expert) and computes
//   h[slot][j] = silu(gate_j . x) * (up_j . x) for them; once the block's h
//   stores have completed, the block makes one atomic arrival.
//
//   B blocks: a block owns ROWS_B output rows d; wave w covers a quarter of
//   them for one half of the k+1 slots. Each wave issues the loads of its
//   down-projection weights right after routing (so they stream from HBM
//   while A runs); wave 0 computes the shared-expert scalar gate
//   sigmoid(se_g . x). After every A arrival the block stages all h (as bf16
//   hi/lo x-operands) in LDS, each wave forms its per-slot down products, and
//   the block combines them per row in rank order:
//   out[d] = sum_{r<k} w_r * (down_r . h_r)[d] + gs * (down_shared . h_shared)[d]
//   (logan-qwen4/src/lib.rs:8692-8711, :7597-7759).
//
// Every wave computes the route itself from the bf16 logits (top-k with the
// key (logit desc, index asc): per-lane sorted keys, k rounds of a DPP wave
// max), so no block waits for another before streaming weights.
//
// Progress: A blocks never wait on another block. Workgroups are dispatched in
// ID order, and every A block precedes every B block, so a B block can only be
// resident after all A blocks were dispatched: the waits always end. They are
// also bounded: after kSpinLimit polls a B block stops waiting, raises the
// sticky error word and finishes without writing its rows (the host can read
// the word with logan_hip_moe_sync_errors()).
//
// Hand-off without L2 maintenance: h is written and read only with
// device-scope (sc1) relaxed atomic stores/loads, which are coherent across
// the XCDs' L2s; an A wave waits for its h stores to complete (s_waitcnt)
// before its arrival atomic, and B reads h only after observing every
// arrival. An agent-scope release/acquire fence would instead write back /
// invalidate the whole L2 of each XCD per wave (buffer_wbl2 / buffer_inv),
// which measured tens of microseconds per launch here.
//
// The arrival counters live in module-scope device memory (zero when the code
// object loads) and the last B block to finish puts them back to zero, so each
// launch starts from zero without a memset. Launches of this kernel on one
// device must therefore not overlap (one stream, or serialised streams).
#include "affine_dev.hpp"
#include "lh_internal.hpp"

namespace lh {

// Arrivals are spread over kArrivalCtrs counters (A block b arrives on
// counter b % kArrivalCtrs), each on its own 256-byte line: same-address
// atomics serialise at the memory side (~40 ns each measured here), so one
// shared counter for every arrival would take tens of microseconds. B waits
// until each counter in use holds its expected count.
constexpr int kArrivalCtrs = 64;
constexpr int kLine = 64;  // u32 per 256-byte line
struct FusedSync {
  uint32_t ctr[kArrivalCtrs][kLine];
  uint32_t b_done[kLine];
  uint32_t error[kLine];
};
__device__ FusedSync g_fused_sync;

constexpr int kFusedMaxSlots = 12;  // k + 1 (routed + shared)
constexpr int kBufWord3 = 0x00020000;  // gfx9 raw buffer resource, 32-bit data format
constexpr int kCpolSc1 = 16;           // cache policy: device scope (sc1)
typedef float float4v __attribute__((ext_vector_type(4)));
constexpr uint32_t kSpinLimit = 1u << 20;

__device__ __forceinline__ uint32_t ld_agent(uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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
  int nctr;        // arrival counters in use
};

constexpr int kWaves = 8;              // waves per block (512 threads)
constexpr int kHalfSlots = (kFusedMaxSlots + 1) / 2;

template <int BITS, int CPLA, int LANESB, int KPL>
__global__ __launch_bounds__(kWaves * 64) void moe_fused_b1_kernel(MoeArgs a, FusedGeom g) {
  constexpr int UA = BITS == 8 ? 2 : 4;      // rows of gate (and of up) per A wave
  constexpr int ROWS_W = 64 / LANESB;        // output rows per B wave
  constexpr int ROWS_B = 4 * ROWS_W;         // output rows per B block (4 row groups x 2 slot halves)
  constexpr int XDW = 36;                    // LDS dwords per (slot, chunk): 16 hi, 16 lo, xs, xsp
  __shared__ __align__(16) uint32_t s_h[kFusedMaxSlots * LANESB * XDW];
  __shared__ float s_y[ROWS_B][kFusedMaxSlots];
  __shared__ uint32_t s_timeout;
  __shared__ float s_gsig;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint16_t *logits = reinterpret_cast<const uint16_t *>(a.logits);
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  UnpackConsts kc;
  kc.init();

  if ((int)blockIdx.x < g.nA_blocks) {
    // ------------------------------------------------------------ phase A
    const int item_raw = blockIdx.x * kWaves + wave;
    const bool active = item_raw < g.nA_waves;
    const int item = active ? item_raw : g.nA_waves - 1;  // idle waves mirror a valid item
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
    if (active && lane < UA && j0 + lane < rows) {
      float v = hv[0];
#pragma unroll
      for (int u = 1; u < UA; ++u) v = lane == u ? hv[u] : v;
      __hip_atomic_store(&hrow[j0 + lane], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);  // h stores complete before the arrival
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_fetch_add(&g_fused_sync.ctr[blockIdx.x % kArrivalCtrs][0], 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  // -------------------------------------------------------------- phase B
  // wave w: row group w % 4 (ROWS_W rows), slot half w / 4
  const int bb = blockIdx.x - g.nA_blocks;
  const int lb = lane % LANESB;           // chunk of a down row
  const int rloc = (wave & 3) * ROWS_W + lane / LANESB;
  const int d = bb * ROWS_B + rloc;
  const bool drow = d < a.D;
  const int half = wave >> 2;
  const int s_lo = half ? (g.slots + 1) / 2 : 0;
  const int s_hi = half ? g.slots : (g.slots + 1) / 2;
  const bool has_shared = a.sdown.m.w != nullptr;

  uint32_t sel[kFusedMaxSlots];
  wave_route_bf16<KPL>(logits, a.E, g.k, sel);

  // issue this wave's down-row loads (slots s_lo .. s_hi-1) now
  uint32_t wv[kHalfSlots][BITS];
  float sc[kHalfSlots], bi[kHalfSlots];
#pragma unroll
  for (int t = 0; t < kHalfSlots; ++t) {
    const int s = s_lo + t;
    const bool sh = s == g.k;
    const DevBank &bd = sh ? a.sdown : a.down;
    uint32_t key = sel[0];
#pragma unroll
    for (int r = 1; r < kFusedMaxSlots; ++r) key = r == s ? sel[r] : key;
    const int e = sh ? 0 : sel_expert(key);
    const int K = sh ? a.sinter : a.inter;
    if (s < s_hi && drow && lb < (K >> 5)) {
      load_chunk<BITS>(wv[t], bd.m.w + (size_t)e * bd.w_stride + (size_t)d * bd.m.row_bytes +
                                  (size_t)lb * (4 * BITS));
      const size_t p = (size_t)e * bd.p_stride + (size_t)d * bd.m.ng + lb / (bd.m.gs >> 5);
      sc[t] = aux_to_f32(bd.m.sc[p], bd.m.fp16);
      bi[t] = aux_to_f32(bd.m.bi[p], bd.m.fp16);
    } else {
#pragma unroll
      for (int q = 0; q < BITS; ++q) wv[t][q] = 0;
      sc[t] = bi[t] = 0.f;
    }
  }

  // shared-expert scalar gate sigmoid(se_g . x) (logan-qwen4/src/lib.rs:7602-7604):
  // wave 0 reads se_g and x as 16-byte loads, all in flight at once
  if (wave == 0) {
    float gsig = 1.0f;
    if (has_shared && a.se_gate_vec) {
      float gd = 0.f;
      const int C = a.D >> 5;
#pragma unroll
      for (int i = 0; i < CPLA; ++i) {
        const int c = lane + 64 * i;
        if (c < C) {
          const uint4 *gv = reinterpret_cast<const uint4 *>(a.se_gate_vec + 32 * c);
          const uint4 *xv = reinterpret_cast<const uint4 *>(a.x + 32 * c);
          uint4 gq[4], xq[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            gq[v] = gv[v];
            xq[v] = xv[v];
          }
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            gd = dot2(gq[v].x, xq[v].x, gd);
            gd = dot2(gq[v].y, xq[v].y, gd);
            gd = dot2(gq[v].z, xq[v].z, gd);
            gd = dot2(gq[v].w, xq[v].w, gd);
          }
        }
      }
      gd = wave_sum_f32(gd);
      gsig = 1.0f / (1.0f + __expf(-gd));
    }
    if (lane == 0) s_gsig = gsig;
  }

  // wait until every arrival counter in use holds its expected count
  if (wave == 0) {
    uint32_t spins = 0, to = 0;
    const int need = lane < g.nctr
                         ? g.nA_blocks / kArrivalCtrs + (lane < g.nA_blocks % kArrivalCtrs ? 1 : 0)
                         : 0;
    bool done = lane >= g.nctr || ld_agent(&g_fused_sync.ctr[lane][0]) == (uint32_t)need;
    while (!__all(done)) {
      __builtin_amdgcn_s_sleep(2);
      if (!done) done = ld_agent(&g_fused_sync.ctr[lane][0]) == (uint32_t)need;
      if (++spins > kSpinLimit) {
        to = 1;
        if (lane == 0)
          __hip_atomic_fetch_or(&g_fused_sync.error[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    if (lane == 0) s_timeout = to;
  }
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);

  // stage h of every slot as x-operands in LDS
  {
    const int CI = hmax >> 5;
    const int items = g.slots * LANESB;
    const __amdgpu_buffer_rsrc_t hrsrc = __builtin_amdgcn_make_buffer_rsrc(
        a.ws, (short)0, g.slots * hmax * 4, kBufWord3);
    for (int it = threadIdx.x; it < items; it += kWaves * 64) {
      const int s = it / LANESB, c = it % LANESB;
      const int K = (has_shared && s == g.k) ? a.sinter : a.inter;
      float xf[32];
      if (c < (K >> 5) && c < CI) {
        // device-scope (sc1) 16-byte loads: coherent with A's sc1 stores
        const int off = (s * hmax + 32 * c) * 4;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const float4v t = __builtin_bit_cast(
              float4v, __builtin_amdgcn_raw_buffer_load_b128(hrsrc, off + 16 * v, 0, kCpolSc1));
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

#pragma unroll
  for (int t = 0; t < kHalfSlots; ++t) {
    const int s = s_lo + t;
    if (s < s_hi) {
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
      unpack_chunk<BITS>(q, wv[t], kc);
      const float acc = pairs_dot(q, hp) + pairs_dot(q, lp);
      float v = chunk_fold<BITS>(acc, sc[t], bi[t], xs, xsp);
      v = group_sum_f32<LANESB>(v);
      if (lb == 0) s_y[rloc][s] = v;
    }
  }
  __syncthreads();

  // rank-ordered combine (logan-qwen4/src/lib.rs:8692-8711) by the first ROWS_B threads
  if ((int)threadIdx.x < ROWS_B) {
    const int r = threadIdx.x;
    const int dd = bb * ROWS_B + r;
    float wr[kFusedMaxSlots];
    const float l0 = sel_logit(sel[0]);
    float wsum = 0.f;
#pragma unroll
    for (int q = 0; q < kFusedMaxSlots; ++q) {
      wr[q] = 0.f;
      if (q < g.k) {
        wr[q] = __expf(sel_logit(sel[q]) - l0);
        wsum += wr[q];
      }
    }
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < kFusedMaxSlots; ++q)
      if (q < g.k) acc = fmaf(s_y[r][q], wr[q] / wsum, acc);
    float o = acc;
    if (has_shared) o = fmaf(s_y[r][g.k], s_gsig, acc);
    if (dd < a.D && !s_timeout) {
      if (a.out_f32)
        reinterpret_cast<float *>(a.out)[dd] = o;
      else
        reinterpret_cast<uint16_t *>(a.out)[dd] = (uint16_t)f32_to_bf16_rne(o);
    }
    if (bb == 0 && r == 0) {
      for (int q = 0; q < g.k; ++q) {
        if (a.idx_out) a.idx_out[q] = sel_expert(sel[q]);
        if (a.w_out) a.w_out[q] = wr[q] / wsum;
      }
    }
  }

  // last B block resets the arrival counters for the next launch
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(&g_fused_sync.b_done[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (uint32_t)g.nB_blocks - 1) {
      for (int c = 0; c < kArrivalCtrs; ++c) st_agent(&g_fused_sync.ctr[c][0], 0u);
      st_agent(&g_fused_sync.b_done[0], 0u);
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
  hipLaunchKernelGGL(kern, dim3(g.nA_blocks + g.nB_blocks), dim3(kWaves * 64), 0, st, a, g);
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
  if (a.se_gate_vec && (reinterpret_cast<uintptr_t>(a.se_gate_vec) & 15) != 0) return 0;
  FusedGeom g;
  g.k = a.k;
  g.slots = slots;
  g.wpr = (a.inter + UA - 1) / UA;
  g.wps = a.sdown.m.w ? (a.sinter + UA - 1) / UA : 0;
  g.nA_waves = g.k * g.wpr + g.wps;
  g.nA_blocks = (g.nA_waves + kWaves - 1) / kWaves;
  g.nctr = g.nA_blocks < kArrivalCtrs ? g.nA_blocks : kArrivalCtrs;
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
  static FusedSync s;
  if (hipMemcpyFromSymbol(&s, HIP_SYMBOL(g_fused_sync), sizeof(s), 0, hipMemcpyDeviceToHost) !=
      hipSuccess)
    return 0xffffffffu;
  uint32_t busy = 0;
  for (int c = 0; c < kArrivalCtrs; ++c) busy |= s.ctr[c][0];
  return s.error[0] | (busy ? 2u : 0u) | (s.b_done[0] ? 4u : 0u);
}

}  // namespace lh
