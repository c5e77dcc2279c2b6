// Single-launch routed-MoE block for one token (B = 1), gfx950.
//
// One kernel, two kinds of blocks, one hand-off:
//
//   A blocks (first in the grid): each wave owns UA rows j of one expert slot
//   (rank r < k of the route, or the shared expert) and computes
//   h[slot][j] = silu(gate_j . x) * (up_j . x) for them; once the block's h
//   stores have completed, the block makes one atomic arrival.
//
//   B blocks: a block owns ROWS_B output rows d; wave w covers half of them
//   for a quarter of the k+1 slots. Each wave issues the shared slot's
//   down-row loads and the shared-expert gate loads before routing and the
//   routed down rows right after it, so they stream from HBM while A runs;
//   wave 0 computes the shared-expert scalar gate sigmoid(se_g . x). After
//   every A arrival the block stages all h (as bf16 hi/lo x-operands) in LDS,
//   each wave forms its per-slot down products, and the block combines them
//   per row in rank order:
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
// The arrival and completion counters live in module-scope device memory
// (zero when the code object loads). B blocks count their completion over
// kDoneCtrs counters and then one top counter; the block that completes the
// count puts every counter back to zero, so each
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
constexpr int kDoneCtrs = 16;  // B completion: block b -> bctr[b % 16], then btop
struct FusedSync {
  uint32_t ctr[kArrivalCtrs][kLine];
  uint32_t bctr[kDoneCtrs][kLine];
  uint32_t btop[kLine];
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

template <int KPL>
__device__ __forceinline__ void route_select(uint32_t (&key)[KPL], int E, int rounds,
                                             uint32_t (&sel)[kFusedMaxSlots]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int e = i * 64 + lane;
    key[i] = e < E ? ((ord16(key[i]) << 16) | (0xffffu - (uint32_t)e)) : 0u;
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

constexpr int kWaves = 8;   // waves per block (512 threads)
constexpr int kQSlots = 3;  // slots per B wave (a quarter of kFusedMaxSlots)

// one slot's down-row chunk and its scale/bias
template <int BITS>
__device__ __forceinline__ void load_down(uint32_t (&w)[BITS], float &sc, float &bi,
                                          const DevBank &bd, int e, int d, int lb, bool live) {
  if (live) {
    load_chunk<BITS>(w, bd.m.w + (size_t)e * bd.w_stride + (size_t)d * bd.m.row_bytes +
                            (size_t)lb * (4 * BITS));
    const size_t p = (size_t)e * bd.p_stride + (size_t)d * bd.m.ng + lb / (bd.m.gs >> 5);
    sc = aux_to_f32(bd.m.sc[p], bd.m.fp16);
    bi = aux_to_f32(bd.m.bi[p], bd.m.fp16);
  } else {
#pragma unroll
    for (int q = 0; q < BITS; ++q) w[q] = 0;
    sc = bi = 0.f;
  }
}

template <int BITS, int CPLA, int LANESB, int KPL>
__global__ __launch_bounds__(kWaves * 64) void moe_fused_b1_kernel(MoeArgs a, FusedGeom g) {
  constexpr int UA = BITS == 8 ? 2 : 4;      // rows of gate (and of up) per A wave
  constexpr int ROWS_W = 64 / LANESB;        // output rows per B wave
  constexpr int ROWS_B = 2 * ROWS_W;         // output rows per B block (2 row groups x 4 slot quarters)
  constexpr int XDW = 36;                    // LDS dwords per (slot, chunk): 16 hi, 16 lo, xs, xsp
  __shared__ __align__(16) uint32_t s_h[kFusedMaxSlots * LANESB * XDW];
  __shared__ float s_y[ROWS_B][kFusedMaxSlots];
  __shared__ uint32_t s_timeout;
  __shared__ float s_gsig;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint16_t *logits = reinterpret_cast<const uint16_t *>(a.logits);
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  const int C = a.D >> 5;
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

    uint32_t key[KPL];
    if (!shared) route_keys<KPL>(logits, a.E, key);
    // x does not depend on the route: in flight together with the logits
    uint4 xq[CPLA][4];
#pragma unroll
    for (int i = 0; i < CPLA; ++i) {
      const int c = lane + 64 * i;
      const uint4 *src = reinterpret_cast<const uint4 *>(a.x + 32 * (c < C ? c : 0));
#pragma unroll
      for (int v = 0; v < 4; ++v) xq[i][v] = src[v];
    }
    int e = 0;
    if (!shared) {
      uint32_t sel[kFusedMaxSlots];
      route_select<KPL>(key, a.E, slot + 1, sel);
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
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint4 q = xq[i][v];
        const bool ok = c < C;
        xb[8 * v + 0] = ok ? q.x & 0xffffu : 0u; xb[8 * v + 1] = ok ? q.x >> 16 : 0u;
        xb[8 * v + 2] = ok ? q.y & 0xffffu : 0u; xb[8 * v + 3] = ok ? q.y >> 16 : 0u;
        xb[8 * v + 4] = ok ? q.z & 0xffffu : 0u; xb[8 * v + 5] = ok ? q.z >> 16 : 0u;
        xb[8 * v + 6] = ok ? q.w & 0xffffu : 0u; xb[8 * v + 7] = ok ? q.w >> 16 : 0u;
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
  // wave w: row group w % 2 (ROWS_W rows), slot quarter w / 2
  const int bb = blockIdx.x - g.nA_blocks;
  const int lb = lane % LANESB;  // chunk of a down row
  const int rloc = (wave & 1) * ROWS_W + lane / LANESB;
  const int d = bb * ROWS_B + rloc;
  const bool drow = d < a.D;
  const int sq = wave >> 1;
  const int s_lo = (g.slots * sq) / 4;
  const int s_hi = (g.slots * (sq + 1)) / 4;
  const bool has_shared = a.sdown.m.w != nullptr;

  uint32_t key[KPL];
  route_keys<KPL>(logits, a.E, key);

  // route-independent loads first: the shared slot's down rows, x and se_g
  uint32_t wv[kQSlots][BITS];
  float sc[kQSlots], bi[kQSlots];
#pragma unroll
  for (int t = 0; t < kQSlots; ++t) {
    const int s = s_lo + t;
    const bool live = has_shared && s == g.k && s < s_hi && drow && lb < (a.sinter >> 5);
    load_down<BITS>(wv[t], sc[t], bi[t], a.sdown, 0, d, lb, live);
  }
  uint4 gq[CPLA][4], xq[CPLA][4];
  const bool do_gate = wave == 0 && has_shared && a.se_gate_vec;
  if (do_gate) {
#pragma unroll
    for (int i = 0; i < CPLA; ++i) {
      const int c = lane + 64 * i;
      const uint4 *gv = reinterpret_cast<const uint4 *>(a.se_gate_vec + 32 * (c < C ? c : 0));
      const uint4 *xv = reinterpret_cast<const uint4 *>(a.x + 32 * (c < C ? c : 0));
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        gq[i][v] = gv[v];
        xq[i][v] = xv[v];
      }
    }
  }
  uint32_t sel[kFusedMaxSlots];
  route_select<KPL>(key, a.E, g.k, sel);
#pragma unroll
  for (int t = 0; t < kQSlots; ++t) {
    const int s = s_lo + t;
    if (s < g.k) {
      uint32_t kk = sel[0];
#pragma unroll
      for (int r = 1; r < kFusedMaxSlots; ++r) kk = r == s ? sel[r] : kk;
      const bool live = s < s_hi && drow && lb < (a.inter >> 5);
      load_down<BITS>(wv[t], sc[t], bi[t], a.down, sel_expert(kk), d, lb, live);
    }
  }
  // shared-expert scalar gate sigmoid(se_g . x) (logan-qwen4/src/lib.rs:7602-7604)
  if (wave == 0) {
    float gsig = 1.0f;
    if (do_gate) {
      float gd = 0.f;
#pragma unroll
      for (int i = 0; i < CPLA; ++i) {
        if (lane + 64 * i < C) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            gd = dot2(gq[i][v].x, xq[i][v].x, gd);
            gd = dot2(gq[i][v].y, xq[i][v].y, gd);
            gd = dot2(gq[i][v].z, xq[i][v].z, gd);
            gd = dot2(gq[i][v].w, xq[i][v].w, gd);
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
  for (int t = 0; t < kQSlots; ++t) {
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

  // completion: the last B block (two-level count) resets every counter
  __syncthreads();
  if (threadIdx.x == 0) {
    const int nb = g.nB_blocks;
    const int c = bb % kDoneCtrs;
    const int nbc = nb < kDoneCtrs ? nb : kDoneCtrs;
    const int needc = nb / kDoneCtrs + (c < nb % kDoneCtrs ? 1 : 0);
    const uint32_t prev =
        __hip_atomic_fetch_add(&g_fused_sync.bctr[c][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (uint32_t)needc - 1) {
      const uint32_t top =
          __hip_atomic_fetch_add(&g_fused_sync.btop[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (top == (uint32_t)nbc - 1) {
        for (int q = 0; q < kArrivalCtrs; ++q) st_agent(&g_fused_sync.ctr[q][0], 0u);
        for (int q = 0; q < kDoneCtrs; ++q) st_agent(&g_fused_sync.bctr[q][0], 0u);
        st_agent(&g_fused_sync.btop[0], 0u);
      }
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
  if ((reinterpret_cast<uintptr_t>(a.x) & 15) != 0) return 0;
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
  const int rows_per_block = 2 * (64 / lanesb);
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
  uint32_t busy = 0, bbusy = s.btop[0];
  for (int c = 0; c < kArrivalCtrs; ++c) busy |= s.ctr[c][0];
  for (int c = 0; c < kDoneCtrs; ++c) bbusy |= s.bctr[c][0];
  return s.error[0] | (busy ? 2u : 0u) | (bbusy ? 4u : 0u);
}

}  // namespace lh
