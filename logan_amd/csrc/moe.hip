// Router top-k and the routed-MoE block (device-native, bf16 activations).
//
// Semantics follow logan-qwen/src/lib.rs:535-593 and
// logan-qwen4/src/lib.rs:7993-8043, :8692-8711, :8759-8815, :7597-7759:
//   probs = softmax(logits); top-k with lower-index ties; weight_r =
//   val_r / sum_{r<k} val_r; h = silu(gate.x) * (up.x); y_r = down.h;
//   out = sum_r (y_r * weight_r) in rank order + sy * sigmoid(se_g.x).
//
// Selection is done on the logits with the key (logit desc, index asc).
// softmax is strictly increasing in the logit wherever exp(l - max) does not
// underflow, so equal logits <=> equal probabilities and the order matches
// the reference's selection on probabilities. Weights are
// exp(l_r - l_0) / sum_{r<k} exp(l_j - l_0), which equals val_r / wsum.
//
// Launch structure (all on one stream):
//   1. moe_route_group_kernel   one block: route every token, shared-expert
//                               gate, group (token, rank) slots by expert
//   2. moe_gateup_kernel        per (expert group, row block): gate and up
//                               rows unpacked once, applied to every token of
//                               the group, SwiGLU fused -> h[slot][j] (f32)
//   3. moe_down_kernel          per (expert group, row block): down rows
//                               unpacked once, applied to h of every slot
//                               -> y[slot][d] (f32)
//   4. moe_combine_kernel       out[t][d] = sum_r w_r y[t,r][d] (rank order)
//                               + gs_t * y[t,shared][d] -> bf16
#include <cstdlib>

#include "affine_dev.hpp"
#include "lh_internal.hpp"

namespace lh {

__device__ __forceinline__ uint32_t ord32(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0;  // -0 == +0, as the reference's comparison
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float unord32(uint32_t o) {
  const uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(u);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m, 64);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ float load_logit(const void *p, int f32, size_t i) {
  return f32 ? reinterpret_cast<const float *>(p)[i]
             : bf16_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
}

constexpr int kMaxE = 1024;  // 16 keys per lane
constexpr int kMaxK = 32;

// One wave selects the top-k of one row of E logits. Rank r's expert and
// logit land in sel_idx[r] / sel_l[r] (LDS, written by lane 0); weights
// w_r = exp(l_r - l_0) / sum_{j<k} exp(l_j - l_0) are written to sel_w[r].
template <bool F32>
__device__ __forceinline__ void wave_topk_t(const void *logits, size_t row_off, int E, int k,
                                            int *sel_idx, float *sel_l, float *sel_w) {
  const int lane = threadIdx.x & 63;
  uint64_t key[16];
  // branch-free loads: out-of-range lanes read element 0 and get key 0
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int e = i * 64 + lane;
    const bool ok = e < E;
    const size_t ei = row_off + (ok ? e : 0);
    const float l = F32 ? reinterpret_cast<const float *>(logits)[ei]
                        : bf16_to_f32(reinterpret_cast<const uint16_t *>(logits)[ei]);
    const uint64_t kk = ((uint64_t)ord32(l) << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
    key[i] = ok ? kk : 0ull;
  }
#pragma unroll 1
  for (int r = 0; r < k; ++r) {
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) best = key[i] > best ? key[i] : best;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint64_t other = shfl_xor_u64(best, o);
      best = other > best ? other : best;
    }
    const int e = (int)(0xffffffffu - (uint32_t)best);
    if (lane == 0) {
      sel_idx[r] = e;
      sel_l[r] = unord32((uint32_t)(best >> 32));
    }
    // keys are unique (the index is part of the key): clear the winner
#pragma unroll
    for (int i = 0; i < 16; ++i) key[i] = key[i] == best ? 0ull : key[i];
  }
  if (lane == 0) {
    float wsum = 0.f;
    const float l0 = sel_l[0];
    for (int r = 0; r < k; ++r) {
      const float ex = __expf(sel_l[r] - l0);
      sel_w[r] = ex;
      wsum += ex;
    }
    for (int r = 0; r < k; ++r) sel_w[r] = sel_w[r] / wsum;
  }
}

__device__ __forceinline__ void wave_topk(const void *logits, int f32, size_t row_off, int E,
                                          int k, int *sel_idx, float *sel_l, float *sel_w) {
  if (f32)
    wave_topk_t<true>(logits, row_off, E, k, sel_idx, sel_l, sel_w);
  else
    wave_topk_t<false>(logits, row_off, E, k, sel_idx, sel_l, sel_w);
}

__global__ __launch_bounds__(256) void route_topk_kernel(const void *logits, int f32, int B, int E,
                                                         int k, int32_t *idx, float *w) {
  __shared__ int s_idx[4][kMaxK];
  __shared__ float s_l[4][kMaxK], s_w[4][kMaxK];
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= B) return;
  wave_topk(logits, f32, (size_t)t * E, E, k, s_idx[wave], s_l[wave], s_w[wave]);
  if ((threadIdx.x & 63) == 0) {
    for (int r = 0; r < k; ++r) {
      idx[(size_t)t * k + r] = s_idx[wave][r];
      w[(size_t)t * k + r] = s_w[wave][r];
    }
  }
}

hipError_t launch_route_topk(const void *logits, int logits_f32, int B, int E, int k, int32_t *idx,
                             float *w, hipStream_t st) {
  if (B <= 0 || E <= 0 || E > kMaxE || k <= 0 || k > kMaxK || k > E) return hipErrorInvalidValue;
  hipLaunchKernelGGL(route_topk_kernel, dim3((B + 3) / 4), dim3(256), 0, st, logits, logits_f32, B,
                     E, k, idx, w);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Workspace layout (all offsets 256-byte aligned).

struct MoeWs {
  int *n_groups;      // [1]  routed groups
  int *group_expert;  // [G]
  int *group_off;     // [G+1] into entries
  int *entries;       // [B*k] routed slot ids, grouped by expert
  int32_t *topk_idx;  // [B*k]
  float *topk_w;      // [B*k]
  float *gs;          // [B]
  float *h;           // [(B*k+B) * hmax]
  float *y;           // [(B*k+B) * D]
  size_t total;
};

static inline size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

static MoeWs moe_ws_layout(void *base, int B, int D, int inter, int sinter, int E, int k) {
  MoeWs w{};
  const size_t G = (size_t)(B * k < E ? B * k : E);
  const size_t slots = (size_t)B * k + B;
  const size_t hmax = (size_t)(inter > sinter ? inter : sinter);
  size_t off = 0;
  char *b = reinterpret_cast<char *>(base);
  auto take = [&](size_t bytes) {
    char *p = b ? b + off : nullptr;
    off += al256(bytes);
    return p;
  };
  w.n_groups = reinterpret_cast<int *>(take(sizeof(int)));
  w.group_expert = reinterpret_cast<int *>(take(sizeof(int) * (G + 1)));
  w.group_off = reinterpret_cast<int *>(take(sizeof(int) * (G + 2)));
  w.entries = reinterpret_cast<int *>(take(sizeof(int) * (size_t)B * k));
  w.topk_idx = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * (size_t)B * k));
  w.topk_w = reinterpret_cast<float *>(take(sizeof(float) * (size_t)B * k));
  w.gs = reinterpret_cast<float *>(take(sizeof(float) * (size_t)B));
  w.h = reinterpret_cast<float *>(take(sizeof(float) * slots * hmax));
  w.y = reinterpret_cast<float *>(take(sizeof(float) * slots * (size_t)D));
  w.total = off;
  return w;
}

size_t moe_workspace_bytes(int B, int D, int inter, int sinter, int E, int k) {
  const size_t general = moe_ws_layout(nullptr, B, D, inter, sinter, E, k).total;
  const size_t fused = moe_fused_workspace_bytes(k + 1, inter, sinter);
  return general > fused ? general : fused;
}

static int g_fused_enabled = -1;

void set_moe_fused_enabled(int on) { g_fused_enabled = on; }

static bool fused_enabled() {
  if (g_fused_enabled < 0) {
    const char *v = getenv("LOGAN_HIP_MOE_FUSED");
    g_fused_enabled = (v && v[0] == '0') ? 0 : 1;
  }
  return g_fused_enabled != 0;
}

// ---------------------------------------------------------------------------
// 1. route + shared gate + grouping (one block of 1024 threads, B <= 64)

constexpr int kGroupThreads = 1024;
constexpr int kMaxB = 64;

__global__ __launch_bounds__(kGroupThreads) void moe_route_group_kernel(MoeArgs a, MoeWs w) {
  __shared__ int s_idx[kMaxB * kMaxK];
  __shared__ int s_cnt[kMaxE];
  __shared__ int s_start[kMaxE];
  __shared__ int s_gid[kMaxE];
  __shared__ int s_wave_tot[kGroupThreads / 64];
  __shared__ float s_l[kGroupThreads / 64][kMaxK], s_w[kGroupThreads / 64][kMaxK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nwaves = kGroupThreads / 64;
  const int nslots = a.B * a.k;

  for (int e = tid; e < a.E; e += kGroupThreads) s_cnt[e] = 0;

  for (int t = wave; t < a.B; t += nwaves) {
    wave_topk(a.logits, a.logits_f32, (size_t)t * a.E, a.E, a.k, &s_idx[t * a.k], s_l[wave],
              s_w[wave]);
    if (lane == 0) {
      for (int r = 0; r < a.k; ++r) {
        const int si = s_idx[t * a.k + r];
        const float sw = s_w[wave][r];
        w.topk_idx[t * a.k + r] = si;
        w.topk_w[t * a.k + r] = sw;
        if (a.idx_out) a.idx_out[t * a.k + r] = si;
        if (a.w_out) a.w_out[t * a.k + r] = sw;
      }
    }
    // shared-expert scalar gate: sigmoid(se_g . x_t) (logan-qwen4/src/lib.rs:7602-7604)
    if (a.sgate.m.w) {
      float g = 0.f;
      if (a.se_gate_vec) {
        for (int j = lane; j < a.D; j += 64)
          g = fmaf(bf16_to_f32(a.se_gate_vec[j]), bf16_to_f32(a.x[(size_t)t * a.D + j]), g);
        g = team_sum<64>(g);
        g = 1.0f / (1.0f + __expf(-g));
      } else {
        g = 1.0f;
      }
      if (lane == 0) w.gs[t] = g;
    }
  }
  __syncthreads();
  for (int i = tid; i < nslots; i += kGroupThreads) atomicAdd(&s_cnt[s_idx[i]], 1);
  __syncthreads();
  // exclusive scans over experts: entry start and group id (E <= 1024 = one per thread)
  {
    const int e = tid;
    const int c = e < a.E ? s_cnt[e] : 0;
    const int f = c > 0 ? 1 : 0;
    // pack (count, flag) into one int: count < 2^20, flag sum < 2^11
    int v = (c << 11) | f;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int n = __shfl_up(incl, o, 64);
      if (lane >= o) incl += n;
    }
    if (lane == 63) s_wave_tot[wave] = incl;
    __syncthreads();
    int prefix = 0;
    for (int q = 0; q < wave; ++q) prefix += s_wave_tot[q];
    const int excl = prefix + incl - v;
    if (e < a.E) {
      s_start[e] = excl >> 11;
      s_gid[e] = excl & 2047;
    }
    if (tid == kGroupThreads - 1) {
      const int tot = prefix + incl;
      *w.n_groups = tot & 2047;
    }
  }
  __syncthreads();
  for (int e = tid; e < a.E; e += kGroupThreads) {
    if (s_cnt[e] > 0) {
      const int g = s_gid[e];
      w.group_expert[g] = e;
      w.group_off[g] = s_start[e];
    }
  }
  if (tid == 0) {
    // group_off[n_groups] = nslots (the routed entries end)
    int ng = 0;
    for (int q = 0; q < nwaves; ++q) ng += s_wave_tot[q] & 2047;
    w.group_off[ng] = nslots;
  }
  // stable placement: position among equal experts follows slot order
  for (int i = tid; i < nslots; i += kGroupThreads) {
    const int e = s_idx[i];
    int before = 0;
    for (int j = 0; j < i; ++j) before += (s_idx[j] == e);
    w.entries[s_start[e] + before] = i;
  }
}

// ---------------------------------------------------------------------------
// 2. gate/up + SwiGLU

struct GroupView {
  const uint8_t *gw, *uw;
  const uint16_t *gsc, *gbi, *usc, *ubi;
  int rows;       // inter of this expert
  int slot_begin, slot_end;
  bool shared;
};

__device__ __forceinline__ bool moe_item_group(const MoeArgs &a, const MoeWs &w, int ng, int ipg,
                                               int ipg_s, int item, int &g, int &rb) {
  if (item < ng * ipg) {
    g = item / ipg;
    rb = item % ipg;
    return true;
  }
  const int si = item - ng * ipg;
  if (a.sgate.m.w && si < ipg_s) {
    g = -1;
    rb = si;
    return true;
  }
  return false;
}

template <int BITS, int LANES, int CPL, int U>
__global__ __launch_bounds__(256) void moe_gateup_kernel(MoeArgs a, MoeWs w, int ipg, int ipg_s) {
  constexpr int TEAMS = 256 / LANES;
  constexpr int RPB = TEAMS * U;  // rows per block
  const int lane = threadIdx.x & (LANES - 1);
  const int team = threadIdx.x / LANES;
  const int C = a.D >> 5;
  const int ng = *w.n_groups;
  const int n_items = ng * ipg + (a.sgate.m.w ? ipg_s : 0);
  UnpackConsts kc;
  kc.init();
  int gidx[CPL];
  bool cval[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + LANES * j;
    cval[j] = c < C;
    gidx[j] = c / (a.gate.m.gs >> 5);
  }

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    int g, rb;
    if (!moe_item_group(a, w, ng, ipg, ipg_s, item, g, rb)) break;
    const bool shared = g < 0;
    const DevBank &bg = shared ? a.sgate : a.gate;
    const DevBank &bu = shared ? a.sup : a.up;
    const int e = shared ? 0 : w.group_expert[g];
    const int rows = shared ? a.sinter : a.inter;
    const int s0 = shared ? 0 : w.group_off[g];
    const int s1 = shared ? a.B : w.group_off[g + 1];
    const uint8_t *gwb = bg.m.w + (size_t)e * bg.w_stride;
    const uint8_t *uwb = bu.m.w + (size_t)e * bu.w_stride;
    const uint16_t *gsc = bg.m.sc + (size_t)e * bg.p_stride;
    const uint16_t *gbi = bg.m.bi + (size_t)e * bg.p_stride;
    const uint16_t *usc = bu.m.sc + (size_t)e * bu.p_stride;
    const uint16_t *ubi = bu.m.bi + (size_t)e * bu.p_stride;
    const int j0 = rb * RPB + team * U;

    uint32_t wg[U][CPL][BITS], wu[U][CPL][BITS];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int row = j0 + u, c = lane + LANES * j;
        if (row < rows && cval[j]) {
          load_chunk<BITS>(wg[u][j], gwb + (size_t)row * bg.m.row_bytes + (size_t)c * (4 * BITS));
          load_chunk<BITS>(wu[u][j], uwb + (size_t)row * bu.m.row_bytes + (size_t)c * (4 * BITS));
        } else {
#pragma unroll
          for (int t = 0; t < BITS; ++t) wg[u][j][t] = wu[u][j][t] = 0;
        }
      }
    float sg[U][CPL], bg_[U][CPL], su[U][CPL], bu_[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int row = j0 + u;
        if (row < rows && cval[j]) {
          const size_t pg = (size_t)row * bg.m.ng + gidx[j];
          const size_t pu = (size_t)row * bu.m.ng + gidx[j];
          sg[u][j] = aux_to_f32(gsc[pg], bg.m.fp16);
          bg_[u][j] = aux_to_f32(gbi[pg], bg.m.fp16);
          su[u][j] = aux_to_f32(usc[pu], bu.m.fp16);
          bu_[u][j] = aux_to_f32(ubi[pu], bu.m.fp16);
        } else {
          sg[u][j] = bg_[u][j] = su[u][j] = bu_[u][j] = 0.f;
        }
      }
    uint32_t qg[U][CPL][16], qu[U][CPL][16];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        unpack_chunk<BITS>(qg[u][j], wg[u][j], kc);
        unpack_chunk<BITS>(qu[u][j], wu[u][j], kc);
      }

    for (int si = s0; si < s1; ++si) {
      const int slot = shared ? a.B * a.k + si : w.entries[si];
      const int t = shared ? si : slot / a.k;
      float pg[U], pu[U];
#pragma unroll
      for (int u = 0; u < U; ++u) pg[u] = pu[u] = 0.f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + LANES * j;
        uint32_t xb[32];
        if (cval[j]) {
          const uint4 *src = reinterpret_cast<const uint4 *>(a.x + (size_t)t * a.D + 32 * c);
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
        for (int u = 0; u < U; ++u) {
          pg[u] += chunk_fold<BITS>(pairs_dot(qg[u][j], xc.p), sg[u][j], bg_[u][j], xc.xs, xc.xsp);
          pu[u] += chunk_fold<BITS>(pairs_dot(qu[u][j], xc.p), su[u][j], bu_[u][j], xc.xs, xc.xsp);
        }
      }
      const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float gv = team_sum<LANES>(pg[u]);
        const float uv = team_sum<LANES>(pu[u]);
        const int row = j0 + u;
        // logan-qwen4/src/lib.rs:8807-8809: h = silu(gate) * up
        if (lane == 0 && row < rows) w.h[(size_t)slot * hmax + row] = silu(gv) * uv;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 3. down projection of h for every slot of a group

template <int BITS, int LANES, int U>
__global__ __launch_bounds__(256) void moe_down_kernel(MoeArgs a, MoeWs w, int ipg) {
  constexpr int TEAMS = 256 / LANES;
  constexpr int RPB = TEAMS * U;
  const int lane = threadIdx.x & (LANES - 1);
  const int team = threadIdx.x / LANES;
  const int ng = *w.n_groups;
  const int n_items = (ng + (a.sdown.m.w ? 1 : 0)) * ipg;
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  UnpackConsts kc;
  kc.init();

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int g = item / ipg, rb = item % ipg;
    const bool shared = g >= ng;
    const DevBank &bd = shared ? a.sdown : a.down;
    const int e = shared ? 0 : w.group_expert[g];
    const int K = shared ? a.sinter : a.inter;  // columns of down
    const int C = K >> 5;
    const int s0 = shared ? 0 : w.group_off[g];
    const int s1 = shared ? a.B : w.group_off[g + 1];
    const uint8_t *wb = bd.m.w + (size_t)e * bd.w_stride;
    const uint16_t *scb = bd.m.sc + (size_t)e * bd.p_stride;
    const uint16_t *bib = bd.m.bi + (size_t)e * bd.p_stride;
    const int d0 = rb * RPB + team * U;
    const bool cval = lane < C;
    const int gi = lane / (bd.m.gs >> 5);

    uint32_t wv[U][BITS];
    float sc[U], bi[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int d = d0 + u;
      if (d < a.D && cval) {
        load_chunk<BITS>(wv[u], wb + (size_t)d * bd.m.row_bytes + (size_t)lane * (4 * BITS));
      } else {
#pragma unroll
        for (int t = 0; t < BITS; ++t) wv[u][t] = 0;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int d = d0 + u;
      if (d < a.D && cval) {
        const size_t p = (size_t)d * bd.m.ng + gi;
        sc[u] = aux_to_f32(scb[p], bd.m.fp16);
        bi[u] = aux_to_f32(bib[p], bd.m.fp16);
      } else {
        sc[u] = bi[u] = 0.f;
      }
    }
    uint32_t q[U][16];
#pragma unroll
    for (int u = 0; u < U; ++u) unpack_chunk<BITS>(q[u], wv[u], kc);

    for (int si = s0; si < s1; ++si) {
      const int slot = shared ? a.B * a.k + si : w.entries[si];
      float xf[32];
      if (cval) {
        const float4 *src = reinterpret_cast<const float4 *>(w.h + (size_t)slot * hmax + 32 * lane);
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
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float acc = pairs_dot(q[u], xh.p) + pairs_dot(q[u], xl.p);
        float v = chunk_fold<BITS>(acc, sc[u], bi[u], xh.xs, xh.xsp);
        v = team_sum<LANES>(v);
        const int d = d0 + u;
        if (lane == 0 && d < a.D) w.y[(size_t)slot * a.D + d] = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 4. rank-ordered combine (logan-qwen4/src/lib.rs:8692-8711)

__global__ __launch_bounds__(256) void moe_combine_kernel(MoeArgs a, MoeWs w) {
  const long long n = (long long)a.B * a.D;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
    const int t = (int)(i / a.D), d = (int)(i % a.D);
    float acc = 0.f;
    for (int r = 0; r < a.k; ++r) {
      const int slot = t * a.k + r;
      acc = fmaf(w.y[(size_t)slot * a.D + d], w.topk_w[slot], acc);
    }
    float o = acc;
    if (a.sdown.m.w) {
      const int slot = a.B * a.k + t;
      o = fmaf(w.y[(size_t)slot * a.D + d], w.gs[t], acc);
    }
    if (a.out_f32)
      reinterpret_cast<float *>(a.out)[i] = o;
    else
      reinterpret_cast<uint16_t *>(a.out)[i] = (uint16_t)f32_to_bf16_rne(o);
  }
}

// ---------------------------------------------------------------------------

template <int BITS>
static int moe_launch_bits(const MoeArgs &a, const MoeWs &w, hipStream_t st) {
  const int Cd = a.D >> 5;
  const int G = a.B * a.k < a.E ? a.B * a.k : a.E;
  // gate/up
  {
    constexpr int U = 2;
    int lanes, cpl;
    if (Cd <= 16) { lanes = 16; cpl = 1; }
    else if (Cd <= 32) { lanes = 32; cpl = 1; }
    else if (Cd <= 64) { lanes = 64; cpl = 1; }
    else if (Cd <= 128) { lanes = 64; cpl = 2; }
    else return 0;
    const int rpb = (256 / lanes) * U;
    const int ipg = (a.inter + rpb - 1) / rpb;
    const int ipg_s = a.sgate.m.w ? (a.sinter + rpb - 1) / rpb : 0;
    const int grid = G * ipg + ipg_s;
    if (lanes == 16) hipLaunchKernelGGL((moe_gateup_kernel<BITS, 16, 1, U>), dim3(grid), dim3(256), 0, st, a, w, ipg, ipg_s);
    else if (lanes == 32) hipLaunchKernelGGL((moe_gateup_kernel<BITS, 32, 1, U>), dim3(grid), dim3(256), 0, st, a, w, ipg, ipg_s);
    else if (cpl == 1) hipLaunchKernelGGL((moe_gateup_kernel<BITS, 64, 1, U>), dim3(grid), dim3(256), 0, st, a, w, ipg, ipg_s);
    else hipLaunchKernelGGL((moe_gateup_kernel<BITS, 64, 2, U>), dim3(grid), dim3(256), 0, st, a, w, ipg, ipg_s);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  // down
  {
    constexpr int U = 2;
    const int kmax = a.inter > a.sinter ? a.inter : a.sinter;
    const int Ci = kmax >> 5;
    int lanes;
    if (Ci <= 16) lanes = 16;
    else if (Ci <= 32) lanes = 32;
    else if (Ci <= 64) lanes = 64;
    else return -1;
    const int rpb = (256 / lanes) * U;
    const int ipg = (a.D + rpb - 1) / rpb;
    const int grid = (G + (a.sdown.m.w ? 1 : 0)) * ipg;
    if (lanes == 16) hipLaunchKernelGGL((moe_down_kernel<BITS, 16, U>), dim3(grid), dim3(256), 0, st, a, w, ipg);
    else if (lanes == 32) hipLaunchKernelGGL((moe_down_kernel<BITS, 32, U>), dim3(grid), dim3(256), 0, st, a, w, ipg);
    else hipLaunchKernelGGL((moe_down_kernel<BITS, 64, U>), dim3(grid), dim3(256), 0, st, a, w, ipg);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  {
    long long n = (long long)a.B * a.D;
    long long blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a, w);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  return 1;
}

static bool bank_ok(const DevBank &b, int O, int I, int bits, int gs) {
  const DevMat &m = b.m;
  if (!m.w || !m.sc || !m.bi) return false;
  if (m.O != O || m.I != I || m.bits != bits || m.gs != gs) return false;
  if (m.gs <= 0 || m.gs % 32 != 0 || m.I % m.gs != 0) return false;
  if ((reinterpret_cast<uintptr_t>(m.w) & 15) != 0) return false;
  if (m.row_bytes != (long long)m.I * m.bits / 8) return false;
  if (b.w_stride % 16 != 0) return false;
  return true;
}

int launch_moe_block(const MoeArgs &a, hipStream_t st) {
  if (a.B <= 0 || a.B > kMaxB || a.E <= 0 || a.E > kMaxE || a.k <= 0 || a.k > kMaxK || a.k > a.E)
    return 0;
  if (a.D <= 0 || a.D % 32 != 0 || a.inter <= 0 || a.inter % 32 != 0) return 0;
  if (!a.x || !a.logits || !a.out || !a.ws) return 0;
  if ((reinterpret_cast<uintptr_t>(a.x) & 15) != 0) return 0;
  const int bits = a.gate.m.bits, gs = a.gate.m.gs;
  if (!(bits == 4 || bits == 5 || bits == 6 || bits == 8)) return 0;
  if (!bank_ok(a.gate, a.inter, a.D, bits, gs) || !bank_ok(a.up, a.inter, a.D, bits, gs)) return 0;
  if (!bank_ok(a.down, a.D, a.inter, bits, a.down.m.gs)) return 0;
  if (a.gate.E < a.E || a.up.E < a.E || a.down.E < a.E) return 0;
  if (a.sgate.m.w) {
    if (a.sinter <= 0 || a.sinter % 32 != 0) return 0;
    if (!bank_ok(a.sgate, a.sinter, a.D, bits, gs) || !bank_ok(a.sup, a.sinter, a.D, bits, gs)) return 0;
    if (!bank_ok(a.sdown, a.D, a.sinter, bits, a.sdown.m.gs)) return 0;
    if (a.sdown.m.gs != a.down.m.gs) return 0;
  }
  const int sinter = a.sgate.m.w ? a.sinter : 0;
  if (a.ws_bytes < moe_workspace_bytes(a.B, a.D, a.inter, sinter, a.E, a.k)) return 0;
  MoeArgs aa = a;
  aa.sinter = sinter;
  if (fused_enabled()) {
    const int rc = launch_moe_fused_b1(aa, st);
    if (rc != 0) return rc;
  }
  MoeWs w = moe_ws_layout(a.ws, a.B, a.D, a.inter, sinter, a.E, a.k);
  hipLaunchKernelGGL(moe_route_group_kernel, dim3(1), dim3(kGroupThreads), 0, st, aa, w);
  if (hipGetLastError() != hipSuccess) return -1;
  switch (bits) {
    case 4: return moe_launch_bits<4>(aa, w, st);
    case 5: return moe_launch_bits<5>(aa, w, st);
    case 6: return moe_launch_bits<6>(aa, w, st);
    case 8: return moe_launch_bits<8>(aa, w, st);
  }
  return 0;
}

}  // namespace lh
