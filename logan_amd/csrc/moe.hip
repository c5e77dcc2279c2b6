// Router top-k and the routed-MoE block (device-native, bf16 activations).
//
// Semantics follow logan-qwen/src/lib.rs:535-593 and
// logan-qwen4/src/lib.rs:7993-8043, :8692-8711, :8759-8815, :7597-7759:
//   probs = softmax(logits); top-k with lower-index ties; weight_r =
//   val_r / sum_{r<k} val_r; h = silu(gate.x) * (up.x); y_r = down.h;
//   out = sum_r (y_r * weight_r) in rank order + sy * sigmoid(se_g.x).
//
// Selection is done on the logits with the key (logit desc, index asc).
// softmax is non-decreasing in the logit, so this order is the reference's
// selection on probabilities unless two different logits round to the same
// probability; route_dev.hpp checks for that and then recomputes the
// reference's probabilities (route_exact). Weights are
// exp(l_r - l_0) / sum_{r<k} exp(l_j - l_0), which equals val_r / wsum up to
// rounding (exactly the reference's val_r / wsum on the recomputed path).
//
// Launch structure (all on one stream):
//   1. moe_route_tok_kernel     one block per token: top-k, shared-expert
//                               gate, x as bf16 pairs
//      moe_group_kernel         one block: group the (token, rank) slots by
//                               expert and cut each expert's rows into
//                               sub-groups of at most kSubTok: one record per
//                               sub-group (expert, first row, rows, tokens)
//                               and a grouped row per slot
//   2. moe_gateup_kernel        per (sub-group, 16 rows): gate and up rows
//                               loaded once, applied to every token of the
//                               sub-group, SwiGLU fused -> h[grouped row][j]
//   3. moe_down_kernel          per (sub-group, 32 rows): down rows loaded
//                               once, applied to h of every row of the
//                               sub-group -> y[grouped row][d] (f32)
//   4. moe_combine_kernel       out[t][d] = sum_r w_r y[row(t,r)][d] (rank
//                               order) + gs_t * y[shared row t][d] -> bf16
// A sub-group's record carries what its blocks need first, so each block
// starts its weight and activation loads after one dependent load. The
// shared expert's blocks (kSubTok tokens each) come first in launches 2 and
// 3: at the end of the grid they ran alone for the last third of each launch.
#include <cstdlib>

#include "affine_dev.hpp"
#include "lh_internal.hpp"
#include "route_dev.hpp"

namespace lh {

// sticky: bit 3 = a routed expert missing from the expert-cache map
static __device__ uint32_t g_moe_map_err;

constexpr int kMaxE = 1024;  // 16 keys per lane
constexpr int kMaxK = 32;

// One wave: top-k of one token's logits; lane r < k ends with rank r's
// expert and weight (route_dev.hpp: wave_topk_lanes).
__device__ __forceinline__ void wave_topk(const void *logits, int f32, size_t row_off, int E,
                                          int k, int &idx, float &w) {
  if (f32) {
    if (E <= 512) wave_topk_lanes<8, true>(logits, row_off, E, k, idx, w);
    else wave_topk_lanes<16, true>(logits, row_off, E, k, idx, w);
  } else {
    if (E <= 512) wave_topk_lanes<8, false>(logits, row_off, E, k, idx, w);
    else wave_topk_lanes<16, false>(logits, row_off, E, k, idx, w);
  }
}

__global__ __launch_bounds__(256) void route_topk_kernel(const void *logits, int f32, int B, int E,
                                                         int k, int32_t *idx, float *w) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= B) return;  // whole waves leave together
  int id;
  float wt;
  wave_topk(logits, f32, (size_t)t * E, E, k, id, wt);
  if (lane < k) {
    idx[(size_t)t * k + lane] = id;
    w[(size_t)t * k + lane] = wt;
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

// Grouped order: the B*k routed (token, rank) slots sorted by expert (one
// group per distinct expert), then the B shared-expert slots. h and y rows
// are stored in grouped order, so a group's rows are contiguous.
constexpr int kRecInts = 8;  // sub-group record: expert, first grouped row, rows, tokens[0..3], 0
// Each expert's tokens are cut into sub-groups of at most kSubTok, so that no
// block of the gate/up and down launches carries many more tokens than the
// others; the shared expert's sub-groups (all B tokens, in order) need no
// record and go first in both launches.
constexpr int kSubTok = 4;
__host__ __device__ inline int max_subgroups(int B, int k, int E) {
  const int nslots = B * k;
  return (nslots < E ? nslots : E) + (nslots + kSubTok - 1) / kSubTok;
}
struct MoeWs {
  int *n_groups;      // [1]  routed sub-groups
  int *rec;           // [max_subgroups][kRecInts]
  int *gpos;          // [B*k] grouped row of slot t*k + r
  int32_t *topk_idx;  // [B*k]
  float *topk_w;      // [B*k]
  float *gs;          // [B]
  uint32_t *xp;       // [B][C][16] x of every token as pre-scaled bf16 pairs
  float *xps;         // [B][C][2]  per chunk: sum x, sum of the paired values
  float *h;           // [(B*k+B) * hmax]
  float *y;           // [(B*k+B) * D]
  size_t total;
};

static inline size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

static MoeWs moe_ws_layout(void *base, int B, int D, int inter, int sinter, int E, int k) {
  MoeWs w{};
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
  w.rec = reinterpret_cast<int *>(take(sizeof(int) * (size_t)max_subgroups(B, k, E) * kRecInts));
  w.gpos = reinterpret_cast<int *>(take(sizeof(int) * (size_t)B * k));
  w.topk_idx = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * (size_t)B * k));
  w.topk_w = reinterpret_cast<float *>(take(sizeof(float) * (size_t)B * k));
  w.gs = reinterpret_cast<float *>(take(sizeof(float) * (size_t)B));
  w.xp = reinterpret_cast<uint32_t *>(take(sizeof(uint32_t) * (size_t)B * (D / 32) * 16));
  w.xps = reinterpret_cast<float *>(take(sizeof(float) * (size_t)B * (D / 32) * 2));
  w.h = reinterpret_cast<float *>(take(sizeof(float) * slots * hmax));
  w.y = reinterpret_cast<float *>(take(sizeof(float) * slots * (size_t)D));
  w.total = off;
  return w;
}

constexpr int kMaxB = 64;  // tokens per launch of the dot2 path (larger batches go in chunks)

// The single-launch B = 1 path's tagged h pairs own the first bytes of the
// workspace; the per-token and MFMA paths lay out their buffers after them,
// so no other path ever writes where a tag is checked.
static size_t fused_region_bytes(int inter, int sinter, int k) {
  return al256(moe_fused_workspace_bytes(k + 1, inter, sinter));
}

size_t moe_workspace_bytes(int B, int D, int inter, int sinter, int E, int k) {
  const size_t general = moe_ws_layout(nullptr, B < kMaxB ? B : kMaxB, D, inter, sinter, E, k).total;
  const size_t mfma = moe_mfma_workspace_bytes(B, D, inter, sinter, E, k);
  return fused_region_bytes(inter, sinter, k) + (general > mfma ? general : mfma);
}

// > 0: one threshold for every code width; 0: the per-width defaults;
// -1: the environment not read yet
static int g_mfma_min_b = -1;

void set_moe_mfma_min_batch(int b) { g_mfma_min_b = b > 0 ? b : 0; }

static int mfma_min_batch(int bits) {
  if (g_mfma_min_b < 0) {
    const char *v = getenv("LOGAN_HIP_MOE_MFMA_MIN_B");
    const int e = v ? atoi(v) : 0;
    g_mfma_min_b = e > 0 ? e : 0;
  }
  if (g_mfma_min_b > 0) return g_mfma_min_b;
  return bits == 4 ? kMfmaMinBatch4Bit : kMfmaMinBatchDefault;
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
// 1. route + shared gate (one block per token), then grouping (one block)

// x of token t as the gate/up kernels' operand: xp[t][c] = make_xchunk_bf16
// of chunk c (pairs, sum x, sum x'), one chunk per lane and step
template <int BITS>
__device__ __forceinline__ void convert_x_token(const MoeArgs &a, const MoeWs &w, int t, int lane) {
  const int C = a.D >> 5;
  for (int c = lane; c < C; c += 64) {
    const uint4 *src = reinterpret_cast<const uint4 *>(a.x + (size_t)t * a.D + 32 * c);
    uint4 xq[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) xq[v] = src[v];
    uint32_t xb[32];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint4 q = xq[v];
      xb[8 * v + 0] = q.x & 0xffffu; xb[8 * v + 1] = q.x >> 16;
      xb[8 * v + 2] = q.y & 0xffffu; xb[8 * v + 3] = q.y >> 16;
      xb[8 * v + 4] = q.z & 0xffffu; xb[8 * v + 5] = q.z >> 16;
      xb[8 * v + 6] = q.w & 0xffffu; xb[8 * v + 7] = q.w >> 16;
    }
    XChunk xc;
    make_xchunk_bf16<BITS>(xc, xb);
    const size_t it = (size_t)t * C + c;
    uint4 *dst = reinterpret_cast<uint4 *>(w.xp + it * 16);
#pragma unroll
    for (int v = 0; v < 4; ++v)
      dst[v] = make_uint4(xc.p[4 * v], xc.p[4 * v + 1], xc.p[4 * v + 2], xc.p[4 * v + 3]);
    w.xps[it * 2] = xc.xs;
    w.xps[it * 2 + 1] = xc.xsp;
  }
}

// One block of two waves per token t = blockIdx.x: wave 0 selects the top-k
// (route_dev.hpp: wave_topk_lanes), wave 1 computes the shared-expert gate
// sigmoid(se_g . x_t) (logan-qwen4/src/lib.rs:7602-7604) and writes x_t in
// the operand form. The tokens' selections run on as many CUs as there are
// tokens (one CU holding all of them spent 0.8 us of VALU per token).
template <int KPL, bool F32, int BITS>
__global__ __launch_bounds__(128) void moe_route_tok_kernel(MoeArgs a, MoeWs w) {
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63;
  if (threadIdx.x < 64) {
    int id;
    float wt;
    wave_topk_lanes<KPL, F32>(a.logits, (size_t)t * a.E, a.E, a.k, id, wt);
    if (lane < a.k) {
      w.topk_idx[t * a.k + lane] = id;
      w.topk_w[t * a.k + lane] = wt;
      if (a.idx_out) a.idx_out[t * a.k + lane] = id;
      if (a.w_out) a.w_out[t * a.k + lane] = wt;
    }
    return;
  }
  if (a.sgate.m.w) {
    float g = 1.0f;
    if (a.se_gate_vec) {
      // 16-byte loads, all in flight (8 bf16 per lane per step)
      const int n8 = a.D >> 3;
      g = 0.f;
      for (int c0 = 0; c0 < n8; c0 += 256) {
        uint4 gq[4], xq[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int c = min(c0 + v * 64 + lane, n8 - 1);
          gq[v] = reinterpret_cast<const uint4 *>(a.se_gate_vec)[c];
          xq[v] = reinterpret_cast<const uint4 *>(a.x + (size_t)t * a.D)[c];
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          if (c0 + v * 64 + lane < n8) {
            g = dot2(gq[v].x, xq[v].x, g);
            g = dot2(gq[v].y, xq[v].y, g);
            g = dot2(gq[v].z, xq[v].z, g);
            g = dot2(gq[v].w, xq[v].w, g);
          }
        }
      }
      g = team_sum<64>(g);
      g = 1.0f / (1.0f + __expf(-g));
    }
    if (lane == 0) w.gs[t] = g;
  }
  convert_x_token<BITS>(a, w, t, lane);
}

constexpr int kGroupThreads = 1024;

// One block: group the (token, rank) slots by expert and cut each expert's
// rows into sub-groups of at most kSubTok: one record per sub-group and a
// grouped row per slot.
__global__ __launch_bounds__(kGroupThreads) void moe_group_kernel(MoeArgs a, MoeWs w) {
  __shared__ int s_idx[kMaxB * kMaxK];
  __shared__ int s_cnt[kMaxE];
  __shared__ int s_start[kMaxE];
  __shared__ int s_gid[kMaxE];
  __shared__ int s_fill[kMaxE];
  __shared__ int s_tok[kMaxB * kMaxK];
  __shared__ int s_gex[kMaxB * kMaxK];
  __shared__ int s_wave_tot[kGroupThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nslots = a.B * a.k;
  for (int i = tid; i < nslots; i += kGroupThreads) s_idx[i] = w.topk_idx[i];
  for (int e = tid; e < a.E; e += kGroupThreads) s_cnt[e] = 0;
  __syncthreads();
  for (int i = tid; i < nslots; i += kGroupThreads) atomicAdd(&s_cnt[s_idx[i]], 1);
  __syncthreads();
  // exclusive scans over experts: first grouped row and first sub-group
  // (E <= 1024 = one per thread)
  {
    const int e = tid;
    const int c = e < a.E ? s_cnt[e] : 0;
    const int f = (c + kSubTok - 1) / kSubTok;
    // pack (count, sub-groups) into one int: count sum <= 2048 < 2^15, sub-group sum < 2^16
    int v = (c << 16) | f;
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
      s_start[e] = excl >> 16;
      s_gid[e] = excl & 0xffff;
    }
    if (tid == kGroupThreads - 1) {
      const int tot = prefix + incl;
      *w.n_groups = tot & 0xffff;
    }
  }
  // placement within a group in arrival order: every row's arithmetic is
  // independent of its position, so the results do not depend on it
  for (int e = tid; e < a.E; e += kGroupThreads) s_fill[e] = 0;
  __syncthreads();
  for (int i = tid; i < nslots; i += kGroupThreads) {
    const int e = s_idx[i];
    const int gp = s_start[e] + atomicAdd(&s_fill[e], 1);
    s_tok[gp] = i / a.k;
    s_gex[gp] = e;
    w.gpos[i] = gp;
  }
  __syncthreads();
  // one record per sub-group: the kSubTok grouped rows from each multiple of
  // kSubTok within an expert's rows
  for (int gp = tid; gp < nslots; gp += kGroupThreads) {
    const int e = s_gex[gp];
    const int rel = gp - s_start[e];
    if (rel % kSubTok == 0) {
      const int c = min(s_cnt[e] - rel, kSubTok);
      int4 *r = reinterpret_cast<int4 *>(w.rec + (size_t)(s_gid[e] + rel / kSubTok) * kRecInts);
      r[0] = make_int4(e, gp, c, s_tok[gp]);
      r[1] = make_int4(c > 1 ? s_tok[gp + 1] : 0, c > 2 ? s_tok[gp + 2] : 0,
                       c > 3 ? s_tok[gp + 3] : 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// 2. gate/up + SwiGLU

// One block: RPB = 16 rows of gate and of up (4 per wave, a wave spans the
// whole row: CPL chunks per lane) of one expert group, applied to every token
// of the group. Loads are issued together, branch-free; x comes pre-paired.
template <int BITS, int CPL>
__global__ __launch_bounds__(256, 3) void moe_gateup_kernel(MoeArgs a, MoeWs w, int ipg, int ipg_s) {
  constexpr int U = 4;
  constexpr int RPB = 4 * U;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int C = a.D >> 5;
  UnpackConsts kc;
  kc.init();
  // the shared expert's sub-groups first, then the routed ones
  const int nsh = a.sgate.m.w ? (a.B + kSubTok - 1) / kSubTok : 0;
  const int item = blockIdx.x;
  const bool shared = item < nsh * ipg_s;
  const int g = shared ? item / ipg_s : (item - nsh * ipg_s) / ipg;
  const int rb = shared ? item % ipg_s : (item - nsh * ipg_s) % ipg;
  // one load round for a routed sub-group: its record carries its tokens
  const int ng = *w.n_groups;
  const int4 rr0 = reinterpret_cast<const int4 *>(w.rec + (size_t)(shared ? 0 : g) * kRecInts)[0];
  const int4 rr1 = reinterpret_cast<const int4 *>(w.rec + (size_t)(shared ? 0 : g) * kRecInts)[1];
  if (!shared && g >= ng) return;
  const int s0 = g * kSubTok;
  const int4 rc0 = shared ? make_int4(0, a.B * a.k + s0, min(kSubTok, a.B - s0), s0) : rr0;
  const int4 rc1 = shared ? make_int4(s0 + 1, s0 + 2, s0 + 3, 0) : rr1;
  const int ge = rc0.x;
  const int off = __builtin_amdgcn_readfirstlane(rc0.y);
  const int cnt = __builtin_amdgcn_readfirstlane(rc0.z);
  const DevMat gm = shared ? a.sgate.m : a.gate.m;
  const DevMat um = shared ? a.sup.m : a.up.m;
  const long long gws = shared ? a.sgate.w_stride : a.gate.w_stride;
  const long long uws = shared ? a.sup.w_stride : a.up.w_stride;
  const long long gps = shared ? a.sgate.p_stride : a.gate.p_stride;
  const long long ups = shared ? a.sup.p_stride : a.up.p_stride;
  int e = __builtin_amdgcn_readfirstlane(ge);
  if (!shared && a.nmap) {  // the expert's block in an expert cache's arena
    bool miss = false;
    e = moe_bank_index<true>(a, e, miss);
    if (miss && threadIdx.x == 0) atomicOr(&g_moe_map_err, 8u);
  }
  const int rows = shared ? a.sinter : a.inter;
  const uint8_t *gwb = gm.w + (size_t)e * gws;
  const uint8_t *uwb = um.w + (size_t)e * uws;
  const uint16_t *gsc = gm.sc + (size_t)e * gps;
  const uint16_t *gbi = gm.bi + (size_t)e * gps;
  const uint16_t *usc = um.sc + (size_t)e * ups;
  const uint16_t *ubi = um.bi + (size_t)e * ups;
  const int j0 = rb * RPB + wave * U;
  const int gshift = __builtin_ctz(gm.gs >> 5);

  uint32_t wg[U][CPL][BITS], wu[U][CPL][BITS];
  uint32_t rsg[U][CPL], rbg[U][CPL], rsu[U][CPL], rbu[U][CPL];
  // loads in the order they are needed (they complete in issue order): token
  // 0's x pairs, the scale/bias words, then the rows' codes
  uint32_t xpn[CPL][16];
  float2 xsn[CPL];
  auto load_x = [&](int t) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const size_t xo = (size_t)t * C + min(lane + 64 * i, C - 1);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint4 q = reinterpret_cast<const uint4 *>(w.xp + xo * 16)[v];
        xpn[i][4 * v] = q.x; xpn[i][4 * v + 1] = q.y; xpn[i][4 * v + 2] = q.z; xpn[i][4 * v + 3] = q.w;
      }
      xsn[i] = reinterpret_cast<const float2 *>(w.xps)[xo];
    }
  };
  load_x(__builtin_amdgcn_readfirstlane(rc0.w));
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int j = min(j0 + u, rows - 1), c = min(lane + 64 * i, C - 1);
      const size_t p = (size_t)j * gm.ng + (c >> gshift);
      rsg[u][i] = ld_stream<uint16_t, true>(gsc + p);
      rbg[u][i] = ld_stream<uint16_t, true>(gbi + p);
      rsu[u][i] = ld_stream<uint16_t, true>(usc + p);
      rbu[u][i] = ld_stream<uint16_t, true>(ubi + p);
    }
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int j = min(j0 + u, rows - 1), c = min(lane + 64 * i, C - 1);
      load_chunk<BITS, true>(wg[u][i], gwb + (size_t)j * gm.row_bytes + (size_t)c * (4 * BITS));
      load_chunk<BITS, true>(wu[u][i], uwb + (size_t)j * um.row_bytes + (size_t)c * (4 * BITS));
    }
  __builtin_amdgcn_sched_barrier(0);
  // the packed rows stay in registers; each token unpacks them again (groups
  // hold one or two tokens in the common case)
  float sg[U][CPL], bg[U][CPL], su[U][CPL], bu[U][CPL];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const bool live = j0 + u < rows && lane + 64 * i < C;
      sg[u][i] = live ? aux_to_f32_sel(rsg[u][i], gm.fp16) : 0.f;
      bg[u][i] = live ? aux_to_f32_sel(rbg[u][i], gm.fp16) : 0.f;
      su[u][i] = live ? aux_to_f32_sel(rsu[u][i], um.fp16) : 0.f;
      bu[u][i] = live ? aux_to_f32_sel(rbu[u][i], um.fp16) : 0.f;
    }
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  for (int i_t = 0; i_t < cnt; ++i_t) {
    // keep the unpack inside the loop (not hoisted into 128 live registers);
    // not before the first token, whose rows start as their own loads land
    if (i_t > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < CPL; ++i)
#pragma unroll
          for (int q = 0; q < BITS; ++q) asm volatile("" : "+v"(wg[u][i][q]), "+v"(wu[u][i][q]));
    }
    if (i_t > 0) load_x(__builtin_amdgcn_readfirstlane(i_t == 1 ? rc1.x : i_t == 2 ? rc1.y : rc1.z));
    float pg[U], pu[U];
#pragma unroll
    for (int u = 0; u < U; ++u) pg[u] = pu[u] = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        uint32_t q[16];
        unpack_chunk<BITS>(q, wg[u][i], kc);
        pg[u] += chunk_fold<BITS>(pairs_dot(q, xpn[i]), sg[u][i], bg[u][i], xsn[i].x, xsn[i].y);
        unpack_chunk<BITS>(q, wu[u][i], kc);
        pu[u] += chunk_fold<BITS>(pairs_dot(q, xpn[i]), su[u][i], bu[u][i], xsn[i].x, xsn[i].y);
      }
    }
    // lane row r (lane / 16) gets row j0 + r: h = silu(gate) * up
    // (logan-qwen4/src/lib.rs:8807-8809)
    const float gv = wave_reduce4(pg[0], pg[1], pg[2], pg[3]);
    const float uv = wave_reduce4(pu[0], pu[1], pu[2], pu[3]);
    const int r = lane >> 4;
    if ((lane & 15) == 0 && j0 + r < rows) w.h[(size_t)(off + i_t) * hmax + j0 + r] = silu(gv) * uv;
  }
}

// ---------------------------------------------------------------------------
// 3. down projection of h for every slot of a group

// output rows per down block: 64 for 4-bit codes with one chunk per lane
// (16 KB of codes per block; 64 rows took 28.6 us against 33.5 us at 32 rows
// and 49.1 us at 16 for config 3, B = 16), 32 otherwise (the 5/6/8-bit code
// extraction of 64 rows needs over 200 registers)
__host__ __device__ constexpr int down_rows(int bits, int lanes) { return bits == 4 && lanes == 16 ? 64 : 32; }

// One block: down_rows output rows d of one expert group's down projection (a row
// per LANES lanes, PASSES rows per lane), applied to h of every slot of the
// group with f32 FMAs: y = scale * sum code*h + bias * sum h.
template <int BITS, int LANES>
__global__ __launch_bounds__(256) void moe_down_kernel(MoeArgs a, MoeWs w, int ipg) {
  constexpr int kHq = LANES / 8;     // float4 of one h row per thread (K <= 32 * LANES)
  constexpr int RPP = 256 / LANES;  // rows per pass of the block
  constexpr int PASSES = down_rows(BITS, LANES) / RPP;
  const int lb = threadIdx.x % LANES;
  const int rsub = threadIdx.x / LANES;
  // the shared expert's sub-groups first, then the routed ones
  const int nsh = a.sdown.m.w ? (a.B + kSubTok - 1) / kSubTok : 0;
  const int item = blockIdx.x;
  const bool shared = item < nsh * ipg;
  const int g = item / ipg - (shared ? 0 : nsh);
  const int rb = item % ipg;
  const int ng = *w.n_groups;
  const int4 rr0 = reinterpret_cast<const int4 *>(w.rec + (size_t)(shared ? 0 : g) * kRecInts)[0];
  if (!shared && g >= ng) return;
  const int rows0 = a.B * a.k + g * kSubTok;
  const int4 rc0 = shared ? make_int4(0, rows0, min(kSubTok, a.B - g * kSubTok), 0) : rr0;
  const int ge = rc0.x;
  const int off = __builtin_amdgcn_readfirstlane(rc0.y);
  const int cnt = __builtin_amdgcn_readfirstlane(rc0.z);
  const DevMat dm = shared ? a.sdown.m : a.down.m;
  const long long dws = shared ? a.sdown.w_stride : a.down.w_stride;
  const long long dps = shared ? a.sdown.p_stride : a.down.p_stride;
  int e = __builtin_amdgcn_readfirstlane(ge);
  if (!shared && a.nmap) {
    bool miss = false;  // (reported by the gate/up blocks)
    e = moe_bank_index<true>(a, e, miss);
  }
  const int K = shared ? a.sinter : a.inter;  // columns of down
  const int Ck = K >> 5;
  const uint8_t *wb = dm.w + (size_t)e * dws;
  const uint16_t *scb = dm.sc + (size_t)e * dps;
  const uint16_t *bib = dm.bi + (size_t)e * dps;
  const int d0 = rb * down_rows(BITS, LANES);
  const int cl = min(lb, Ck - 1);
  const int gi = cl / (dm.gs >> 5);

  uint32_t wv[PASSES][BITS];
  uint32_t rs[PASSES], rbi[PASSES];
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  // loads in the order they are needed (they complete in issue order): the
  // sub-group's first h row (K floats, 2 per thread for K <= 512), the
  // scale/bias words, then the rows' codes
  auto load_h = [&](int row, float4 (&hq)[kHq]) {
#pragma unroll
    for (int v = 0; v < kHq; ++v) {
      const int o = threadIdx.x + 256 * v;
      hq[v] = o < 8 * Ck ? reinterpret_cast<const float4 *>(w.h + (size_t)row * hmax)[o]
                         : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  float4 hq[kHq];
  load_h(off, hq);
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int d = min(d0 + p * RPP + rsub, a.D - 1);
    rs[p] = ld_stream<uint16_t, true>(scb + (size_t)d * dm.ng + gi);
    rbi[p] = ld_stream<uint16_t, true>(bib + (size_t)d * dm.ng + gi);
  }
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int d = min(d0 + p * RPP + rsub, a.D - 1);
    load_chunk<BITS, true>(wv[p], wb + (size_t)d * dm.row_bytes + (size_t)cl * (4 * BITS));
  }
  __builtin_amdgcn_sched_barrier(0);
  float sc[PASSES], bi[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const bool live = d0 + p * RPP + rsub < a.D && lb < Ck;
    sc[p] = live ? aux_to_f32_sel(rs[p], dm.fp16) : 0.f;
    bi[p] = live ? aux_to_f32_sel(rbi[p], dm.fp16) : 0.f;
  }
  __shared__ __align__(16) float s_h[32 * LANES];
  for (int i_t = 0; i_t < cnt; ++i_t) {
    // h of the row through LDS once per block (each of the RPP row groups
    // needs all of it); float4 v of chunk c sits at 8c + ((v + c) & 7), so
    // that the LANES lanes of a row, reading 128 bytes apart, spread over
    // the banks (down 29.5 -> 26.7 us for config 3, B = 16)
    if (i_t > 0) load_h(off + i_t, hq);
#pragma unroll
    for (int v = 0; v < kHq; ++v) {
      const int o = threadIdx.x + 256 * v;
      if (o < 8 * Ck) reinterpret_cast<float4 *>(s_h)[(o & ~7) | ((o + (o >> 3)) & 7)] = hq[v];
    }
    __syncthreads();
    float xf[32];
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float4 t = reinterpret_cast<const float4 *>(s_h)[8 * cl + ((v + cl) & 7)];
      xf[4 * v + 0] = t.x; xf[4 * v + 1] = t.y; xf[4 * v + 2] = t.z; xf[4 * v + 3] = t.w;
    }
    __syncthreads();
    float xt[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) xt[v] = xf[v] + xf[v + 16];
#pragma unroll
    for (int q = 8; q > 0; q >>= 1)
#pragma unroll
      for (int v = 0; v < q; ++v) xt[v] += xt[v + q];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      float v = fmaf(sc[p], codes_dot<BITS>(wv[p], xf), bi[p] * xt[0]);
      v = team_sum<LANES>(v);
      const int d = d0 + p * RPP + rsub;
      if (lb == 0 && d < a.D) w.y[(size_t)(off + i_t) * a.D + d] = v;
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
    // the shared expert's row and gate do not depend on the routes: in flight
    // with the first round (shared rows follow the routed ones)
    float ysh = 0.f, gs = 0.f;
    if (a.sdown.m.w) {
      ysh = w.y[(size_t)(a.B * a.k + t) * a.D + d];
      gs = w.gs[t];
    }
    // sixteen ranks' rows and weights, then their outputs, in flight at a
    // time, added in rank order
    for (int r0 = 0; r0 < a.k; r0 += 16) {
      int gp[16];
      float wt[16], yv[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        gp[j] = 0;
        wt[j] = 0.f;
        if (r0 + j < a.k) {
          gp[j] = w.gpos[t * a.k + r0 + j];
          wt[j] = w.topk_w[t * a.k + r0 + j];
        }
      }
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (r0 + j < a.k) yv[j] = w.y[(size_t)gp[j] * a.D + d];
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (r0 + j < a.k) acc = fmaf(yv[j], wt[j], acc);
    }
    float o = acc;
    if (a.sdown.m.w) o = fmaf(ysh, gs, acc);
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
  const int msub = max_subgroups(a.B, a.k, a.E);
  const int nsh = a.sgate.m.w ? (a.B + kSubTok - 1) / kSubTok : 0;
  // gate/up: 16 rows per block, the shared expert's sub-groups and every
  // possible routed sub-group (blocks of sub-groups that did not form leave
  // at once)
  {
    const int ipg = (a.inter + 15) / 16;
    const int ipg_s = a.sgate.m.w ? (a.sinter + 15) / 16 : 0;
    const int grid = nsh * ipg_s + msub * ipg;
    if (Cd <= 64)
      hipLaunchKernelGGL((moe_gateup_kernel<BITS, 1>), dim3(grid), dim3(256), 0, st, a, w, ipg, ipg_s);
    else if (Cd <= 128)
      hipLaunchKernelGGL((moe_gateup_kernel<BITS, 2>), dim3(grid), dim3(256), 0, st, a, w, ipg, ipg_s);
    else
      return 0;
    if (hipGetLastError() != hipSuccess) return -1;
  }
  // down: down_rows(BITS, LANES) rows per block
  {
    const int kmax = a.inter > a.sinter ? a.inter : a.sinter;
    const int Ci = kmax >> 5;
    if (Ci > 32) return -1;
    const int rows = Ci <= 16 ? down_rows(BITS, 16) : down_rows(BITS, 32);
    const int ipg = (a.D + rows - 1) / rows;
    const int grid = (nsh + msub) * ipg;
    if (Ci <= 16) hipLaunchKernelGGL((moe_down_kernel<BITS, 16>), dim3(grid), dim3(256), 0, st, a, w, ipg);
    else hipLaunchKernelGGL((moe_down_kernel<BITS, 32>), dim3(grid), dim3(256), 0, st, a, w, ipg);
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

uint32_t moe_map_errors() {
  uint32_t v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_moe_map_err), sizeof(v), 0, hipMemcpyDeviceToHost) !=
      hipSuccess)
    return 0xffffffffu;
  return v;
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

template <int BITS>
static void launch_route_tok_bits(const MoeArgs &a, const MoeWs &w, hipStream_t st) {
  const dim3 g(a.B), b(128);
  if (a.logits_f32) {
    if (a.E <= 512) hipLaunchKernelGGL((moe_route_tok_kernel<8, true, BITS>), g, b, 0, st, a, w);
    else hipLaunchKernelGGL((moe_route_tok_kernel<16, true, BITS>), g, b, 0, st, a, w);
  } else {
    if (a.E <= 512) hipLaunchKernelGGL((moe_route_tok_kernel<8, false, BITS>), g, b, 0, st, a, w);
    else hipLaunchKernelGGL((moe_route_tok_kernel<16, false, BITS>), g, b, 0, st, a, w);
  }
}

static int launch_route_tok(const MoeArgs &a, const MoeWs &w, int bits, hipStream_t st) {
  switch (bits) {
    case 4: launch_route_tok_bits<4>(a, w, st); break;
    case 5: launch_route_tok_bits<5>(a, w, st); break;
    case 6: launch_route_tok_bits<6>(a, w, st); break;
    default: launch_route_tok_bits<8>(a, w, st); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_moe_block(const MoeArgs &a, hipStream_t st) {
  if (a.B <= 0 || a.B > kMaxBatch || a.E <= 0 || a.E > kMaxE || a.k <= 0 || a.k > kMaxK || a.k > a.E)
    return 0;
  if ((long long)a.B * a.k > kMaxBatchSlots) return 0;
  if (a.D <= 0 || a.D % 32 != 0 || a.inter <= 0 || a.inter % 32 != 0) return 0;
  if (a.D > 4096 || a.inter > 1024 || a.sinter > 1024) return 0;  // kernel shapes below
  if (!a.x || !a.logits || !a.out || !a.ws) return 0;
  if ((reinterpret_cast<uintptr_t>(a.x) & 15) != 0) return 0;
  const int bits = a.gate.m.bits, gs = a.gate.m.gs;
  if (!(bits == 4 || bits == 5 || bits == 6 || bits == 8)) return 0;
  if (!bank_ok(a.gate, a.inter, a.D, bits, gs) || !bank_ok(a.up, a.inter, a.D, bits, gs)) return 0;
  if (!bank_ok(a.down, a.D, a.inter, bits, a.down.m.gs)) return 0;
  if (a.nmap < 0 || a.nmap > kMoeMapMax) return 0;
  if (a.nmap == 0 && (a.gate.E < a.E || a.up.E < a.E || a.down.E < a.E)) return 0;
  for (int i = 0; i < a.nmap; ++i)  // cache blocks: inside every bank view
    if (a.map_b[i] < 0 || a.map_b[i] >= a.gate.E || a.map_b[i] >= a.up.E || a.map_b[i] >= a.down.E)
      return 0;
  // a map covers the experts of one token's route: B = 1, on the fused or
  // per-token path (the token-batch MFMA path never takes B = 1)
  if (a.nmap > 0 && a.B != 1) return 0;
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
  const size_t fz = fused_region_bytes(a.inter, sinter, a.k);
  if (fused_enabled()) {
    MoeArgs af = aa;
    af.ws_bytes = fz;
    const int rc = launch_moe_fused_b1(af, st);
    if (rc != 0) return rc;
  }
  aa.ws = reinterpret_cast<char *>(a.ws) + fz;
  aa.ws_bytes = a.ws_bytes - fz;
  if (a.B >= mfma_min_batch(bits)) {
    const int rc = launch_moe_mfma(aa, st);
    if (rc != 0) return rc;
  }
  // dot2 path, at most kMaxB tokens per pass (the passes reuse the workspace
  // in stream order)
  for (int b0 = 0; b0 < a.B; b0 += kMaxB) {
    MoeArgs c = aa;
    c.B = a.B - b0 < kMaxB ? a.B - b0 : kMaxB;
    c.x = a.x + (size_t)b0 * a.D;
    c.logits = reinterpret_cast<const char *>(a.logits) + (size_t)b0 * a.E * (a.logits_f32 ? 4 : 2);
    c.out = reinterpret_cast<char *>(a.out) + (size_t)b0 * a.D * (a.out_f32 ? 4 : 2);
    if (a.idx_out) c.idx_out = a.idx_out + (size_t)b0 * a.k;
    if (a.w_out) c.w_out = a.w_out + (size_t)b0 * a.k;
    MoeWs w = moe_ws_layout(aa.ws, c.B, a.D, a.inter, sinter, a.E, a.k);
    if (launch_route_tok(c, w, bits, st) != 0) return -1;
    hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(kGroupThreads), 0, st, c, w);
    if (hipGetLastError() != hipSuccess) return -1;
    int rc = 0;
    switch (bits) {
      case 4: rc = moe_launch_bits<4>(c, w, st); break;
      case 5: rc = moe_launch_bits<5>(c, w, st); break;
      case 6: rc = moe_launch_bits<6>(c, w, st); break;
      case 8: rc = moe_launch_bits<8>(c, w, st); break;
    }
    if (rc != 1) return rc;
  }
  return 1;
}

}  // namespace lh
