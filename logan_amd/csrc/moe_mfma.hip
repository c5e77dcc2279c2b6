// Routed-MoE block for token batches on MFMA (prefill chunks, large decode
// batches): the same semantics as moe.hip (logan-qwen/src/lib.rs:535-593,
// logan-qwen4/src/lib.rs:8692-8711, :8759-8815, :7597-7759), with the
// per-expert products on v_mfma_f32_16x16x32_bf16 so that an expert's
// weights are read once for up to 16 of its tokens at a time.
//
// Launches (one stream):
//   1. moe_mroute_kernel       one wave per token: top-k (lower-index ties),
//                              normalised weights, shared-expert gate
//   2. moe_mgroup_kernel       one block: group the (token, rank) slots by
//                              expert and cut each group into tiles of at most
//                              16 slots; the shared expert gets tiles of 16
//                              tokens ahead of the routed ones
//   3. moe_gateup_mfma_kernel  per (tile, 64 rows): the tile's x rows staged
//                              in LDS, gate and up rows of 16 per wave, SwiGLU
//                              fused; h stored as two bf16 planes (hi, lo with
//                              h = hi + lo to 2^-17) in grouped row order
//      moe_gateup_lds_kernel   above 128 tokens (4/8-bit, groups of 64): the
//                              weights streamed through a per-wave LDS ring,
//                              whole-tile blocks and then 128-row ones
//   4. moe_down_mfma_kernel    per (tile, 128 rows): h hi/lo staged in LDS,
//                              two MFMA passes (hi, lo), y in grouped order
//      moe_down_lds_kernel     above 128 tokens: the LDS ring again,
//                              whole-tile blocks and then 512-row ones
//   5. moe_mcombine_kernel     out[t] = sum_r w_r y[row(t, r)] (rank order)
//                              + gs_t y[shared row t]
// Numerics: codes exact, activations exact (x bf16; h to 2^-17), f32
// accumulation, per-group scale/bias folded after each 64-code step (the
// group sizes are multiples of 64).
#include "lh_internal.hpp"
#include "mfma_dev.hpp"
#include "route_dev.hpp"

namespace lh {

constexpr int kMTok = 16;          // slots per tile
#ifndef MOE_CHUNK
#define MOE_CHUNK 2048
#endif
constexpr int kMChunk = MOE_CHUNK;  // x codes staged in LDS at a time (gate/up)
constexpr int kMDownK = 512;       // largest down K (expert intermediate size)
constexpr int kMMaxSlots = 65536;  // B * k
constexpr int kMMaxE = 1024;
constexpr int kMGroupThreads = 1024;
constexpr int kMGroupKeep = 8;     // routed slots per grouping thread held in registers

struct MoeMWs {
  int *n_tiles;       // [1]
  int4 *tiles;        // [max_tiles] (expert or -1 for shared, first grouped row, slots, 0)
  int *tok;           // [B*k] token of each grouped routed row
  int *gpos;          // [B*k] grouped row of slot t*k + r
  int32_t *topk_idx;  // [B*k]
  float *topk_w;      // [B*k]
  float *gs;          // [B]
  uint16_t *xop;      // [B * D] x in the 4-bit operand order (a_nibble_order per 8)
  uint16_t *h_hi;     // [(B*k + B) * hmax] bf16, stored in the operand order
  uint16_t *h_lo;     // [(B*k + B) * hmax] bf16
  float *y;           // [(B*k + B) * D]
  int max_tiles;
  size_t total;
};

static inline size_t al256m(size_t v) { return (v + 255) & ~(size_t)255; }

static MoeMWs moe_mws_layout(void *base, int B, int D, int inter, int sinter, int E, int k) {
  MoeMWs w{};
  const size_t nsl = (size_t)B * k;
  const size_t slots = nsl + B;
  const size_t hmax = (size_t)(inter > sinter ? inter : sinter);
  const int G = (int)(nsl < (size_t)E ? nsl : (size_t)E);
  w.max_tiles = (int)((nsl + kMTok - 1) / kMTok) + G + (B + kMTok - 1) / kMTok;
  size_t off = 0;
  char *b = reinterpret_cast<char *>(base);
  auto take = [&](size_t bytes) {
    char *p = b ? b + off : nullptr;
    off += al256m(bytes);
    return p;
  };
  w.n_tiles = reinterpret_cast<int *>(take(sizeof(int)));
  w.tiles = reinterpret_cast<int4 *>(take(sizeof(int4) * (size_t)w.max_tiles));
  w.tok = reinterpret_cast<int *>(take(sizeof(int) * nsl));
  w.gpos = reinterpret_cast<int *>(take(sizeof(int) * nsl));
  w.topk_idx = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * nsl));
  w.topk_w = reinterpret_cast<float *>(take(sizeof(float) * nsl));
  w.gs = reinterpret_cast<float *>(take(sizeof(float) * (size_t)B));
  w.xop = reinterpret_cast<uint16_t *>(take(sizeof(uint16_t) * (size_t)B * D));
  w.h_hi = reinterpret_cast<uint16_t *>(take(sizeof(uint16_t) * slots * hmax));
  w.h_lo = reinterpret_cast<uint16_t *>(take(sizeof(uint16_t) * slots * hmax));
  w.y = reinterpret_cast<float *>(take(sizeof(float) * slots * (size_t)D));
  w.total = off;
  return w;
}

size_t moe_mfma_workspace_bytes(int B, int D, int inter, int sinter, int E, int k) {
  return moe_mws_layout(nullptr, B, D, inter, sinter, E, k).total;
}

// ---------------------------------------------------------------------------
// 1. routing and the shared-expert gate, one wave per token

constexpr int kMRouteXr = 4;  // x granules (8 bf16) per lane held across the routing

template <int KPL, bool F32>
__global__ __launch_bounds__(256) void moe_mroute_kernel(MoeArgs a, MoeMWs w) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= a.B) return;  // whole waves leave together
  // the token's first 64 x kMRouteXr granules of x (and of the shared gate
  // vector), loaded before the routing so that their latency overlaps it
  const int n8 = a.D >> 3;
  const bool op4 = a.gate.m.bits == 4;
  const bool gdot = a.sgate.m.w && a.se_gate_vec;
  const uint4 *xs = reinterpret_cast<const uint4 *>(a.x + (size_t)t * a.D);
  const uint4 *gv = reinterpret_cast<const uint4 *>(a.se_gate_vec);
  uint4 xr[kMRouteXr], gr[kMRouteXr];
#pragma unroll
  for (int q = 0; q < kMRouteXr; ++q) {
    const int c = lane + 64 * q;
    xr[q] = make_uint4(0u, 0u, 0u, 0u);
    gr[q] = make_uint4(0u, 0u, 0u, 0u);
    if (c < n8 && (op4 || gdot)) xr[q] = xs[c];
    if (c < n8 && gdot) gr[q] = gv[c];
  }
  int id;
  float wt;
  wave_topk_lanes<KPL, F32>(a.logits, (size_t)t * a.E, a.E, a.k, id, wt);
  if (lane < a.k) {
    const size_t s = (size_t)t * a.k + lane;
    w.topk_idx[s] = id;
    w.topk_w[s] = wt;
    if (a.idx_out) a.idx_out[s] = id;
    if (a.w_out) a.w_out[s] = wt;
  }
  if (op4) {
    // x in the operand order of 4-bit codes: pairs (x_p, x_{p+4}) of every 8
    uint4 *xd = reinterpret_cast<uint4 *>(w.xop + (size_t)t * a.D);
#pragma unroll
    for (int q = 0; q < kMRouteXr; ++q) {
      const int c = lane + 64 * q;
      if (c < n8) xd[c] = __builtin_bit_cast(uint4, a_nibble_order(xr[q]));
    }
    for (int c = lane + 64 * kMRouteXr; c < n8; c += 64) xd[c] = __builtin_bit_cast(uint4, a_nibble_order(xs[c]));
  }
  if (a.sgate.m.w) {
    // sigmoid(se_g . x_t) (logan-qwen4/src/lib.rs:7602-7604), 8 bf16 per lane per load
    float g = 1.0f;
    if (gdot) {
      float acc = 0.f;
#pragma unroll
      for (int q = 0; q < kMRouteXr; ++q) {
        acc = dot2(gr[q].x, xr[q].x, acc);
        acc = dot2(gr[q].y, xr[q].y, acc);
        acc = dot2(gr[q].z, xr[q].z, acc);
        acc = dot2(gr[q].w, xr[q].w, acc);
      }
      for (int c = lane + 64 * kMRouteXr; c < n8; c += 64) {
        const uint4 gq = gv[c], xq = xs[c];
        acc = dot2(gq.x, xq.x, acc);
        acc = dot2(gq.y, xq.y, acc);
        acc = dot2(gq.z, xq.z, acc);
        acc = dot2(gq.w, xq.w, acc);
      }
      acc = wave_sum_f32(acc);
      g = 1.0f / (1.0f + __expf(-acc));
    }
    if (lane == 0) w.gs[t] = g;
  }
}

// ---------------------------------------------------------------------------
// 2. grouping into tiles (one block)

__global__ __launch_bounds__(kMGroupThreads) void moe_mgroup_kernel(MoeArgs a, MoeMWs w) {
  __shared__ int s_cnt[kMMaxE];
  __shared__ int s_start[kMMaxE];
  __shared__ int s_tbase[kMMaxE];
  __shared__ int s_fill[kMMaxE];
  __shared__ int s_wave_tot[kMGroupThreads / 64];
  __shared__ int s_routed_tiles;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nslots = a.B * a.k;
  for (int e = tid; e < kMMaxE; e += kMGroupThreads) {
    s_cnt[e] = 0;
    s_fill[e] = 0;
  }
  __syncthreads();
  // the first kMGroupKeep slots of each thread stay in registers for the
  // placement below (one global read of the routes instead of two)
  int keep[kMGroupKeep];
#pragma unroll
  for (int q = 0; q < kMGroupKeep; ++q) {
    const int i = tid + q * kMGroupThreads;
    keep[q] = i < nslots ? w.topk_idx[i] : 0;
  }
#pragma unroll
  for (int q = 0; q < kMGroupKeep; ++q)
    if (tid + q * kMGroupThreads < nslots) atomicAdd(&s_cnt[keep[q]], 1);
  for (int i = tid + kMGroupKeep * kMGroupThreads; i < nslots; i += kMGroupThreads) atomicAdd(&s_cnt[w.topk_idx[i]], 1);
  __syncthreads();
  {
    // exclusive scan over experts of (slots << 14 | tiles): slots <= 2^16,
    // tiles <= 2^12 + 2^10
    const int e = tid;
    const int c = e < a.E ? s_cnt[e] : 0;
    const int v = (c << 14) | ((c + kMTok - 1) / kMTok);
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
      s_start[e] = excl >> 14;
      s_tbase[e] = excl & 16383;
    }
    if (tid == kMGroupThreads - 1) s_routed_tiles = (prefix + incl) & 16383;
  }
  __syncthreads();
  // placement in arrival order (each row's arithmetic is independent of it)
#pragma unroll
  for (int q = 0; q < kMGroupKeep; ++q) {
    const int i = tid + q * kMGroupThreads;
    if (i < nslots) {
      const int e = keep[q];
      const int gp = s_start[e] + atomicAdd(&s_fill[e], 1);
      w.tok[gp] = i / a.k;
      w.gpos[i] = gp;
    }
  }
  for (int i = tid + kMGroupKeep * kMGroupThreads; i < nslots; i += kMGroupThreads) {
    const int e = w.topk_idx[i];
    const int gp = s_start[e] + atomicAdd(&s_fill[e], 1);
    w.tok[gp] = i / a.k;
    w.gpos[i] = gp;
  }
  // the shared expert's tiles first, then the routed ones (the launches
  // give the first tiles whole-tile blocks)
  const int R = s_routed_tiles;
  const int S = a.sgate.m.w ? (a.B + kMTok - 1) / kMTok : 0;
  for (int e = tid; e < a.E; e += kMGroupThreads) {
    const int c = s_cnt[e];
    for (int tt = 0; tt * kMTok < c; ++tt)
      w.tiles[S + s_tbase[e] + tt] = make_int4(e, s_start[e] + kMTok * tt, min(kMTok, c - kMTok * tt), 0);
  }
  for (int tt = tid; tt < S; tt += kMGroupThreads)
    w.tiles[tt] = make_int4(-1, nslots + kMTok * tt, min(kMTok, a.B - kMTok * tt), 0);
  if (tid == 0) *w.n_tiles = R + S;
}

// ---------------------------------------------------------------------------
// 3. gate/up + SwiGLU: block = (tile, 16 * WAVES rows), wave = 16 rows of gate
//    and up; batches of GU 64-code steps double-buffered in registers

#ifndef MOE_GU
#define MOE_GU 4
#endif
// Two block shapes: 8 waves (128 rows, one block per CU) for large batches,
// 4 waves (64 rows) with two blocks resident per CU for batches of up to
// kMGuSmallB tokens, whose few tiles per expert leave the chip short of
// blocks (config 4 B = 32: 140 -> 128 µs per 5-bit layer; the B = 512
// prefill chunk 2 % slower with 4 waves)
#ifndef MOE_GU_WAVES
#define MOE_GU_WAVES 8
#endif
#ifndef MOE_GU_MINW
#define MOE_GU_MINW 1  // minimum waves per SIMD (register cap) of the 8-wave shape
#endif
constexpr int kMGuSmallB = 128;

// scale/bias words of GU steps for one lane's row: with 64-code groups the GU
// consecutive u16 come in one load
template <int GU, bool GS64>
struct AuxRun {
  uint32_t s[GS64 ? GU / 2 : GU], b[GS64 ? GU / 2 : GU];
  __device__ __forceinline__ void load(const uint16_t *sr, const uint16_t *br, int st, int gsteps) {
    if constexpr (GS64) {
      static_assert(GU == 2 || GU == 4 || GU == 8, "aux run of 2, 4 or 8 steps");
      if constexpr (GU == 8) {
        const uint4 vs = *reinterpret_cast<const uint4 *>(sr + st);
        const uint4 vb = *reinterpret_cast<const uint4 *>(br + st);
        s[0] = vs.x; s[1] = vs.y; s[2] = vs.z; s[3] = vs.w;
        b[0] = vb.x; b[1] = vb.y; b[2] = vb.z; b[3] = vb.w;
      } else if constexpr (GU == 4) {
        const uint2 vs = *reinterpret_cast<const uint2 *>(sr + st);
        const uint2 vb = *reinterpret_cast<const uint2 *>(br + st);
        s[0] = vs.x; s[1] = vs.y; b[0] = vb.x; b[1] = vb.y;
      } else {
        s[0] = *reinterpret_cast<const uint32_t *>(sr + st);
        b[0] = *reinterpret_cast<const uint32_t *>(br + st);
      }
    } else {
#pragma unroll
      for (int u = 0; u < GU; ++u) {
        s[u] = sr[(st + u) / gsteps];
        b[u] = br[(st + u) / gsteps];
      }
    }
  }
  __device__ __forceinline__ uint32_t sw(int u) const {
    if constexpr (GS64) return (s[u >> 1] >> (16 * (u & 1))) & 0xffffu;
    else return s[u];
  }
  __device__ __forceinline__ uint32_t bw(int u) const {
    if constexpr (GS64) return (b[u >> 1] >> (16 * (u & 1))) & 0xffffu;
    else return b[u];
  }
};

template <int BITS, int GU, bool GS64>
struct GuBatch {
  SkRaw<BITS> g[GU], u[GU];
  AuxRun<GU, GS64> ag, au;
};

template <int BITS, int GU, int WAVES, bool GS64, bool FP16>
__global__ __launch_bounds__(WAVES * 64, WAVES <= 4 ? 2 : MOE_GU_MINW) void moe_gateup_mfma_kernel(MoeArgs a, MoeMWs w, int ipt) {
  __shared__ __align__(16) uint16_t sx[kMTok * kMChunk];
  constexpr int NT = WAVES * 64;
  constexpr int RPB = 16 * WAVES;
  using S = MfmaStep<BITS>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int tile = blockIdx.x / ipt, rb = blockIdx.x % ipt;
  if (tile >= *w.n_tiles) return;
  const int4 tr = w.tiles[tile];
  const int e = __builtin_amdgcn_readfirstlane(tr.x);
  const int row0 = __builtin_amdgcn_readfirstlane(tr.y);
  const int cnt = __builtin_amdgcn_readfirstlane(tr.z);
  const bool shared = e < 0;
  const int rows = shared ? a.sinter : a.inter;
  if (rb * RPB >= rows) return;
  const DevBank &gbk = shared ? a.sgate : a.gate;
  const DevBank &ubk = shared ? a.sup : a.up;
  const size_t eo = shared ? 0 : (size_t)e;
  const int j = min(rb * RPB + wave * 16 + r16, rows - 1);
  const uint8_t *gw = gbk.m.w + eo * gbk.w_stride + (size_t)j * gbk.m.row_bytes;
  const uint8_t *uw = ubk.m.w + eo * ubk.w_stride + (size_t)j * ubk.m.row_bytes;
  const uint16_t *gsr = gbk.m.sc + eo * gbk.p_stride + (size_t)j * gbk.m.ng;
  const uint16_t *gbr = gbk.m.bi + eo * gbk.p_stride + (size_t)j * gbk.m.ng;
  const uint16_t *usr = ubk.m.sc + eo * ubk.p_stride + (size_t)j * ubk.m.ng;
  const uint16_t *ubr = ubk.m.bi + eo * ubk.p_stride + (size_t)j * ubk.m.ng;
  const int gsteps = gbk.m.gs >> 6;
  const int nslots = a.B * a.k;
  const int chunk = a.D < kMChunk ? a.D : kMChunk;
  const int nch = a.D / chunk;
  const int bpc = (chunk >> 6) / GU;  // batches per chunk
  const uint16_t *xsrc = BITS == 4 ? w.xop : a.x;  // x in the operand order
  UnpackConsts kc;
  kc.init();
  const bf16x8_t ones = mfma_ones();
  f32x4_t accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
  // the tile's token indices, read once (the x staging loads then depend on
  // LDS only and are all in flight together); rows past the tile repeat its
  // last token
  __shared__ int s_tok[kMTok];
  if (tid < kMTok) s_tok[tid] = shared ? row0 - nslots + min(tid, cnt - 1) : w.tok[row0 + min(tid, cnt - 1)];
  __syncthreads();

  auto issue = [&](int st, GuBatch<BITS, GU, GS64> &B) {
#pragma unroll
    for (int u = 0; u < GU; ++u) {
      const int k = (st + u) * 64 + 16 * g;
      S::load_raw(B.g[u], gw, k);
      S::load_raw(B.u[u], uw, k);
    }
    B.ag.load(gsr, gbr, st, gsteps);
    B.au.load(usr, ubr, st, gsteps);
  };
  auto step = [&](int stc, const GuBatch<BITS, GU, GS64> &B) {
#pragma unroll
    for (int u = 0; u < GU; ++u) {
      bf16x8_t a0, a1, b0, b1;
      S::a_ops(sx + r16 * chunk, ((stc + u) * 64 + 16 * g) >> 3, r16, a0, a1);
      const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      f32x4_t xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, ones, z, 0, 0, 0);
      xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, ones, xs, 0, 0, 0);
      S::b_ops(B.g[u], kc, b0, b1);
      f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, z, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, d, 0, 0, 0);
      S::fold(accg, d, xs, aux_f32<FP16>(B.ag.sw(u)), aux_f32<FP16>(B.ag.bw(u)));
      S::b_ops(B.u[u], kc, b0, b1);
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, z, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, d, 0, 0, 0);
      S::fold(accu, d, xs, aux_f32<FP16>(B.au.sw(u)), aux_f32<FP16>(B.au.bw(u)));
    }
  };

  for (int c = 0; c < nch; ++c) {
    const int s0 = c * chunk >> 6;
    GuBatch<BITS, GU, GS64> B0, B1;
    issue(s0, B0);
    // stage x of the tile's tokens, codes [c*chunk, (c+1)*chunk), straight
    // into LDS: lane granule pg of the 16-row tile is physical granule P of
    // row m, which holds logical granule P ^ (m & 15)
    if (c > 0) __syncthreads();
    {
      constexpr int NV = kMTok * kMChunk / 8 / NT;
      const int gpr = chunk >> 3;  // granules per row (>= 32)
      auto dma = [&](int base) {
        const int pg = base + lane;
        const int m = pg / gpr, qq = swz(m, pg % gpr);
        lds_dma16(xsrc + (size_t)s_tok[m] * a.D + c * chunk + 8 * qq, sx + 8 * base);
      };
      // rows from cnt on are not staged: their LDS rows keep what an earlier
      // block left there, and feed only MFMA output rows that are not stored
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (NT * i + 64 * wave < cnt * gpr) dma(NT * i + 64 * wave);
      lds_dma_wait();
    }
    __syncthreads();
    // issues past the chunk end reload its last batch (unconditional, so the
    // in-order vmcnt stays exact)
    for (int b = 0; b < bpc; b += 2) {
      issue(s0 + GU * min(b + 1, bpc - 1), B1);
      __builtin_amdgcn_sched_barrier(0);
      step(GU * b, B0);
      issue(s0 + GU * min(b + 2, bpc - 1), B0);
      __builtin_amdgcn_sched_barrier(0);
      if (b + 1 < bpc) step(GU * (b + 1), B1);
    }
  }
  // h = silu(gate) * up (logan-qwen4/src/lib.rs:8807-8809) as hi + lo bf16,
  // each at its place in the down pass's operand order
  const int jj = rb * RPB + wave * 16 + r16;
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  if (jj < rows) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 4 * g + i;
      if (m < cnt) {
        const float h = silu(accg[i]) * accu[i];
        const uint32_t hi = f32_to_bf16_rne(h);
        const uint32_t lo = f32_to_bf16_rne(h - bf16_to_f32(hi));
        const size_t o = (size_t)(row0 + m) * hmax + S::op_pos(jj);
        w.h_hi[o] = (uint16_t)hi;
        w.h_lo[o] = (uint16_t)lo;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 3b. gate/up with the weights staged in LDS (4- and 8-bit codes, 8 waves, the
//     large-batch shape). The register form above has each lane load its own
//     8 or 16 bytes of 16 rows per step: one load instruction touches 16
//     lines 32 bytes at a time, the same line again on each of the next
//     three steps, and 8 waves x 32 rows of lines in flight per CU do not
//     stay in its L1. Here each wave copies its 16 gate and 16 up rows batch
//     by batch (128 bytes of every row: 4 steps of 4-bit codes, 2 of 8-bit)
//     straight into a private LDS ring with global_load_lds: 8 lanes cover
//     one row's 128 bytes, so each instruction reads whole lines of 8 rows,
//     each line once. Scale/bias words, the x tile, the MFMA steps and the
//     fold are those of the register form.

// Direct global -> LDS copies whose LDS writes the compiler does not see, so it
// inserts no waits for them before LDS reads (it would wait for every copy in
// flight, the ring's next batches included); the kernels wait with vmcnt
// themselves. Lane l writes its 16 (4) bytes at lds + 16 l (4 l); lds is the
// wave-uniform LDS byte address.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const uint8_t *)p);
}
__device__ __forceinline__ void lds_copy16(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(src), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void lds_copy4(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(src), "s"(lds) : "memory", "m0");
}

// One slot of a wave's LDS ring: a batch of two 16-row groups (m = 0, 1) x
// 128 bytes of BITS-bit codes (GU steps of 64), groups of 64 codes. Bytes
// [2048 m, 2048 m + 2048): group m's rows, 128 bytes each, the 16-byte chunk
// c of row r at position c ^ (r & 7) (the 16 rows of an MFMA operand read
// spread over the banks); then the scale and bias words of the GU steps:
// 4-bit: [128 m + 0: m's scales (8 bytes per row) | +128: biases] per group,
// 8-bit: [64 (2m): m's scales (4 bytes per row) | 64 (2m + 1): biases].
template <int BITS>
struct RingSlot {
  static_assert(BITS == 4 || BITS == 8, "128-byte row batches of 4- or 8-bit codes");
  static constexpr int GU = BITS == 4 ? 4 : 2;  // steps per batch
  static constexpr int BYTES = 4096 + (BITS == 4 ? 512 : 256);
  static constexpr int NI = BITS == 4 ? 6 : 5;  // copies per batch

  // the copies of one batch into slot d: row pointers wr[i] (rows 8 i + lane / 8
  // of the slot, already at the batch's first byte plus the lane's source chunk
  // 16 ((lane & 7) ^ (lane >> 3))), scale/bias pointers of the batch (aux1
  // 4-bit only) as laid out by aux_ptr
  static __device__ __forceinline__ void issue(uint32_t d, const uint8_t *wr[4], const uint16_t *aux0,
                                               const uint16_t *aux1) {
    lds_copy16(wr[0], d);
    lds_copy16(wr[1], d + 1024);
    lds_copy16(wr[2], d + 2048);
    lds_copy16(wr[3], d + 3072);
    lds_copy4(aux0, d + 4096);
    if constexpr (BITS == 4) lds_copy4(aux1, d + 4096 + 256);
  }
  // the lane's first scale/bias word to copy (u16 index of the batch's first
  // step added per batch) for groups whose rows are rowm[0], rowm[1] + (the
  // lane's row inside its group, chosen here): 4-bit: copy m, lanes 0-31
  // scales, 32-63 biases, row (l & 31) / 2, dword l & 1; 8-bit: one copy,
  // lanes 0-15 group 0 scales, 16-31 its biases, 32-63 group 1 likewise, row l & 15
  static __device__ __forceinline__ void aux_ptr(int lane, const DevBank &b0, const DevBank &b1,
                                                 size_t eo, const int (&rowm)[2], int rmax,
                                                 const uint16_t *(&aux)[2]) {
    if constexpr (BITS == 4) {
      const int rl = (lane & 31) >> 1;
      const int r0 = min(rowm[0] + rl, rmax), r1 = min(rowm[1] + rl, rmax);
      aux[0] = (lane < 32 ? b0.m.sc : b0.m.bi) + eo * b0.p_stride + (size_t)r0 * b0.m.ng + 2 * (lane & 1);
      aux[1] = (lane < 32 ? b1.m.sc : b1.m.bi) + eo * b1.p_stride + (size_t)r1 * b1.m.ng + 2 * (lane & 1);
    } else {
      const int m = lane >> 5;
      const DevBank &bk = m ? b1 : b0;
      const int r = min(rowm[m] + (lane & 15), rmax);
      aux[0] = (((lane >> 4) & 1) ? bk.m.bi : bk.m.sc) + eo * bk.p_stride + (size_t)r * bk.m.ng;
      aux[1] = aux[0];
    }
  }
  // the lane's 16 codes of step u, group m (lane = 16 g + r16)
  static __device__ __forceinline__ void raw(const uint8_t *slot, int m, int u, int r16, int g,
                                             SkRaw<BITS> &r) {
    const uint8_t *row = slot + m * 2048 + r16 * 128;
    if constexpr (BITS == 4) {
      const int c = 2 * u + (g >> 1);
      r.v = *reinterpret_cast<const uint2 *>(row + ((c ^ (r16 & 7)) << 4) + 8 * (g & 1));
    } else {
      const int c = 4 * u + g;
      r.v = *reinterpret_cast<const uint4 *>(row + ((c ^ (r16 & 7)) << 4));
    }
  }
  // output row r16's scale / bias words of the batch's steps, two u16 per word
  static __device__ __forceinline__ void aux(const uint8_t *slot, int r16, uint32_t (&sw)[2][GU / 2],
                                             uint32_t (&bw)[2][GU / 2]) {
    if constexpr (BITS == 4) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const uint2 s2 = *reinterpret_cast<const uint2 *>(slot + 4096 + 256 * m + 8 * r16);
        const uint2 b2 = *reinterpret_cast<const uint2 *>(slot + 4096 + 256 * m + 128 + 8 * r16);
        sw[m][0] = s2.x; sw[m][1] = s2.y;
        bw[m][0] = b2.x; bw[m][1] = b2.y;
      }
    } else {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        sw[m][0] = *reinterpret_cast<const uint32_t *>(slot + 4096 + 128 * m + 4 * r16);
        bw[m][0] = *reinterpret_cast<const uint32_t *>(slot + 4096 + 128 * m + 64 + 4 * r16);
      }
    }
  }
  // step u's u16 of a word pair
  template <bool FP16>
  static __device__ __forceinline__ float word(const uint32_t (&v)[GU / 2], int u) {
    return aux_f32<FP16>((v[u >> 1] >> (16 * (u & 1))) & 0xffffu);
  }
};

// As with the down blocks below, one 8-wave block fills a CU (the x tile and
// the ring), so blocks run in rounds and each pays its start (x tile, first
// batch) and end. When x fits one chunk, the first tiles take whole-tile
// blocks (all the tile's 128-row groups, one after another in each wave, the
// x tile staged once and the ring running on from one group into the next)
// and the last kMGuSmallUnits (tile, 128-row group) units follow as one-group
// blocks, taken by the CUs whose whole-tile blocks end first.

constexpr int kMGuSmallUnits = 256;  // one round on 256 CUs

template <int BITS, bool FP16>
__global__ __launch_bounds__(512, 1) void moe_gateup_lds_kernel(MoeArgs a, MoeMWs w, int ipt) {
  constexpr int WAVES = 8, NT = WAVES * 64, RPB = 16 * WAVES;
  using R = RingSlot<BITS>;
  constexpr int GU = R::GU, NB = 2;  // two batches in a wave's ring
  __shared__ __align__(16) uint16_t sx[kMTok * kMChunk];
  // sums of the tile's x over each 64-code step of the chunk (the fold's bias
  // term), formed once per chunk for all the block's row groups
  __shared__ __align__(16) float sxs[kMChunk / 64][kMTok];
  __shared__ __align__(16) uint8_t swt[NB][WAVES][R::BYTES];
  __shared__ int s_tok[kMTok];
  using S = MfmaStep<BITS>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int chunk = a.D < kMChunk ? a.D : kMChunk;
  const int nch = a.D / chunk;
  // blocks [0, nbt) take whole tiles (ipt row groups); then the tiles from
  // nbt on one 128-row group per block
  const int nt = __builtin_amdgcn_readfirstlane(*w.n_tiles);
  const int units = nt * ipt;
  const int nbt = nch == 1 && units > kMGuSmallUnits ? (units - kMGuSmallUnits) / ipt : 0;
  const int bid = blockIdx.x;
  int tile, rg0, nrg;
  if (bid < nbt) {
    tile = bid;
    rg0 = 0;
    nrg = ipt;
  } else {
    tile = nbt + (bid - nbt) / ipt;
    rg0 = (bid - nbt) % ipt;
    nrg = 1;
  }
  if (tile >= nt) return;
  const int4 tr = w.tiles[tile];
  const int e = __builtin_amdgcn_readfirstlane(tr.x);
  const int row0 = __builtin_amdgcn_readfirstlane(tr.y);
  const int cnt = __builtin_amdgcn_readfirstlane(tr.z);
  const bool shared = e < 0;
  const int rows = shared ? a.sinter : a.inter;
  if (rg0 * RPB >= rows) return;
  nrg = min(nrg, (rows + RPB - 1) / RPB - rg0);
  const DevBank &gbk = shared ? a.sgate : a.gate;
  const DevBank &ubk = shared ? a.sup : a.up;
  const size_t eo = shared ? 0 : (size_t)e;
  const int jw0 = rg0 * RPB + wave * 16;  // the wave's first row (row group rg0)
  const int rmax = rows - 1;
  // the banks' fields, read here: such a load inside the ring loop would wait
  // for every copy in flight. Ring group 0 = the gate rows, group 1 = the same
  // rows of up: rows jr + lane / 8 and jr + 8 + lane / 8 at the lane's source
  // chunk; scale / bias words as RingSlot::aux_ptr lays them out.
  const int lr = lane >> 3, sc = 16 * ((lane & 7) ^ lr);
  const uint8_t *const gb = gbk.m.w + eo * gbk.w_stride + sc;
  const uint8_t *const ub = ubk.m.w + eo * ubk.w_stride + sc;
  const size_t grb = gbk.m.row_bytes, urb = ubk.m.row_bytes;
  const uint16_t *ab0, *ab1;
  int arl, ang0, ang1;
  if constexpr (BITS == 4) {
    ab0 = (lane < 32 ? gbk.m.sc : gbk.m.bi) + eo * gbk.p_stride + 2 * (lane & 1);
    ab1 = (lane < 32 ? ubk.m.sc : ubk.m.bi) + eo * ubk.p_stride + 2 * (lane & 1);
    arl = (lane & 31) >> 1;
    ang0 = gbk.m.ng;
    ang1 = ubk.m.ng;
  } else {
    const bool up = lane >= 32;
    const bool bias = (lane >> 4) & 1;
    ab0 = up ? (bias ? ubk.m.bi : ubk.m.sc) + eo * ubk.p_stride
             : (bias ? gbk.m.bi : gbk.m.sc) + eo * gbk.p_stride;
    ab1 = ab0;
    arl = lane & 15;
    ang0 = up ? ubk.m.ng : gbk.m.ng;
    ang1 = ang0;
  }
  const int nslots = a.B * a.k;
  const int bpc = (chunk >> 6) / GU;  // batches per chunk
  const int nbc = nrg * bpc;          // batches of a chunk over the block's row groups
  const uint16_t *xsrc = BITS == 4 ? w.xop : a.x;  // x in the operand order
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  UnpackConsts kc;
  kc.init();
  const bf16x8_t ones = mfma_ones();
  f32x4_t acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};  // gate, up
  if (tid < kMTok) s_tok[tid] = shared ? row0 - nslots + min(tid, cnt - 1) : w.tok[row0 + min(tid, cnt - 1)];
  __syncthreads();

  // the next batch of chunk c to copy (uniform): index in the chunk's row
  // group major sequence, ring slot, row group, batch in the chunk (bytes
  // [128 (c bpc + ibl), + 128) of every row, steps GU (c bpc + ibl) on). Past
  // the chunk's last batch the cursor stays there and the copy repeats that
  // batch into its own slot (the same bytes, so step() reads them whether or
  // not the copy has landed), which keeps the count of copies behind every
  // batch at NI.
  const uint32_t ring0 = __builtin_amdgcn_readfirstlane(lds_addr(&swt[0][wave][0]));
  int ib = 0, is = 0, ir = 0, ibl = 0;
  // the copy sources of row group ir at byte 0 of its rows, formed when the
  // cursor enters the group
  const uint8_t *cw[4];
  const uint16_t *ca0, *ca1;
  auto set_rows = [&]() {
    const int jr = jw0 + ir * RPB;
    const int jl0 = min(jr + lr, rmax), jl1 = min(jr + 8 + lr, rmax), ja = min(jr + arl, rmax);
    cw[0] = gb + (size_t)jl0 * grb;
    cw[1] = gb + (size_t)jl1 * grb;
    cw[2] = ub + (size_t)jl0 * urb;
    cw[3] = ub + (size_t)jl1 * urb;
    ca0 = ab0 + (size_t)ja * ang0;
    ca1 = ab1 + (size_t)ja * ang1;
  };
  auto issue_next = [&](int c) {
    const uint32_t d = __builtin_amdgcn_readfirstlane(ring0 + (uint32_t)is * (WAVES * R::BYTES));
    const int kb = c * bpc + ibl;
    const size_t o = (size_t)128 * kb;
    const uint8_t *wr[4] = {cw[0] + o, cw[1] + o, cw[2] + o, cw[3] + o};
    R::issue(d, wr, ca0 + kb * GU, ca1 + kb * GU);
    if (ib < nbc - 1) {
      ++ib;
      is ^= 1;
      if (++ibl == bpc) {
        ibl = 0;
        ++ir;
        set_rows();
      }
    }
  };
  auto step = [&](const uint8_t *slot, int bl) {
    uint32_t sw[2][GU / 2], bw[2][GU / 2];
    R::aux(slot, r16, sw, bw);
#pragma unroll
    for (int u = 0; u < GU; ++u) {
      bf16x8_t a0, a1, b0, b1;
      S::a_ops(sx + r16 * chunk, ((bl * GU + u) * 64 + 16 * g) >> 3, r16, a0, a1);
      const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      const float4 xv = *reinterpret_cast<const float4 *>(&sxs[bl * GU + u][4 * g]);
      const f32x4_t xs = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        SkRaw<BITS> rw;
        R::raw(slot, m, u, r16, g, rw);
        S::b_ops(rw, kc, b0, b1);
        f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, z, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, d, 0, 0, 0);
        S::fold(acc[m], d, xs, R::template word<FP16>(sw[m], u), R::template word<FP16>(bw[m], u));
      }
    }
  };

  for (int c = 0; c < nch; ++c) {
    // the x tile's copies and the chunk's first batch, then one full wait
    if (c > 0) __syncthreads();
    {
      constexpr int NV = kMTok * kMChunk / 8 / NT;
      const int gpr = chunk >> 3;  // granules per row (>= 32)
      auto dma = [&](int base) {
        const int pg = base + lane;
        const int m = pg / gpr, qq = swz(m, pg % gpr);
        lds_dma16(xsrc + (size_t)s_tok[m] * a.D + c * chunk + 8 * qq, sx + 8 * base);
      };
      // rows from cnt on are not staged: their LDS rows keep what an earlier
      // block left there, and feed only MFMA output rows that are not stored
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (NT * i + 64 * wave < cnt * gpr) dma(NT * i + 64 * wave);
    }
    ib = 0;
    is = 0;
    ir = 0;
    ibl = 0;
    set_rows();
    issue_next(c);
    lds_dma_wait();
    __syncthreads();
    // the step sums of x: wave w forms steps w, w + 8, ... (one MFMA pair
    // against ones each; lanes of one 16-lane row hold the same four tokens)
    for (int u = wave; u < (chunk >> 6); u += WAVES) {
      bf16x8_t a0, a1;
      S::a_ops(sx + r16 * chunk, (u * 64 + 16 * g) >> 3, r16, a0, a1);
      const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      f32x4_t xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, ones, z, 0, 0, 0);
      xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, ones, xs, 0, 0, 0);
      if (r16 == 0) *reinterpret_cast<float4 *>(&sxs[u][4 * g]) = make_float4(xs[0], xs[1], xs[2], xs[3]);
    }
    __syncthreads();
    // batch b + 1 in flight while batch b is multiplied: wait for all but the
    // NI copies of the batch issued last
    int cs = 0;  // ring slot of the batch multiplied
    for (int rg = 0; rg < nrg; ++rg) {
      for (int bl = 0; bl < bpc; ++bl) {
        issue_next(c);
        lds_dma_wait_behind<R::NI>();
        step(&swt[cs][wave][0], bl);
        cs ^= 1;
      }
      if (c == nch - 1) {
        // h = silu(gate) * up (logan-qwen4/src/lib.rs:8807-8809) as hi + lo
        // bf16, each at its place in the down pass's operand order
        const int jj = jw0 + rg * RPB + r16;
        if (jj < rows) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = 4 * g + i;
            if (m < cnt) {
              const float h = silu(acc[0][i]) * acc[1][i];
              const uint32_t hi = f32_to_bf16_rne(h);
              const uint32_t lo = f32_to_bf16_rne(h - bf16_to_f32(hi));
              const size_t o = (size_t)(row0 + m) * hmax + S::op_pos(jj);
              w.h_hi[o] = (uint16_t)hi;
              w.h_lo[o] = (uint16_t)lo;
            }
          }
        }
#pragma unroll
        for (int m = 0; m < 2; ++m) acc[m] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
    }
  }
  lds_dma_wait();  // no copy into LDS outlives the block
}

// ---------------------------------------------------------------------------
// 4. down: block = (tile, 128 rows), wave = 2 x 16 rows, K <= 512: h copied
//    into LDS first, then every scale/bias and weight load of the wave, and
//    each step waits only for its own weights

template <int BITS, bool FP16>
__global__ __launch_bounds__(256) void moe_down_mfma_kernel(MoeArgs a, MoeMWs w, int ipt) {
  constexpr int NS = kMDownK / 64;  // steps at most
  __shared__ __align__(16) uint16_t shi[kMTok * kMDownK];
  __shared__ __align__(16) uint16_t slo[kMTok * kMDownK];
  using S = MfmaStep<BITS>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int tile = blockIdx.x / ipt, rb = blockIdx.x % ipt;
  if (tile >= *w.n_tiles) return;
  const int4 tr = w.tiles[tile];
  const int e = __builtin_amdgcn_readfirstlane(tr.x);
  const int row0 = __builtin_amdgcn_readfirstlane(tr.y);
  const int cnt = __builtin_amdgcn_readfirstlane(tr.z);
  const bool shared = e < 0;
  const DevBank &dbk = shared ? a.sdown : a.down;
  const int K = shared ? a.sinter : a.inter;
  const size_t eo = shared ? 0 : (size_t)e;
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  const int steps = K >> 6;
  const int gsteps = dbk.m.gs >> 6;
  // scale/bias as dwords of two steps when every step is its own group
  const bool pair_aux = __builtin_amdgcn_readfirstlane(gsteps == 1 && (dbk.m.ng & 1) == 0);
  SkRaw<BITS> wr[2][NS];
  uint32_t sr[2][NS], br[2][NS];
  {
    // stage h (hi, lo) of the tile's rows straight into LDS, first: loads
    // complete in issue order, so the steps' weights (issued last) may still
    // be in flight when the copies are waited for (physical granule P of row
    // m holds logical granule P ^ (m & 15))
    constexpr int NQ = kMTok * kMDownK / 8 / 256;
    const int gpr = K >> 3;  // >= 16
    auto dma = [&](int base) {
      const int pg = base + lane;
      const int m = pg / gpr, qq = swz(m, pg % gpr);
      const size_t o = (size_t)(row0 + min(m, cnt - 1)) * hmax + 8 * qq;
      lds_dma16(w.h_hi + o, shi + 8 * base);
      lds_dma16(w.h_lo + o, slo + 8 * base);
    };
    // rows from cnt on are not staged (they feed only output rows not stored)
#pragma unroll
    for (int i = 0; i < NQ; ++i)
      if (256 * i + 64 * wave < cnt * gpr) dma(256 * i + 64 * wave);
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int d = min(rb * 128 + wave * 32 + 16 * r + r16, a.D - 1);
    const uint16_t *srow = dbk.m.sc + eo * dbk.p_stride + (size_t)d * dbk.m.ng;
    const uint16_t *brow = dbk.m.bi + eo * dbk.p_stride + (size_t)d * dbk.m.ng;
    if (pair_aux) {
#pragma unroll
      for (int u = 0; u < NS; u += 2) {
        const int q = min(u, steps - 2);
        // the dword of steps (u, u + 1) in slot u, split where it is used
        sr[r][u] = *reinterpret_cast<const uint32_t *>(srow + q);
        br[r][u] = *reinterpret_cast<const uint32_t *>(brow + q);
        sr[r][u + 1] = 0;
        br[r][u + 1] = 0;
      }
    } else {
#pragma unroll
      for (int u = 0; u < NS; ++u) {
        const int gi = min(u, steps - 1) / gsteps;
        sr[r][u] = srow[gi];
        br[r][u] = brow[gi];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int d = min(rb * 128 + wave * 32 + 16 * r + r16, a.D - 1);
    const uint8_t *wrow = dbk.m.w + eo * dbk.w_stride + (size_t)d * dbk.m.row_bytes;
#pragma unroll
    for (int u = 0; u < NS; ++u) S::load_raw(wr[r][u], wrow, min(u, steps - 1) * 64 + 16 * g);
  }
  __builtin_amdgcn_sched_barrier(0);
  // at least 2 * NS weight loads follow the copies
  lds_dma_wait_behind<2 * NS>();
  __syncthreads();
  UnpackConsts kc;
  kc.init();
  const bf16x8_t ones = mfma_ones();
  f32x4_t acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    if (u < steps) {
      const int q0 = (u * 64 + 16 * g) >> 3;
      bf16x8_t h0, h1, l0, l1;
      S::a_ops(shi + r16 * K, q0, r16, h0, h1);
      S::a_ops(slo + r16 * K, q0, r16, l0, l1);
      const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      f32x4_t xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h0, ones, z, 0, 0, 0);
      xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h1, ones, xs, 0, 0, 0);
      xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l0, ones, xs, 0, 0, 0);
      xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l1, ones, xs, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        bf16x8_t b0, b1;
        S::b_ops(wr[r][u], kc, b0, b1);
        f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h0, b0, z, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h1, b1, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l0, b0, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l1, b1, d, 0, 0, 0);
        const uint32_t sw = pair_aux ? (sr[r][u & ~1] >> (16 * (u & 1))) & 0xffffu : sr[r][u];
        const uint32_t bw = pair_aux ? (br[r][u & ~1] >> (16 * (u & 1))) & 0xffffu : br[r][u];
        S::fold(acc[r], d, xs, aux_f32<FP16>(sw), aux_f32<FP16>(bw));
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int d = rb * 128 + wave * 32 + 16 * r + r16;
    if (d >= a.D) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 4 * g + i;
      if (m < cnt) w.y[(size_t)(row0 + m) * a.D + d] = acc[r][i];
    }
  }
}

// ---------------------------------------------------------------------------
// 4b. down with the weights staged in LDS (4- and 8-bit codes, groups of 64,
//     K a multiple of 128 code bytes): 8 waves, each wave a run of 32-row
//     pairs of 16-row groups. h (hi, lo) is staged once per block (the
//     register form stages it per 128 rows), and each wave streams its rows'
//     codes batch by batch through a three-slot ring of RingSlot batches
//     (group 0 = rows 32 p + [0, 16), group 1 = rows 32 p + [16, 32) of pair
//     p), two batches in flight while one is multiplied, the ring running on
//     from one pair into the next. The sums of h over each step (the fold's
//     bias term) are formed once and kept.
//
//     One block per CU (the ring and the h tile fill its LDS), so blocks run
//     in rounds and a block's start (h copy, first batches) and end (last
//     batches multiplied, nothing in flight) are paid per block. A block over
//     a whole tile (all D rows, npw = D / 256 pairs per wave) pays them once
//     per tile (config-5 chunk: 39 us per 2048-row block against 4 x 13.1 us
//     for 512-row blocks), but 544 such blocks on 256 CUs leave most of the
//     last round idle. So the first tiles take whole-tile blocks and the last
//     kMDownSmallUnits 512-row units (npw = 2) follow them in grid order: the
//     CUs whose whole-tile blocks end first take the small ones (config-5
//     chunk: 118-119 us per layer with 512-row blocks only, 98 us so; 110 us
//     with 128 small units, 103 with 512).

constexpr int kMDownLdsRows = 512;      // rows of a small block (32 x 2 pairs x 8 waves)
constexpr int kMDownSmallUnits = 256;   // 512-row units left to small blocks (one round on 256 CUs)

template <int BITS, bool FP16>
__global__ __launch_bounds__(512, 1) void moe_down_lds_kernel(MoeArgs a, MoeMWs w, int upt) {
  constexpr int WAVES = 8, NT = WAVES * 64;
  using R = RingSlot<BITS>;
  constexpr int GU = R::GU, NB = 3;
  constexpr int NS = kMDownK / 64;      // steps at most
  constexpr int KBM = NS / GU;           // batches per pair at most
  __shared__ __align__(16) uint16_t shi[kMTok * kMDownK];
  __shared__ __align__(16) uint16_t slo[kMTok * kMDownK];
  __shared__ __align__(16) uint8_t swt[NB][WAVES][R::BYTES];
  using S = MfmaStep<BITS>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  // blocks [0, nbt) take whole tiles; then the tiles from nbt on in 512-row
  // units (upt = ceil(D / 512) per tile; the grid holds max_tiles x upt)
  const int nt = __builtin_amdgcn_readfirstlane(*w.n_tiles);
  const int units = nt * upt;
  const int nbt = units > kMDownSmallUnits ? (units - kMDownSmallUnits) / upt : 0;
  const int bid = blockIdx.x;
  int tile, rb, npw;
  if (bid < nbt) {
    tile = bid;
    rb = 0;
    npw = 2 * upt;
  } else {
    tile = nbt + (bid - nbt) / upt;
    rb = (bid - nbt) % upt;
    npw = 2;
  }
  if (tile >= nt) return;
  const int4 tr = w.tiles[tile];
  const int e = __builtin_amdgcn_readfirstlane(tr.x);
  const int row0 = __builtin_amdgcn_readfirstlane(tr.y);
  const int cnt = __builtin_amdgcn_readfirstlane(tr.z);
  const bool shared = e < 0;
  const DevBank &dbk = shared ? a.sdown : a.down;
  const int K = shared ? a.sinter : a.inter;
  const size_t eo = shared ? 0 : (size_t)e;
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  const int kbn = (K >> 6) / GU;  // batches per pair
  const int nbw = npw * kbn;      // batches of the wave
  const int jw = rb * kMDownLdsRows + wave * 32 * npw;  // the wave's first row
  const int dmax = a.D - 1;
  // the bank's fields, read here: such a load inside the ring loop would wait
  // for every copy in flight. Pair p's batch kb: rows jw + 32 p + 8 i + lane / 8
  // (i < 4) at byte 128 kb + the lane's source chunk; scale / bias words as
  // RingSlot::aux_ptr lays them out (the lane's row arl, arl1 of the pair).
  const int lr = lane >> 3;
  const uint8_t *const wb = dbk.m.w + eo * dbk.w_stride + 16 * ((lane & 7) ^ lr);
  const size_t rbytes = dbk.m.row_bytes;
  const int ng = dbk.m.ng;
  const uint16_t *ab;
  int arl, arl1;
  if constexpr (BITS == 4) {
    ab = (lane < 32 ? dbk.m.sc : dbk.m.bi) + eo * dbk.p_stride + 2 * (lane & 1);
    arl = (lane & 31) >> 1;
    arl1 = arl + 16;
  } else {
    ab = (((lane >> 4) & 1) ? dbk.m.bi : dbk.m.sc) + eo * dbk.p_stride;
    arl = 16 * (lane >> 5) + (lane & 15);
    arl1 = arl;
  }
  // the next batch to copy (uniform): index, ring slot, pair, k batch. Past the
  // wave's last batch the cursor stays there and the copy repeats that batch
  // into its own slot (the same bytes), which keeps the count of copies behind
  // every batch at 2 NI.
  const uint32_t ring0 = __builtin_amdgcn_readfirstlane(lds_addr(&swt[0][wave][0]));
  int ib = 0, is = 0, ip = 0, ik = 0;
  // the copy sources of pair ip at byte 0 of its rows, formed when the cursor
  // enters the pair
  const uint8_t *cw[4];
  const uint16_t *ca0, *ca1;
  auto set_pair = [&]() {
    const int rp = jw + 32 * ip;
#pragma unroll
    for (int i = 0; i < 4; ++i) cw[i] = wb + (size_t)min(rp + 8 * i + lr, dmax) * rbytes;
    ca0 = ab + (size_t)min(rp + arl, dmax) * ng;
    ca1 = ab + (size_t)min(rp + arl1, dmax) * ng;
  };
  set_pair();
  auto issue_next = [&]() {
    const uint32_t d = __builtin_amdgcn_readfirstlane(ring0 + (uint32_t)is * (WAVES * R::BYTES));
    const size_t o = (size_t)128 * ik;
    const uint8_t *wr[4] = {cw[0] + o, cw[1] + o, cw[2] + o, cw[3] + o};
    R::issue(d, wr, ca0 + ik * GU, ca1 + ik * GU);
    if (ib < nbw - 1) {
      ++ib;
      is = is == NB - 1 ? 0 : is + 1;
      if (++ik == kbn) {
        ik = 0;
        ++ip;
        set_pair();
      }
    }
  };
  {
    // stage h (hi, lo) of the tile's rows (physical granule P of row m holds
    // logical granule P ^ (m & 15))
    constexpr int NQ = kMTok * kMDownK / 8 / NT;
    const int gpr = K >> 3;
    auto dma = [&](int base) {
      const int pg = base + lane;
      const int m = pg / gpr, qq = swz(m, pg % gpr);
      const size_t o = (size_t)(row0 + min(m, cnt - 1)) * hmax + 8 * qq;
      lds_dma16(w.h_hi + o, shi + 8 * base);
      lds_dma16(w.h_lo + o, slo + 8 * base);
    };
    // rows from cnt on are not staged (they feed only output rows not stored)
#pragma unroll
    for (int i = 0; i < NQ; ++i)
      if (NT * i + 64 * wave < cnt * gpr) dma(NT * i + 64 * wave);
  }
  // the ring's first two batches behind the h copies (a wave with no rows
  // inside D copies clamped rows and stores nothing)
  issue_next();
  issue_next();
  lds_dma_wait_behind<2 * R::NI>();
  __syncthreads();
  UnpackConsts kc;
  kc.init();
  const bf16x8_t ones = mfma_ones();
  // sum of h over each step's 64 k (hi and lo): the fold's bias term
  f32x4_t xs[NS];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    if (u < kbn * GU) {
      bf16x8_t h0, h1, l0, l1;
      const int q0 = (u * 64 + 16 * g) >> 3;
      S::a_ops(shi + r16 * K, q0, r16, h0, h1);
      S::a_ops(slo + r16 * K, q0, r16, l0, l1);
      const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      xs[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h0, ones, z, 0, 0, 0);
      xs[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h1, ones, xs[u], 0, 0, 0);
      xs[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l0, ones, xs[u], 0, 0, 0);
      xs[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l1, ones, xs[u], 0, 0, 0);
    }
  }
  int cs = 0;  // ring slot of the batch multiplied
  for (int p = 0; p < npw; ++p) {
    f32x4_t acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kb = 0; kb < KBM; ++kb) {
      if (kb < kbn) {
        // two batches in flight behind this one
        issue_next();
        lds_dma_wait_behind<2 * R::NI>();
        const uint8_t *slot = &swt[cs][wave][0];
        cs = cs == NB - 1 ? 0 : cs + 1;
        uint32_t sw[2][GU / 2], bw[2][GU / 2];
        R::aux(slot, r16, sw, bw);
#pragma unroll
        for (int ul = 0; ul < GU; ++ul) {
          const int u = kb * GU + ul;
          const int q0 = (u * 64 + 16 * g) >> 3;
          bf16x8_t h0, h1, l0, l1;
          S::a_ops(shi + r16 * K, q0, r16, h0, h1);
          S::a_ops(slo + r16 * K, q0, r16, l0, l1);
          const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            SkRaw<BITS> rw;
            bf16x8_t b0, b1;
            R::raw(slot, m, ul, r16, g, rw);
            S::b_ops(rw, kc, b0, b1);
            f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h0, b0, z, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h1, b1, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l0, b0, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l1, b1, d, 0, 0, 0);
            S::fold(acc[m], d, xs[u], R::template word<FP16>(sw[m], ul),
                    R::template word<FP16>(bw[m], ul));
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int d = jw + 32 * p + 16 * m + r16;
      if (d < a.D) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 4 * g + i;
          if (t < cnt) w.y[(size_t)(row0 + t) * a.D + d] = acc[m][i];
        }
      }
    }
  }
  lds_dma_wait();  // no copy into LDS outlives the block
}

// ---------------------------------------------------------------------------
// 5. rank-ordered combine (logan-qwen4/src/lib.rs:8692-8711)

constexpr int kMCombRanks = 16;  // ranks' rows in flight per round (top-k up to 16 in one)

__global__ __launch_bounds__(256) void moe_mcombine_kernel(MoeArgs a, MoeMWs w) {
  // four consecutive outputs per thread (D % 4 == 0)
  const int D4 = a.D >> 2;
  // with D a multiple of 256 a wave's 64 outputs share one token, whose route
  // words are then read once per wave
  const bool wave_tok = (D4 & 63) == 0;
  const long long n = (long long)a.B * D4;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
    int t = (int)(i / D4);
    if (wave_tok) t = __builtin_amdgcn_readfirstlane(t);
    const int d = 4 * (int)(i - (long long)t * D4);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    // the shared expert's row and gate do not depend on the routes: in flight
    // with the first round
    float gs = 0.f;
    float4 vs = make_float4(0.f, 0.f, 0.f, 0.f);
    if (a.sdown.m.w) {
      gs = w.gs[t];
      vs = *reinterpret_cast<const float4 *>(w.y + ((size_t)a.B * a.k + t) * a.D + d);
    }
    // a round's routed rows and weights, then all its rows' outputs in
    // flight together, added in rank order (logan-qwen4/src/lib.rs:8692-8711)
    for (int r0 = 0; r0 < a.k; r0 += kMCombRanks) {
      int gp[kMCombRanks];
      float wt[kMCombRanks];
      float4 yv[kMCombRanks];
#pragma unroll
      for (int j = 0; j < kMCombRanks; ++j) {
        gp[j] = 0;
        wt[j] = 0.f;
        if (r0 + j < a.k) {
          gp[j] = w.gpos[t * a.k + r0 + j];
          wt[j] = w.topk_w[t * a.k + r0 + j];
        }
      }
#pragma unroll
      for (int j = 0; j < kMCombRanks; ++j)
        if (r0 + j < a.k) yv[j] = *reinterpret_cast<const float4 *>(w.y + (size_t)gp[j] * a.D + d);
#pragma unroll
      for (int j = 0; j < kMCombRanks; ++j) {
        if (r0 + j < a.k) {
          acc.x = fmaf(yv[j].x, wt[j], acc.x);
          acc.y = fmaf(yv[j].y, wt[j], acc.y);
          acc.z = fmaf(yv[j].z, wt[j], acc.z);
          acc.w = fmaf(yv[j].w, wt[j], acc.w);
        }
      }
    }
    if (a.sdown.m.w) {
      acc.x = fmaf(vs.x, gs, acc.x);
      acc.y = fmaf(vs.y, gs, acc.y);
      acc.z = fmaf(vs.z, gs, acc.z);
      acc.w = fmaf(vs.w, gs, acc.w);
    }
    const size_t o = (size_t)t * a.D + d;
    if (a.out_f32) {
      *reinterpret_cast<float4 *>(reinterpret_cast<float *>(a.out) + o) = acc;
    } else {
      uint2 p;
      p.x = f32_to_bf16_rne(acc.x) | (f32_to_bf16_rne(acc.y) << 16);
      p.y = f32_to_bf16_rne(acc.z) | (f32_to_bf16_rne(acc.w) << 16);
      *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(a.out) + o) = p;
    }
  }
}

// ---------------------------------------------------------------------------

static bool mbank_ok(const DevBank &b) {
  const DevMat &m = b.m;
  if (m.bits < 4 || m.bits > 8 || m.bits == 7) return false;
  if (m.gs <= 0 || m.gs % 64 != 0 || m.I % m.gs != 0) return false;
  const uintptr_t need = m.bits == 4 ? 7 : m.bits == 8 ? 15 : 3;
  if ((reinterpret_cast<uintptr_t>(m.w) & need) != 0 || (m.row_bytes & (long long)need) != 0) return false;
  if ((b.w_stride & (long long)need) != 0) return false;
  // scale/bias runs are read as 4- or 8-byte words
  if (((reinterpret_cast<uintptr_t>(m.sc) | reinterpret_cast<uintptr_t>(m.bi)) & 7) != 0) return false;
  if ((b.p_stride & 7) != 0) return false;
  return true;
}

bool moe_mfma_supported(const MoeArgs &a) {
  if (a.B <= 0 || (long long)a.B * a.k > kMMaxSlots || a.E > kMMaxE) return false;
  // the combine writes four outputs per store
  if ((reinterpret_cast<uintptr_t>(a.out) & (a.out_f32 ? 15 : 7)) != 0) return false;
  // whole batches of MOE_GU steps per LDS chunk
  if (a.D % (64 * MOE_GU) != 0 || (a.D > kMChunk && a.D % kMChunk != 0)) return false;
  if (a.inter % 128 != 0 || a.inter > kMDownK) return false;
  if (!mbank_ok(a.gate) || !mbank_ok(a.up) || !mbank_ok(a.down)) return false;
  // one scale/bias type per pass (gate/up and the shared gate/up; down and
  // the shared down)
  if (a.up.m.fp16 != a.gate.m.fp16) return false;
  if (a.sgate.m.w && (a.sgate.m.fp16 != a.gate.m.fp16 || a.sup.m.fp16 != a.gate.m.fp16 ||
                      a.sdown.m.fp16 != a.down.m.fp16))
    return false;
  if (a.up.m.bits != a.gate.m.bits || a.down.m.bits != a.gate.m.bits) return false;
  if (a.sgate.m.w) {
    if (a.sinter % 128 != 0 || a.sinter > kMDownK) return false;
    if (!mbank_ok(a.sgate) || !mbank_ok(a.sup) || !mbank_ok(a.sdown)) return false;
    if (a.sgate.m.bits != a.gate.m.bits || a.sup.m.bits != a.gate.m.bits ||
        a.sdown.m.bits != a.gate.m.bits)
      return false;
  }
  return true;
}

template <int BITS, int WV>
static hipError_t moe_gateup_launch(const MoeArgs &a, const MoeMWs &w, hipStream_t st) {
  const int kmax = a.inter > a.sinter ? a.inter : a.sinter;
  {
    const int ipt = (kmax + 16 * WV - 1) / (16 * WV);
    // one aligned load of GU consecutive u16 scale (bias) words per batch
    const bool gs64 = a.gate.m.gs == 64 && (!a.sgate.m.w || a.sgate.m.gs == 64) &&
                      a.gate.m.ng % (MOE_GU < 4 ? 4 : MOE_GU) == 0;
    const dim3 grid(w.max_tiles * ipt), block(WV * 64);
    if constexpr (WV == 8 && (BITS == 4 || BITS == 8)) {
      // the large-batch shape with the weights staged in LDS (groups of 64)
      if (gs64 && a.gate.m.gs == 64) {
        if (a.gate.m.fp16) hipLaunchKernelGGL((moe_gateup_lds_kernel<BITS, true>), grid, block, 0, st, a, w, ipt);
        else hipLaunchKernelGGL((moe_gateup_lds_kernel<BITS, false>), grid, block, 0, st, a, w, ipt);
        return hipGetLastError();
      }
    }
    if (a.gate.m.fp16) {
      if (gs64) hipLaunchKernelGGL((moe_gateup_mfma_kernel<BITS, MOE_GU, WV, true, true>), grid, block, 0, st, a, w, ipt);
      else hipLaunchKernelGGL((moe_gateup_mfma_kernel<BITS, MOE_GU, WV, false, true>), grid, block, 0, st, a, w, ipt);
    } else {
      if (gs64) hipLaunchKernelGGL((moe_gateup_mfma_kernel<BITS, MOE_GU, WV, true, false>), grid, block, 0, st, a, w, ipt);
      else hipLaunchKernelGGL((moe_gateup_mfma_kernel<BITS, MOE_GU, WV, false, false>), grid, block, 0, st, a, w, ipt);
    }
  }
  return hipGetLastError();
}

template <int BITS>
static hipError_t moe_down_launch(const MoeArgs &a, const MoeMWs &w, hipStream_t st) {
  if constexpr (BITS == 4 || BITS == 8) {
    // the large-batch shape with the weights staged in LDS: groups of 64, K a
    // multiple of one batch (128 code bytes) on the routed and shared experts
    constexpr int KB = 128 * 8 / BITS;
    const bool lds = a.B > kMGuSmallB && a.down.m.gs == 64 && a.inter % KB == 0 &&
                     (!a.sdown.m.w || (a.sdown.m.gs == 64 && a.sinter % KB == 0));
    if (lds) {
      const int upt = (a.D + kMDownLdsRows - 1) / kMDownLdsRows;
      if (a.down.m.fp16)
        hipLaunchKernelGGL((moe_down_lds_kernel<BITS, true>), dim3(w.max_tiles * upt), dim3(512), 0, st, a, w, upt);
      else
        hipLaunchKernelGGL((moe_down_lds_kernel<BITS, false>), dim3(w.max_tiles * upt), dim3(512), 0, st, a, w, upt);
      return hipGetLastError();
    }
  }
  const int ipt = (a.D + 127) / 128;
  if (a.down.m.fp16)
    hipLaunchKernelGGL((moe_down_mfma_kernel<BITS, true>), dim3(w.max_tiles * ipt), dim3(256), 0, st, a, w, ipt);
  else
    hipLaunchKernelGGL((moe_down_mfma_kernel<BITS, false>), dim3(w.max_tiles * ipt), dim3(256), 0, st, a, w, ipt);
  return hipGetLastError();
}

template <int BITS>
static int moe_mfma_launch_bits(const MoeArgs &a, const MoeMWs &w, hipStream_t st) {
  const hipError_t ge = a.B <= kMGuSmallB ? moe_gateup_launch<BITS, 4>(a, w, st)
                                          : moe_gateup_launch<BITS, MOE_GU_WAVES>(a, w, st);
  if (ge != hipSuccess) return -1;
  if (moe_down_launch<BITS>(a, w, st) != hipSuccess) return -1;
  {
    long long n = (long long)a.B * (a.D >> 2);
    long long blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(moe_mcombine_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a, w);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  return 1;
}

// a.sinter is 0 when there is no shared expert; the caller has validated the
// banks against the block geometry.
int launch_moe_mfma(const MoeArgs &a, hipStream_t st) {
  if (!moe_mfma_supported(a)) return 0;
  if (a.ws_bytes < moe_mfma_workspace_bytes(a.B, a.D, a.inter, a.sinter, a.E, a.k)) return 0;
  const MoeMWs w = moe_mws_layout(a.ws, a.B, a.D, a.inter, a.sinter, a.E, a.k);
  const dim3 rgrid((a.B + 3) / 4);
  if (a.logits_f32) {
    if (a.E <= 512) hipLaunchKernelGGL((moe_mroute_kernel<8, true>), rgrid, dim3(256), 0, st, a, w);
    else hipLaunchKernelGGL((moe_mroute_kernel<16, true>), rgrid, dim3(256), 0, st, a, w);
  } else {
    if (a.E <= 512) hipLaunchKernelGGL((moe_mroute_kernel<8, false>), rgrid, dim3(256), 0, st, a, w);
    else hipLaunchKernelGGL((moe_mroute_kernel<16, false>), rgrid, dim3(256), 0, st, a, w);
  }
  if (hipGetLastError() != hipSuccess) return -1;
  hipLaunchKernelGGL(moe_mgroup_kernel, dim3(1), dim3(kMGroupThreads), 0, st, a, w);
  if (hipGetLastError() != hipSuccess) return -1;
  switch (a.gate.m.bits) {
    case 4: return moe_mfma_launch_bits<4>(a, w, st);
    case 5: return moe_mfma_launch_bits<5>(a, w, st);
    case 6: return moe_mfma_launch_bits<6>(a, w, st);
    default: return moe_mfma_launch_bits<8>(a, w, st);
  }
}

}  // namespace lh
