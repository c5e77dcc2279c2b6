// Single-launch routed-MoE block for one token (B = 1), gfx950.
//
// One kernel, two kinds of blocks, one hand-off:
//
//   A blocks (first in the grid): each wave owns UA rows j of one expert slot
//   (rank r < k of the route, or the shared expert) and computes
//   h[slot][j] = silu(gate_j . x) * (up_j . x) for them. It stores each h as
//   a 64-bit (value, tag) pair, where tag names the launch, and adds one
//   arrival on the slot's counters right behind the stores. Nothing on the
//   A side waits for its stores to land.
//
//   B blocks: a block owns ROWS_B output rows d; wave w owns slots w and
//   w + 8 for all of them. Each wave issues the shared slot's down-row loads
//   and the shared-expert gate loads before the route is known and the routed
//   down rows right after it, so they stream from HBM while A runs; the last wave
//   computes the shared-expert scalar gate sigmoid(se_g . x). While A runs,
//   each wave turns its down codes into exact f16 pairs. Per slot, a wave
//   waits for the slot's arrivals, reads the slot's h pairs until every tag
//   is this launch's (an arrival can overtake the stores it counts) and forms
//   the down products of its rows, one f16 x f32 fma per code. The
//   block then combines them per row in rank order:
//   out[d] = sum_{r<k} w_r * (down_r . h_r)[d] + gs * (down_shared . h_shared)[d]
//   (logan-qwen4/src/lib.rs:8692-8711, :7597-7759).
//
// Weights and their scale/bias words are read with non-temporal loads: they
// are read once per launch, and kept out of L2 they do not displace what the
// launch reads again (logits, x, the hand-off lines, its code): 14.1 -> 13.3
// us per config-3 layer.
//
// Routing, from the router logits, bf16 or f32 (top-k with the key (logit
// desc, index asc): per-lane sorted keys, k rounds of a DPP wave max, and the
// reference's probability arithmetic instead where a tie in probability could
// reorder it): each A block's wave 0 selects its own slot's expert, so no A
// block waits before streaming weights. B block 0's wave 0 selects every rank
// and publishes the route (expert and combine weight per rank) as tagged
// 16-byte records; the other B blocks read them, their routed down-row loads
// behind it (the shared slot's are issued first). One selecting B wave
// instead of one per B block: the 256 B waves' selection rounds competed for
// the CUs with the A blocks' routing (13.33 -> 13.21 us per config-3 layer).
//
// Progress: A blocks never wait on another block, and B block 0 waits for
// none before it publishes the route. Workgroups are dispatched in ID order,
// every A block precedes every B block and B block 0 the other B blocks, so
// a block can only be resident after the blocks it waits for were
// dispatched: the waits always end. They are
// also bounded: after kSpinLimit polls a B wave stops waiting, raises the
// sticky error word and its block finishes without writing its rows (the
// host can read the word with logan_hip_moe_sync_errors(); results of later
// launches are then not guaranteed either).
//
// Hand-off without L2 maintenance: h pairs and counters are written and
// read only with device-scope (sc1) relaxed atomics / loads, which are
// coherent across the XCDs' L2s. An h pair's tag names its launch, so pairs
// left by earlier launches never pass the tag check. An agent-scope
// release/acquire fence would instead write back / invalidate the whole L2
// of each XCD per wave (buffer_wbl2 / buffer_inv), which measured tens of
// microseconds per launch here.
//
// Launch numbers without a completion count: every block takes a ticket
// from one of kTickets 64-bit counters (block b from counter b % kTickets);
// the launch number is ticket >> kTicketShift. The block that takes a
// counter's last ticket of the launch adds what is left to the next multiple
// of 2^kTicketShift, and counters that no block of a small grid uses are
// advanced by one launch as well, so every block of the next launch again
// reads one launch number. Launches of this kernel on one device must
// therefore not overlap: the next launch starts only after this one has
// ended, its realigning atomics included (the launcher orders launches that
// come on different streams, see fused_launch).
// Arrival counters come in two sets used by alternate launches; each launch
// zeroes the set the next one will use. All of this lives in module-scope
// device memory (zero when the code object loads), so no launch needs a
// memset and nothing is left to count once the outputs are written.
#include <mutex>

#include "affine_dev.hpp"
#include "lh_internal.hpp"
#include "route_dev.hpp"

namespace lh {

constexpr int kFusedMaxSlots = 12;  // k + 1 (routed + shared)
// Each slot's arrivals are spread over kSubCtrs counters (the i-th A block of
// a slot arrives on counter i % kSubCtrs), each on its own 256-byte line:
// same-address atomics serialise at the memory side (~40 ns each measured
// here). Launch tickets likewise go over kTickets counters.
constexpr int kSubCtrs = 4;
constexpr int kLine = 64;  // u32 per 256-byte line
constexpr int kTickets = 64;
constexpr int kTicketShift = 20;  // tickets per launch and counter stay below 2^20
struct FusedSync {
  unsigned long long tk[kTickets][kLine / 2];
  uint32_t ctr[2][kFusedMaxSlots][kSubCtrs][kLine];
  uint32_t error[kLine];
};
__device__ FusedSync g_fused_sync;

constexpr int kBufWord3 = 0x00020000;  // gfx9 raw buffer resource, 32-bit data format
constexpr int kCpolSc1 = 16;           // cache policy: device scope (sc1)
// h pairs rotate over kSlices workspace slices (slice = launch % kSlices), so
// a line that an XCD's L2 still holds from an earlier launch is many launches
// old; B reads pairs through L2 first and re-reads with sc1 on a stale tag.
constexpr int kSlices = 16;
typedef float float4v __attribute__((ext_vector_type(4)));
constexpr uint32_t kSpinLimit = 1u << 20;

__device__ __forceinline__ uint32_t ld_agent(uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------- stage timeline
// A build with -DLOGAN_HIP_TIMELINE records, per block, s_memrealtime stamps
// (100 MHz) of its stages for the last two launches (slot = launch number &
// 1), read back with logan_hip_fused_timeline(). A blocks: start, route
// known, gate/up weights consumed (wave 0), arrival added (last wave). B
// blocks: start, route known, then the latest wave's arrivals seen, h read
// and down products formed, and the end. Default builds contain none of it.
#ifdef LOGAN_HIP_TIMELINE
// one 128-byte line per block (blocks sharing a line slowed the launch by ~5 us)
constexpr int kTlBlocks = 1024, kTlStamps = 16;
__device__ unsigned long long g_fused_tl[2][kTlBlocks][kTlStamps];
#define TL_NOW() __builtin_amdgcn_s_memrealtime()
#define TL_PUT(lid, i, v)                                                      \
  do {                                                                         \
    if (blockIdx.x < (unsigned)kTlBlocks) g_fused_tl[(lid) & 1][blockIdx.x][i] = (v); \
  } while (0)
// stamps go to LDS at once (held in registers they would spill)
#define TL_LDS                                 \
  __shared__ unsigned long long s_tl[3][kWaves]; \
  __shared__ unsigned long long s_tlb[3]
#define TL_BLOCK(i)                              \
  do {                                           \
    if (threadIdx.x == 0) s_tlb[i] = TL_NOW();   \
  } while (0)
#define TL_WAVE(i) \
  do {             \
    if (lane == 0) s_tl[i][wave] = TL_NOW(); \
  } while (0)
#define TL_PUT_WAVES(lid, i, j)                                              \
  do {                                                                       \
    unsigned long long m_ = 0;                                               \
    for (int w_ = 0; w_ < kWaves; ++w_) m_ = s_tl[j][w_] > m_ ? s_tl[j][w_] : m_; \
    TL_PUT(lid, i, m_);                                                      \
  } while (0)
#else
#define TL_NOW() 0ull
#define TL_PUT(lid, i, v) ((void)0)
#define TL_LDS
#define TL_BLOCK(i) ((void)0)
#define TL_WAVE(i) ((void)0)
#define TL_PUT_WAVES(lid, i, j) ((void)0)
#endif

// ---------------------------------------------------------------- kernel

struct FusedGeom {
  int k;           // routed experts
  int slots;       // k + (shared ? 1 : 0)
  int wpr;         // A waves per routed slot
  int wps;         // A waves for the shared slot
  int nA_blocks;
  int nB_blocks;
};

#ifndef FUSED_PASSES
#define FUSED_PASSES 2
#endif
constexpr int kWaves = 8;  // waves per block (512 threads)

// gate/up rows per A wave: fewer where a lane's weight registers would spill
__host__ __device__ constexpr int fused_ua(int bits, int cpla) {
  return (bits == 8 || (cpla == 2 && bits >= 5)) ? 2 : 4;
}
constexpr int kSlotsPerWave = (kFusedMaxSlots + kWaves - 1) / kWaves;  // B: slots w, w + 8

// One down-row chunk and its raw scale/bias. Branch-free: a dead lane loads
// row 0 / chunk 0 of the same expert, and its scale and bias are zeroed where
// they are used, so the loads of all slots and passes stay in flight together.
template <int BITS>
__device__ __forceinline__ void load_down(uint32_t (&w)[BITS], uint32_t &scr, uint32_t &bir,
                                          const DevBank &bd, int e, int d, int lb, bool live) {
  const int dd = live ? d : 0, ll = live ? lb : 0;
  load_chunk<BITS, true>(w, bd.m.w + (size_t)e * bd.w_stride + (size_t)dd * bd.m.row_bytes +
                                (size_t)ll * (4 * BITS));
  const size_t p = (size_t)e * bd.p_stride + (size_t)dd * bd.m.ng + ll / (bd.m.gs >> 5);
  scr = ld_stream<uint16_t, true>(bd.m.sc + p);
  bir = ld_stream<uint16_t, true>(bd.m.bi + p);
}

// The down products of one slot from f32 h and packed codes converted at
// use (the instantiations without room for pre-converted codes): h goes
// through the wave's LDS row to chunk-per-lane, then
// sum_k (code_k * sc + bi) * h_k = sc * sum_k code_k h_k + bi * sum_k h_k.
template <int BITS, int PASSES, int RPP, int LANESB, int VPL, int SLOTS>
__device__ __forceinline__ void down_slot_f32(const MoeArgs &a, int s, bool sh, int d0, int lb, int rsub,
                                              float *row, const float (&hv)[VPL],
                                              const uint32_t (&wv)[PASSES][BITS], const uint32_t (&rsc)[PASSES],
                                              const uint32_t (&rbi)[PASSES], float (&s_y)[RPP * PASSES][SLOTS]) {
  const int lane = threadIdx.x & 63;
  const int K = sh ? a.sinter : a.inter;
#pragma unroll
  for (int v = 0; v < VPL; v += 4)
    *reinterpret_cast<float4 *>(row + VPL * lane + v) = make_float4(hv[v], hv[v + 1], hv[v + 2], hv[v + 3]);
  __builtin_amdgcn_wave_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  float xf[32];
#pragma unroll
  for (int v = 0; v < 32; v += 4) {
    const float4 f = *reinterpret_cast<const float4 *>(row + 32 * lb + v);
    xf[v] = f.x; xf[v + 1] = f.y; xf[v + 2] = f.z; xf[v + 3] = f.w;
  }
  __builtin_amdgcn_wave_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  float xt[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) xt[v] = xf[v] + xf[v + 16];
#pragma unroll
  for (int w = 8; w > 0; w >>= 1)
#pragma unroll
    for (int v = 0; v < w; ++v) xt[v] += xt[v + w];
  const float xs = xt[0];
  const DevBank &bd = sh ? a.sdown : a.down;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const bool live = d0 + p * RPP + rsub < a.D && lb < (K >> 5);
    const float sc = live ? aux_to_f32(rsc[p], bd.m.fp16) : 0.f;
    const float bi = live ? aux_to_f32(rbi[p], bd.m.fp16) : 0.f;
    float v = fmaf(sc, codes_dot<BITS>(wv[p], xf), bi * xs);
    v = group_sum_f32<LANESB>(v);
    if (lb == 0) s_y[p * RPP + rsub][s] = v;
  }
}

// VPL consecutive (value, tag) pairs from byte offset off; positions at or
// beyond n (n may be <= 0) read as 0 and are not checked. True when every
// checked tag is `tag`.
template <int VPL, int CPOL>
__device__ __forceinline__ bool read_pairs(__amdgpu_buffer_rsrc_t rs, int off, int n,
                                           uint32_t tag, float (&hv)[VPL]) {
  bool ok = true;
#pragma unroll
  for (int v = 0; v < VPL / 2; ++v) {
    const uint4 q =
        __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * v, 0, CPOL));
    ok = ok && (2 * v >= n || q.y == tag) && (2 * v + 1 >= n || q.w == tag);
    hv[2 * v] = 2 * v < n ? __uint_as_float(q.x) : 0.f;
    hv[2 * v + 1] = 2 * v + 1 < n ? __uint_as_float(q.z) : 0.f;
  }
  return ok;
}

// This block's ticket (thread 0; the value is used later, so the atomic's
// round trip overlaps the block's first loads).
__device__ __forceinline__ unsigned long long take_ticket() {
  return __hip_atomic_fetch_add(&g_fused_sync.tk[blockIdx.x % kTickets][0], 1ull, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
}

// Launch number from the ticket; the holder of a counter's last ticket of
// this launch realigns the counter for the next launch, and counters no
// block of a small grid uses are advanced by one launch too (counter
// j >= gridDim.x by block j mod gridDim.x), so all counters stay in step.
__device__ __forceinline__ uint32_t launch_number(unsigned long long t) {
  const int j = blockIdx.x % kTickets;
  const unsigned long long n = (gridDim.x - 1 - j) / kTickets + 1;  // blocks on counter j
  if ((t & ((1ull << kTicketShift) - 1)) == n - 1)
    __hip_atomic_fetch_add(&g_fused_sync.tk[j][0], (1ull << kTicketShift) - n, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  for (int u = blockIdx.x + gridDim.x; u < kTickets; u += gridDim.x)
    __hip_atomic_fetch_add(&g_fused_sync.tk[u][0], 1ull << kTicketShift, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  return (uint32_t)(t >> kTicketShift);
}

// tag of a launch's h pairs: odd, so zeroed memory never passes, and mixed
// with a constant so that the small integers and ordinary floats a
// workspace may hold from earlier use do not look like a recent launch's tag
constexpr uint32_t kTagMix = 0x6A09E666u;  // even: the tag stays odd
__device__ __forceinline__ uint32_t launch_tag(uint32_t lid) { return ((lid << 1) | 1u) ^ kTagMix; }

// expected arrivals on sub-counter q of a slot with n A waves
__device__ __forceinline__ uint32_t sub_need(int n, int q) {
  return (uint32_t)(n / kSubCtrs + (q < n % kSubCtrs ? 1 : 0));
}

template <int BITS, int CPLA, int LANESB, int KPL, bool LF>
// LF: f32 router logits (64-bit selection keys), else bf16.
// Two 8-wave blocks per CU (4 waves per SIMD, <= 128 VGPRs) so all A and B
// blocks of a config-3 launch are resident at once; the D > 2048 variants
// hold two x chunks per lane and would spill there.
__global__ __launch_bounds__(kWaves * 64, CPLA == 1 ? 4 : 2) void moe_fused_b1_kernel(MoeArgs a, FusedGeom g) {
  constexpr int UA = fused_ua(BITS, CPLA);     // rows of gate (and of up) per A wave
  constexpr int RPP = 64 / LANESB;            // B rows per pass of a wave
  constexpr int PASSES = FUSED_PASSES;        // B passes (rows held per lane, per slot)
  constexpr int ROWS_B = RPP * PASSES;        // output rows per B block
  constexpr int VPL = LANESB / 2;             // h pairs per lane when reading a slot
  __shared__ __align__(16) float s_hv[kWaves][32 * LANESB];
  __shared__ float s_y[ROWS_B][kFusedMaxSlots];
  __shared__ uint32_t s_to[kWaves];
  __shared__ uint32_t s_sel[kFusedMaxSlots];  // route keys, computed once per block
  __shared__ float s_w[kFusedMaxSlots];       // B: combine weights by rank
  __shared__ __align__(16) uint32_t s_xp[64 * CPLA][16];  // A: x pairs per chunk
  __shared__ __align__(16) float s_xs[64 * CPLA][kWaves];  // A: partial sums of x
  __shared__ __align__(16) float s_xsp[64 * CPLA][kWaves]; // A: partial sums of x' (pairs)
  __shared__ uint32_t s_left;  // A: waves of the block still running
  __shared__ uint32_t s_lid;   // launch number
  __shared__ uint32_t s_rto;   // B: the route did not arrive
  __shared__ float s_gsig;
  TL_LDS;

  const int lane = threadIdx.x & 63;
  // wave-uniform for the compiler too, so per-slot bank selection and
  // addressing stay scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  using RK = WaveKeys<KPL, LF>;
  using Key = typename RK::K;
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  const int C = a.D >> 5;
  UnpackConsts kc;
  kc.init();

  if ((int)blockIdx.x < g.nA_blocks) {
    // ------------------------------------------------------------ phase A
    TL_BLOCK(0);
    const int item = blockIdx.x * kWaves + wave;
    const bool shared = item >= g.k * g.wpr;
    const int slot = shared ? g.k : item / g.wpr;
    const int jb = shared ? item - g.k * g.wpr : item % g.wpr;
    const int rows = shared ? a.sinter : a.inter;

    unsigned long long tk = 0;
    if (threadIdx.x == 0) tk = take_ticket();
    // every wave of an A block serves the same slot: wave 0 routes for all
    RK rk;
    if (!shared && wave == 0) rk.load(a.logits, a.E);
    // x does not depend on the route: in flight together with the logits
    uint4 xq[CPLA][4];
#pragma unroll
    for (int i = 0; i < CPLA; ++i) {
      const int c = lane + 64 * i;
      const uint4 *src = reinterpret_cast<const uint4 *>(a.x + 32 * (c < C ? c : 0));
#pragma unroll
      for (int v = 0; v < 4; ++v) xq[i][v] = src[v];
    }
    if (threadIdx.x == 0) s_left = kWaves;
    // x as pre-scaled bf16 pairs, converted once per block: wave w converts
    // pairs 2w and 2w+1 of every chunk into LDS, with its partial sums
#pragma unroll
    for (int i = 0; i < CPLA; ++i) {
      const int c = lane + 64 * i;
      const bool ok = c < C;
      uint32_t xb[32];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint4 q = xq[i][v];
        xb[8 * v + 0] = q.x & 0xffffu; xb[8 * v + 1] = q.x >> 16;
        xb[8 * v + 2] = q.y & 0xffffu; xb[8 * v + 3] = q.y >> 16;
        xb[8 * v + 4] = q.z & 0xffffu; xb[8 * v + 5] = q.z >> 16;
        xb[8 * v + 6] = q.w & 0xffffu; xb[8 * v + 7] = q.w >> 16;
      }
      // (pair index compile-time in each unrolled body: no dynamic register indexing)
#pragma unroll
      for (int pp = 0; pp < 16; pp += 2) {
        if ((pp >> 1) == wave) {
          uint32_t w0, w1;
          float s0, sp0, s1, sp1;
          xpair_bf16<BITS>(xb, pp, w0, s0, sp0);
          xpair_bf16<BITS>(xb, pp + 1, w1, s1, sp1);
          s_xp[c][pp] = ok ? w0 : 0u;
          s_xp[c][pp + 1] = ok ? w1 : 0u;
          s_xs[c][wave] = ok ? s0 + s1 : 0.f;
          s_xsp[c][wave] = ok ? sp0 + sp1 : 0.f;
        }
      }
    }
    if (!shared && wave == 0) {
      int ex = -1;
      if constexpr (LF) {
        // 32-bit keys first (route_dev.hpp: select_fast / fast_ok)
        uint32_t fs[kFusedMaxSlots + 1];
        rk.select_fast(a.E, slot + 1, fs);
        float v, m;
        if (rk.fast_ok(fs, slot, v, m)) {
          uint32_t ks = fs[0];
#pragma unroll
          for (int r = 1; r < kFusedMaxSlots; ++r) ks = r == slot ? fs[r] : ks;
          ex = RK::expert32(ks);
        }
      }
      if (ex < 0) {
      Key sel[kFusedMaxSlots];
      rk.select(a.E, slot + 1, sel);
      Key mine = sel[0];
#pragma unroll
      for (int r = 1; r < kFusedMaxSlots; ++r) mine = r == slot ? sel[r] : mine;
      ex = RK::expert(mine);
      // a probability tie the logit order cannot see (route_dev.hpp): this
      // slot's rank then comes from the reference's own arithmetic
      const float m = RK::logit(sel[0]), ls = RK::logit(mine);
      if (LF || !bf16_rank_tie_free(m, ls)) {
        // consecutive selected ranks checked lane-parallel (lane r: ranks r,
        // r + 1), the unselected keys per lane
        Key kr = 0;
#pragma unroll
        for (int r = 0; r < kFusedMaxSlots; ++r) kr = lane == r ? sel[r] : kr;
        const float lr = RK::logit(kr), lnext = __shfl(lr, (lane + 1) & 63, 64);
        bool cand = lane < slot && tie_pair(lr, lnext, m);
#pragma unroll
        for (int i = 0; i < KPL; ++i)
          cand = cand || (rk.key[i] != Key(0) && tie_other(RK::logit(rk.key[i]), ls, m));
        if (__any(cand) || tie_global(m, ls)) {
          const RouteLane rl = route_exact<KPL, LF>(a.logits, 0, a.E, a.k);
          ex = __builtin_amdgcn_readlane(rl.idx, slot);
        }
      }
      }
      if (lane == 0) s_sel[0] = 0xffffu - (uint32_t)ex;
    }
    if (threadIdx.x == 0) s_lid = launch_number(tk);
    __syncthreads();
    int e = shared ? 0 : sel_expert(__builtin_amdgcn_readfirstlane(s_sel[0]));
    if (!shared && a.nmap) {  // the expert's block in an expert cache's arena
      bool miss = false;
      e = moe_bank_index<false>(a, e, miss);
      if (miss && threadIdx.x == 0)
        __hip_atomic_fetch_or(&g_fused_sync.error[0], 8u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const uint32_t lid = __builtin_amdgcn_readfirstlane(s_lid);
    TL_BLOCK(1);
    // bank fields copied once (scalar) rather than re-read per use
    const DevMat gm = shared ? a.sgate.m : a.gate.m;
    const DevMat um = shared ? a.sup.m : a.up.m;
    const long long gws = shared ? a.sgate.w_stride : a.gate.w_stride;
    const long long uws = shared ? a.sup.w_stride : a.up.w_stride;
    const long long gps = shared ? a.sgate.p_stride : a.gate.p_stride;
    const long long ups = shared ? a.sup.p_stride : a.up.p_stride;
    const uint8_t *gw = gm.w + (size_t)e * gws;
    const uint8_t *uw = um.w + (size_t)e * uws;
    const uint16_t *gsc = gm.sc + (size_t)e * gps;
    const uint16_t *gbi = gm.bi + (size_t)e * gps;
    const uint16_t *usc = um.sc + (size_t)e * ups;
    const uint16_t *ubi = um.bi + (size_t)e * ups;
    const int j0 = jb * UA;
    const int gsh = __builtin_ctz(gm.gs >> 5);  // group sizes are 32 * 2^n

    // branch-free loads (clamped row / chunk; dead lanes get zero scale and
    // bias where they are used), the scale/bias words before the codes: loads
    // complete in issue order, so row u's products wait only for its chunks
    uint32_t wg[UA][CPLA][BITS], wu[UA][CPLA][BITS];
    uint32_t rsg[UA][CPLA], rbg[UA][CPLA], rsu[UA][CPLA], rbu[UA][CPLA];
#pragma unroll
    for (int u = 0; u < UA; ++u)
#pragma unroll
      for (int i = 0; i < CPLA; ++i) {
        const int j = min(j0 + u, rows - 1), c = min(lane + 64 * i, C - 1);
        const size_t p = (size_t)j * gm.ng + (c >> gsh);
        rsg[u][i] = ld_stream<uint16_t, true>(gsc + p);
        rbg[u][i] = ld_stream<uint16_t, true>(gbi + p);
        rsu[u][i] = ld_stream<uint16_t, true>(usc + p);
        rbu[u][i] = ld_stream<uint16_t, true>(ubi + p);
      }
#pragma unroll
    for (int u = 0; u < UA; ++u)
#pragma unroll
      for (int i = 0; i < CPLA; ++i) {
        const int j = min(j0 + u, rows - 1), c = min(lane + 64 * i, C - 1);
        load_chunk<BITS, true>(wg[u][i], gw + (size_t)j * gm.row_bytes + (size_t)c * (4 * BITS));
        load_chunk<BITS, true>(wu[u][i], uw + (size_t)j * um.row_bytes + (size_t)c * (4 * BITS));
      }
    const uint32_t tag = launch_tag(lid);
    // keep every load above issued before any of their consumers
    __builtin_amdgcn_sched_barrier(0);
    float pg[UA], pu[UA];
#pragma unroll
    for (int u = 0; u < UA; ++u) pg[u] = pu[u] = 0.f;
#pragma unroll
    for (int i = 0; i < CPLA; ++i) {
      const int c = lane + 64 * i;
      uint32_t xp[16];
#pragma unroll
      for (int v = 0; v < 16; v += 4) {
        const uint4 t = *reinterpret_cast<const uint4 *>(&s_xp[c][v]);
        xp[v] = t.x; xp[v + 1] = t.y; xp[v + 2] = t.z; xp[v + 3] = t.w;
      }
      const float4 s0 = *reinterpret_cast<const float4 *>(&s_xs[c][0]);
      const float4 s1 = *reinterpret_cast<const float4 *>(&s_xs[c][4]);
      const float4 q0 = *reinterpret_cast<const float4 *>(&s_xsp[c][0]);
      const float4 q1 = *reinterpret_cast<const float4 *>(&s_xsp[c][4]);
      const float xs = ((s0.x + s0.y) + (s0.z + s0.w)) + ((s1.x + s1.y) + (s1.z + s1.w));
      const float xsp = ((q0.x + q0.y) + (q0.z + q0.w)) + ((q1.x + q1.y) + (q1.z + q1.w));
#pragma unroll
      for (int u = 0; u < UA; ++u) {
        const bool live = j0 + u < rows && c < C;
        const float sg = live ? aux_to_f32_sel(rsg[u][i], gm.fp16) : 0.f;
        const float bg = live ? aux_to_f32_sel(rbg[u][i], gm.fp16) : 0.f;
        const float su = live ? aux_to_f32_sel(rsu[u][i], um.fp16) : 0.f;
        const float bu = live ? aux_to_f32_sel(rbu[u][i], um.fp16) : 0.f;
        uint32_t q[16];
        unpack_chunk<BITS>(q, wg[u][i], kc);
        pg[u] += chunk_fold<BITS>(pairs_dot(q, xp), sg, bg, xs, xsp);
        unpack_chunk<BITS>(q, wu[u][i], kc);
        pu[u] += chunk_fold<BITS>(pairs_dot(q, xp), su, bu, xs, xsp);
      }
    }
    // wave totals: lane row r (r = lane / 16) ends up with row j0 + r's h
    // (logan-qwen4/src/lib.rs:8807-8809: h = silu(gate) * up)
    TL_BLOCK(2);
    float hval;
    if constexpr (UA == 4) {
      const float gv = wave_reduce4(pg[0], pg[1], pg[2], pg[3]);
      const float uv = wave_reduce4(pu[0], pu[1], pu[2], pu[3]);
      hval = silu(gv) * uv;
    } else {
      static_assert(UA == 2, "A rows per wave");
      const float t = wave_reduce4(pg[0], pg[1], pu[0], pu[1]);  // rows: g0, g1, u0, u1
      const float up = __int_as_float(__builtin_amdgcn_ds_bpermute((lane + 32) << 2, __float_as_int(t)));
      hval = silu(t) * up;
    }
    const int slice = (int)(lid % kSlices);
    uint64_t *hrow = reinterpret_cast<uint64_t *>(a.ws) + ((size_t)slice * g.slots + slot) * hmax;
    const int r = lane >> 4;
    if ((lane & 15) == 0 && r < UA && j0 + r < rows) {
      const uint64_t pr = ((uint64_t)tag << 32) | __float_as_uint(hval);
      __hip_atomic_store(&hrow[j0 + r], pr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // The block's last wave to get here adds the block's arrival, right
    // behind the stores and without waiting for them (B checks the tags).
    if (threadIdx.x == 0) {
      TL_PUT(lid, 0, s_tlb[0]);
      TL_PUT(lid, 1, s_tlb[1]);
      TL_PUT(lid, 2, s_tlb[2]);
    }
    if (lane == 0 && atomicSub(&s_left, 1u) == 1u) {
      TL_PUT(lid, 3, TL_NOW());
      const int first = shared ? g.k * g.wpr / kWaves : slot * (g.wpr / kWaves);
      __hip_atomic_fetch_add(&g_fused_sync.ctr[lid & 1][slot][(blockIdx.x - first) % kSubCtrs][0], 1u,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }

  // -------------------------------------------------------------- phase B
  // lane: chunk lb of row rsub within each pass; wave: slots wave, wave + 8
  TL_BLOCK(0);
  const int bb = blockIdx.x - g.nA_blocks;
  const int lb = lane % LANESB;
  const int rsub = lane / LANESB;
  const int d0 = bb * ROWS_B;
  const bool has_shared = a.sdown.m.w != nullptr;

  // B block 0's wave 0 routes and publishes the route; the other B blocks
  // read it (one wave selecting instead of one per block: the selection
  // rounds of 256 waves competed with the A blocks' own routing)
  unsigned long long tk = 0;
  if (threadIdx.x == 0) tk = take_ticket();
  const bool pub = bb == 0;
  RK rk;
  if (pub && wave == 0) rk.load(a.logits, a.E);

  // route-independent loads first: the shared slot's down rows
  uint32_t wv[kSlotsPerWave][PASSES][BITS];
  uint32_t rsc[kSlotsPerWave][PASSES], rbi[kSlotsPerWave][PASSES];
#pragma unroll
  for (int t = 0; t < kSlotsPerWave; ++t) {
    const int s = wave + t * kWaves;
    if (has_shared && s == g.k) {
#pragma unroll
      for (int p = 0; p < PASSES; ++p) {
        const int d = d0 + p * RPP + rsub;
        const bool live = d < a.D && lb < (a.sinter >> 5);
        load_down<BITS>(wv[t][p], rsc[t][p], rbi[t][p], a.sdown, 0, d, lb, live);
      }
    }
  }
  float wr = 0.f;
  uint32_t enc = 0u;  // publisher: 0xffff - expert of rank `lane`, 0 past the route
  if (pub && wave == 0) {
    bool routed = false;
    if constexpr (LF) {
      // 32-bit keys first (route_dev.hpp: select_fast / fast_ok)
      uint32_t fs[kFusedMaxSlots + 1];
      rk.select_fast(a.E, g.k, fs);
      float v, m;
      if (rk.fast_ok(fs, g.k - 1, v, m)) {
        uint32_t kr = 0u;
#pragma unroll
        for (int r = 0; r < kFusedMaxSlots; ++r) kr = lane == r ? fs[r] : kr;
        // combine weights, one rank per lane (logan-qwen4/src/lib.rs:8694)
        const float ev = lane < g.k ? __expf(v - m) : 0.f;
        wr = ev / wave_sum_f32(ev);
        enc = lane < g.k ? 0xffffu - (uint32_t)RK::expert32(kr) : 0u;
        routed = true;
      }
    }
    if (!routed) {
    Key sel0[kFusedMaxSlots];
    rk.select(a.E, g.k, sel0);
    Key mine = 0;
#pragma unroll
    for (int r = 0; r < kFusedMaxSlots; ++r) mine = lane == r ? sel0[r] : mine;
    const float m = RK::logit(sel0[0]);
    float llast = m;
#pragma unroll
    for (int r = 0; r < kFusedMaxSlots; ++r) llast = r == g.k - 1 ? RK::logit(sel0[r]) : llast;
    bool exact = false;
    if (LF || !bf16_ranks_tie_free(m, llast)) {
      // consecutive selected ranks checked lane-parallel (lane r: ranks r,
      // r + 1), the unselected keys per lane
      const float lr = RK::logit(mine), lnext = __shfl(lr, (lane + 1) & 63, 64);
      bool cand = lane + 1 < g.k && tie_pair(lr, lnext, m);
#pragma unroll
      for (int i = 0; i < KPL; ++i)
        cand = cand || (rk.key[i] != Key(0) && tie_other(RK::logit(rk.key[i]), llast, m));
      exact = __any(cand) || tie_global(m, llast);
    }
    if (exact) {
      // a probability tie the logit order cannot see (route_dev.hpp)
      const RouteLane rl = route_exact<KPL, LF>(a.logits, 0, a.E, g.k);
      enc = lane < g.k ? 0xffffu - (uint32_t)rl.idx : 0u;
      wr = rl.w;
    } else {
      // combine weights, one rank per lane (logan-qwen4/src/lib.rs:8694):
      // w_r = exp(l_r - l_0) / sum_{r<k} exp(l_r - l_0)
      const float ev = lane < g.k ? __expf(RK::logit(mine) - m) : 0.f;
      wr = ev / wave_sum_f32(ev);
      enc = lane < g.k ? 0xffffu - (uint32_t)RK::expert(mine) : 0u;
    }
    }
    if (lane < kFusedMaxSlots) s_sel[lane] = enc;
    if (lane < kFusedMaxSlots) s_w[lane] = wr;
    if (lane < g.k) {
      if (a.idx_out) a.idx_out[lane] = sel_expert(enc);
      if (a.w_out) a.w_out[lane] = wr;
    }
  }
  if (threadIdx.x == 0) s_lid = launch_number(tk);
  __syncthreads();
  const uint32_t lid = __builtin_amdgcn_readfirstlane(s_lid);
  const uint32_t tag = launch_tag(lid);
  // The route records: 16 bytes (0xffff - expert, tag, weight bits, tag) per
  // rank, in kSlices rotating slices after the h pairs of the workspace.
  char *const rbase = reinterpret_cast<char *>(a.ws) + (size_t)kSlices * g.slots * hmax * sizeof(uint64_t);
  const __amdgpu_buffer_rsrc_t rrs =
      __builtin_amdgcn_make_buffer_rsrc(rbase, (short)0, kSlices * kFusedMaxSlots * 16, kBufWord3);
  const int roff = ((int)(lid % kSlices) * kFusedMaxSlots + (lane < kFusedMaxSlots ? lane : 0)) * 16;
  if (pub && wave == 0 && lane < g.k) {
    // device-scope 64-bit halves, each carrying the tag
    uint64_t *rec = reinterpret_cast<uint64_t *>(rbase + roff);
    const uint64_t tg = (uint64_t)tag << 32;
    __hip_atomic_store(rec, tg | enc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(rec + 1, tg | __float_as_uint(wr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!pub && wave == 0) {
    // read the ranks' records with device-scope loads until every tag is this
    // launch's (the few record lines stay in an XCD's L2 from earlier
    // launches, so a first read through L2 would mostly find stale tags)
    const bool mine = lane < g.k;
    uint4 q = make_uint4(0u, 0u, 0u, 0u);
    bool ok = !mine;
    if (mine) {
      q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rrs, roff, 0, kCpolSc1));
      ok = q.y == tag && q.w == tag;
    }
    uint32_t rto = 0;
    for (uint32_t spins = 0; !__all(ok);) {
      __builtin_amdgcn_s_sleep(1);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if (++spins > kSpinLimit) {
        rto = 1;
        break;
      }
      if (!ok) {
        q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rrs, roff, 0, kCpolSc1));
        ok = q.y == tag && q.w == tag;
      }
    }
    // a route that never came: expert 0 everywhere (valid addresses), no output
    if (lane < kFusedMaxSlots) s_sel[lane] = mine ? (rto ? 0xffffu : q.x) : 0u;
    if (lane < kFusedMaxSlots) s_w[lane] = mine && !rto ? __uint_as_float(q.z) : 0.f;
    if (lane == 0) s_rto = rto;
    if (rto && lane == 0)
      __hip_atomic_fetch_or(&g_fused_sync.error[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (pub && wave == 0 && lane == 0) s_rto = 0u;
  __syncthreads();
  TL_BLOCK(1);
  // zero the arrival counters the next launch uses (the previous launch,
  // their last user, has ended): counter j by block j mod nB
  if (wave == 0) {
    const int j = bb + g.nB_blocks * lane;
    if (j < kFusedMaxSlots * kSubCtrs) st_agent(&g_fused_sync.ctr[(lid + 1) & 1][j / kSubCtrs][j % kSubCtrs][0], 0u);
  }
#pragma unroll
  for (int t = 0; t < kSlotsPerWave; ++t) {
    const int s = wave + t * kWaves;
    if (s < g.k) {
      const uint32_t kk = __builtin_amdgcn_readfirstlane(s_sel[s]);
      bool miss = false;  // (reported by the A blocks, which route the same way)
      const int e = moe_bank_index<false>(a, sel_expert(kk), miss);
#pragma unroll
      for (int p = 0; p < PASSES; ++p) {
        const int d = d0 + p * RPP + rsub;
        const bool live = d < a.D && lb < (a.inter >> 5);
        load_down<BITS>(wv[t][p], rsc[t][p], rbi[t][p], a.down, e, d, lb, live);
      }
    }
  }
  // shared-expert gate loads after the down rows, by the last wave (one slot
  // fewer than wave 0 when slots > kWaves)
  uint4 gq[CPLA][4], xq[CPLA][4];
  const bool do_gate = wave == kWaves - 1 && has_shared && a.se_gate_vec;
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
  __builtin_amdgcn_sched_barrier(0);
  // shared-expert scalar gate sigmoid(se_g . x) (logan-qwen4/src/lib.rs:7602-7604)
  if (wave == kWaves - 1) {
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

  // While the gate/up blocks run, turn this wave's down codes into exact f16
  // pairs and its scale/bias words into f32, so that after the hand-off each
  // code costs one v_fma_mix_f32 (f16 code x f32 h + f32). The empty asm
  // operands keep the conversion here, ahead of the wait (the compiler would
  // otherwise sink it to the first use, behind the hand-off).
  // (Not with 32-lane down rows at one x chunk per lane: their h pairs
  // already fill the 128-register budget of that instantiation.)
  constexpr bool kPreF16 = !(LANESB == 32 && CPLA == 1);
  uint32_t cp[kSlotsPerWave][PASSES][16];
  float fsc[kSlotsPerWave][PASSES], fbi[kSlotsPerWave][PASSES];
#pragma unroll
  for (int t = 0; t < kSlotsPerWave && kPreF16; ++t) {
    const int s = wave + t * kWaves;
    const bool sh = has_shared && s == g.k;
    const int K = sh ? a.sinter : a.inter;
    const int fp16 = sh ? a.sdown.m.fp16 : a.down.m.fp16;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const bool live = s < g.slots && d0 + p * RPP + rsub < a.D && lb < (K >> 5);
      fsc[t][p] = live ? aux_to_f32(rsc[t][p], fp16) : 0.f;
      fbi[t][p] = live ? aux_to_f32(rbi[t][p], fp16) : 0.f;
      codes_to_f16<BITS>(wv[t][p], cp[t][p]);
#pragma unroll
      for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(cp[t][p][i]));
      asm volatile("" : "+v"(fsc[t][p]), "+v"(fbi[t][p]));
    }
  }

  // Wait for the arrivals of this wave's slots (lane 4 t + q polls
  // sub-counter q of slot wave + 8 t), read their tagged h together until
  // every tag is this launch's, then form the down products slot by slot.
  static_assert(kSlotsPerWave * kSubCtrs <= 64, "one poll lane per sub-counter");
  uint32_t to = 0;
  {
    const int t = lane / kSubCtrs, q = lane % kSubCtrs;
    const int s = wave + t * kWaves;
    const bool mine = t < kSlotsPerWave && s < g.slots;
    const int nb = ((has_shared && s == g.k) ? g.wps : g.wpr) / kWaves;  // A blocks of slot s
    const uint32_t need = mine ? sub_need(nb, q) : 0u;
    uint32_t *cp = &g_fused_sync.ctr[lid & 1][mine ? s : 0][q][0];
    bool done = !mine || ld_agent(cp) >= need;
    uint32_t spins = 0;
    while (!__all(done)) {
      __builtin_amdgcn_s_sleep(2);
      if (!done) done = ld_agent(cp) >= need;
      if (++spins > kSpinLimit) {
        to = 1;
        break;
      }
    }
  }
  TL_WAVE(0);
  // lane covers h[VPL*lane .. VPL*lane + VPL) of each slot: first through
  // L2, then (stale or not yet landed) with device-scope loads
  const int slice = (int)(lid % kSlices);
  const __amdgpu_buffer_rsrc_t hrsrc = __builtin_amdgcn_make_buffer_rsrc(
      a.ws, (short)0, kSlices * g.slots * hmax * 8, kBufWord3);
  float hv[kSlotsPerWave][VPL];
  bool ok = true;
  if (!to) {
#pragma unroll
    for (int t = 0; t < kSlotsPerWave; ++t) {
      const int s = wave + t * kWaves;
      const int K = s < g.slots ? ((has_shared && s == g.k) ? a.sinter : a.inter) : 0;
      const int off = ((slice * g.slots + (s < g.slots ? s : 0)) * hmax + VPL * lane) * 8;
      ok = read_pairs<VPL, 0>(hrsrc, off, K - VPL * lane, tag, hv[t]) && ok;
    }
  }
  for (uint32_t spins = 0; !to && !__all(ok);) {
    __builtin_amdgcn_s_sleep(1);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (++spins > kSpinLimit) {
      to = 1;
      break;
    }
    ok = true;
#pragma unroll
    for (int t = 0; t < kSlotsPerWave; ++t) {
      const int s = wave + t * kWaves;
      const int K = s < g.slots ? ((has_shared && s == g.k) ? a.sinter : a.inter) : 0;
      const int off = ((slice * g.slots + (s < g.slots ? s : 0)) * hmax + VPL * lane) * 8;
      ok = read_pairs<VPL, kCpolSc1>(hrsrc, off, K - VPL * lane, tag, hv[t]) && ok;
    }
  }
  TL_WAVE(1);
  if (to && lane == 0)
    __hip_atomic_fetch_or(&g_fused_sync.error[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int t = 0; t < kSlotsPerWave; ++t) {
    const int s = wave + t * kWaves;
    if (s < g.slots && !to && !kPreF16) {
      down_slot_f32<BITS, PASSES, RPP, LANESB, VPL>(a, s, has_shared && s == g.k, d0, lb, rsub, s_hv[wave],
                                                  hv[t], wv[t], rsc[t], rbi[t], s_y);
    } else if (s < g.slots && !to) {
      // through this wave's LDS row to chunk-per-lane (h of chunk lb)
      float *row = s_hv[wave];
#pragma unroll
      for (int v = 0; v < VPL; v += 4)
        *reinterpret_cast<float4 *>(row + VPL * lane + v) =
            make_float4(hv[t][v], hv[t][v + 1], hv[t][v + 2], hv[t][v + 3]);
      // sum of h over chunk c, which lanes LPC c .. LPC c + LPC - 1 hold
      constexpr int LPC = 32 / VPL;
      static_assert(LPC == 2 || LPC == 4, "h pairs per lane");
      float hs = 0.f;
#pragma unroll
      for (int v = 0; v < VPL; ++v) hs += hv[t][v];
      hs += __shfl_xor(hs, 1);
      if constexpr (LPC == 4) hs += __shfl_xor(hs, 2);
      const float xs = __shfl(hs, LPC * lb);
      __builtin_amdgcn_wave_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      float acc[PASSES];
#pragma unroll
      for (int p = 0; p < PASSES; ++p) acc[p] = 0.f;
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const float4 f = *reinterpret_cast<const float4 *>(row + 32 * lb + 4 * v);
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
          const half2v c0 = __builtin_bit_cast(half2v, cp[t][p][2 * v]);
          const half2v c1 = __builtin_bit_cast(half2v, cp[t][p][2 * v + 1]);
          acc[p] = fmaf((float)c0.x, f.x, acc[p]);
          acc[p] = fmaf((float)c0.y, f.y, acc[p]);
          acc[p] = fmaf((float)c1.x, f.z, acc[p]);
          acc[p] = fmaf((float)c1.y, f.w, acc[p]);
        }
      }
      __builtin_amdgcn_wave_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
      for (int p = 0; p < PASSES; ++p) {
        // sum_k (code_k * sc + bi) * h_k = sc * sum_k code_k h_k + bi * sum_k h_k
        float v = fmaf(fsc[t][p], acc[p], fbi[t][p] * xs);
        v = group_sum_f32<LANESB>(v);
        if (lb == 0) s_y[p * RPP + rsub][s] = v;
      }
    }
  }
  if (lane == 0) s_to[wave] = to;
  TL_WAVE(2);
  __syncthreads();
  if (threadIdx.x == 0) {
    TL_PUT(lid, 0, s_tlb[0]);
    TL_PUT(lid, 1, s_tlb[1]);
    TL_PUT_WAVES(lid, 2, 0);
    TL_PUT_WAVES(lid, 3, 1);
    TL_PUT_WAVES(lid, 4, 2);
  }

  // rank-ordered combine (logan-qwen4/src/lib.rs:8692-8711) by the first ROWS_B threads
  if ((int)threadIdx.x < ROWS_B) {
    const int r = threadIdx.x;
    const int dd = d0 + r;
    uint32_t anyto = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) anyto |= s_to[w];
    anyto |= s_rto;
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < kFusedMaxSlots; ++q)
      if (q < g.k) acc = fmaf(s_y[r][q], s_w[q], acc);
    float o = acc;
    if (has_shared) o = fmaf(s_y[r][g.k], s_gsig, acc);
    if (dd < a.D && !anyto) {
      if (a.out_f32)
        reinterpret_cast<float *>(a.out)[dd] = o;
      else
        reinterpret_cast<uint16_t *>(a.out)[dd] = (uint16_t)f32_to_bf16_rne(o);
    }
  }
  if (threadIdx.x == 0) TL_PUT(lid, 5, TL_NOW());

}

// ---------------------------------------------------------------- launch

size_t moe_fused_workspace_bytes(int slots, int inter, int sinter) {
  const size_t hmax = (size_t)(inter > sinter ? inter : sinter);
  // (value, tag) h pairs, then the published route records
  return (size_t)kSlices * slots * hmax * sizeof(uint64_t) + (size_t)kSlices * kFusedMaxSlots * 16;
}

// Launches of this kernel on one device share the module-scope ticket and
// arrival counters, so they must not overlap. Launches on one stream are
// ordered by the stream; when a launch comes on another stream than the
// previous one, it first waits (hipStreamWaitEvent) for an event recorded
// after that launch. Launches recorded into a graph are ordered by the
// graph's stream; replays of such a graph must not overlap other launches
// of this kernel on the device (nothing is recorded or waited for while a
// stream captures).
namespace {
constexpr int kMaxDevices = 64;
struct FusedOrder {
  hipStream_t last = nullptr;
  hipEvent_t ev = nullptr;
  bool pending = false;  // ev marks the end of the last launch
};
std::mutex g_order_mtx;
FusedOrder g_order[kMaxDevices];
}  // namespace

template <int BITS, int CPLA, int LANESB, int KPL, bool LF>
static int fused_launch(const MoeArgs &a, const FusedGeom &g, hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess) return 0;
  const bool capturing = cap != hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lk(g_order_mtx);
  FusedOrder &o = g_order[dev];
  if (!capturing && o.pending && o.last != st && hipStreamWaitEvent(st, o.ev, 0) != hipSuccess)
    return -1;
  auto kern = moe_fused_b1_kernel<BITS, CPLA, LANESB, KPL, LF>;
  hipLaunchKernelGGL(kern, dim3(g.nA_blocks + g.nB_blocks), dim3(kWaves * 64), 0, st, a, g);
  if (hipGetLastError() != hipSuccess) return -1;
  o.last = st;
  o.pending = false;
  if (!capturing) {
    if (!o.ev && hipEventCreateWithFlags(&o.ev, hipEventDisableTiming) != hipSuccess) return 1;
    o.pending = hipEventRecord(o.ev, st) == hipSuccess;
  }
  return 1;
}

template <int BITS, int CPLA, int LANESB>
static int fused_kpl(const MoeArgs &a, const FusedGeom &g, hipStream_t st) {
  if (a.logits_f32) {
    if (a.E <= 512) return fused_launch<BITS, CPLA, LANESB, 8, true>(a, g, st);
    if (a.E <= 1024) return fused_launch<BITS, CPLA, LANESB, 16, true>(a, g, st);
    return 0;
  }
  if (a.E <= 512) return fused_launch<BITS, CPLA, LANESB, 8, false>(a, g, st);
  if (a.E <= 1024) return fused_launch<BITS, CPLA, LANESB, 16, false>(a, g, st);
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
  if (a.B != 1) return 0;
  const int slots = a.k + (a.sdown.m.w ? 1 : 0);
  if (slots > kFusedMaxSlots || a.E > 1024) return 0;
  const int hmax = a.inter > a.sinter ? a.inter : a.sinter;
  if (a.ws_bytes < moe_fused_workspace_bytes(slots, a.inter, a.sinter)) return 0;
  if ((reinterpret_cast<uintptr_t>(a.ws) & 15) != 0 || (hmax & 3) != 0) return 0;
  const int UA = fused_ua(a.gate.m.bits, (a.D >> 5) <= 64 ? 1 : 2);
  if (a.se_gate_vec && (reinterpret_cast<uintptr_t>(a.se_gate_vec) & 15) != 0) return 0;
  if ((reinterpret_cast<uintptr_t>(a.x) & 15) != 0) return 0;
  const int gs32 = a.gate.m.gs >> 5;  // A indexes groups with a shift
  if ((gs32 & (gs32 - 1)) != 0) return 0;
  FusedGeom g;
  g.k = a.k;
  g.slots = slots;
  g.wpr = (a.inter + UA - 1) / UA;
  g.wps = a.sdown.m.w ? (a.sinter + UA - 1) / UA : 0;
  // whole A blocks per slot (inter and sinter are multiples of 32)
  if (g.wpr % kWaves != 0 || g.wps % kWaves != 0) return 0;
  g.nA_blocks = (g.k * g.wpr + g.wps) / kWaves;
  const int Ci = hmax >> 5;
  const int lanesb = Ci <= 16 ? 16 : 32;
  const int rows_per_block = (64 / lanesb) * FUSED_PASSES;  // RPP * PASSES
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
  // between launches every ticket counter sits on the same launch boundary
  uint32_t off = 0, apart = 0;
  for (int j = 0; j < kTickets; ++j) {
    off |= (s.tk[j][0] & ((1ull << kTicketShift) - 1)) != 0;
    apart |= (s.tk[j][0] >> kTicketShift) != (s.tk[0][0] >> kTicketShift);
  }
  return s.error[0] | (off ? 2u : 0u) | (apart ? 4u : 0u);
}

}  // namespace lh

#ifdef LOGAN_HIP_TIMELINE
// [2][1024][16] u64 stamps of the timeline build (see above); 0 on success
extern "C" int logan_hip_fused_timeline(unsigned long long *out, size_t bytes) {
  if (bytes < sizeof(lh::g_fused_tl)) return -1;
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(lh::g_fused_tl), sizeof(lh::g_fused_tl), 0,
                             hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
#endif
