// Small-batch MLX-affine product on MFMA with K split across blocks:
// y[m] = W x[m] for 3 <= M <= 32 activation rows (same numerics as
// gemv_mfma.hip: exact codes, f32 accumulation, per-group scale and bias
// folded after each 64-code step).
//
// Block (rb, ks) owns rows [128 rb, 128 rb + 128) (8 waves x 16 rows) and
// codes [512 ks, 512 ks + 512). Its x rows for that K range are staged once
// in LDS (in the operand order of the code width) and feed all 8 waves, so
// the activation traffic is 1/8 of a wave-private load; every wave issues
// its x staging loads, its scale/bias words and then all eight of its 64-code
// steps' weight loads before its first wait. Each block writes its partial
// sums for its (token, row) pairs into a scratch slot, and a second kernel
// adds the K partials in order (deterministic) into y. (The last-arriving
// block of a row block adding them instead, behind device-scope atomics,
// measured slower: 87.9 against 84.4 us for a config-2 layer at M = 8, since
// one block then reads every partial of its rows in series.)
//
// Scratch: kSkSlots module-scope slots of kSkSlotFloats floats, leased from
// a SlotRing: launches on any streams that would overlap on a slot are
// ordered on the device.
#include <atomic>
#include <type_traits>

#include "affine_dev.hpp"
#include "lh_internal.hpp"
#include "mfma_dev.hpp"

namespace lh {

constexpr int kSkKc = 512;   // codes per block
constexpr int kSkSteps = kSkKc / 64;
constexpr int kSkRows = 128;  // rows per block
constexpr int kSkSlots = 4;
constexpr size_t kSkSlotFloats = size_t(1) << 21;  // 8 MB per slot

static __device__ __align__(256) float g_sk_part[kSkSlots * kSkSlotFloats];

struct SplitParams {
  const uint8_t *w;
  const uint16_t *sc;
  const uint16_t *bi;
  const uint16_t *x;
  long long row_bytes;
  int N, K, ng, gsteps, x_stride, M, slot;
  size_t part_off;  // this product's partials within the slot
};

// Products that share x (same K, code width, group size and sidecar type),
// one grid: block b belongs to product i for start[i] <= b < start[i + 1].
constexpr int kSkMultiMax = 8;
struct SplitMulti {
  SplitParams m[kSkMultiMax];
  int start[kSkMultiMax + 1];
  int n;
};
struct ReduceMulti {
  void *y[kSkMultiMax];
  size_t part_off[kSkMultiMax];
  int N[kSkMultiMax];
  int y_stride[kSkMultiMax];
  int start[kSkMultiMax + 1];  // prefix sums of M * N
  int n, KS, M, slot, y_bf16;
  int swiglu;  // products 0 (gate) and 1 (up) reduce to y[0] = silu(gate) * up
};

template <int BITS, int MT, bool FP16, bool AUX8>
__device__ __forceinline__ void splitk_block(const SplitParams &p, int rb) {
  __shared__ __align__(16) uint16_t sx[16 * MT * kSkKc];
  using S = MfmaStep<BITS>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int ks = blockIdx.y;
  const int k0 = ks * kSkKc;
  const int n = rb * kSkRows + wave * 16 + r16;
  const int row = min(n, p.N - 1);
  const uint8_t *wrow = p.w + (size_t)row * p.row_bytes;
  const uint16_t *srow = p.sc + (size_t)row * p.ng;
  const uint16_t *brow = p.bi + (size_t)row * p.ng;

  // Loads in the order they are needed: x rows m < M for codes [k0, k0 + 512)
  // (64 granules of 8 per row), the scale/bias words, then the eight steps'
  // weights. Loads complete in issue order (vmcnt), so x is staged and each
  // 64-code step starts as soon as its own weights land; with the weights
  // first, staging x waited for all 64 KB of the block's weights and no step
  // overlapped the loads (3.6 us of loads, then 1.2 us of MFMA per block).
  constexpr int NV = 16 * MT * (kSkKc / 8) / 512;
  uint4 v[NV];
  {
    const int lim = p.M * (kSkKc / 8);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int q = min(tid + 512 * i, lim - 1);
      const int m = q >> 6, qq = q & 63;
      v[i] = *reinterpret_cast<const uint4 *>(p.x + (size_t)m * p.x_stride + k0 + 8 * qq);
    }
  }
  uint32_t sr[kSkSteps], br[kSkSteps];
  uint4 vs, vb;
  if constexpr (AUX8) {
    // groups of 64: the 8 steps' u16 words are one aligned 16-byte run
    vs = *reinterpret_cast<const uint4 *>(srow + (k0 >> 6));
    vb = *reinterpret_cast<const uint4 *>(brow + (k0 >> 6));
  } else {
#pragma unroll
    for (int u = 0; u < kSkSteps; ++u) {
      const int gi = ((k0 >> 6) + u) / p.gsteps;
      sr[u] = srow[gi];
      br[u] = brow[gi];
    }
  }
  SkRaw<BITS> wr[kSkSteps];
#pragma unroll
  for (int u = 0; u < kSkSteps; ++u) S::load_raw(wr[u], wrow, k0 + u * 64 + 16 * g);
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the first wait
  if constexpr (AUX8) {
    const uint32_t ws[4] = {vs.x, vs.y, vs.z, vs.w}, wb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
    for (int u = 0; u < kSkSteps; ++u) {
      sr[u] = (ws[u >> 1] >> (16 * (u & 1))) & 0xffffu;
      br[u] = (wb[u >> 1] >> (16 * (u & 1))) & 0xffffu;
    }
  }
  // unconditional stores (granules past row M - 1 fill LDS rows no stored
  // output depends on), so no load is sunk into a guarded store
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = tid + 512 * i;
    const int m = q >> 6, qq = q & 63;
    const uint4 o = BITS == 4 ? __builtin_bit_cast(uint4, a_nibble_order(v[i])) : v[i];
    *reinterpret_cast<uint4 *>(sx + m * kSkKc + 8 * swz(m, qq)) = o;
  }
  __syncthreads();

  UnpackConsts kc;
  kc.init();
  const bf16x8_t ones = mfma_ones();
  f32x4_t acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kSkSteps; ++u) {
    bf16x8_t b0, b1;
    S::b_ops(wr[u], kc, b0, b1);
    const float s = aux_f32<FP16>(sr[u]), b = aux_f32<FP16>(br[u]);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      bf16x8_t a0, a1;
      const int m = 16 * t + r16;
      S::a_ops(sx + m * kSkKc, (u * 64 + 16 * g) >> 3, m, a0, a1);
      const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      f32x4_t xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, ones, z, 0, 0, 0);
      xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, ones, xs, 0, 0, 0);
      f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, z, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, d, 0, 0, 0);
      S::fold(acc[t], d, xs, s, b);
    }
  }
  if (n >= p.N) return;
  float *part = g_sk_part + (size_t)p.slot * kSkSlotFloats + p.part_off + (size_t)ks * p.M * p.N;
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * t + 4 * g + i;
      if (m < p.M) part[(size_t)m * p.N + n] = acc[t][i];
    }
}

template <int BITS, int MT, bool FP16, bool AUX8>
__global__ __launch_bounds__(512) void skinny_splitk_kernel(SplitParams p) {
  splitk_block<BITS, MT, FP16, AUX8>(p, blockIdx.x);
}

template <int BITS, int MT, bool FP16, bool AUX8>
__global__ __launch_bounds__(512) void skinny_splitk_multi_kernel(SplitMulti mp) {
  int i = 0;
  while (i + 1 < mp.n && (int)blockIdx.x >= mp.start[i + 1]) ++i;
  splitk_block<BITS, MT, FP16, AUX8>(mp.m[i], blockIdx.x - mp.start[i]);
}

__global__ __launch_bounds__(256) void splitk_reduce_kernel(int slot, int KS, int M, int N, void *y,
                                                            int y_stride, int y_bf16) {
  const float *part = g_sk_part + (size_t)slot * kSkSlotFloats;
  const int MN = M * N;  // <= kSkSlotFloats
  for (int i = blockIdx.x * 256 + threadIdx.x; i < MN; i += gridDim.x * 256) {
    // eight partials in flight at a time, added in K order
    float s = 0.f;
    for (int k0 = 0; k0 < KS; k0 += 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = part[min(k0 + j, KS - 1) * MN + i];
#pragma unroll
      for (int j = 0; j < 8; ++j) s += k0 + j < KS ? v[j] : 0.f;
    }
    const int m = i / N, n = i - m * N;
    if (y_bf16)
      reinterpret_cast<uint16_t *>(y)[(size_t)m * y_stride + n] = (uint16_t)f32_to_bf16_rne(s);
    else
      reinterpret_cast<float *>(y)[(size_t)m * y_stride + n] = s;
  }
}

// The reduce of several products in one grid (each element added in K order,
// as in splitk_reduce_kernel).
__global__ __launch_bounds__(256) void splitk_reduce_multi_kernel(ReduceMulti r) {
  const float *part = g_sk_part + (size_t)r.slot * kSkSlotFloats;
  if (r.swiglu) {
    // h = silu(gate) * up (logan-qwen4/src/lib.rs:8803-8812), each sum in K order
    const int MN = r.M * r.N[0];
    const float *pg = part + r.part_off[0], *pu = part + r.part_off[1];
    for (int i = blockIdx.x * 256 + threadIdx.x; i < MN; i += gridDim.x * 256) {
      float sg = 0.f, su = 0.f;
      for (int k0 = 0; k0 < r.KS; k0 += 8) {
        float vg[8], vu[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          vg[q] = pg[(size_t)min(k0 + q, r.KS - 1) * MN + i];
          vu[q] = pu[(size_t)min(k0 + q, r.KS - 1) * MN + i];
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          sg += k0 + q < r.KS ? vg[q] : 0.f;
          su += k0 + q < r.KS ? vu[q] : 0.f;
        }
      }
      const float hv = silu(sg) * su;
      const int m = i / r.N[0], nn = i - m * r.N[0];
      if (r.y_bf16)
        reinterpret_cast<uint16_t *>(r.y[0])[(size_t)m * r.y_stride[0] + nn] = (uint16_t)f32_to_bf16_rne(hv);
      else
        reinterpret_cast<float *>(r.y[0])[(size_t)m * r.y_stride[0] + nn] = hv;
    }
    return;
  }
  const int total = r.start[r.n];
  for (int i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
    int j = 0;
    while (j + 1 < r.n && i >= r.start[j + 1]) ++j;
    const int li = i - r.start[j];
    const int MN = r.M * r.N[j];
    const float *pj = part + r.part_off[j];
    float s = 0.f;
    for (int k0 = 0; k0 < r.KS; k0 += 8) {
      float v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = pj[(size_t)min(k0 + q, r.KS - 1) * MN + li];
#pragma unroll
      for (int q = 0; q < 8; ++q) s += k0 + q < r.KS ? v[q] : 0.f;
    }
    const int m = li / r.N[j], nn = li - m * r.N[j];
    if (r.y_bf16)
      reinterpret_cast<uint16_t *>(r.y[j])[(size_t)m * r.y_stride[j] + nn] = (uint16_t)f32_to_bf16_rne(s);
    else
      reinterpret_cast<float *>(r.y[j])[(size_t)m * r.y_stride[j] + nn] = s;
  }
}

// ---------------------------------------------------------------------------
// gate/up + SwiGLU over the full K, for the pairs with enough rows to fill the
// chip without a K split (the config-2 4096 -> 2 x 14336 product): block b
// owns row indices [64 b, 64 b + 64); waves 0-3 stream those gate rows and
// waves 4-7 the same up rows, 16 each, over all of K in chunks of 512 codes.
// Each chunk's x rows are staged once in LDS (double-buffered, the layout of
// splitk_block) and its weights, scale and bias words are issued one chunk
// ahead of their MFMAs. The gate waves hand their sums to the up waves
// through LDS, which write h = silu(gate) * up (logan-qwen4/src/lib.rs
// :8807-8809): no partial sums and no reduce launch.
#ifndef FULLK_WPM
#define FULLK_WPM 4
#endif
constexpr int kFkWpm = FULLK_WPM;     // waves per matrix in a block
constexpr int kFkRows = 16 * kFkWpm;  // row indices per block
constexpr int kFkThreads = 128 * kFkWpm;

struct FullKParams {
  const uint8_t *w[2];  // gate, up
  const uint16_t *sc[2];
  const uint16_t *bi[2];
  const uint16_t *x;
  void *h;
  long long row_bytes;
  int N, K, ng, gsteps, x_stride, M, h_stride, h_bf16;
};

template <int BITS, int MT, bool AUX8>
struct FkChunk {
  static constexpr int NV = 16 * MT * (kSkKc / 8) / kFkThreads;  // x granules per thread
  uint4 v[NV];
  SkRaw<BITS> wr[kSkSteps];
  uint32_t sr[AUX8 ? 1 : kSkSteps], br[AUX8 ? 1 : kSkSteps];
  uint4 vs, vb;
};

template <int BITS, int MT, bool FP16, bool AUX8>
__global__ __launch_bounds__(kFkThreads) void swiglu_fullk_kernel(FullKParams p) {
  __shared__ __align__(16) uint16_t sx[2][16 * MT * kSkKc];
  __shared__ float sg[kFkWpm][64][4 * MT];
  using S = MfmaStep<BITS>;
  using C = FkChunk<BITS, MT, AUX8>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int mat = wave / kFkWpm;  // 0: gate, 1: up
  const int n = blockIdx.x * kFkRows + (wave % kFkWpm) * 16 + r16;
  const int row = min(n, p.N - 1);
  const uint8_t *wrow = (mat ? p.w[1] : p.w[0]) + (size_t)row * p.row_bytes;
  const uint16_t *srow = (mat ? p.sc[1] : p.sc[0]) + (size_t)row * p.ng;
  const uint16_t *brow = (mat ? p.bi[1] : p.bi[0]) + (size_t)row * p.ng;
  const int nch = p.K / kSkKc;
  const int lim = p.M * (kSkKc / 8);

  // loads of chunk c in the order they are needed: x, scale/bias, weights
  auto issue = [&](int c, C &q) {
    const int k0 = c * kSkKc;
#pragma unroll
    for (int i = 0; i < C::NV; ++i) {
      const int gq = min(tid + kFkThreads * i, lim - 1);
      q.v[i] = *reinterpret_cast<const uint4 *>(p.x + (size_t)(gq >> 6) * p.x_stride + k0 + 8 * (gq & 63));
    }
    if constexpr (AUX8) {
      q.vs = *reinterpret_cast<const uint4 *>(srow + (k0 >> 6));
      q.vb = *reinterpret_cast<const uint4 *>(brow + (k0 >> 6));
    } else {
#pragma unroll
      for (int u = 0; u < kSkSteps; ++u) {
        const int gi = ((k0 >> 6) + u) / p.gsteps;
        q.sr[u] = srow[gi];
        q.br[u] = brow[gi];
      }
    }
#pragma unroll
    for (int u = 0; u < kSkSteps; ++u) S::load_raw(q.wr[u], wrow, k0 + u * 64 + 16 * g);
  };
  // x of a chunk into LDS buffer b (granules past row M - 1 fill rows no
  // stored output depends on)
  auto stage = [&](const C &q, int b) {
#pragma unroll
    for (int i = 0; i < C::NV; ++i) {
      const int gq = tid + kFkThreads * i;
      const int m = gq >> 6, qq = gq & 63;
      const uint4 o = BITS == 4 ? __builtin_bit_cast(uint4, a_nibble_order(q.v[i])) : q.v[i];
      *reinterpret_cast<uint4 *>(sx[b] + m * kSkKc + 8 * swz(m, qq)) = o;
    }
  };
  UnpackConsts kc;
  kc.init();
  const bf16x8_t ones = mfma_ones();
  f32x4_t acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const C &q, int b) {
#pragma unroll
    for (int u = 0; u < kSkSteps; ++u) {
      uint32_t su, bu;
      if constexpr (AUX8) {
        const uint32_t ws[4] = {q.vs.x, q.vs.y, q.vs.z, q.vs.w}, wb[4] = {q.vb.x, q.vb.y, q.vb.z, q.vb.w};
        su = (ws[u >> 1] >> (16 * (u & 1))) & 0xffffu;
        bu = (wb[u >> 1] >> (16 * (u & 1))) & 0xffffu;
      } else {
        su = q.sr[u];
        bu = q.br[u];
      }
      bf16x8_t b0, b1;
      S::b_ops(q.wr[u], kc, b0, b1);
      const float sf = aux_f32<FP16>(su), bf = aux_f32<FP16>(bu);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        bf16x8_t a0, a1;
        const int m = 16 * t + r16;
        S::a_ops(sx[b] + m * kSkKc, (u * 64 + 16 * g) >> 3, m, a0, a1);
        const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
        f32x4_t xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, ones, z, 0, 0, 0);
        xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, ones, xs, 0, 0, 0);
        f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, z, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, d, 0, 0, 0);
        S::fold(acc[t], d, xs, sf, bf);
      }
    }
  };

  // two chunks per trip, so each register set is a fixed one: chunk c is
  // multiplied from LDS buffer c & 1 while chunk c + 1's loads are in flight
  C qa, qb;
  issue(0, qa);
  stage(qa, 0);
  if (nch > 1) issue(1, qb);
  __syncthreads();
  for (int c = 0; c < nch; c += 2) {
    compute(qa, 0);
    if (c + 1 < nch) stage(qb, 1);
    if (c + 2 < nch) issue(c + 2, qa);
    __syncthreads();
    if (c + 1 < nch) {
      compute(qb, 1);
      if (c + 2 < nch) stage(qa, 0);
      if (c + 3 < nch) issue(c + 3, qb);
      __syncthreads();
    }
  }

  // accumulator element i of lane l: token 16 t + 4 (l / 16) + i, row n
  if (mat == 0) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) sg[wave][lane][4 * t + i] = acc[t][i];
  }
  __syncthreads();
  if (mat == 1 && n < p.N) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 16 * t + 4 * g + i;
        if (m >= p.M) continue;
        const float hv = silu(sg[wave - kFkWpm][lane][4 * t + i]) * acc[t][i];
        if (p.h_bf16)
          reinterpret_cast<uint16_t *>(p.h)[(size_t)m * p.h_stride + n] = (uint16_t)f32_to_bf16_rne(hv);
        else
          reinterpret_cast<float *>(p.h)[(size_t)m * p.h_stride + n] = hv;
      }
  }
}

// ---------------------------------------------------------------------------
// Small-batch product (3..8 tokens) with K split across the waves of one
// block instead of across blocks: block b owns rows [16 b, 16 b + 16), and
// each of its W waves owns a run of cpw 512-code chunks (K = 512 W cpw). The
// waves' K ranges are disjoint, so each wave stages its own x rows: per
// chunk, one coalesced 1 KB load per row (MX rows, MX = 4 or 8; rows past
// M - 1 repeat row M - 1 and their outputs are discarded) into an LDS tile
// of its own, read back in the MFMA operand order. A wave keeps one chunk of
// weights in flight behind the step it computes (a step's registers are
// reissued for the next chunk as soon as the step's products have read them)
// and the next chunk's x one chunk ahead. The waves' sums meet in LDS and
// are added in K order (wave 0 first, the order the K-split reduce adds its
// partials in), and the block writes y: no partial sums and no reduce
// launch.
//
// Measured against a plain read of the same bytes in the same pattern (9 us
// for the config-2 down product, 4096 x 14336 codes): the kernel's loads
// alone run at that rate and its arithmetic alone (8-bit code conversion,
// MFMA, fold) takes 7.5 us, and the two add up rather than overlap. Each CU
// holds a bounded number of vector-memory instructions in flight; a wave
// with more outstanding waits at issue and cannot compute meanwhile. Holding
// two chunks per wave in registers (next chunk issued before the current
// one's products) made the issue stalls longer, not the layer faster
// (per-wave s_memrealtime stamps: up to 8 us before a wave's first chunk
// was accepted), and copying x with global_load_lds makes the compiler wait
// for every load before each LDS read.
#ifndef SKINNY_KWAVE
#define SKINNY_KWAVE 1
#endif
constexpr bool kSkinnyKwave = SKINNY_KWAVE != 0;
constexpr int kKwMaxW = 8;

struct KwaveParams {
  const uint8_t *w;
  const uint16_t *sc;
  const uint16_t *bi;
  const uint16_t *x;
  void *y;
  long long row_bytes;
  int N, ng, gsteps, x_stride, M, cpw, y_stride, y_bf16;
};

// dynamic LDS of the kernel: W waves x 2 buffers x MX rows x 512 bf16
__host__ __device__ constexpr size_t kwave_lds_bytes(int W, int MX) {
  return (size_t)W * 2 * MX * kSkKc * 2;
}

template <int BITS, int MX, bool FP16, bool AUX8>
__global__ __launch_bounds__(64 * kKwMaxW) void skinny_kwave_kernel(KwaveParams p) {
  using S = MfmaStep<BITS>;
  extern __shared__ __align__(16) uint16_t kw_lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int W = blockDim.x >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int n = blockIdx.x * 16 + r16;
  const int row = min(n, p.N - 1);
  const uint8_t *wrow = p.w + (size_t)row * p.row_bytes;
  const uint16_t *srow = p.sc + (size_t)row * p.ng;
  const uint16_t *brow = p.bi + (size_t)row * p.ng;
  const int kb = wave * p.cpw * kSkKc;
  uint16_t *sxw = kw_lds + (size_t)wave * 2 * MX * kSkKc;  // this wave's two x tiles
  const int mr = min(r16, MX - 1);                          // operand row read by this lane

  SkRaw<BITS> wr[kSkSteps];
  uint4 xg[MX];                          // x granule `lane` of rows 0..MX-1 of a chunk
  uint4 vs, vb;                          // AUX8: the chunk's 8 scale / bias words
  uint32_t sr[kSkSteps], br[kSkSteps];  // otherwise one word per step
  auto issue_aux = [&](int k0) {
    if constexpr (AUX8) {
      vs = *reinterpret_cast<const uint4 *>(srow + (k0 >> 6));
      vb = *reinterpret_cast<const uint4 *>(brow + (k0 >> 6));
    } else {
#pragma unroll
      for (int u = 0; u < kSkSteps; ++u) {
        const int gi = ((k0 >> 6) + u) / p.gsteps;
        sr[u] = srow[gi];
        br[u] = brow[gi];
      }
    }
  };
  auto issue_w = [&](int u, int k0) { S::load_raw(wr[u], wrow, k0 + u * 64 + 16 * g); };
  // every load unconditional (rows past M - 1 repeat row M - 1), so the
  // compiler's wait counts stay exact
  auto issue_x = [&](int k0) {
#pragma unroll
    for (int m = 0; m < MX; ++m)
      xg[m] = *reinterpret_cast<const uint4 *>(p.x + (size_t)min(m, p.M - 1) * p.x_stride + k0 + 8 * lane);
  };
  auto store_x = [&](int buf) {
    uint16_t *t = sxw + buf * MX * kSkKc;
#pragma unroll
    for (int m = 0; m < MX; ++m) {
      const uint4 o = BITS == 4 ? __builtin_bit_cast(uint4, a_nibble_order(xg[m])) : xg[m];
      *reinterpret_cast<uint4 *>(t + m * kSkKc + 8 * swz(m, lane)) = o;
    }
  };

  UnpackConsts kc;
  kc.init();
  const bf16x8_t ones = mfma_ones();
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  // one chunk's eight steps from x tile `buf`; with REISSUE each step's
  // weight registers are loaded again for the chunk at knext once the step's
  // products have read them (the last chunk is peeled off, so no load is
  // conditional)
  auto chunk = [&](auto reissue, int buf, int knext) {
    constexpr bool REISSUE = decltype(reissue)::value;
    uint32_t scur[kSkSteps], bcur[kSkSteps];
    if constexpr (AUX8) {
      const uint32_t ws[4] = {vs.x, vs.y, vs.z, vs.w}, wb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
      for (int u = 0; u < kSkSteps; ++u) {
        scur[u] = (ws[u >> 1] >> (16 * (u & 1))) & 0xffffu;
        bcur[u] = (wb[u >> 1] >> (16 * (u & 1))) & 0xffffu;
      }
    } else {
#pragma unroll
      for (int u = 0; u < kSkSteps; ++u) {
        scur[u] = sr[u];
        bcur[u] = br[u];
      }
    }
    if constexpr (REISSUE) issue_aux(knext);
    const uint16_t *rowp = sxw + buf * MX * kSkKc + mr * kSkKc;
#pragma unroll
    for (int u = 0; u < kSkSteps; ++u) {
      bf16x8_t b0, b1, a0, a1;
      S::b_ops(wr[u], kc, b0, b1);
      S::a_ops(rowp, (u * 64 + 16 * g) >> 3, mr, a0, a1);
      const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      f32x4_t xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, ones, z, 0, 0, 0);
      xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, ones, xs, 0, 0, 0);
      f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, z, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, d, 0, 0, 0);
      // the reissue after the step's operands are formed, so the loads land
      // in place (no copies, and no waits, at the loop head); the barrier
      // keeps it there (the scheduler would otherwise sink every load of the
      // next chunk below the last step: one round trip per chunk)
      if constexpr (REISSUE) issue_w(u, knext);
      __builtin_amdgcn_sched_barrier(0);
      S::fold(acc, d, xs, aux_f32<FP16>(scur[u]), aux_f32<FP16>(bcur[u]));
    }
  };

  issue_x(kb);
  issue_aux(kb);
#pragma unroll
  for (int u = 0; u < kSkSteps; ++u) issue_w(u, kb);
  store_x(0);
  // x one chunk ahead (the last chunk's x is read again on the last round)
  issue_x(kb + min(1, p.cpw - 1) * kSkKc);
  for (int c = 0; c + 1 < p.cpw; ++c) {
    chunk(std::true_type{}, c & 1, kb + (c + 1) * kSkKc);
    store_x((c + 1) & 1);
    issue_x(kb + min(c + 2, p.cpw - 1) * kSkKc);
  }
  chunk(std::false_type{}, (p.cpw - 1) & 1, 0);

  // the waves' sums, added in K order
  __syncthreads();
  float *red = reinterpret_cast<float *>(kw_lds);  // [W][4][64]
#pragma unroll
  for (int i = 0; i < 4; ++i) red[(wave * 4 + i) * 64 + lane] = acc[i];
  __syncthreads();
  if (tid < 256) {
    const int i = tid >> 6, l = tid & 63;
    float s = 0.f;
    for (int w = 0; w < W; ++w) s += red[(w * 4 + i) * 64 + l];
    const int m = 4 * (l >> 4) + i, nn = blockIdx.x * 16 + (l & 15);
    if (m < p.M && nn < p.N) {
      if (p.y_bf16)
        reinterpret_cast<uint16_t *>(p.y)[(size_t)m * p.y_stride + nn] = (uint16_t)f32_to_bf16_rne(s);
      else
        reinterpret_cast<float *>(p.y)[(size_t)m * p.y_stride + nn] = s;
    }
  }
}

// waves per block for nch 512-code chunks, `blocks` blocks and MX x rows:
// the largest divisor of nch in [4, 8] that leaves each wave at least two
// chunks (the config-2 o product, 8 chunks: 6.7 us with 4 waves of two
// against 7.6 us with 8 of one) and keeps the whole grid resident on the 256
// CUs (the kernel holds up to about 200 VGPRs: two waves per SIMD, 2048
// waves; and the blocks of one CU share its 160 KB of LDS); failing that,
// the largest that fits; 0 if none
static int kwave_waves(int nch, int blocks, int MX) {
  const int per_cu = (blocks + 255) / 256;
  auto fits = [&](int w) {
    return nch % w == 0 && (long long)blocks * w <= 2048 &&
           (size_t)per_cu * kwave_lds_bytes(w, MX) <= 160 * 1024;
  };
  for (int w = kKwMaxW; w >= 4; --w)
    if (fits(w) && nch / w >= 2) return w;
  for (int w = kKwMaxW; w >= 4; --w)
    if (fits(w)) return w;
  return 0;
}

static int kwave_mx(int M) { return M <= 4 ? 4 : 8; }

bool affine_kwave_supported(const DevMat &m, int M) {
  if (!kSkinnyKwave) return false;
  if (m.bits < 4 || m.bits > 8 || m.bits == 7) return false;
  if (M < 3 || M > 8 || m.I % kSkKc != 0) return false;
  if (m.gs <= 0 || m.gs % 64 != 0 || m.I % m.gs != 0) return false;
  if (m.row_bytes != (long long)m.I * m.bits / 8) return false;
  const uintptr_t need = m.bits == 4 ? 7 : m.bits == 8 ? 15 : 3;
  if ((reinterpret_cast<uintptr_t>(m.w) & need) != 0 || (m.row_bytes & (long long)need) != 0) return false;
  // at least 256 blocks of 16 rows (one per CU); fewer rows fill the chip
  // better with the K split across blocks
  if (m.O < 16 * 256) return false;
  return kwave_waves(m.I / kSkKc, (m.O + 15) / 16, kwave_mx(M)) != 0;
}

template <int BITS, int MX, bool FP16, bool AUX8>
static void kwave_launch_t(const KwaveParams &p, int W, hipStream_t st) {
  auto *k = skinny_kwave_kernel<BITS, MX, FP16, AUX8>;
  const size_t lds = kwave_lds_bytes(W, MX);
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(k),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     (int)kwave_lds_bytes(kKwMaxW, MX));
  (void)attr;
  hipLaunchKernelGGL(k, dim3((p.N + 15) / 16), dim3(64 * W), lds, st, p);
}

template <int BITS, int MX>
static void kwave_launch_mx(const KwaveParams &p, int W, bool fp16, bool aux8, hipStream_t st) {
  if (fp16) {
    if (aux8) kwave_launch_t<BITS, MX, true, true>(p, W, st);
    else kwave_launch_t<BITS, MX, true, false>(p, W, st);
  } else {
    if (aux8) kwave_launch_t<BITS, MX, false, true>(p, W, st);
    else kwave_launch_t<BITS, MX, false, false>(p, W, st);
  }
}

template <int BITS>
static void kwave_launch_bits(const KwaveParams &p, int W, bool fp16, bool aux8, hipStream_t st) {
  if (kwave_mx(p.M) == 4) kwave_launch_mx<BITS, 4>(p, W, fp16, aux8, st);
  else kwave_launch_mx<BITS, 8>(p, W, fp16, aux8, st);
}

hipError_t launch_affine_kwave(const DevMat &m, const uint16_t *x, int x_stride, int M, void *y,
                               int y_stride, int y_bf16, hipStream_t st) {
  if (!affine_kwave_supported(m, M)) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return hipErrorInvalidValue;
  const int nch = m.I / kSkKc, W = kwave_waves(nch, (m.O + 15) / 16, kwave_mx(M));
  KwaveParams p;
  p.w = m.w;
  p.sc = m.sc;
  p.bi = m.bi;
  p.x = x;
  p.y = y;
  p.row_bytes = m.row_bytes;
  p.N = m.O;
  p.ng = m.ng;
  p.gsteps = m.gs / 64;
  p.x_stride = x_stride;
  p.M = M;
  p.cpw = nch / W;
  p.y_stride = y_stride;
  p.y_bf16 = y_bf16;
  const bool aux8 = m.gs == 64 && (m.ng % 8) == 0 &&
                    ((reinterpret_cast<uintptr_t>(m.sc) | reinterpret_cast<uintptr_t>(m.bi)) & 15) == 0;
  switch (m.bits) {
    case 4: kwave_launch_bits<4>(p, W, m.fp16, aux8, st); break;
    case 5: kwave_launch_bits<5>(p, W, m.fp16, aux8, st); break;
    case 6: kwave_launch_bits<6>(p, W, m.fp16, aux8, st); break;
    default: kwave_launch_bits<8>(p, W, m.fp16, aux8, st); break;
  }
  return hipGetLastError();
}

bool affine_splitk_supported(const DevMat &m, int M) {
  if (m.bits < 4 || m.bits > 8 || m.bits == 7) return false;
  if (M < 3 || M > 32 || m.I % kSkKc != 0) return false;
  if (m.gs <= 0 || m.gs % 64 != 0 || m.I % m.gs != 0) return false;
  if (m.row_bytes != (long long)m.I * m.bits / 8) return false;
  const uintptr_t need = m.bits == 4 ? 7 : m.bits == 8 ? 15 : 3;
  if ((reinterpret_cast<uintptr_t>(m.w) & need) != 0 || (m.row_bytes & (long long)need) != 0) return false;
  const size_t KS = (size_t)m.I / kSkKc;
  return KS * (size_t)M * (size_t)m.O <= kSkSlotFloats;
}

template <int BITS, int MT>
static void splitk_launch_t(const SplitParams &p, bool fp16, bool aux8, hipStream_t st) {
  const dim3 grid((p.N + kSkRows - 1) / kSkRows, p.K / kSkKc);
  if (fp16) {
    if (aux8) hipLaunchKernelGGL((skinny_splitk_kernel<BITS, MT, true, true>), grid, dim3(512), 0, st, p);
    else hipLaunchKernelGGL((skinny_splitk_kernel<BITS, MT, true, false>), grid, dim3(512), 0, st, p);
  } else {
    if (aux8) hipLaunchKernelGGL((skinny_splitk_kernel<BITS, MT, false, true>), grid, dim3(512), 0, st, p);
    else hipLaunchKernelGGL((skinny_splitk_kernel<BITS, MT, false, false>), grid, dim3(512), 0, st, p);
  }
}

template <int BITS>
static void splitk_launch_bits(const SplitParams &p, bool fp16, bool aux8, hipStream_t st) {
  if (p.M <= 16) splitk_launch_t<BITS, 1>(p, fp16, aux8, st);
  else splitk_launch_t<BITS, 2>(p, fp16, aux8, st);
}

static SlotRing g_sk_slots(kSkSlots);

hipError_t launch_affine_splitk(const DevMat &m, const uint16_t *x, int x_stride, int M, void *y,
                                int y_stride, int y_bf16, hipStream_t st) {
  if (!affine_splitk_supported(m, M)) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return hipErrorInvalidValue;
  SplitParams p;
  p.w = m.w;
  p.sc = m.sc;
  p.bi = m.bi;
  p.x = x;
  p.row_bytes = m.row_bytes;
  p.N = m.O;
  p.K = m.I;
  p.ng = m.ng;
  p.gsteps = m.gs / 64;
  p.x_stride = x_stride;
  p.M = M;
  SlotRing::Lease lease;
  {
    const hipError_t le = g_sk_slots.take(st, lease);
    if (le != hipSuccess) return le;
  }
  p.slot = lease.slot();
  p.part_off = 0;
  // 16-byte runs of eight u16 scale/bias words per 512 codes
  const bool aux8 = m.gs == 64 && (m.ng % 8) == 0 &&
                    ((reinterpret_cast<uintptr_t>(m.sc) | reinterpret_cast<uintptr_t>(m.bi)) & 15) == 0;
  switch (m.bits) {
    case 4: splitk_launch_bits<4>(p, m.fp16, aux8, st); break;
    case 5: splitk_launch_bits<5>(p, m.fp16, aux8, st); break;
    case 6: splitk_launch_bits<6>(p, m.fp16, aux8, st); break;
    default: splitk_launch_bits<8>(p, m.fp16, aux8, st); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t MN = (size_t)M * m.O;
  size_t blocks = (MN + 255) / 256;
  if (blocks > 2048) blocks = 2048;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p.slot, m.I / kSkKc, M,
                     m.O, y, y_stride, y_bf16);
  e = hipGetLastError();
  const hipError_t le = lease.done();
  return e != hipSuccess ? e : le;
}

template <int BITS, int MT>
static void splitk_multi_launch_t(const SplitMulti &mp, int KS, bool fp16, bool aux8, hipStream_t st) {
  const dim3 grid(mp.start[mp.n], KS);
  if (fp16) {
    if (aux8) hipLaunchKernelGGL((skinny_splitk_multi_kernel<BITS, MT, true, true>), grid, dim3(512), 0, st, mp);
    else hipLaunchKernelGGL((skinny_splitk_multi_kernel<BITS, MT, true, false>), grid, dim3(512), 0, st, mp);
  } else {
    if (aux8) hipLaunchKernelGGL((skinny_splitk_multi_kernel<BITS, MT, false, true>), grid, dim3(512), 0, st, mp);
    else hipLaunchKernelGGL((skinny_splitk_multi_kernel<BITS, MT, false, false>), grid, dim3(512), 0, st, mp);
  }
}

template <int BITS>
static void splitk_multi_launch_bits(const SplitMulti &mp, int KS, int M, bool fp16, bool aux8,
                                     hipStream_t st) {
  if (M <= 16) splitk_multi_launch_t<BITS, 1>(mp, KS, fp16, aux8, st);
  else splitk_multi_launch_t<BITS, 2>(mp, KS, fp16, aux8, st);
}

bool affine_splitk_multi_supported(const DevMat *ms, int n, int M) {
  if (n < 1 || n > kSkMultiMax) return false;
  size_t floats = 0;
  for (int i = 0; i < n; ++i) {
    const DevMat &m = ms[i];
    if (!affine_splitk_supported(m, M)) return false;
    if (m.I != ms[0].I || m.bits != ms[0].bits || m.gs != ms[0].gs || m.fp16 != ms[0].fp16) return false;
    floats += (size_t)(m.I / kSkKc) * M * m.O;
  }
  return floats <= kSkSlotFloats;
}

// ys[i][M][O_i] = x . W_i^T for products that share x: one K-split launch and
// one reduce launch for all of them (gate/up, q/k/v) instead of two launches
// per product.
hipError_t launch_affine_splitk_multi(const DevMat *ms, int n, const uint16_t *x, int x_stride, int M,
                                      void *const *ys, int y_bf16, hipStream_t st, int swiglu_stride) {
  const bool swiglu = swiglu_stride > 0;
  if (swiglu && (n != 2 || ms[0].O != ms[1].O)) return hipErrorInvalidValue;
  if (!affine_splitk_multi_supported(ms, n, M)) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return hipErrorInvalidValue;
  SplitMulti mp{};
  ReduceMulti r{};
  const int KS = ms[0].I / kSkKc;
  SlotRing::Lease lease;
  {
    const hipError_t le = g_sk_slots.take(st, lease);
    if (le != hipSuccess) return le;
  }
  const int slot = lease.slot();
  bool aux8 = true;
  size_t off = 0;
  for (int i = 0; i < n; ++i) {
    const DevMat &m = ms[i];
    aux8 = aux8 && m.gs == 64 && (m.ng % 8) == 0 &&
           ((reinterpret_cast<uintptr_t>(m.sc) | reinterpret_cast<uintptr_t>(m.bi)) & 15) == 0;
    SplitParams &p = mp.m[i];
    p.w = m.w;
    p.sc = m.sc;
    p.bi = m.bi;
    p.x = x;
    p.row_bytes = m.row_bytes;
    p.N = m.O;
    p.K = m.I;
    p.ng = m.ng;
    p.gsteps = m.gs / 64;
    p.x_stride = x_stride;
    p.M = M;
    p.slot = slot;
    p.part_off = off;
    r.y[i] = ys[i];
    r.part_off[i] = off;
    r.N[i] = m.O;
    r.y_stride[i] = m.O;
    off += (size_t)KS * M * m.O;
    mp.start[i + 1] = mp.start[i] + (m.O + kSkRows - 1) / kSkRows;
    r.start[i + 1] = r.start[i] + M * m.O;
  }
  mp.n = r.n = n;
  r.KS = KS;
  r.M = M;
  r.slot = slot;
  r.y_bf16 = y_bf16;
  r.swiglu = swiglu ? 1 : 0;
  if (swiglu) r.y_stride[0] = swiglu_stride;
  switch (ms[0].bits) {
    case 4: splitk_multi_launch_bits<4>(mp, KS, M, ms[0].fp16, aux8, st); break;
    case 5: splitk_multi_launch_bits<5>(mp, KS, M, ms[0].fp16, aux8, st); break;
    case 6: splitk_multi_launch_bits<6>(mp, KS, M, ms[0].fp16, aux8, st); break;
    default: splitk_multi_launch_bits<8>(mp, KS, M, ms[0].fp16, aux8, st); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  size_t blocks = ((size_t)(swiglu ? r.start[1] : r.start[n]) + 255) / 256;
  if (blocks > 2048) blocks = 2048;
  hipLaunchKernelGGL(splitk_reduce_multi_kernel, dim3((unsigned)blocks), dim3(256), 0, st, r);
  e = hipGetLastError();
  const hipError_t le = lease.done();
  return e != hipSuccess ? e : le;
}

// The full-K pair serves gate/up pairs of one geometry whose 64-row blocks
// cover at least three quarters of the CUs (N >= 12288), at up to 16 tokens
// (one 16-token MFMA tile: more would spill registers); other pairs keep the
// K split.
bool swiglu_fullk_supported(const DevMat &g, const DevMat &u, int M) {
  if (M > 16) return false;
  if (!affine_splitk_supported(g, M) || !affine_splitk_supported(u, M)) return false;
  if (g.I != u.I || g.O != u.O || g.bits != u.bits || g.gs != u.gs || g.fp16 != u.fp16 ||
      g.row_bytes != u.row_bytes)
    return false;
  return g.O >= 12288;
}

template <int BITS, int MT>
static void fullk_launch_t(const FullKParams &p, bool fp16, bool aux8, hipStream_t st) {
  const dim3 grid((p.N + kFkRows - 1) / kFkRows);
  if (fp16) {
    if (aux8) hipLaunchKernelGGL((swiglu_fullk_kernel<BITS, MT, true, true>), grid, dim3(kFkThreads), 0, st, p);
    else hipLaunchKernelGGL((swiglu_fullk_kernel<BITS, MT, true, false>), grid, dim3(kFkThreads), 0, st, p);
  } else {
    if (aux8) hipLaunchKernelGGL((swiglu_fullk_kernel<BITS, MT, false, true>), grid, dim3(kFkThreads), 0, st, p);
    else hipLaunchKernelGGL((swiglu_fullk_kernel<BITS, MT, false, false>), grid, dim3(kFkThreads), 0, st, p);
  }
}

template <int BITS>
static void fullk_launch_bits(const FullKParams &p, bool fp16, bool aux8, hipStream_t st) {
  fullk_launch_t<BITS, 1>(p, fp16, aux8, st);
}

hipError_t launch_swiglu_fullk(const DevMat &g, const DevMat &u, const uint16_t *x, int x_stride, int M,
                               void *h, int h_stride, int h_bf16, hipStream_t st) {
  if (!swiglu_fullk_supported(g, u, M)) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return hipErrorInvalidValue;
  FullKParams p;
  p.w[0] = g.w;
  p.w[1] = u.w;
  p.sc[0] = g.sc;
  p.sc[1] = u.sc;
  p.bi[0] = g.bi;
  p.bi[1] = u.bi;
  p.x = x;
  p.h = h;
  p.row_bytes = g.row_bytes;
  p.N = g.O;
  p.K = g.I;
  p.ng = g.ng;
  p.gsteps = g.gs / 64;
  p.x_stride = x_stride;
  p.M = M;
  p.h_stride = h_stride;
  p.h_bf16 = h_bf16;
  const bool aux8 = g.gs == 64 && (g.ng % 8) == 0 &&
                    ((reinterpret_cast<uintptr_t>(g.sc) | reinterpret_cast<uintptr_t>(g.bi) |
                      reinterpret_cast<uintptr_t>(u.sc) | reinterpret_cast<uintptr_t>(u.bi)) & 15) == 0;
  switch (g.bits) {
    case 4: fullk_launch_bits<4>(p, g.fp16, aux8, st); break;
    case 5: fullk_launch_bits<5>(p, g.fp16, aux8, st); break;
    case 6: fullk_launch_bits<6>(p, g.fp16, aux8, st); break;
    default: fullk_launch_bits<8>(p, g.fp16, aux8, st); break;
  }
  return hipGetLastError();
}

}  // namespace lh
