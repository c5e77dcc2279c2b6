// Prefill / large-batch product with MLX-affine weights on MFMA (gfx950):
//   y[m][n] = sum_k x[m][k] * bf16(code[n][k] * scale[n][k/gs] + bias[n][k/gs])
// the semantics of logan-metal's QMM (backend_metal.mm:1480-1560: each
// dequantised weight rounded to bf16 in threadgroup memory, bf16 x bf16
// products accumulated in f32, bf16 output).
//
// One block computes a 64 x 64 tile of y (4 waves, each a 32 x 32 tile with
// v_mfma_f32_32x32x16_bf16). Per 64-wide k step the block dequantises its 64
// weight rows into LDS (codes -> f32 fma -> v_cvt_pk_bf16_f32), while every
// lane loads its x operands straight from global memory (x rows are re-read
// by the N/64 blocks of a row block and stay in L2). Operand layout of the
// 32x32x16 instruction (checked on the device): lane l holds row (col) l % 32
// and 8 consecutive k at offset 8 * (l / 32) of each 16-wide k slice; the
// result's element i of lane l is row 8 * (i / 4) + 4 * (l / 32) + i % 4,
// column l % 32.
#include <algorithm>
#include <atomic>

#include "affine_dev.hpp"
#include "lh_internal.hpp"

namespace lh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct GemmParams {
  const uint8_t *w;
  const uint16_t *sc;
  const uint16_t *bi;
  const uint16_t *x;
  void *y;
  long long row_bytes;
  int M, N, K, ng, gs, fp16, x_stride, y_stride, y_bf16;
};

constexpr int kTile = 64;        // block tile (m and n) and k step
constexpr int kLdsStride = 72;   // bf16 per LDS row: 64 + 8 pad (no bank conflicts)

// Codes per dequantising thread: 16 (4 per row of 64) for widths whose
// 16-code runs start on a dword boundary; 5-bit runs of 32 codes (2 per row).
template <int BITS>
struct DeqGeom {
  static constexpr int CPT = BITS == 5 ? 32 : 16;
  static constexpr int THREADS = kTile * (kTile / CPT);  // 256 or 128
  static constexpr int DW = CPT * BITS / 32;             // dwords of codes
};

template <int BITS>
__device__ __forceinline__ uint32_t code_of(const uint32_t (&w)[DeqGeom<BITS>::DW], int j) {
  const int bit = j * BITS, i = bit >> 5, sh = bit & 31;
  uint32_t c = w[i] >> sh;
  if (sh + BITS > 32) c |= w[i + 1] << (32 - sh);
  return c & ((1u << BITS) - 1u);
}

// Split-K: the blocks of one tile that share a k range write f32 partial
// sums part[z][m][n] into one of kQSlots module-scope slots (taken round-robin
// per call, so calls whose executions overlap on one device stay correct
// while at most kQSlots are in flight); qmm_reduce_kernel adds them in z
// order and writes y. slot < 0: one k range, y written directly.
constexpr int kQSlots = 2;
constexpr size_t kQSlotFloats = size_t(1) << 23;  // 32 MB per slot
static __device__ __align__(256) float g_qmm_part[kQSlots * kQSlotFloats];

__device__ __forceinline__ void qmm_store(const GemmParams &p, int slot, int z, int m, int n,
                                          float v) {
  if (slot >= 0)
    g_qmm_part[(size_t)slot * kQSlotFloats + ((size_t)z * p.M + m) * p.N + n] = v;
  else if (p.y_bf16)
    reinterpret_cast<__bf16 *>(p.y)[(size_t)m * p.y_stride + n] = (__bf16)v;
  else
    reinterpret_cast<float *>(p.y)[(size_t)m * p.y_stride + n] = v;
}

__global__ __launch_bounds__(256) void qmm_reduce_kernel(GemmParams p, int slot, int KS) {
  const float *part = g_qmm_part + (size_t)slot * kQSlotFloats;
  const size_t MN = (size_t)p.M * p.N;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < MN; i += (size_t)gridDim.x * 256) {
    float v[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) v[z] = z < KS ? part[z * MN + i] : 0.f;
    float s = v[0];
#pragma unroll
    for (int z = 1; z < 16; ++z) s += z < KS ? v[z] : 0.f;  // in k order
    const int m = (int)(i / p.N), n = (int)(i % p.N);
    if (p.y_bf16)
      reinterpret_cast<__bf16 *>(p.y)[(size_t)m * p.y_stride + n] = (__bf16)s;
    else
      reinterpret_cast<float *>(p.y)[(size_t)m * p.y_stride + n] = s;
  }
}

template <int BITS>
__global__ __launch_bounds__(256) void affine_qmm_kernel(GemmParams p, int ksteps, int slot) {
  using G = DeqGeom<BITS>;
  __shared__ __align__(16) __bf16 sW[kTile * kLdsStride];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bm0 = blockIdx.x * kTile, bn0 = blockIdx.y * kTile;
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5, l32 = lane & 31;

  // dequantising role: row n = tid / (64 / CPT), codes [kq, kq + CPT)
  const int dn = tid / (kTile / G::CPT);
  const int kq = (tid % (kTile / G::CPT)) * G::CPT;
  const bool deq = tid < G::THREADS;
  const int nrow = min(bn0 + dn, p.N - 1);
  const uint8_t *wrow = p.w + (size_t)nrow * p.row_bytes;
  const uint16_t *srow = p.sc + (size_t)nrow * p.ng;
  const uint16_t *brow = p.bi + (size_t)nrow * p.ng;

  // x operand row of this lane (clamped; rows past M are never stored)
  const int xm = min(bm0 + wm * 32 + l32, p.M - 1);
  const uint16_t *xrow = p.x + (size_t)xm * p.x_stride;

  // software pipeline: the loads of step k0 + 64 are issued before step k0 is
  // dequantised and multiplied
  // (two register buffers with compile-time indices: the loop body is
  // unrolled by two steps)
  uint32_t wv0[G::DW], wv1[G::DW];
  uint32_t sr0 = 0, br0 = 0, sr1 = 0, br1 = 0;
  uint4 xa0[4], xa1[4];
  auto issue = [&](int k0, uint32_t (&wv)[G::DW], uint32_t &sraw, uint32_t &braw, uint4 (&xa)[4]) {
    if (deq) {
      const uint32_t *src = reinterpret_cast<const uint32_t *>(wrow + (size_t)(k0 + kq) * BITS / 8);
#pragma unroll
      for (int i = 0; i < G::DW; ++i) wv[i] = src[i];
      const int gidx = (k0 + kq) / p.gs;
      sraw = srow[gidx];
      braw = brow[gidx];
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      xa[ks] = *reinterpret_cast<const uint4 *>(xrow + k0 + 16 * ks + 8 * half);
  };
  f32x16 acc = {};
  auto step = [&](const uint32_t (&wv)[G::DW], uint32_t sraw, uint32_t braw, const uint4 (&xa)[4]) {
    if (deq) {
      const float s = aux_to_f32_sel(sraw, p.fp16), b = aux_to_f32_sel(braw, p.fp16);
      uint32_t packed[G::CPT / 2];
#pragma unroll
      for (int j = 0; j < G::CPT; j += 2) {
        bf16x2 v;
        v[0] = (__bf16)fmaf((float)code_of<BITS>(wv, j), s, b);
        v[1] = (__bf16)fmaf((float)code_of<BITS>(wv, j + 1), s, b);
        packed[j / 2] = __builtin_bit_cast(uint32_t, v);
      }
      uint4 *dst = reinterpret_cast<uint4 *>(sW + dn * kLdsStride + kq);
#pragma unroll
      for (int v = 0; v < G::CPT / 8; ++v)
        dst[v] = make_uint4(packed[4 * v], packed[4 * v + 1], packed[4 * v + 2], packed[4 * v + 3]);
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 a = __builtin_bit_cast(bf16x8, xa[ks]);
      const bf16x8 b = *reinterpret_cast<const bf16x8 *>(sW + (wn * 32 + l32) * kLdsStride + 16 * ks +
                                                        8 * half);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
    }
    __syncthreads();
  };
  const int z = blockIdx.z;
  const int kb = z * ksteps * kTile, ke = min(p.K, kb + ksteps * kTile);
  issue(kb, wv0, sr0, br0, xa0);
  for (int k0 = kb; k0 < ke; k0 += 2 * kTile) {
    if (k0 + kTile < ke) issue(k0 + kTile, wv1, sr1, br1, xa1);
    __builtin_amdgcn_sched_barrier(0);
    step(wv0, sr0, br0, xa0);
    if (k0 + kTile < ke) {
      if (k0 + 2 * kTile < ke) issue(k0 + 2 * kTile, wv0, sr0, br0, xa0);
      __builtin_amdgcn_sched_barrier(0);
      step(wv1, sr1, br1, xa1);
    }
  }
  // store: element i of this lane is (row 8*(i/4) + 4*half + i%4, col l32)
  const int n = bn0 + wn * 32 + l32;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int m = bm0 + wm * 32 + 8 * (i / 4) + 4 * half + (i % 4);
    if (m < p.M && n < p.N) qmm_store(p, slot, z, m, n, acc[i]);
  }
}

// ---------------------------------------------------------------------------
// Large tiles: 128 x 128 output per 256-thread block (each wave 64 x 64 as
// 2 x 2 MFMA tiles), so every weight is dequantised once per 128 tokens. Per
// 64-k step the block writes the x tile and the dequantised W tile into one
// of two LDS stages while the MFMAs read the other; the next step's global
// loads are issued into registers before the current step's MFMAs, one
// barrier per step. (x read straight into MFMA operand registers instead of
// through LDS measured 1.7x slower: each load instruction then touches 32
// rows.) Blocks are numbered so that the M tiles of one N tile share an XCD
// (block id mod 8) and meet the weight tile in that XCD's L2.
constexpr int kQ2 = 128;     // tile rows (m) and columns (n)
constexpr int kQ2Ld = 72;    // bf16 per LDS row: 64 + 8 pad
#ifndef QMM_MIN_TILES
#define QMM_MIN_TILES 192
#endif
constexpr int kQ2MinTiles = QMM_MIN_TILES;
constexpr int kQTargetBlocks = 512;  // about two blocks per CU
static std::atomic<unsigned> g_qmm_next{0};

template <int BITS>
__global__ __launch_bounds__(256) void affine_qmm128_kernel(GemmParams p, int mtiles, int ntiles,
                                                            int ksteps, int slot) {
  // two stages: step s reads stage s % 2 while stage (s + 1) % 2 is filled
  __shared__ __align__(16) __bf16 sA[2][kQ2 * kQ2Ld];
  __shared__ __align__(16) __bf16 sB[2][kQ2 * kQ2Ld];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5, l32 = lane & 31;
  // XCD-grouped tile order
  const int L = blockIdx.x;
  const int grp = L / (8 * mtiles), rem = L % (8 * mtiles);
  const int nt = grp * 8 + rem % 8, mt = rem / 8;
  if (nt >= ntiles) return;
  const int bm0 = mt * kQ2, bn0 = nt * kQ2;

  // loader role: row lr of both tiles, codes / activations [32 lh, 32 lh + 32)
  const int lr = tid >> 1, lh = tid & 1;
  const uint16_t *xrow = p.x + (size_t)min(bm0 + lr, p.M - 1) * p.x_stride + 32 * lh;
  const int wrw = min(bn0 + lr, p.N - 1);
  const uint8_t *wrow = p.w + (size_t)wrw * p.row_bytes;
  const uint16_t *srow = p.sc + (size_t)wrw * p.ng;
  const uint16_t *brow = p.bi + (size_t)wrw * p.ng;
  struct Loads {
    uint4 x0, x1, x2, x3;
    uint32_t w[BITS];
    uint32_t s, b;
  };
  auto issue = [&](int k0) {
    Loads r;
    const uint4 *xs = reinterpret_cast<const uint4 *>(xrow + k0);
    r.x0 = xs[0];
    r.x1 = xs[1];
    r.x2 = xs[2];
    r.x3 = xs[3];
    load_chunk<BITS>(r.w, wrow + (size_t)(k0 + 32 * lh) * BITS / 8);
    const int gi = (k0 + 32 * lh) / p.gs;
    r.s = srow[gi];
    r.b = brow[gi];
    return r;
  };
  auto commit = [&](const Loads &r, int st) {
    uint4 *da = reinterpret_cast<uint4 *>(sA[st] + lr * kQ2Ld + 32 * lh);
    da[0] = r.x0;
    da[1] = r.x1;
    da[2] = r.x2;
    da[3] = r.x3;
    const float s = aux_to_f32_sel(r.s, p.fp16), b = aux_to_f32_sel(r.b, p.fp16);
    uint32_t pk[16];
#pragma unroll
    for (int j = 0; j < 32; j += 2) {
      // codes j, j + 1 of the 32-code chunk (LSB-first stream)
      uint32_t c[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int bit = (j + q) * BITS, i = bit >> 5, sh = bit & 31;
        uint32_t v = r.w[i] >> sh;
        if (sh + BITS > 32) v |= r.w[i + 1] << (32 - sh);
        c[q] = v & ((1u << BITS) - 1u);
      }
      bf16x2 v;
      v[0] = (__bf16)fmaf((float)c[0], s, b);
      v[1] = (__bf16)fmaf((float)c[1], s, b);
      pk[j / 2] = __builtin_bit_cast(uint32_t, v);
    }
    uint4 *db = reinterpret_cast<uint4 *>(sB[st] + lr * kQ2Ld + 32 * lh);
#pragma unroll
    for (int v = 0; v < 4; ++v) db[v] = make_uint4(pk[4 * v], pk[4 * v + 1], pk[4 * v + 2], pk[4 * v + 3]);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
  auto mfma_step = [&](int st) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const bf16x8 *>(sA[st] + (wm * 64 + 32 * i + l32) * kQ2Ld + 16 * ks +
                                                 8 * half);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const bf16x8 *>(sB[st] + (wn * 64 + 32 * j + l32) * kQ2Ld + 16 * ks +
                                                 8 * half);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };
  // per step: the MFMAs read stage s % 2 while the next step's operands
  // (loaded during the previous step) are dequantised into the other stage,
  // then the loads of step s + 2 are issued; one barrier per step (stage
  // (s + 1) % 2 was last read in step s - 1, before that step's barrier).
  // (Loads issued three steps ahead measured no faster.)
  const int z = blockIdx.y;
  const int kb = z * ksteps * 64, nst = (min(p.K, kb + ksteps * 64) - kb) / 64;
  Loads cur = issue(kb);
  commit(cur, 0);
  cur = issue(kb + 64 * min(1, nst - 1));
  __syncthreads();
  for (int s = 0; s < nst; ++s) {
    mfma_step(s & 1);
    if (s + 1 < nst) {
      commit(cur, (s + 1) & 1);
      cur = issue(kb + 64 * min(s + 2, nst - 1));
    }
    __syncthreads();
  }
  // element e of tile (i, j): row 32 i + 8 (e / 4) + 4 half + e % 4, column 32 j + l32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = bn0 + wn * 64 + 32 * j + l32;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = bm0 + wm * 64 + 32 * i + 8 * (e / 4) + 4 * half + (e % 4);
        if (m < p.M && n < p.N) qmm_store(p, slot, z, m, n, acc[i][j][e]);
      }
    }
}

bool affine_qmm_supported(const DevMat &m) {
  if (!(m.bits == 4 || m.bits == 5 || m.bits == 6 || m.bits == 8)) return false;
  if (m.I <= 0 || m.I % kTile != 0 || m.O <= 0) return false;
  if (m.gs <= 0 || m.gs % 32 != 0 || m.I % m.gs != 0) return false;
  if (m.row_bytes != (long long)m.I * m.bits / 8) return false;
  if ((m.row_bytes & 3) != 0 || (reinterpret_cast<uintptr_t>(m.w) & 3) != 0) return false;
  return true;
}

hipError_t launch_affine_qmm(const DevMat &m, const uint16_t *x, int x_stride, int M, void *y,
                             int y_stride, int y_bf16, hipStream_t st) {
  if (!affine_qmm_supported(m) || M <= 0) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return hipErrorInvalidValue;
  GemmParams p;
  p.w = m.w;
  p.sc = m.sc;
  p.bi = m.bi;
  p.x = x;
  p.y = y;
  p.row_bytes = m.row_bytes;
  p.M = M;
  p.N = m.O;
  p.K = m.I;
  p.ng = m.ng;
  p.gs = m.gs;
  p.fp16 = m.fp16;
  p.x_stride = x_stride;
  p.y_stride = y_stride;
  p.y_bf16 = y_bf16;
  // Large tiles when their grid alone keeps the chip busy, else 64 x 64
  // tiles (four times the blocks); grids still short of about two blocks per
  // CU split K as well (at most 16 ways, partials within one slot).
  const int ksteps_all = m.I / 64;
  const int mt = (M + kQ2 - 1) / kQ2, nt = (m.O + kQ2 - 1) / kQ2;
  const bool big = M > kTile && m.O >= kQ2 && (mt * nt >= kQ2MinTiles || m.I >= 512);
  const int tiles = big ? mt * nt : ((M + kTile - 1) / kTile) * ((m.O + kTile - 1) / kTile);
  int split = 1;
  while (split < 16 && tiles * split < kQTargetBlocks && 2 * split <= ksteps_all &&
         (size_t)(2 * split) * M * m.O <= kQSlotFloats)
    split *= 2;
  const int ksteps = (ksteps_all + split - 1) / split;
  split = (ksteps_all + ksteps - 1) / ksteps;
  const int slot = split > 1 ? (int)(g_qmm_next.fetch_add(1, std::memory_order_relaxed) % kQSlots) : -1;
  if (big) {
    const dim3 grid(((nt + 7) / 8) * 8 * mt, split);
    switch (m.bits) {
      case 4: hipLaunchKernelGGL(affine_qmm128_kernel<4>, grid, dim3(256), 0, st, p, mt, nt, ksteps, slot); break;
      case 5: hipLaunchKernelGGL(affine_qmm128_kernel<5>, grid, dim3(256), 0, st, p, mt, nt, ksteps, slot); break;
      case 6: hipLaunchKernelGGL(affine_qmm128_kernel<6>, grid, dim3(256), 0, st, p, mt, nt, ksteps, slot); break;
      case 8: hipLaunchKernelGGL(affine_qmm128_kernel<8>, grid, dim3(256), 0, st, p, mt, nt, ksteps, slot); break;
    }
  } else {
    const dim3 grid((M + kTile - 1) / kTile, (m.O + kTile - 1) / kTile, split);
    switch (m.bits) {
      case 4: hipLaunchKernelGGL(affine_qmm_kernel<4>, grid, dim3(256), 0, st, p, ksteps, slot); break;
      case 5: hipLaunchKernelGGL(affine_qmm_kernel<5>, grid, dim3(256), 0, st, p, ksteps, slot); break;
      case 6: hipLaunchKernelGGL(affine_qmm_kernel<6>, grid, dim3(256), 0, st, p, ksteps, slot); break;
      case 8: hipLaunchKernelGGL(affine_qmm_kernel<8>, grid, dim3(256), 0, st, p, ksteps, slot); break;
    }
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || split == 1) return e;
  const size_t mn = (size_t)M * m.O;
  const int rblocks = (int)std::min<size_t>((mn + 255) / 256, 4096);
  hipLaunchKernelGGL(qmm_reduce_kernel, dim3(rblocks), dim3(256), 0, st, p, slot, split);
  return hipGetLastError();
}

}  // namespace lh
