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
#include "mfma_dev.hpp"

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
// sums part[z][m][n] into one of kQSlots module-scope slots (a SlotRing
// lease: calls on any streams that would overlap on a slot are ordered on
// the device); qmm_reduce_kernel adds them in z order and writes y.
// slot < 0: one k range, y written directly.
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

// all KS loads of a thread issued before the first add; V = 4 when rows are
// a multiple of 4 columns (16-byte partial loads), the y store then one 8- or
// 16-byte store when y rows are 16-byte aligned (yvec)
template <int KS, int V>
__global__ __launch_bounds__(256) void qmm_reduce_kernel(GemmParams p, int slot, int yvec) {
  typedef float fv __attribute__((ext_vector_type(V)));
  const float *part = g_qmm_part + (size_t)slot * kQSlotFloats;
  const size_t MN = (size_t)p.M * p.N, nv = MN / V;
  for (size_t v = (size_t)blockIdx.x * 256 + threadIdx.x; v < nv; v += (size_t)gridDim.x * 256) {
    const size_t i = v * V;
    fv t[KS];
#pragma unroll
    for (int z = 0; z < KS; ++z) t[z] = __builtin_nontemporal_load(reinterpret_cast<const fv *>(part + z * MN + i));
    fv s = t[0];
#pragma unroll
    for (int z = 1; z < KS; ++z) s += t[z];  // in k order
    const size_t o = (i / p.N) * p.y_stride + i % p.N;
    if (p.y_bf16) {
      __bf16 *y = reinterpret_cast<__bf16 *>(p.y) + o;
      if constexpr (V == 4) {
        if (yvec) {
          typedef __bf16 b4 __attribute__((ext_vector_type(4)));
          *reinterpret_cast<b4 *>(y) = b4{(__bf16)s[0], (__bf16)s[1], (__bf16)s[2], (__bf16)s[3]};
          continue;
        }
      }
#pragma unroll
      for (int e = 0; e < V; ++e) y[e] = (__bf16)s[e];
    } else {
      float *y = reinterpret_cast<float *>(p.y) + o;
      if constexpr (V == 4) {
        if (yvec) {
          *reinterpret_cast<fv *>(y) = s;
          continue;
        }
      }
#pragma unroll
      for (int e = 0; e < V; ++e) y[e] = s[e];
    }
  }
}

template <int V>
static void launch_qmm_reduce(const GemmParams &p, int slot, int KS, hipStream_t st) {
  const size_t nv = (size_t)p.M * p.N / V;
  const dim3 grid((unsigned)std::min<size_t>((nv + 255) / 256, 4096));
  const int es = p.y_bf16 ? 2 : 4;
  const int yvec = (reinterpret_cast<uintptr_t>(p.y) & 15) == 0 && ((long long)p.y_stride * es) % 16 == 0;
  switch (KS) {
#define LH_QRED(k) \
  case k: hipLaunchKernelGGL((qmm_reduce_kernel<k, V>), grid, dim3(256), 0, st, p, slot, yvec); break;
    LH_QRED(2) LH_QRED(3) LH_QRED(4) LH_QRED(5) LH_QRED(6) LH_QRED(7) LH_QRED(8) LH_QRED(9)
    LH_QRED(10) LH_QRED(11) LH_QRED(12) LH_QRED(13) LH_QRED(14) LH_QRED(15) LH_QRED(16)
#undef LH_QRED
    default: break;
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
static SlotRing g_qmm_slots(kQSlots);

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

// ---------------------------------------------------------------------------
// 256 x 128 tiles for M >= 256, over up to kQMultiMax matrices that read the
// same x (q/k/v, qkvz/ba) in one grid. 512 threads, waves 4 (m) x 2 (n), each
// 64 x 64 as 2 x 2 v_mfma_f32_32x32x16_bf16 tiles, so every dequantised weight
// serves 256 tokens (half the VALU per MFMA of the 128-row tiles).
//   * step s's x rows and the codes / scale / bias of its weights are loaded
//     into one of two register sets two steps ahead, then written to LDS
//     stage s & 1 (the weights dequantised to bf16) one step ahead, and
//     multiplied after the barrier that follows: one barrier per step, and
//     the loads of the next two steps stay in flight across it;
//   * LDS rows are 144 bytes (64 bf16 + 16 bytes of padding), so the 16
//     lanes an operand read serves per clock (rows r .. r + 15 at one k
//     offset) start on 16 different 4-bank groups of the 64 banks.
constexpr int kQ3M = 256, kQ3N = 128;
constexpr int kQ3Ld = 72;  // u16 per LDS row: 64 + 8 of padding
constexpr int kQMultiMax = 8;

struct QmmMat {
  const uint8_t *w;
  const uint16_t *sc;
  const uint16_t *bi;
  void *y;
  long long row_bytes;
  int N, ng, y_stride, col0;  // col0: first column of this matrix in split partial rows
};
struct QmmMulti {
  QmmMat m[kQMultiMax];
  int tile_start[kQMultiMax + 1];  // first 128-column tile of matrix i
  const uint16_t *x;
  int n, M, K, gs, fp16, x_stride, y_bf16, part_N;
  int vec;  // bit 0: y rows take 16-byte stores; bit 1: partial rows do
};

template <int BITS>
struct Q3Raw {
  uint32_t w[BITS == 4 ? 2 : BITS == 8 ? 4 : 3];
  uint32_t s, b;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t q3_rsrc(const void *p, long long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                           (int)(bytes > 0x7fffffffLL ? 0x7fffffffLL : bytes),
                                           0x00020000);
}

// 16 codes [k, k + 16) of a row (k a multiple of 16) and their group's scale
// and bias: exactly three buffer loads
template <int BITS>
__device__ __forceinline__ void q3_load(Q3Raw<BITS> &r, __amdgpu_buffer_rsrc_t wr,
                                        __amdgpu_buffer_rsrc_t sr, __amdgpu_buffer_rsrc_t br,
                                        int rowoff, int poff, int k) {
  if constexpr (BITS == 4) {
    const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wr, rowoff + (k >> 1), 0, 0));
    r.w[0] = v.x;
    r.w[1] = v.y;
  } else if constexpr (BITS == 8) {
    const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, rowoff + k, 0, 0));
    r.w[0] = v.x;
    r.w[1] = v.y;
    r.w[2] = v.z;
    r.w[3] = v.w;
  } else {
    typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
    const u32x3 v = __builtin_bit_cast(
        u32x3, __builtin_amdgcn_raw_buffer_load_b96(wr, rowoff + 4 * ((k * BITS) >> 5), 0, 0));
    r.w[0] = v.x;
    r.w[1] = v.y;
    r.w[2] = v.z;
  }
  r.s = __builtin_amdgcn_raw_buffer_load_b16(sr, poff, 0, 0);
  r.b = __builtin_amdgcn_raw_buffer_load_b16(br, poff, 0, 0);
}

// bf16(code * s + b) of the 16 codes, packed in pairs (code order); sh is the
// bit where the first 5-bit code starts (0 or 16)
template <int BITS>
__device__ __forceinline__ void q3_dequant(const Q3Raw<BITS> &r, int sh, bool fp16, uint32_t (&pk)[8]) {
  const float s = aux_to_f32_sel(r.s, fp16), b = aux_to_f32_sel(r.b, fp16);
  float f[16];
  if constexpr (BITS == 4) {
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const uint32_t lo = r.w[d] & 0x0F0F0F0Fu, hi = (r.w[d] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[8 * d + 2 * i] = (float)((lo >> (8 * i)) & 255u);
        f[8 * d + 2 * i + 1] = (float)((hi >> (8 * i)) & 255u);
      }
    }
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) f[4 * d + i] = (float)((r.w[d] >> (8 * i)) & 255u);
  } else {
    const uint32_t win[3] = {__builtin_amdgcn_alignbit(r.w[1], r.w[0], sh),
                             __builtin_amdgcn_alignbit(r.w[2], r.w[1], sh), r.w[2] >> sh};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int bit = j * BITS, i = bit >> 5, o = bit & 31;
      uint32_t v = win[i] >> o;
      if (o + BITS > 32) v |= win[i + 1] << (32 - o);
      f[j] = (float)(v & ((1u << BITS) - 1u));
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    bf16x2 v;
    v[0] = (__bf16)fmaf(f[2 * j], s, b);
    v[1] = (__bf16)fmaf(f[2 * j + 1], s, b);
    pk[j] = __builtin_bit_cast(uint32_t, v);
  }
}

template <int N>
__device__ __forceinline__ void q3_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// sums the KS partial slices of a split product in k order (z = 0, 1, ...):
// all KS loads of a thread are issued before the first add. V = 4: a thread
// takes 4 consecutive columns of one row with 16-byte loads (partial rows and
// every matrix's first column a multiple of 4 columns, vec bit 1), so the 4
// never cross a matrix or a row; the y store is then one 8- or 16-byte store
// when y rows are 16-byte aligned (vec bit 0).
template <int KS, int V>
__global__ __launch_bounds__(256) void qmm_reduce_multi_kernel(QmmMulti p, int slot) {
  typedef float fv __attribute__((ext_vector_type(V)));
  const float *part = g_qmm_part + (size_t)slot * kQSlotFloats;
  const size_t MN = (size_t)p.M * p.part_N, nv = MN / V;
  for (size_t v = (size_t)blockIdx.x * 256 + threadIdx.x; v < nv; v += (size_t)gridDim.x * 256) {
    const size_t i = v * V;
    fv t[KS];
#pragma unroll
    for (int z = 0; z < KS; ++z) t[z] = __builtin_nontemporal_load(reinterpret_cast<const fv *>(part + z * MN + i));
    fv s = t[0];
#pragma unroll
    for (int z = 1; z < KS; ++z) s += t[z];  // in k order
    const int m = (int)(i / p.part_N), c = (int)(i % p.part_N);
    int mi = 0;
#pragma unroll
    for (int u = 1; u < kQMultiMax; ++u) mi = u < p.n && c >= p.m[u].col0 ? u : mi;
    const QmmMat &q = p.m[mi];
    const size_t o = (size_t)m * q.y_stride + (c - q.col0);
    if (p.y_bf16) {
      __bf16 *y = reinterpret_cast<__bf16 *>(q.y) + o;
      if constexpr (V == 4) {
        if (p.vec & 1) {
          typedef __bf16 b4 __attribute__((ext_vector_type(4)));
          *reinterpret_cast<b4 *>(y) = b4{(__bf16)s[0], (__bf16)s[1], (__bf16)s[2], (__bf16)s[3]};
          continue;
        }
      }
#pragma unroll
      for (int e = 0; e < V; ++e) y[e] = (__bf16)s[e];
    } else {
      float *y = reinterpret_cast<float *>(q.y) + o;
      if constexpr (V == 4) {
        if (p.vec & 1) {
          *reinterpret_cast<fv *>(y) = s;
          continue;
        }
      }
#pragma unroll
      for (int e = 0; e < V; ++e) y[e] = s[e];
    }
  }
}

template <int V>
static void launch_qmm_reduce_multi(const QmmMulti &p, int slot, int KS, hipStream_t st) {
  const size_t nv = (size_t)p.M * p.part_N / V;
  const dim3 grid((unsigned)std::min<size_t>((nv + 255) / 256, 4096));
  switch (KS) {
#define LH_QRED(k) \
  case k: hipLaunchKernelGGL((qmm_reduce_multi_kernel<k, V>), grid, dim3(256), 0, st, p, slot); break;
    LH_QRED(2) LH_QRED(3) LH_QRED(4) LH_QRED(5) LH_QRED(6) LH_QRED(7) LH_QRED(8) LH_QRED(9)
    LH_QRED(10) LH_QRED(11) LH_QRED(12) LH_QRED(13) LH_QRED(14) LH_QRED(15) LH_QRED(16)
#undef LH_QRED
    default: break;
  }
}

template <int BITS>
__global__ __launch_bounds__(512) void affine_qmm256_kernel(QmmMulti p, int mtiles, int ntiles,
                                                            int ksteps, int slot) {
  __shared__ __align__(16) uint16_t sX[2][kQ3M * kQ3Ld];
  __shared__ __align__(16) uint16_t sW[2][kQ3N * kQ3Ld];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5, l32 = lane & 31;
  // XCD-grouped tile order: the M tiles of one N tile share an XCD's L2
  const int L = blockIdx.x;
  const int grp = L / (8 * mtiles), rem = L % (8 * mtiles);
  const int nt = grp * 8 + rem % 8, mt = rem / 8;
  if (nt >= ntiles) return;
  int mi = 0;
#pragma unroll
  for (int t = 1; t < kQMultiMax; ++t) mi = t < p.n && nt >= p.tile_start[t] ? t : mi;
  mi = __builtin_amdgcn_readfirstlane(mi);
  const QmmMat &mat = p.m[mi];
  const int bm0 = mt * kQ3M, bn0 = (nt - p.tile_start[mi]) * kQ3N;
  const int N = mat.N;

  // dequantising role: row wr of the W tile, codes [16 q, 16 q + 16) of each step
  const int wr = tid >> 2, q = tid & 3;
  const int nrow = min(bn0 + wr, N - 1);
  const __amdgpu_buffer_rsrc_t wrs = q3_rsrc(mat.w, (long long)N * mat.row_bytes);
  const __amdgpu_buffer_rsrc_t srs = q3_rsrc(mat.sc, (long long)N * mat.ng * 2);
  const __amdgpu_buffer_rsrc_t brs = q3_rsrc(mat.bi, (long long)N * mat.ng * 2);
  const int rowoff = (int)((long long)nrow * mat.row_bytes);
  const int prow = nrow * mat.ng;
  const int gsh = __builtin_ctz(p.gs);  // group sizes are powers of two here
  const int sh5 = (BITS == 5 && (q & 1)) ? 16 : 0;  // 5-bit run start inside its first dword
  const int wdst = wr * kQ3Ld;

  // x staging role: 16-byte granules g = 512 i + tid (i < 4) of the 256 x 8
  // tile
  const uint16_t *xsrc[4];
  int xdst[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int g = 512 * i + tid;
    const int r = g >> 3, lg = g & 7;
    xsrc[i] = p.x + (size_t)min(bm0 + r, p.M - 1) * p.x_stride + 8 * lg;
    xdst[i] = r * kQ3Ld + 8 * lg;
  }

  const int z = blockIdx.y;
  const int kb = z * ksteps * 64;
  const int nst = (min(p.K, kb + ksteps * 64) - kb) >> 6;

  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  struct Set {
    u32x4 x[4];  // native vectors: a HIP uint4 array copy would stay in memory
    Q3Raw<BITS> w;
  };
  auto load = [&](int s, Set &r) {
    const int k0 = kb + 64 * s;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.x[i] = *reinterpret_cast<const u32x4 *>(xsrc[i] + k0);
    const int k = k0 + 16 * q;
    q3_load<BITS>(r.w, wrs, srs, brs, rowoff, 2 * (prow + (k >> gsh)), k);
  };
  auto stage = [&](const Set &r, int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4 *>(sX[st] + xdst[i]) = r.x[i];
    uint32_t pk[8];
    q3_dequant<BITS>(r.w, sh5, p.fp16 != 0, pk);
    uint16_t *d = sW[st] + wdst;
    *reinterpret_cast<uint4 *>(d + 16 * q) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    *reinterpret_cast<uint4 *>(d + 16 * q + 8) = make_uint4(pk[4], pk[5], pk[6], pk[7]);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
  auto mfma = [&](int st) {
    const uint16_t *xa = sX[st] + (wm * 64 + l32) * kQ3Ld;
    const uint16_t *wb = sW[st] + (wn * 64 + l32) * kQ3Ld;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int g = 16 * ks + 8 * half;
      bf16x8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const bf16x8 *>(xa + 32 * kQ3Ld * i + g);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const bf16x8 *>(wb + 32 * kQ3Ld * j + g);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };
  auto barrier = [&]() {
    // nothing moves across a step boundary (the scheduler would otherwise
    // hoist the next set's conversions and wait for loads meant to stay in
    // flight); the LDS writes of this wave are done, then the barrier alone
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };

  // Step s's x and W pass through a register set loaded two steps earlier,
  // are written (W dequantised) into LDS stage s & 1 one step ahead, and
  // multiplied after the barrier that follows. Iteration s: barrier; the
  // MFMAs of step s (they run in the matrix pipe while the same wave goes
  // on); stage step s + 1 from its set into the other stage; load step s + 3
  // into that set.
  Set ra, rb;
  load(0, ra);
  if (nst > 1) load(1, rb);
  stage(ra, 0);
  if (nst > 2) load(2, ra);
  int s = 0;
  // steady state, two steps per trip so each register set is a fixed one
  for (; s + 4 < nst; s += 2) {
    barrier();
    mfma(0);
    stage(rb, 1);
    load(s + 3, rb);
    barrier();
    mfma(1);
    stage(ra, 0);
    load(s + 4, ra);
  }
  // tail: the last (at most four) steps, s even here; written out so that
  // each register set stays a fixed one
  if (s < nst) {
    barrier();
    mfma(0);
    if (s + 1 < nst) stage(rb, 1);
    if (s + 3 < nst) load(s + 3, rb);
  }
  if (s + 1 < nst) {
    barrier();
    mfma(1);
    if (s + 2 < nst) stage(ra, 0);
    if (s + 4 < nst) load(s + 4, ra);
  }
  if (s + 2 < nst) {
    barrier();
    mfma(0);
    if (s + 3 < nst) stage(rb, 1);
  }
  if (s + 3 < nst) {
    barrier();
    mfma(1);
  }

  // Output through LDS, 32 rows of the wave's tile at a time: the wave
  // writes them as f32 rows of 72 floats (element e of MFMA tile (i, j) is
  // row 8 (e / 4) + 4 half + e % 4, column 32 j + l32), then stores whole
  // rows with 16-byte stores (8 bf16 or 4 f32 per lane); ragged or unaligned
  // edges take element stores.
  constexpr int kTs = 72;
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();  // every wave is done with the operand tiles
  float *tb = reinterpret_cast<float *>(&sX[0][0]) + wave * (32 * kTs);
  const bool split = slot >= 0;
  float *part = split ? g_qmm_part + (size_t)slot * kQSlotFloats + (size_t)z * p.M * p.part_N + mat.col0
                      : nullptr;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        tb[(8 * (e / 4) + 4 * half + (e % 4)) * kTs + 32 * j + l32] = acc[i][j][e];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    const int m0 = bm0 + wm * 64 + 32 * i, n0 = bn0 + wn * 64;
    if (!split && p.y_bf16) {
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int r = 8 * it + (lane >> 3), c = 8 * (lane & 7);
        const float4 u = *reinterpret_cast<const float4 *>(tb + r * kTs + c);
        const float4 v = *reinterpret_cast<const float4 *>(tb + r * kTs + c + 4);
        const int m = m0 + r, n = n0 + c;
        if (m >= p.M) continue;
        __bf16 *dst = reinterpret_cast<__bf16 *>(mat.y) + (size_t)m * mat.y_stride + n;
        const float f[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
        if ((p.vec & 1) && n + 8 <= N) {
          bf16x8 o;
#pragma unroll
          for (int t = 0; t < 8; ++t) o[t] = (__bf16)f[t];
          *reinterpret_cast<bf16x8 *>(dst) = o;
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t)
            if (n + t < N) dst[t] = (__bf16)f[t];
        }
      }
    } else {
      const bool vec = split ? (p.vec & 2) != 0 : (p.vec & 1) != 0;
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int r = 4 * it + (lane >> 4), c = 4 * (lane & 15);
        const float4 u = *reinterpret_cast<const float4 *>(tb + r * kTs + c);
        const int m = m0 + r, n = n0 + c;
        if (m >= p.M) continue;
        float *dst = split ? part + (size_t)m * p.part_N + n
                           : reinterpret_cast<float *>(mat.y) + (size_t)m * mat.y_stride + n;
        if (vec && n + 4 <= N) {
          *reinterpret_cast<float4 *>(dst) = u;
        } else {
          const float f[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (n + t < N) dst[t] = f[t];
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
  }
}

// ---------------------------------------------------------------------------
// The same 256 x 128 tiles with 16 waves (1024 threads): waves 8 (m) x 2 (n),
// each a 32 x 64 tile (1 x 2 v_mfma_f32_32x32x16_bf16 tiles), each thread
// dequantising 8 codes and staging 2 granules of x per step. Same LDS layout,
// tile order and one-barrier-per-step pipeline as affine_qmm256_kernel, at
// <= 128 registers so that four waves share a SIMD instead of two: the step's
// chain of LDS reads -> MFMAs and loads -> dequantisation -> LDS writes ->
// barrier then overlaps across twice the waves.
template <int BITS>
struct Q8Raw {
  uint32_t w[BITS == 4 ? 1 : 2];
  uint32_t s, b;
};

// 8 codes [k, k + 8) of a row (k a multiple of 8) and their group's scale
// and bias
template <int BITS>
__device__ __forceinline__ void q8_load(Q8Raw<BITS> &r, __amdgpu_buffer_rsrc_t wr,
                                        __amdgpu_buffer_rsrc_t sr, __amdgpu_buffer_rsrc_t br,
                                        int rowoff, int poff, int k) {
  if constexpr (BITS == 4) {
    r.w[0] = __builtin_amdgcn_raw_buffer_load_b32(wr, rowoff + (k >> 1), 0, 0);
  } else if constexpr (BITS == 8) {
    const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wr, rowoff + k, 0, 0));
    r.w[0] = v.x;
    r.w[1] = v.y;
  } else {
    // the dword holding the first code; the 8 codes end within the next one
    const uint2 v = __builtin_bit_cast(
        uint2, __builtin_amdgcn_raw_buffer_load_b64(wr, rowoff + 4 * ((k * BITS) >> 5), 0, 0));
    r.w[0] = v.x;
    r.w[1] = v.y;
  }
  r.s = __builtin_amdgcn_raw_buffer_load_b16(sr, poff, 0, 0);
  r.b = __builtin_amdgcn_raw_buffer_load_b16(br, poff, 0, 0);
}

// bf16(code * s + b) of the 8 codes, packed in pairs (code order); sh is the
// bit of the first code within r.w[0] (5/6-bit)
template <int BITS>
__device__ __forceinline__ void q8_dequant(const Q8Raw<BITS> &r, int sh, bool fp16, uint32_t (&pk)[4]) {
  const float s = aux_to_f32_sel(r.s, fp16), b = aux_to_f32_sel(r.b, fp16);
  float f[8];
  if constexpr (BITS == 4) {
    const uint32_t lo = r.w[0] & 0x0F0F0F0Fu, hi = (r.w[0] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = (float)((lo >> (8 * i)) & 255u);
      f[2 * i + 1] = (float)((hi >> (8 * i)) & 255u);
    }
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) f[4 * d + i] = (float)((r.w[d] >> (8 * i)) & 255u);
  } else {
    const uint32_t win[2] = {__builtin_amdgcn_alignbit(r.w[1], r.w[0], sh), r.w[1] >> sh};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int bit = j * BITS, i = bit >> 5, o = bit & 31;
      uint32_t v = win[i] >> o;
      if (o + BITS > 32) v |= win[i + 1] << (32 - o);
      f[j] = (float)(v & ((1u << BITS) - 1u));
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bf16x2 v;
    v[0] = (__bf16)fmaf(f[2 * j], s, b);
    v[1] = (__bf16)fmaf(f[2 * j + 1], s, b);
    pk[j] = __builtin_bit_cast(uint32_t, v);
  }
}

template <int BITS>
__global__ __launch_bounds__(1024) void affine_qmm256w_kernel(QmmMulti p, int mtiles, int ntiles,
                                                              int ksteps, int slot) {
  __shared__ __align__(16) uint16_t sX[2][kQ3M * kQ3Ld];
  __shared__ __align__(16) uint16_t sW[2][kQ3N * kQ3Ld];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5, l32 = lane & 31;
  const int L = blockIdx.x;
  const int grp = L / (8 * mtiles), rem = L % (8 * mtiles);
  const int nt = grp * 8 + rem % 8, mt = rem / 8;
  if (nt >= ntiles) return;
  int mi = 0;
#pragma unroll
  for (int t = 1; t < kQMultiMax; ++t) mi = t < p.n && nt >= p.tile_start[t] ? t : mi;
  mi = __builtin_amdgcn_readfirstlane(mi);
  const QmmMat &mat = p.m[mi];
  const int bm0 = mt * kQ3M, bn0 = (nt - p.tile_start[mi]) * kQ3N;
  const int N = mat.N;

  // dequantising role: row wr of the W tile, codes [8 q, 8 q + 8) of each step
  const int wr = tid >> 3, q = tid & 7;
  const int nrow = min(bn0 + wr, N - 1);
  const __amdgpu_buffer_rsrc_t wrs = q3_rsrc(mat.w, (long long)N * mat.row_bytes);
  const __amdgpu_buffer_rsrc_t srs = q3_rsrc(mat.sc, (long long)N * mat.ng * 2);
  const __amdgpu_buffer_rsrc_t brs = q3_rsrc(mat.bi, (long long)N * mat.ng * 2);
  const int rowoff = (int)((long long)nrow * mat.row_bytes);
  const int prow = nrow * mat.ng;
  const int gsh = __builtin_ctz(p.gs);
  // first code's bit within its dword: (8 q * BITS) mod 32 (k0 is a multiple of 64)
  const int shq = (8 * q * BITS) & 31;
  const int wdst = wr * kQ3Ld + 8 * q;

  // x staging role: 16-byte granules g = 1024 i + tid (i < 2) of the 256 x 8 tile
  const uint16_t *xsrc[2];
  int xdst[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int g = 1024 * i + tid;
    const int r = g >> 3, lg = g & 7;
    xsrc[i] = p.x + (size_t)min(bm0 + r, p.M - 1) * p.x_stride + 8 * lg;
    xdst[i] = r * kQ3Ld + 8 * lg;
  }

  const int z = blockIdx.y;
  const int kb = z * ksteps * 64;
  const int nst = (min(p.K, kb + ksteps * 64) - kb) >> 6;

  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  struct Set {
    u32x4 x[2];
    Q8Raw<BITS> w;
  };
  auto load = [&](int s, Set &r) {
    const int k0 = kb + 64 * s;
#pragma unroll
    for (int i = 0; i < 2; ++i) r.x[i] = *reinterpret_cast<const u32x4 *>(xsrc[i] + k0);
    const int k = k0 + 8 * q;
    q8_load<BITS>(r.w, wrs, srs, brs, rowoff, 2 * (prow + (k >> gsh)), k);
  };
  auto stage = [&](const Set &r, int st) {
#pragma unroll
    for (int i = 0; i < 2; ++i) *reinterpret_cast<u32x4 *>(sX[st] + xdst[i]) = r.x[i];
    uint32_t pk[4];
    q8_dequant<BITS>(r.w, shq, p.fp16 != 0, pk);
    *reinterpret_cast<uint4 *>(sW[st] + wdst) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  };

  f32x16 acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) acc[j] = f32x16{};
  auto mfma = [&](int st) {
    const uint16_t *xa = sX[st] + (wm * 32 + l32) * kQ3Ld;
    const uint16_t *wb = sW[st] + (wn * 64 + l32) * kQ3Ld;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int g = 16 * ks + 8 * half;
      const bf16x8 a = *reinterpret_cast<const bf16x8 *>(xa + g);
      bf16x8 b[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const bf16x8 *>(wb + 32 * kQ3Ld * j + g);
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[j], acc[j], 0, 0, 0);
    }
  };
  auto barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };

  // as affine_qmm256_kernel: step s's operands pass through a register set
  // loaded two steps earlier and LDS stage s & 1 written one step ahead
  Set ra, rb;
  load(0, ra);
  if (nst > 1) load(1, rb);
  stage(ra, 0);
  if (nst > 2) load(2, ra);
  int s = 0;
  for (; s + 4 < nst; s += 2) {
    barrier();
    mfma(0);
    stage(rb, 1);
    load(s + 3, rb);
    barrier();
    mfma(1);
    stage(ra, 0);
    load(s + 4, ra);
  }
  if (s < nst) {
    barrier();
    mfma(0);
    if (s + 1 < nst) stage(rb, 1);
    if (s + 3 < nst) load(s + 3, rb);
  }
  if (s + 1 < nst) {
    barrier();
    mfma(1);
    if (s + 2 < nst) stage(ra, 0);
    if (s + 4 < nst) load(s + 4, ra);
  }
  if (s + 2 < nst) {
    barrier();
    mfma(0);
    if (s + 3 < nst) stage(rb, 1);
  }
  if (s + 3 < nst) {
    barrier();
    mfma(1);
  }

  // element e of tile j: row 8 (e / 4) + 4 half + e % 4 of the wave's 32,
  // column 32 j + l32 of its 64; lanes 0-31 store 32 consecutive columns
  const bool split = slot >= 0;
  float *part = split ? g_qmm_part + (size_t)slot * kQSlotFloats + (size_t)z * p.M * p.part_N + mat.col0
                      : nullptr;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = bn0 + wn * 64 + 32 * j + l32;
    if (n >= N) continue;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = bm0 + wm * 32 + 8 * (e / 4) + 4 * half + (e % 4);
      if (m >= p.M) continue;
      if (split)
        part[(size_t)m * p.part_N + n] = acc[j][e];
      else if (p.y_bf16)
        reinterpret_cast<__bf16 *>(mat.y)[(size_t)m * mat.y_stride + n] = (__bf16)acc[j][e];
      else
        reinterpret_cast<float *>(mat.y)[(size_t)m * mat.y_stride + n] = acc[j][e];
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

// 256 x 128 tiles: every matrix supported, the same K / bits / group size /
// aux type, power-of-two group sizes (the kernel shifts), at least 256 rows
// of x, and offsets of every matrix within 2 GiB (32-bit buffer offsets)
static bool qmm256_ok(const DevMat *ms, int n, int M) {
  if (M < kQ3M || n < 1 || n > kQMultiMax) return false;
  for (int i = 0; i < n; ++i) {
    const DevMat &m = ms[i];
    if (!affine_qmm_supported(m)) return false;
    if (m.I != ms[0].I || m.bits != ms[0].bits || m.gs != ms[0].gs || m.fp16 != ms[0].fp16) return false;
    if ((m.gs & (m.gs - 1)) != 0 || (long long)m.O * m.row_bytes > 0x7fffffffLL) return false;
    if ((reinterpret_cast<uintptr_t>(m.w) & 15) != 0) return false;
  }
  return true;
}

// 16 waves per block where K is split (short k ranges: the 2048-row output
// projections, 23 -> 19.6 us), 8 where it is not (the 12352-row grids of one
// k range, 45.4 -> 43 us)

static hipError_t launch_qmm256(const DevMat *ms, int n, const uint16_t *x, int x_stride, int M,
                                void *const *ys, const int *y_strides, int y_bf16, hipStream_t st) {
  QmmMulti p;
  p.x = x;
  p.n = n;
  p.M = M;
  p.K = ms[0].I;
  p.gs = ms[0].gs;
  p.fp16 = ms[0].fp16;
  p.x_stride = x_stride;
  p.y_bf16 = y_bf16;
  int tiles = 0, cols = 0;
  for (int i = 0; i < kQMultiMax; ++i) {
    if (i < n) {
      p.m[i] = QmmMat{ms[i].w, ms[i].sc, ms[i].bi, ys[i], ms[i].row_bytes, ms[i].O, ms[i].ng,
                      y_strides[i], cols};
      p.tile_start[i] = tiles;
      tiles += (ms[i].O + kQ3N - 1) / kQ3N;
      cols += ms[i].O;
    } else {
      p.m[i] = p.m[0];
      p.tile_start[i] = tiles;
    }
  }
  p.tile_start[kQMultiMax] = tiles;
  p.part_N = cols;
  bool yv = true, pv = (cols & 3) == 0;
  for (int i = 0; i < n; ++i) {
    const int es = y_bf16 ? 2 : 4;
    yv = yv && (reinterpret_cast<uintptr_t>(ys[i]) & 15) == 0 && ((long long)y_strides[i] * es) % 16 == 0;
    pv = pv && (p.m[i].col0 & 3) == 0;
  }
  p.vec = (yv ? 1 : 0) | (pv ? 2 : 0);
  const int mt = (M + kQ3M - 1) / kQ3M;
  const int ksteps_all = p.K / 64;
  // split K while the grid is short of one block per CU and each k range
  // keeps at least 8 steps
  int split = 1;
  while (split < 16 && mt * tiles * split < 192 && ksteps_all / (2 * split) >= 8 &&
         (size_t)(2 * split) * M * cols <= kQSlotFloats)
    split *= 2;
  const int ksteps = (ksteps_all + split - 1) / split;
  split = (ksteps_all + ksteps - 1) / ksteps;
  SlotRing::Lease lease;
  if (split > 1) {
    const hipError_t le = g_qmm_slots.take(st, lease);
    if (le != hipSuccess) return le;
  }
  const int slot = split > 1 ? lease.slot() : -1;
  const dim3 grid(((tiles + 7) / 8) * 8 * mt, split);
  if (split > 1) {
    switch (ms[0].bits) {
      case 4: hipLaunchKernelGGL(affine_qmm256w_kernel<4>, grid, dim3(1024), 0, st, p, mt, tiles, ksteps, slot); break;
      case 5: hipLaunchKernelGGL(affine_qmm256w_kernel<5>, grid, dim3(1024), 0, st, p, mt, tiles, ksteps, slot); break;
      case 6: hipLaunchKernelGGL(affine_qmm256w_kernel<6>, grid, dim3(1024), 0, st, p, mt, tiles, ksteps, slot); break;
      case 8: hipLaunchKernelGGL(affine_qmm256w_kernel<8>, grid, dim3(1024), 0, st, p, mt, tiles, ksteps, slot); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (ms[0].bits) {
      case 4: hipLaunchKernelGGL(affine_qmm256_kernel<4>, grid, dim3(512), 0, st, p, mt, tiles, ksteps, slot); break;
      case 5: hipLaunchKernelGGL(affine_qmm256_kernel<5>, grid, dim3(512), 0, st, p, mt, tiles, ksteps, slot); break;
      case 6: hipLaunchKernelGGL(affine_qmm256_kernel<6>, grid, dim3(512), 0, st, p, mt, tiles, ksteps, slot); break;
      case 8: hipLaunchKernelGGL(affine_qmm256_kernel<8>, grid, dim3(512), 0, st, p, mt, tiles, ksteps, slot); break;
      default: return hipErrorInvalidValue;
    }
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || split == 1) return e;
  if (p.vec & 2)
    launch_qmm_reduce_multi<4>(p, slot, split, st);
  else
    launch_qmm_reduce_multi<1>(p, slot, split, st);
  e = hipGetLastError();
  const hipError_t le = lease.done();
  return e != hipSuccess ? e : le;
}

hipError_t launch_affine_qmm_multi(const DevMat *ms, int n, const uint16_t *x, int x_stride, int M,
                                   void *const *ys, int y_bf16, hipStream_t st) {
  if (n < 1 || n > kQMultiMax || M <= 0) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return hipErrorInvalidValue;
  int strides[kQMultiMax];
  for (int i = 0; i < n; ++i) strides[i] = ms[i].O;
  if (qmm256_ok(ms, n, M)) return launch_qmm256(ms, n, x, x_stride, M, ys, strides, y_bf16, st);
  for (int i = 0; i < n; ++i) {
    const hipError_t e = launch_affine_qmm(ms[i], x, x_stride, M, ys[i], ms[i].O, y_bf16, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_affine_qmm(const DevMat &m, const uint16_t *x, int x_stride, int M, void *y,
                             int y_stride, int y_bf16, hipStream_t st) {
  if (!affine_qmm_supported(m) || M <= 0) return hipErrorInvalidValue;
  if (qmm256_ok(&m, 1, M) && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (x_stride & 7) == 0) {
    void *ys[1] = {y};
    const int strides[1] = {y_stride};
    return launch_qmm256(&m, 1, x, x_stride, M, ys, strides, y_bf16, st);
  }
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
  SlotRing::Lease lease;
  if (split > 1) {
    const hipError_t le = g_qmm_slots.take(st, lease);
    if (le != hipSuccess) return le;
  }
  const int slot = split > 1 ? lease.slot() : -1;
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
  if ((m.O & 3) == 0)
    launch_qmm_reduce<4>(p, slot, split, st);
  else
    launch_qmm_reduce<1>(p, slot, split, st);
  e = hipGetLastError();
  const hipError_t le = lease.done();
  return e != hipSuccess ? e : le;
}

}  // namespace lh
