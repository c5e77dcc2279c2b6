// Dense MLX-affine GEMV kernels for gfx950.
//
//  * gemv_bf16_kernel: the decode hot path. A "team" of LANES lanes owns one
//    weight row at a time; lane l owns chunks c = l + LANES*j (32 codes each),
//    so a team's loads of one row are contiguous 16-32 B per lane. The x
//    operand of the lane's chunks is built once (bf16 pairs in the unpack
//    order) and kept in VGPRs for every row the team visits. U rows are
//    loaded before any is consumed to keep several 128-bit loads in flight
//    per lane. The team sum is a butterfly over LANES lanes. For rows of up
//    to 64 chunks the weights and their scale/bias words are read with
//    non-temporal loads (read once per launch; x and the code stay in L2).
//  * gemv_generic_kernel: any bits/group size, f32 activations, f32 output,
//    per-element exact dequantisation (code*scale+bias, as
//    logan-qwen4/src/lib.rs:3752-3762); serves the f32 host ABI and shapes
//    without a fast kernel. Up to 16 descriptors per launch.
//  * dequant_kernel: writes code*scale+bias per element (bit-exact probe).
#include "affine_dev.hpp"
#include "lh_internal.hpp"

namespace lh {

struct GemvParams {
  const uint8_t *w;
  const uint16_t *sc;
  const uint16_t *bi;
  const uint16_t *x;
  void *y;
  long long row_bytes;
  int I, O, ng, gsc;  // gsc = chunks per group
  int gsc_shift;      // log2(gsc) when gsc is a power of two, else -1
  int fp16, x_stride, M, y_stride, y_bf16;
  // SW (SwiGLU) form: the up matrix, same geometry as w
  const uint8_t *w2;
  const uint16_t *sc2;
  const uint16_t *bi2;
};

// SPLIT > 1: SPLIT teams share one row, each over a contiguous K segment of
// LANES*CPL chunks; their partial sums meet in LDS and are added in segment
// order.
// XF: the activation is one f32 row (a.x points at floats); its two operand
// rows are hi = bf16(x) and lo = bf16(x - hi) (|x - hi - lo| <= 2^-18 |x|),
// split in registers, and their partial sums are added before the team
// reduction, so the kernel writes one f32 (or bf16) output row (MT == 2).
// SW: SwiGLU form. Team row u alternates between the gate matrix (w, even u)
// and the up matrix (w2, odd u) at the same row index j = (r0 + u) / 2, and
// the team writes h[m][j] = silu(gate_j . x) * (up_j . x) (logan-qwen4/src
// /lib.rs:8803-8812) instead of the two products; the grid covers 2 * O rows.
template <int BITS, int LANES, int CPL, int U, int MT, int SPLIT, bool XF = false, bool SW = false>
__device__ __forceinline__ void gemv_bf16_body(const GemvParams &a, int bid) {
  static_assert(!XF || MT == 2, "f32 activations use the two-row operand form");
  static_assert(!SW || (U % 2 == 0 && !XF), "SwiGLU pairs whole teams of bf16 rows");
  constexpr int MO = XF ? 1 : MT;  // output rows
  constexpr int TEAMS = 256 / LANES;
  constexpr int ROWTEAMS = TEAMS / SPLIT;
  const int lane = threadIdx.x & (LANES - 1);
  const int team = threadIdx.x / LANES;
  const int rteam = team / SPLIT, seg = team % SPLIT;
  const int cbase = seg * LANES * CPL;
  const int C = a.I >> 5;
  UnpackConsts kc;
  kc.init();
  __shared__ float s_part[SPLIT > 1 ? TEAMS * U * MT : 1];
  // non-temporal weight loads for the short-row shapes (config 1: 3.39 ->
  // 3.30 us) and the two-wave rows of narrow codes (config-5 decode, 4-bit
  // K = 4096 output projections: 1090-1097 -> 1066-1070 us per token); the
  // long-row 8-bit shapes measured slower with them (config-2 layer at
  // M = 1: 52 -> 62 us, 55 -> 59 us with the 4096-code products alone)
  constexpr bool NT = (SPLIT == 1 && CPL == 1) || (SPLIT == 2 && CPL == 1 && !SW && BITS < 8);

  // Loads are branch-free (row and chunk clamped into the matrix, x rows
  // clamped to M) and issued in the order they are needed: x, the raw
  // scale/bias words, then every weight chunk, all in flight together; the
  // values of dead lanes are masked where they are used. Loads complete in
  // issue order (vmcnt), so the x conversion and the scale/bias conversion
  // wait for their own loads alone and row u's products for its chunks.
  int gidx[CPL];
  bool cval[CPL];
  int cc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = cbase + lane + LANES * j;
    cval[j] = c < C;
    cc[j] = cval[j] ? c : C - 1;
    gidx[j] = a.gsc_shift >= 0 ? cc[j] >> a.gsc_shift : cc[j] / a.gsc;
  }

  uint4 xr[MT][CPL][4];
  if constexpr (XF) {
    // 32 f32 per chunk: xr[0] and xr[1] hold its first and second half
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint4 *src =
          reinterpret_cast<const uint4 *>(reinterpret_cast<const float *>(a.x) + 32 * cc[j]);
#pragma unroll
      for (int v = 0; v < 8; ++v) xr[v >> 2][j][v & 3] = src[v];
    }
  } else {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int mm = m < a.M ? m : a.M - 1;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const uint4 *src = reinterpret_cast<const uint4 *>(a.x + (size_t)mm * a.x_stride + 32 * cc[j]);
#pragma unroll
        for (int v = 0; v < 4; ++v) xr[m][j][v] = src[v];
      }
    }
  }

  // the grid covers O exactly once: block b owns rows [b*ROWTEAMS*U, ...)
  {
    const int r0 = bid * (ROWTEAMS * U) + rteam * U;
    uint32_t wv[U][CPL][BITS];
    uint32_t scr[U][CPL], bir[U][CPL];
    // row index and matrix of team row u (SW: gate / up alternately)
    auto row_of = [&](int u) { return SW ? (r0 >> 1) + (u >> 1) : r0 + u; };
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = min(row_of(u), a.O - 1);
      const uint16_t *scp = (SW && (u & 1)) ? a.sc2 : a.sc;
      const uint16_t *bip = (SW && (u & 1)) ? a.bi2 : a.bi;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const size_t pi = (size_t)row * a.ng + gidx[j];
        scr[u][j] = ld_stream<uint16_t, NT>(scp + pi);
        bir[u][j] = ld_stream<uint16_t, NT>(bip + pi);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = min(row_of(u), a.O - 1);
      const uint8_t *wp = (SW && (u & 1)) ? a.w2 : a.w;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        load_chunk<BITS, NT>(wv[u][j], wp + (size_t)row * a.row_bytes + (size_t)cc[j] * (4 * BITS));
    }
    // keep every load above issued before any of their consumers
    __builtin_amdgcn_sched_barrier(0);
    XChunk xc[MT][CPL];
    if constexpr (XF) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        uint32_t xh[32], xl[32];
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const uint4 t = xr[v >> 2][j][v & 3];
          const uint32_t w4[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float f = cval[j] ? __uint_as_float(w4[q]) : 0.f;
            const uint32_t hi = f32_to_bf16_rne(f);
            xh[4 * v + q] = hi;
            xl[4 * v + q] = f32_to_bf16_rne(f - bf16_to_f32(hi));  // f - hi is exact
          }
        }
        make_xchunk_bf16<BITS>(xc[0][j], xh);
        make_xchunk_bf16<BITS>(xc[1][j], xl);
      }
    } else {
#pragma unroll
      for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const bool ok = cval[j] && m < a.M;
          uint32_t xb[32];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const uint4 t = xr[m][j][v];
            xb[8 * v + 0] = ok ? t.x & 0xffffu : 0u; xb[8 * v + 1] = ok ? t.x >> 16 : 0u;
            xb[8 * v + 2] = ok ? t.y & 0xffffu : 0u; xb[8 * v + 3] = ok ? t.y >> 16 : 0u;
            xb[8 * v + 4] = ok ? t.z & 0xffffu : 0u; xb[8 * v + 5] = ok ? t.z >> 16 : 0u;
            xb[8 * v + 6] = ok ? t.w & 0xffffu : 0u; xb[8 * v + 7] = ok ? t.w >> 16 : 0u;
          }
          make_xchunk_bf16<BITS>(xc[m][j], xb);
        }
      }
    }
    float scv[U][CPL], biv[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const bool live = row_of(u) < a.O && cval[j];
        scv[u][j] = live ? aux_to_f32(scr[u][j], a.fp16) : 0.f;
        biv[u][j] = live ? aux_to_f32(bir[u][j], a.fp16) : 0.f;
      }
    float part[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int m = 0; m < MT; ++m) part[u][m] = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        uint32_t q[16];
        unpack_chunk<BITS>(q, wv[u][j], kc);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const float acc = pairs_dot(q, xc[m][j].p);
          part[u][m] += chunk_fold<BITS>(acc, scv[u][j], biv[u][j], xc[m][j].xs, xc[m][j].xsp);
        }
      }
    }
    if constexpr (XF) {
#pragma unroll
      for (int u = 0; u < U; ++u) part[u][0] += part[u][1];  // y = W.hi + W.lo
    }
    if constexpr (LANES == 64 && SPLIT == 1 && U * MO >= 2 && !SW) {
      // four (row, token) sums per wave_reduce4; row r of lanes gets value r
      constexpr int NV = U * MO;
      float vals[NV];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int m = 0; m < MO; ++m) vals[u * MO + m] = part[u][m];
      const int rr = lane >> 4;
#pragma unroll
      for (int g0 = 0; g0 < NV; g0 += 4) {
        const float t = wave_reduce4(vals[g0], g0 + 1 < NV ? vals[g0 + 1] : 0.f,
                                     g0 + 2 < NV ? vals[g0 + 2] : 0.f,
                                     g0 + 3 < NV ? vals[g0 + 3] : 0.f);
        const int idx = g0 + rr;
        const int u = idx / MO, m = idx % MO;
        const int row = r0 + u;
        if ((lane & 15) == 0 && idx < NV && row < a.O && (XF || m < a.M)) {
          if (a.y_bf16)
            reinterpret_cast<uint16_t *>(a.y)[(size_t)m * a.y_stride + row] =
                (uint16_t)f32_to_bf16_rne(t);
          else
            reinterpret_cast<float *>(a.y)[(size_t)m * a.y_stride + row] = t;
        }
      }
    } else {
      float tot[U][MO];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int m = 0; m < MO; ++m) tot[u][m] = team_sum<LANES>(part[u][m]);
      if constexpr (SPLIT > 1) {
        if (lane == 0) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int m = 0; m < MO; ++m) s_part[(team * U + u) * MT + m] = tot[u][m];
        }
        __syncthreads();
        if (seg == 0 && lane == 0) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int m = 0; m < MO; ++m) {
              float v = tot[u][m];
#pragma unroll
              for (int s = 1; s < SPLIT; ++s) v += s_part[((team + s) * U + u) * MT + m];
              tot[u][m] = v;
            }
        }
        __syncthreads();
      }
#pragma unroll
      for (int u = 0; u < U; u += SW ? 2 : 1) {
        const int row = row_of(u);
#pragma unroll
        for (int m = 0; m < MO; ++m) {
          // SW: h = silu(gate) * up of the pair (u, u + 1)
          const float v = SW ? silu(tot[u][m]) * tot[u + (SW ? 1 : 0)][m] : tot[u][m];
          if (seg == 0 && lane == 0 && row < a.O && (XF || m < a.M)) {
            if (a.y_bf16)
              reinterpret_cast<uint16_t *>(a.y)[(size_t)m * a.y_stride + row] =
                  (uint16_t)f32_to_bf16_rne(v);
            else
              reinterpret_cast<float *>(a.y)[(size_t)m * a.y_stride + row] = v;
          }
        }
      }
    }
  }
}

template <int BITS, int LANES, int CPL, int U, int MT, int SPLIT, bool XF>
__global__ __launch_bounds__(256) void gemv_bf16_kernel(GemvParams a) {
  gemv_bf16_body<BITS, LANES, CPL, U, MT, SPLIT, XF>(a, blockIdx.x);
}

template <int BITS, int LANES, int CPL, int U, int MT, int SPLIT>
__global__ __launch_bounds__(256) void gemv_swiglu_kernel(GemvParams a) {
  gemv_bf16_body<BITS, LANES, CPL, U, MT, SPLIT, false, true>(a, blockIdx.x);
}

// Up to kMultiMax matrices sharing one activation in one launch: block b
// serves the matrix whose block range holds it.
constexpr int kMultiMax = 8;
struct GemvMultiDesc {
  const uint8_t *w;
  const uint16_t *sc;
  const uint16_t *bi;
  const uint16_t *x;  // this matrix's activation rows, or nullptr: the shared x
  void *y;
  long long row_bytes;
  int O, ng;
};
struct GemvMultiParams {
  GemvParams common;  // I, gsc, gsc_shift, fp16, x, x_stride, M, y_bf16
  GemvMultiDesc d[kMultiMax];
  int block_start[kMultiMax + 1];
  int n;
};

template <int BITS, int LANES, int CPL, int U, int MT, int SPLIT, bool XF>
__global__ __launch_bounds__(256) void gemv_bf16_multi_kernel(GemvMultiParams mp) {
  int i = 0;
  while (i + 1 < mp.n && (int)blockIdx.x >= mp.block_start[i + 1]) ++i;
  GemvParams a = mp.common;
  a.w = mp.d[i].w;
  a.sc = mp.d[i].sc;
  a.bi = mp.d[i].bi;
  a.y = mp.d[i].y;
  if (mp.d[i].x) a.x = mp.d[i].x;
  a.row_bytes = mp.d[i].row_bytes;
  a.O = mp.d[i].O;
  a.ng = mp.d[i].ng;
  a.y_stride = mp.d[i].O;
  gemv_bf16_body<BITS, LANES, CPL, U, MT, SPLIT, XF>(a, blockIdx.x - mp.block_start[i]);
}

template <int BITS, int LANES, int CPL, int MT, int SPLIT, int U, bool XF>
static hipError_t gemv_launch_t(const GemvParams &p, hipStream_t st, GemvMultiParams *mp) {
  constexpr int rows_per_block = (256 / LANES / SPLIT) * U;
  if (mp) {
    mp->block_start[0] = 0;
    for (int i = 0; i < mp->n; ++i)
      mp->block_start[i + 1] = mp->block_start[i] + (mp->d[i].O + rows_per_block - 1) / rows_per_block;
    for (int i = mp->n + 1; i <= kMultiMax; ++i) mp->block_start[i] = mp->block_start[mp->n];
    hipLaunchKernelGGL((gemv_bf16_multi_kernel<BITS, LANES, CPL, U, MT, SPLIT, XF>),
                       dim3(mp->block_start[mp->n]), dim3(256), 0, st, *mp);
    return hipGetLastError();
  }
  const int blocks = (p.O + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((gemv_bf16_kernel<BITS, LANES, CPL, U, MT, SPLIT, XF>), dim3(blocks), dim3(256),
                     0, st, p);
  return hipGetLastError();
}

// Rows longer than 64 chunks are split across waves (SPLIT) rather than
// given more chunks per lane: one chunk per lane and two rows per team keep
// registers low, so more waves - and more loads - are in flight. Measured at
// the config-2 / config-5 shapes (8-bit 14336x4096: 14.5 -> 13.0 us; 8-bit
// 4096x14336: 18.8 -> 15.6 us; 4-bit 2048x4096: 4.5 -> 3.7 us). Rows of up
// to 64 chunks keep four rows per team (two measured faster launched back to
// back, slower inside a graph).
template <int BITS, int MT, bool XF>
static hipError_t gemv_dispatch_shape(const GemvParams &p, hipStream_t st, GemvMultiParams *mp) {
  const int C = p.I >> 5;
  if (C <= 16) return gemv_launch_t<BITS, 16, 1, MT, 1, 4, XF>(p, st, mp);
  if (C <= 32) return gemv_launch_t<BITS, 32, 1, MT, 1, 4, XF>(p, st, mp);
  if (C <= 64) return gemv_launch_t<BITS, 64, 1, MT, 1, 4, XF>(p, st, mp);
  if (C <= 128) return gemv_launch_t<BITS, 64, 1, MT, 2, 2, XF>(p, st, mp);
  if (C <= 256) return gemv_launch_t<BITS, 64, 1, MT, 4, 2, XF>(p, st, mp);
  if (C <= 512) return gemv_launch_t<BITS, 64, 2, MT, 4, 2, XF>(p, st, mp);
  return hipErrorInvalidValue;
}

template <int MT, bool XF = false>
static hipError_t gemv_dispatch_bits(const GemvParams &p, int bits, hipStream_t st,
                                     GemvMultiParams *mp = nullptr) {
  switch (bits) {
    case 4: return gemv_dispatch_shape<4, MT, XF>(p, st, mp);
    case 5: return gemv_dispatch_shape<5, MT, XF>(p, st, mp);
    case 6: return gemv_dispatch_shape<6, MT, XF>(p, st, mp);
    case 8: return gemv_dispatch_shape<8, MT, XF>(p, st, mp);
  }
  return hipErrorInvalidValue;
}

bool gemv_bf16_supported(const DevMat &m) {
  if (!(m.bits == 4 || m.bits == 5 || m.bits == 6 || m.bits == 8)) return false;
  if (m.gs <= 0 || m.gs % 32 != 0 || m.I % m.gs != 0) return false;
  if ((m.I >> 5) > 512) return false;
  if ((reinterpret_cast<uintptr_t>(m.w) & 15) != 0) return false;
  // every chunk must start on the alignment load_chunk assumes
  const long long cb = 4ll * m.bits;
  if (m.row_bytes % cb != 0) return false;
  return true;
}

hipError_t launch_gemv_bf16(const DevMat &m, const uint16_t *x, int x_stride, int M, void *y,
                            int y_stride, int y_bf16, hipStream_t st) {
  if (!gemv_bf16_supported(m) || M <= 0) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0)
    return hipErrorInvalidValue;
  GemvParams p;
  p.w = m.w;
  p.sc = m.sc;
  p.bi = m.bi;
  p.row_bytes = m.row_bytes;
  p.I = m.I;
  p.O = m.O;
  p.ng = m.ng;
  p.gsc = m.gs / 32;
  p.gsc_shift = (p.gsc & (p.gsc - 1)) == 0 ? __builtin_ctz(p.gsc) : -1;
  p.fp16 = m.fp16;
  p.x_stride = x_stride;
  p.y_stride = y_stride;
  p.y_bf16 = y_bf16;
  // token blocks of at most 2 rows of x per launch of the dot2 kernel
  auto dot2_rows = [&](int r0, int nr) -> hipError_t {
    for (int m0 = r0; m0 < r0 + nr; m0 += 2) {
      const int mt = r0 + nr - m0 >= 2 ? 2 : 1;
      p.x = x + (size_t)m0 * x_stride;
      p.M = mt;
      p.y = y_bf16 ? (void *)(reinterpret_cast<uint16_t *>(y) + (size_t)m0 * y_stride)
                   : (void *)(reinterpret_cast<float *>(y) + (size_t)m0 * y_stride);
      hipError_t e = mt == 2 ? gemv_dispatch_bits<2>(p, m.bits, st, nullptr)
                             : gemv_dispatch_bits<1>(p, m.bits, st, nullptr);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  };
  if (M < 3) return dot2_rows(0, M);
  // three or more activation rows: MFMA paths that read each weight once per
  // 32 rows of x (the K-split form shares each block's x rows across 128
  // weight rows; the wave-private form needs 4/8-bit codes)
  for (int m0 = 0; m0 < M; m0 += 32) {
    const int mc = min(32, M - m0);
    void *ym = y_bf16 ? (void *)(reinterpret_cast<uint16_t *>(y) + (size_t)m0 * y_stride)
                      : (void *)(reinterpret_cast<float *>(y) + (size_t)m0 * y_stride);
    const uint16_t *xm = x + (size_t)m0 * x_stride;
    hipError_t e;
    if (mc >= 3 && affine_kwave_supported(m, mc))
      e = launch_affine_kwave(m, xm, x_stride, mc, ym, y_stride, y_bf16, st);
    else if (mc >= 3 && affine_splitk_supported(m, mc))
      e = launch_affine_splitk(m, xm, x_stride, mc, ym, y_stride, y_bf16, st);
    else if (affine_skinny_supported(m))
      e = launch_affine_skinny(m, xm, x_stride, mc, ym, y_stride, y_bf16, st);
    else
      e = dot2_rows(m0, mc);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// ---- gate/up + SwiGLU in one product (h = silu(gate . x) * (up . x)) ----

template <int BITS, int LANES, int CPL, int MT, int SPLIT, int U>
static hipError_t swiglu_launch_t(const GemvParams &p, hipStream_t st) {
  constexpr int rows_per_block = (256 / LANES / SPLIT) * U;  // gate and up rows together
  const int blocks = (2 * p.O + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((gemv_swiglu_kernel<BITS, LANES, CPL, U, MT, SPLIT>), dim3(blocks), dim3(256), 0,
                     st, p);
  return hipGetLastError();
}

template <int BITS, int MT>
static hipError_t swiglu_dispatch_shape(const GemvParams &p, hipStream_t st) {
  const int C = p.I >> 5;
  if (C <= 16) return swiglu_launch_t<BITS, 16, 1, MT, 1, 4>(p, st);
  if (C <= 32) return swiglu_launch_t<BITS, 32, 1, MT, 1, 4>(p, st);
  if (C <= 64) return swiglu_launch_t<BITS, 64, 1, MT, 1, 4>(p, st);
  if (C <= 128) return swiglu_launch_t<BITS, 64, 1, MT, 2, 2>(p, st);
  if (C <= 256) return swiglu_launch_t<BITS, 64, 1, MT, 4, 2>(p, st);
  if (C <= 512) return swiglu_launch_t<BITS, 64, 2, MT, 4, 2>(p, st);
  return hipErrorInvalidValue;
}

template <int MT>
static hipError_t swiglu_dispatch_bits(const GemvParams &p, int bits, hipStream_t st) {
  switch (bits) {
    case 4: return swiglu_dispatch_shape<4, MT>(p, st);
    case 5: return swiglu_dispatch_shape<5, MT>(p, st);
    case 6: return swiglu_dispatch_shape<6, MT>(p, st);
    case 8: return swiglu_dispatch_shape<8, MT>(p, st);
  }
  return hipErrorInvalidValue;
}

#ifndef SWIGLU_FULLK
#define SWIGLU_FULLK 1
#endif
constexpr bool kSwigluFullK = SWIGLU_FULLK != 0;

hipError_t launch_gemv_swiglu(const DevMat &g, const DevMat &u, const uint16_t *x, int x_stride, int M,
                              void *h, int h_stride, int h_bf16, hipStream_t st) {
  if (!gemv_bf16_supported(g) || !gemv_bf16_supported(u) || M <= 0) return hipErrorInvalidValue;
  if (g.I != u.I || g.O != u.O || g.bits != u.bits || g.gs != u.gs || g.fp16 != u.fp16 ||
      g.row_bytes != u.row_bytes)
    return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return hipErrorInvalidValue;
  // 3..32 tokens: the K-split pair, its reduce forming h
  const DevMat gu[2] = {g, u};
  for (int m0 = 0; m0 < M; m0 += 32) {
    const int mc = min(32, M - m0);
    if (mc >= 3 && kSwigluFullK && swiglu_fullk_supported(g, u, mc)) {
      void *hm = h_bf16 ? (void *)(reinterpret_cast<uint16_t *>(h) + (size_t)m0 * h_stride)
                        : (void *)(reinterpret_cast<float *>(h) + (size_t)m0 * h_stride);
      const hipError_t e = launch_swiglu_fullk(g, u, x + (size_t)m0 * x_stride, x_stride, mc, hm, h_stride,
                                               h_bf16, st);
      if (e != hipSuccess) return e;
      continue;
    }
    if (mc >= 3 && affine_splitk_multi_supported(gu, 2, mc)) {
      void *hm = h_bf16 ? (void *)(reinterpret_cast<uint16_t *>(h) + (size_t)m0 * h_stride)
                        : (void *)(reinterpret_cast<float *>(h) + (size_t)m0 * h_stride);
      void *const ys[2] = {hm, hm};
      const hipError_t e = launch_affine_splitk_multi(gu, 2, x + (size_t)m0 * x_stride, x_stride, mc,
                                                      ys, h_bf16, st, h_stride);
      if (e != hipSuccess) return e;
      continue;
    }
    // token pairs through the dot2 kernel
    GemvParams p;
    p.w = g.w;
    p.sc = g.sc;
    p.bi = g.bi;
    p.w2 = u.w;
    p.sc2 = u.sc;
    p.bi2 = u.bi;
    p.row_bytes = g.row_bytes;
    p.I = g.I;
    p.O = g.O;
    p.ng = g.ng;
    p.gsc = g.gs / 32;
    p.gsc_shift = (p.gsc & (p.gsc - 1)) == 0 ? __builtin_ctz(p.gsc) : -1;
    p.fp16 = g.fp16;
    p.x_stride = x_stride;
    p.y_stride = h_stride;
    p.y_bf16 = h_bf16;
    for (int t = m0; t < m0 + mc; t += 2) {
      const int mt = m0 + mc - t >= 2 ? 2 : 1;
      p.x = x + (size_t)t * x_stride;
      p.M = mt;
      p.y = h_bf16 ? (void *)(reinterpret_cast<uint16_t *>(h) + (size_t)t * h_stride)
                   : (void *)(reinterpret_cast<float *>(h) + (size_t)t * h_stride);
      const hipError_t e = mt == 2 ? swiglu_dispatch_bits<2>(p, g.bits, st) : swiglu_dispatch_bits<1>(p, g.bits, st);
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// Matrices sharing x (same I, bits, group size, aux type): one launch per
// token pair through the dot2 kernel; 3..32 tokens one K-split launch and one
// reduce for all of them where the K-split form applies, otherwise the MFMA
// path matrix by matrix.
// xs (optional): per-matrix activations, each [M][x_stride], instead of the
// shared x.
static hipError_t gemv_bf16_multi_impl(const DevMat *ms, void *const *ys, int n, const uint16_t *x,
                                       const uint16_t *const *xs, int x_stride, int M, int y_bf16,
                                       hipStream_t st) {
  if (n <= 0 || n > kMultiMax || M <= 0) return hipErrorInvalidValue;
  for (int i = 0; i < n; ++i) {
    if (!gemv_bf16_supported(ms[i]) || ms[i].I != ms[0].I || ms[i].bits != ms[0].bits ||
        ms[i].gs != ms[0].gs || ms[i].fp16 != ms[0].fp16 || !ys[i])
      return hipErrorInvalidValue;
    const uint16_t *xi = xs ? xs[i] : x;
    if (!xi || (reinterpret_cast<uintptr_t>(xi) & 15) != 0) return hipErrorInvalidValue;
  }
  if ((x_stride & 7) != 0) return hipErrorInvalidValue;
  // 3..32 tokens: one K-split launch and one reduce for all the products
  if (!xs && M >= 3 && M <= 32 && n > 1 && affine_splitk_multi_supported(ms, n, M))
    return launch_affine_splitk_multi(ms, n, x, x_stride, M, ys, y_bf16, st);
  if (M >= 3 && (xs || affine_skinny_supported(ms[0]))) {
    for (int i = 0; i < n; ++i) {
      hipError_t e = launch_gemv_bf16(ms[i], xs ? xs[i] : x, x_stride, M, ys[i], ms[i].O, y_bf16, st);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  GemvMultiParams mp{};
  GemvParams &p = mp.common;
  p.I = ms[0].I;
  p.gsc = ms[0].gs / 32;
  p.gsc_shift = (p.gsc & (p.gsc - 1)) == 0 ? __builtin_ctz(p.gsc) : -1;
  p.fp16 = ms[0].fp16;
  p.x_stride = x_stride;
  p.y_bf16 = y_bf16;
  mp.n = n;
  for (int m0 = 0; m0 < M; m0 += 2) {
    const int mt = M - m0 >= 2 ? 2 : 1;
    p.x = x + (size_t)m0 * x_stride;
    p.M = mt;
    for (int i = 0; i < n; ++i) {
      mp.d[i].x = xs ? xs[i] + (size_t)m0 * x_stride : nullptr;
      mp.d[i].w = ms[i].w;
      mp.d[i].sc = ms[i].sc;
      mp.d[i].bi = ms[i].bi;
      mp.d[i].row_bytes = ms[i].row_bytes;
      mp.d[i].O = ms[i].O;
      mp.d[i].ng = ms[i].ng;
      mp.d[i].y = y_bf16 ? (void *)(reinterpret_cast<uint16_t *>(ys[i]) + (size_t)m0 * ms[i].O)
                         : (void *)(reinterpret_cast<float *>(ys[i]) + (size_t)m0 * ms[i].O);
    }
    hipError_t e = mt == 2 ? gemv_dispatch_bits<2>(p, ms[0].bits, st, &mp)
                           : gemv_dispatch_bits<1>(p, ms[0].bits, st, &mp);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_gemv_bf16_multi(const DevMat *ms, void *const *ys, int n, const uint16_t *x,
                                  int x_stride, int M, int y_bf16, hipStream_t st) {
  return gemv_bf16_multi_impl(ms, ys, n, x, nullptr, x_stride, M, y_bf16, st);
}

hipError_t launch_gemv_bf16_multi_x(const DevMat *ms, const uint16_t *const *xs, void *const *ys,
                                    int n, int x_stride, int M, int y_bf16, hipStream_t st) {
  if (!xs) return hipErrorInvalidValue;
  return gemv_bf16_multi_impl(ms, ys, n, nullptr, xs, x_stride, M, y_bf16, st);
}

// One f32 activation row per matrix (xs[i], or the shared x when xs is
// null), f32 or bf16 output rows: the XF form of the dot2 kernel, all
// matrices (same I, bits, group size, aux type) in one launch.
hipError_t launch_gemv_f32x_multi(const DevMat *ms, const float *x, const float *const *xs,
                                  void *const *ys, int n, int y_bf16, hipStream_t st) {
  if (n <= 0 || n > kMultiMax) return hipErrorInvalidValue;
  for (int i = 0; i < n; ++i) {
    if (!gemv_bf16_supported(ms[i]) || ms[i].I != ms[0].I || ms[i].bits != ms[0].bits ||
        ms[i].gs != ms[0].gs || ms[i].fp16 != ms[0].fp16 || !ys[i])
      return hipErrorInvalidValue;
    const float *xi = xs ? xs[i] : x;
    if (!xi || (reinterpret_cast<uintptr_t>(xi) & 15) != 0) return hipErrorInvalidValue;
  }
  GemvMultiParams mp{};
  GemvParams &p = mp.common;
  p.I = ms[0].I;
  p.gsc = ms[0].gs / 32;
  p.gsc_shift = (p.gsc & (p.gsc - 1)) == 0 ? __builtin_ctz(p.gsc) : -1;
  p.fp16 = ms[0].fp16;
  p.x = reinterpret_cast<const uint16_t *>(x);
  p.x_stride = p.I;
  p.M = 2;
  p.y_bf16 = y_bf16;
  mp.n = n;
  for (int i = 0; i < n; ++i) {
    mp.d[i].x = xs ? reinterpret_cast<const uint16_t *>(xs[i]) : nullptr;
    mp.d[i].w = ms[i].w;
    mp.d[i].sc = ms[i].sc;
    mp.d[i].bi = ms[i].bi;
    mp.d[i].row_bytes = ms[i].row_bytes;
    mp.d[i].O = ms[i].O;
    mp.d[i].ng = ms[i].ng;
    mp.d[i].y = ys[i];
  }
  if (n == 1) {  // the single-matrix kernel
    p.w = ms[0].w;
    p.sc = ms[0].sc;
    p.bi = ms[0].bi;
    p.row_bytes = ms[0].row_bytes;
    p.O = ms[0].O;
    p.ng = ms[0].ng;
    p.y = ys[0];
    p.y_stride = ms[0].O;
    if (xs) p.x = reinterpret_cast<const uint16_t *>(xs[0]);
    return gemv_dispatch_bits<2, true>(p, ms[0].bits, st, nullptr);
  }
  return gemv_dispatch_bits<2, true>(p, ms[0].bits, st, &mp);
}

// ---------------------------------------------------------------------------
// Generic exact-dequant GEMV (f32 activations), descriptor-batched.

__device__ __forceinline__ uint32_t code_generic(const uint8_t *row, int col, int bits) {
  const int bit = col * bits;
  const int wi = bit >> 5, sh = bit & 31;
  const uint32_t *wr = reinterpret_cast<const uint32_t *>(row);
  uint64_t comb = wr[wi];
  if (sh + bits > 32) comb |= (uint64_t)wr[wi + 1] << 32;
  return (uint32_t)((comb >> sh) & ((1ull << bits) - 1ull));
}

__global__ __launch_bounds__(256) void gemv_generic_kernel(GenBatch b) {
  int di = 0;
#pragma unroll 1
  while (di + 1 < b.n && (int)blockIdx.x >= b.block_start[di + 1]) ++di;
  const GenDesc &d = b.d[di];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = (blockIdx.x - b.block_start[di]) * kGenRowsPerBlock + wave;
  if (row >= d.O) return;
  const uint8_t *wr = d.w + (size_t)row * d.row_bytes;
  const int ng = d.I / d.gs;
  for (int s = 0; s < d.S; ++s) {
    const float *xs = d.x + (size_t)s * d.x_stride;
    const float *us = d.xmode ? d.up + (size_t)s * d.x_stride : nullptr;
    float acc = 0.f;
    for (int c = lane; c < d.I; c += 64) {
      const int g = row * ng + c / d.gs;
      const float sc = aux_to_f32(d.sc[g], d.fp16);
      const float bi = aux_to_f32(d.bi[g], d.fp16);
      const float wv = fmaf((float)code_generic(wr, c, d.bits), sc, bi);
      float xv = xs[c];
      if (d.xmode) xv = (xv / (1.0f + expf(-xv))) * us[c];
      acc = fmaf(wv, xv, acc);
    }
    acc = team_sum<64>(acc);
    if (lane == 0) d.y[(size_t)s * d.y_stride + row] = acc;
  }
}

hipError_t launch_gemv_generic(const GenBatch &b, hipStream_t st) {
  if (b.n <= 0 || b.n > kMaxDescs) return hipErrorInvalidValue;
  const int blocks = b.block_start[b.n];
  if (blocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(gemv_generic_kernel, dim3(blocks), dim3(256), 0, st, b);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void dequant_kernel(DevMat m, int row0, int nrows, float *out) {
  const long long n = (long long)nrows * m.I;
  for (long long e = (long long)blockIdx.x * 256 + threadIdx.x; e < n; e += (long long)gridDim.x * 256) {
    const int r = (int)(e / m.I), c = (int)(e % m.I);
    const int row = row0 + r;
    const int g = row * m.ng + c / m.gs;
    const float code = (float)code_generic(m.w + (size_t)row * m.row_bytes, c, m.bits);
    // separate multiply and add, as the reference (colisource.rs:852)
    const float prod = __fmul_rn(code, aux_to_f32(m.sc[g], m.fp16));
    out[e] = __fadd_rn(prod, aux_to_f32(m.bi[g], m.fp16));
  }
}

hipError_t launch_dequant(const DevMat &m, int row0, int nrows, float *out, hipStream_t st) {
  if (nrows <= 0) return hipSuccess;
  const long long n = (long long)nrows * m.I;
  long long blocks = (n + 255) / 256;
  if (blocks > 65535) blocks = 65535;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, st, m, row0, nrows, out);
  return hipGetLastError();
}

}  // namespace lh
