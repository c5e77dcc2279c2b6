// Dense Llama / MiniCPM5 decode layer (logan-metal's coli_metal_llama_layer,
// logan-metal/metal/backend_metal.mm:2652-2779; the CPU form it must agree
// with is logan-llama/src/model.rs:786-905), for one token at position pos:
//
//   xn = rmsnorm(x, in_norm); q, k, v = Wq xn, Wk xn, Wv xn
//   rope(q, k) at pos (pairs j, j + hd/2; angle pos / theta^(2j/hd))
//   K[pos], V[pos] = k, v
//   per head h (kv head h / (H/KH)): s_t = q.K[t] / sqrt(hd), t <= pos;
//     p = softmax(s); att_h = sum_t p_t V[t]
//   x += Wo att; pn = rmsnorm(x, post_norm)
//   x += Wdown (silu(Wgate pn) * Wup pn)
//
// The residual stream, K/V cache and every intermediate stay f32. Weights
// are bf16 values: fmt 5 holds them raw ([O][I] bf16), fmt 15 holds MLX
// affine-8 codes with bf16 scale/bias per 64 columns, each weight formed
// as RNE_bf16(code * scale + bias) on the fly — what the reference's
// affine-8 QMV computes (spark_qmv_affine8_fast, backend_metal.mm
// :1143-1193) and what logan-llama's loader stores for fmt 5
// (logan-llama/src/weights.rs:441-516; code * scale is exact in f32, so one
// fma gives the same value). Products of a bf16 weight with an f32
// activation run on v_dot2_f32_bf16 with the activation split into bf16
// hi + lo halves (|x - hi - lo| <= 2^-18 |x|); the producers of every GEMV
// input (the RMSNorms, the attention, the SwiGLU) write those halves
// directly.
#include <cmath>

#include "affine_dev.hpp"
#include "lh_internal.hpp"

namespace lh {

namespace {

constexpr int kLT = 256;  // threads per block

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// hi/lo bf16 halves of f32 v, stored at hl[i] and hl[n + i]
__device__ __forceinline__ void put_hl(uint16_t *hl, int n, int i, float v) {
  const uint32_t hi = f32_to_bf16_rne(v);
  hl[i] = (uint16_t)hi;
  hl[n + i] = (uint16_t)f32_to_bf16_rne(v - bf16_to_f32(hi));  // v - hi is exact
}

// Device-scope (sc1) stores and loads: coherent across the XCDs' L2s, for
// values one block of a running kernel hands to another (an agent-scope
// fence would write back / invalidate the whole L2 instead).
__device__ __forceinline__ void st_dev(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float *p) {
  return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ float block_sum(float v, float *red) {
  v = team_sum<64>(v);
  __syncthreads();  // red may still be read by a previous reduction
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < kLT / 64; ++i) t += red[i];
  return t;
}

__device__ float block_max(float v, float *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < kLT / 64; ++i) t = fmaxf(t, red[i]);
  return t;
}

}  // namespace

// out = hi/lo halves of x * (1 / sqrt(sum x^2 / n + eps)) * w (a_rmsnorm,
// backend_metal.mm:705-714; rms_norm_into, logan-llama/src/model.rs
// :1067-1073). One block; n a multiple of 4; loads unrolled so each thread's
// are in flight together. Also zeroes ctr[0, nctr) (the attention's
// per-kv-head counters, when this is the layer's first kernel). (Forming the
// norm inside the product blocks instead, the input one in every q/k/v block
// and the post-attention one in the output projection's last block,
// measured 1.5-2.5 us slower per config-2 layer.)
__global__ __launch_bounds__(kLT) void rmsnorm_hl_kernel(const float *x, const float *w, int n,
                                                         float eps, uint16_t *out, int *ctr, int nctr) {
  __shared__ float red[kLT / 64];
  for (int i = threadIdx.x; i < nctr; i += kLT) ctr[i] = 0;
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  const float4 *w4 = reinterpret_cast<const float4 *>(w);
  const int n4 = n >> 2;
  float s = 0.f;
#pragma unroll 4
  for (int i = threadIdx.x; i < n4; i += kLT) {
    const float4 v = x4[i];
    s = fmaf(v.x, v.x, s);
    s = fmaf(v.y, v.y, s);
    s = fmaf(v.z, v.z, s);
    s = fmaf(v.w, v.w, s);
  }
  const float tot = block_sum(s, red);
  const float r = 1.0f / sqrtf(tot / (float)n + eps);
#pragma unroll 4
  for (int i = threadIdx.x; i < n4; i += kLT) {
    const float4 v = x4[i], g = w4[i];
    put_hl(out, n, 4 * i, v.x * r * g.x);
    put_hl(out, n, 4 * i + 1, v.y * r * g.y);
    put_hl(out, n, 4 * i + 2, v.z * r * g.z);
    put_hl(out, n, 4 * i + 3, v.w * r * g.w);
  }
}

// ---- dense GEMV: y[r] = (res ? res[r] : 0) + sum_j w[r][j] x[j] ----------
//
// A block of NT threads owns DU rows; its waves split the 16-column chunks of
// those rows (thread i: chunks i, i + NT, ...). With NCH = 1 (K <= 16 NT) a
// thread loads its one chunk; with NCH = 0 (any K) it keeps the next chunk's
// loads in flight while it uses the current one. The wave partials of a row
// are added in wave order.
template <int FMT, int DU, int NT, int NCH>
__global__ __launch_bounds__(NT) void dense_gemv_kernel(DenseBatch b) {
  int di = 0;
  while (di + 1 < b.n && (int)blockIdx.x >= b.block_start[di + 1]) ++di;
  const DenseDesc d = b.d[di];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // a SwiGLU pair's block holds rows [r0, r0 + DU / 2) of gate (u < DU / 2)
  // and of up; every row's sum is formed as for a single product
  const bool pair = d.w2 != nullptr;
  const int rpb = pair ? DU / 2 : DU;
  const int r0 = ((int)blockIdx.x - b.block_start[di]) * rpb;
  const int C = d.I >> 4;
  const uint16_t *xh = d.xhl, *xl = d.xhl + d.I;
  constexpr int WD = FMT == 5 ? 8 : 4;  // dwords of one row's 16-column chunk
  struct Chunk {
    uint32_t w[DU][WD];
    uint32_t sb[FMT == 5 ? 1 : DU];  // fmt 15: scale | bias << 16
    uint32_t hi[8], lo[8];
  };
  auto load = [&](int c, Chunk &k) {
    const int cc = c < C ? c : C - 1;
#pragma unroll
    for (int u = 0; u < DU; ++u) {
      const bool second = pair && u >= DU / 2;
      const int row = min(r0 + (second ? u - DU / 2 : u), d.O - 1);
      const void *wm = second ? d.w2 : d.w;
      if constexpr (FMT == 5) {
        const uint4 *p = reinterpret_cast<const uint4 *>(
            reinterpret_cast<const uint16_t *>(wm) + (size_t)row * d.I + 16 * (size_t)cc);
        const uint4 a = p[0], bq = p[1];
        k.w[u][0] = a.x; k.w[u][1] = a.y; k.w[u][2] = a.z; k.w[u][3] = a.w;
        k.w[u][4] = bq.x; k.w[u][5] = bq.y; k.w[u][6] = bq.z; k.w[u][7] = bq.w;
      } else {
        // fmt 15: non-temporal loads (codes and scale/bias words are read
        // once per launch): config-2 layer 79.5-80.7 -> 76.3-76.8 us; the
        // raw bf16 rows of fmt 5 measured slower with them (105-107 -> 116 us)
        const uint4 a = ld_stream<uint4, true>(reinterpret_cast<const uint4 *>(
            reinterpret_cast<const uint8_t *>(wm) + (size_t)row * d.I + 16 * (size_t)cc));
        k.w[u][0] = a.x; k.w[u][1] = a.y; k.w[u][2] = a.z; k.w[u][3] = a.w;
        const size_t g = (size_t)row * (d.I >> 6) + (cc >> 2);
        k.sb[u] = (uint32_t)ld_stream<uint16_t, true>((second ? d.sc2 : d.sc) + g) |
                  ((uint32_t)ld_stream<uint16_t, true>((second ? d.bi2 : d.bi) + g) << 16);
      }
    }
    const uint4 *ph = reinterpret_cast<const uint4 *>(xh + 16 * (size_t)cc);
    const uint4 *pl = reinterpret_cast<const uint4 *>(xl + 16 * (size_t)cc);
    const uint4 h0 = ph[0], h1 = ph[1], l0 = pl[0], l1 = pl[1];
    k.hi[0] = h0.x; k.hi[1] = h0.y; k.hi[2] = h0.z; k.hi[3] = h0.w;
    k.hi[4] = h1.x; k.hi[5] = h1.y; k.hi[6] = h1.z; k.hi[7] = h1.w;
    k.lo[0] = l0.x; k.lo[1] = l0.y; k.lo[2] = l0.z; k.lo[3] = l0.w;
    k.lo[4] = l1.x; k.lo[5] = l1.y; k.lo[6] = l1.z; k.lo[7] = l1.w;
  };
  float acc[DU];
#pragma unroll
  for (int u = 0; u < DU; ++u) acc[u] = 0.f;
  auto use = [&](int c, const Chunk &k) {
    if (c >= C) return;
#pragma unroll
    for (int u = 0; u < DU; ++u) {
      uint32_t pr[8];
      if constexpr (FMT == 5) {
#pragma unroll
        for (int q = 0; q < 8; ++q) pr[q] = k.w[u][q];
      } else {
        const float sc = bf16_to_f32(k.sb[u] & 0xffffu), bi = bf16_to_f32(k.sb[u] >> 16);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t v = k.w[u][q];
          const float w0 = fmaf(sc, (float)(v & 0xffu), bi);
          const float w1 = fmaf(sc, (float)((v >> 8) & 0xffu), bi);
          const float w2 = fmaf(sc, (float)((v >> 16) & 0xffu), bi);
          const float w3 = fmaf(sc, (float)(v >> 24), bi);
          pr[2 * q] = pk_bf16(w0, w1);
          pr[2 * q + 1] = pk_bf16(w2, w3);
        }
      }
      float a = acc[u];
#pragma unroll
      for (int q = 0; q < 8; ++q) a = dot2(pr[q], k.hi[q], a);
#pragma unroll
      for (int q = 0; q < 8; ++q) a = dot2(pr[q], k.lo[q], a);
      acc[u] = a;
    }
  };
  int c = threadIdx.x;
  if constexpr (NCH == 1) {
    Chunk k0;
    load(c, k0);
    use(c, k0);
  } else {
    static_assert(NCH == 0, "one chunk up front, or the loop");
    Chunk k0, k1;
    load(c, k0);
    for (; c < C; c += 2 * NT) {
      load(c + NT, k1);
      use(c, k0);
      load(c + 2 * NT, k0);
      use(c + NT, k1);
    }
  }
  __shared__ float red[NT / 64][DU];
#pragma unroll
  for (int u = 0; u < DU; ++u) {
    const float t = team_sum<64>(acc[u]);
    if (lane == 0) red[wave][u] = t;
  }
  __syncthreads();
  auto row_sum = [&](int u) {
    float t = red[0][u];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) t += red[w][u];
    return t;
  };
  if (pair) {
    // h = silu(gate) * up (logan-llama/src/model.rs:888-890) as hi/lo halves
    const int row = r0 + threadIdx.x;
    if (threadIdx.x < DU / 2 && row < d.O)
      put_hl(d.hhl, d.O, row, silu(row_sum(threadIdx.x)) * row_sum(threadIdx.x + DU / 2));
  } else if (threadIdx.x < DU) {
    const float t = row_sum(threadIdx.x);
    const int row = r0 + threadIdx.x;
    if (row < d.O) d.y[row] = d.res ? d.res[row] + t : t;
  }
}

bool dense_supported(int fmt, int O, int I, const void *w) {
  if (O <= 0 || I <= 0 || (reinterpret_cast<uintptr_t>(w) & 15) != 0) return false;
  if (fmt == 5) return I % 16 == 0;
  if (fmt == 15) return I % 64 == 0;
  return false;
}

hipError_t launch_dense_gemv(DenseBatch &b, int fmt, hipStream_t st) {
  if (b.n <= 0 || b.n > kDenseMaxDescs) return hipErrorInvalidValue;
  // by the longest K: at most one 16-column chunk per thread (K <= 4096): 8
  // rows per block, each thread's loads issued at once; longer: 4 rows, the
  // next chunk in flight while one is used (two chunks per thread of 512
  // threads measured no faster for the 4096 x 14336 down product)
  int kmax = 0;
  for (int i = 0; i < b.n; ++i) kmax = b.d[i].I > kmax ? b.d[i].I : kmax;
  const bool one = kmax <= 16 * kLT;
  const int rows_per_block = one ? 8 : 4;
  b.block_start[0] = 0;
  for (int i = 0; i < b.n; ++i) {
    const DenseDesc &d = b.d[i];
    if (!dense_supported(fmt, d.O, d.I, d.w) || !d.xhl) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(d.xhl) & 15) != 0) return hipErrorInvalidValue;
    if (fmt == 15 && (!d.sc || !d.bi)) return hipErrorInvalidValue;
    const bool pair = d.w2 != nullptr;
    if (pair ? !dense_supported(fmt, d.O, d.I, d.w2) || !d.hhl || (fmt == 15 && (!d.sc2 || !d.bi2))
             : !d.y)
      return hipErrorInvalidValue;
    const int rpb = pair ? rows_per_block / 2 : rows_per_block;
    b.block_start[i + 1] = b.block_start[i] + (d.O + rpb - 1) / rpb;
  }
  const dim3 grid(b.block_start[b.n]), block(kLT);
  if (fmt == 5) {
    if (one) hipLaunchKernelGGL((dense_gemv_kernel<5, 8, kLT, 1>), grid, block, 0, st, b);
    else hipLaunchKernelGGL((dense_gemv_kernel<5, 4, kLT, 0>), grid, block, 0, st, b);
  } else {
    if (one) hipLaunchKernelGGL((dense_gemv_kernel<15, 8, kLT, 1>), grid, block, 0, st, b);
    else hipLaunchKernelGGL((dense_gemv_kernel<15, 4, kLT, 0>), grid, block, 0, st, b);
  }
  return hipGetLastError();
}

// ---- the layer's small kernels --------------------------------------------

// Attention for one token at position pos over T = pos + 1 cached positions,
// with RoPE and the cache store fused in (logan-llama/src/model.rs:786-869;
// llama_qkv_rope, llama_cache_store, llama_attn_score, spark_softmax,
// llama_attn_ctx: backend_metal.mm:1290-1408):
//   RoPE on q and k (pairs j, j + hd/2, angle pos / theta^(2j/hd));
//   K[pos], V[pos] = k, v;
//   per head h (kv head h / G, G = H / KH): s_t = q.K[t] / sqrt(hd), t <= pos;
//   p = softmax(s); att_h = sum_t p_t V[t], stored as hi/lo halves.
// Block (kv head kh, slice sl of kAttnTS positions) serves the G query heads
// of kh, so each K/V row is read once: the angles' cos/sin formed once per
// block, RoPE on the G q rows and, in the slice holding pos, on the new k row
// (that block alone stores k and v at pos; the slice's own reads of position
// pos take them from LDS), the scores (kAttnTP threads per position, a part
// of the row each), per head the slice max m, l = sum exp(s - m) and
// o = sum exp(s_t - m) V[t]. The last block of kh to finish (a counter per kv
// head, zeroed by the layer's first kernel and reset by that block) joins the
// slices in order, rescaling each by exp(m_slice - m_max), and writes o / l.
// positions per slice (32: 1.5-2.5 us per config-2 layer below 64; 16 no
// better than 32)
constexpr int kAttnTS = 32;
constexpr int kAttnTP = kLT / kAttnTS;  // threads per position in the scores
constexpr int kAttnGMax = 16;  // query heads per kv head

__global__ __launch_bounds__(kLT) void attn_kernel(float *qkv, float *kc, float *vc, float *part,
                                                   int *ctr, uint16_t *att, int H, int KH, int hd,
                                                   int pos, float theta) {
  static_assert(kAttnTP * kAttnTS == kLT && (kAttnTP == 4 || kAttnTP == 8 || kAttnTP == 16),
                "threads per position");
  __shared__ float cs[128], sn[128];          // cos / sin of the hd/2 angles
  __shared__ float qs[kAttnGMax * 256 / 4];  // G roped q rows (G * hd <= 1024)
  __shared__ float kn[256], vn[256];          // the new k (roped) and v rows
  __shared__ float es[kAttnGMax][kAttnTS];   // exp(s - m) per head and position
  __shared__ float ml[kAttnGMax][2];
  __shared__ float red[kLT / 64 * 1024];      // per wave and head: o partials (G * hd <= 1024)
  __shared__ int s_last;
  const int kh = blockIdx.x, sl = blockIdx.y, S = gridDim.y;
  const int G = H / KH, half = hd >> 1, qdim = H * hd, kvdim = KH * hd;
  const int T = pos + 1, t0 = sl * kAttnTS, nt = min(kAttnTS, T - t0);
  const bool has_pos = pos < t0 + kAttnTS;  // the last slice
  const int tid = threadIdx.x;
  // every load of the block first: the K and V rows of the slice (position pos
  // read too, and replaced by the new rows below), the q pairs and the new k, v
  // scores: position t, its row's part qd of hd / kAttnTP values (q4 float4)
  const int t = tid / kAttnTP, qd = tid % kAttnTP, q4 = hd / (4 * kAttnTP);
  const int C4 = hd >> 2, PG = kLT / C4, c4 = tid % C4, pg = tid / C4;  // o: column, group
  constexpr int NPM = kAttnTS / 4;  // positions per thread in o at most (hd <= 256)
  constexpr int KQ = 64 / kAttnTP;   // float4 of a row part at most (hd <= 256)
  const int np = kAttnTS / PG;
  float4 kv[KQ], vv[NPM];
  {
    const int tt = t0 + min(t, nt - 1);
    const float4 *krow = reinterpret_cast<const float4 *>(kc + (size_t)tt * kvdim + kh * hd);
#pragma unroll
    for (int i = 0; i < KQ; ++i)
      if (i < q4) kv[i] = krow[qd * q4 + i];
#pragma unroll
    for (int i = 0; i < NPM; ++i) {
      if (i < np) {
        const int tv = t0 + min(pg + PG * i, nt - 1);
        vv[i] = reinterpret_cast<const float4 *>(vc + (size_t)tv * kvdim + kh * hd)[c4];
      }
    }
  }
  float qa[2], qb[2];  // pairs tid and tid + kLT of the G q rows (G * hd / 2 <= 512)
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int i = tid + r * kLT;
    if (i < G * half) {
      const float *q = qkv + (kh * G + i / half) * hd + i % half;
      qa[r] = q[0];
      qb[r] = q[half];
    }
  }
  float ka = 0.f, kb = 0.f, vnew = 0.f;
  if (has_pos) {
    if (tid < half) {
      ka = qkv[qdim + kh * hd + tid];
      kb = qkv[qdim + kh * hd + tid + half];
    }
    if (tid < hd) vnew = qkv[qdim + kvdim + kh * hd + tid];
  }
  if (tid < half) {
    // the angle as the CPU path forms it, in f32: pos / powf(theta, 2j / hd)
    const float ex = __fdiv_rn((float)(2 * tid), (float)hd);
    const float pw = (float)pow((double)theta, (double)ex);
    const float ang = __fdiv_rn((float)pos, pw);
    const float co = (float)cos((double)ang), si = (float)sin((double)ang);
    cs[tid] = co;
    sn[tid] = si;
    if (has_pos) {
      // the new k row, roped, and v: into LDS and (this block alone) the cache
      const float ra = ka * co - kb * si, rb = ka * si + kb * co;
      float *kr = kc + (size_t)pos * kvdim + kh * hd;
      kn[tid] = ra;
      kn[tid + half] = rb;
      kr[tid] = ra;
      kr[tid + half] = rb;
    }
  }
  if (has_pos && tid < hd) {
    vn[tid] = vnew;
    vc[(size_t)pos * kvdim + kh * hd + tid] = vnew;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int i = tid + r * kLT;
    if (i < G * half) {
      const int g = i / half, j = i % half;
      qs[g * hd + j] = qa[r] * cs[j] - qb[r] * sn[j];
      qs[g * hd + j + half] = qa[r] * sn[j] + qb[r] * cs[j];
    }
  }
  if (has_pos) {
    // position pos: the new rows, not the cache's
    if (t0 + min(t, nt - 1) == pos) {
#pragma unroll
      for (int i = 0; i < KQ; ++i)
        if (i < q4) kv[i] = reinterpret_cast<const float4 *>(kn)[qd * q4 + i];
    }
#pragma unroll
    for (int i = 0; i < NPM; ++i)
      if (i < np && t0 + min(pg + PG * i, nt - 1) == pos) vv[i] = reinterpret_cast<const float4 *>(vn)[c4];
  }
  __syncthreads();
  // scores: position t, the row's quarter qd (hd / 16 float4)
  const float rs = sqrtf((float)hd);
  for (int g = 0; g < G; ++g) {
    const float *q = qs + g * hd + 4 * qd * q4;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < KQ; ++i) {
      if (i < q4) {
        acc = fmaf(q[4 * i], kv[i].x, acc);
        acc = fmaf(q[4 * i + 1], kv[i].y, acc);
        acc = fmaf(q[4 * i + 2], kv[i].z, acc);
        acc = fmaf(q[4 * i + 3], kv[i].w, acc);
      }
    }
#pragma unroll
    for (int o = 1; o < kAttnTP; o <<= 1) acc += __shfl_xor(acc, o, 64);
    if (qd == 0) es[g][t] = __fdiv_rn(acc, rs);
  }
  __syncthreads();
  // softmax over the slice, one wave per head
  const int lane = tid & 63, wave = tid >> 6;
  for (int g = wave; g < G; g += kLT / 64) {
    const float sc = lane < kAttnTS ? es[g][lane] : 0.f;
    float mx = lane < nt ? sc : -INFINITY;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const float e = lane < nt ? __expf(sc - mx) : 0.f;
    const float l = team_sum<64>(e);
    if (lane < kAttnTS) es[g][lane] = e;
    if (lane == 0) {
      ml[g][0] = mx;
      ml[g][1] = l;
    }
  }
  __syncthreads();
  // o = sum_t e_t V[t]: column float4 c4, positions pg, pg + PG, ...; the
  // position groups of a wave added by shuffles, then the waves' in wave order
  for (int g = 0; g < G; ++g) {
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < NPM; ++i) {
      if (i < np) {
        const float e = es[g][pg + PG * i];  // 0 past the slice's positions
        o.x = fmaf(e, vv[i].x, o.x);
        o.y = fmaf(e, vv[i].y, o.y);
        o.z = fmaf(e, vv[i].z, o.z);
        o.w = fmaf(e, vv[i].w, o.w);
      }
    }
    for (int off = C4; off < 64; off <<= 1) {
      o.x += __shfl_xor(o.x, off, 64);
      o.y += __shfl_xor(o.y, off, 64);
      o.z += __shfl_xor(o.z, off, 64);
      o.w += __shfl_xor(o.w, off, 64);
    }
    if (lane < C4) reinterpret_cast<float4 *>(red)[(wave * G + g) * C4 + c4] = o;
  }
  __syncthreads();
  // The slice partials go out as device-scope stores and the joining block
  // reads them with device-scope loads; each block's stores complete (vmcnt)
  // before its counter increment.
  for (int i = tid; i < G * hd; i += kLT) {
    const int g = i / hd, d = i % hd;
    float v = 0.f;
    for (int w = 0; w < kLT / 64; ++w) v += red[(w * G + g) * hd + d];
    float *pr = part + ((size_t)(kh * G + g) * S + sl) * (hd + 2);
    st_dev(pr + 2 + d, v);
    if (d == 0) {
      st_dev(pr, ml[g][0]);
      st_dev(pr + 1, ml[g][1]);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // the last block of kv head kh joins its heads' slices
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(&ctr[kh], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
  __syncthreads();
  if (!s_last) return;
  for (int i = tid; i < G * hd; i += kLT) {
    const int h = kh * G + i / hd, d = i % hd;
    const float *pr = part + (size_t)h * S * (hd + 2);
    // slices in groups of 8, their (m, l, o) loads in flight together
    float m = -INFINITY;
    for (int s0 = 0; s0 < S; s0 += 8) {
      float mv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) mv[j] = s0 + j < S ? ld_dev(pr + (size_t)(s0 + j) * (hd + 2)) : -INFINITY;
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, mv[j]);
    }
    float l = 0.f, o = 0.f;
    for (int s0 = 0; s0 < S; s0 += 8) {
      float mv[8], lv[8], ov[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (s0 + j < S) {
          const float *q = pr + (size_t)(s0 + j) * (hd + 2);
          mv[j] = ld_dev(q);
          lv[j] = ld_dev(q + 1);
          ov[j] = ld_dev(q + 2 + d);
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (s0 + j < S) {
          const float f = __expf(mv[j] - m);
          l = fmaf(lv[j], f, l);
          o = fmaf(ov[j], f, o);
        }
      }
    }
    put_hl(att, qdim, h * hd + d, __fdiv_rn(o, l));
  }
  if (tid == 0) __hip_atomic_store(&ctr[kh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// h = silu(g) * u (logan-llama/src/model.rs:888-890; moe_silu,
// backend_metal.mm:698-699) as hi/lo halves
__global__ __launch_bounds__(kLT) void silu_mul_hl_kernel(const float *g, const float *u, int n,
                                                          uint16_t *out) {
  const int i = blockIdx.x * kLT + threadIdx.x;
  if (i < n) put_hl(out, n, i, silu(g[i]) * u[i]);
}

// ---- the layer ---------------------------------------------------------------

namespace {
inline size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

struct LlamaWs {
  uint16_t *xhl, *atthl, *pnhl, *hhl;
  float *qkv, *part, *mg, *mu;
  int *ctr;
};

size_t llama_ws_layout(const LlamaDims &m, int T, uint8_t *base, LlamaWs *w) {
  const int qdim = m.H * m.hd, kvdim = m.KH * m.hd;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    uint8_t *p = base ? base + off : nullptr;
    off += al256(bytes);
    return p;
  };
  uint8_t *xhl = take((size_t)2 * m.D * 2), *qkv = take((size_t)(qdim + 2 * kvdim) * 4);
  const int S = (T + kAttnTS - 1) / kAttnTS;
  uint8_t *prt = take((size_t)m.H * S * (m.hd + 2) * 4), *att = take((size_t)2 * qdim * 2);
  uint8_t *pn = take((size_t)2 * m.D * 2), *mg = take((size_t)m.inter * 4);
  uint8_t *mu = take((size_t)m.inter * 4), *hh = take((size_t)2 * m.inter * 2);
  uint8_t *ctr = take((size_t)m.KH * 4);  // the attention's, per kv head
  if (w) {
    w->ctr = reinterpret_cast<int *>(ctr);
    w->xhl = reinterpret_cast<uint16_t *>(xhl);
    w->qkv = reinterpret_cast<float *>(qkv);
    w->part = reinterpret_cast<float *>(prt);
    w->atthl = reinterpret_cast<uint16_t *>(att);
    w->pnhl = reinterpret_cast<uint16_t *>(pn);
    w->mg = reinterpret_cast<float *>(mg);
    w->mu = reinterpret_cast<float *>(mu);
    w->hhl = reinterpret_cast<uint16_t *>(hh);
  }
  return off;
}

DenseDesc ddesc(const DenseMat &m, const uint16_t *xhl, float *y, const float *res) {
  DenseDesc d{};
  d.w = m.w;
  d.sc = m.sc;
  d.bi = m.bi;
  d.xhl = xhl;
  d.y = y;
  d.res = res;
  d.O = m.O;
  d.I = m.I;
  return d;
}

// matrices reading one activation, grouped into launches by format
hipError_t launch_dense_set(const DenseMat *ms, const DenseDesc *ds, int n, hipStream_t st) {
  for (int fmt : {5, 15}) {
    DenseBatch b{};
    for (int i = 0; i < n; ++i)
      if (ms[i].fmt == fmt) b.d[b.n++] = ds[i];
    if (b.n == 0) continue;
    hipError_t e = launch_dense_gemv(b, fmt, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}
}  // namespace

size_t llama_workspace_bytes(const LlamaDims &m, int T) { return llama_ws_layout(m, T, nullptr, nullptr); }

bool llama_supported(const LlamaDims &m, const DenseMat mats[7]) {
  if (m.D <= 0 || m.inter <= 0 || m.H <= 0 || m.KH <= 0 || m.H % m.KH != 0) return false;
  // head size 32, 64, 128 or 256 (float4 columns that divide the block, and
  // a float4 per score thread),
  // at most kAttnGMax query heads per kv head, G * hd <= 1024
  const int G = m.H / m.KH;
  if (m.hd < 4 * kAttnTP || m.hd > 256 || (m.hd & (m.hd - 1)) != 0 || G > kAttnGMax || G * m.hd > 1024 ||
      !(m.theta > 0.f) || !(m.eps > 0.f))
    return false;
  if (m.D % 16 != 0) return false;  // the norms' float4 loads; the GEMVs need it too
  const int qdim = m.H * m.hd, kvdim = m.KH * m.hd;
  const int ei[7] = {m.D, m.D, m.D, qdim, m.D, m.D, m.inter};
  const int eo[7] = {qdim, kvdim, kvdim, m.D, m.inter, m.inter, m.D};
  for (int i = 0; i < 7; ++i) {
    const DenseMat &d = mats[i];
    if (d.I != ei[i] || d.O != eo[i] || !dense_supported(d.fmt, d.O, d.I, d.w)) return false;
    if (d.fmt == 15 && (!d.sc || !d.bi)) return false;
  }
  return true;
}

hipError_t launch_llama_layer(const DenseMat mats[7], const float *in_norm, const float *post_norm,
                              const LlamaDims &m, float *x, float *kc, float *vc, int pos,
                              void *ws, hipStream_t st) {
  if (!llama_supported(m, mats) || pos < 0 || !x || !kc || !vc || !ws || !in_norm || !post_norm)
    return hipErrorInvalidValue;
  // the attention reads cache rows as float4
  if ((reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc)) & 15) return hipErrorInvalidValue;
  const int T = pos + 1, qdim = m.H * m.hd, kvdim = m.KH * m.hd;
  LlamaWs w;
  llama_ws_layout(m, T, reinterpret_cast<uint8_t *>(ws), &w);
  hipLaunchKernelGGL(rmsnorm_hl_kernel, dim3(1), dim3(kLT), 0, st, x, in_norm, m.D, m.eps, w.xhl,
                     w.ctr, m.KH);
  const DenseDesc qkv[3] = {ddesc(mats[0], w.xhl, w.qkv, nullptr),
                            ddesc(mats[1], w.xhl, w.qkv + qdim, nullptr),
                            ddesc(mats[2], w.xhl, w.qkv + qdim + kvdim, nullptr)};
  hipError_t e = launch_dense_set(mats, qkv, 3, st);
  if (e != hipSuccess) return e;
  const int S = (T + kAttnTS - 1) / kAttnTS;
  hipLaunchKernelGGL(attn_kernel, dim3(m.KH, S), dim3(kLT), 0, st, w.qkv, kc, vc, w.part, w.ctr,
                     w.atthl, m.H, m.KH, m.hd, pos, m.theta);
  const DenseDesc od = ddesc(mats[3], w.atthl, x, x);
  e = launch_dense_set(mats + 3, &od, 1, st);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(rmsnorm_hl_kernel, dim3(1), dim3(kLT), 0, st, x, post_norm, m.D, m.eps, w.pnhl,
                     nullptr, 0);
  if (mats[4].fmt == mats[5].fmt) {
    // gate and up as one SwiGLU pair: h straight from the product
    DenseDesc gu = ddesc(mats[4], w.pnhl, nullptr, nullptr);
    gu.w2 = mats[5].w;
    gu.sc2 = mats[5].sc;
    gu.bi2 = mats[5].bi;
    gu.hhl = w.hhl;
    e = launch_dense_set(mats + 4, &gu, 1, st);
    if (e != hipSuccess) return e;
  } else {
    const DenseDesc gu[2] = {ddesc(mats[4], w.pnhl, w.mg, nullptr), ddesc(mats[5], w.pnhl, w.mu, nullptr)};
    e = launch_dense_set(mats + 4, gu, 2, st);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(silu_mul_hl_kernel, dim3((m.inter + kLT - 1) / kLT), dim3(kLT), 0, st, w.mg,
                       w.mu, m.inter, w.hhl);
  }
  const DenseDesc dd = ddesc(mats[6], w.hhl, x, x);
  e = launch_dense_set(mats + 6, &dd, 1, st);
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

}  // namespace lh
