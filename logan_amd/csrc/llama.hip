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
constexpr int kDU = 4;    // rows per block in the dense GEMV

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

// ---- dense GEMV: y[r] = (res ? res[r] : 0) + sum_j w[r][j] x[j] ----------
//
// A block owns kDU rows; its 4 waves split the 16-column chunks of those
// rows (wave w, lane l: chunks 64 w + l, + 256, ...), the next chunk's loads
// in flight while the current one is used; the 4 wave partials of a row are
// added in wave order.
template <int FMT>
__global__ __launch_bounds__(kLT) void dense_gemv_kernel(DenseBatch b) {
  int di = 0;
  while (di + 1 < b.n && (int)blockIdx.x >= b.block_start[di + 1]) ++di;
  const DenseDesc d = b.d[di];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = ((int)blockIdx.x - b.block_start[di]) * kDU;
  const int C = d.I >> 4;
  const uint16_t *xh = d.xhl, *xl = d.xhl + d.I;
  constexpr int WD = FMT == 5 ? 8 : 4;  // dwords of one row's 16-column chunk
  struct Chunk {
    uint32_t w[kDU][WD];
    uint32_t sb[FMT == 5 ? 1 : kDU];  // fmt 15: scale | bias << 16
    uint32_t hi[8], lo[8];
  };
  auto load = [&](int c, Chunk &k) {
    const int cc = c < C ? c : C - 1;
#pragma unroll
    for (int u = 0; u < kDU; ++u) {
      const int row = min(r0 + u, d.O - 1);
      if constexpr (FMT == 5) {
        const uint4 *p = reinterpret_cast<const uint4 *>(
            reinterpret_cast<const uint16_t *>(d.w) + (size_t)row * d.I + 16 * (size_t)cc);
        const uint4 a = p[0], bq = p[1];
        k.w[u][0] = a.x; k.w[u][1] = a.y; k.w[u][2] = a.z; k.w[u][3] = a.w;
        k.w[u][4] = bq.x; k.w[u][5] = bq.y; k.w[u][6] = bq.z; k.w[u][7] = bq.w;
      } else {
        const uint4 a = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint8_t *>(d.w) +
                                                         (size_t)row * d.I + 16 * (size_t)cc);
        k.w[u][0] = a.x; k.w[u][1] = a.y; k.w[u][2] = a.z; k.w[u][3] = a.w;
        const size_t g = (size_t)row * (d.I >> 6) + (cc >> 2);
        k.sb[u] = (uint32_t)d.sc[g] | ((uint32_t)d.bi[g] << 16);
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
  float acc[kDU];
#pragma unroll
  for (int u = 0; u < kDU; ++u) acc[u] = 0.f;
  auto use = [&](int c, const Chunk &k) {
    if (c >= C) return;
#pragma unroll
    for (int u = 0; u < kDU; ++u) {
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
  Chunk k0, k1;
  int c = wave * 64 + lane;
  load(c, k0);
  for (; c < C; c += 512) {
    load(c + 256, k1);
    use(c, k0);
    load(c + 512, k0);
    use(c + 256, k1);
  }
  __shared__ float red[kLT / 64][kDU];
#pragma unroll
  for (int u = 0; u < kDU; ++u) {
    const float t = team_sum<64>(acc[u]);
    if (lane == 0) red[wave][u] = t;
  }
  __syncthreads();
  if (threadIdx.x < kDU) {
    const int row = r0 + threadIdx.x;
    float t = red[0][threadIdx.x];
#pragma unroll
    for (int w = 1; w < kLT / 64; ++w) t += red[w][threadIdx.x];
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
  constexpr int rows_per_block = kDU;
  b.block_start[0] = 0;
  for (int i = 0; i < b.n; ++i) {
    const DenseDesc &d = b.d[i];
    if (!dense_supported(fmt, d.O, d.I, d.w) || !d.xhl || !d.y) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(d.xhl) & 15) != 0) return hipErrorInvalidValue;
    if (fmt == 15 && (!d.sc || !d.bi)) return hipErrorInvalidValue;
    b.block_start[i + 1] = b.block_start[i] + (d.O + rows_per_block - 1) / rows_per_block;
  }
  const dim3 grid(b.block_start[b.n]);
  if (fmt == 5) hipLaunchKernelGGL(dense_gemv_kernel<5>, grid, dim3(kLT), 0, st, b);
  else hipLaunchKernelGGL(dense_gemv_kernel<15>, grid, dim3(kLT), 0, st, b);
  return hipGetLastError();
}

// ---- the layer's small kernels --------------------------------------------

// out = hi/lo halves of x * (1 / sqrt(sum x^2 / n + eps)) * w (a_rmsnorm,
// backend_metal.mm:705-714; rms_norm_into, logan-llama/src/model.rs
// :1067-1073). One block; n a multiple of 4; loads unrolled so each thread's
// are in flight together.
__global__ __launch_bounds__(kLT) void rmsnorm_hl_kernel(const float *x, const float *w, int n,
                                                         float eps, uint16_t *out) {
  __shared__ float red[kLT / 64];
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

// RoPE on the q and k heads of qkv [q | k | v] (pairs j, j + hd/2, angle
// pos / theta^(2j/hd), logan-llama/src/model.rs:786-796, :1087-1100;
// llama_qkv_rope, backend_metal.mm:1328-1356), then K[pos] = k, V[pos] = v
// (llama_cache_store :1358-1368).
__global__ __launch_bounds__(kLT) void rope_store_kernel(float *qkv, float *kc, float *vc, int H,
                                                         int KH, int hd, int pos, float theta) {
  const int half = hd >> 1, qdim = H * hd, kvdim = KH * hd;
  const int rope_tasks = (H + KH) * half;
  const int t = blockIdx.x * kLT + threadIdx.x;
  if (t < rope_tasks) {
    const int head = t / half, j = t % half;
    // the angle as the CPU path forms it, in f32: pos / powf(theta, 2j / hd)
    const float ex = __fdiv_rn((float)(2 * j), (float)hd);
    const float pw = (float)pow((double)theta, (double)ex);
    const float ang = __fdiv_rn((float)pos, pw);
    const float co = (float)cos((double)ang), si = (float)sin((double)ang);
    float *v = qkv + (head < H ? head * hd : qdim + (head - H) * hd);
    const float a = v[j], bb = v[j + half];
    const float ra = a * co - bb * si, rb = a * si + bb * co;
    v[j] = ra;
    v[j + half] = rb;
    if (head >= H) {
      float *kr = kc + (size_t)pos * kvdim + (head - H) * hd;
      kr[j] = ra;
      kr[j + half] = rb;
    }
  } else if (t < rope_tasks + kvdim) {
    const int i = t - rope_tasks;
    vc[(size_t)pos * kvdim + i] = qkv[qdim + kvdim + i];
  }
}

// Attention over T = pos + 1 cached positions (logan-llama/src/model.rs
// :838-869; llama_attn_score / spark_softmax / llama_attn_ctx,
// backend_metal.mm:1290-1302, :1370-1408): s_t = q.K[t] / sqrt(hd),
// p = softmax(s), att = sum_t p_t V[t], split over T in slices of kAttnTS
// positions. Block (h, slice) forms its slice's scores, their max m, the
// sum l of exp(s - m) and o = sum exp(s_t - m) V[t]; a second kernel joins
// the slices in order, rescaling each by exp(m_slice - m_max), and writes
// att = o / l as hi/lo halves.
constexpr int kAttnQ = 16;   // q values per lane: head_dim <= 256
constexpr int kAttnTS = 64;  // positions per slice

__global__ __launch_bounds__(kLT) void attn_slice_kernel(const float *qkv, const float *kc,
                                                         const float *vc, float *part, int H,
                                                         int KH, int hd, int T) {
  __shared__ float red[kLT / 64];
  __shared__ float es[kAttnTS];
  __shared__ float ps[kLT];
  const int h = blockIdx.x, sl = blockIdx.y, S = gridDim.y;
  const int kh = h / (H / KH), kvdim = KH * hd;
  const int t0 = sl * kAttnTS, nt = min(kAttnTS, T - t0);
  const int sub = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const float *q = qkv + h * hd;
  const float rs = sqrtf((float)hd);
  float qr[kAttnQ];
#pragma unroll
  for (int i = 0; i < kAttnQ; ++i) qr[i] = sub + 16 * i < hd ? q[sub + 16 * i] : 0.f;
  const float *kb = kc + kh * hd + sub;
  // scores: 16 groups of 16 lanes, 4 positions per group, loads together
  float a[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = t0 + min(16 * j + grp, nt - 1);
    const float *k = kb + (size_t)t * kvdim;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kAttnQ; ++i)
      if (sub + 16 * i < hd) acc = fmaf(qr[i], k[16 * i], acc);
    a[j] = acc;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float sc = __fdiv_rn(team_sum<16>(a[j]), rs);
    a[j] = sc;
    if (16 * j + grp < nt) mx = fmaxf(mx, sc);
  }
  mx = block_max(mx, red);
  float l = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tl = 16 * j + grp;
    const float e = tl < nt ? __expf(a[j] - mx) : 0.f;
    if (sub == 0) es[tl] = e;
    if (sub == 0) l += e;
  }
  l = block_sum(l, red);  // its barriers publish es[]
  // o[d] = sum_t e_t V[t][d]: P partitions of hd threads, positions p, p + P, ...
  const int P = kLT / hd;
  const int d = threadIdx.x % hd, p = threadIdx.x / hd;
  float o = 0.f;
  if (p < P) {
    const float *vcol = vc + (size_t)t0 * kvdim + kh * hd + d;
#pragma unroll 8
    for (int t = p; t < nt; t += P) o = fmaf(es[t], vcol[(size_t)t * kvdim], o);
  }
  ps[threadIdx.x] = o;
  __syncthreads();
  float *pr = part + ((size_t)h * S + sl) * (hd + 2);
  if (threadIdx.x < hd) {
    float v = 0.f;
    for (int pp = 0; pp < P; ++pp) v += ps[pp * hd + threadIdx.x];
    pr[2 + threadIdx.x] = v;
  }
  if (threadIdx.x == 0) {
    pr[0] = mx;
    pr[1] = l;
  }
}

__global__ __launch_bounds__(kLT) void attn_join_kernel(const float *part, uint16_t *att, int H,
                                                        int hd, int S) {
  const int i = blockIdx.x * kLT + threadIdx.x;
  if (i >= H * hd) return;
  const int h = i / hd, d = i % hd;
  const float *pr = part + (size_t)h * S * (hd + 2);
  float m = -INFINITY;
  for (int sl = 0; sl < S; ++sl) m = fmaxf(m, pr[(size_t)sl * (hd + 2)]);
  float l = 0.f, o = 0.f;
  for (int sl = 0; sl < S; ++sl) {
    const float *q = pr + (size_t)sl * (hd + 2);
    const float f = __expf(q[0] - m);
    l = fmaf(q[1], f, l);
    o = fmaf(q[2 + d], f, o);
  }
  put_hl(att, H * hd, i, __fdiv_rn(o, l));
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
  if (w) {
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
  if (m.hd <= 0 || m.hd % 2 != 0 || m.hd > 16 * kAttnQ || !(m.theta > 0.f) || !(m.eps > 0.f))
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
  const int T = pos + 1, qdim = m.H * m.hd, kvdim = m.KH * m.hd;
  LlamaWs w;
  llama_ws_layout(m, T, reinterpret_cast<uint8_t *>(ws), &w);
  hipLaunchKernelGGL(rmsnorm_hl_kernel, dim3(1), dim3(kLT), 0, st, x, in_norm, m.D, m.eps, w.xhl);
  const DenseDesc qkv[3] = {ddesc(mats[0], w.xhl, w.qkv, nullptr),
                            ddesc(mats[1], w.xhl, w.qkv + qdim, nullptr),
                            ddesc(mats[2], w.xhl, w.qkv + qdim + kvdim, nullptr)};
  hipError_t e = launch_dense_set(mats, qkv, 3, st);
  if (e != hipSuccess) return e;
  const int rs_tasks = (m.H + m.KH) * (m.hd / 2) + kvdim;
  hipLaunchKernelGGL(rope_store_kernel, dim3((rs_tasks + kLT - 1) / kLT), dim3(kLT), 0, st, w.qkv,
                     kc, vc, m.H, m.KH, m.hd, pos, m.theta);
  const int S = (T + kAttnTS - 1) / kAttnTS;
  hipLaunchKernelGGL(attn_slice_kernel, dim3(m.H, S), dim3(kLT), 0, st, w.qkv, kc, vc, w.part,
                     m.H, m.KH, m.hd, T);
  hipLaunchKernelGGL(attn_join_kernel, dim3((m.H * m.hd + kLT - 1) / kLT), dim3(kLT), 0, st,
                     w.part, w.atthl, m.H, m.hd, S);
  const DenseDesc od = ddesc(mats[3], w.atthl, x, x);
  e = launch_dense_set(mats + 3, &od, 1, st);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(rmsnorm_hl_kernel, dim3(1), dim3(kLT), 0, st, x, post_norm, m.D, m.eps, w.pnhl);
  const DenseDesc gu[2] = {ddesc(mats[4], w.pnhl, w.mg, nullptr), ddesc(mats[5], w.pnhl, w.mu, nullptr)};
  e = launch_dense_set(mats + 4, gu, 2, st);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(silu_mul_hl_kernel, dim3((m.inter + kLT - 1) / kLT), dim3(kLT), 0, st, w.mg,
                     w.mu, m.inter, w.hhl);
  const DenseDesc dd = ddesc(mats[6], w.hhl, x, x);
  e = launch_dense_set(mats + 6, &dd, 1, st);
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

}  // namespace lh
