// C ABI of logan-hip: host-pointer drop-in for logan-metal's affine/MoE entry
// points plus the device-native (HBM-resident) entry points.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/logan_hip.h"
#include "lh_internal.hpp"

struct LoganHipTensor {
  uint8_t *w = nullptr;
  uint16_t *sc = nullptr;
  uint16_t *bi = nullptr;
  int fmt = 0, I = 0, O = 0, gs = 0, bits = 0, fp16 = 0;
  int planes = 0;  // MXFP4 planes (fmt 7 / 9 / 10: 1 / 2 / 3); 0 for affine codes
  size_t wbytes = 0, abytes = 0;
};

namespace {

std::mutex g_mtx;
bool g_tried = false;
bool g_ok = false;
int g_dev = -1;
hipStream_t g_stream = nullptr;
hipEvent_t g_prof_ev0 = nullptr, g_prof_ev1 = nullptr;
size_t g_tensor_count = 0, g_tensor_bytes = 0;
bool g_prof_on = false;
uint64_t g_prof[4] = {0, 0, 0, 0};  // encode, submit, wait, kernel

struct DevBuf {
  void *p = nullptr;
  size_t n = 0;
  // Grows the buffer; the caller guarantees no in-flight work uses it.
  bool ensure(size_t bytes) {
    if (bytes <= n) return true;
    if (p) hipFree(p);
    p = nullptr;
    n = 0;
    if (hipMalloc(&p, bytes) != hipSuccess) {
      p = nullptr;
      return false;
    }
    n = bytes;
    return true;
  }
  void release() {
    if (p) hipFree(p);
    p = nullptr;
    n = 0;
  }
};
DevBuf g_xbuf, g_ybuf, g_ws;
DevBuf g_hlbuf, g_y2buf;  // hi/lo activation pairs and pair products of matmul_multi

// Pinned host staging (hipHostMalloc) for the host-pointer entry points: the
// caller's pageable rows are copied into it on the host and DMA'd from it
// asynchronously, results come back into it (pageable source or destination
// made each copy a staged, synchronous transfer: config-1 drop-in matmul
// 39-48 -> 32 us wall per call).
struct HostBuf {
  void *p = nullptr;
  size_t n = 0;
  // Grows the buffer; the caller guarantees no in-flight copy uses it.
  bool ensure(size_t bytes) {
    if (bytes <= n) return true;
    if (p) hipHostFree(p);
    p = nullptr;
    n = 0;
    if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) {
      p = nullptr;
      return false;
    }
    n = bytes;
    return true;
  }
  void release() {
    if (p) hipHostFree(p);
    p = nullptr;
    n = 0;
  }
};
HostBuf g_hxbuf, g_hybuf;  // matmul_multi's x rows in, y rows out

// Device buffers of one route-island submission: x [D], gate/up outputs
// [2 K M], expert outputs [K D], and the pinned host staging of x and of the
// outputs. Each pending handle owns one set from the pool until
// finish/discard, so calls made between begin and finish (the shared
// expert, other GEMVs, another begin) never touch it.
struct RouteBufs {
  DevBuf x, gu, out;
  HostBuf hx, hout;
  void release() {
    x.release();
    gu.release();
    out.release();
    hx.release();
    hout.release();
  }
};
std::vector<RouteBufs *> g_route_pool;  // idle sets

RouteBufs *route_bufs_take(size_t xb, size_t gub, size_t outb) {
  RouteBufs *b = nullptr;
  if (!g_route_pool.empty()) {
    b = g_route_pool.back();
    g_route_pool.pop_back();
  } else {
    b = new (std::nothrow) RouteBufs();
    if (!b) return nullptr;
  }
  if (!b->x.ensure(xb) || !b->gu.ensure(gub) || !b->out.ensure(outb) || !b->hx.ensure(xb) ||
      !b->hout.ensure(outb)) {
    g_route_pool.push_back(b);
    return nullptr;
  }
  return b;
}

struct RoutePending {
  hipEvent_t ev = nullptr;
  hipEvent_t pev0 = nullptr, pev1 = nullptr;  // around the kernels, when profiling
  RouteBufs *bufs = nullptr;
  int K = 0, D = 0;
};

// back to the pool once the submission's work has retired
void route_release_locked(RoutePending *p) {
  if (p->ev) {
    hipEventSynchronize(p->ev);
    hipEventDestroy(p->ev);
  }
  if (p->pev0) hipEventDestroy(p->pev0);
  if (p->pev1) hipEventDestroy(p->pev1);
  if (p->bufs) g_route_pool.push_back(p->bufs);
  delete p;
}

using clk = std::chrono::steady_clock;
inline uint64_t now_ns() {
  return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
             clk::now().time_since_epoch())
      .count();
}

// Workspace of logan_hip_moe_block_static: a file-scope device array (each
// device that runs the library holds its own copy until the process ends).
// In host code `scratch` only names the variable; its device address comes
// from hipGetSymbolAddress, once per device, with that device current.
constexpr size_t kStaticScratchBytes = LOGAN_HIP_MOE_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mtx;
void *g_scratch_ptr[kMaxDevices];

// The current device's copy of `scratch` (nullptr when it cannot be had).
void *scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mtx);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

bool init_locked() {
  if (g_tried) return g_ok;
  g_tried = true;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return false;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return false;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    std::fprintf(stderr, "[logan-hip] device %d is %s, library is built for gfx950\n", dev,
                 prop.gcnArchName);
    return false;
  }
  if (hipSetDevice(dev) != hipSuccess) return false;
  if (!scratch_on_current_device()) return false;
  // default-priority stream
  if (hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) return false;
  if (hipEventCreate(&g_prof_ev0) != hipSuccess || hipEventCreate(&g_prof_ev1) != hipSuccess)
    return false;
  g_dev = dev;
  g_ok = true;
  return true;
}

// fmt -> (bits, fp16, effective group size); false for non-affine codes.
bool fmt_info(int fmt, int gs_in, int &bits, int &fp16, int &gs) {
  static const int kBits[5] = {4, 5, 6, 8, 4};
  if (fmt == 15) {
    bits = 8;
    fp16 = 0;
    gs = 64;
    return true;
  }
  if (fmt >= 16 && fmt <= 20) {
    bits = kBits[fmt - 16];
    fp16 = 0;
  } else if (fmt >= 21 && fmt <= 24) {
    bits = kBits[fmt - 21];
    fp16 = 1;
  } else {
    return false;
  }
  gs = gs_in;
  return gs > 0;
}

// MXFP4 fmt -> number of stacked planes (backend_metal.mm:1860-1863); 0 otherwise
int mx_planes(int fmt) { return fmt == 7 ? 1 : fmt == 9 ? 2 : fmt == 10 ? 3 : 0; }

bool fmt_known(int fmt, int gs_in) {
  int bits, fp16, gs;
  return mx_planes(fmt) > 0 || fmt_info(fmt, gs_in, bits, fp16, gs);
}

bool geom_ok(long long I, long long O, int bits, int gs) {
  if (I <= 0 || O <= 0 || gs <= 0) return false;
  if (I % gs != 0) return false;
  if ((I * bits) % 32 != 0) return false;
  return true;
}

// Create (first use) or validate the device copy of one affine tensor.
// Returns nullptr on decline.
LoganHipTensor *resolve_mxfp4_locked(LoganHipTensor **slot, const void *weights,
                                     const void *aux, int fmt, int I, int O);

LoganHipTensor *resolve_bf16_locked(LoganHipTensor **slot, const void *weights, int I, int O);

LoganHipTensor *resolve_tensor_locked(LoganHipTensor **slot, const void *weights,
                                      const void *aux, int fmt, int I, int O, int gs_in) {
  if (mx_planes(fmt)) return resolve_mxfp4_locked(slot, weights, aux, fmt, I, O);
  if (fmt == 5) return resolve_bf16_locked(slot, weights, I, O);
  int bits, fp16, gs;
  if (!fmt_info(fmt, gs_in, bits, fp16, gs)) return nullptr;
  if (!geom_ok(I, O, bits, gs)) return nullptr;
  LoganHipTensor *t = slot ? *slot : nullptr;
  if (t) {
    if (t->planes || t->fmt == 5 || t->I != I || t->O != O || t->bits != bits || t->fp16 != fp16 ||
        t->gs != gs)
      return nullptr;
    return t;
  }
  if (!weights || !aux) return nullptr;
  t = new LoganHipTensor();
  t->fmt = fmt;
  t->I = I;
  t->O = O;
  t->gs = gs;
  t->bits = bits;
  t->fp16 = fp16;
  t->wbytes = (size_t)O * ((size_t)I * bits / 8);
  const size_t pbytes = (size_t)O * (I / gs) * 2;
  t->abytes = 2 * pbytes;
  if (hipMalloc(&t->w, t->wbytes) != hipSuccess) {
    delete t;
    return nullptr;
  }
  if (hipMalloc(&t->sc, t->abytes) != hipSuccess) {
    hipFree(t->w);
    delete t;
    return nullptr;
  }
  t->bi = t->sc + pbytes / 2;
  if (hipMemcpy(t->w, weights, t->wbytes, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(t->sc, aux, t->abytes, hipMemcpyHostToDevice) != hipSuccess) {
    hipFree(t->w);
    hipFree(t->sc);
    delete t;
    return nullptr;
  }
  g_tensor_count++;
  g_tensor_bytes += t->wbytes + t->abytes;
  if (slot) *slot = t;
  return t;
}

// MXFP4 tensors (fmt 7 / 9 / 10): codes [planes][O][I/2] and E8M0 scale
// bytes [planes][O][I/32], planes back to back as the reference lays them
// out (backend_metal.mm:460-470). The kernels take I a multiple of 32; other
// widths decline.
LoganHipTensor *resolve_mxfp4_locked(LoganHipTensor **slot, const void *weights,
                                     const void *aux, int fmt, int I, int O) {
  const int planes = mx_planes(fmt);
  if (planes == 0 || I <= 0 || O <= 0 || I % 32 != 0) return nullptr;
  LoganHipTensor *t = slot ? *slot : nullptr;
  if (t) return (t->planes == planes && t->I == I && t->O == O) ? t : nullptr;
  if (!weights || !aux) return nullptr;
  t = new LoganHipTensor();
  t->fmt = fmt;
  t->I = I;
  t->O = O;
  t->gs = 32;
  t->bits = 4;
  t->planes = planes;
  t->wbytes = (size_t)planes * O * (I / 2);
  t->abytes = (size_t)planes * O * (I / 32);
  void *sc = nullptr;
  if (hipMalloc(&t->w, t->wbytes) != hipSuccess) {
    delete t;
    return nullptr;
  }
  if (hipMalloc(&sc, t->abytes) != hipSuccess) {
    hipFree(t->w);
    delete t;
    return nullptr;
  }
  t->sc = reinterpret_cast<uint16_t *>(sc);
  if (hipMemcpy(t->w, weights, t->wbytes, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(sc, aux, t->abytes, hipMemcpyHostToDevice) != hipSuccess) {
    hipFree(t->w);
    hipFree(sc);
    delete t;
    return nullptr;
  }
  g_tensor_count++;
  g_tensor_bytes += t->wbytes + t->abytes;
  if (slot) *slot = t;
  return t;
}

// Raw bf16 weights (fmt 5, [O][I], backend_metal.mm:1865): served by the
// dense kernel, which takes I a multiple of 16; other widths decline.
LoganHipTensor *resolve_bf16_locked(LoganHipTensor **slot, const void *weights, int I, int O) {
  if (I <= 0 || O <= 0 || I % 16 != 0) return nullptr;
  LoganHipTensor *t = slot ? *slot : nullptr;
  if (t) return (t->fmt == 5 && t->I == I && t->O == O) ? t : nullptr;
  if (!weights) return nullptr;
  t = new LoganHipTensor();
  t->fmt = 5;
  t->I = I;
  t->O = O;
  t->bits = 16;
  t->wbytes = (size_t)O * I * 2;
  if (hipMalloc(&t->w, t->wbytes) != hipSuccess) {
    delete t;
    return nullptr;
  }
  if (hipMemcpy(t->w, weights, t->wbytes, hipMemcpyHostToDevice) != hipSuccess) {
    hipFree(t->w);
    delete t;
    return nullptr;
  }
  g_tensor_count++;
  g_tensor_bytes += t->wbytes;
  if (slot) *slot = t;
  return t;
}

lh::DenseMat dense_mat(const LoganHipTensor *t) {
  lh::DenseMat m{};
  m.w = t->w;
  m.sc = t->fmt == 15 ? t->sc : nullptr;
  m.bi = t->fmt == 15 ? t->bi : nullptr;
  m.fmt = t->fmt;
  m.O = t->O;
  m.I = t->I;
  return m;
}

// Dense (fmt 5) products, x as bf16 hi/lo halves, in launches of up to 8.
hipError_t launch_dense5(const std::vector<lh::DenseDesc> &ds, hipStream_t st) {
  for (size_t b0 = 0; b0 < ds.size(); b0 += lh::kDenseMaxDescs) {
    lh::DenseBatch b{};
    b.n = (int)std::min(ds.size() - b0, (size_t)lh::kDenseMaxDescs);
    for (int i = 0; i < b.n; ++i) b.d[i] = ds[b0 + i];
    hipError_t e = lh::launch_dense_gemv(b, 5, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

lh::Mx4Desc mx_desc(const LoganHipTensor *t, const void *x, void *y) {
  lh::Mx4Desc d{};
  d.w = t->w;
  d.sc = reinterpret_cast<const uint8_t *>(t->sc);
  d.x = x;
  d.y = y;
  d.wplane = (long long)t->O * (t->I / 2);
  d.splane = (long long)t->O * (t->I / 32);
  d.O = t->O;
  d.I = t->I;
  d.planes = t->planes;
  return d;
}

// MXFP4 products (f32 activations and outputs) in launches of up to 16.
hipError_t launch_mx_descs(const std::vector<lh::Mx4Desc> &ds, hipStream_t st) {
  for (size_t b0 = 0; b0 < ds.size(); b0 += lh::kMx4MaxDescs) {
    lh::Mx4Batch b{};
    b.n = (int)std::min(ds.size() - b0, (size_t)lh::kMx4MaxDescs);
    for (int i = 0; i < b.n; ++i) b.d[i] = ds[b0 + i];
    b.y_bf16 = 0;
    hipError_t e = lh::launch_mxfp4_gemv(b, true, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

lh::GenDesc gen_desc(const LoganHipTensor *t, const float *x, const float *up, float *y, int S,
                     int x_stride, int y_stride, int xmode) {
  lh::GenDesc d{};
  d.w = t->w;
  d.sc = t->sc;
  d.bi = t->bi;
  d.x = x;
  d.up = up;
  d.y = y;
  d.row_bytes = (long long)t->I * t->bits / 8;
  d.I = t->I;
  d.O = t->O;
  d.gs = t->gs;
  d.bits = t->bits;
  d.fp16 = t->fp16;
  d.S = S;
  d.x_stride = x_stride;
  d.y_stride = y_stride;
  d.xmode = xmode;
  return d;
}

// Launch descriptors in batches of 16.
hipError_t launch_descs(const std::vector<lh::GenDesc> &ds, hipStream_t st) {
  for (size_t b0 = 0; b0 < ds.size(); b0 += lh::kMaxDescs) {
    lh::GenBatch b{};
    b.n = (int)std::min(ds.size() - b0, (size_t)lh::kMaxDescs);
    b.block_start[0] = 0;
    for (int i = 0; i < b.n; ++i) {
      b.d[i] = ds[b0 + i];
      b.block_start[i + 1] =
          b.block_start[i] + (b.d[i].O + lh::kGenRowsPerBlock - 1) / lh::kGenRowsPerBlock;
    }
    hipError_t e = lh::launch_gemv_generic(b, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

void prof_add(int i, uint64_t v) {
  if (g_prof_on) g_prof[i] += v;
}

// After a synchronising wait: fold the device time between the two events.
void prof_kernel_time() {
  if (!g_prof_on) return;
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, g_prof_ev0, g_prof_ev1) == hipSuccess)
    g_prof[3] += (uint64_t)(ms * 1e6);
}

lh::DevMat devmat(const LoganHipAffine &a) {
  lh::DevMat m{};
  m.w = reinterpret_cast<const uint8_t *>(a.weights);
  m.sc = reinterpret_cast<const uint16_t *>(a.scales);
  m.bi = reinterpret_cast<const uint16_t *>(a.biases);
  m.I = a.I;
  m.O = a.O;
  m.gs = a.group_size;
  m.bits = a.bits;
  m.fp16 = a.aux_fp16;
  m.row_bytes = (long long)a.I * a.bits / 8;
  m.ng = a.group_size > 0 ? a.I / a.group_size : 0;
  return m;
}

lh::DevMat tensor_mat(const LoganHipTensor *t) {
  lh::DevMat m{};
  m.w = t->w;
  m.sc = t->sc;
  m.bi = t->bi;
  m.I = t->I;
  m.O = t->O;
  m.gs = t->gs;
  m.bits = t->bits;
  m.fp16 = t->fp16;
  m.row_bytes = (long long)t->I * t->bits / 8;
  m.ng = t->gs > 0 ? t->I / t->gs : 0;  // raw bf16 tensors have no groups
  return m;
}

// staging offsets in elements, rounded so every sub-buffer is 256-byte aligned
inline size_t al_elems(size_t n, size_t esize) {
  const size_t per = 256 / esize;
  return (n + per - 1) / per * per;
}

// Products that share one activation (hi/lo row pairs xhl, 2 S rows) on the
// bf16 kernels, grouped into multi-matrix launches of like geometry.
hipError_t launch_shared_x_groups(const std::vector<lh::DevMat> &ms, const std::vector<void *> &ys,
                                  const uint16_t *xhl, int I, int M2, hipStream_t st) {
  std::vector<char> done(ms.size(), 0);
  for (size_t i = 0; i < ms.size(); ++i) {
    if (done[i]) continue;
    lh::DevMat gm[lh::kGemvMultiMax];
    void *gy[lh::kGemvMultiMax];
    int n = 0;
    for (size_t j = i; j < ms.size() && n < lh::kGemvMultiMax; ++j) {
      if (done[j] || ms[j].bits != ms[i].bits || ms[j].gs != ms[i].gs || ms[j].fp16 != ms[i].fp16)
        continue;
      gm[n] = ms[j];
      gy[n] = ys[j];
      ++n;
      done[j] = 1;
    }
    hipError_t e = lh::launch_gemv_bf16_multi(gm, gy, n, xhl, I, M2, 0, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// One f32 activation row per product (xs[i]) on the dot2 kernel's f32 form,
// grouped into multi-matrix launches of like geometry; outputs f32.
hipError_t launch_f32x_groups(const std::vector<lh::DevMat> &ms, const std::vector<const float *> &xs,
                              const std::vector<void *> &ys, hipStream_t st) {
  std::vector<char> done(ms.size(), 0);
  for (size_t i = 0; i < ms.size(); ++i) {
    if (done[i]) continue;
    lh::DevMat gm[lh::kGemvMultiMax];
    const float *gx[lh::kGemvMultiMax];
    void *gy[lh::kGemvMultiMax];
    int n = 0;
    for (size_t j = i; j < ms.size() && n < lh::kGemvMultiMax; ++j) {
      if (done[j] || ms[j].I != ms[i].I || ms[j].bits != ms[i].bits || ms[j].gs != ms[i].gs ||
          ms[j].fp16 != ms[i].fp16)
        continue;
      gm[n] = ms[j];
      gx[n] = xs[j];
      gy[n] = ys[j];
      ++n;
      done[j] = 1;
    }
    hipError_t e = lh::launch_gemv_f32x_multi(gm, nullptr, gx, gy, n, 0, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

bool affine_ok(const LoganHipAffine *a) {
  if (!a || !a->weights || !a->scales || !a->biases) return false;
  if (!(a->bits == 4 || a->bits == 5 || a->bits == 6 || a->bits == 8)) return false;
  return geom_ok(a->I, a->O, a->bits, a->group_size);
}

lh::DevBank devbank(const LoganHipAffineBank &b) {
  lh::DevBank d{};
  LoganHipAffine a{b.weights, b.scales, b.biases, b.O, b.I, b.bits, b.group_size, b.aux_fp16};
  d.m = devmat(a);
  d.w_stride = (long long)b.O * d.m.row_bytes;
  d.p_stride = (long long)b.O * d.m.ng;
  d.E = b.E;
  return d;
}

int rc_from(hipError_t e) { return e == hipSuccess ? 1 : -1; }


}  // namespace

extern "C" {

int logan_hip_init(void) {
  std::lock_guard<std::mutex> lk(g_mtx);
  return init_locked() ? 1 : 0;
}

int logan_hip_available(void) {
  std::lock_guard<std::mutex> lk(g_mtx);
  return g_ok ? 1 : 0;
}

void logan_hip_shutdown(void) {
  std::lock_guard<std::mutex> lk(g_mtx);
  if (!g_ok) return;
  hipStreamSynchronize(g_stream);
  g_xbuf.release();
  g_ybuf.release();
  g_ws.release();
  g_hxbuf.release();
  g_hybuf.release();
  for (RouteBufs *b : g_route_pool) {
    b->release();
    delete b;
  }
  g_route_pool.clear();
}

void logan_hip_stats(size_t *tensor_count, size_t *tensor_bytes) {
  std::lock_guard<std::mutex> lk(g_mtx);
  if (tensor_count) *tensor_count = g_tensor_count;
  if (tensor_bytes) *tensor_bytes = g_tensor_bytes;
}

int logan_hip_mem_info(size_t *used_bytes, size_t *total_bytes) {
  std::lock_guard<std::mutex> lk(g_mtx);
  if (!g_ok) return 0;
  size_t fr = 0, tot = 0;
  if (hipMemGetInfo(&fr, &tot) != hipSuccess) return 0;
  if (used_bytes) *used_bytes = tot - fr;
  if (total_bytes) *total_bytes = tot;
  return 1;
}

void logan_hip_profile_set_on(int on) {
  std::lock_guard<std::mutex> lk(g_mtx);
  g_prof_on = on != 0;
}

void logan_hip_profile_reset(void) {
  std::lock_guard<std::mutex> lk(g_mtx);
  for (auto &v : g_prof) v = 0;
}

void logan_hip_profile_get(uint64_t *encode_ns, uint64_t *submit_ns, uint64_t *wait_ns,
                           uint64_t *kernel_ns) {
  std::lock_guard<std::mutex> lk(g_mtx);
  if (encode_ns) *encode_ns = g_prof[0];
  if (submit_ns) *submit_ns = g_prof[1];
  if (wait_ns) *wait_ns = g_prof[2];
  if (kernel_ns) *kernel_ns = g_prof[3];
}

int logan_hip_matmul(LoganHipTensor **tensor, float *y, const float *x, const void *weights,
                     const void *scales, int fmt, int S, int I, int O, int gs) {
  if (!tensor || !y || !x || S <= 0) return 0;
  LoganHipMatmulDesc d{};
  d.tensor = *tensor;
  d.y = y;
  d.weights = weights;
  d.scales = reinterpret_cast<const float *>(scales);
  d.fmt = fmt;
  d.I = I;
  d.O = O;
  d.gs = gs;
  d.x = nullptr;
  d.S = S;
  const int rc = logan_hip_matmul_multi(x, S, &d, 1);
  *tensor = d.tensor;
  return rc;
}

int logan_hip_matmul_multi(const float *x, int S, LoganHipMatmulDesc *descs, int count) {
  if (!descs || count <= 0 || count > 16) return 0;
  std::lock_guard<std::mutex> lk(g_mtx);
  if (!g_ok) return 0;
  uint64_t t0 = now_ns();
  // shared activation: every descriptor without its own x must agree on I
  int shared_I = -1;
  for (int i = 0; i < count; ++i) {
    const LoganHipMatmulDesc &d = descs[i];
    if (!d.y) return 0;
    if (!d.x) {
      if (!x || S <= 0) return 0;
      if (shared_I >= 0 && shared_I != d.I) return 0;
      shared_I = d.I;
    } else if (d.S <= 0) {
      return 0;
    }
  }
  std::vector<LoganHipTensor *> ts(count);
  for (int i = 0; i < count; ++i) {
    ts[i] = resolve_tensor_locked(&descs[i].tensor, descs[i].weights, descs[i].scales,
                                  descs[i].fmt, descs[i].I, descs[i].O, descs[i].gs);
    if (!ts[i]) return 0;
  }
  // staging (f32): shared x, then private x's; outputs concatenated. Products
  // whose geometry the bf16 kernels take run there: a one-row activation on
  // the dot2 kernel's f32 form (the row split into bf16 hi + lo in
  // registers, both halves' products added), several rows as bf16 (hi, lo)
  // row pairs through the row-batched kernels with each output row re-joined
  // as y = y_hi + y_lo. The rest take the exact per-element kernel.
  std::vector<lh::DevMat> mat(count);
  std::vector<char> fast(count), dense5(count);
  bool shared_pairs = false;
  for (int i = 0; i < count; ++i) {
    mat[i] = tensor_mat(ts[i]);
    dense5[i] = ts[i]->fmt == 5;
    fast[i] = !ts[i]->planes && !dense5[i] && lh::gemv_bf16_supported(mat[i]);
    shared_pairs = shared_pairs || (!descs[i].x && ((fast[i] && S > 1) || dense5[i]));
  }
  size_t xn = shared_I > 0 ? al_elems((size_t)S * shared_I, 4) : 0, yn = 0;
  size_t hln = shared_pairs ? al_elems((size_t)2 * S * shared_I, 2) : 0, y2n = 0;
  std::vector<size_t> xoff(count, 0), yoff(count, 0), hloff(count, 0), y2off(count, 0);
  for (int i = 0; i < count; ++i) {
    const int s = descs[i].x ? descs[i].S : S;
    if (descs[i].x) {
      xoff[i] = xn;
      xn += al_elems((size_t)s * descs[i].I, 4);
      if ((fast[i] && s > 1) || dense5[i]) {
        hloff[i] = hln;
        hln += al_elems((size_t)2 * s * descs[i].I, 2);
      }
    }
    yoff[i] = yn;
    yn += al_elems((size_t)s * descs[i].O, 4);
    if (fast[i] && s > 1) {
      y2off[i] = y2n;
      y2n += al_elems((size_t)2 * s * descs[i].O, 4);
    }
  }
  if (!g_xbuf.ensure(xn * 4 + 16) || !g_ybuf.ensure(yn * 4 + 16)) return 0;
  if (hln && (!g_hlbuf.ensure(hln * 2 + 16) || !g_y2buf.ensure(y2n * 4 + 16))) return 0;
  float *dx = reinterpret_cast<float *>(g_xbuf.p);
  float *dy = reinterpret_cast<float *>(g_ybuf.p);
  uint16_t *dhl = reinterpret_cast<uint16_t *>(g_hlbuf.p);
  float *dy2 = reinterpret_cast<float *>(g_y2buf.p);
  std::vector<lh::GenDesc> ds;
  std::vector<lh::Mx4Desc> mxs;  // MXFP4: one descriptor per activation row
  std::vector<lh::DenseDesc> d5s;  // raw bf16: one descriptor per activation row
  lh::HiloBatch split{}, join{};
  std::vector<lh::DevMat> shared_m, row_m;
  std::vector<void *> shared_y, row_y;
  std::vector<const float *> row_x;
  if (shared_pairs) split.j[split.n++] = lh::HiloJob{dx, dhl, S, shared_I};
  for (int i = 0; i < count; ++i) {
    const int s = descs[i].x ? descs[i].S : S;
    const float *xs = descs[i].x ? dx + xoff[i] : dx;
    if (ts[i]->planes) {
      for (int r = 0; r < s; ++r)
        mxs.push_back(mx_desc(ts[i], xs + (size_t)r * ts[i]->I, dy + yoff[i] + (size_t)r * ts[i]->O));
    } else if (dense5[i]) {
      const uint16_t *hl = descs[i].x ? dhl + hloff[i] : dhl;
      if (descs[i].x) split.j[split.n++] = lh::HiloJob{xs, dhl + hloff[i], s, descs[i].I};
      for (int r = 0; r < s; ++r) {
        lh::DenseDesc dd{};
        dd.w = ts[i]->w;
        dd.xhl = hl + (size_t)2 * r * ts[i]->I;
        dd.y = dy + yoff[i] + (size_t)r * ts[i]->O;
        dd.O = ts[i]->O;
        dd.I = ts[i]->I;
        d5s.push_back(dd);
      }
    } else if (!fast[i]) {
      ds.push_back(gen_desc(ts[i], xs, nullptr, dy + yoff[i], s, ts[i]->I, ts[i]->O, 0));
    } else if (s == 1) {
      row_m.push_back(mat[i]);
      row_x.push_back(xs);
      row_y.push_back(dy + yoff[i]);
    } else {
      if (descs[i].x) split.j[split.n++] = lh::HiloJob{xs, dhl + hloff[i], s, descs[i].I};
      else {
        shared_m.push_back(mat[i]);
        shared_y.push_back(dy2 + y2off[i]);
      }
      join.j[join.n++] = lh::HiloJob{dy2 + y2off[i], dy + yoff[i], s, descs[i].O};
    }
  }
  uint64_t t1 = now_ns();
  prof_add(0, t1 - t0);
  // every row in through one pinned staging copy (the previous call's copies
  // ended with its stream synchronisation)
  if (!g_hxbuf.ensure(xn * 4 + 16) || !g_hybuf.ensure(yn * 4 + 16)) return 0;
  float *hx = reinterpret_cast<float *>(g_hxbuf.p);
  float *hy = reinterpret_cast<float *>(g_hybuf.p);
  if (shared_I > 0) memcpy(hx, x, (size_t)S * shared_I * 4);
  for (int i = 0; i < count; ++i)
    if (descs[i].x) memcpy(hx + xoff[i], descs[i].x, (size_t)descs[i].S * descs[i].I * 4);
  hipError_t e = hipMemcpyAsync(dx, hx, xn * 4, hipMemcpyHostToDevice, g_stream);
  if (e != hipSuccess) return -1;
  if (g_prof_on) hipEventRecord(g_prof_ev0, g_stream);
  if (!row_m.empty()) e = launch_f32x_groups(row_m, row_x, row_y, g_stream);
  if (e == hipSuccess && split.n) e = lh::launch_hilo_split(split, g_stream);
  if (e == hipSuccess && !shared_m.empty())
    e = launch_shared_x_groups(shared_m, shared_y, dhl, shared_I, 2 * S, g_stream);
  for (int i = 0; i < count && e == hipSuccess; ++i)
    if (fast[i] && descs[i].x && descs[i].S > 1)
      e = lh::launch_gemv_bf16(mat[i], dhl + hloff[i], descs[i].I, 2 * descs[i].S, dy2 + y2off[i],
                               descs[i].O, 0, g_stream);
  if (e == hipSuccess && !ds.empty()) e = launch_descs(ds, g_stream);
  if (e == hipSuccess && !mxs.empty()) e = launch_mx_descs(mxs, g_stream);
  if (e == hipSuccess && !d5s.empty()) e = launch_dense5(d5s, g_stream);
  if (e == hipSuccess && join.n) e = lh::launch_hilo_join(join, g_stream);
  if (e != hipSuccess) return -1;
  if (g_prof_on) hipEventRecord(g_prof_ev1, g_stream);
  uint64_t t2 = now_ns();
  prof_add(1, t2 - t1);
  e = hipMemcpyAsync(hy, dy, yn * 4, hipMemcpyDeviceToHost, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  if (e != hipSuccess) return -1;
  for (int i = 0; i < count; ++i) {
    const int s = descs[i].x ? descs[i].S : S;
    memcpy(descs[i].y, hy + yoff[i], (size_t)s * descs[i].O * 4);
  }
  prof_add(2, now_ns() - t2);
  prof_kernel_time();
  return 1;
}

void *logan_hip_moe_route_begin(uint64_t model_id, int layer, LoganHipMatmulDesc *descs, int count,
                                const float *x, int D, int M) {
  (void)model_id;
  (void)layer;
  if (!descs || count <= 0 || count > 16 || !x || D <= 0 || M <= 0) return nullptr;
  const int K = count;
  const int expected_I[3] = {D, D, M};
  const int expected_O[3] = {M, M, D};
  for (int i = 0; i < K; ++i)
    for (int r = 0; r < 3; ++r) {
      const LoganHipMatmulDesc &d = descs[i * 3 + r];
      if (!fmt_known(d.fmt, d.gs)) return nullptr;
      if (d.I != expected_I[r] || d.O != expected_O[r]) return nullptr;
    }
  std::lock_guard<std::mutex> lk(g_mtx);
  if (!g_ok) return nullptr;
  uint64_t t0 = now_ns();
  std::vector<LoganHipTensor *> ts((size_t)K * 3);
  for (int i = 0; i < K * 3; ++i) {
    ts[i] = resolve_tensor_locked(&descs[i].tensor, descs[i].weights, descs[i].scales,
                                  descs[i].fmt, descs[i].I, descs[i].O, descs[i].gs);
    if (!ts[i]) return nullptr;
  }
  // fast path: every matrix an MXFP4 one or one the bf16 kernels take (f32
  // x split into bf16 hi/lo in registers, f32 products); h = silu(g) * u
  // between the two stages. MXFP4 matrices need it (no fused-SwiGLU form).
  std::vector<lh::DevMat> mat((size_t)K * 3);
  bool fast = true, any_mx = false;
  for (int i = 0; i < K * 3; ++i) {
    mat[i] = tensor_mat(ts[i]);
    any_mx = any_mx || ts[i]->planes;
    fast = fast && (ts[i]->planes || lh::gemv_bf16_supported(mat[i]));
  }
  fast = fast && M % 4 == 0;  // 16-byte aligned per-expert h rows
  if (any_mx && !fast) return nullptr;
  RoutePending *p = new (std::nothrow) RoutePending();
  if (!p) return nullptr;
  p->bufs = route_bufs_take((size_t)D * 4 + 16, (size_t)2 * K * M * 4 + 16, (size_t)K * D * 4 + 16);
  if (!p->bufs || hipEventCreateWithFlags(&p->ev, hipEventDisableTiming) != hipSuccess) {
    p->ev = nullptr;
    route_release_locked(p);
    return nullptr;
  }
  p->K = K;
  p->D = D;
  float *dx = reinterpret_cast<float *>(p->bufs->x.p);
  float *gu = reinterpret_cast<float *>(p->bufs->gu.p);
  float *out = reinterpret_cast<float *>(p->bufs->out.p);
  uint64_t t1 = now_ns();
  memcpy(p->bufs->hx.p, x, (size_t)D * 4);
  hipError_t e = hipMemcpyAsync(dx, p->bufs->hx.p, (size_t)D * 4, hipMemcpyHostToDevice, g_stream);
  if (g_prof_on && hipEventCreate(&p->pev0) == hipSuccess && hipEventCreate(&p->pev1) == hipSuccess)
    hipEventRecord(p->pev0, g_stream);
  if (fast) {
    // gate/up products (f32 x on the dot2 kernel's f32 form) -> gu [K][M]
    // and gu [K][M] + K M; h = silu(g) * u in place; downs read h -> out[e]
    std::vector<lh::DevMat> gum, dm;
    std::vector<const float *> gux, dxs;
    std::vector<void *> guy, dys;
    std::vector<lh::Mx4Desc> gmx, dmx;
    auto add = [&](int j, const float *xi, float *yi, bool down) {
      if (ts[j]->planes) {
        (down ? dmx : gmx).push_back(mx_desc(ts[j], xi, yi));
        return;
      }
      (down ? dm : gum).push_back(mat[j]);
      (down ? dxs : gux).push_back(xi);
      (down ? dys : guy).push_back(yi);
    };
    for (int i = 0; i < K; ++i) {
      add(i * 3 + 0, dx, gu + (size_t)i * M, false);
      add(i * 3 + 1, dx, gu + (size_t)K * M + (size_t)i * M, false);
      add(i * 3 + 2, gu + (size_t)i * M, out + (size_t)i * D, true);
    }
    prof_add(0, t1 - t0);
    if (e == hipSuccess && !gum.empty()) e = launch_f32x_groups(gum, gux, guy, g_stream);
    if (e == hipSuccess && !gmx.empty()) e = launch_mx_descs(gmx, g_stream);
    if (e == hipSuccess) e = lh::launch_silu_mul(gu, gu + (size_t)K * M, (long long)K * M, false, g_stream);
    if (e == hipSuccess && !dm.empty()) e = launch_f32x_groups(dm, dxs, dys, g_stream);
    if (e == hipSuccess && !dmx.empty()) e = launch_mx_descs(dmx, g_stream);
  } else {
    // gate -> gu[i*M], up -> gu[K*M + i*M]; down(silu(gate)*up) -> out[i*D]
    std::vector<lh::GenDesc> s1, s2;
    for (int i = 0; i < K; ++i) {
      s1.push_back(gen_desc(ts[i * 3 + 0], dx, nullptr, gu + (size_t)i * M, 1, D, M, 0));
      s1.push_back(gen_desc(ts[i * 3 + 1], dx, nullptr, gu + (size_t)K * M + (size_t)i * M, 1, D, M, 0));
      s2.push_back(gen_desc(ts[i * 3 + 2], gu + (size_t)i * M, gu + (size_t)K * M + (size_t)i * M,
                            out + (size_t)i * D, 1, M, D, 1));
    }
    prof_add(0, now_ns() - t0);
    if (e == hipSuccess) e = launch_descs(s1, g_stream);
    if (e == hipSuccess) e = launch_descs(s2, g_stream);
  }
  if (p->pev1) hipEventRecord(p->pev1, g_stream);
  // the expert outputs come back into the handle's pinned buffer in stream
  // order; finish waits for the event and copies them out on the host
  if (e == hipSuccess)
    e = hipMemcpyAsync(p->bufs->hout.p, out, (size_t)K * D * 4, hipMemcpyDeviceToHost, g_stream);
  if (e == hipSuccess) e = hipEventRecord(p->ev, g_stream);
  prof_add(1, now_ns() - t1);
  if (e != hipSuccess) {
    // submitted work may be partially queued: drain it; a decline would hide
    // a real failure, so the handle is still returned and finish reports -1
    hipStreamSynchronize(g_stream);
    p->K = -1;
    return p;
  }
  return p;
}

int logan_hip_moe_route_finish(void *pending, float *out, int count) {
  if (!pending) return 0;
  RoutePending *p = reinterpret_cast<RoutePending *>(pending);
  std::lock_guard<std::mutex> lk(g_mtx);
  int rc = 1;
  const uint64_t t0 = now_ns();
  if (p->K < 0) {
    rc = -1;
  } else if (!out || count <= 0) {
    hipEventSynchronize(p->ev);
    rc = 0;
  } else if (hipEventSynchronize(p->ev) != hipSuccess) {
    rc = -1;
  } else {
    const int K = std::min(count, p->K);
    memcpy(out, p->bufs->hout.p, (size_t)K * p->D * 4);
  }
  prof_add(2, now_ns() - t0);
  float ms = 0.f;
  if (g_prof_on && p->pev1 && hipEventElapsedTime(&ms, p->pev0, p->pev1) == hipSuccess)
    g_prof[3] += (uint64_t)(ms * 1e6);
  route_release_locked(p);
  return rc;
}

void logan_hip_moe_route_discard(void *pending) {
  if (!pending) return;
  RoutePending *p = reinterpret_cast<RoutePending *>(pending);
  std::lock_guard<std::mutex> lk(g_mtx);
  route_release_locked(p);
}

void logan_hip_moe_route_drop_model(uint64_t model_id) {
  (void)model_id;
  std::lock_guard<std::mutex> lk(g_mtx);
  if (!g_ok) return;
  // idle buffer sets only; those of pending handles return on finish/discard
  for (RouteBufs *b : g_route_pool) {
    b->release();
    delete b;
  }
  g_route_pool.clear();
}

int logan_hip_shared_expert(uint64_t model_id, int layer, LoganHipMatmulDesc *descs, int count,
                            const float *x, float *out, int D, int Iinter) {
  (void)model_id;
  (void)layer;
  if (!descs || count != 3 || !x || !out || D <= 0 || Iinter <= 0) return 0;
  void *p = logan_hip_moe_route_begin(0, 0, descs, 1, x, D, Iinter);
  if (!p) return 0;
  return logan_hip_moe_route_finish(p, out, 1);
}

void logan_hip_shared_expert_drop_model(uint64_t model_id) { logan_hip_moe_route_drop_model(model_id); }

// ---- dense Llama decode layer, host pointers (backend_metal.mm:2495-2791) ----
//
// One context per (model, layer): the norm weights' device copies, the
// layer's K/V cache (f32, grown in steps of 256 tokens), staging for x and
// the workspace. A call must come at the position the context has reached
// (pos == tokens so far), as the reference requires (:2643).
namespace {
struct LlamaCtx {
  uint64_t model_id = 0;
  int layer = -1;
  lh::LlamaDims dims{};
  const float *host_in_norm = nullptr, *host_post_norm = nullptr;
  float *in_norm = nullptr, *post_norm = nullptr, *kc = nullptr, *vc = nullptr;
  int tokens = 0, cap = 0;
  DevBuf x, ws;
  void release() {
    hipFree(in_norm);
    hipFree(post_norm);
    hipFree(kc);
    hipFree(vc);
    in_norm = post_norm = kc = vc = nullptr;
    x.release();
    ws.release();
  }
};
std::vector<LlamaCtx *> g_llama;

bool llama_same(const lh::LlamaDims &a, const lh::LlamaDims &b) {
  return a.D == b.D && a.inter == b.inter && a.H == b.H && a.KH == b.KH && a.hd == b.hd &&
         a.theta == b.theta && a.eps == b.eps;
}

bool llama_grow_locked(LlamaCtx *c, int need) {
  if (need <= c->cap) return true;
  const int cap = (need + 255) / 256 * 256;
  const size_t kv = (size_t)c->dims.KH * c->dims.hd;
  float *nk = nullptr, *nv = nullptr;
  if (hipMalloc(&nk, (size_t)cap * kv * 4) != hipSuccess) return false;
  if (hipMalloc(&nv, (size_t)cap * kv * 4) != hipSuccess) {
    hipFree(nk);
    return false;
  }
  if (c->tokens > 0 &&
      (hipMemcpyAsync(nk, c->kc, (size_t)c->tokens * kv * 4, hipMemcpyDeviceToDevice, g_stream) != hipSuccess ||
       hipMemcpyAsync(nv, c->vc, (size_t)c->tokens * kv * 4, hipMemcpyDeviceToDevice, g_stream) != hipSuccess ||
       hipStreamSynchronize(g_stream) != hipSuccess)) {
    hipFree(nk);
    hipFree(nv);
    return false;
  }
  hipFree(c->kc);
  hipFree(c->vc);
  c->kc = nk;
  c->vc = nv;
  c->cap = cap;
  return true;
}

LlamaCtx *llama_ctx_locked(uint64_t model_id, int layer, const float *in_norm, const float *post_norm,
                           const lh::LlamaDims &dims) {
  for (LlamaCtx *c : g_llama) {
    if (c->model_id != model_id || c->layer != layer) continue;
    if (c->host_in_norm != in_norm || c->host_post_norm != post_norm || !llama_same(c->dims, dims))
      return nullptr;
    return c;
  }
  if (!model_id || layer < 0) return nullptr;
  LlamaCtx *c = new (std::nothrow) LlamaCtx();
  if (!c) return nullptr;
  c->model_id = model_id;
  c->layer = layer;
  c->dims = dims;
  c->host_in_norm = in_norm;
  c->host_post_norm = post_norm;
  const size_t nb = (size_t)dims.D * 4;
  if (hipMalloc(&c->in_norm, nb) != hipSuccess || hipMalloc(&c->post_norm, nb) != hipSuccess ||
      hipMemcpy(c->in_norm, in_norm, nb, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(c->post_norm, post_norm, nb, hipMemcpyHostToDevice) != hipSuccess ||
      !c->x.ensure(nb) || !llama_grow_locked(c, 1)) {
    c->release();
    delete c;
    return nullptr;
  }
  g_llama.push_back(c);
  return c;
}
}  // namespace

int logan_hip_host_llama_layer(uint64_t model_id, int layer, LoganHipMatmulDesc *descs, int count,
                               float *x, float *k_out, float *v_out, const float *in_norm,
                               const float *post_norm, int D, int inter, int H, int KH, int hd,
                               int pos, float theta, float eps) {
  if (!descs || count != 7 || !x || !k_out || !v_out || !in_norm || !post_norm || pos < 0) return 0;
  const lh::LlamaDims dims{D, inter, H, KH, hd, theta, eps};
  const int qdim = H * hd, kvdim = KH * hd;
  const int ei[7] = {D, D, D, qdim, D, D, inter};
  const int eo[7] = {qdim, kvdim, kvdim, D, inter, inter, D};
  for (int i = 0; i < 7; ++i)
    if ((descs[i].fmt != 5 && descs[i].fmt != 15) || descs[i].I != ei[i] || descs[i].O != eo[i])
      return 0;
  std::lock_guard<std::mutex> lk(g_mtx);
  if (!g_ok) return 0;
  const uint64_t t0 = now_ns();
  LoganHipTensor *ts[7];
  lh::DenseMat mats[7];
  for (int i = 0; i < 7; ++i) {
    ts[i] = resolve_tensor_locked(&descs[i].tensor, descs[i].weights, descs[i].scales, descs[i].fmt,
                                  descs[i].I, descs[i].O, descs[i].fmt == 15 ? 64 : 0);
    if (!ts[i]) return 0;
    mats[i] = dense_mat(ts[i]);
  }
  if (!lh::llama_supported(dims, mats)) return 0;
  LlamaCtx *c = llama_ctx_locked(model_id, layer, in_norm, post_norm, dims);
  if (!c || c->tokens != pos || !llama_grow_locked(c, pos + 1)) return 0;
  if (!c->ws.ensure(lh::llama_workspace_bytes(dims, pos + 1))) return 0;
  // x in, then x, k and v out, through the pinned staging buffers
  if (!g_hxbuf.ensure((size_t)D * 4) || !g_hybuf.ensure((size_t)(D + 2 * kvdim) * 4)) return 0;
  float *hx = reinterpret_cast<float *>(g_hxbuf.p);
  float *hy = reinterpret_cast<float *>(g_hybuf.p);
  float *dx = reinterpret_cast<float *>(c->x.p);
  const uint64_t t1 = now_ns();
  prof_add(0, t1 - t0);
  memcpy(hx, x, (size_t)D * 4);
  hipError_t e = hipMemcpyAsync(dx, hx, (size_t)D * 4, hipMemcpyHostToDevice, g_stream);
  if (e == hipSuccess && g_prof_on) hipEventRecord(g_prof_ev0, g_stream);
  if (e == hipSuccess)
    e = lh::launch_llama_layer(mats, c->in_norm, c->post_norm, dims, dx, c->kc, c->vc, pos, c->ws.p,
                               g_stream);
  if (e == hipSuccess && g_prof_on) hipEventRecord(g_prof_ev1, g_stream);
  const uint64_t t2 = now_ns();
  prof_add(1, t2 - t1);
  if (e == hipSuccess) e = hipMemcpyAsync(hy, dx, (size_t)D * 4, hipMemcpyDeviceToHost, g_stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(hy + D, c->kc + (size_t)pos * kvdim, (size_t)kvdim * 4, hipMemcpyDeviceToHost,
                       g_stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(hy + D + kvdim, c->vc + (size_t)pos * kvdim, (size_t)kvdim * 4,
                       hipMemcpyDeviceToHost, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  if (e != hipSuccess) {
    hipStreamSynchronize(g_stream);
    return -1;
  }
  memcpy(x, hy, (size_t)D * 4);
  memcpy(k_out, hy + D, (size_t)kvdim * 4);
  memcpy(v_out, hy + D + kvdim, (size_t)kvdim * 4);
  prof_add(2, now_ns() - t2);
  prof_kernel_time();
  c->tokens = pos + 1;
  return 1;
}

void logan_hip_host_llama_drop_model(uint64_t model_id) {
  if (!model_id) return;
  std::lock_guard<std::mutex> lk(g_mtx);
  if (!g_ok) return;
  hipStreamSynchronize(g_stream);
  for (auto it = g_llama.begin(); it != g_llama.end();) {
    if ((*it)->model_id == model_id) {
      (*it)->release();
      delete *it;
      it = g_llama.erase(it);
    } else {
      ++it;
    }
  }
}

void logan_hip_tensor_free(LoganHipTensor *t) {
  if (!t) return;
  std::lock_guard<std::mutex> lk(g_mtx);
  if (g_ok) hipStreamSynchronize(g_stream);  // queued work may still read the tensor
  if (t->w) hipFree(t->w);
  if (t->sc) hipFree(t->sc);
  if (g_tensor_count) g_tensor_count--;
  g_tensor_bytes -= std::min(g_tensor_bytes, t->wbytes + t->abytes);
  delete t;
}

size_t logan_hip_tensor_bytes(const LoganHipTensor *t) { return t ? t->wbytes + t->abytes : 0; }

// Host-pointer element-wise ops (backend_metal.mm:2147-2204): stage the
// operands in HBM, run the kernel, copy the result back, wait.
namespace {
int host_ew(float *dst, size_t n_dst, const float *src, size_t n_src,
            hipError_t (*run)(float *, const float *, hipStream_t, const void *), const void *arg) {
  std::lock_guard<std::mutex> lk(g_mtx);
  if (!g_ok) return 0;
  if (!g_xbuf.ensure(n_dst * 4 + 16) || !g_ybuf.ensure(n_src * 4 + 16)) return 0;
  if (!g_hxbuf.ensure(n_dst * 4 + 16) || !g_hybuf.ensure(n_src * 4 + 16)) return 0;
  float *dd = reinterpret_cast<float *>(g_xbuf.p);
  float *ds = reinterpret_cast<float *>(g_ybuf.p);
  // through the pinned staging buffers: dst in and out of g_hxbuf, src in
  // from g_hybuf (the copies run in stream order)
  float *hd = reinterpret_cast<float *>(g_hxbuf.p);
  float *hs = reinterpret_cast<float *>(g_hybuf.p);
  memcpy(hd, dst, n_dst * 4);
  memcpy(hs, src, n_src * 4);
  hipError_t e = hipMemcpyAsync(dd, hd, n_dst * 4, hipMemcpyHostToDevice, g_stream);
  if (e == hipSuccess) e = hipMemcpyAsync(ds, hs, n_src * 4, hipMemcpyHostToDevice, g_stream);
  if (e == hipSuccess) e = run(dd, ds, g_stream, arg);
  if (e == hipSuccess) e = hipMemcpyAsync(hd, dd, n_dst * 4, hipMemcpyDeviceToHost, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  if (e != hipSuccess) {
    hipStreamSynchronize(g_stream);
    return -1;
  }
  memcpy(dst, hd, n_dst * 4);
  return 1;
}
struct RmsArg {
  int n, nrows;
  float eps;
};
}  // namespace

int logan_hip_host_rmsnorm(float *x, const float *w, int n, int nrows, float eps) {
  if (!x || !w || n <= 0 || nrows <= 0) return 0;
  const RmsArg arg{n, nrows, eps};
  return host_ew(x, (size_t)n * nrows, w, (size_t)n,
                 [](float *d, const float *s, hipStream_t st, const void *a) {
                   const RmsArg &r = *reinterpret_cast<const RmsArg *>(a);
                   return lh::launch_rmsnorm(d, s, r.n, r.nrows, r.eps, st);
                 },
                 &arg);
}

int logan_hip_host_add(float *y, const float *a, int n) {
  if (!y || !a || n <= 0) return 0;
  const long long nn = n;
  return host_ew(y, (size_t)n, a, (size_t)n,
                 [](float *d, const float *s, hipStream_t st, const void *a) {
                   return lh::launch_add(d, s, *reinterpret_cast<const long long *>(a), st);
                 },
                 &nn);
}

int logan_hip_host_silu_mul(float *g, const float *u, int n) {
  if (!g || !u || n <= 0) return 0;
  const long long nn = n;
  return host_ew(g, (size_t)n, u, (size_t)n,
                 [](float *d, const float *s, hipStream_t st, const void *a) {
                   return lh::launch_silu_mul(d, s, *reinterpret_cast<const long long *>(a), false,
                                              st);
                 },
                 &nn);
}

// ---------------------------------------------------------------------------

int logan_hip_affine_gemv(const LoganHipAffine *w, const void *x, int M, int x_stride, void *y,
                          int y_stride, int y_dtype, void *stream) {
  if (!affine_ok(w) || !x || !y || M <= 0 || x_stride < w->I || y_stride < w->O) return 0;
  if (y_dtype != LOGAN_HIP_F32 && y_dtype != LOGAN_HIP_BF16) return 0;
  const lh::DevMat m = devmat(*w);
  if (!lh::gemv_bf16_supported(m)) return 0;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return 0;
  return rc_from(lh::launch_gemv_bf16(m, reinterpret_cast<const uint16_t *>(x), x_stride, M, y,
                                      y_stride, y_dtype == LOGAN_HIP_BF16,
                                      reinterpret_cast<hipStream_t>(stream)));
}

int logan_hip_affine_gemv_multi(const LoganHipAffine *ws, int count, const void *x, int M,
                                int x_stride, void *const *ys, int y_dtype, void *stream) {
  if (!ws || !ys || !x || count <= 0 || count > 8 || M <= 0) return 0;
  if (y_dtype != LOGAN_HIP_F32 && y_dtype != LOGAN_HIP_BF16) return 0;
  lh::DevMat ms[8];
  for (int i = 0; i < count; ++i) {
    if (!affine_ok(&ws[i]) || !ys[i] || x_stride < ws[i].I) return 0;
    ms[i] = devmat(ws[i]);
    if (!lh::gemv_bf16_supported(ms[i])) return 0;
    if (ms[i].I != ms[0].I || ms[i].bits != ms[0].bits || ms[i].gs != ms[0].gs ||
        ms[i].fp16 != ms[0].fp16)
      return 0;
  }
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return 0;
  return rc_from(lh::launch_gemv_bf16_multi(ms, ys, count, reinterpret_cast<const uint16_t *>(x),
                                            x_stride, M, y_dtype == LOGAN_HIP_BF16,
                                            reinterpret_cast<hipStream_t>(stream)));
}

int logan_hip_affine_qmm(const LoganHipAffine *w, const void *x, int M, int x_stride, void *y,
                         int y_stride, int y_dtype, void *stream) {
  if (!affine_ok(w) || !x || !y || M <= 0 || x_stride < w->I || y_stride < w->O) return 0;
  if (y_dtype != LOGAN_HIP_F32 && y_dtype != LOGAN_HIP_BF16) return 0;
  const lh::DevMat m = devmat(*w);
  if (!lh::affine_qmm_supported(m)) return 0;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return 0;
  return rc_from(lh::launch_affine_qmm(m, reinterpret_cast<const uint16_t *>(x), x_stride, M, y,
                                       y_stride, y_dtype == LOGAN_HIP_BF16,
                                       reinterpret_cast<hipStream_t>(stream)));
}

int logan_hip_affine_gemv_swiglu(const LoganHipAffine *gate, const LoganHipAffine *up,
                                 const void *x, int M, int x_stride, void *h, int h_stride,
                                 int h_dtype, void *stream) {
  if (!affine_ok(gate) || !affine_ok(up) || !x || !h || M <= 0) return 0;
  if (x_stride < gate->I || h_stride < gate->O) return 0;
  if (h_dtype != LOGAN_HIP_F32 && h_dtype != LOGAN_HIP_BF16) return 0;
  const lh::DevMat g = devmat(*gate), u = devmat(*up);
  if (!lh::gemv_bf16_supported(g) || !lh::gemv_bf16_supported(u)) return 0;
  if (g.I != u.I || g.O != u.O || g.bits != u.bits || g.gs != u.gs || g.fp16 != u.fp16) return 0;
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return 0;
  return rc_from(lh::launch_gemv_swiglu(g, u, reinterpret_cast<const uint16_t *>(x), x_stride, M, h,
                                        h_stride, h_dtype == LOGAN_HIP_BF16,
                                        reinterpret_cast<hipStream_t>(stream)));
}

int logan_hip_affine_qmm_multi(const LoganHipAffine *ws, int count, const void *x, int M,
                               int x_stride, void *const *ys, int y_dtype, void *stream) {
  if (!ws || !ys || !x || count <= 0 || count > 8 || M <= 0) return 0;
  if (y_dtype != LOGAN_HIP_F32 && y_dtype != LOGAN_HIP_BF16) return 0;
  lh::DevMat ms[8];
  for (int i = 0; i < count; ++i) {
    if (!affine_ok(&ws[i]) || !ys[i] || x_stride < ws[i].I) return 0;
    ms[i] = devmat(ws[i]);
    if (!lh::affine_qmm_supported(ms[i])) return 0;
    if (ms[i].I != ms[0].I || ms[i].bits != ms[0].bits || ms[i].gs != ms[0].gs ||
        ms[i].fp16 != ms[0].fp16)
      return 0;
  }
  if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_stride & 7) != 0) return 0;
  return rc_from(lh::launch_affine_qmm_multi(ms, count, reinterpret_cast<const uint16_t *>(x),
                                             x_stride, M, ys, y_dtype == LOGAN_HIP_BF16,
                                             reinterpret_cast<hipStream_t>(stream)));
}

int logan_hip_silu_mul(void *g, const void *u, long long n, int dtype, void *stream) {
  if (!g || !u || n <= 0) return 0;
  if (dtype != LOGAN_HIP_F32 && dtype != LOGAN_HIP_BF16) return 0;
  if (((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(u)) & 15) != 0) return 0;
  return rc_from(lh::launch_silu_mul(g, u, n, dtype == LOGAN_HIP_BF16,
                                     reinterpret_cast<hipStream_t>(stream)));
}

int logan_hip_affine_gemv_f32(const LoganHipAffine *w, const float *x, int M, int x_stride,
                              float *y, int y_stride, void *stream) {
  if (!affine_ok(w) || !x || !y || M <= 0 || x_stride < w->I || y_stride < w->O) return 0;
  LoganHipTensor t;
  t.w = const_cast<uint8_t *>(reinterpret_cast<const uint8_t *>(w->weights));
  t.sc = const_cast<uint16_t *>(reinterpret_cast<const uint16_t *>(w->scales));
  t.bi = const_cast<uint16_t *>(reinterpret_cast<const uint16_t *>(w->biases));
  t.I = w->I;
  t.O = w->O;
  t.gs = w->group_size;
  t.bits = w->bits;
  t.fp16 = w->aux_fp16;
  std::vector<lh::GenDesc> ds{gen_desc(&t, x, nullptr, y, M, x_stride, y_stride, 0)};
  return rc_from(launch_descs(ds, reinterpret_cast<hipStream_t>(stream)));
}

int logan_hip_affine_dequant(const LoganHipAffine *w, int row0, int nrows, float *out,
                             void *stream) {
  if (!affine_ok(w) || !out || row0 < 0 || nrows < 0 || row0 + nrows > w->O) return 0;
  return rc_from(lh::launch_dequant(devmat(*w), row0, nrows, out,
                                    reinterpret_cast<hipStream_t>(stream)));
}

int logan_hip_route_topk(const void *logits, int logits_dtype, int B, int E, int k, int32_t *idx,
                         float *w, void *stream) {
  if (!logits || !idx || !w || B <= 0 || E <= 0 || E > 1024 || k <= 0 || k > 32 || k > E) return 0;
  if (logits_dtype != LOGAN_HIP_F32 && logits_dtype != LOGAN_HIP_BF16) return 0;
  return rc_from(lh::launch_route_topk(logits, logits_dtype == LOGAN_HIP_F32, B, E, k, idx, w,
                                       reinterpret_cast<hipStream_t>(stream)));
}

static bool fill_moe_args(const LoganHipMoeBlock *blk, lh::MoeArgs &a) {
  if (!blk) return false;
  a = lh::MoeArgs{};
  a.gate = devbank(blk->gate);
  a.up = devbank(blk->up);
  a.down = devbank(blk->down);
  if (blk->shared_gate.weights) {
    a.sgate = devbank(blk->shared_gate);
    a.sup = devbank(blk->shared_up);
    a.sdown = devbank(blk->shared_down);
    a.sinter = blk->shared_gate.O;
  }
  a.se_gate_vec = reinterpret_cast<const uint16_t *>(blk->shared_gate_vec);
  a.D = blk->gate.I;
  a.inter = blk->gate.O;
  a.E = blk->gate.E;
  a.k = blk->top_k;
  return a.D > 0 && a.inter > 0 && a.E > 0 && a.k > 0;
}

size_t logan_hip_moe_workspace_bytes(const LoganHipMoeBlock *blk, int B) {
  lh::MoeArgs a;
  if (!fill_moe_args(blk, a) || B <= 0) return 0;
  return lh::moe_workspace_bytes(B, a.D, a.inter, a.sgate.m.w ? a.sinter : 0, a.E, a.k);
}

// the MoE launch on the caller's workspace, or on the library-owned one
static int run_moe_block(lh::MoeArgs &a, void *workspace, size_t workspace_bytes, void *stream) {
  const size_t need =
      lh::moe_workspace_bytes(a.B, a.D, a.inter, a.sgate.m.w ? a.sinter : 0, a.E, a.k);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (workspace) {
    if (workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255) != 0) return 0;
    a.ws = workspace;
    a.ws_bytes = workspace_bytes;
    return lh::launch_moe_block(a, st);
  }
  std::lock_guard<std::mutex> lk(g_mtx);
  if (g_ws.n < need) {
    // the old buffer may still be read by queued work on any stream
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    if (!g_ws.ensure(need)) return 0;
  }
  a.ws = g_ws.p;
  a.ws_bytes = g_ws.n;
  return lh::launch_moe_block(a, st);
}

int logan_hip_moe_block(const LoganHipMoeBlock *blk, const void *x, const void *logits,
                        int logits_dtype, int B, void *out, int out_dtype, int32_t *idx_out,
                        float *w_out, void *workspace, size_t workspace_bytes, void *stream) {
  lh::MoeArgs a;
  if (!fill_moe_args(blk, a) || !x || !logits || !out || B <= 0) return 0;
  if (logits_dtype != LOGAN_HIP_F32 && logits_dtype != LOGAN_HIP_BF16) return 0;
  if (out_dtype != LOGAN_HIP_F32 && out_dtype != LOGAN_HIP_BF16) return 0;
  a.x = reinterpret_cast<const uint16_t *>(x);
  a.logits = logits;
  a.logits_f32 = logits_dtype == LOGAN_HIP_F32;
  a.B = B;
  a.out = out;
  a.out_f32 = out_dtype == LOGAN_HIP_F32;
  a.idx_out = idx_out;
  a.w_out = w_out;
  return run_moe_block(a, workspace, workspace_bytes, stream);
}

int logan_hip_moe_block_cached(const LoganHipMoeBlock *blk, const LoganHipExpertCache *c,
                               const int32_t *experts, const int32_t *blocks, int k, const void *x,
                               const void *logits, int logits_dtype, void *out, int out_dtype,
                               int32_t *idx_out, float *w_out, void *workspace,
                               size_t workspace_bytes, void *stream) {
  lh::MoeArgs a;
  if (!fill_moe_args(blk, a) || !c || !experts || !blocks || !x || !logits || !out) return 0;
  if (k != a.k || k < 1 || k > lh::kMoeMapMax) return 0;
  if (logits_dtype != LOGAN_HIP_F32 && logits_dtype != LOGAN_HIP_BF16) return 0;
  if (out_dtype != LOGAN_HIP_F32 && out_dtype != LOGAN_HIP_BF16) return 0;
  // the routed banks: views of the cache's blocks, in the caller's geometry
  const lh::DevBank want[3] = {a.gate, a.up, a.down};
  int nblocks = 0;
  if (!lh::expert_cache_banks(c, &a.gate, &a.up, &a.down, &nblocks)) return 0;
  const lh::DevBank *got[3] = {&a.gate, &a.up, &a.down};
  for (int m = 0; m < 3; ++m) {
    const lh::DevMat &w = want[m].m, &g = got[m]->m;
    if (w.O != g.O || w.I != g.I || w.bits != g.bits || w.gs != g.gs || w.fp16 != g.fp16) return 0;
  }
  a.nmap = k;
  for (int r = 0; r < k; ++r) {
    if (experts[r] < 0 || experts[r] >= a.E || blocks[r] < 0 || blocks[r] >= nblocks) return 0;
    a.map_e[r] = experts[r];
    a.map_b[r] = blocks[r];
  }
  a.x = reinterpret_cast<const uint16_t *>(x);
  a.logits = logits;
  a.logits_f32 = logits_dtype == LOGAN_HIP_F32;
  a.B = 1;
  a.out = out;
  a.out_f32 = out_dtype == LOGAN_HIP_F32;
  a.idx_out = idx_out;
  a.w_out = w_out;
  return run_moe_block(a, workspace, workspace_bytes, stream);
}

int logan_hip_moe_block_routed(const LoganHipMoeBlock *blk, const LoganHipAffine *router,
                               const void *x, int B, float *logits, void *out, int out_dtype,
                               int32_t *idx_out, float *w_out, void *workspace,
                               size_t workspace_bytes, void *stream) {
  lh::MoeArgs a;
  if (!fill_moe_args(blk, a) || !affine_ok(router) || !x || !logits || B <= 0) return 0;
  if (router->O != a.E || router->I != a.D) return 0;
  const lh::DevMat rm = devmat(*router);
  if (!lh::gemv_bf16_supported(rm) || (reinterpret_cast<uintptr_t>(x) & 15) != 0 || (a.D & 7) != 0)
    return 0;
  if (B > lh::kMaxBatch) return 0;
  // the router product, then the block on its f32 logits (stream order)
  const hipError_t e = lh::launch_gemv_bf16(rm, reinterpret_cast<const uint16_t *>(x), a.D, B,
                                            logits, a.E, 0, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return -1;
  return logan_hip_moe_block(blk, x, logits, LOGAN_HIP_F32, B, out, out_dtype, idx_out, w_out,
                             workspace, workspace_bytes, stream);
}

int logan_hip_moe_block_static(const LoganHipMoeBlock *blk, const void *x, const void *logits,
                               int logits_dtype, int B, void *out, int out_dtype, int32_t *idx_out,
                               float *w_out, void *stream) {
  lh::MoeArgs a;
  if (!fill_moe_args(blk, a) || !x || !logits || !out || B <= 0) return 0;
  if (logits_dtype != LOGAN_HIP_F32 && logits_dtype != LOGAN_HIP_BF16) return 0;
  if (out_dtype != LOGAN_HIP_F32 && out_dtype != LOGAN_HIP_BF16) return 0;
  const size_t need =
      lh::moe_workspace_bytes(B, a.D, a.inter, a.sgate.m.w ? a.sinter : 0, a.E, a.k);
  if (need > kStaticScratchBytes) {
    std::fprintf(stderr,
                 "[logan-hip] moe_block_static: B=%d needs a %zu-byte workspace; the static "
                 "scratch holds %zu bytes (use logan_hip_moe_block with a workspace)\n",
                 B, need, kStaticScratchBytes);
    return 0;
  }
  void *ws = scratch_on_current_device();
  if (!ws) return 0;
  a.x = reinterpret_cast<const uint16_t *>(x);
  a.logits = logits;
  a.logits_f32 = logits_dtype == LOGAN_HIP_F32;
  a.B = B;
  a.out = out;
  a.out_f32 = out_dtype == LOGAN_HIP_F32;
  a.idx_out = idx_out;
  a.w_out = w_out;
  a.ws = ws;
  a.ws_bytes = kStaticScratchBytes;
  return lh::launch_moe_block(a, reinterpret_cast<hipStream_t>(stream));
}

int logan_hip_mxfp4_gemv(const LoganHipMxfp4 *ws, int count, const void *const *xs, int x_dtype,
                         void *const *ys, int y_dtype, void *stream) {
  if (!ws || !xs || !ys || count <= 0 || count > lh::kMx4MaxDescs) return 0;
  if ((x_dtype != LOGAN_HIP_F32 && x_dtype != LOGAN_HIP_BF16) ||
      (y_dtype != LOGAN_HIP_F32 && y_dtype != LOGAN_HIP_BF16))
    return 0;
  lh::Mx4Batch b{};
  b.n = count;
  b.y_bf16 = y_dtype == LOGAN_HIP_BF16;
  for (int i = 0; i < count; ++i) {
    const LoganHipMxfp4 &m = ws[i];
    if (!m.codes || !m.scales || m.planes < 1 || m.planes > 3) return 0;
    if (!lh::mxfp4_supported(m.O, m.I, m.codes)) return 0;
    if (!xs[i] || !ys[i] || (reinterpret_cast<uintptr_t>(xs[i]) & 15) != 0) return 0;
    lh::Mx4Desc &d = b.d[i];
    d.w = reinterpret_cast<const uint8_t *>(m.codes);
    d.sc = reinterpret_cast<const uint8_t *>(m.scales);
    d.x = xs[i];
    d.y = ys[i];
    d.wplane = (long long)m.O * (m.I / 2);
    d.splane = (long long)m.O * (m.I / 32);
    d.O = m.O;
    d.I = m.I;
    d.planes = m.planes;
  }
  return rc_from(lh::launch_mxfp4_gemv(b, x_dtype == LOGAN_HIP_F32, reinterpret_cast<hipStream_t>(stream)));
}

int logan_hip_mxfp4_dequant(const LoganHipMxfp4 *w, int row0, int nrows, float *out, void *stream) {
  if (!w || !w->codes || !w->scales || !out || !lh::mxfp4_supported(w->O, w->I, w->codes)) return 0;
  if (row0 < 0 || nrows <= 0 || row0 + nrows > w->O) return 0;
  return rc_from(lh::launch_mxfp4_dequant(reinterpret_cast<const uint8_t *>(w->codes),
                                          reinterpret_cast<const uint8_t *>(w->scales), w->O, w->I,
                                          row0, nrows, out, reinterpret_cast<hipStream_t>(stream)));
}

static bool dense_from(const LoganHipDense &a, lh::DenseMat &m) {
  if (!a.weights || (a.fmt != 5 && a.fmt != 15)) return false;
  if (a.fmt == 15 && (!a.scales || !a.biases)) return false;
  m.w = a.weights;
  m.sc = a.fmt == 15 ? reinterpret_cast<const uint16_t *>(a.scales) : nullptr;
  m.bi = a.fmt == 15 ? reinterpret_cast<const uint16_t *>(a.biases) : nullptr;
  m.fmt = a.fmt;
  m.O = a.O;
  m.I = a.I;
  return true;
}

static bool llama_from(const LoganHipLlamaLayer *L, lh::DenseMat mats[7], lh::LlamaDims &dims) {
  if (!L) return false;
  const LoganHipDense *ds[7] = {&L->q, &L->k, &L->v, &L->o, &L->gate, &L->up, &L->down};
  for (int i = 0; i < 7; ++i)
    if (!dense_from(*ds[i], mats[i])) return false;
  dims = lh::LlamaDims{L->D, L->inter, L->heads, L->kv_heads, L->head_dim, L->theta, L->eps};
  return lh::llama_supported(dims, mats);
}

size_t logan_hip_llama_workspace_bytes(const LoganHipLlamaLayer *L, int pos) {
  lh::DenseMat mats[7];
  lh::LlamaDims dims;
  if (pos < 0 || !llama_from(L, mats, dims)) return 0;
  return lh::llama_workspace_bytes(dims, pos + 1);
}

int logan_hip_llama_layer(const LoganHipLlamaLayer *L, float *x, int pos, void *ws, size_t ws_bytes,
                          void *stream) {
  lh::DenseMat mats[7];
  lh::LlamaDims dims;
  if (!x || !ws || pos < 0 || !llama_from(L, mats, dims)) return 0;
  if (!L->in_norm || !L->post_norm || !L->k_cache || !L->v_cache || pos >= L->cache_tokens) return 0;
  // x and the norm weights are read as float4, the workspace's activation
  // pairs as 16-byte vectors
  const auto a16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!a16(x) || !a16(L->in_norm) || !a16(L->post_norm) || !a16(ws)) return 0;
  if (ws_bytes < lh::llama_workspace_bytes(dims, pos + 1)) return 0;
  return rc_from(lh::launch_llama_layer(mats, L->in_norm, L->post_norm, dims, x, L->k_cache,
                                        L->v_cache, pos, ws, reinterpret_cast<hipStream_t>(stream)));
}

void logan_hip_set_moe_fused(int on) { lh::set_moe_fused_enabled(on ? 1 : 0); }

uint32_t logan_hip_moe_sync_errors(void) { return lh::moe_fused_sync_errors() | lh::moe_map_errors(); }

void logan_hip_set_moe_mfma_min_batch(int b) { lh::set_moe_mfma_min_batch(b); }

const char *logan_hip_version(void) { return "logan-hip 0.1.0 (gfx950)"; }

}  // extern "C"
