// MLX quantized weights from a safetensors checkpoint into HBM.
//
// The reference reads each matrix (or one expert's slice of a stacked
// switch_mlp bank) into host memory (load_mlx_quantized_wt /
// load_mlx_quantized_expert_wt, logan-qwen4/src/lib.rs:11818-12078) and the
// Metal backend wraps those bytes later. Here the validated byte ranges move
// straight into one device allocation per load: the file is read with
// parallel pread()s into a ring of pinned staging slots, and each filled slot
// is copied to HBM with an async DMA on the loader's own stream while the
// next slot is read. The device image is the file's bytes unchanged (the MLX
// layouts are what every kernel here reads), so a bank of all E experts lands
// as the [E][O][I*bits/8] / [E][O][I/gs] stacks the MoE block takes.
#include <hip/hip_runtime.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <thread>
#include <vector>

#include "../../include/logan_hip.h"
#include "stfile.hpp"

namespace lh {
namespace st {
bool plan_lookup(const LoganHipStFile *h, const File **f);
bool pread_all(int fd, uint64_t off, void *dst, size_t n);
}  // namespace st
}  // namespace lh

namespace lh {
namespace ld {

constexpr int kMaxReaders = 8;  // pread threads per slot

std::mutex g_load_mtx;  // one load at a time per process (the staging ring is shared)
Stager g_stage;

std::mutex &load_mutex() { return g_load_mtx; }
Stager &stager() { return g_stage; }

bool stager_ready(std::string *err) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    *err = "no HIP device";
    return false;
  }
  if (g_stage.ready && g_stage.dev == dev) return true;
  if (g_stage.ready) {  // another device is current now: rebuild on it
    for (int i = 0; i < kSlots; ++i) {
      hipEventDestroy(g_stage.ev[i]);
      hipHostFree(g_stage.buf[i]);
    }
    hipStreamDestroy(g_stage.st);
    g_stage = Stager();
  }
  if (hipStreamCreateWithFlags(&g_stage.st, hipStreamNonBlocking) != hipSuccess) {
    *err = "hipStreamCreate failed";
    return false;
  }
  for (int i = 0; i < kSlots; ++i) {
    if (hipHostMalloc(&g_stage.buf[i], kSlotBytes, hipHostMallocDefault) != hipSuccess ||
        hipEventCreateWithFlags(&g_stage.ev[i], hipEventDisableTiming) != hipSuccess) {
      *err = "pinned staging allocation failed";
      for (int j = 0; j <= i; ++j) {
        if (g_stage.buf[j]) hipHostFree(g_stage.buf[j]);
        if (g_stage.ev[j]) hipEventDestroy(g_stage.ev[j]);
      }
      hipStreamDestroy(g_stage.st);
      g_stage = Stager();
      return false;
    }
  }
  unsigned hw = std::thread::hardware_concurrency();
  g_stage.readers = (int)std::max(1u, std::min<unsigned>(kMaxReaders, hw ? hw / 2 : 1));
  g_stage.dev = dev;
  g_stage.ready = true;
  return true;
}

// read [off, off + n) of fd into dst with up to `readers` threads
bool parallel_read(int fd, uint64_t off, char *dst, size_t n, int readers) {
  const size_t kMinPiece = 4u << 20;
  int t = (int)std::min<size_t>((size_t)readers, std::max<size_t>(1, n / kMinPiece));
  if (t <= 1) return lh::st::pread_all(fd, off, dst, n);
  std::vector<std::thread> th;
  std::vector<char> ok((size_t)t, 0);
  const size_t piece = (n + (size_t)t - 1) / (size_t)t;
  for (int i = 0; i < t; ++i) {
    size_t a = (size_t)i * piece, b = std::min(n, a + piece);
    th.emplace_back([&, i, a, b] { ok[(size_t)i] = lh::st::pread_all(fd, off + a, dst + a, b - a); });
  }
  bool all = true;
  for (int i = 0; i < t; ++i) {
    th[(size_t)i].join();
    all = all && ok[(size_t)i];
  }
  return all;
}

// Move one file range into device memory through the staging ring. Slots
// are reused only after their previous DMA has completed.
bool stage_region(const lh::st::File &f, const lh::st::Region &r, char *ddst, int *slot,
                  std::string *err) {
  uint64_t done = 0;
  while (done < r.len) {
    const int s = *slot;
    *slot = (s + 1) % kSlots;
    if (g_stage.pending[s] && hipEventSynchronize(g_stage.ev[s]) != hipSuccess) {
      *err = "staging copy failed";
      return false;
    }
    g_stage.pending[s] = false;
    const size_t n = (size_t)std::min<uint64_t>(kSlotBytes, r.len - done);
    if (!parallel_read(f.fds[(size_t)r.shard], r.file_off + done, (char *)g_stage.buf[s], n,
                       g_stage.readers)) {
      *err = f.paths[(size_t)r.shard] + ": read failed";
      return false;
    }
    if (hipMemcpyAsync(ddst + done, g_stage.buf[s], n, hipMemcpyHostToDevice, g_stage.st) !=
            hipSuccess ||
        hipEventRecord(g_stage.ev[s], g_stage.st) != hipSuccess) {
      *err = "hipMemcpyAsync to device failed";
      return false;
    }
    g_stage.pending[s] = true;
    done += n;
  }
  return true;
}

}  // namespace ld
}  // namespace lh

namespace {

using namespace lh::ld;

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

int load_plan(const lh::st::File &f, const lh::st::QuantPlan &p, LoganHipQuantWt *out) {
  std::lock_guard<std::mutex> lk(g_load_mtx);
  std::string err;
  if (!stager_ready(&err)) {
    lh::set_last_error(err);
    return -1;
  }
  const size_t wb = align256(p.w.len), sb = align256(p.sc.len), bb = align256(p.bi.len);
  char *base = nullptr;
  if (hipMalloc((void **)&base, wb + sb + bb) != hipSuccess) {
    lh::set_last_error("hipMalloc of " + std::to_string(wb + sb + bb) + " bytes failed");
    return -1;
  }
  int slot = 0;
  bool ok = stage_region(f, p.w, base, &slot, &err) && stage_region(f, p.sc, base + wb, &slot, &err) &&
            (p.bi.len == 0 || stage_region(f, p.bi, base + wb + sb, &slot, &err));
  // every slot's DMA must finish before the ring (or the result) is used again
  if (hipStreamSynchronize(g_stage.st) != hipSuccess && ok) {
    ok = false;
    err = "staging copy failed";
  }
  for (int i = 0; i < kSlots; ++i) g_stage.pending[i] = false;
  if (!ok) {
    hipFree(base);
    lh::set_last_error(err);
    return -1;
  }
  memset(out, 0, sizeof(*out));
  out->kind = p.kind;
  out->E = p.E;
  out->O = p.O;
  out->I = p.I;
  out->bits = p.bits;
  out->group_size = p.group_size;
  out->aux_fp16 = p.aux_fp16;
  out->weights = base;
  out->scales = base + wb;
  out->biases = p.bi.len ? base + wb + sb : nullptr;
  out->weight_bytes = p.w.len;
  out->scale_bytes = p.sc.len;
  out->bias_bytes = p.bi.len;
  out->owner = base;
  return 1;
}

}  // namespace

extern "C" {

int logan_hip_load_mlx_quantized(const LoganHipStFile *st, const char *name, int O, int I,
                                 LoganHipQuantWt *out) {
  const lh::st::File *f = nullptr;
  if (!lh::st::plan_lookup(st, &f) || !name || !out) {
    lh::set_last_error("null argument");
    return 0;
  }
  lh::st::QuantPlan p;
  std::string err;
  if (!lh::st::plan_dense(*f, name, O, I, &p, &err)) {
    lh::set_last_error(err);
    return 0;
  }
  return load_plan(*f, p, out);
}

int logan_hip_load_mlx_quantized_experts(const LoganHipStFile *st, const char *name, int e0,
                                         int count, int experts, int O, int I,
                                         LoganHipQuantWt *out) {
  const lh::st::File *f = nullptr;
  if (!lh::st::plan_lookup(st, &f) || !name || !out) {
    lh::set_last_error("null argument");
    return 0;
  }
  lh::st::QuantPlan p;
  std::string err;
  if (!lh::st::plan_experts(*f, name, e0, count, experts, O, I, &p, &err)) {
    lh::set_last_error(err);
    return 0;
  }
  return load_plan(*f, p, out);
}

void logan_hip_quant_free(LoganHipQuantWt *w) {
  if (!w) return;
  if (w->owner) hipFree(w->owner);
  memset(w, 0, sizeof(*w));
}

}  // extern "C"
