// Route-driven expert cache in HBM: the reference's EXP-069 RouteCache and
// EXP-067 RouteArena (logan-qwen4/src/lib.rs:12110-12300, builders
// :12959-13140, fetch :12697-12903) for banks that are not kept resident.
//
// One device allocation holds fixed-size expert blocks. Each block carries
// one routed expert's gate, up and down matrices (packed weights, scales,
// biases) in the order of the reference's io_plan (:13550-13590), each part
// 256-byte aligned here so the kernels' 128-bit loads stay aligned. Blocks
// [L * blocks_per_layer, (L + 1) * blocks_per_layer) are layer L's retention
// cache (tags, a replacement cursor, hit/miss/eviction counts); the last
// 2 * topk blocks are the route arena, one set of topk per layer parity,
// where route ranks the cache does not retain are streamed. A fetch reserves
// the route's first min(blocks_per_layer, k) ranks in the cache (each block
// the route claims is pinned, so a later rank's miss never evicts it),
// streams the misses and the tail into their blocks through the loader's
// pinned staging ring on the loader's stream, after the caller stream's
// earlier work (which may still read those blocks), and makes the caller
// stream wait for the copies. The MoE block then reads the experts through
// the (expert, block) map of the route (logan_hip_moe_block_cached): the
// routed banks become views of the allocation with the block stride.
#include <hip/hip_runtime.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/logan_hip.h"
#include "lh_internal.hpp"
#include "stfile.hpp"

namespace lh {
namespace st {
bool plan_lookup(const LoganHipStFile *h, const File **f);
bool pread_all(int fd, uint64_t off, void *dst, size_t n);
}  // namespace st
}  // namespace lh

namespace {

inline size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

const char *const kRole[3] = {"gate_proj", "up_proj", "down_proj"};

// one layer's three stacked banks, resolved once: expert e's part j of
// matrix m is (shard, off[m][j] + e * len[m][j], len[m][j])
struct LayerPlan {
  bool ok = false;
  int shard[3][3] = {};
  uint64_t off[3][3] = {}, len[3][3] = {};
};

}  // namespace

struct LoganHipExpertCache {
  int dev = 0;
  const lh::st::File *f = nullptr;  // borrowed: the StFile outlives the cache
  int layers = 0, experts = 0, D = 0, H = 0, blocks = 0, topk = 0;
  int bits = 0, gs[3] = {}, fp16 = 0;
  uint64_t plen[3][3] = {};   // bytes of part j of matrix m for one expert
  size_t poff[3][3] = {};     // its offset in a block
  size_t stride = 0;          // bytes per block
  char *base = nullptr;       // HBM
  size_t bytes = 0;
  std::vector<LayerPlan> plans;
  // RouteCache state (lib.rs:12145-12168): tags[L][b] = expert or -1
  std::vector<std::vector<int32_t>> tags;
  std::vector<int> next;
  uint64_t generation = 0, hits = 0, misses = 0, evictions = 0, streamed = 0, loaded = 0;
  hipEvent_t ev_before = nullptr, ev_done = nullptr;
  std::mutex mu;

  int total_blocks() const { return layers * blocks + 2 * topk; }
  int arena_block(int layer, int rank) const { return layers * blocks + (layer % 2) * topk + rank; }
};

namespace {

// The three bank names of a layer (io_plan's prefix, lib.rs:13557).
std::string bank_name(int layer, int m) {
  return "model.layers." + std::to_string(layer) + ".mlp.switch_mlp." + kRole[m] + ".weight";
}

// the layer's banks through the loader's checks (load_mlx_quantized_expert_wt,
// lib.rs:11939-12078), and their agreement with the cache's layout
// (RouteArena::layout_matches, :12266-12275)
bool layer_plan(LoganHipExpertCache *c, int layer, std::string *err) {
  LayerPlan &lp = c->plans[(size_t)layer];
  if (lp.ok) return true;
  for (int m = 0; m < 3; ++m) {
    const int O = m == 2 ? c->D : c->H, I = m == 2 ? c->H : c->D;
    lh::st::QuantPlan p;
    if (!lh::st::plan_experts(*c->f, bank_name(layer, m), 0, 1, c->experts, O, I, &p, err))
      return false;
    if (p.kind != LOGAN_HIP_WT_AFFINE) {
      *err = bank_name(layer, m) + ": the expert cache serves MLX affine banks only";
      return false;
    }
    if (p.bits != c->bits || p.group_size != c->gs[m] || p.aux_fp16 != c->fp16 ||
        p.w.len != c->plen[m][0] || p.sc.len != c->plen[m][1] || p.bi.len != c->plen[m][2]) {
      *err = bank_name(layer, m) + ": expert layout differs from the cache's";
      return false;
    }
    const lh::st::Region r[3] = {p.w, p.sc, p.bi};
    for (int j = 0; j < 3; ++j) {
      lp.shard[m][j] = r[j].shard;
      lp.off[m][j] = r[j].file_off;
      lp.len[m][j] = r[j].len;
    }
  }
  lp.ok = true;
  return true;
}

struct Job {
  int layer, expert, block;
};

// read one expert's nine parts into its block image at dst (host)
bool read_job(const LoganHipExpertCache *c, const Job &j, char *dst) {
  const LayerPlan &lp = c->plans[(size_t)j.layer];
  for (int m = 0; m < 3; ++m)
    for (int p = 0; p < 3; ++p) {
      const uint64_t n = lp.len[m][p];
      const uint64_t off = lp.off[m][p] + (uint64_t)j.expert * n;
      if (!lh::st::pread_all(c->f->fds[(size_t)lp.shard[m][p]], off, dst + c->poff[m][p], n))
        return false;
    }
  return true;
}

// Stream the jobs' block images into HBM through the staging ring, after
// the work already queued on `st`; `st` then waits for the copies. Caller
// holds c->mu.
int run_jobs(LoganHipExpertCache *c, const std::vector<Job> &jobs, hipStream_t st, std::string *err) {
  if (jobs.empty()) return 1;
  std::lock_guard<std::mutex> lk(lh::ld::load_mutex());
  if (!lh::ld::stager_ready(err)) return -1;
  lh::ld::Stager &g = lh::ld::stager();
  // the blocks may still be read by kernels queued on st
  if (hipEventRecord(c->ev_before, st) != hipSuccess ||
      hipStreamWaitEvent(g.st, c->ev_before, 0) != hipSuccess) {
    *err = "expert cache: stream ordering failed";
    return -1;
  }
  const size_t per_slot = lh::ld::kSlotBytes / c->stride;
  int slot = 0;
  for (size_t j0 = 0; j0 < jobs.size(); j0 += per_slot) {
    const size_t n = std::min(per_slot, jobs.size() - j0);
    if (g.pending[slot] && hipEventSynchronize(g.ev[slot]) != hipSuccess) {
      *err = "expert cache: staging copy failed";
      return -1;
    }
    g.pending[slot] = false;
    char *buf = reinterpret_cast<char *>(g.buf[slot]);
    // one reader thread per expert image, up to the ring's reader count; each
    // image's copy is queued as soon as it is read, so reads and copies overlap
    const int t = (int)std::min<size_t>(n, (size_t)std::max(1, g.readers));
    std::vector<char> ok(n, 0);
    auto work = [&](int w) {
      for (size_t i = (size_t)w; i < n; i += (size_t)t) {
        char *src = buf + i * c->stride;
        if (!read_job(c, jobs[j0 + i], src)) continue;
        char *dst = c->base + (size_t)jobs[j0 + i].block * c->stride;
        ok[i] = hipMemcpyAsync(dst, src, c->stride, hipMemcpyHostToDevice, g.st) == hipSuccess ? 1 : 2;
      }
    };
    if (t == 1) {
      work(0);
    } else {
      std::vector<std::thread> th;
      for (int w = 0; w < t; ++w) th.emplace_back(work, w);
      for (auto &x : th) x.join();
    }
    // the slot's event after every copy queued from it, even on failure
    const hipError_t re = hipEventRecord(g.ev[slot], g.st);
    g.pending[slot] = re == hipSuccess;
    for (size_t i = 0; i < n; ++i)
      if (ok[i] != 1) {
        *err = ok[i] == 0 ? "expert cache: read of layer " + std::to_string(jobs[j0 + i].layer) +
                                " expert " + std::to_string(jobs[j0 + i].expert) + " failed"
                          : std::string("expert cache: hipMemcpyAsync failed");
        return -1;
      }
    if (re != hipSuccess) {
      *err = "expert cache: event record failed";
      return -1;
    }
    slot = (slot + 1) % lh::ld::kSlots;
  }
  if (hipEventRecord(c->ev_done, g.st) != hipSuccess || hipStreamWaitEvent(st, c->ev_done, 0) != hipSuccess) {
    *err = "expert cache: stream ordering failed";
    return -1;
  }
  c->loaded += (uint64_t)jobs.size() * c->stride;
  return 1;
}

// layer count as try_build_route_cache derives it (lib.rs:12965-12975): one
// more than the largest N of a `language_model.model.layers.N.` name (the
// `model.layers.N.` spelling counts too)
int count_layers(const lh::st::File &f) {
  int n = 0;
  for (const auto &kv : f.tensors) {
    for (const char *pre : {"language_model.model.layers.", "model.layers."}) {
      const size_t pl = strlen(pre);
      if (kv.first.compare(0, pl, pre) != 0) continue;
      const size_t dot = kv.first.find('.', pl);
      if (dot == std::string::npos || dot == pl) continue;
      const std::string num = kv.first.substr(pl, dot - pl);
      if (num.find_first_not_of("0123456789") != std::string::npos || num.size() > 6) continue;
      n = std::max(n, std::stoi(num) + 1);
    }
  }
  return n;
}

}  // namespace

namespace lh {

// the routed banks as views of the cache's blocks (for the MoE entry)
bool expert_cache_banks(const LoganHipExpertCache *c, DevBank *g, DevBank *u, DevBank *d, int *nblocks) {
  if (!c || !c->base) return false;
  DevBank *b[3] = {g, u, d};
  for (int m = 0; m < 3; ++m) {
    DevMat &dm = b[m]->m;
    dm.O = m == 2 ? c->D : c->H;
    dm.I = m == 2 ? c->H : c->D;
    dm.bits = c->bits;
    dm.gs = c->gs[m];
    dm.fp16 = c->fp16;
    dm.row_bytes = (long long)dm.I * dm.bits / 8;
    dm.ng = dm.I / dm.gs;
    dm.w = reinterpret_cast<const uint8_t *>(c->base + c->poff[m][0]);
    dm.sc = reinterpret_cast<const uint16_t *>(c->base + c->poff[m][1]);
    dm.bi = reinterpret_cast<const uint16_t *>(c->base + c->poff[m][2]);
    b[m]->w_stride = (long long)c->stride;
    b[m]->p_stride = (long long)(c->stride / 2);
    b[m]->E = c->total_blocks();
  }
  *nblocks = c->total_blocks();
  return true;
}

}  // namespace lh

extern "C" {

LoganHipExpertCache *logan_hip_expert_cache_create(const LoganHipStFile *st, int layers, int experts,
                                                   int d_model, int d_hidden, int blocks_per_layer,
                                                   int topk) {
  const lh::st::File *f = nullptr;
  if (!lh::st::plan_lookup(st, &f) || !f) {
    lh::set_last_error("null argument");
    return nullptr;
  }
  if (experts < 1 || d_model < 1 || d_hidden < 1 || blocks_per_layer < 0 || topk < 1 ||
      topk > lh::kMoeMapMax || layers < 0) {
    lh::set_last_error("expert cache: invalid geometry");
    return nullptr;
  }
  if (layers == 0) layers = count_layers(*f);
  if (layers == 0) {
    lh::set_last_error("could not determine layer count from the tensor table");
    return nullptr;
  }
  auto *c = new LoganHipExpertCache();
  c->f = f;
  c->layers = layers;
  c->experts = experts;
  c->D = d_model;
  c->H = d_hidden;
  c->blocks = blocks_per_layer;
  c->topk = topk;
  std::string err;
  // the block layout from layer 0's banks (lib.rs:12979: io_plan(0, 0, ...))
  size_t cur = 0;
  for (int m = 0; m < 3; ++m) {
    const int O = m == 2 ? d_model : d_hidden, I = m == 2 ? d_hidden : d_model;
    lh::st::QuantPlan p;
    if (!lh::st::plan_experts(*f, bank_name(0, m), 0, 1, experts, O, I, &p, &err) ||
        p.kind != LOGAN_HIP_WT_AFFINE) {
      if (err.empty()) err = bank_name(0, m) + ": the expert cache serves MLX affine banks only";
      lh::set_last_error(err);
      delete c;
      return nullptr;
    }
    if (m == 0) {
      c->bits = p.bits;
      c->fp16 = p.aux_fp16;
    } else if (p.bits != c->bits || p.aux_fp16 != c->fp16) {
      lh::set_last_error(bank_name(0, m) + ": bit width or sidecar type differs from gate_proj");
      delete c;
      return nullptr;
    }
    c->gs[m] = p.group_size;
    const uint64_t len[3] = {p.w.len, p.sc.len, p.bi.len};
    for (int j = 0; j < 3; ++j) {
      c->plen[m][j] = len[j];
      c->poff[m][j] = cur;
      cur += al256(len[j]);
    }
  }
  c->stride = cur;
  if (c->stride > lh::ld::kSlotBytes) {
    lh::set_last_error("expert cache: an expert block exceeds a staging slot");
    delete c;
    return nullptr;
  }
  c->plans.resize((size_t)layers);
  c->tags.assign((size_t)layers, std::vector<int32_t>((size_t)blocks_per_layer, -1));
  c->next.assign((size_t)layers, 0);
  c->bytes = (size_t)c->total_blocks() * c->stride;
  if (hipGetDevice(&c->dev) != hipSuccess || hipMalloc((void **)&c->base, c->bytes) != hipSuccess ||
      hipEventCreateWithFlags(&c->ev_before, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&c->ev_done, hipEventDisableTiming) != hipSuccess) {
    lh::set_last_error("expert cache: device allocation of " + std::to_string(c->bytes) +
                       " bytes failed");
    logan_hip_expert_cache_destroy(c);
    return nullptr;
  }
  return c;
}

void logan_hip_expert_cache_destroy(LoganHipExpertCache *c) {
  if (!c) return;
  if (c->base) {
    // queued kernels and copies may still use the blocks
    (void)hipDeviceSynchronize();
    (void)hipFree(c->base);
  }
  if (c->ev_before) (void)hipEventDestroy(c->ev_before);
  if (c->ev_done) (void)hipEventDestroy(c->ev_done);
  delete c;
}

int logan_hip_expert_cache_fetch(LoganHipExpertCache *c, int layer, const int32_t *experts, int k,
                                 int32_t *blocks_out, void *stream) {
  if (!c || !experts || !blocks_out || k < 1 || k > c->topk || layer < 0 || layer >= c->layers) {
    lh::set_last_error("expert cache: invalid fetch");
    return 0;
  }
  for (int r = 0; r < k; ++r)
    if (experts[r] < 0 || experts[r] >= c->experts) {
      lh::set_last_error("expert cache: expert id " + std::to_string(experts[r]) + " out of range");
      return 0;
    }
  std::lock_guard<std::mutex> lk(c->mu);
  std::string err;
  if (!layer_plan(c, layer, &err)) {  // declined: layout mismatch or a bad bank
    lh::set_last_error(err);
    return 0;
  }
  // the cache's share: ranks 0 .. retain-1 (cache_fetch_route, :12720-12790)
  const int cap = c->blocks, retain = std::min(cap, k);
  std::vector<int32_t> &tags = c->tags[(size_t)layer];
  std::vector<char> pinned((size_t)std::max(cap, 1), 0);
  std::vector<Job> jobs;
  std::vector<int> missed;  // cache blocks filled by this fetch
  for (int r = 0; r < retain; ++r) {
    // RouteCache::reserve (:12190-12228)
    int b = -1;
    for (int i = 0; i < cap; ++i)
      if (tags[(size_t)i] == experts[r]) {
        b = i;
        break;
      }
    if (b >= 0) {
      ++c->hits;
    } else {
      const int start = c->next[(size_t)layer] % cap;
      for (int off = 0; off < cap; ++off) {
        const int cc = (start + off) % cap;
        if (!pinned[(size_t)cc]) {
          b = cc;
          break;
        }
      }
      if (b < 0) {  // cannot happen with retain <= cap
        lh::set_last_error("expert cache: no unpinned block");
        return 0;
      }
      if (tags[(size_t)b] >= 0) ++c->evictions;
      tags[(size_t)b] = experts[r];
      c->next[(size_t)layer] = (b + 1) % cap;
      ++c->generation;
      ++c->misses;
      jobs.push_back(Job{layer, experts[r], layer * cap + b});
      missed.push_back(b);
    }
    pinned[(size_t)b] = 1;
    blocks_out[r] = layer * cap + b;
  }
  // the rest streams through this layer parity's arena (arena_submit_range,
  // :13257-13303: block parity * topk + rank)
  for (int r = retain; r < k; ++r) {
    const int b = c->arena_block(layer, r);
    jobs.push_back(Job{layer, experts[r], b});
    blocks_out[r] = b;
    ++c->streamed;
  }
  const int rc = run_jobs(c, jobs, reinterpret_cast<hipStream_t>(stream), &err);
  if (rc != 1) {
    // blocks whose load may not have happened must not hit later
    for (int b : missed) tags[(size_t)b] = -1;
    lh::set_last_error(err);
  }
  return rc;
}

void logan_hip_expert_cache_stats(const LoganHipExpertCache *c, LoganHipExpertCacheStats *out) {
  if (!out) return;
  memset(out, 0, sizeof(*out));
  if (!c) return;
  std::lock_guard<std::mutex> lk(const_cast<LoganHipExpertCache *>(c)->mu);
  out->hits = c->hits;
  out->misses = c->misses;
  out->evictions = c->evictions;
  out->streamed = c->streamed;
  out->bytes_loaded = c->loaded;
  out->generation = c->generation;
  out->block_bytes = c->stride;
  out->device_bytes = c->bytes;
  out->layers = c->layers;
  out->blocks_per_layer = c->blocks;
  out->topk = c->topk;
}

int logan_hip_expert_cache_tags(const LoganHipExpertCache *c, int layer, int32_t *tags_out) {
  if (!c || !tags_out || layer < 0 || layer >= c->layers) return 0;
  std::lock_guard<std::mutex> lk(const_cast<LoganHipExpertCache *>(c)->mu);
  for (int b = 0; b < c->blocks; ++b) tags_out[b] = c->tags[(size_t)layer][(size_t)b];
  return 1;
}

}  // extern "C"
