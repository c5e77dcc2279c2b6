// Safetensors checkpoint index (header parse, shard map, name aliases) and
// the geometry rules of the MLX quantized loaders, shared by stfile.hip (host
// parsing and validation) and loader.hip (upload into HBM).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace lh {
namespace st {

struct Tensor {
  int shard = 0;
  std::vector<uint64_t> shape;
  std::string dtype;
  uint64_t offset = 0;  // absolute byte offset in the shard file
  uint64_t len = 0;     // payload bytes
};

struct File {
  std::vector<int> fds;  // one read-only descriptor per shard
  std::vector<std::string> paths;
  std::map<std::string, Tensor> tensors;
  ~File();
};

// Bytes per element of a dtype the reader accepts, 0 for any other.
int element_bytes(const std::string &dtype);

// Parse + validate; nullptr with *err set on failure.
File *open_file(const std::string &path, std::string *err);
File *open_dir(const std::string &dir, std::string *err);

// Rust `{:?}` spelling of a shape, e.g. "[512, 512, 256]".
std::string shape_str(const std::vector<uint64_t> &s);

// One contiguous byte range of a tensor payload to move.
struct Region {
  int shard = -1;
  uint64_t file_off = 0, len = 0;
};

// What a quantized load resolves to, before any byte moves.
struct QuantPlan {
  int kind = 0;  // 1 affine, 2 MXFP4
  int E = 0;     // experts covered (1 for a dense matrix)
  int O = 0, I = 0, bits = 0, group_size = 0, aux_fp16 = 0;
  Region w, sc, bi;  // bi.len == 0 for MXFP4
};

// load_mlx_quantized_wt's checks (logan-qwen4/src/lib.rs:11818-11937).
bool plan_dense(const File &f, const std::string &name, long long o, long long i, QuantPlan *p,
                std::string *err);
// load_mlx_quantized_expert_wt's checks (lib.rs:11939-12078) for experts
// [e0, e0 + ne) of a stacked bank of `experts`.
bool plan_experts(const File &f, const std::string &name, long long e0, long long ne,
                  long long experts, long long o, long long i, QuantPlan *p, std::string *err);

}  // namespace st

// The loader's pinned staging ring (loader.hip), shared by the expert cache's
// fills: kSlots pinned host slots filled by pread()s and drained by async
// copies on the loader's own stream, one event per slot.
namespace ld {
constexpr size_t kSlotBytes = 32u << 20;  // one staging slot
constexpr int kSlots = 4;                 // reads run up to 3 slots ahead of the DMA
struct Stager {
  bool ready = false;
  int dev = -1;
  hipStream_t st = nullptr;
  void *buf[kSlots] = {};
  hipEvent_t ev[kSlots] = {};
  bool pending[kSlots] = {};
  int readers = 1;
};
// held for a whole load (the ring is shared)
std::mutex &load_mutex();
Stager &stager();
// the ring on the current device (built on first use); false with *err set
bool stager_ready(std::string *err);
// [off, off + n) of fd into dst with up to `readers` threads
bool parallel_read(int fd, uint64_t off, char *dst, size_t n, int readers);
}  // namespace ld

// Thread-local message of the last failed loader/stfile call.
void set_last_error(const std::string &m);

}  // namespace lh
