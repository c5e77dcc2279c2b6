// Internal (C++) launch interface shared by the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace lh {

// ---- scratch slots shared by launches on any stream of one device ----
// Split products write partial sums into a module-scope slot with one kernel
// and add them up with a second on the same stream. SlotRing hands the slots
// out round-robin; a lease holds its slot's host lock from take() until
// done(), makes its stream wait (on the device) for the event the slot's
// previous user recorded after its last kernel on the slot, and done()
// records the lease's own event there. Launches on different streams
// therefore never overlap on a slot, whatever their number. Inside a stream
// capture neither the wait nor the record is made: a captured graph's slot
// is fixed at capture time and its replays are ordered by their own stream
// only (a replay that overlaps another call on another stream may share the
// slot).
class SlotRing {
 public:
  static constexpr int kMaxSlots = 8, kMaxDevices = 16;
  explicit SlotRing(int nslots) : n_(nslots) {}
  class Lease {
   public:
    Lease() = default;
    Lease(const Lease &) = delete;
    Lease &operator=(const Lease &) = delete;
    ~Lease() { (void)release(true); }
    int slot() const { return slot_; }
    // after the last kernel that touches the slot: record, unlock (the
    // destructor does the same for a lease left held on an error path)
    hipError_t done() { return release(true); }

   private:
    friend class SlotRing;
    hipError_t release(bool record);
    SlotRing *ring_ = nullptr;
    int dev_ = 0, slot_ = -1;
    bool capturing_ = false;
    hipStream_t st_ = nullptr;
  };
  // takes the next slot for stream st (blocks while another host thread
  // holds it); on failure lease.slot() < 0
  hipError_t take(hipStream_t st, Lease &lease);

 private:
  struct Dev;
  Dev *dev(int d);
  int n_;
  Dev *devs_[kMaxDevices] = {};
};

// One MLX-affine matrix resident in device memory.
struct DevMat {
  const uint8_t *w;     // rows * row_bytes, 16-byte aligned
  const uint16_t *sc;   // rows * ng
  const uint16_t *bi;   // rows * ng
  int I, O, gs, bits, fp16;
  long long row_bytes;  // I*bits/8
  int ng;               // I/gs
};

// ---- fast dense GEMV: bf16 activations [M, I], y [M, O] (bf16 or f32) ----
// Returns hipSuccess, or hipErrorInvalidValue when the geometry has no fast
// kernel (caller then uses the generic kernel).
hipError_t launch_gemv_bf16(const DevMat &m, const uint16_t *x, int x_stride, int M,
                            void *y, int y_stride, int y_bf16, hipStream_t st);
bool gemv_bf16_supported(const DevMat &m);
// up to 8 matrices sharing x (same I, bits, group size, aux type); ys[i] is
// [M][O_i]
hipError_t launch_gemv_bf16_multi(const DevMat *ms, void *const *ys, int n, const uint16_t *x,
                                  int x_stride, int M, int y_bf16, hipStream_t st);
// same, each matrix with its own activation rows xs[i] [M][x_stride]
hipError_t launch_gemv_bf16_multi_x(const DevMat *ms, const uint16_t *const *xs, void *const *ys,
                                    int n, int x_stride, int M, int y_bf16, hipStream_t st);
constexpr int kGemvMultiMax = 8;
// one f32 activation row per matrix (xs[i], or the shared x when xs is
// null) on the dot2 kernel, split in registers into bf16 (hi, lo) operands
// (|x - hi - lo| <= 2^-18 |x|); ys[i] [O_i] f32 (y_bf16 0) or bf16
hipError_t launch_gemv_f32x_multi(const DevMat *ms, const float *x, const float *const *xs,
                                  void *const *ys, int n, int y_bf16, hipStream_t st);

// ---- f32 activations on the bf16 kernels: each f32 row x becomes the bf16
// row pair (hi, lo) = (bf16(x), bf16(x - hi)), the products run on 2 rows
// per activation row with f32 outputs, and each output row is y = y_hi + y_lo
// (|x - hi - lo| <= 2^-18 |x|)
struct HiloJob {
  const float *src;  // [rows][n] f32
  void *dst;         // split: uint16_t [2 rows][n]; join: float [rows][n]
  int rows, n;
};
constexpr int kHiloMaxJobs = 32;
struct HiloBatch {
  HiloJob j[kHiloMaxJobs];
  int n;
};
// split: dst = bf16 (hi, lo) row pairs of src; join: dst = src[2r] + src[2r+1]
hipError_t launch_hilo_split(const HiloBatch &b, hipStream_t st);
hipError_t launch_hilo_join(const HiloBatch &b, hipStream_t st);


// ---- prefill / large-batch product on MFMA: bf16-rounded dequantised
// weights (the reference QMM semantics), x bf16 [M, I], y [M, O] ----
hipError_t launch_affine_qmm(const DevMat &m, const uint16_t *x, int x_stride, int M, void *y,
                             int y_stride, int y_bf16, hipStream_t st);
bool affine_qmm_supported(const DevMat &m);
// up to 8 matrices sharing x (same I, bits, group size, aux type) in one
// grid where the 256-row tiles apply, else one launch per matrix; ys[i] is
// [M][O_i]
hipError_t launch_affine_qmm_multi(const DevMat *ms, int n, const uint16_t *x, int x_stride, int M,
                                   void *const *ys, int y_bf16, hipStream_t st);
bool affine_skinny_supported(const DevMat &m);
hipError_t launch_affine_skinny(const DevMat &m, const uint16_t *x, int x_stride, int M, void *y,
                                int y_stride, int y_bf16, hipStream_t st);
// K split across blocks (gemv_splitk.hip): I % 512 == 0, groups of 64k,
// 3 <= M <= 32; partial sums in module-scope scratch slots
bool affine_splitk_multi_supported(const DevMat *ms, int n, int M);
// swiglu_stride > 0: n == 2 (gate, up) and the reduce writes
// ys[0][M][swiglu_stride] = silu(gate) * up instead of the two products
hipError_t launch_affine_splitk_multi(const DevMat *ms, int n, const uint16_t *x, int x_stride, int M,
                                      void *const *ys, int y_bf16, hipStream_t st,
                                      int swiglu_stride = 0);
// h[M][h_stride] = silu(gate . x) * (up . x) in one product (gate and up of
// the same geometry): the dot2 kernel with gate/up row pairs for token pairs,
// the K-split pair with a SwiGLU reduce for 3..32 tokens
hipError_t launch_gemv_swiglu(const DevMat &g, const DevMat &u, const uint16_t *x, int x_stride, int M,
                              void *h, int h_stride, int h_bf16, hipStream_t st);
// gate/up + SwiGLU for 3..16 tokens over the full K (no partial sums), for
// pairs with at least 12288 rows
bool swiglu_fullk_supported(const DevMat &g, const DevMat &u, int M);
hipError_t launch_swiglu_fullk(const DevMat &g, const DevMat &u, const uint16_t *x, int x_stride, int M,
                               void *h, int h_stride, int h_bf16, hipStream_t st);
// K split across the waves of a block (3..8 tokens, at least 4096 rows,
// I / 512 with a divisor in [4, 8]): y written by the one launch
bool affine_kwave_supported(const DevMat &m, int M);
hipError_t launch_affine_kwave(const DevMat &m, const uint16_t *x, int x_stride, int M, void *y,
                               int y_stride, int y_bf16, hipStream_t st);
bool affine_splitk_supported(const DevMat &m, int M);
hipError_t launch_affine_splitk(const DevMat &m, const uint16_t *x, int x_stride, int M, void *y,
                                int y_stride, int y_bf16, hipStream_t st);
hipError_t launch_silu_mul(void *g, const void *u, long long n, bool bf16, hipStream_t st);
// in-place RMSNorm of nrows rows of n floats with weight w[n]; y += a
hipError_t launch_rmsnorm(float *x, const float *w, int n, int nrows, float eps, hipStream_t st);
hipError_t launch_add(float *y, const float *a, long long n, hipStream_t st);

// ---- generic GEMV over up to 16 descriptors, f32 activations ----
struct GenDesc {
  const uint8_t *w;
  const uint16_t *sc;
  const uint16_t *bi;
  const float *x;       // [S, x_stride]; with xmode 1 this is the gate input
  const float *up;      // xmode 1: x_eff = silu(x) * up
  float *y;             // [S, y_stride]
  long long row_bytes;
  int I, O, gs, bits, fp16, S, x_stride, y_stride, xmode;
};
constexpr int kMaxDescs = 16;
struct GenBatch {
  GenDesc d[kMaxDescs];
  int block_start[kMaxDescs + 1];
  int n;
};
constexpr int kGenRowsPerBlock = 4;
hipError_t launch_gemv_generic(const GenBatch &b, hipStream_t st);

// ---- MXFP4 (fmt 7; 2 / 3 residual planes = fmt 9 / 10) GEMV ----
struct Mx4Desc {
  const uint8_t *w;            // [planes][O][I/2], 16-byte aligned
  const uint8_t *sc;           // [planes][O][I/32] E8M0 bytes
  const void *x;               // [I] f32 or bf16, 16-byte aligned
  void *y;                     // [O] f32 or bf16
  long long wplane, splane;    // bytes between planes
  int O, I, planes;
};
constexpr int kMx4MaxDescs = 16;
struct Mx4Batch {
  Mx4Desc d[kMx4MaxDescs];
  int block_start[kMx4MaxDescs + 1];
  int n;
  int y_bf16;
};
bool mxfp4_supported(int O, int I, const void *w);
hipError_t launch_mxfp4_gemv(Mx4Batch &b, bool x_f32, hipStream_t st);
hipError_t launch_mxfp4_dequant(const uint8_t *w, const uint8_t *sc, int O, int I, int row0,
                                int nrows, float *out, hipStream_t st);

// ---- dense bf16-valued GEMV (fmt 5 raw bf16, fmt 15 affine-8 g64 with
// every weight rounded to bf16) and the Llama decode layer ----
struct DenseDesc {
  const void *w;                  // fmt 5: bf16 [O][I]; fmt 15: u8 [O][I]; 16-byte aligned
  const uint16_t *sc, *bi;        // fmt 15: bf16 [O][I/64] each
  const uint16_t *xhl;            // [2][I]: bf16 hi then lo halves of the f32 activation
  float *y;                       // [O]
  const float *res;               // y = res + W x when set (may alias y)
  int O, I;
  // SwiGLU pair when w2 is set: w is gate, w2 up (same format and shape);
  // instead of y, hhl[2][O] receives the hi/lo halves of silu(W x) * (W2 x)
  const void *w2;
  const uint16_t *sc2, *bi2;
  uint16_t *hhl;
};
constexpr int kDenseMaxDescs = 8;
struct DenseBatch {
  DenseDesc d[kDenseMaxDescs];
  int block_start[kDenseMaxDescs + 1];
  int n;
};
bool dense_supported(int fmt, int O, int I, const void *w);
hipError_t launch_dense_gemv(DenseBatch &b, int fmt, hipStream_t st);

struct DenseMat {
  const void *w;
  const uint16_t *sc, *bi;
  int fmt, O, I;
};
struct LlamaDims {
  int D, inter, H, KH, hd;
  float theta, eps;
};
// mats: q, k, v, o, gate, up, down
bool llama_supported(const LlamaDims &m, const DenseMat mats[7]);
size_t llama_workspace_bytes(const LlamaDims &m, int T);
hipError_t launch_llama_layer(const DenseMat mats[7], const float *in_norm, const float *post_norm,
                              const LlamaDims &m, float *x, float *kc, float *vc, int pos,
                              void *ws, hipStream_t st);

// ---- exact dequantisation of rows [row0, row0+nrows) to f32 ----
hipError_t launch_dequant(const DevMat &m, int row0, int nrows, float *out, hipStream_t st);

// ---- router: softmax top-k on logits [B, E] (bf16 or f32) ----
hipError_t launch_route_topk(const void *logits, int logits_f32, int B, int E, int k,
                             int32_t *idx, float *w, hipStream_t st);

// ---- routed-MoE block, device-native ----
struct DevBank {
  DevMat m;               // one expert's geometry; w/sc/bi point at expert 0
  long long w_stride;     // bytes between experts
  long long p_stride;     // u16 elements between experts' params
  int E;
};
struct MoeArgs {
  DevBank gate, up, down;          // routed
  DevBank sgate, sup, sdown;       // shared (E = 1); sgate.m.w == nullptr: none
  const uint16_t *se_gate_vec;     // bf16 [D] or nullptr (gate = 1)
  const uint16_t *x;               // bf16 [B, D]
  const void *logits;              // [B, E]
  int logits_f32;
  int B, D, inter, sinter, E, k;
  void *out;                       // [B, D], bf16 or f32 (out_f32)
  int out_f32;
  int32_t *idx_out;                // optional [B, k]
  float *w_out;                    // optional [B, k]
  void *ws;                        // workspace
  size_t ws_bytes;
  // Routed experts held in an expert cache's arena (expert_cache.hip): the
  // routed banks are views of its blocks (block stride as w_stride /
  // p_stride) and expert map_e[i] sits in block map_b[i]. nmap == 0: the
  // banks hold every expert, indexed by expert id.
  int nmap;
  int32_t map_e[32], map_b[32];
};
constexpr int kMoeMapMax = 32;
// The bank index of routed expert e: its block when a map is set (an expert
// missing from the map reads block map_b[0], so the launch stays in bounds,
// and sets *miss), else e itself.
// CONST_IDX: the map is read at constant indices only (an unrolled scan of
// all kMoeMapMax entries). In the per-token kernels, which also select bank
// references inside the by-value MoeArgs at run time, a scan at run-time
// indices makes the compiler copy the whole MoeArgs to scratch in every
// thread (4x slower); in the fused B = 1 kernel the run-time scan stays in
// registers and the unrolled one costs 11 % of its time. The kernels' scratch
// use is checked by a CPU test.
template <bool CONST_IDX>
__device__ __forceinline__ int moe_bank_index(const MoeArgs &a, int e, bool &miss) {
  if (a.nmap == 0) return e;
  int b = -1;
  if constexpr (CONST_IDX) {
#pragma unroll
    for (int i = 0; i < kMoeMapMax; ++i) b = i < a.nmap && a.map_e[i] == e ? a.map_b[i] : b;
  } else {
    for (int i = 0; i < a.nmap; ++i) b = a.map_e[i] == e ? a.map_b[i] : b;
  }
  miss = b < 0;
  return b < 0 ? a.map_b[0] : b;
}
size_t moe_workspace_bytes(int B, int D, int inter, int sinter, int E, int k);
// single-launch B = 1 path (moe_fused.hip): 1 launched, 0 not applicable
int launch_moe_fused_b1(const MoeArgs &a, hipStream_t st);
size_t moe_fused_workspace_bytes(int slots, int inter, int sinter);
// sticky error bits of the fused path (bit 0: a wait timed out; bits 1-2:
// arrival counters not at rest; bit 3: a routed expert missing from the
// expert-cache map)
uint32_t moe_fused_sync_errors();
// bit 3 of the same word for the per-token path (moe.hip)
uint32_t moe_map_errors();
// 0 disables the fused B = 1 path (LOGAN_HIP_MOE_FUSED=0); default on
void set_moe_fused_enabled(int on);
// token-batch path on MFMA (moe_mfma.hip): 4/5/6/8-bit codes, groups of 64k,
// D % 128 == 0, inter and sinter <= 512 and % 128 == 0; 1 launched, 0 not
// applicable, -1 launch failure
constexpr int kMaxBatch = 4096;         // tokens per moe_block call
constexpr int kMaxBatchSlots = 65536;   // tokens * top_k
// smallest batch on the MFMA path by code width (measured crossovers with the
// per-token path, config-3 shapes: 4-bit between 48 and 64 tokens, 5/6-bit
// below 24)
constexpr int kMfmaMinBatchDefault = 24;
constexpr int kMfmaMinBatch4Bit = 56;
bool moe_mfma_supported(const MoeArgs &a);
int launch_moe_mfma(const MoeArgs &a, hipStream_t st);
size_t moe_mfma_workspace_bytes(int B, int D, int inter, int sinter, int E, int k);
// smallest batch that takes the MFMA path for every code width
// (LOGAN_HIP_MOE_MFMA_MIN_B); b <= 0 restores the per-width defaults
void set_moe_mfma_min_batch(int b);
// 1 ok, 0 unsupported geometry (nothing launched), -1 launch failure
int launch_moe_block(const MoeArgs &a, hipStream_t st);
}  // namespace lh

struct LoganHipExpertCache;
namespace lh {
// the routed banks as views of an expert cache's blocks (expert_cache.hip);
// *nblocks = blocks in the cache's allocation
bool expert_cache_banks(const LoganHipExpertCache *c, DevBank *g, DevBank *u, DevBank *d, int *nblocks);

}  // namespace lh
