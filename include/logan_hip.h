/*
 * logan-hip: MI355X (gfx950) backend for Logan's quantized decode hot path —
 * the MLX-affine 4/5/6/8-bit dequant-GEMV and the routed-expert MoE block.
 *
 * C ABI. Two layers:
 *
 *  1. Host-pointer drop-in for the subset of logan-metal's C ABI that the
 *     Qwen/Llama/Spark runtimes use on this path
 *     (logan-metal/metal/backend_metal.h). Same argument meaning, same return
 *     convention: 1 = success, 0 = declined before anything was submitted
 *     (caller keeps its CPU path, no state changed), -1 = failure after
 *     submission. Activations and outputs are host f32 arrays; packed weights
 *     and their [scales][biases] sidecar are host byte arrays uploaded to HBM
 *     once on first use and cached behind an opaque tensor handle that the
 *     caller keeps and frees (backend_metal.h:59-66, :180).
 *     The library also exports logan-metal's own C names for every function
 *     its Rust FFI blocks declare (include/logan_metal_ffi.h): those of this
 *     layer forward here, the rest are advisory or decline.
 *
 *  2. Device-native entry points (`logan_hip_affine_*`, `logan_hip_route_topk`,
 *     `logan_hip_moe_block*`): every pointer is device memory already resident
 *     in HBM, activations/outputs bf16, work enqueued on the caller's HIP
 *     stream (`stream` is a hipStream_t; NULL = the null stream). These have no
 *     direct logan-metal counterpart: they are the HBM-resident form of the
 *     same operations (cited per function) and what the benchmarks time.
 *
 * Formats (fmt codes of backend_metal.mm:206-213, logan-metal/src/lib.rs:860-880):
 *   15      affine-8, group 64, bf16 sidecar (Spark/MLX raw bytes)
 *   16..19  affine 4/5/6/8-bit, bf16 sidecar;  20 = 4-bit (Q4 FMA variant, same math)
 *   21..24  affine 4/5/6/8-bit, fp16 sidecar
 * Packed weights: O rows of I*bits/8 bytes, one LSB-first little-endian u32
 * bitstream per row (logan-qwen4/src/lib.rs:3688-3701). Sidecar: O*(I/gs) u16
 * scales followed by O*(I/gs) u16 biases (backend_metal.mm:218-220).
 * Dequantised weight: code*scale + bias (logan-qwen4/src/lib.rs:3703-3727).
 *
 * Threading: every entry point of layer 1 serialises on one process-wide
 * mutex (as backend_metal.mm:1678). Each pending route-island handle owns its
 * device buffers until finish/discard, so other calls (the shared expert,
 * GEMVs, further begins) may run between a begin and its finish.
 */
#ifndef LOGAN_HIP_H
#define LOGAN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Layer 1: host-pointer drop-in                                             */
/* ------------------------------------------------------------------------ */

typedef struct LoganHipTensor LoganHipTensor;

/* Replaces coli_metal_init (backend_metal.h:22; backend_metal.mm:1934-2045).
 * 1 when a gfx950 device is usable, else 0. Idempotent. */
int logan_hip_init(void);
/* Replaces coli_metal_available (backend_metal.h:35). */
int logan_hip_available(void);
/* Replaces coli_metal_shutdown (backend_metal.h:34). Frees staging buffers;
 * tensor handles stay valid until freed. */
void logan_hip_shutdown(void);
/* Replaces coli_metal_stats (backend_metal.h:37): live tensor count/bytes. */
void logan_hip_stats(size_t *tensor_count, size_t *tensor_bytes);
/* Replaces coli_metal_mem_info (backend_metal.h:38). 1 ok, 0 unavailable. */
int logan_hip_mem_info(size_t *used_bytes, size_t *total_bytes);

/* Replace coli_metal_profile_set_on/reset/get (backend_metal.h:42-45).
 * encode = host time building launches, submit = enqueue time, wait = host
 * blocking time, kernel = device time between events around each call. */
void logan_hip_profile_set_on(int on);
void logan_hip_profile_reset(void);
void logan_hip_profile_get(uint64_t *encode_ns, uint64_t *submit_ns, uint64_t *wait_ns,
                           uint64_t *kernel_ns);

/* Replaces coli_metal_matmul (backend_metal.h:63-66) for the affine formats.
 * y[S,O] = x[S,I] . W^T with W the dequantised affine matrix. `scales` is the
 * [scales][biases] sidecar. gs is ignored for fmt 15 (fixed 64). Other fmt
 * codes decline with 0. The first call uploads W and the sidecar to HBM and
 * stores the handle in *tensor; later calls with the same handle reuse it
 * (weights assumed stable, backend_metal.h:59-60). A handle whose geometry
 * differs from the call declines. */
int logan_hip_matmul(LoganHipTensor **tensor, float *y, const float *x, const void *weights,
                     const void *scales, int fmt, int S, int I, int O, int gs);

/* Same layout as ColiMetalMatmulDesc (backend_metal.h:68-88). */
typedef struct LoganHipMatmulDesc {
  LoganHipTensor *tensor;
  float *y;
  const void *weights;
  const float *scales; /* [scales][biases] u16 sidecar, typed as in the reference */
  int fmt;
  int I;
  int O;
  int gs;
  const float *x; /* NULL: use the function-level x */
  int S;
} LoganHipMatmulDesc;

/* Replaces coli_metal_matmul_multi (backend_metal.h:100-101): up to 16
 * independent GEMVs in one submission, one wait. Descriptors with x == NULL
 * use the shared x/S. Updates descs[n].tensor. */
int logan_hip_matmul_multi(const float *x, int S, LoganHipMatmulDesc *descs, int count);

/* Replace coli_metal_moe_route_begin/finish/discard/drop_model
 * (backend_metal.h:163-168; backend_metal.mm:3749-3911). `descs` holds exactly
 * count*3 descriptors, expert-major [e0.gate, e0.up, e0.down, e1.gate, ...],
 * gate/up [M rows, D cols], down [D rows, M cols]; count = K <= 16 experts.
 * One submission: K gate + K up GEMVs, SwiGLU h = silu(g)*u, K down GEMVs.
 * begin returns an opaque pending handle (NULL = pre-submit decline);
 * finish waits and writes the K expert outputs (count*D floats, expert-major);
 * the caller does its own rank-ordered weighted reduction. fmt 7 (MXFP4) and
 * 21..24 as the reference, and 16..19 (bf16 sidecars) as well, mixed per
 * matrix. */
void *logan_hip_moe_route_begin(uint64_t model_id, int layer, LoganHipMatmulDesc *descs, int count,
                                const float *x, int D, int M);
int logan_hip_moe_route_finish(void *pending, float *out, int count);
void logan_hip_moe_route_discard(void *pending);
void logan_hip_moe_route_drop_model(uint64_t model_id);

/* Replaces coli_metal_shared_mxfp4 (backend_metal.h:146-149): descs =
 * [gate, up, down] (count == 3) of fmt 7 (MXFP4) or affine, out[D] =
 * down(silu(gate.x) * (up.x)). The scalar shared-expert gate stays with the
 * caller (logan-qwen4/src/lib.rs:7602-7604). */
int logan_hip_shared_expert(uint64_t model_id, int layer, LoganHipMatmulDesc *descs, int count,
                            const float *x, float *out, int D, int Iinter);
void logan_hip_shared_expert_drop_model(uint64_t model_id);

/* Replaces coli_metal_llama_layer / coli_metal_llama_drop_model
 * (backend_metal.h:102-115, backend_metal.mm:2495-2791): one dense
 * Llama/MiniCPM5 decode layer on x[D] in place. descs are exactly
 * [q, k, v, o, gate, up, down] of fmt 5 (raw bf16) or 15 (affine-8 g64, each
 * weight rounded to bf16 as the reference's QMV does); RMSNorm, RoPE,
 * attention over the layer's GPU-held f32 K/V cache, residuals and SwiGLU
 * run on the device, and the position's K and V rows (after RoPE) come back
 * in k_out / v_out [kv_heads * head_dim]. Calls for one (model_id, layer)
 * must come in position order (pos = tokens so far, else 0); drop_model
 * frees the caches. head_dim even and <= 256. 1 ok, 0 declined, -1 failure. */
int logan_hip_host_llama_layer(uint64_t model_id, int layer, LoganHipMatmulDesc *descs, int count,
                               float *x, float *k_out, float *v_out, const float *in_norm,
                               const float *post_norm, int D, int inter, int heads, int kv_heads,
                               int head_dim, int pos, float theta, float eps);
void logan_hip_host_llama_drop_model(uint64_t model_id);

/* Host-pointer element-wise ops on the GPU (stage in HBM, run, copy back,
 * wait): in-place RMSNorm of nrows rows of n floats,
 * x = x * (1 / sqrt(mean(x^2) + eps)) * w (replaces coli_metal_rmsnorm,
 * backend_metal.h:24, backend_metal.mm:2147-2166 with kernel a_rmsnorm
 * :705-714); y += a (coli_metal_add, backend_metal.mm:2168-2185); the SwiGLU
 * g = silu(g) * u (coli_metal_silu_mul, :2187-2204). 1 ok, 0 declined,
 * -1 failure. */
int logan_hip_host_rmsnorm(float *x, const float *w, int n, int nrows, float eps);
int logan_hip_host_add(float *y, const float *a, int n);
int logan_hip_host_silu_mul(float *g, const float *u, int n);

/* Replace coli_metal_tensor_free / coli_metal_tensor_bytes (backend_metal.h:180-181). */
void logan_hip_tensor_free(LoganHipTensor *tensor);
size_t logan_hip_tensor_bytes(const LoganHipTensor *tensor);

/* ------------------------------------------------------------------------ */
/* Layer 2: device-native (HBM-resident, bf16)                              */
/* ------------------------------------------------------------------------ */

enum { LOGAN_HIP_F32 = 0, LOGAN_HIP_BF16 = 1 };

/* One affine matrix in device memory (the MLX dense layout,
 * logan-qwen4/src/lib.rs:11818-11937): weights [O][I*bits/8] (16-byte
 * aligned), scales [O][I/gs] u16, biases [O][I/gs] u16. */
typedef struct LoganHipAffine {
  const void *weights;
  const void *scales;
  const void *biases;
  int O;
  int I;
  int bits;       /* 4, 5, 6, 8 */
  int group_size; /* multiple of 32 dividing I for the fast kernels */
  int aux_fp16;   /* 0: bf16 sidecars, 1: fp16 */
} LoganHipAffine;

/* y[M][y_stride] = x[M][x_stride] . W^T  (matmul_mlx_affine_storage,
 * logan-qwen4/src/lib.rs:3729-3764, per activation row). x bf16, y bf16 or
 * f32 (y_dtype). f32 accumulation. 1 ok, 0 unsupported geometry, -1 launch
 * failure. With M >= 3 (I a multiple of 512, groups of 64k) the product may
 * be split over K, its partial sums passing through one of 4 library-owned
 * scratch slots: a call waits on the device (an event wait on its stream)
 * for the previous user of its slot, so calls on any number of streams stay
 * correct. Calls made inside a stream capture skip that wait: replays of a
 * captured graph are ordered by their own stream only. */
int logan_hip_affine_gemv(const LoganHipAffine *w, const void *x, int M, int x_stride, void *y,
                          int y_stride, int y_dtype, void *stream);

/* Up to 8 matrices that read the same activation (q/k/v, gate/up, ...) in
 * one launch: ys[i][M][O_i] = x[M][x_stride] . W_i^T, each as
 * logan_hip_affine_gemv. The reference encodes its batch of GEMVs into one
 * command buffer (coli_metal_matmul_multi,
 * logan-metal/metal/backend_metal.mm:2290-2493, up to 16 descriptors each
 * with its own x); here the shared x is read once per block and the
 * matrices' row blocks form one grid (for 3..32 rows of x where the K-split
 * form applies: one K-split grid and one partial-sum reduction for all the
 * matrices, through the same scratch slots as logan_hip_affine_gemv). Every
 * matrix has the same I, bits, group_size and aux type. 1 ok, 0 unsupported,
 * -1 launch failure. */
int logan_hip_affine_gemv_multi(const LoganHipAffine *ws, int count, const void *x, int M,
                                int x_stride, void *const *ys, int y_dtype, void *stream);

/* The dense MLP's gate/up pair and its SwiGLU as one product:
 * h[M][h_stride] = silu(gate . x) * (up . x), silu(v) = v / (1 + exp(-v)),
 * from the f32 accumulators (logan-qwen4/src/lib.rs:8803-8812; replaces the
 * two GEMVs plus coli_metal_silu_mul of the reference's dense layer,
 * logan-metal/metal/backend_metal.mm:2187-2203). gate and up share I, O,
 * bits, group_size and aux type. Token pairs take the dot2 kernel with each
 * team computing a gate row and its up row; 3..32 tokens the K-split pair,
 * whose reduction forms h. h bf16 (RNE) or f32. 1 ok, 0 unsupported, -1
 * launch failure. */
int logan_hip_affine_gemv_swiglu(const LoganHipAffine *gate, const LoganHipAffine *up,
                                 const void *x, int M, int x_stride, void *h, int h_stride,
                                 int h_dtype, void *stream);

/* Prefill / large-batch form of the same product on MFMA, with the
 * reference QMM's numerics (logan-metal/metal/backend_metal.mm:1480-1560,
 * spark_qmm_affine8_t16o8): every dequantised weight code*scale + bias is
 * rounded to bf16 (RNE) before bf16 x bf16 products are accumulated in f32.
 * x bf16 [M][x_stride], y bf16 (RNE) or f32. I must be a multiple of 64 and
 * group_size a multiple of 32. 1 ok, 0 unsupported geometry, -1 launch
 * failure. Grids short of blocks split K and pass partial sums through one
 * of 2 library-owned scratch slots, ordered across streams as in
 * logan_hip_affine_gemv (the same capture caveat applies). */
int logan_hip_affine_qmm(const LoganHipAffine *w, const void *x, int M, int x_stride, void *y,
                         int y_stride, int y_dtype, void *stream);

/* Up to 8 matrices that read the same x (q/k/v, qkvz/ba of a prefill
 * chunk) as one product: ys[i][M][O_i] = x . bf16(W_i)^T, each as
 * logan_hip_affine_qmm. With M >= 256 and power-of-two group sizes their
 * column tiles form one grid (the reference encodes its batch of products
 * into one command buffer, backend_metal.mm:2290-2493); otherwise one launch
 * per matrix. Every matrix has the same I, bits, group_size and aux type. 1
 * ok, 0 unsupported, -1 launch failure. Split grids share
 * logan_hip_affine_qmm's scratch slots and their cross-stream ordering. */
int logan_hip_affine_qmm_multi(const LoganHipAffine *ws, int count, const void *x, int M,
                               int x_stride, void *const *ys, int y_dtype, void *stream);

/* SwiGLU between a dense gate/up pair and the down projection, in place:
 * g[i] = silu(g[i]) * u[i], silu(v) = v / (1 + exp(-v)), f32 arithmetic
 * (replaces coli_metal_silu_mul, logan-metal/metal/backend_metal.mm
 * :2187-2203, kernel moe_silu :698-699). dtype LOGAN_HIP_F32 or
 * LOGAN_HIP_BF16 (bf16 result rounded RNE); g and u 16-byte aligned device
 * pointers of n elements. 1 ok, 0 bad arguments, -1 launch failure. */
int logan_hip_silu_mul(void *g, const void *u, long long n, int dtype, void *stream);

/* Same product with f32 activations and f32 output, exact per-element
 * dequantisation (any group size dividing I). */
int logan_hip_affine_gemv_f32(const LoganHipAffine *w, const float *x, int M, int x_stride,
                              float *y, int y_stride, void *stream);

/* out[nrows][I] = code*scale + bias for rows [row0, row0+nrows), f32 — the
 * dequantised-weight oracle form (logan-qwen4/src/colisource.rs:779-856),
 * for bit-exact checks. */
int logan_hip_affine_dequant(const LoganHipAffine *w, int row0, int nrows, float *out,
                             void *stream);

/* One MXFP4 matrix in device memory (logan-metal fmt 7; planes 2 / 3 are
 * fmt 9 / 10, the residual expansions whose products add,
 * backend_metal.mm:438-490, 1860-1863, 1888-1890): codes
 * [planes][O][I/2] (element 2j in the low nibble of byte j, E2M1; 16-byte
 * aligned), scales [planes][O][I/32] E8M0 bytes (scale = 2^(byte - 127)). I a
 * multiple of 32. */
typedef struct LoganHipMxfp4 {
  const void *codes;
  const void *scales;
  int O;
  int I;
  int planes; /* 1, 2, 3 */
} LoganHipMxfp4;

/* ys[i][O_i] = W_i . xs[i] for up to 16 matrices, each with its own
 * activation, in one launch (the fmt 7/9/10 GEMV of backend_metal.mm
 * :438-490, as coli_metal_matmul_multi batches it, :2290-2493). xs 16-byte
 * aligned, x_dtype LOGAN_HIP_F32 (split in registers into bf16 hi + lo,
 * |x - hi - lo| <= 2^-18 |x|) or LOGAN_HIP_BF16; y f32 or bf16 (RNE); f32
 * accumulation, each 32-column group's sum scaled once by its power of two.
 * 1 ok, 0 unsupported, -1 launch failure. */
int logan_hip_mxfp4_gemv(const LoganHipMxfp4 *ws, int count, const void *const *xs, int x_dtype,
                         void *const *ys, int y_dtype, void *stream);

/* out[nrows][I] = E2M1(code) * 2^(scale - 127) of plane 0, rows
 * [row0, row0+nrows), f32, through the decode instruction the GEMV uses —
 * for bit-exact checks of the decode. */
int logan_hip_mxfp4_dequant(const LoganHipMxfp4 *w, int row0, int nrows, float *out, void *stream);

/* One matrix of the dense decode layer in device memory: fmt 5 = raw bf16
 * weights [O][I] (I a multiple of 16); fmt 15 = MLX affine-8 codes u8 [O][I]
 * with bf16 scales and biases [O][I/64] each (I a multiple of 64), every
 * weight taken as RNE_bf16(code * scale + bias). 16-byte aligned. */
typedef struct LoganHipDense {
  const void *weights;
  const void *scales;
  const void *biases;
  int O;
  int I;
  int fmt;
} LoganHipDense;

/* A dense Llama layer in device memory: its seven matrices, f32 norm
 * weights [D], and the caller's f32 K/V cache [cache_tokens][kv_heads *
 * head_dim] (K rows stored after RoPE). */
typedef struct LoganHipLlamaLayer {
  LoganHipDense q, k, v, o, gate, up, down;
  const float *in_norm;
  const float *post_norm;
  float *k_cache;
  float *v_cache;
  int cache_tokens;
  int D, inter, heads, kv_heads, head_dim;
  float theta, eps;
} LoganHipLlamaLayer;

/* Workspace bytes of logan_hip_llama_layer at position pos (0 if the layer
 * is unsupported). */
size_t logan_hip_llama_workspace_bytes(const LoganHipLlamaLayer *L, int pos);

/* The decode layer of logan_hip_host_llama_layer on device buffers: x[D] f32
 * in place, K[pos] and V[pos] written to the caches (pos < cache_tokens),
 * attention over positions 0..pos. x, the two norm weights and ws must be
 * 16-byte aligned. 1 ok, 0 unsupported (or unaligned), -1 launch failure. */
int logan_hip_llama_layer(const LoganHipLlamaLayer *L, float *x, int pos, void *ws, size_t ws_bytes,
                          void *stream);

/* Router: per token, softmax over E logits then top-k with lower-index ties
 * (logan-qwen4/src/lib.rs:7993-8043); idx[B][k] in rank order, w[B][k] =
 * val_r / sum_{r<k} val (:8694). logits_dtype LOGAN_HIP_F32/BF16; E <= 1024,
 * k <= 32. */
int logan_hip_route_topk(const void *logits, int logits_dtype, int B, int E, int k, int32_t *idx,
                         float *w, void *stream);

/* A stack of E experts' matrices (MLX switch_mlp layout,
 * logan-qwen4/src/lib.rs:11939-12078): expert e's weights start at
 * weights + e*O*(I*bits/8), its params at e*O*(I/gs) elements. */
typedef struct LoganHipAffineBank {
  const void *weights;
  const void *scales;
  const void *biases;
  int E;
  int O;
  int I;
  int bits;
  int group_size;
  int aux_fp16;
} LoganHipAffineBank;

/* Routed-MoE block (logan-qwen/src/lib.rs:535-593; logan-qwen4/src/lib.rs
 * :8692-8711, :8758-8815, :7597-7759). Routed banks gate/up [E][inter][D],
 * down [E][D][inter]. Shared expert: shared_gate/up/down with E == 1
 * (weights NULL = no shared expert); shared_gate_vec bf16 [D] is the scalar
 * gate row (NULL = gate 1.0). Shared banks must use the routed bits and
 * group sizes. */
typedef struct LoganHipMoeBlock {
  LoganHipAffineBank gate, up, down;
  LoganHipAffineBank shared_gate, shared_up, shared_down;
  const void *shared_gate_vec;
  int top_k;
} LoganHipMoeBlock;

/* Device workspace bytes for B tokens. */
size_t logan_hip_moe_workspace_bytes(const LoganHipMoeBlock *blk, int B);

/* out[B][D] = MoE(x[B][D] bf16, logits[B][E]); out_dtype LOGAN_HIP_BF16
 * (RNE of the f32 result) or LOGAN_HIP_F32. idx_out [B][k] and w_out [B][k]
 * are optional (NULL) copies of the routing. workspace: device memory of at
 * least logan_hip_moe_workspace_bytes(blk, B) bytes (256-byte aligned), or
 * NULL to use a library-owned buffer (allocated on growth). B <= 4096,
 * B * k <= 65536, E <= 1024, k <= 32. 1 ok, 0 unsupported geometry,
 * -1 failure. */
int logan_hip_moe_block(const LoganHipMoeBlock *blk, const void *x, const void *logits,
                        int logits_dtype, int B, void *out, int out_dtype, int32_t *idx_out,
                        float *w_out, void *workspace, size_t workspace_bytes, void *stream);

/* The routed-MoE block with the router on device: logits[B][E] = x . router^T
 * with f32 accumulation and f32 results (logan-qwen4/src/lib.rs:7990-7991,
 * `matmul(&mut logits, x, &layer.router)` before softmax_row), written to
 * `logits` (device f32 [B][E], caller-provided), then logan_hip_moe_block on
 * those f32 logits (routing bit-exact against the reference's selection on
 * the same logits). router: E rows of D columns, any geometry
 * logan_hip_affine_gemv takes (MLX checkpoints keep it at 8-bit g64). Other
 * arguments as logan_hip_moe_block. 1 ok, 0 unsupported, -1 failure. */
int logan_hip_moe_block_routed(const LoganHipMoeBlock *blk, const LoganHipAffine *router,
                               const void *x, int B, float *logits, void *out, int out_dtype,
                               int32_t *idx_out, float *w_out, void *workspace,
                               size_t workspace_bytes, void *stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): logan_hip_moe_block without a workspace argument. Its
 * workspace is a library-owned file-scope device array of
 * LOGAN_HIP_MOE_STATIC_SCRATCH_BYTES on each device (held until the process
 * ends); the call allocates nothing. Calls whose workspace would exceed it
 * (B above a few hundred tokens at the config-3 shapes: 57 MB at B = 512)
 * return 0 and print why. Every call on a device shares that device's array:
 * calls whose executions overlap on one device (other streams) race. */
#define LOGAN_HIP_MOE_STATIC_SCRATCH_BYTES (64u << 20)
int logan_hip_moe_block_static(const LoganHipMoeBlock *blk, const void *x, const void *logits,
                               int logits_dtype, int B, void *out, int out_dtype,
                               int32_t *idx_out, float *w_out, void *stream);

/* Controls of the routed-MoE block's single-launch B = 1 path (one kernel
 * with an in-kernel hand-off between the gate/up and down phases). It is on
 * by default (LOGAN_HIP_MOE_FUSED=0 in the environment turns it off);
 * set_moe_fused(0/1) overrides, like the reference's LOGAN_MOE_ISLAND switch
 * (logan-qwen4/src/lib.rs:14907-14922). Launches of that path on one device
 * must not overlap. sync_errors returns its sticky error word for the
 * current device: 0 = healthy; bit 0 = a phase hand-off wait timed out (the
 * output of that call was not valid); bit 1 = a launch counter not on a
 * launch boundary, bit 2 = launch counters out of step (both checked between
 * launches); bit 3 = a routed expert missing from logan_hip_moe_block_cached's
 * map (that call's output was not valid). */
void logan_hip_set_moe_fused(int on);
uint32_t logan_hip_moe_sync_errors(void);

/* Batches of at least this many tokens take the routed-MoE block's MFMA
 * path (4/5/6/8-bit codes with group sizes that are multiples of 64; each
 * expert's weights read once per 16 of its tokens); smaller batches and
 * other geometries take the per-token dot-product path in passes of up to
 * 64 tokens. b > 0 sets one threshold for every code width; b <= 0
 * restores the defaults: 56 tokens for 4-bit codes, 24 for 5/6/8-bit
 * (LOGAN_HIP_MOE_MFMA_MIN_B from the environment, when set, replaces them).
 * Both paths follow the same reference semantics (logan-qwen4/src/lib.rs
 * :8692-8711, :8759-8815); this control has no counterpart in the
 * reference (its batched path is host-side, lib.rs:9714-9721). */
void logan_hip_set_moe_mfma_min_batch(int b);

/* ------------------------------------------------------------------------ */
/* Layer 3: MLX quantized weights from a safetensors checkpoint into HBM     */
/* ------------------------------------------------------------------------ */

/* Message of the last call of this layer that returned 0, -1 or NULL on the
 * calling thread (the reference's Err(String) text for a rejected tensor). */
const char *logan_hip_last_error(void);

typedef struct LoganHipStFile LoganHipStFile;

/* StFile::open (logan-qwen4/src/lib.rs:508-531): one .safetensors file,
 * header checked as parse_shard does (:326-421: header inside the file,
 * known dtype, data_offsets inside the file, span == elements x width).
 * NULL on error. */
LoganHipStFile *logan_hip_st_open(const char *path);
/* StFile::open_dir (lib.rs:537-595): every shard named by
 * model.safetensors.index.json (sorted, deduplicated), or model.safetensors;
 * names under model.language_model. / language_model.model. /
 * language_model.lm_head. also answer to the engine's model. / lm_head.
 * spelling (register, :460-503). NULL on error. */
LoganHipStFile *logan_hip_st_open_dir(const char *dir);
void logan_hip_st_close(LoganHipStFile *st);
/* shard_count (lib.rs:598-600) */
int logan_hip_st_shard_count(const LoganHipStFile *st);
/* shape_of (lib.rs:946-948) plus dtype and payload bytes: 1 found, 0 absent.
 * shape receives up to max_dims dims, *ndim the tensor's rank. */
int logan_hip_st_tensor(const LoganHipStFile *st, const char *name, char *dtype, size_t dtype_cap,
                        uint64_t *shape, int max_dims, int *ndim, uint64_t *nbytes);
/* dtype_counts (lib.rs:671-680): distinct payloads of one dtype. */
int logan_hip_st_dtype_count(const LoganHipStFile *st, const char *dtype);
/* payload_range (lib.rs:726-760) into host memory: 1 ok, 0 rejected, -1 read
 * failure. */
int logan_hip_st_read(const LoganHipStFile *st, const char *name, uint64_t within, uint64_t len,
                      void *dst);

enum { LOGAN_HIP_WT_AFFINE = 1, LOGAN_HIP_WT_MXFP4 = 2 };

/* A quantized weight (WtBytes::MlxAffine / WtBytes::Mxfp4,
 * logan-qwen4/src/lib.rs:1560-1580) resident in HBM: the file's bytes
 * unchanged, E experts stacked (E = 1 for a dense matrix). Affine: weights
 * [E][O][I*bits/8], scales and biases u16 [E][O][I/group_size] (bf16, or
 * fp16 when aux_fp16). MXFP4: weights [E][O][I/2], scales E8M0 bytes
 * [E][O][ceil(I/32)], biases NULL. One device allocation, 256-byte aligned
 * parts, released by logan_hip_quant_free. */
typedef struct LoganHipQuantWt {
  int kind; /* LOGAN_HIP_WT_AFFINE or LOGAN_HIP_WT_MXFP4 */
  int E;
  int O;
  int I;
  int bits;
  int group_size;
  int aux_fp16;
  const void *weights;
  const void *scales;
  const void *biases;
  uint64_t weight_bytes, scale_bytes, bias_bytes;
  void *owner;
} LoganHipQuantWt;

/* load_mlx_quantized_wt (logan-qwen4/src/lib.rs:11818-11937) into HBM:
 * `name` is the U32 [O, words] packed weight ending in .weight; bits =
 * words*32/I must be 4, 5, 6 or 8; a BF16/F16 `.scales` [O, groups] with an
 * identical `.biases` makes it affine (group_size = I/groups), a U8 `.scales`
 * [O, ceil(I/32)] with 4-bit codes makes it MXFP4. 1 ok; 0 rejected (the
 * reference's conditions and message, logan_hip_last_error), nothing
 * allocated; -1 read or device failure. Blocking; calls serialise. */
int logan_hip_load_mlx_quantized(const LoganHipStFile *st, const char *name, int O, int I,
                                 LoganHipQuantWt *out);
/* load_mlx_quantized_expert_wt (lib.rs:11939-12078) for the `count`
 * consecutive experts e0 .. e0+count-1 of a stacked switch_mlp bank U32
 * [experts, O, words] (count = 1 is the reference's one-expert read;
 * count = experts makes the whole bank resident in one transfer). Same
 * return convention. */
int logan_hip_load_mlx_quantized_experts(const LoganHipStFile *st, const char *name, int e0,
                                         int count, int experts, int O, int I,
                                         LoganHipQuantWt *out);
/* The same checks without reading or allocating anything: fills kind,
 * geometry and the byte counts (pointers NULL). 1 accepted, 0 rejected. */
int logan_hip_plan_mlx_quantized(const LoganHipStFile *st, const char *name, int O, int I,
                                 LoganHipQuantWt *out);
int logan_hip_plan_mlx_quantized_experts(const LoganHipStFile *st, const char *name, int e0,
                                         int count, int experts, int O, int I,
                                         LoganHipQuantWt *out);
void logan_hip_quant_free(LoganHipQuantWt *w);

/* ---- Route-driven expert cache (banks not kept resident) ----------------
 * The reference's EXP-069 RouteCache and EXP-067 RouteArena
 * (logan-qwen4/src/lib.rs:12110-12300; builders try_build_route_cache /
 * try_build_route_arena :12959-13140; cache_fetch_route :12697-12903) in
 * one HBM allocation of expert blocks. A block holds one routed expert's
 * gate, up and down matrices (packed weights, scales, biases) in io_plan's
 * order (:13550-13590), each part 256-byte aligned. Each layer owns
 * blocks_per_layer retained blocks (the reference's LOGAN_ROUTE_CACHE
 * blocks: tags, a replacement cursor that skips the blocks the current
 * route has claimed, hit / miss / eviction counts); 2 x topk more blocks are
 * the route arena (one set of topk per layer parity) for the ranks the
 * cache does not retain. Affine banks only. */
typedef struct LoganHipExpertCache LoganHipExpertCache;

typedef struct LoganHipExpertCacheStats {
  uint64_t hits, misses, evictions; /* retained ranks (:12775-12789) */
  uint64_t streamed;                /* ranks loaded through the route arena */
  uint64_t bytes_loaded;            /* host -> HBM bytes of all fills */
  uint64_t generation;              /* bumped per block reuse (:12163) */
  uint64_t block_bytes, device_bytes;
  int layers, blocks_per_layer, topk;
} LoganHipExpertCacheStats;

/* Blocks sized from layer 0 expert 0's banks
 * model.layers.{L}.mlp.switch_mlp.{gate,up,down}_proj of `st` (stacked
 * [experts] banks, gate/up d_hidden x d_model, down d_model x d_hidden, the
 * loader's checks). layers 0: counted from the tensor table as
 * try_build_route_cache does (:12965-12975). blocks_per_layer 0: every rank
 * streams through the arena. topk <= 32. `st` must stay open while the
 * cache lives. NULL on error (logan_hip_last_error). */
LoganHipExpertCache *logan_hip_expert_cache_create(const LoganHipStFile *st, int layers, int experts,
                                                   int d_model, int d_hidden, int blocks_per_layer,
                                                   int topk);
/* Waits for the device, frees the blocks. */
void logan_hip_expert_cache_destroy(LoganHipExpertCache *c);
/* cache_fetch_route for one token's route experts[0..k-1] (rank order) of
 * `layer`: ranks below min(blocks_per_layer, k) are looked up / reserved in
 * the layer's cache (RouteCache::reserve, :12190-12228), the others take the
 * layer parity's arena blocks; misses and arena ranks are read from the
 * checkpoint through the loader's pinned staging ring and copied on the
 * loader's stream after the work already queued on `stream` (which may
 * still read those blocks), and `stream` then waits for the copies (the
 * host returns once the reads are staged). blocks_out[r] = the block of rank
 * r, for logan_hip_moe_block_cached. 1 ok; 0 declined (k > topk, an id out
 * of range, a layer whose banks differ from the cache's layout); -1 read or
 * device failure (the blocks this call claimed are dropped from the cache;
 * the reference disables its cache instead). Calls on one cache
 * serialise. */
int logan_hip_expert_cache_fetch(LoganHipExpertCache *c, int layer, const int32_t *experts, int k,
                                 int32_t *blocks_out, void *stream);
void logan_hip_expert_cache_stats(const LoganHipExpertCache *c, LoganHipExpertCacheStats *out);
/* The layer's block tags (expert per retained block, -1 empty) into
 * tags_out[blocks_per_layer]. 1 ok, 0 bad arguments. */
int logan_hip_expert_cache_tags(const LoganHipExpertCache *c, int layer, int32_t *tags_out);

/* logan_hip_moe_block for one token (B = 1) whose routed experts come from
 * an expert cache: experts[r] / blocks[r] are the route and the blocks
 * logan_hip_expert_cache_fetch returned (the engine's authoritative route,
 * e.g. logan_hip_route_topk on the same logits, so the block's own routing
 * selects the same experts). blk supplies top_k (== k), the shared expert,
 * its gate vector and the routed geometry (gate.E = experts, O, I, bits,
 * group_size, aux_fp16 equal to the cache's); its routed weight pointers are
 * not read. The output is bit-identical to logan_hip_moe_block on resident
 * banks holding the same bytes. A routed expert missing from the map sets
 * bit 3 of logan_hip_moe_sync_errors (the launch reads a mapped block, in
 * bounds). 1 ok, 0 unsupported, -1 failure. */
int logan_hip_moe_block_cached(const LoganHipMoeBlock *blk, const LoganHipExpertCache *c,
                               const int32_t *experts, const int32_t *blocks, int k, const void *x,
                               const void *logits, int logits_dtype, void *out, int out_dtype,
                               int32_t *idx_out, float *w_out, void *workspace,
                               size_t workspace_bytes, void *stream);

/* Library version string. */
const char *logan_hip_version(void);

#ifdef __cplusplus
}
#endif
#endif /* LOGAN_HIP_H */
