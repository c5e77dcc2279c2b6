/*
 * logan-metal's C ABI as exported by liblogan_hip.so: every function that the
 * Rust FFI blocks of logan-metal/src/lib.rs declare (`unsafe extern "C"` at
 * :198-481, :2795-2818, :3382-3585), with the C form of the Rust signature,
 * so that block links against this library unchanged. tests/golden/
 * ffi_symbols.json holds the reference's declarations (names, parameter
 * types, lines) and tests/test_ffi_surface.py checks this header and the
 * library's exports against it.
 *
 * Three kinds of entry:
 *  - implemented: the same operation on the GPU, forwarding to the
 *    logan_hip_* entry point named (include/logan_hip.h), with the
 *    reference's 1 / 0 / -1 return convention;
 *  - advisory: host-memory registration, which this library does not need;
 *  - declining: operations outside the quantized-decode hot path (ANE and
 *    IOSurface bridges, GDN/HC/MLA/Spark layers, MetalIO streaming,
 *    Apple8 tiles, BNNS), returning what the reference's non-macOS build
 *    returns to its callers (logan-metal/src/lib.rs:4322-5069: nothing is
 *    done, the caller keeps its CPU path).
 * Out-parameters of declining and advisory functions are left untouched
 * unless stated.
 */
#ifndef LOGAN_METAL_FFI_H
#define LOGAN_METAL_FFI_H

#include <stddef.h>
#include <stdint.h>

#include "logan_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ColiMetalTensor is the opaque handle of the host-pointer layer;
 * ColiMetalMatmulDesc (ColiMetalMatmulDescRaw, logan-metal/src/lib.rs:124-139;
 * backend_metal.h:68-88) has LoganHipMatmulDesc's layout. */
typedef LoganHipTensor ColiMetalTensor;
typedef LoganHipMatmulDesc ColiMetalMatmulDesc;
/* only passed by pointer to declining functions */
typedef struct ColiMetalioRegion ColiMetalioRegion;
typedef struct ColiMetalioStats ColiMetalioStats;
typedef struct ColiApple8MetalioExpert ColiApple8MetalioExpert;

/* ---- implemented: forward to the logan_hip_* entry point named ---------- */

/* lib.rs:253 -> logan_hip_init */
int32_t coli_metal_init(void);
/* lib.rs:254 -> logan_hip_available */
int32_t coli_metal_available(void);
/* lib.rs:255 -> logan_hip_profile_set_on */
void coli_metal_profile_set_on(int32_t on);
/* lib.rs:256 -> logan_hip_profile_reset */
void coli_metal_profile_reset(void);
/* lib.rs:257 -> logan_hip_profile_get */
void coli_metal_profile_get(uint64_t *encode, uint64_t *submit, uint64_t *wait, uint64_t *kernel);
/* lib.rs:263 -> logan_hip_matmul */
int32_t coli_metal_matmul(ColiMetalTensor **tensor, float *y, const float *x, const void *weights,
                          const float *scales, int32_t fmt, int32_t s, int32_t i, int32_t o,
                          int32_t gs);
/* lib.rs:279 -> logan_hip_matmul_multi */
int32_t coli_metal_matmul_multi(const float *x, int32_t s, ColiMetalMatmulDesc *descs,
                                int32_t count);
/* lib.rs:443 -> logan_hip_shared_expert */
int32_t coli_metal_shared_mxfp4(uint64_t model_id, int32_t layer, ColiMetalMatmulDesc *descs,
                                int32_t count, const float *x, float *out, int32_t d,
                                int32_t iinter);
/* lib.rs:453 -> logan_hip_shared_expert_drop_model */
void coli_metal_shared_mxfp4_drop_model(uint64_t model_id);
/* lib.rs:285 -> logan_hip_host_llama_layer */
int32_t coli_metal_llama_layer(uint64_t model_id, int32_t layer, ColiMetalMatmulDesc *descs,
                               int32_t count, float *x, float *k_out, float *v_out,
                               const float *input_norm, const float *post_norm, int32_t d,
                               int32_t inter, int32_t heads, int32_t kv_heads, int32_t head_dim,
                               int32_t pos, float theta, float eps);
/* lib.rs:304 -> logan_hip_host_llama_drop_model */
void coli_metal_llama_drop_model(uint64_t model_id);
/* lib.rs:454 -> logan_hip_host_rmsnorm */
int32_t coli_metal_rmsnorm(float *x, const float *w, int32_t n, int32_t nrows, float eps);
/* lib.rs:455 -> logan_hip_host_add */
int32_t coli_metal_add(float *y, const float *a, int32_t n);
/* lib.rs:456 -> logan_hip_host_silu_mul */
int32_t coli_metal_silu_mul(float *g, const float *u, int32_t n);
/* lib.rs:457 -> logan_hip_tensor_free */
void coli_metal_tensor_free(ColiMetalTensor *tensor);
/* lib.rs:458 -> logan_hip_shutdown */
void coli_metal_shutdown(void);
/* lib.rs:3440 -> logan_hip_moe_route_begin */
void *coli_metal_moe_route_begin(uint64_t model_id, int32_t layer, ColiMetalMatmulDesc *descs,
                                 int32_t count, const float *x, int32_t d, int32_t m);
/* lib.rs:3449 -> logan_hip_moe_route_finish */
int32_t coli_metal_moe_route_finish(void *pending, float *out, int32_t count);
/* lib.rs:3450 -> logan_hip_moe_route_discard */
void coli_metal_moe_route_discard(void *pending);
/* lib.rs:3451 -> logan_hip_moe_route_drop_model */
void coli_metal_moe_route_drop_model(uint64_t model_id);

/* ---- advisory (weights are copied to HBM on first use, so registration
 *      changes nothing): register/unregister do nothing, ptr_registered
 *      returns 0, wrap_stats reports zeros ---------------------------------- */

/* lib.rs:275 */
void coli_metal_wrap_stats(uint64_t *calls, uint64_t *zero_copy, uint64_t *copy_bytes,
                           uint64_t *bytes_created);
/* lib.rs:276 */
void coli_metal_register(void *base, size_t len);
/* lib.rs:277 */
void coli_metal_unregister(void *base);
/* lib.rs:278 */
int32_t coli_metal_ptr_registered(const void *base);

/* ---- out of this library's scope: decline as the reference's non-macOS
 *      build does, so the caller keeps its CPU path (value returned in the
 *      comment; no-op for void functions; out-parameters are left untouched) */

/* lib.rs:199: NULL */
void *logan_metal_shared_surface_wrap(void *raw_surface, size_t logical_bytes);
/* lib.rs:203: no-op */
void logan_metal_shared_surface_free(void *handle);
/* lib.rs:204: NULL */
void *logan_metal_shared_surface_contents(void *handle);
/* lib.rs:205: 0 */
size_t logan_metal_shared_surface_length(void *handle);
/* lib.rs:206: 0 */
size_t logan_metal_shared_surface_allocation_length(void *handle);
/* lib.rs:207: NULL */
void *logan_metal_ane_dynamic_pack_create(void *qkv_surface, void *aux_surface,
                                          const uint16_t *wqkv, const uint16_t *wz,
                                          const uint16_t *wa, const uint16_t *wb, uint32_t hidden,
                                          uint32_t spatial, uint32_t qkv_rows, uint32_t z_rows,
                                          uint32_t ab_rows, uint32_t qkv_stride,
                                          uint32_t aux_stride, uint32_t qkv_offset,
                                          uint32_t z_offset, uint32_t a_offset, uint32_t b_offset);
/* lib.rs:226: 0 */
int32_t logan_metal_ane_dynamic_pack_run(void *handle, const float *x, double *gpu_ms);
/* lib.rs:231: NULL */
void *logan_metal_ane_dynamic_pack_begin(void *handle, const float *x, void *signal_event,
                                         uint64_t signal_value);
/* lib.rs:237: 0 */
int32_t logan_metal_ane_dynamic_pack_finish(void *pending, double *gpu_ms);
/* lib.rs:238: no-op */
void logan_metal_ane_dynamic_pack_discard(void *pending);
/* lib.rs:239: no-op */
void logan_metal_ane_dynamic_pack_free(void *handle);
/* lib.rs:240: NULL */
void *logan_metal_gdn_conv_silu_create(void *input_handle, void *output_handle,
                                       const float *weights, size_t channels, size_t spatial,
                                       size_t kernel);
/* lib.rs:248: 0 */
int32_t logan_metal_gdn_conv_silu_run(void *handle);
/* lib.rs:249: NULL */
void *logan_metal_gdn_conv_silu_begin(void *handle);
/* lib.rs:250: 0 */
int32_t logan_metal_gdn_conv_silu_finish(void *handle, double *gpu_ms);
/* lib.rs:251: no-op */
void logan_metal_gdn_conv_silu_free(void *handle);
/* lib.rs:305: 0 */
int32_t coli_metal_gdn_mxfp4(uint64_t model_id, int32_t layer, ColiMetalMatmulDesc *descs,
                             int32_t count, const float *x, float *out, const float *a_log,
                             const float *dt_bias, const float *conv_w, const float *norm_w,
                             float *state, float *conv_state, int32_t d, int32_t kheads, int32_t kd,
                             int32_t vheads, int32_t vd, int32_t kk, int32_t output_gate,
                             float eps);
/* lib.rs:327: no-op */
void coli_metal_gdn_mxfp4_drop_model(uint64_t model_id);
/* lib.rs:328: 0 */
int32_t coli_metal_hc_mix(uint64_t model_id, ColiMetalMatmulDesc *descs, int32_t count,
                          const float *normed, float *out, float *inject, int32_t d, int32_t hc,
                          int32_t lr);
/* lib.rs:339: no-op */
void coli_metal_hc_drop_model(uint64_t model_id);
/* lib.rs:340: 0 */
int32_t coli_metal_spark_layer(uint64_t model_id, int32_t layer, ColiMetalMatmulDesc *descs,
                               int32_t count, float *x, const float *input_norm,
                               const float *post_norm, int32_t d, int32_t inter, int32_t heads,
                               int32_t kv_heads, int32_t head_dim, int32_t sliding, int32_t window,
                               int32_t pos, int32_t rotary_dim, float theta, float eps);
/* lib.rs:360: 0 */
int32_t coli_metal_spark_token_begin(uint64_t model_id, const float *x, int32_t d, int32_t pos);
/* lib.rs:361: 0 */
int32_t coli_metal_spark_layer_encode(uint64_t model_id, int32_t layer, ColiMetalMatmulDesc *descs,
                                      int32_t count, const float *input_norm,
                                      const float *post_norm, int32_t d, int32_t inter,
                                      int32_t heads, int32_t kv_heads, int32_t head_dim,
                                      int32_t sliding, int32_t window, int32_t pos,
                                      int32_t rotary_dim, float theta, float eps);
/* lib.rs:380: 0 */
int32_t coli_metal_spark_token_end(uint64_t model_id, float *x, int32_t d, int32_t pos);
/* lib.rs:381: 0 */
int32_t coli_metal_spark_token_end_top1(uint64_t model_id, ColiMetalMatmulDesc *head,
                                        const float *norm, uint32_t *token, int32_t d,
                                        int32_t vocab, int32_t pos, float eps);
/* lib.rs:391: 0 */
int32_t coli_metal_spark_token_end_logits(uint64_t model_id, ColiMetalMatmulDesc *head,
                                          const float *norm, float *logits, int32_t d,
                                          int32_t vocab, int32_t pos, float eps);
/* lib.rs:401: no-op */
void coli_metal_spark_token_abort(uint64_t model_id);
/* lib.rs:402: 0 */
int32_t coli_metal_spark_prefill_begin(uint64_t model_id, const float *x, int32_t s, int32_t d,
                                       int32_t base);
/* lib.rs:409: 0 */
int32_t coli_metal_spark_prefill_layer_encode(uint64_t model_id, int32_t layer,
                                              ColiMetalMatmulDesc *descs, int32_t count,
                                              const float *input_norm, const float *post_norm,
                                              int32_t d, int32_t inter, int32_t heads,
                                              int32_t kv_heads, int32_t head_dim, int32_t sliding,
                                              int32_t window, int32_t base, int32_t s,
                                              int32_t rotary_dim, float theta, float eps);
/* lib.rs:429: 0 */
int32_t coli_metal_spark_prefill_end(uint64_t model_id, int32_t base, int32_t s);
/* lib.rs:430: 0 */
int32_t coli_metal_spark_prefill_end_logits(uint64_t model_id, ColiMetalMatmulDesc *head,
                                            const float *norm, float *logits, int32_t d,
                                            int32_t vocab, int32_t base, int32_t s, float eps);
/* lib.rs:441: no-op */
void coli_metal_spark_prefill_abort(uint64_t model_id);
/* lib.rs:442: no-op */
void coli_metal_spark_drop_model(uint64_t model_id);
/* lib.rs:459: 0 */
int32_t coli_bnns_bf16_matmul(const uint16_t *w, const float *x, float *y, int32_t o, int32_t i);
/* lib.rs:466: 0 */
int32_t coli_bnns_bf16_matmul_batch(const uint16_t *w, const float *x, float *y, int32_t s,
                                    int32_t o, int32_t i);
/* lib.rs:474: 0 */
int32_t coli_bnns_f16_matmul(const uint16_t *w, const uint16_t *x, float *y, int32_t o, int32_t i);
/* lib.rs:2796: 0 */
int32_t metalio_init(void);
/* lib.rs:2797: 0 */
int32_t metalio_active(void);
/* lib.rs:2798: no-op */
void metalio_shutdown(void);
/* lib.rs:2799: -1 */
int32_t metalio_file_add(const char *path);
/* lib.rs:2800: -1 */
int32_t metalio_slot_alloc(size_t max_bytes);
/* lib.rs:2801: 0 */
int32_t metalio_slot_alloc_alias(void *base, size_t len);
/* lib.rs:2802: no-op */
void metalio_slot_free(int32_t slot);
/* lib.rs:2803: NULL */
void *metalio_slot_ptr(int32_t slot);
/* lib.rs:2804: 0 */
size_t metalio_slot_bytes(int32_t slot);
/* lib.rs:2805: -1 */
int64_t metalio_loadv(int32_t slot, const ColiMetalioRegion *regions, int32_t count, int32_t kind);
/* lib.rs:2811: -1 */
int32_t metalio_wait(int64_t event_value);
/* lib.rs:2812: 0 */
int64_t metalio_batch_barrier(void);
/* lib.rs:2813: -1 */
int32_t metalio_batch_wait(int64_t event_value, const int32_t *slots, int32_t count);
/* lib.rs:2814: no-op */
void metalio_slot_consumed(int32_t slot);
/* lib.rs:2815: no-op */
void metalio_prefetch_demanded(int32_t slot);
/* lib.rs:2816: -1 */
int32_t metalio_probe(int32_t slot);
/* lib.rs:2817: no-op */
void metalio_stats(ColiMetalioStats *out);
/* lib.rs:3383: 0 */
int32_t coli_apple8_metalio_direct_init(void);
/* lib.rs:3384: no-op */
void coli_apple8_metalio_direct_shutdown(void);
/* lib.rs:3385: 0 */
int32_t coli_apple8_metalio_matmul_slot(int32_t slot, size_t slot_offset, size_t matrix_bytes,
                                        const float *x, float *y, int32_t s, int32_t i, int32_t o);
/* lib.rs:3395: 0 */
int32_t coli_apple8_metalio_swiglu_slot(int32_t slot, size_t gate_offset, size_t gate_bytes,
                                        size_t up_offset, size_t up_bytes, size_t down_offset,
                                        size_t down_bytes, const float *x, float *y, int32_t s,
                                        int32_t hidden, int32_t intermediate);
/* lib.rs:3409: 0 */
int32_t coli_apple8_metalio_moe_rows(const ColiApple8MetalioExpert *experts,
                                     const int32_t *row_offsets, int32_t expert_count,
                                     const float *x, float *y, int32_t total_rows, int32_t hidden,
                                     int32_t intermediate);
/* lib.rs:3419: 0 */
int32_t coli_apple8_metalio_moe_topk(const ColiApple8MetalioExpert *experts,
                                     const float *route_weights, int32_t expert_count,
                                     const float *x, float *y, int32_t hidden,
                                     int32_t intermediate);
/* lib.rs:3428: 0 */
int32_t coli_apple8_metalio_moe_topk_begin(const ColiApple8MetalioExpert *experts,
                                           const float *route_weights, int32_t expert_count,
                                           const float *x, int32_t hidden, int32_t intermediate,
                                           void **pending_out);
/* lib.rs:3437: 0 */
int32_t coli_apple8_metalio_moe_topk_finish(void *pending, float *y);
/* lib.rs:3438: no-op */
void coli_apple8_metalio_moe_topk_discard(void *pending);
/* lib.rs:3453: 0 */
int32_t coli_metal_qwen_attn_decode(const float *q, int32_t heads, int32_t kv_heads, int32_t hd,
                                    int32_t max_t, int32_t nsel, float scale, float *out,
                                    const float *kvk_host, const float *kvv_host);
/* lib.rs:3465: no-op */
void coli_apple8_metalio_profile_get(uint64_t *encode_ns, uint64_t *submit_ns, uint64_t *wait_ns,
                                     uint64_t *kernel_ns, uint64_t *fused_calls,
                                     uint64_t *fused_experts);
/* lib.rs:3473: no-op */
void coli_apple8_metalio_profile_detail_get(uint64_t *gdn_wait_ns, uint64_t *gdn_kernel_ns,
                                            uint64_t *gdn_calls, uint64_t *moe_wait_ns,
                                            uint64_t *moe_kernel_ns, uint64_t *moe_calls);
/* lib.rs:3482: 0 */
int32_t coli_apple8_metalio_bf16_matmul(const uint16_t *w, const float *x, float *y, int32_t s,
                                        int32_t o, int32_t i);
/* lib.rs:3491: no-op */
void coli_apple8_metalio_gdn_drop_model(uint64_t model_id);
/* lib.rs:3492: NULL */
void *coli_apple8_metalio_ane_fence_create(uint64_t value, void **shared_backing_out);
/* lib.rs:3496: 0 */
int32_t coli_apple8_metalio_ane_fence_set_value(void *handle, uint64_t value);
/* lib.rs:3497: NULL */
void *coli_apple8_metalio_ane_fence_metal_event(void *handle);
/* lib.rs:3498: no-op */
void coli_apple8_metalio_ane_fence_free(void *handle);
/* lib.rs:3499: 0 */
int32_t coli_apple8_metalio_gdn_begin(uint64_t model_id, int32_t layer, const float *x,
                                      const uint16_t *wqkv, const uint16_t *wz, const uint16_t *wa,
                                      const uint16_t *wb, const uint16_t *wout, const float *a_log,
                                      const float *dt_bias, const float *conv_w,
                                      const float *norm_w, float *state, float *conv_state,
                                      int32_t d, int32_t kheads, int32_t kd, int32_t vheads,
                                      int32_t vd, int32_t kk, int32_t output_gate, float eps,
                                      void **pending_out);
/* lib.rs:3524: 0 */
int32_t coli_apple8_metalio_gdn_ane_begin(uint64_t model_id, int32_t layer, void *qkv_surface,
                                          size_t qkv_bytes, void *z_surface, size_t z_bytes,
                                          void *a_surface, size_t a_bytes, void *b_surface,
                                          size_t b_bytes, int32_t spatial, const uint16_t *wqkv,
                                          const uint16_t *wz, const uint16_t *wa,
                                          const uint16_t *wb, const uint16_t *wout,
                                          const float *a_log, const float *dt_bias,
                                          const float *conv_w, const float *norm_w, float *state,
                                          float *conv_state, int32_t d, int32_t kheads, int32_t kd,
                                          int32_t vheads, int32_t vd, int32_t kk,
                                          int32_t output_gate, float eps, void *ane_fence,
                                          void **pending_out);
/* lib.rs:3558: 0 */
int32_t coli_apple8_metalio_gdn_finish(void *pending, float *out);
/* lib.rs:3559: no-op */
void coli_apple8_metalio_gdn_discard(void *pending);
/* lib.rs:3560: 0 */
int32_t coli_apple8_metalio_gdn_token(uint64_t model_id, int32_t layer, const float *x, float *out,
                                      const uint16_t *wqkv, const uint16_t *wz, const uint16_t *wa,
                                      const uint16_t *wb, const uint16_t *wout, const float *a_log,
                                      const float *dt_bias, const float *conv_w,
                                      const float *norm_w, float *state, float *conv_state,
                                      int32_t d, int32_t kheads, int32_t kd, int32_t vheads,
                                      int32_t vd, int32_t kk, int32_t output_gate, float eps);

/* ---- backend_metal.h entries outside the Rust block, also exported ---- */

/* backend_metal.h:37 -> logan_hip_stats */
void coli_metal_stats(size_t *tensor_count, size_t *tensor_bytes);
/* backend_metal.h:38 -> logan_hip_mem_info */
int coli_metal_mem_info(size_t *used_bytes, size_t *total_bytes);
/* backend_metal.h:181 -> logan_hip_tensor_bytes */
size_t coli_metal_tensor_bytes(const ColiMetalTensor *tensor);

#ifdef __cplusplus
}
#endif
#endif /* LOGAN_METAL_FFI_H */
