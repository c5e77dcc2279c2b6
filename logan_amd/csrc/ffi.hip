// logan-metal's C symbol names (include/logan_metal_ffi.h): every function
// of the Rust FFI blocks in logan-metal/src/lib.rs (:198-481, :2795-2818,
// :3382-3585), so that block links against liblogan_hip.so unchanged.
// Implemented names forward to the logan_hip_* entry point of the same
// meaning; the rest are advisory or decline the way the reference's non-macOS
// build does (logan-metal/src/lib.rs:4322-5069), leaving the caller on its CPU
// path. MetalIO ids and event values decline with -1 (its callers test
// `< 0` / `!= 0`, lib.rs:2890-2990, :3050, :3301), the batch barrier with 0
// (callers test `> 0`, :2862-2864).
#include <hip/hip_runtime.h>

#include "../../include/logan_metal_ffi.h"

extern "C" {

// ---- implemented

int32_t coli_metal_init(void) { return logan_hip_init(); }
int32_t coli_metal_available(void) { return logan_hip_available(); }
void coli_metal_shutdown(void) { logan_hip_shutdown(); }
void coli_metal_profile_set_on(int32_t on) { logan_hip_profile_set_on(on); }
void coli_metal_profile_reset(void) { logan_hip_profile_reset(); }
void coli_metal_profile_get(uint64_t *encode, uint64_t *submit, uint64_t *wait, uint64_t *kernel) {
  logan_hip_profile_get(encode, submit, wait, kernel);
}
int32_t coli_metal_matmul(ColiMetalTensor **tensor, float *y, const float *x, const void *weights,
                          const float *scales, int32_t fmt, int32_t s, int32_t i, int32_t o,
                          int32_t gs) {
  return logan_hip_matmul(tensor, y, x, weights, scales, fmt, s, i, o, gs);
}
int32_t coli_metal_matmul_multi(const float *x, int32_t s, ColiMetalMatmulDesc *descs,
                                int32_t count) {
  return logan_hip_matmul_multi(x, s, descs, count);
}
int32_t coli_metal_shared_mxfp4(uint64_t model_id, int32_t layer, ColiMetalMatmulDesc *descs,
                                int32_t count, const float *x, float *out, int32_t d,
                                int32_t iinter) {
  return logan_hip_shared_expert(model_id, layer, descs, count, x, out, d, iinter);
}
void coli_metal_shared_mxfp4_drop_model(uint64_t model_id) {
  logan_hip_shared_expert_drop_model(model_id);
}
int32_t coli_metal_llama_layer(uint64_t model_id, int32_t layer, ColiMetalMatmulDesc *descs,
                               int32_t count, float *x, float *k_out, float *v_out,
                               const float *input_norm, const float *post_norm, int32_t d,
                               int32_t inter, int32_t heads, int32_t kv_heads, int32_t head_dim,
                               int32_t pos, float theta, float eps) {
  return logan_hip_host_llama_layer(model_id, layer, descs, count, x, k_out, v_out, input_norm,
                                    post_norm, d, inter, heads, kv_heads, head_dim, pos, theta, eps);
}
void coli_metal_llama_drop_model(uint64_t model_id) { logan_hip_host_llama_drop_model(model_id); }
int32_t coli_metal_rmsnorm(float *x, const float *w, int32_t n, int32_t nrows, float eps) {
  return logan_hip_host_rmsnorm(x, w, n, nrows, eps);
}
int32_t coli_metal_add(float *y, const float *a, int32_t n) { return logan_hip_host_add(y, a, n); }
int32_t coli_metal_silu_mul(float *g, const float *u, int32_t n) {
  return logan_hip_host_silu_mul(g, u, n);
}
void coli_metal_tensor_free(ColiMetalTensor *tensor) { logan_hip_tensor_free(tensor); }
void *coli_metal_moe_route_begin(uint64_t model_id, int32_t layer, ColiMetalMatmulDesc *descs,
                                 int32_t count, const float *x, int32_t d, int32_t m) {
  return logan_hip_moe_route_begin(model_id, layer, descs, count, x, d, m);
}
int32_t coli_metal_moe_route_finish(void *pending, float *out, int32_t count) {
  return logan_hip_moe_route_finish(pending, out, count);
}
void coli_metal_moe_route_discard(void *pending) { logan_hip_moe_route_discard(pending); }
void coli_metal_moe_route_drop_model(uint64_t model_id) {
  logan_hip_moe_route_drop_model(model_id);
}
void coli_metal_stats(size_t *tensor_count, size_t *tensor_bytes) {
  logan_hip_stats(tensor_count, tensor_bytes);
}
int coli_metal_mem_info(size_t *used_bytes, size_t *total_bytes) {
  return logan_hip_mem_info(used_bytes, total_bytes);
}
size_t coli_metal_tensor_bytes(const ColiMetalTensor *tensor) {
  return logan_hip_tensor_bytes(tensor);
}

// ---- advisory: weights are copied to HBM on first use, so there is nothing
// to register; nothing is ever wrapped zero-copy

void coli_metal_wrap_stats(uint64_t *calls, uint64_t *zero_copy, uint64_t *copy_bytes,
                           uint64_t *bytes_created) {
  if (calls) *calls = 0;
  if (zero_copy) *zero_copy = 0;
  if (copy_bytes) *copy_bytes = 0;
  if (bytes_created) *bytes_created = 0;
}
void coli_metal_register(void *, size_t) {}
void coli_metal_unregister(void *) {}
int32_t coli_metal_ptr_registered(const void *) { return 0; }

// ---- declining (outside the quantized-decode hot path)

void *logan_metal_shared_surface_wrap(void *, size_t) { return nullptr; }
void logan_metal_shared_surface_free(void *) {}
void *logan_metal_shared_surface_contents(void *) { return nullptr; }
size_t logan_metal_shared_surface_length(void *) { return 0; }
size_t logan_metal_shared_surface_allocation_length(void *) { return 0; }
void *logan_metal_ane_dynamic_pack_create(void *, void *, const uint16_t *, const uint16_t *,
                                          const uint16_t *, const uint16_t *, uint32_t, uint32_t,
                                          uint32_t, uint32_t, uint32_t, uint32_t, uint32_t,
                                          uint32_t, uint32_t, uint32_t,
                                          uint32_t) { return nullptr; }
int32_t logan_metal_ane_dynamic_pack_run(void *, const float *, double *) { return 0; }
void *logan_metal_ane_dynamic_pack_begin(void *, const float *, void *,
                                         uint64_t) { return nullptr; }
int32_t logan_metal_ane_dynamic_pack_finish(void *, double *) { return 0; }
void logan_metal_ane_dynamic_pack_discard(void *) {}
void logan_metal_ane_dynamic_pack_free(void *) {}
void *logan_metal_gdn_conv_silu_create(void *, void *, const float *, size_t, size_t,
                                       size_t) { return nullptr; }
int32_t logan_metal_gdn_conv_silu_run(void *) { return 0; }
void *logan_metal_gdn_conv_silu_begin(void *) { return nullptr; }
int32_t logan_metal_gdn_conv_silu_finish(void *, double *) { return 0; }
void logan_metal_gdn_conv_silu_free(void *) {}
int32_t coli_metal_gdn_mxfp4(uint64_t, int32_t, ColiMetalMatmulDesc *, int32_t, const float *,
                             float *, const float *, const float *, const float *, const float *,
                             float *, float *, int32_t, int32_t, int32_t, int32_t, int32_t, int32_t,
                             int32_t, float) { return 0; }
void coli_metal_gdn_mxfp4_drop_model(uint64_t) {}
int32_t coli_metal_hc_mix(uint64_t, ColiMetalMatmulDesc *, int32_t, const float *, float *, float *,
                          int32_t, int32_t, int32_t) { return 0; }
void coli_metal_hc_drop_model(uint64_t) {}
int32_t coli_metal_spark_layer(uint64_t, int32_t, ColiMetalMatmulDesc *, int32_t, float *,
                               const float *, const float *, int32_t, int32_t, int32_t, int32_t,
                               int32_t, int32_t, int32_t, int32_t, int32_t, float,
                               float) { return 0; }
int32_t coli_metal_spark_token_begin(uint64_t, const float *, int32_t, int32_t) { return 0; }
int32_t coli_metal_spark_layer_encode(uint64_t, int32_t, ColiMetalMatmulDesc *, int32_t,
                                      const float *, const float *, int32_t, int32_t, int32_t,
                                      int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, float,
                                      float) { return 0; }
int32_t coli_metal_spark_token_end(uint64_t, float *, int32_t, int32_t) { return 0; }
int32_t coli_metal_spark_token_end_top1(uint64_t, ColiMetalMatmulDesc *, const float *, uint32_t *,
                                        int32_t, int32_t, int32_t, float) { return 0; }
int32_t coli_metal_spark_token_end_logits(uint64_t, ColiMetalMatmulDesc *, const float *, float *,
                                          int32_t, int32_t, int32_t, float) { return 0; }
void coli_metal_spark_token_abort(uint64_t) {}
int32_t coli_metal_spark_prefill_begin(uint64_t, const float *, int32_t, int32_t,
                                       int32_t) { return 0; }
int32_t coli_metal_spark_prefill_layer_encode(uint64_t, int32_t, ColiMetalMatmulDesc *, int32_t,
                                              const float *, const float *, int32_t, int32_t,
                                              int32_t, int32_t, int32_t, int32_t, int32_t, int32_t,
                                              int32_t, int32_t, float, float) { return 0; }
int32_t coli_metal_spark_prefill_end(uint64_t, int32_t, int32_t) { return 0; }
int32_t coli_metal_spark_prefill_end_logits(uint64_t, ColiMetalMatmulDesc *, const float *, float *,
                                            int32_t, int32_t, int32_t, int32_t,
                                            float) { return 0; }
void coli_metal_spark_prefill_abort(uint64_t) {}
void coli_metal_spark_drop_model(uint64_t) {}
int32_t coli_bnns_bf16_matmul(const uint16_t *, const float *, float *, int32_t,
                              int32_t) { return 0; }
int32_t coli_bnns_bf16_matmul_batch(const uint16_t *, const float *, float *, int32_t, int32_t,
                                    int32_t) { return 0; }
int32_t coli_bnns_f16_matmul(const uint16_t *, const uint16_t *, float *, int32_t,
                             int32_t) { return 0; }
int32_t metalio_init(void) { return 0; }
int32_t metalio_active(void) { return 0; }
void metalio_shutdown(void) {}
int32_t metalio_file_add(const char *) { return -1; }
int32_t metalio_slot_alloc(size_t) { return -1; }
int32_t metalio_slot_alloc_alias(void *, size_t) { return -1; }
void metalio_slot_free(int32_t) {}
void *metalio_slot_ptr(int32_t) { return nullptr; }
size_t metalio_slot_bytes(int32_t) { return 0; }
int64_t metalio_loadv(int32_t, const ColiMetalioRegion *, int32_t, int32_t) { return -1; }
int32_t metalio_wait(int64_t) { return -1; }
int64_t metalio_batch_barrier(void) { return 0; }
int32_t metalio_batch_wait(int64_t, const int32_t *, int32_t) { return -1; }
void metalio_slot_consumed(int32_t) {}
void metalio_prefetch_demanded(int32_t) {}
int32_t metalio_probe(int32_t) { return -1; }
void metalio_stats(ColiMetalioStats *) {}
int32_t coli_apple8_metalio_direct_init(void) { return 0; }
void coli_apple8_metalio_direct_shutdown(void) {}
int32_t coli_apple8_metalio_matmul_slot(int32_t, size_t, size_t, const float *, float *, int32_t,
                                        int32_t, int32_t) { return 0; }
int32_t coli_apple8_metalio_swiglu_slot(int32_t, size_t, size_t, size_t, size_t, size_t, size_t,
                                        const float *, float *, int32_t, int32_t,
                                        int32_t) { return 0; }
int32_t coli_apple8_metalio_moe_rows(const ColiApple8MetalioExpert *, const int32_t *, int32_t,
                                     const float *, float *, int32_t, int32_t,
                                     int32_t) { return 0; }
int32_t coli_apple8_metalio_moe_topk(const ColiApple8MetalioExpert *, const float *, int32_t,
                                     const float *, float *, int32_t, int32_t) { return 0; }
int32_t coli_apple8_metalio_moe_topk_begin(const ColiApple8MetalioExpert *, const float *, int32_t,
                                           const float *, int32_t, int32_t, void **) { return 0; }
int32_t coli_apple8_metalio_moe_topk_finish(void *, float *) { return 0; }
void coli_apple8_metalio_moe_topk_discard(void *) {}
int32_t coli_metal_qwen_attn_decode(const float *, int32_t, int32_t, int32_t, int32_t, int32_t,
                                    float, float *, const float *, const float *) { return 0; }
void coli_apple8_metalio_profile_get(uint64_t *, uint64_t *, uint64_t *, uint64_t *, uint64_t *,
                                     uint64_t *) {}
void coli_apple8_metalio_profile_detail_get(uint64_t *, uint64_t *, uint64_t *, uint64_t *,
                                            uint64_t *, uint64_t *) {}
int32_t coli_apple8_metalio_bf16_matmul(const uint16_t *, const float *, float *, int32_t, int32_t,
                                        int32_t) { return 0; }
void coli_apple8_metalio_gdn_drop_model(uint64_t) {}
void *coli_apple8_metalio_ane_fence_create(uint64_t, void **) { return nullptr; }
int32_t coli_apple8_metalio_ane_fence_set_value(void *, uint64_t) { return 0; }
void *coli_apple8_metalio_ane_fence_metal_event(void *) { return nullptr; }
void coli_apple8_metalio_ane_fence_free(void *) {}
int32_t coli_apple8_metalio_gdn_begin(uint64_t, int32_t, const float *, const uint16_t *,
                                      const uint16_t *, const uint16_t *, const uint16_t *,
                                      const uint16_t *, const float *, const float *, const float *,
                                      const float *, float *, float *, int32_t, int32_t, int32_t,
                                      int32_t, int32_t, int32_t, int32_t, float,
                                      void **) { return 0; }
int32_t coli_apple8_metalio_gdn_ane_begin(uint64_t, int32_t, void *, size_t, void *, size_t, void *,
                                          size_t, void *, size_t, int32_t, const uint16_t *,
                                          const uint16_t *, const uint16_t *, const uint16_t *,
                                          const uint16_t *, const float *, const float *,
                                          const float *, const float *, float *, float *, int32_t,
                                          int32_t, int32_t, int32_t, int32_t, int32_t, int32_t,
                                          float, void *, void **) { return 0; }
int32_t coli_apple8_metalio_gdn_finish(void *, float *) { return 0; }
void coli_apple8_metalio_gdn_discard(void *) {}
int32_t coli_apple8_metalio_gdn_token(uint64_t, int32_t, const float *, float *, const uint16_t *,
                                      const uint16_t *, const uint16_t *, const uint16_t *,
                                      const uint16_t *, const float *, const float *, const float *,
                                      const float *, float *, float *, int32_t, int32_t, int32_t,
                                      int32_t, int32_t, int32_t, int32_t, float) { return 0; }

}  // extern "C"
