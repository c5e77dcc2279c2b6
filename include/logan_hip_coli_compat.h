/*
 * logan-metal C symbol names exported by liblogan_hip.so for the subset of
 * backend_metal.h this library implements. Each forwards to the logan_hip_*
 * entry point of the same meaning (include/logan_hip.h), so the FFI block in
 * logan-metal/src/lib.rs (:198-460) links against this library unchanged.
 * ColiMetalTensor is LoganHipTensor; ColiMetalMatmulDesc has the layout of
 * LoganHipMatmulDesc (backend_metal.h:68-88).
 */
#ifndef LOGAN_HIP_COLI_COMPAT_H
#define LOGAN_HIP_COLI_COMPAT_H

#include "logan_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

int coli_metal_init(void);                                       /* backend_metal.h:22 */
int coli_metal_available(void);                                  /* backend_metal.h:35 */
void coli_metal_shutdown(void);                                  /* backend_metal.h:34 */
void coli_metal_stats(size_t *tensor_count, size_t *tensor_bytes); /* backend_metal.h:37 */
int coli_metal_mem_info(size_t *used_bytes, size_t *total_bytes); /* backend_metal.h:38 */
void coli_metal_profile_set_on(int on);                          /* backend_metal.h:42 */
void coli_metal_profile_reset(void);                             /* backend_metal.h:43 */
void coli_metal_profile_get(uint64_t *encode_ns, uint64_t *submit_ns, uint64_t *wait_ns,
                            uint64_t *kernel_ns);                /* backend_metal.h:44-45 */
int coli_metal_matmul(LoganHipTensor **tensor, float *y, const float *x, const void *weights,
                      const float *scales, int fmt, int S, int I, int O,
                      int gs);                                   /* backend_metal.h:63-66 */
int coli_metal_matmul_multi(const float *x, int S, LoganHipMatmulDesc *descs,
                            int count);                          /* backend_metal.h:100-101 */
void *coli_metal_moe_route_begin(uint64_t model_id, int layer, LoganHipMatmulDesc *descs,
                                 int count, const float *x, int D, int M); /* backend_metal.h:163-165 */
int coli_metal_moe_route_finish(void *pending, float *out, int count); /* backend_metal.h:166 */
void coli_metal_moe_route_discard(void *pending);                /* backend_metal.h:167 */
void coli_metal_moe_route_drop_model(uint64_t model_id);         /* backend_metal.h:168 */
int coli_metal_shared_mxfp4(uint64_t model_id, int layer, LoganHipMatmulDesc *descs, int count,
                            const float *x, float *out, int D, int Iinter); /* backend_metal.h:146-148 */
void coli_metal_shared_mxfp4_drop_model(uint64_t model_id);      /* backend_metal.h:149 */
void coli_metal_tensor_free(LoganHipTensor *tensor);             /* backend_metal.h:180 */
size_t coli_metal_tensor_bytes(const LoganHipTensor *tensor);    /* backend_metal.h:181 */

#ifdef __cplusplus
}
#endif
#endif
