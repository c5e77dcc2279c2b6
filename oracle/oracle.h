/*
 * CPU oracle for the logan-hip quantized-decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference
 * (mateocabanal/logan) CPU arithmetic for the MLX-affine dequant-GEMV and the
 * routed-MoE block. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or the reported CPU
 * baseline. The shipped library never calls into it.
 *
 * Every function names the reference file:line it follows. The reference is
 * Rust; Rust f32 arithmetic is IEEE single precision without contraction, so
 * this file is compiled with -ffp-contract=off and no fast-math.
 */
#ifndef LOGAN_ORACLE_H
#define LOGAN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* logan-qwen4/src/ggufsource.rs:1968-1991 (IEEE fp16 -> f32, exact). */
float lo_f16_to_f32(uint16_t bits);
/* logan-core/src/math.rs:279-283 (f32 -> bf16 bits, round-to-nearest-even). */
uint16_t lo_f32_to_bf16(float f);
/* logan-core/src/math.rs:289-291 (bf16 bits -> f32, exact). */
float lo_bf16_to_f32(uint16_t b);

/* logan-qwen4/src/lib.rs:3688-3701: code of `column` in one packed row. */
uint32_t lo_affine_code(const uint8_t *row, size_t column, int bits);
/* logan-qwen4/src/lib.rs:3678-3686: scale/bias element `index` (bf16 or fp16). */
float lo_affine_param(const uint8_t *bytes, size_t index, int fp16);

/* logan-qwen4/src/lib.rs:3703-3727 and src/colisource.rs:779-856: dequantised
 * rows [row0, row0+nrows) into out[nrows*cols]. Returns 0 on success, -1 on an
 * invalid geometry (colisource.rs:788-833 error cases). */
int lo_affine_dequant(float *out, const uint8_t *w, const uint8_t *scales,
                      const uint8_t *biases, size_t rows, size_t cols, int bits,
                      size_t group_size, int fp16, size_t row0, size_t nrows);

/* logan-qwen4/src/lib.rs:3729-3764: y[o] = sum_j w[o,j] x[j], sequential f32
 * sum in column order, single thread. */
void lo_affine_gemv(float *y, const float *x, const uint8_t *w,
                    const uint8_t *scales, const uint8_t *biases, size_t o,
                    size_t i, int bits, size_t group_size, int fp16);
/* Same arithmetic per row, rows split over `threads` workers as the reference
 * splits rows over threads (logan-qwen4/src/lib.rs:3785-3807). */
void lo_affine_gemv_mt(float *y, const float *x, const uint8_t *w,
                       const uint8_t *scales, const uint8_t *biases, size_t o,
                       size_t i, int bits, size_t group_size, int fp16,
                       int threads);

/* logan-spark/src/lib.rs:346-367: affine-8, group 64, aux = [bf16 scales]
 * [bf16 biases]; per group acc += sc*dot + bi*xsum[g]; y rounded to bf16
 * (returned as the rounded f32 value, lib.rs:254-258). */
void lo_spark_affine8_gemv(float *y, const float *x, const uint8_t *w,
                           const uint8_t *aux, size_t o, size_t i);

/* logan-metal/metal/backend_metal.mm:1480-1560: prefill product with the
 * dequantised weights rounded to bf16, f32 accumulation; y[m][o]. */
void lo_affine_qmm_bf16(float *y, const float *x, const uint8_t *w,
                        const uint8_t *scales, const uint8_t *biases, size_t m,
                        size_t o, size_t i, int bits, size_t group_size,
                        int fp16);

/* logan-qwen4/src/lib.rs:4516-4518. */
float lo_mxfp4_value(uint8_t code, uint8_t scale_byte);
void lo_mxfp4_gemv(float *y, const float *x, const uint8_t *w, const uint8_t *sc, size_t o,
                   size_t i);
void lo_mxfp4_gemv_stacked(float *y, const float *x, const uint8_t *w, const uint8_t *sc,
                           size_t o, size_t i, int stacks);
/* logan-llama/src/model.rs:1025-1033 over bf16-valued weights (fmt 5 raw
 * bf16, fmt 15 affine-8 g64 rounded to bf16). */
void lo_dense_gemv(float *y, const float *x, const void *w, const uint16_t *sc,
                   const uint16_t *bi, int fmt, size_t O, size_t I);
/* logan-llama/src/model.rs:786-905, one token at position pos. */
int lo_llama_layer(float *x, float *kc, float *vc, int pos, const void *const *w,
                   const uint16_t *const *sc, const uint16_t *const *bi, const int *fmt,
                   const float *in_norm, const float *post_norm, int D, int inter, int H, int KH,
                   int hd, float theta, float eps);
void lo_rmsnorm(float *x, const float *w, size_t n, size_t nrows, float eps);
void lo_add(float *y, const float *a, size_t n);
float lo_silu(float x);
void lo_silu_mul(float *g, const float *u, size_t n);
/* logan-qwen4/src/lib.rs:4558-4574 (= logan-qwen/src/lib.rs:260-276). */
void lo_softmax_row(float *x, size_t n);
/* logan-qwen4/src/lib.rs:7993-8043 (= logan-qwen/src/lib.rs:545-557):
 * selection top-k on probabilities with lower-index ties. `probs` is
 * softmax output [n]; writes idx[k], val[k] in rank order; returns
 * wsum = sum val[0..k) in rank order. */
float lo_topk(const float *probs, size_t n, size_t k, int32_t *idx, float *val);

/* One routed-MoE block for one token (logan-qwen/src/lib.rs:535-593,
 * logan-qwen4/src/lib.rs:8758-8815 + :8692-8711 + :7597-7759):
 *   probs = softmax(logits); top-k; per rank r: h = silu(gate.x) * (up.x);
 *   y = down.h; acc += y * (val[r]/wsum); shared: gs = sigmoid(se_g.x),
 *   sy = se_down(silu(se_gate.x) * se_up.x); out = acc + sy*gs.
 * Expert banks are MLX switch_mlp stacks: expert e of a bank with O rows and
 * I columns starts at weights + e*O*(I*bits/8), params at e*O*(I/gs)
 * (logan-qwen4/src/lib.rs:12001-12019). se_g is f32 [D] (NULL: no shared
 * expert; then out = acc). */
typedef struct lo_bank {
  const uint8_t *w, *scales, *biases;
  size_t o, i;
  int bits;
  size_t group_size;
  int fp16;
} lo_bank;

void lo_moe_token(float *out, const float *x, const float *logits, size_t E,
                  size_t k, size_t D, const lo_bank *gate, const lo_bank *up,
                  const lo_bank *down, const lo_bank *se_gate,
                  const lo_bank *se_up, const lo_bank *se_down,
                  const float *se_g, int32_t *idx_out, float *w_out);

/* Row-threaded variant of lo_moe_token for the CPU baseline: every GEMV's rows
 * are split over `threads` workers; the reduction order per row is unchanged. */
void lo_moe_token_mt(float *out, const float *x, const float *logits, size_t E,
                     size_t k, size_t D, const lo_bank *gate, const lo_bank *up,
                     const lo_bank *down, const lo_bank *se_gate,
                     const lo_bank *se_up, const lo_bank *se_down,
                     const float *se_g, int32_t *idx_out, float *w_out,
                     int threads);

#ifdef __cplusplus
}
#endif
#endif
