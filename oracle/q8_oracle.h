/*
 * q8_oracle.h -- CPU restatement of the reference's Q8 matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only to check
 * results (or, for bench.py, as the timed restated-reference CPU path).  The product
 * library (madi_amd) never links, loads or calls it.
 *
 * Every routine works on the reference's NATURAL Q8_0 layout:
 *   qs     int8  [N][K]      row-major, out-major (= safetensors [out][in])
 *   scales fp16  [N][K/32]   one scale per 32-element K block
 *   w[n][k] = qs[n*K + k] * scales[n*(K/32) + k/32]
 * (reference: engine/metal/encoder.zig:21, engine/metal/decoder.zig:22).
 *
 * fp16 values travel as their uint16_t bit patterns.
 *
 * Parity pins (what checks each function; see tests/test_oracle.py):
 *   f16 <-> f32 conversion ...... exhaustive against numpy's float16 casts
 *   dequant ..................... exhaustive q x scale grid against numpy
 *   gemm / gemv ................. fp64 accumulation bound, K=32 closed form,
 *                                 one-hot and all-ones inputs, brute force on
 *                                 the reference's 50x64x96 case, planted-
 *                                 mistake mutants
 *   gelu_erf .................... math.erf (A&S 7.1.26 error bound 1.5e-7)
 *   quantize .................... round-half-away knife edges, |q|<=127,
 *                                 block max maps to 127, all-zero block -> 1.0
 *   fnv1a64 ..................... published FNV-1a 64-bit test vectors
 *   flash_enc ................... fp64 softmax attention within the bound the
 *                                 f16 rounding of P allows, uniform attention
 *                                 (q = 0) = mean of the value rows, one-hot
 *                                 peaked attention, key-order and head
 *                                 independence, planted-mistake mutants
 */
#ifndef MADI_Q8_ORACLE_H
#define MADI_Q8_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ORACLE_EPI_NONE = 0,
  ORACLE_EPI_BIAS = 1,
  ORACLE_EPI_BIAS_GELU = 2,
  ORACLE_EPI_BIAS_RES = 3
};

float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
void oracle_f16_to_f32_array(float *dst, const uint16_t *src, size_t n);
void oracle_f32_to_f16_array(uint16_t *dst, const float *src, size_t n);

float oracle_gelu_erf(float x);

void oracle_dequant_q8_f16(uint16_t *out_kn, const int8_t *qs, const uint16_t *scales,
                           uint32_t n, uint32_t k);

void oracle_q8_gemm_rows(float *c_rows, const uint16_t *a, const int8_t *qs,
                         const uint16_t *scales, const float *bias, int epilogue,
                         uint32_t m, uint32_t n, uint32_t k, const uint32_t *rows,
                         uint32_t n_rows, int threads);

void oracle_q8_gemm_f16(uint16_t *c, const uint16_t *a, const int8_t *qs,
                        const uint16_t *scales, const float *bias, int epilogue,
                        uint32_t m, uint32_t n, uint32_t k, int threads);

void oracle_q8_gemv(float *out, const float *x, const int8_t *qs, const uint16_t *scales,
                    const float *bias, int epilogue, uint32_t n, uint32_t k, int threads);

void oracle_q8_gemv_qkv(float *q_out, const float *x, const int8_t *qs,
                        const uint16_t *scales, const float *qb, const float *vb,
                        float *kc, float *vc, uint32_t pos, uint32_t d);

void oracle_q8_proj(float *out, const float *in, const int8_t *qs, const uint16_t *scales,
                    uint32_t m, uint32_t n, uint32_t k, int threads);

void oracle_quantize_q8(int8_t *qs, uint16_t *scales, const uint16_t *w_f16,
                        uint32_t rows, uint32_t dim);

uint64_t oracle_fnv1a64(uint64_t seed, const uint8_t *bytes, size_t n);
uint64_t oracle_fnv_q8(uint64_t seed, const int8_t *qs, size_t nq, const uint16_t *scales,
                       size_t nsc);

void oracle_emb_row_q8(float *out, const int8_t *qs, const uint16_t *scales, uint32_t tok,
                       uint32_t dim);
/* decoder_ops.metal:614-633 emb_pe_rows_q8: rows tokens[0..m) of the natural-layout
 * table plus positional rows pos0..pos0+m-1 of pe ([*][dim] f32). */
void oracle_emb_pe_rows_q8(float *out, const int8_t *qs, const uint16_t *scales,
                           const uint32_t *tokens, const float *pe, uint32_t dim, uint32_t pos0,
                           uint32_t m);

void oracle_gemm_f16(uint16_t *c, const uint16_t *a, const uint16_t *b, uint32_t m,
                     uint32_t n, uint32_t k, float alpha, float beta, int threads);

/* m4_gemm.metal:268-407 m4_flash_enc: bidirectional attention, head dim 64, over
 * q, k, v f16 [seq][nh*64] (head hd in columns hd*64..), f16 out of the same shape. */
void oracle_flash_enc_f16(uint16_t *out, const uint16_t *q, const uint16_t *k,
                          const uint16_t *v, uint32_t seq, uint32_t nh, int threads);

#ifdef __cplusplus
}
#endif
#endif
