/*
 * issue.c -- a compiled issue loop over the C ABI (libmadi_issue.so).
 *
 * The engine issues its operator calls from compiled code: the decode loop
 * (engine/metal/transcribe.zig:2783-2800), the batched decode step (:2380-2400)
 * and the encoder's layer loop (engine/metal/encoder.zig:256-303) are Zig.
 * A Python loop over the same calls measures the interpreter as much as the
 * GPU (each ctypes call costs a few microseconds of host time, about the GPU
 * time of a small decoder projection).  This file replays a call list that
 * the caller builds once -- one record per library call, with the call's
 * arguments -- `reps` times from C, so a measured sequence is issued at the
 * rate compiled code issues it.  It adds no operation of its own.
 */
#include <stddef.h>
#include <stdint.h>

#include "madi_q8.h"

enum {
  ISSUE_GEMV = 0,        /* madi_q8_gemv(out, x, qs, sc, n, k)                      */
  ISSUE_GEMV_BIAS = 1,   /* madi_q8_gemv_bias(out, x, qs, sc, bias, n, k)           */
  ISSUE_GEMV_EPI = 2,    /* madi_q8_gemv_epi(f, out, x, qs, sc, bias, n, k)         */
  ISSUE_QKV = 3,         /* madi_q8_gemv_qkv(q, x, qs, sc, qb, vb, kc, vc, pos, d)  */
  ISSUE_LOGIT = 4,       /* madi_q8_logit_gemv(logits, qs, sc, x, vocab, dim)       */
  ISSUE_PPROJ = 5,       /* madi_q8_pproj(out, in, qs, sc, m, n, k)                 */
  ISSUE_DEQ = 6,         /* madi_q8_dequant_f16(wdq, qs, sc, n, k)                  */
  ISSUE_M4 = 7,          /* madi_m4_gemm(f, a, b, c, bias, m, n, k)                 */
  ISSUE_Q8_GEMM = 8,     /* madi_q8_gemm(a, qs, sc, c, bias, m, n, k, epi)          */
  ISSUE_MATMUL_F16 = 9,  /* madi_matmul_f16(a, b, c, m, n, k, 1, 0)                 */
  ISSUE_FLASH = 10,      /* madi_flash_enc_f16(out, q, k, v, seq, nh)               */
};

/* One call: its kind and up to ten arguments in declaration order (pointers
 * and sizes alike widened to 64 bits). */
typedef struct {
  int32_t op;
  int32_t pad;
  uint64_t a[10];
} madi_issue_op;

#define P(i) ((void *)(uintptr_t)o->a[i])
#define F(i) ((float *)(uintptr_t)o->a[i])
#define U(i) ((uint32_t)o->a[i])

static int issue_one(const madi_issue_op *o) {
  switch (o->op) {
  case ISSUE_GEMV: return madi_q8_gemv(F(0), F(1), P(2), P(3), U(4), U(5));
  case ISSUE_GEMV_BIAS: return madi_q8_gemv_bias(F(0), F(1), P(2), P(3), F(4), U(5), U(6));
  case ISSUE_GEMV_EPI:
    return madi_q8_gemv_epi((int)o->a[0], F(1), F(2), P(3), P(4), F(5), U(6), U(7));
  case ISSUE_QKV:
    return madi_q8_gemv_qkv(F(0), F(1), P(2), P(3), F(4), F(5), F(6), F(7),
                            (const uint32_t *)P(8), U(9));
  case ISSUE_LOGIT: return madi_q8_logit_gemv(F(0), P(1), P(2), F(3), U(4), U(5));
  case ISSUE_PPROJ: return madi_q8_pproj(F(0), F(1), P(2), P(3), U(4), U(5), U(6));
  case ISSUE_DEQ: return madi_q8_dequant_f16(P(0), P(1), P(2), U(3), U(4));
  case ISSUE_M4: return madi_m4_gemm((int)o->a[0], P(1), P(2), P(3), F(4), U(5), U(6), U(7));
  case ISSUE_Q8_GEMM:
    return madi_q8_gemm(P(0), P(1), P(2), P(3), F(4), U(5), U(6), U(7), (int)o->a[8]);
  case ISSUE_MATMUL_F16:
    return madi_matmul_f16(P(0), P(1), P(2), (int)o->a[3], (int)o->a[4], (int)o->a[5], 1.0f, 0.0f);
  case ISSUE_FLASH: return madi_flash_enc_f16(P(0), P(1), P(2), P(3), U(4), U(5));
  default: return MADI_ERR_ARG;
  }
}

/* Issue ops[0..n) in order, `reps` times.  Returns 0, or the first failing
 * call's return code with its index (rep * n + i) in *failed_at. */
int madi_issue_run(const madi_issue_op *ops, int n, int reps, int64_t *failed_at) {
  for (int r = 0; r < reps; ++r)
    for (int i = 0; i < n; ++i) {
      const int rc = issue_one(&ops[i]);
      if (rc != MADI_OK) {
        if (failed_at) *failed_at = (int64_t)r * n + i;
        return rc;
      }
    }
  return MADI_OK;
}
