// f16gemm.hip -- the boundary's plain fp16 GEMMs on pre-dequantised weights.
//
// The engine keeps F16 GEMM entry points for callers that hold an F16 weight
// (the encoder's F16 cache, the batched decode's WF16 copy): kM4 / kM4Bias
// (engine/metal/encoder.zig:125-136 -> m4_gemm_nn / m4_gemm_bias /
// m4_gemm_bias_gelu, kernels/m4_gemm.metal:19-115) and matmulF16Batched
// (metal_backend.zig:120 -> mtl_matmul_f16_enc, metal_backend.h:103).  These
// are plain library GEMMs: rocBLAS gemm_ex with f16 operands and fp32
// accumulation, on the library's stream.  The bias epilogues follow the
// reference's kernels, which round the product to f16 first and then add the
// f32 bias (and apply GELU) in one elementwise pass over the f16 result.
#include <rocblas/rocblas.h>

#include "common.h"

namespace madi {

namespace {
rocblas_handle g_blas = nullptr;

int blas(rocblas_handle *h, const char *what) {
  if (!g_blas && rocblas_create_handle(&g_blas) != rocblas_status_success) {
    g_blas = nullptr;
    return fail(MADI_ERR_INIT, "%s: rocblas_create_handle failed", what);
  }
  if (rocblas_set_stream(g_blas, stream()) != rocblas_status_success)
    return fail(MADI_ERR_DISPATCH, "%s: rocblas_set_stream failed", what);
  *h = g_blas;
  return MADI_OK;
}

// C[M][N] = alpha * A[M][K] . B[K][N] + beta * C, all row-major f16: the
// column-major product C^T = B^T A^T with the operands as stored.
int gemm_f16(const char *what, const void *a, const void *b, void *c, uint32_t m, uint32_t n,
             uint32_t k, float alpha, float beta) {
  rocblas_handle h;
  if (int rc = blas(&h, what)) return rc;
  const rocblas_status st = rocblas_gemm_ex(
      h, rocblas_operation_none, rocblas_operation_none, (rocblas_int)n, (rocblas_int)m,
      (rocblas_int)k, &alpha, b, rocblas_datatype_f16_r, (rocblas_int)n, a, rocblas_datatype_f16_r,
      (rocblas_int)k, &beta, c, rocblas_datatype_f16_r, (rocblas_int)n, c, rocblas_datatype_f16_r,
      (rocblas_int)n, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (st != rocblas_status_success)
    return fail(MADI_ERR_DISPATCH, "%s: rocblas_gemm_ex failed (%s)", what, rocblas_status_to_string(st));
  return MADI_OK;
}

// C[M][N] (f32) = A[M][K] (f16) . B[K][N] (f16), row-major, fp32 accumulation
// (rocBLAS with f16 inputs and an f32 result).
int gemm_f16_f32out(const char *what, const void *a, const void *b, float *c, uint32_t m,
                    uint32_t n, uint32_t k) {
  rocblas_handle h;
  if (int rc = blas(&h, what)) return rc;
  const float alpha = 1.0f, beta = 0.0f;
  const rocblas_status st = rocblas_gemm_ex(
      h, rocblas_operation_none, rocblas_operation_none, (rocblas_int)n, (rocblas_int)m,
      (rocblas_int)k, &alpha, b, rocblas_datatype_f16_r, (rocblas_int)n, a, rocblas_datatype_f16_r,
      (rocblas_int)k, &beta, c, rocblas_datatype_f32_r, (rocblas_int)n, c, rocblas_datatype_f32_r,
      (rocblas_int)n, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (st != rocblas_status_success)
    return fail(MADI_ERR_DISPATCH, "%s: rocblas_gemm_ex failed (%s)", what, rocblas_status_to_string(st));
  return MADI_OK;
}

// The operands the fused Q8 GEMM needs (16-byte aligned A, C and bias, whole
// 32-row panels, K a multiple of 64, and madi_q8_gemm's 32-bit buffer limits:
// A, W and one 128-row C tile below 2 GiB); otherwise a recorded weight is
// materialised and the library GEMM runs.
inline bool fusable(const void *a, const void *c, const float *bias, uint32_t m, uint32_t n,
                    uint32_t k) {
  return aligned(a, 16) && aligned(c, 16) && (!bias || aligned(bias, 16)) && n % kPanelRows == 0 &&
         k % kChunkK == 0 && (uint64_t)m * k * 2 < (1ull << 31) && (uint64_t)n * k < (1ull << 31) &&
         (uint64_t)n * 256 < (1ull << 31);
}

// dst[i] = f16(src[i]) (round to nearest even), the engine's f32 -> f16 staging
__global__ __launch_bounds__(256) void to_f16_kernel(f16 *__restrict__ dst,
                                                     const float *__restrict__ src, size_t count) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) dst[i] = (f16)src[i];
}

// c[r][col] = f16(epi(float(c[r][col]) + bias[col])), m4_gemm.metal:79-85 / 108-114
template <bool GELU>
__global__ __launch_bounds__(256) void bias_epilogue_kernel(f16 *__restrict__ c,
                                                            const float *__restrict__ bias,
                                                            uint32_t n, size_t count) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  float v = (float)c[i] + bias[i % n];
  if constexpr (GELU) v = gelu_erf(v);
  c[i] = (f16)v;
}
}  // namespace

void f16gemm_cleanup() {
  if (g_blas) (void)rocblas_destroy_handle(g_blas);
  g_blas = nullptr;
}

}  // namespace madi

using namespace madi;

extern "C" int madi_f16_gemm(const void *a, const void *b, void *c, const float *bias, uint32_t m,
                             uint32_t n, uint32_t k, int epilogue) {
  if (!a || !b || !c) return fail(MADI_ERR_NULL, "madi_f16_gemm: null pointer");
  if (epilogue != MADI_EPI_NONE && epilogue != MADI_EPI_BIAS && epilogue != MADI_EPI_BIAS_GELU)
    return fail(MADI_ERR_ARG, "madi_f16_gemm: unknown epilogue %d", epilogue);
  if (epilogue != MADI_EPI_NONE && !bias) return fail(MADI_ERR_NULL, "madi_f16_gemm: null bias");
  if (m == 0 || n == 0 || k == 0 || m > 0x7fffffffu || n > 0x7fffffffu || k > 0x7fffffffu)
    return fail(MADI_ERR_SHAPE, "madi_f16_gemm: m=%u n=%u k=%u", m, n, k);
  if (!aligned(a, 2) || !aligned(b, 2) || !aligned(c, 2) || (bias && !aligned(bias, 4)))
    return fail(MADI_ERR_ALIGN, "madi_f16_gemm: misaligned operand");
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_f16_gemm: madi_init has not succeeded");
  // b is the F16 [K][N] that kDeq recorded for a Q8 weight [N][K]: the fused Q8
  // GEMM runs on that weight (one rounding of acc + bias, the Q8-direct
  // kernel's epilogue, m4_gemm.metal:180-186) and b is never written
  const void *qs, *sc;
  if (fusable(a, c, bias, m, n, k) && deferred_lookup(b, n, k, &qs, &sc))
    return fused_gemm(a, qs, sc, c, bias, m, n, k, epilogue);
  if (int rc = deferred_before_read(a, (size_t)m * k * 2)) return rc;
  if (int rc = deferred_before_read(b, (size_t)k * n * 2)) return rc;
  if (int rc = deferred_before_write(c, (size_t)m * n * 2)) return rc;
  if (int rc = gemm_f16("madi_f16_gemm", a, b, c, m, n, k, 1.0f, 0.0f)) return rc;
  if (epilogue == MADI_EPI_NONE) return MADI_OK;
  const size_t count = (size_t)m * n;
  const dim3 grid((unsigned)((count + 255) / 256));
  if (epilogue == MADI_EPI_BIAS)
    hipLaunchKernelGGL(bias_epilogue_kernel<false>, grid, dim3(256), 0, stream(),
                       static_cast<f16 *>(c), bias, n, count);
  else
    hipLaunchKernelGGL(bias_epilogue_kernel<true>, grid, dim3(256), 0, stream(),
                       static_cast<f16 *>(c), bias, n, count);
  return check_launch("madi_f16_gemm(epilogue)");
}

extern "C" int madi_matmul_f16(const void *a, const void *b, void *c, int m, int n, int k,
                               float alpha, float beta) {
  if (!a || !b || !c) return fail(MADI_ERR_NULL, "madi_matmul_f16: null pointer");
  if (m <= 0 || n <= 0 || k <= 0)
    return fail(MADI_ERR_SHAPE, "madi_matmul_f16: m=%d n=%d k=%d", m, n, k);
  if (!aligned(a, 2) || !aligned(b, 2) || !aligned(c, 2))
    return fail(MADI_ERR_ALIGN, "madi_matmul_f16: misaligned operand");
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_matmul_f16: madi_init has not succeeded");
  // b is the F16 [K][N] copy deqW16 recorded for a Q8 weight [N][K]: the
  // product runs from the Q8 weight and b is never written.  Few rows (the
  // batched decode's logits, B = 8 or 16 over the vocab's 51866 rows,
  // transcribe.zig:2391-2394) take the batched projection kernel, which
  // handles any N; many rows on whole panels (the cross-attention K and V of
  // the encoder output, transcribe.zig:2440-2448) the fused GEMM.
  const void *qs, *sc;
  const uint32_t um = (uint32_t)m, un = (uint32_t)n, uk = (uint32_t)k;
  if (alpha == 1.0f && beta == 0.0f && deferred_lookup(b, un, uk, &qs, &sc)) {
    if (skinny_f16_prefers_gemm(um, un, uk) && fusable(a, c, nullptr, um, un, uk))
      return madi_q8_gemm(a, qs, sc, c, nullptr, um, un, uk, MADI_EPI_NONE);
    if (skinny_f16_ok(a, qs, c, um, un, uk)) {
      if (int rc = deferred_before_read(a, (size_t)um * uk * 2)) return rc;
      if (int rc = deferred_before_write(c, (size_t)um * un * 2)) return rc;
      return q8_skinny_f16io(a, qs, sc, c, um, un, uk);
    }
  }
  const size_t mn = (size_t)m * n * 2;
  if (int rc = deferred_before_read(a, (size_t)m * k * 2)) return rc;
  if (int rc = deferred_before_read(b, (size_t)k * n * 2)) return rc;
  if (beta != 0.0f)
    if (int rc = deferred_before_read(c, mn)) return rc;
  if (int rc = deferred_before_write(c, mn)) return rc;
  return gemm_f16("madi_matmul_f16", a, b, c, (uint32_t)m, (uint32_t)n, (uint32_t)k, alpha, beta);
}

extern "C" int madi_proj_f16w(float *out, const float *in, const void *w16, void *stage16,
                              uint32_t m, uint32_t n, uint32_t k) {
  if (!out || !in || !w16) return fail(MADI_ERR_NULL, "madi_proj_f16w: null pointer");
  if (m == 0 || n == 0 || k == 0 || m > 0x7fffffffu || n > 0x7fffffffu || k > 0x7fffffffu)
    return fail(MADI_ERR_SHAPE, "madi_proj_f16w: m=%u n=%u k=%u", m, n, k);
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_proj_f16w: madi_init has not succeeded");
  // w16 is a recorded F16 copy of a Q8 weight (deqW16 at decode start): the
  // batched projection runs from the Q8 weight, one kernel
  const void *qs, *sc;
  if (aligned(in, 16) && aligned(out, 4) && deferred_lookup(w16, n, k, &qs, &sc))
    return madi_q8_pproj(out, in, qs, sc, m, n, k);
  // a true F16 weight: the reference's f32 -> f16 staging, then an f16 GEMM
  // with an f32 result
  if (!stage16) return fail(MADI_ERR_NULL, "madi_proj_f16w: null staging buffer for an F16 weight");
  if (!aligned(w16, 2) || !aligned(stage16, 2) || !aligned(in, 4) || !aligned(out, 4))
    return fail(MADI_ERR_ALIGN, "madi_proj_f16w: misaligned operand");
  const size_t count = (size_t)m * k;
  if (int rc = deferred_before_read(in, count * 4)) return rc;
  if (int rc = deferred_before_read(w16, (size_t)k * n * 2)) return rc;
  if (int rc = deferred_before_write(stage16, count * 2)) return rc;
  if (int rc = deferred_before_write(out, (size_t)m * n * 4)) return rc;
  hipLaunchKernelGGL(to_f16_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream(),
                     static_cast<f16 *>(stage16), in, count);
  if (int rc = check_launch("madi_proj_f16w(stage)")) return rc;
  return gemm_f16_f32out("madi_proj_f16w", stage16, w16, out, m, n, k);
}
