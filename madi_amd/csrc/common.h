// common.h -- shared host and device helpers of the gfx950 Q8 matmul library.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "madi_q8.h"

namespace madi {

// ---------------------------------------------------------------- host side
// Records a message for madi_last_error() and returns `code`.
int fail(int code, const char *fmt, ...);
int check_launch(const char *what);
bool initialized();
hipStream_t stream();
// Compute units of the device (256 on an MI355X).
int cu_count();
// The library's split-K workspace: `partial_bytes` of fp32 partial sums and
// `counters` arrival counters that are zero whenever no kernel is using them.
// Grows on demand (a grow waits for the device; an outgrown buffer is kept,
// not freed, because graphs captured earlier still name it); all of them are
// freed by madi_cleanup.
int workspace(size_t partial_bytes, size_t counters, float **partials, uint32_t **cnt);
// Releases the fp16 GEMM's rocBLAS handle (madi_cleanup).
void f16gemm_cleanup();
// The MFMA GEMM with f32 activations (rounded to f16) and an f32 result, for
// the batched projection's many-row calls (gemm.hip); shapes checked by the caller.
int q8_gemm_f32io(const float *in, const void *qs, const void *scales, float *out, uint32_t m,
                  uint32_t n, uint32_t k);
// f16 rows through the batched projection kernel, f16 result (skinny.hip)
int q8_skinny_f16io(const void *in, const void *qs, const void *scales, void *out, uint32_t m,
                    uint32_t n, uint32_t k);
bool skinny_f16_ok(const void *in, const void *qs, const void *out, uint32_t m, uint32_t n,
                   uint32_t k);
bool skinny_f16_prefers_gemm(uint32_t m, uint32_t n, uint32_t k);
// Several outputs of one Q8 GEMM: columns [s*n, (s+1)*n) of the product go to
// c[s] (row pitch n, f16) with bias b[s] -- the encoder's q, k and v
// projections from one stacked weight, launched once into their three
// buffers.  n == 0: a single output.
constexpr int kMaxSegs = 3;
struct OutSeg {
  void *c[kMaxSegs];
  const float *b[kMaxSegs];
  uint32_t n;
};
// madi_q8_gemm into segments (gemm.hip).  Returns kSegUnsupported, having
// launched nothing, where the shape's kernel writes one output only (K split
// across workgroups, the in-workgroup K split, the persistent tile loop) or
// the segment width is not a whole number of the launch's tiles.
constexpr int kSegUnsupported = 1;
int q8_gemm_seg(const void *a, const void *qs, const void *scales, const OutSeg &seg, uint32_t m,
                uint32_t n, uint32_t k, int epilogue);
// Resolves the current device's address of the allocation-free GEMM's fixed
// scratch array and clears its counters (madi_init).
int gemm_scratch_init();

// Deferred dequantisation (boundary.hip).  madi_q8_dequant_f16 records
// (wdq -> Q8 weight) instead of writing wdq; an F16 GEMM whose weight is
// exactly a recorded wdq runs the fused Q8 kernel.  Every entry point calls
// deferred_before_write on the device memory it writes (records whose wdq it
// overwrites are retired; records whose Q8 source it overwrites are
// materialised first) and deferred_before_read on F16 memory it reads other
// than through that lookup (a recorded wdq is materialised first).
// deferred_record returns 1 when it recorded, 0 when deferral is off (the
// caller dequantises now), or an error code.
int deferred_record(void *wdq, const void *qs, const void *sc, uint32_t n, uint32_t k);
bool deferred_lookup(const void *wdq, uint32_t n, uint32_t k, const void **qs, const void **sc);
int deferred_before_write(const void *ptr, size_t bytes);
int deferred_before_read(const void *ptr, size_t bytes);
// madi_free: records whose Q8 source lies in the freed memory are materialised,
// records whose wdq lies in it are dropped.  Returns 1 when it launched a
// dequantisation that reads the memory about to be freed.
int deferred_before_free(const void *ptr, size_t bytes);
// Materialises every record and forgets them (madi_cleanup).
int deferred_flush_all();
// The held q|k|v group (boundary.hip): launched now, if any.
int group_flush();
// The fused route of the F16 GEMM entry points on a recorded wdq: may hold
// the GEMM to launch it together with the next q|k|v slices (boundary.hip).
int fused_gemm(const void *a, const void *qs, const void *sc, void *c, const float *bias, uint32_t m,
               uint32_t n, uint32_t k, int epi);
// Launches the transposed dequantisation Q8 -> F16 [K][N] (layout.hip).
// dequantise into wdq the elements with index in [lo, hi) (layout.hip)
int dequant_launch(void *wdq, const void *qs, const void *sc, uint32_t n, uint32_t k, size_t lo,
                   size_t hi);
// Bytes from p to the end of the live madi_alloc allocation that contains p,
// 0 if no such allocation contains it.
size_t alloc_extent(const void *p);

inline bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ---------------------------------------------------------------- device side
typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Panel layout geometry (see madi_q8.h).
constexpr uint32_t kPanelRows = 32;
constexpr uint32_t kChunkK = 64;

__host__ __device__ inline uint32_t panel_rows(uint32_t n, uint32_t p) {
  uint32_t left = n - p * kPanelRows;
  return left < kPanelRows ? left : kPanelRows;
}
// byte offset of chunk c of panel p in the panel-layout qs buffer
__host__ __device__ inline size_t panel_chunk_qs(uint32_t k, uint32_t p, uint32_t rows,
                                                 uint32_t c) {
  return (size_t)p * kPanelRows * k + (size_t)c * rows * kChunkK;
}
// element offset of chunk c of panel p in the panel-layout scales buffer
__host__ __device__ inline size_t panel_chunk_sc(uint32_t k, uint32_t p, uint32_t rows,
                                                 uint32_t c) {
  return (size_t)p * kPanelRows * (k / 32) + (size_t)c * 2 * rows;
}

// q_pair: two biased bytes (q + 128) of `w`, selected by `sel`, to the exact
// fp16 pair (q0, q1).  The perm builds the fp16 bit patterns 0x64uu = 1024 + u
// for each byte u, so x - 1152 = q exactly.  dequant_pair: times the fp16
// scale pair `s2`; one IEEE fp16 multiply of the exact operands gives
// fp16_rne(q * s), the reference's half(float(q) * float(s))
// (q8_gemm.metal:26) bit for bit.
__device__ inline f16x2 q_pair(uint32_t w, uint32_t sel) {
  const f16x2 bias = {(f16)-1152.0f, (f16)-1152.0f};
  return __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, w, sel)) + bias;
}
__device__ inline f16x2 dequant_pair(uint32_t w, uint32_t sel, f16x2 s2) {
  return q_pair(w, sel) * s2;
}
// byte selectors for v_perm_b32(0x64646464, w, sel): (b0,b1) and (b2,b3)
constexpr uint32_t kSelLo = 0x04010400u;
constexpr uint32_t kSelHi = 0x04030402u;

// 16 biased bytes -> 16 dequantised fp16 (two MFMA k-steps of 8)
__device__ inline void dequant16(const u32x4 &w, f16 s, f16x8 &lo, f16x8 &hi) {
  const f16x2 s2 = {s, s};
  f16x2 a0 = dequant_pair(w.x, kSelLo, s2), a1 = dequant_pair(w.x, kSelHi, s2);
  f16x2 a2 = dequant_pair(w.y, kSelLo, s2), a3 = dequant_pair(w.y, kSelHi, s2);
  f16x2 b0 = dequant_pair(w.z, kSelLo, s2), b1 = dequant_pair(w.z, kSelHi, s2);
  f16x2 b2 = dequant_pair(w.w, kSelLo, s2), b3 = dequant_pair(w.w, kSelHi, s2);
  lo = (f16x8){a0.x, a0.y, a1.x, a1.y, a2.x, a2.y, a3.x, a3.y};
  hi = (f16x8){b0.x, b0.y, b1.x, b1.y, b2.x, b2.y, b3.x, b3.y};
}

// erf-form GELU, Abramowitz & Stegun 7.1.26, the formula of
// engine/metal/kernels/graph_helpers.metal:460-473 and m4_gemm.metal:43-56.
__device__ inline float gelu_erf(float xv) {
  float z = xv * 0.7071067811865476f;
  float az = __builtin_fabsf(z);
  float sign = (z < 0.0f) ? -1.0f : 1.0f;
  float t = 1.0f / __builtin_fmaf(az, 0.3275911f, 1.0f);
  float poly = __builtin_fmaf(1.061405429f, t, -1.453152027f);
  poly = __builtin_fmaf(poly, t, 1.421413741f);
  poly = __builtin_fmaf(poly, t, -0.284496736f);
  poly = __builtin_fmaf(poly, t, 0.254829592f);
  poly = poly * t;
  float ex = exp2f(__builtin_fmaxf(-az * az * 1.4426950408889634f, -80.0f));
  float erf = sign * (1.0f - poly * ex);
  return 0.5f * xv * (1.0f + erf);
}

// The same erf-form GELU in fewer instructions, for epilogues that apply it
// to every element of a tile (128 values per lane in the GEMM): with
// z = x / sqrt(2), 1 / (1 + p|z|) takes p / sqrt(2) against |x| (one FMA and
// the hardware reciprocal, 1 ulp), e^(-z^2) is the hardware exp2 of
// (x * -log2(e) / 2) * x (it returns 0 where that underflows, where
// erf(|z|) is 1 in fp32 anyway), and x/2 (1 + sign(x) erf(|z|)) is
// x/2 + |x/2| erf(|z|), one FMA.  Differs from gelu_erf by a few fp32 ulps,
// far inside one rounding of the f16 result.
__device__ inline float gelu_erf_fast(float xv) {
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(__builtin_fabsf(xv), 0.23164189f, 1.0f));
  float poly = __builtin_fmaf(1.061405429f, t, -1.453152027f);
  poly = __builtin_fmaf(poly, t, 1.421413741f);
  poly = __builtin_fmaf(poly, t, -0.284496736f);
  poly = __builtin_fmaf(poly, t, 0.254829592f);
  poly = poly * t;
  const float ex = __builtin_amdgcn_exp2f((xv * -0.72134752044448170f) * xv);
  const float erf_abs = __builtin_fmaf(-poly, ex, 1.0f);  // erf(|z|)
  const float hx = 0.5f * xv;
  return __builtin_fmaf(__builtin_fabsf(hx), erf_abs, hx);
}

}  // namespace madi
