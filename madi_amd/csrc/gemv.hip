// gemv.hip -- decoder Q8 GEMV family (M = 1), HBM-bound.
//
// Replaces gemv_q8 / _bias / _bias_gelu / _bias_res / _qkv and logit_gemv_q8
// (engine/metal/kernels/graph_helpers.metal:320-558).  The reference runs one
// 32-lane simdgroup per output row reading char4 + float4; here a 256-thread
// workgroup streams two 32-row panels of the panel layout: every wave64 load
// instruction moves one contiguous KiB (16 bytes per lane, 128-bit loads) and
// each lane (h, r) accumulates the 32-weight block of row r, K-half h, of each
// 64-wide chunk.  The four waves split K; the two K-halves meet with one
// cross-lane shuffle and the four waves through LDS.
//
// Activations are staged once per workgroup in LDS as f32 and read as broadcast
// 128-bit LDS loads shared by both panels.  The stored bytes are u = q + 128:
// per block the lane forms sum_i x_i * u_i - 128 * sum_i x_i (the x sums are
// staged with x), then multiplies by the block's scale, the same
// (partial * scale) structure as the reference's kernels.
#include "common.h"

using namespace madi;

namespace {

#ifndef MADI_GEMV_PPW
#define MADI_GEMV_PPW 1
#endif
#ifndef MADI_GEMV_UNROLL
#define MADI_GEMV_UNROLL 5
#endif
constexpr int kPanelsPerWG = MADI_GEMV_PPW;
constexpr int kUnroll = MADI_GEMV_UNROLL;  // chunks whose loads are in flight together
constexpr uint32_t kMaxK = 12288;

enum GemvMode { kPlain = 0, kBias = 1, kBiasGelu = 2, kBiasRes = 3, kQkv = 4 };

struct GemvArgs {
  float *out;
  const void *x;
  const uint8_t *qs;
  const f16 *sc;
  const float *bias;
  uint32_t n, k;
  // QKV epilogue (graph_helpers.metal:527-558)
  const float *qb, *vb;
  float *kc, *vc;
  const uint32_t *pos;
};

__device__ inline float byte_f(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xffu); }

struct Batch {
  u32x4 w[kUnroll][kPanelsPerWG][2];
  f16 s[kUnroll][kPanelsPerWG];
};

// Issue the loads of chunks [c, min(c + kUnroll, c1)) of the workgroup's panels.
__device__ inline void load_batch(Batch &b, const GemvArgs &a, uint32_t K, uint32_t c,
                                  uint32_t c1, uint32_t p0, const uint32_t *R, const bool *live,
                                  uint32_t h, uint32_t r) {
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
#pragma unroll
    for (int t = 0; t < kPanelsPerWG; ++t) {
      if (c + u < c1 && live[t]) {
        const uint32_t p = p0 + t, Rt = R[t];
        const uint8_t *blk = a.qs + panel_chunk_qs(K, p, Rt, c + u);
        b.w[u][t][0] = *reinterpret_cast<const u32x4 *>(blk + (h * Rt + r) * 16);
        b.w[u][t][1] = *reinterpret_cast<const u32x4 *>(blk + ((2 + h) * Rt + r) * 16);
        b.s[u][t] = a.sc[panel_chunk_sc(K, p, Rt, c + u) + h * Rt + r];
      }
    }
}

template <typename XT, int MODE>
__global__ __launch_bounds__(256) void q8_gemv_kernel(GemvArgs a) {
  extern __shared__ float smem[];
  const uint32_t K = a.k, C = K / kChunkK;
  float *xs = smem;                 // [K]
  float *xsum = smem + K;           // [C][2]: sum of each 32-wide half-chunk
  float *red = xsum + 2 * C;        // [4 waves][kPanelsPerWG * 32]

  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t h = lane >> 5, r = lane & 31;
  const uint32_t np = (a.n + kPanelRows - 1) / kPanelRows;
  const uint32_t p0 = blockIdx.x * kPanelsPerWG;

  uint32_t R[kPanelsPerWG];
  bool live[kPanelsPerWG];
#pragma unroll
  for (int t = 0; t < kPanelsPerWG; ++t) {
    const uint32_t p = p0 + t;
    R[t] = p < np ? panel_rows(a.n, p) : 0;
    live[t] = r < R[t];
  }
  const uint32_t c0 = (wave * C) / 4, c1 = ((wave + 1) * C) / 4;

  // The first weight batch does not depend on x: put it in flight before the
  // x prologue so the activation staging hides under HBM latency.
  Batch b;
  load_batch(b, a, K, c0, c1, p0, R, live, h, r);

  // Stage x as f32; each 32-lane group also reduces one 32-wide block sum.
  const XT *x = static_cast<const XT *>(a.x);
  for (uint32_t i = threadIdx.x; i < K; i += 256) {
    const float v = (float)x[i];
    xs[i] = v;
    float sum = v;
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 32);
    if ((i & 31) == 0) xsum[i >> 5] = sum;
  }
  __syncthreads();

  float acc[kPanelsPerWG] = {};
  for (uint32_t c = c0; c < c1; c += kUnroll) {
    if (c != c0) load_batch(b, a, K, c, c1, p0, R, live, h, r);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (c + u >= c1) break;
      const f32x4 *xv = reinterpret_cast<const f32x4 *>(xs + (c + u) * kChunkK + h * 32);
      f32x4 xr[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) xr[q] = xv[q];
      const float xsm = xsum[(c + u) * 2 + h];
#pragma unroll
      for (int t = 0; t < kPanelsPerWG; ++t) {
        if (!live[t]) continue;
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const u32x4 ww = b.w[u][t][j];
          const uint32_t wd[4] = {ww.x, ww.y, ww.z, ww.w};
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const f32x4 xq = xr[j * 4 + d];
            part = __builtin_fmaf(xq.x, byte_f(wd[d], 0), part);
            part = __builtin_fmaf(xq.y, byte_f(wd[d], 1), part);
            part = __builtin_fmaf(xq.z, byte_f(wd[d], 2), part);
            part = __builtin_fmaf(xq.w, byte_f(wd[d], 3), part);
          }
        }
        part = __builtin_fmaf(-128.0f, xsm, part);
        acc[t] = __builtin_fmaf(part, (float)b.s[u][t], acc[t]);
      }
    }
  }

#pragma unroll
  for (int t = 0; t < kPanelsPerWG; ++t) {
    acc[t] += __shfl_xor(acc[t], 32);
    if (h == 0) red[wave * (kPanelsPerWG * 32) + t * 32 + r] = acc[t];
  }
  __syncthreads();
  if (threadIdx.x >= kPanelsPerWG * 32) return;
  const uint32_t t = threadIdx.x / 32, rr = threadIdx.x % 32;
  if (p0 + t >= np || rr >= panel_rows(a.n, p0 + t)) return;
  const uint32_t stride = kPanelsPerWG * 32;
  const float v = red[threadIdx.x] + red[stride + threadIdx.x] + red[2 * stride + threadIdx.x] +
                  red[3 * stride + threadIdx.x];
  const uint32_t nrow = (p0 + t) * kPanelRows + rr;
  if constexpr (MODE == kPlain) {
    a.out[nrow] = v;
  } else if constexpr (MODE == kBias) {
    a.out[nrow] = v + a.bias[nrow];
  } else if constexpr (MODE == kBiasGelu) {
    a.out[nrow] = gelu_erf(v + a.bias[nrow]);
  } else if constexpr (MODE == kBiasRes) {
    a.out[nrow] = a.out[nrow] + v + a.bias[nrow];
  } else {  // kQkv: a.n = 3D, a.k = D
    const uint32_t D = a.k, pos = a.pos[0];
    if (nrow < D)
      a.out[nrow] = v + a.qb[nrow];
    else if (nrow < 2 * D)
      a.kc[(size_t)pos * D + (nrow - D)] = v;
    else
      a.vc[(size_t)pos * D + (nrow - 2 * D)] = v + a.vb[nrow - 2 * D];
  }
}

template <typename XT, int MODE>
int launch(const char *what, const GemvArgs &a) {
  if (!a.out || !a.x || !a.qs || !a.sc) return fail(MADI_ERR_NULL, "%s: null pointer", what);
  if ((MODE == kBias || MODE == kBiasGelu || MODE == kBiasRes) && !a.bias)
    return fail(MADI_ERR_NULL, "%s: null bias", what);
  if (a.n == 0 || a.k == 0 || a.k % kChunkK)
    return fail(MADI_ERR_SHAPE, "%s: n=%u k=%u (need n > 0, k a positive multiple of 64)", what, a.n, a.k);
  if (a.k > kMaxK) return fail(MADI_ERR_SHAPE, "%s: k=%u exceeds %u", what, a.k, kMaxK);
  if (!aligned(a.qs, 16) || !aligned(a.sc, 2) || !aligned(a.x, sizeof(XT)))
    return fail(MADI_ERR_ALIGN, "%s: qs needs 16-byte alignment", what);
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "%s: madi_init has not succeeded", what);
  const uint32_t np = (a.n + kPanelRows - 1) / kPanelRows;
  const uint32_t grid = (np + kPanelsPerWG - 1) / kPanelsPerWG;
  const size_t lds = (a.k + 2 * (a.k / kChunkK) + 4 * kPanelsPerWG * 32) * sizeof(float);
  hipLaunchKernelGGL((q8_gemv_kernel<XT, MODE>), dim3(grid), dim3(256), lds, stream(), a);
  return check_launch(what);
}

GemvArgs args(float *out, const void *x, const void *qs, const void *scales, const float *bias,
              uint32_t n, uint32_t k) {
  GemvArgs a{};
  a.out = out;
  a.x = x;
  a.qs = static_cast<const uint8_t *>(qs);
  a.sc = static_cast<const f16 *>(scales);
  a.bias = bias;
  a.n = n;
  a.k = k;
  return a;
}

}  // namespace

extern "C" int madi_q8_gemv(float *out, const float *x, const void *qs, const void *scales,
                            uint32_t n, uint32_t k) {
  return launch<float, kPlain>("madi_q8_gemv", args(out, x, qs, scales, nullptr, n, k));
}

extern "C" int madi_q8_gemv_bias(float *out, const float *x, const void *qs, const void *scales,
                                 const float *bias, uint32_t n, uint32_t k) {
  return launch<float, kBias>("madi_q8_gemv_bias", args(out, x, qs, scales, bias, n, k));
}

extern "C" int madi_q8_gemv_bias_gelu(float *out, const float *x, const void *qs,
                                      const void *scales, const float *bias, uint32_t n,
                                      uint32_t k) {
  return launch<float, kBiasGelu>("madi_q8_gemv_bias_gelu", args(out, x, qs, scales, bias, n, k));
}

extern "C" int madi_q8_gemv_bias_res(float *out, const float *x, const void *qs,
                                     const void *scales, const float *bias, uint32_t n,
                                     uint32_t k) {
  return launch<float, kBiasRes>("madi_q8_gemv_bias_res", args(out, x, qs, scales, bias, n, k));
}

extern "C" int madi_q8_gemv_qkv(float *q_out, const float *x, const void *qs, const void *scales,
                                const float *qb, const float *vb, float *kc, float *vc,
                                const uint32_t *pos, uint32_t d) {
  if (!qb || !vb || !kc || !vc || !pos) return fail(MADI_ERR_NULL, "madi_q8_gemv_qkv: null pointer");
  if (d == 0 || d % kChunkK) return fail(MADI_ERR_SHAPE, "madi_q8_gemv_qkv: d=%u must be a positive multiple of 64", d);
  GemvArgs a = args(q_out, x, qs, scales, nullptr, 3 * d, d);
  a.qb = qb;
  a.vb = vb;
  a.kc = kc;
  a.vc = vc;
  a.pos = pos;
  return launch<float, kQkv>("madi_q8_gemv_qkv", a);
}

extern "C" int madi_q8_logit_gemv(float *logits, const void *qs, const void *scales,
                                  const float *x, uint32_t vocab, uint32_t dim) {
  return launch<float, kPlain>("madi_q8_logit_gemv", args(logits, x, qs, scales, nullptr, vocab, dim));
}

extern "C" int madi_q8_gemv_f16x(float *out, const void *x_f16, const void *qs,
                                 const void *scales, const float *bias, uint32_t n, uint32_t k,
                                 int epilogue) {
  const GemvArgs a = args(out, x_f16, qs, scales, bias, n, k);
  switch (epilogue) {
  case MADI_EPI_NONE: return launch<f16, kPlain>("madi_q8_gemv_f16x", a);
  case MADI_EPI_BIAS: return launch<f16, kBias>("madi_q8_gemv_f16x", a);
  case MADI_EPI_BIAS_GELU: return launch<f16, kBiasGelu>("madi_q8_gemv_f16x", a);
  case MADI_EPI_BIAS_RES: return launch<f16, kBiasRes>("madi_q8_gemv_f16x", a);
  default: return fail(MADI_ERR_ARG, "madi_q8_gemv_f16x: unknown epilogue %d", epilogue);
  }
}
