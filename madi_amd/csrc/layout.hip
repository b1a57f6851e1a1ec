// layout.hip -- load-time work on the CDNA4 panel layout: repack of natural Q8
// rows, F16 -> Q8 quantisation straight into panels, the weight identity hash,
// the transposed F16 dequant, and Q8 embedding-row gathers.
#include <string.h>

#include "common.h"

using namespace madi;

namespace {

int check_q8_shape(const char *what, uint32_t n, uint32_t k) {
  if (n == 0 || k == 0) return fail(MADI_ERR_SHAPE, "%s: empty weight (n=%u k=%u)", what, n, k);
  if (k % kChunkK != 0)
    return fail(MADI_ERR_SHAPE, "%s: k=%u is not a multiple of %u (panel layout)", what, k, kChunkK);
  return MADI_OK;
}

// natural index of the byte stored at panel-layout unit (p, c, j, h, r), byte i
inline size_t natural_qs_index(uint32_t k, uint32_t p, uint32_t c, uint32_t j, uint32_t h,
                               uint32_t r, uint32_t i) {
  return (size_t)(p * kPanelRows + r) * k + c * kChunkK + h * 32 + j * 16 + i;
}

}  // namespace

// ------------------------------------------------------------------ host repack
extern "C" int madi_q8_repack_host(void *dst_qs, void *dst_scales, const void *qs,
                                   const void *scales, uint32_t n, uint32_t k) {
  if (!dst_qs || !dst_scales || !qs || !scales) return fail(MADI_ERR_NULL, "madi_q8_repack_host: null pointer");
  if (int rc = check_q8_shape("madi_q8_repack_host", n, k)) return rc;
  const int8_t *src = static_cast<const int8_t *>(qs);
  const uint16_t *ssrc = static_cast<const uint16_t *>(scales);
  uint8_t *dst = static_cast<uint8_t *>(dst_qs);
  uint16_t *sdst = static_cast<uint16_t *>(dst_scales);
  const uint32_t np = (n + kPanelRows - 1) / kPanelRows, nc = k / kChunkK, nb = k / 32;
  for (uint32_t p = 0; p < np; ++p) {
    const uint32_t R = panel_rows(n, p);
    for (uint32_t c = 0; c < nc; ++c) {
      uint8_t *blk = dst + panel_chunk_qs(k, p, R, c);
      uint16_t *sblk = sdst + panel_chunk_sc(k, p, R, c);
      for (uint32_t j = 0; j < 2; ++j)
        for (uint32_t h = 0; h < 2; ++h)
          for (uint32_t r = 0; r < R; ++r) {
            uint8_t *u = blk + ((2 * j + h) * R + r) * 16;
            for (uint32_t i = 0; i < 16; ++i)
              u[i] = (uint8_t)(src[natural_qs_index(k, p, c, j, h, r, i)] + 128);
          }
      for (uint32_t h = 0; h < 2; ++h)
        for (uint32_t r = 0; r < R; ++r)
          sblk[h * R + r] = ssrc[(size_t)(p * kPanelRows + r) * nb + 2 * c + h];
    }
  }
  return MADI_OK;
}

extern "C" int madi_q8_unpack_host(void *dst_qs, void *dst_scales, const void *tiled_qs,
                                   const void *tiled_scales, uint32_t n, uint32_t k) {
  if (!dst_qs || !dst_scales || !tiled_qs || !tiled_scales)
    return fail(MADI_ERR_NULL, "madi_q8_unpack_host: null pointer");
  if (int rc = check_q8_shape("madi_q8_unpack_host", n, k)) return rc;
  const uint8_t *src = static_cast<const uint8_t *>(tiled_qs);
  const uint16_t *ssrc = static_cast<const uint16_t *>(tiled_scales);
  int8_t *dst = static_cast<int8_t *>(dst_qs);
  uint16_t *sdst = static_cast<uint16_t *>(dst_scales);
  const uint32_t np = (n + kPanelRows - 1) / kPanelRows, nc = k / kChunkK, nb = k / 32;
  for (uint32_t p = 0; p < np; ++p) {
    const uint32_t R = panel_rows(n, p);
    for (uint32_t c = 0; c < nc; ++c) {
      const uint8_t *blk = src + panel_chunk_qs(k, p, R, c);
      const uint16_t *sblk = ssrc + panel_chunk_sc(k, p, R, c);
      for (uint32_t j = 0; j < 2; ++j)
        for (uint32_t h = 0; h < 2; ++h)
          for (uint32_t r = 0; r < R; ++r) {
            const uint8_t *u = blk + ((2 * j + h) * R + r) * 16;
            for (uint32_t i = 0; i < 16; ++i)
              dst[natural_qs_index(k, p, c, j, h, r, i)] = (int8_t)(u[i] - 128);
          }
      for (uint32_t h = 0; h < 2; ++h)
        for (uint32_t r = 0; r < R; ++r)
          sdst[(size_t)(p * kPanelRows + r) * nb + 2 * c + h] = sblk[h * R + r];
    }
  }
  return MADI_OK;
}

// ------------------------------------------------------------------ device repack
// One thread per natural 16-byte unit (reads coalesced along the row).
// Natural rows -> panel layout on the device.  Grid (panels, ceil(K / 256)):
// a workgroup moves one panel's rows over four 64-wide chunks.  The rows are
// read whole (8 lanes per 256-byte row segment, 32 bytes each, flipped to
// q + 128) into an LDS tile; the units then leave in the panel layout's own
// order, so consecutive lanes write consecutive 16-byte units (the four
// chunks of a full panel are 8 KiB contiguous).  The scales (8 per row) go
// straight to their panel positions.
constexpr uint32_t kRepackChunks = 4;
constexpr uint32_t kRepackPitch = kRepackChunks * kChunkK + 16;  // LDS row bytes

// The staged tile (row r's stored bytes q + 128 of chunks c0 .. c0 + chunks - 1
// at r * kRepackPitch) out to panel p in the panel layout's own order: unit v
// of the group is chunk v >> 7, then (j, h) as 2j + h, then row r, so
// consecutive lanes write consecutive 16-byte units.
__device__ inline void write_panel_units(uint8_t *__restrict__ dq, const uint8_t *tile, uint32_t k,
                                         uint32_t p, uint32_t R, uint32_t c0, uint32_t chunks,
                                         uint32_t t) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t v = t + 256 * i, cl = v >> 7, jh = (v >> 5) & 3, r = v & 31;
    if (cl < chunks && r < R) {
      const uint32_t j = jh >> 1, h = jh & 1;
      *reinterpret_cast<u32x4 *>(dq + panel_chunk_qs(k, p, R, c0 + cl) + (jh * R + r) * 16) =
          *reinterpret_cast<const u32x4 *>(tile + r * kRepackPitch + cl * kChunkK + h * 32 + j * 16);
    }
  }
}

__global__ __launch_bounds__(256) void q8_repack_kernel(uint8_t *__restrict__ dq,
                                                        uint16_t *__restrict__ ds,
                                                        const int8_t *__restrict__ src,
                                                        const uint16_t *__restrict__ ssrc,
                                                        uint32_t n, uint32_t k) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kPanelRows * kRepackPitch];
  const uint32_t p = blockIdx.x, cg = blockIdx.y, t = threadIdx.x;
  const uint32_t R = panel_rows(n, p);
  const uint32_t c0 = cg * kRepackChunks, nc = k / kChunkK;
  const uint32_t chunks = nc - c0 < kRepackChunks ? nc - c0 : kRepackChunks;
  const u32x4 flip = {0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
  {
    const uint32_t r = t >> 3, q = t & 7;  // 32 bytes per lane: columns 32q .. 32q + 31
    if (r < R && q < 2 * chunks) {
      const int8_t *row = src + (size_t)(p * kPanelRows + r) * k + c0 * kChunkK + q * 32;
      u32x4 a = *reinterpret_cast<const u32x4 *>(row), b = *reinterpret_cast<const u32x4 *>(row + 16);
      *reinterpret_cast<u32x4 *>(tile + r * kRepackPitch + q * 32) = a ^ flip;
      *reinterpret_cast<u32x4 *>(tile + r * kRepackPitch + q * 32 + 16) = b ^ flip;
    }
    // scales: row r's blocks 8cg .. 8cg + 7
    const uint32_t b = t & 7;
    if (r < R && b < 2 * chunks) {
      const uint32_t cl = b >> 1, h = b & 1;
      ds[panel_chunk_sc(k, p, R, c0 + cl) + h * R + r] =
          ssrc[(size_t)(p * kPanelRows + r) * (k / 32) + c0 * 2 + b];
    }
  }
  __syncthreads();
  write_panel_units(dq, tile, k, p, R, c0, chunks, t);
}

static bool overlaps(const void *a, size_t na, const void *b, size_t nb) {
  uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + nb && y < x + na;
}

extern "C" int madi_q8_repack(void *dst_qs, void *dst_scales, const void *qs, const void *scales,
                              uint32_t n, uint32_t k) {
  if (!dst_qs || !dst_scales || !qs || !scales) return fail(MADI_ERR_NULL, "madi_q8_repack: null pointer");
  if (int rc = check_q8_shape("madi_q8_repack", n, k)) return rc;
  if (!aligned(dst_qs, 16) || !aligned(qs, 16) || !aligned(dst_scales, 2) || !aligned(scales, 2))
    return fail(MADI_ERR_ALIGN, "madi_q8_repack: qs buffers need 16-byte alignment");
  const size_t nq = (size_t)n * k, ns = (size_t)n * (k / 32);
  if (overlaps(dst_qs, nq, qs, nq) || overlaps(dst_scales, ns * 2, scales, ns * 2))
    return fail(MADI_ERR_ARG, "madi_q8_repack: source and destination overlap");
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_q8_repack: madi_init has not succeeded");
  if (int rc = deferred_before_write(dst_qs, nq)) return rc;
  if (int rc = deferred_before_write(dst_scales, ns * 2)) return rc;
  const uint32_t np = (n + kPanelRows - 1) / kPanelRows;
  const uint32_t groups = (k / kChunkK + kRepackChunks - 1) / kRepackChunks;
  hipLaunchKernelGGL(q8_repack_kernel, dim3(np, groups), dim3(256), 0, stream(),
                     static_cast<uint8_t *>(dst_qs), static_cast<uint16_t *>(dst_scales),
                     static_cast<const int8_t *>(qs), static_cast<const uint16_t *>(scales), n, k);
  return check_launch("madi_q8_repack");
}

// ------------------------------------------------------------------ quantise F16 -> panel Q8
// quantInto (engine/metal/transcribe.zig:309-326) and quantize_q8.py:27-40 on
// the device, writing straight into the panel layout.  One thread per
// (row, 32-block): scale = max|w| / 127 in f32 (1.0 for an all-zero block),
// stored as f16; q = clamp(round_half_away(w * (1 / scale)), -127, 127), all
// in correctly rounded f32 as the Zig loop does.
// Grid (panels, ceil(K / 256)), as the repack: lane (r, b) of a workgroup
// quantises row r's block b of four chunks (32 f16, 8 lanes per 512-byte row
// segment), writes its scale to the panel position and its 32 stored bytes
// to an LDS tile, from which the units leave in panel order.
__global__ __launch_bounds__(256) void q8_quantize_kernel(uint8_t *__restrict__ dst_q,
                                                          uint16_t *__restrict__ dst_s,
                                                          const uint16_t *__restrict__ src,
                                                          uint32_t n, uint32_t k) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kPanelRows * kRepackPitch];
  const uint32_t p = blockIdx.x, cg = blockIdx.y, t = threadIdx.x;
  const uint32_t R = panel_rows(n, p);
  const uint32_t c0 = cg * kRepackChunks, nc = k / kChunkK;
  const uint32_t chunks = nc - c0 < kRepackChunks ? nc - c0 : kRepackChunks;
  const uint32_t r = t >> 3, b = t & 7;  // row r, block 8cg + b
  if (r < R && b < 2 * chunks) {
    const u32x4 *s4 = reinterpret_cast<const u32x4 *>(
        src + (size_t)(p * kPanelRows + r) * k + (size_t)(c0 * 2 + b) * 32);
    float w[32];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f16x8 v = __builtin_bit_cast(f16x8, s4[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) w[8 * i + e] = (float)v[e];
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float a = __builtin_fabsf(w[i]);
      mx = a > mx ? a : mx;
    }
    const float scale = mx > 0.0f ? __fdiv_rn(mx, 127.0f) : 1.0f;
    const float inv = __frcp_rn(scale);
    uint32_t word[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      uint32_t packed = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float q = roundf(__fmul_rn(w[4 * d + e], inv));
        q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
        packed |= (uint32_t)((int)q + 128) << (8 * e);  // stored biased: q + 128
      }
      word[d] = packed;
    }
    const uint32_t cl = b >> 1, h = b & 1;
    uint8_t *row = tile + r * kRepackPitch + cl * kChunkK + h * 32;
    *reinterpret_cast<u32x4 *>(row) = (u32x4){word[0], word[1], word[2], word[3]};
    *reinterpret_cast<u32x4 *>(row + 16) = (u32x4){word[4], word[5], word[6], word[7]};
    dst_s[panel_chunk_sc(k, p, R, c0 + cl) + h * R + r] = __builtin_bit_cast(uint16_t, (f16)scale);
  }
  __syncthreads();
  write_panel_units(dst_q, tile, k, p, R, c0, chunks, t);
}

extern "C" int madi_q8_quantize(void *dst_qs, void *dst_scales, const void *w_f16, uint32_t n,
                                uint32_t k) {
  if (!dst_qs || !dst_scales || !w_f16) return fail(MADI_ERR_NULL, "madi_q8_quantize: null pointer");
  if (int rc = check_q8_shape("madi_q8_quantize", n, k)) return rc;
  if (!aligned(dst_qs, 16) || !aligned(w_f16, 16) || !aligned(dst_scales, 2))
    return fail(MADI_ERR_ALIGN, "madi_q8_quantize: qs and w need 16-byte alignment");
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_q8_quantize: madi_init has not succeeded");
  const size_t blocks = (size_t)n * (k / 32);
  if (int rc = deferred_before_write(dst_qs, (size_t)n * k)) return rc;
  if (int rc = deferred_before_write(dst_scales, blocks * 2)) return rc;
  const uint32_t np = (n + kPanelRows - 1) / kPanelRows;
  const uint32_t groups = (k / kChunkK + kRepackChunks - 1) / kRepackChunks;
  hipLaunchKernelGGL(q8_quantize_kernel, dim3(np, groups), dim3(256), 0, stream(),
                     static_cast<uint8_t *>(dst_qs), static_cast<uint16_t *>(dst_scales),
                     static_cast<const uint16_t *>(w_f16), n, k);
  return check_launch("madi_q8_quantize");
}

// ------------------------------------------------------------------ weight identity (host)
// fnvQ8 (engine/metal/transcribe.zig:131-140): FNV-1a 64 over the natural-layout
// qs bytes, then the scales' little-endian bytes, continuing from `seed`.
extern "C" uint64_t madi_q8_fnv(uint64_t seed, const void *qs, size_t nq, const void *scales,
                                size_t nsc) {
  uint64_t x = seed;
  const uint8_t *b = static_cast<const uint8_t *>(qs);
  for (size_t i = 0; i < nq; ++i) x = (x ^ b[i]) * 0x100000001b3ull;
  b = static_cast<const uint8_t *>(scales);
  for (size_t i = 0; i < nsc * 2; ++i) x = (x ^ b[i]) * 0x100000001b3ull;
  return x;
}

// ------------------------------------------------------------------ dequant -> F16 [K][N]
// grid (ceil(panels / 4), K / 64): a workgroup dequantises four panels (128
// columns n of the output) for one 64-wide chunk of K into an LDS tile, then
// writes the tile out row by row.  Loading, lane (panel, j, h, row pair)
// takes the panel-layout units of rows r and r+1 (32 contiguous bytes) and
// writes each k's two values as one 4-byte LDS word.  Storing, each output
// row k of the tile is 256 contiguous bytes: 16-byte stores (16 lanes per
// row) where N % 8 == 0 and the output is 16-byte aligned (every encoder
// shape), else 2-byte stores with n fastest (128 contiguous bytes per wave
// instruction; the 51866-row vocab).  Only the elements with index in
// [lo, hi) are written (the whole matrix, [0, n*k), for kDeq; a window when
// part of the destination has since been overwritten).
constexpr uint32_t kDeqPanels = 4;
// LDS row pitch: 128 f16 plus 16 bytes, so consecutive rows start in
// different banks and every 16-byte piece stays aligned
constexpr uint32_t kDeqPitch = kDeqPanels * kPanelRows * 2 + 16;

__global__ __launch_bounds__(256) void q8_dequant_f16_kernel(f16 *__restrict__ out,
                                                             const uint8_t *__restrict__ qs,
                                                             const f16 *__restrict__ sc,
                                                             uint32_t n, uint32_t k, size_t lo,
                                                             size_t hi, uint32_t vec) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kChunkK * kDeqPitch];
  const uint32_t np = (n + kPanelRows - 1) / kPanelRows;
  const uint32_t g = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
  {
    // one wave per panel; 16 lanes per (j, h), each with rows 2rp, 2rp + 1
    const uint32_t pl = t >> 6, jh = (t >> 4) & 3, rp = t & 15;
    const uint32_t p = g * kDeqPanels + pl, r = 2 * rp;
    if (p < np) {
      const uint32_t R = panel_rows(n, p);
      if (r < R) {
        const uint32_t j = jh >> 1, h = jh & 1;
        const uint8_t *u = qs + panel_chunk_qs(k, p, R, c) + ((2 * j + h) * R + r) * 16;
        const f16 *s = sc + panel_chunk_sc(k, p, R, c) + h * R + r;
        const bool two = r + 1 < R;
        f16x8 a0, a1, b0 = {}, b1 = {};
        dequant16(*reinterpret_cast<const u32x4 *>(u), s[0], a0, a1);
        if (two) dequant16(*reinterpret_cast<const u32x4 *>(u + 16), s[1], b0, b1);
        const uint32_t k0 = h * 32 + j * 16, col = pl * kPanelRows + r;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          *reinterpret_cast<f16x2 *>(tile + (k0 + i) * kDeqPitch + col * 2) = (f16x2){a0[i], b0[i]};
          *reinterpret_cast<f16x2 *>(tile + (k0 + 8 + i) * kDeqPitch + col * 2) = (f16x2){a1[i], b1[i]};
        }
      }
    }
  }
  __syncthreads();
  const uint32_t n0 = g * kDeqPanels * kPanelRows;
  if (vec) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint32_t idx = t + 256 * s, kr = idx >> 4, c8 = idx & 15, nn = n0 + c8 * 8;
      if (nn >= n) continue;  // N % 8 == 0: a group is wholly inside or outside
      const size_t e = (size_t)(c * kChunkK + kr) * n + nn;
      const f16x8 v = *reinterpret_cast<const f16x8 *>(tile + kr * kDeqPitch + c8 * 16);
      if (e >= lo && e + 8 <= hi) {
        *reinterpret_cast<f16x8 *>(out + e) = v;
      } else if (e + 8 > lo && e < hi) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (e + i >= lo && e + i < hi) out[e + i] = v[i];
      }
    }
  } else {
    for (int s = 0; s < 32; ++s) {
      const uint32_t idx = t + 256 * s, kr = idx >> 7, nl = idx & 127, nn = n0 + nl;
      if (nn >= n) continue;
      const size_t e = (size_t)(c * kChunkK + kr) * n + nn;
      if (e >= lo && e < hi) out[e] = *reinterpret_cast<const f16 *>(tile + kr * kDeqPitch + nl * 2);
    }
  }
}

namespace madi {
int dequant_launch(void *wdq, const void *qs, const void *scales, uint32_t n, uint32_t k,
                   size_t lo, size_t hi) {
  const uint32_t np = (n + kPanelRows - 1) / kPanelRows;
  if (hi > (size_t)n * k) hi = (size_t)n * k;
  const uint32_t vec = n % 8 == 0 && aligned(wdq, 16) ? 1u : 0u;
  hipLaunchKernelGGL(q8_dequant_f16_kernel, dim3((np + kDeqPanels - 1) / kDeqPanels, k / kChunkK),
                     dim3(256), 0, stream(), static_cast<f16 *>(wdq),
                     static_cast<const uint8_t *>(qs), static_cast<const f16 *>(scales), n, k, lo,
                     hi, vec);
  return check_launch("madi_q8_dequant_f16");
}
}  // namespace madi

// kDeq / deqW16.  With deferral on (the default) this records the pair and
// returns: the F16 GEMM that consumes wdq runs the fused Q8 kernel instead,
// and wdq is written only if something else reads it (boundary.hip).
extern "C" int madi_q8_dequant_f16(void *wdq, const void *qs, const void *scales, uint32_t n,
                                   uint32_t k) {
  if (!wdq || !qs || !scales) return fail(MADI_ERR_NULL, "madi_q8_dequant_f16: null pointer");
  if (int rc = check_q8_shape("madi_q8_dequant_f16", n, k)) return rc;
  if (!aligned(qs, 16) || !aligned(scales, 2) || !aligned(wdq, 2))
    return fail(MADI_ERR_ALIGN, "madi_q8_dequant_f16: qs needs 16-byte alignment");
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_q8_dequant_f16: madi_init has not succeeded");
  const int rec = deferred_record(wdq, qs, scales, n, k);
  if (rec != 0) return rec < 0 ? rec : MADI_OK;
  return dequant_launch(wdq, qs, scales, n, k, 0, (size_t)n * k);
}

// ------------------------------------------------------------------ embedding rows
__device__ inline float panel_weight(const uint8_t *qs, const f16 *sc, uint32_t n, uint32_t k,
                                     uint32_t row, uint32_t d) {
  const uint32_t p = row / kPanelRows, r = row % kPanelRows, R = panel_rows(n, p);
  const uint32_t c = d / kChunkK, kk = d % kChunkK, h = kk / 32, j = (kk % 32) / 16, i = kk % 16;
  const int q = (int)qs[panel_chunk_qs(k, p, R, c) + ((2 * j + h) * R + r) * 16 + i] - 128;
  const float s = (float)sc[panel_chunk_sc(k, p, R, c) + h * R + r];
  return (float)q * s;
}

// gpu_emb_lookup_q8 / emb_lookup_indirect_q8 semantics (graph_helpers.metal:354-383).
// `n_rows` bounds the token: an out-of-range token writes nothing (the
// reference reads out of bounds there; this library refuses instead).
__global__ __launch_bounds__(256) void q8_emb_row_kernel(float *__restrict__ out,
                                                         const uint8_t *__restrict__ qs,
                                                         const f16 *__restrict__ sc,
                                                         const uint32_t *__restrict__ tok_ptr,
                                                         const uint32_t *__restrict__ tokens,
                                                         const uint32_t *__restrict__ pos_ptr,
                                                         uint32_t n_rows, uint32_t dim) {
  const uint32_t tok = tokens ? tokens[pos_ptr[0]] : tok_ptr[0];
  if (tok >= n_rows) return;
  for (uint32_t d = threadIdx.x; d < dim; d += 256) out[d] = panel_weight(qs, sc, n_rows, dim, tok, d);
}

static int emb_common(const char *what, float *out, const void *qs, const void *scales,
                      const uint32_t *tok_ptr, const uint32_t *tokens, const uint32_t *pos_ptr,
                      uint32_t n_rows, uint32_t dim) {
  if (!out || !qs || !scales) return fail(MADI_ERR_NULL, "%s: null pointer", what);
  if (dim == 0 || dim % kChunkK) return fail(MADI_ERR_SHAPE, "%s: dim=%u must be a positive multiple of 64", what, dim);
  if (n_rows == 0) return fail(MADI_ERR_SHAPE, "%s: empty table", what);
  if (!aligned(qs, 16) || !aligned(scales, 2) || !aligned(out, 4))
    return fail(MADI_ERR_ALIGN, "%s: misaligned pointer", what);
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "%s: madi_init has not succeeded", what);
  if (int rc = deferred_before_write(out, (size_t)dim * 4)) return rc;
  hipLaunchKernelGGL(q8_emb_row_kernel, dim3(1), dim3(256), 0, stream(), out,
                     static_cast<const uint8_t *>(qs), static_cast<const f16 *>(scales), tok_ptr,
                     tokens, pos_ptr, n_rows, dim);
  return check_launch(what);
}

// emb_pe_rows_q8 semantics (engine/metal/kernels/decoder_ops.metal:614-633), the
// sequence prefill's embedding (decoder.zig:460-467): out[m][d] =
// f32(q) * f32(s) of row tokens[m] + pe[(pos0 + m) * dim + d].  One workgroup
// per row; a thread takes one 16-byte unit of the panel layout (16
// consecutive d of one quantisation block), so each row is read as whole
// units and written as 64-byte runs.  The product is exact in f32 (8 x 11
// significant bits), so the one rounding is the add, as in the reference.  A
// token >= n_rows leaves its row untouched.
__global__ __launch_bounds__(256) void q8_emb_pe_rows_kernel(
    float *__restrict__ out, const uint8_t *__restrict__ qs, const f16 *__restrict__ sc,
    const uint32_t *__restrict__ tokens, const float *__restrict__ pe, uint32_t n_rows,
    uint32_t dim, uint32_t pos0) {
  const uint32_t m = blockIdx.x;
  const uint32_t tok = tokens[m];
  if (tok >= n_rows) return;
  const uint32_t p = tok / kPanelRows, r = tok % kPanelRows, R = panel_rows(n_rows, p);
  const float *per = pe + (size_t)(pos0 + m) * dim;
  float *o = out + (size_t)m * dim;
  for (uint32_t u = threadIdx.x; u < dim / 16; u += blockDim.x) {
    const uint32_t d0 = u * 16, c = d0 / kChunkK, h = (d0 % kChunkK) / 32, j = (d0 % 32) / 16;
    const u32x4 w = *reinterpret_cast<const u32x4 *>(qs + panel_chunk_qs(dim, p, R, c) +
                                                     ((2 * j + h) * R + r) * 16);
    const float s = (float)sc[panel_chunk_sc(dim, p, R, c) + h * R + r];
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const f32x4 e = *reinterpret_cast<const f32x4 *>(per + d0 + 4 * v);
      f32x4 res;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int q = (int)((words[v] >> (8 * b)) & 0xffu) - 128;
        res[b] = (float)q * s + e[b];
      }
      *reinterpret_cast<f32x4 *>(o + d0 + 4 * v) = res;
    }
  }
}

extern "C" int madi_q8_emb_pe_rows(float *out, const void *qs, const void *scales,
                                   const uint32_t *tokens, const float *pe, uint32_t dim,
                                   uint32_t pos0, uint32_t m, uint32_t vocab) {
  const char *what = "madi_q8_emb_pe_rows";
  if (!out || !qs || !scales || !tokens || !pe) return fail(MADI_ERR_NULL, "%s: null pointer", what);
  if (dim == 0 || dim % kChunkK) return fail(MADI_ERR_SHAPE, "%s: dim=%u must be a positive multiple of 64", what, dim);
  if (vocab == 0) return fail(MADI_ERR_SHAPE, "%s: empty table", what);
  if (m == 0) return MADI_OK;
  if (m > 65535u) return fail(MADI_ERR_SHAPE, "%s: m=%u exceeds 65535 rows", what, m);
  if ((uint64_t)vocab * dim >= (1ull << 32))
    return fail(MADI_ERR_SHAPE, "%s: vocab=%u dim=%u exceeds the 4 GiB table limit", what, vocab, dim);
  if (!aligned(qs, 16) || !aligned(scales, 2) || !aligned(out, 16) || !aligned(pe, 16))
    return fail(MADI_ERR_ALIGN, "%s: qs, out and pe need 16-byte alignment", what);
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "%s: madi_init has not succeeded", what);
  if (int rc = deferred_before_write(out, (size_t)m * dim * 4)) return rc;
  hipLaunchKernelGGL(q8_emb_pe_rows_kernel, dim3(m), dim3(dim / 16 < 256 ? 64 * ((dim / 16 + 63) / 64) : 256),
                     0, stream(), out, static_cast<const uint8_t *>(qs),
                     static_cast<const f16 *>(scales), tokens, pe, vocab, dim, pos0);
  return check_launch(what);
}

extern "C" int madi_q8_emb_lookup(float *out, const void *qs, const void *scales,
                                  const uint32_t *tok_ptr, uint32_t vocab, uint32_t dim) {
  if (!tok_ptr) return fail(MADI_ERR_NULL, "madi_q8_emb_lookup: null tok_ptr");
  return emb_common("madi_q8_emb_lookup", out, qs, scales, tok_ptr, nullptr, nullptr, vocab, dim);
}

extern "C" int madi_q8_emb_lookup_indirect(float *out, const void *qs, const void *scales,
                                           const uint32_t *tokens, const uint32_t *pos_ptr,
                                           uint32_t vocab, uint32_t dim) {
  if (!tokens || !pos_ptr) return fail(MADI_ERR_NULL, "madi_q8_emb_lookup_indirect: null pointer");
  return emb_common("madi_q8_emb_lookup_indirect", out, qs, scales, nullptr, tokens, pos_ptr,
                    vocab, dim);
}
