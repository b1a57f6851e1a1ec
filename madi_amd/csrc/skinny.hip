// skinny.hip -- Q8 projection of a few activation rows: the batched decode
// GEMV (M = B token rows, 2..32 per pass), HBM-bound on the weights.
//
// Replaces the reference's pproj (engine/metal/decoder.zig:427-432) and the
// per-slot batched projections it feeds (decodeBlockBatched, prefill): there
// the Q8 weight is dequantised into an F16 [K][N] scratch (kDeq), the f32 rows
// are converted to f16 (kCvt32), MPS multiplies them, and kCvt16 widens the
// f16 result.  Here one kernel reads the Q8 panels once and keeps the
// arithmetic of that pipeline on the MFMA: activations rounded to f16 (the
// kCvt32 staging), weights dequantised to fp16_rne(q * s) (kDeq), fp32
// accumulation; the sum is written as f32 without the f16 output staging (the
// one rounding the pipeline adds after the product, dropped: it only moves
// the result away from the fp32 reference of test_batchproj.zig:72-78).
//
// Workgroup: one 32-row weight panel x one slice of 32 activation rows, four
// waves splitting K like the GEMV.  Per 64-wide K chunk a wave loads the
// panel's two 16-byte units per lane (lane (h, r): row r's 32 weights of
// quantisation block h) and its scale, plus 32 f32 activations per lane (lane
// (h, c): row c of the slice, the same 32 k), converts both to fp16 fragments
// and runs four v_mfma_f32_32x32x16_f16 with the weight as the A operand (rows
// n) and the activations as B (columns m).  K order of step s: k = 32h + 8s +
// e for both operands, as in the GEMM.  Activation rows past M load as zeros
// (their lanes' offsets fall outside the buffer resource), so small M costs
// no extra memory traffic.  Each wave keeps a two-chunk window in flight; the
// four K partial tiles meet in LDS and every wave stores one quarter.
#include "common.h"

using namespace madi;

namespace {

constexpr int kWaves = 4;   // K quarters per panel
constexpr int kWin = 2;     // chunks in flight per wave
constexpr uint32_t kSlice = 32;  // activation rows per workgroup

typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ inline rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// One chunk's loads for a lane: two weight units, the block scale and the 32
// activations of its (row, block) pair.
struct Chunk {
  u32x4 w[2];
  uint32_t s;
  f32x4 x[8];
};

__device__ inline void load_chunk(Chunk &b, rsrc_t wq, rsrc_t ws, rsrc_t xr, uint32_t K,
                                  uint32_t c, uint32_t p, uint32_t R, uint32_t w_voff,
                                  uint32_t s_voff, uint32_t x_voff) {
  const uint32_t so = (uint32_t)panel_chunk_qs(K, p, R, c);
  b.w[0] = __builtin_amdgcn_raw_buffer_load_b128(wq, w_voff, so, 0);
  b.w[1] = __builtin_amdgcn_raw_buffer_load_b128(wq, w_voff + 2 * R * 16, so, 0);
  b.s = __builtin_amdgcn_raw_buffer_load_b16(ws, s_voff, (uint32_t)panel_chunk_sc(K, p, R, c) * 2, 0);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    b.x[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, x_voff + i * 16, c * kChunkK * 4, 0));
}

// acc += W(chunk) . X(chunk)^T over the four k-steps; step s uses half (s & 1)
// of weight unit s >> 1
__device__ inline void accumulate(const Chunk &b, f32x16 &acc) {
  const f16 sc = __builtin_bit_cast(f16, (uint16_t)b.s);
  const f16x2 s2 = {sc, sc};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const u32x4 u = b.w[s >> 1];
    const uint32_t b0 = (s & 1) ? u.z : u.x, b1 = (s & 1) ? u.w : u.y;
    const f16x2 a0 = dequant_pair(b0, kSelLo, s2), a1 = dequant_pair(b0, kSelHi, s2);
    const f16x2 a2 = dequant_pair(b1, kSelLo, s2), a3 = dequant_pair(b1, kSelHi, s2);
    const f16x8 wf = {a0.x, a0.y, a1.x, a1.y, a2.x, a2.y, a3.x, a3.y};
    const f32x4 lo = b.x[2 * s], hi = b.x[2 * s + 1];
    const f16x8 xf = {(f16)lo.x, (f16)lo.y, (f16)lo.z, (f16)lo.w,
                      (f16)hi.x, (f16)hi.y, (f16)hi.z, (f16)hi.w};
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf, xf, acc, 0, 0, 0);
  }
}

struct SkinnyArgs {
  float *out;
  const float *x;
  const uint8_t *qs;
  const f16 *sc;
  uint32_t m, n, k;
  uint32_t panels, slices;
};

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void q8_skinny_kernel(
    SkinnyArgs a) {
  __shared__ __attribute__((aligned(16))) f32x4 red[kWaves][4][64];  // [wave][g][lane]

  // Consecutive workgroups go to different XCDs (round-robin).  Map the
  // slices of one panel to one XCD so they share its weights in that L2:
  // workgroup b runs on XCD b % 8 and takes panel 8 * ((b / 8) / S) + b % 8,
  // slice (b / 8) % S.
  const uint32_t b = blockIdx.x, S = a.slices;
  const uint32_t p = 8 * ((b / 8) / S) + b % 8, slice = (b / 8) % S;
  if (p >= a.panels) return;

  const uint32_t K = a.k, C = K / kChunkK;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t h = lane >> 5, r = lane & 31;
  const uint32_t R = panel_rows(a.n, p);
  const uint32_t c0 = (wave * C) / kWaves, c1 = ((wave + 1) * C) / kWaves;

  // Lanes past a partial panel's last row read row R-1 (in bounds; their sums
  // are never stored).  The activation resource covers the slice's rows that
  // exist, so rows past M read zeros.
  const uint32_t rr = r < R ? r : R - 1;
  const uint32_t w_voff = (h * R + rr) * 16, s_voff = (h * R + rr) * 2;
  const uint32_t m0 = slice * kSlice;
  const uint32_t rows = a.m - m0 < kSlice ? a.m - m0 : kSlice;
  const rsrc_t wq = make_rsrc(a.qs, a.n * K), ws = make_rsrc(a.sc, a.n * (K / 32) * 2);
  const rsrc_t xr = make_rsrc(a.x + (size_t)m0 * K, rows * K * 4);
  const uint32_t x_voff = r * K * 4 + h * 32 * 4;

  Chunk win[kWin];
#pragma unroll
  for (int i = 0; i < kWin; ++i)
    if (c0 + i < c1) load_chunk(win[i], wq, ws, xr, K, c0 + i, p, R, w_voff, s_voff, x_voff);
  f32x16 acc = {};
#pragma unroll 1
  for (uint32_t c = c0; c < c1; c += kWin) {
#pragma unroll
    for (int i = 0; i < kWin; ++i) {
      if (c + i < c1) {
        accumulate(win[i], acc);
        if (c + i + kWin < c1)
          load_chunk(win[i], wq, ws, xr, K, c + i + kWin, p, R, w_voff, s_voff, x_voff);
      }
    }
  }

  // Lane (h, c) holds D[n][m] for m = m0 + c and n = 32p + 8g + 4h + e
  // (acc[4g + e]).  Wave w sums group g = w over the four K quarters.
#pragma unroll
  for (int g = 0; g < 4; ++g)
    red[wave][g][lane] = (f32x4){acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]};
  __syncthreads();
  const f32x4 v = red[0][wave][lane] + red[1][wave][lane] + red[2][wave][lane] + red[3][wave][lane];
  const uint32_t m = m0 + r;
  const uint32_t nl = wave * 8 + h * 4;  // panel-local row of v.x
  if (m >= a.m) return;
  float *o = a.out + (size_t)m * a.n + p * kPanelRows + nl;
  if (nl + 4 <= R) {
    o[0] = v.x;
    o[1] = v.y;
    o[2] = v.z;
    o[3] = v.w;
  } else {
    if (nl + 0 < R) o[0] = v.x;
    if (nl + 1 < R) o[1] = v.y;
    if (nl + 2 < R) o[2] = v.z;
  }
}

}  // namespace

extern "C" int madi_q8_pproj(float *out, const float *in, const void *qs, const void *scales,
                             uint32_t m, uint32_t n, uint32_t k) {
  if (!out || !in || !qs || !scales) return fail(MADI_ERR_NULL, "madi_q8_pproj: null pointer");
  if (m == 0 || n == 0 || k == 0 || k % kChunkK)
    return fail(MADI_ERR_SHAPE, "madi_q8_pproj: m=%u n=%u k=%u (need m, n > 0, k a positive multiple of 64)", m, n, k);
  // buffer offsets are 32-bit: W (n*k bytes) and one slice of activations
  // (32*k*4 bytes) must stay below 2 GiB
  if ((uint64_t)n * k >= (1ull << 31) || (uint64_t)kSlice * k * 4 >= (1ull << 31))
    return fail(MADI_ERR_SHAPE, "madi_q8_pproj: n=%u k=%u exceeds the 2 GiB operand limit", n, k);
  if (!aligned(qs, 16) || !aligned(scales, 2) || !aligned(in, 16) || !aligned(out, 4))
    return fail(MADI_ERR_ALIGN, "madi_q8_pproj: qs and in need 16-byte alignment");
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_q8_pproj: madi_init has not succeeded");
  SkinnyArgs a{};
  a.out = out;
  a.x = in;
  a.qs = static_cast<const uint8_t *>(qs);
  a.sc = static_cast<const f16 *>(scales);
  a.m = m;
  a.n = n;
  a.k = k;
  a.panels = (n + kPanelRows - 1) / kPanelRows;
  a.slices = (m + kSlice - 1) / kSlice;
  const uint32_t grid = (a.panels + 7) / 8 * 8 * a.slices;
  hipLaunchKernelGGL(q8_skinny_kernel, dim3(grid), dim3(256), 0, stream(), a);
  return check_launch("madi_q8_pproj");
}
