// gemm.hip -- fused Q8 GEMM for the encoder projections (M = 1500 per window).
//
// C[M][N] (f16) = epi(A[M][K] (f16) . deq(W)[N][K]^T), fp32 accumulation on
// v_mfma_f32_32x32x16_f16.  Replaces the encoder's kDeq + kM4/kM4Bias pairs
// (engine/metal/encoder.zig:262-301) and the reference's fused Q8 designs
// mul_mm_q8 (kernels/q8_gemm.metal:29-102) and m4_gemm_q8_bias_gelu
// (kernels/m4_gemm.metal:131-189).
//
// Workgroup tile: 256 weight rows (8 panels) x 32*MT activation rows, four
// waves.  The weight is the MFMA A operand (rows = n) and the activations the
// B operand (columns = m), so each lane's 16 fp32 results cover four runs of
// four consecutive n and are stored as 8-byte f16x4 writes.
//
// Per 64-wide K chunk a stage of LDS holds, all written by direct-to-LDS DMA
// (global_load_lds_dwordx4, no VGPR staging):
//   W  8 panels x 2 KiB int8 (the panel layout's chunk blocks, copied verbatim)
//   S  8 panels x 128 B fp16 scales
//   A  MT m-tiles x 4 k-steps x 1 KiB, in MFMA B-operand order (lane l holds
//      A[m0 + 32i + l%32][k0 + 32(l/32) + 8s .. +8])
// NSTAGES stages form a ring so loads run NSTAGES-1 chunks ahead of the math.
// Wave w owns panels 2w, 2w+1: it reads its 2 x 2 KiB of int8 and 2 x 128 B of
// scales, dequantises them in registers (v_perm_b32 + packed fp16 add/mul,
// bit-exact fp16_rne(q*s)) and runs 2 x MT x 4 MFMAs per chunk.
//
// K ordering: MFMA k-slot (lane half h, slot e) of step s holds k = 32h + 8s + e
// for BOTH operands, so each lane's weight slice of a chunk lies in one
// quantisation block (one scale per lane per chunk); any k permutation shared
// by both operands leaves the product unchanged.
#include "common.h"

using namespace madi;

namespace {

constexpr int kPanelsPerTile = 8;
constexpr int kWBytes = kPanelsPerTile * 2048;
constexpr int kSBytes = kPanelsPerTile * 128;

template <int MT>
struct Geometry {
  static constexpr int kABytes = MT * 4 * 1024;
  static constexpr int kStage = kWBytes + kSBytes + kABytes;
  static constexpr int kLoadsPerStage = 4 + MT + 1;  // per wave: W, A, S instructions
};

template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ inline void dma16(const void *src, void *lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_wave_base, 16, 0, 0);
}

template <int MT>
__device__ inline void issue_stage(uint8_t *stage, const f16 *__restrict__ A,
                                   const uint8_t *__restrict__ qs, const f16 *__restrict__ sc,
                                   uint32_t M, uint32_t K, uint32_t m0, uint32_t p0,
                                   uint32_t np, uint32_t c, uint32_t wave, uint32_t lane) {
  uint8_t *Ws = stage;
  uint8_t *Ss = stage + kWBytes;
  uint8_t *As = stage + kWBytes + kSBytes;
  // W: wave w copies chunk blocks b = 4w..4w+3 (panel b/2, half b%2)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t b = wave * 4 + i, t = b >> 1, j = b & 1;
    uint32_t p = p0 + t;
    p = p < np ? p : np - 1;  // panels past N: valid bytes, results never stored
    const uint8_t *src = qs + panel_chunk_qs(K, p, kPanelRows, c) + j * 1024 + lane * 16;
    dma16(src, Ws + t * 2048 + j * 1024);
  }
  // A: wave w copies blocks b = w*MT .. w*MT+MT-1, block b = (m-tile b/4, step b%4)
  const uint32_t h = lane >> 5, r = lane & 31;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const uint32_t b = wave * MT + i, mi = b >> 2, s = b & 3;
    uint32_t m = m0 + mi * 32 + r;
    m = m < M ? m : M - 1;  // rows past M: valid bytes, results never stored
    const f16 *src = A + (size_t)m * K + c * kChunkK + h * 32 + s * 8;
    dma16(src, As + b * 1024);
  }
  // S: wave w copies the 2 x 128 B scale blocks of panels 2w, 2w+1 (16 lanes)
  if (lane < 16) {
    const uint32_t t = wave * 2 + (lane >> 3), q = lane & 7;
    uint32_t p = p0 + t;
    p = p < np ? p : np - 1;
    const f16 *src = sc + panel_chunk_sc(K, p, kPanelRows, c) + q * 8;
    dma16(src, Ss + wave * 256);
  }
}

template <int MT, int EPI, int NSTAGES>
__global__ __launch_bounds__(256) void q8_gemm_kernel(const f16 *__restrict__ A,
                                                      const uint8_t *__restrict__ qs,
                                                      const f16 *__restrict__ sc,
                                                      f16 *__restrict__ Cout,
                                                      const float *__restrict__ bias, uint32_t M,
                                                      uint32_t N, uint32_t K, uint32_t tiles_m,
                                                      uint32_t tiles_n, uint32_t group_m) {
  using G = Geometry<MT>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NSTAGES * G::kStage];

  // ---- tile order: consecutive workgroups go to different XCDs (round-robin),
  // so renumber to give each XCD a contiguous run, then walk that run in
  // groups of `group_m` M-tiles so an XCD's tiles share A rows and W panels
  // in its own L2.
  const uint32_t T = tiles_m * tiles_n;
  uint32_t bid = blockIdx.x;
  if (T % 8 == 0) bid = (bid % 8) * (T / 8) + bid / 8;
  const uint32_t per_group = group_m * tiles_n;
  const uint32_t gi = bid / per_group, first_m = gi * group_m;
  const uint32_t gm = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
  const uint32_t tm = first_m + (bid % per_group) % gm;
  const uint32_t tn = (bid % per_group) / gm;

  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t m0 = tm * 32 * MT, p0 = tn * kPanelsPerTile;
  const uint32_t np = N / kPanelRows, nchunks = K / kChunkK;

  f32x16 acc[2][MT];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[t][i] = (f32x16){};

#pragma unroll
  for (int st = 0; st < NSTAGES - 1; ++st)
    if (st < (int)nchunks)
      issue_stage<MT>(smem + st * G::kStage, A, qs, sc, M, K, m0, p0, np, st, wave, lane);

  for (uint32_t c = 0; c < nchunks; ++c) {
    // chunk c's DMA (this wave's part) has landed once at most the later
    // stages' loads are outstanding; the barrier makes every wave's part visible
    // and frees the slot the next issue overwrites.
    if (c + NSTAGES - 2 < nchunks)
      wait_vmcnt<(NSTAGES - 2) * G::kLoadsPerStage>();
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    {
      const uint32_t cn = c + NSTAGES - 1;
      if (cn < nchunks)
        issue_stage<MT>(smem + (cn % NSTAGES) * G::kStage, A, qs, sc, M, K, m0, p0, np, cn,
                        wave, lane);
    }
    const uint8_t *stage = smem + (c % NSTAGES) * G::kStage;
    const uint8_t *Ws = stage;
    const f16 *Ss = reinterpret_cast<const f16 *>(stage + kWBytes);
    const uint8_t *As = stage + kWBytes + kSBytes;

    f16x8 wf[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t tp = wave * 2 + t;
      const u32x4 u0 = *reinterpret_cast<const u32x4 *>(Ws + tp * 2048 + lane * 16);
      const u32x4 u1 = *reinterpret_cast<const u32x4 *>(Ws + tp * 2048 + 1024 + lane * 16);
      const f16 s = Ss[tp * 64 + lane];
      dequant16(u0, s, wf[t][0], wf[t][1]);
      dequant16(u1, s, wf[t][2], wf[t][3]);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      f16x8 bf[MT];
#pragma unroll
      for (int i = 0; i < MT; ++i)
        bf[i] = *reinterpret_cast<const f16x8 *>(As + (i * 4 + s) * 1024 + lane * 16);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < MT; ++i)
          acc[t][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[t][s], bf[i], acc[t][i], 0, 0, 0);
    }
  }

  // ---- epilogue: lane holds D[n][m] for m = l%32, n = 8g + 4(l/32) + (0..3)
  const uint32_t h = lane >> 5, col = lane & 31;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const uint32_t nb = (p0 + wave * 2 + t) * kPanelRows;
    if (nb >= N) continue;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const uint32_t m = m0 + i * 32 + col;
      if (m >= M) continue;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t n = nb + g * 8 + h * 4;
        float v[4] = {acc[t][i][g * 4 + 0], acc[t][i][g * 4 + 1], acc[t][i][g * 4 + 2],
                      acc[t][i][g * 4 + 3]};
        if constexpr (EPI != MADI_EPI_NONE) {
          const f32x4 b4 = *reinterpret_cast<const f32x4 *>(bias + n);
          v[0] += b4.x;
          v[1] += b4.y;
          v[2] += b4.z;
          v[3] += b4.w;
          if constexpr (EPI == MADI_EPI_BIAS_GELU) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gelu_erf(v[e]);
          }
        }
        const f16x4 o = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
        *reinterpret_cast<f16x4 *>(Cout + (size_t)m * N + n) = o;
      }
    }
  }
}

template <int MT, int EPI>
int launch_gemm(const f16 *A, const uint8_t *qs, const f16 *sc, f16 *C, const float *bias,
                uint32_t M, uint32_t N, uint32_t K) {
  constexpr int NSTAGES = MT >= 4 ? 3 : 4;
  const uint32_t tiles_m = (M + 32 * MT - 1) / (32 * MT);
  const uint32_t tiles_n = (N + 255) / 256;
  const uint32_t group_m = tiles_m < 6 ? tiles_m : 6;
  hipLaunchKernelGGL((q8_gemm_kernel<MT, EPI, NSTAGES>), dim3(tiles_m * tiles_n), dim3(256), 0,
                     stream(), A, qs, sc, C, bias, M, N, K, tiles_m, tiles_n, group_m);
  return check_launch("madi_q8_gemm");
}

template <int MT>
int dispatch_epi(int epi, const f16 *A, const uint8_t *qs, const f16 *sc, f16 *C,
                 const float *bias, uint32_t M, uint32_t N, uint32_t K) {
  switch (epi) {
  case MADI_EPI_NONE: return launch_gemm<MT, MADI_EPI_NONE>(A, qs, sc, C, bias, M, N, K);
  case MADI_EPI_BIAS: return launch_gemm<MT, MADI_EPI_BIAS>(A, qs, sc, C, bias, M, N, K);
  case MADI_EPI_BIAS_GELU: return launch_gemm<MT, MADI_EPI_BIAS_GELU>(A, qs, sc, C, bias, M, N, K);
  default: return fail(MADI_ERR_ARG, "madi_q8_gemm: unknown epilogue %d", epi);
  }
}

}  // namespace

extern "C" int madi_q8_gemm(const void *a, const void *qs, const void *scales, void *c,
                            const float *bias, uint32_t m, uint32_t n, uint32_t k, int epilogue) {
  if (!a || !qs || !scales || !c) return fail(MADI_ERR_NULL, "madi_q8_gemm: null pointer");
  if (epilogue != MADI_EPI_NONE && !bias) return fail(MADI_ERR_NULL, "madi_q8_gemm: null bias");
  if (epilogue == MADI_EPI_BIAS_RES)
    return fail(MADI_ERR_ARG, "madi_q8_gemm: the residual epilogue exists for the GEMV only");
  if (m == 0 || n == 0 || k == 0 || n % kPanelRows || k % kChunkK)
    return fail(MADI_ERR_SHAPE, "madi_q8_gemm: m=%u n=%u k=%u (need n %% 32 == 0, k %% 64 == 0)", m, n, k);
  if (!aligned(a, 16) || !aligned(qs, 16) || !aligned(scales, 16) || !aligned(c, 8) ||
      (bias && !aligned(bias, 16)))
    return fail(MADI_ERR_ALIGN, "madi_q8_gemm: a/qs/scales/bias need 16-byte, c 8-byte alignment");
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_q8_gemm: madi_init has not succeeded");
  const f16 *A = static_cast<const f16 *>(a);
  const uint8_t *Q = static_cast<const uint8_t *>(qs);
  const f16 *S = static_cast<const f16 *>(scales);
  f16 *C = static_cast<f16 *>(c);
  if (m <= 32) return dispatch_epi<1>(epilogue, A, Q, S, C, bias, m, n, k);
  if (m <= 64) return dispatch_epi<2>(epilogue, A, Q, S, C, bias, m, n, k);
  return dispatch_epi<4>(epilogue, A, Q, S, C, bias, m, n, k);
}
