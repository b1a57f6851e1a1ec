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
//   A  32*MT rows x 128 B (64 f16), row-major with the 16-byte chunks of row r
//      XOR-swizzled by (r >> 1) & 7; each DMA instruction copies 8 whole rows
//      (eight 128-byte lines, fully coalesced), and the MFMA fragment reads
//      (16 consecutive rows, one chunk each) hit 16 distinct bank groups
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
constexpr int kWaves = 8;  // two waves per SIMD
constexpr int kWBytes = kPanelsPerTile * 2048;
constexpr int kSBytes = kPanelsPerTile * 128;
constexpr int NSTAGES = 4;

template <int MT>
struct Geometry {
  static constexpr int kABytes = MT * 4 * 1024;
  static constexpr int kStage = kWBytes + kSBytes + kABytes;
  // DMA instructions per wave per stage: two weight halves of its panel, its
  // share of the A row groups, and scales (see issue_stage)
  static constexpr int kLoadsPerStage = MT == 1 ? 3 : 2 + MT / 2 + 1;
};

template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ inline void dma16(const void *src, void *lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_wave_base, 16, 0, 0);
}

// XOR swizzle of the A tile's 16-byte chunks within row `row`
__device__ inline uint32_t a_swz(uint32_t row) { return (row >> 1) & 7; }

// DMA of one ring stage (chunk c), in four parts.  Wave v copies: part 0/1,
// the two 1 KiB halves of panel v's chunk block; part 2, its A row groups
// (8 rows x 128 B each, fully coalesced) g = v, v+8, ... < 4*MT; part 3 the
// scales: its own panel's 128 B (MT >= 2), or, for MT == 1 where waves 4..7
// have no row group, 256 B covering panels 2(v-4), 2(v-4)+1.  Every wave
// issues Geometry<MT>::kLoadsPerStage instructions per stage.  The parts ride
// between the MFMAs of the four k-steps, so the vector-memory pipe drains
// while the matrix pipe is busy.
template <int MT>
__device__ inline void issue_part(uint8_t *stage, int part, const f16 *__restrict__ A,
                                  const uint8_t *__restrict__ qs, const f16 *__restrict__ sc,
                                  uint32_t M, uint32_t K, uint32_t m0, uint32_t p0, uint32_t np,
                                  uint32_t c, uint32_t wave, uint32_t lane) {
  uint8_t *Ws = stage;
  uint8_t *Ss = stage + kWBytes;
  uint8_t *As = stage + kWBytes + kSBytes;
  if (part < 2) {
    uint32_t p = p0 + wave;
    p = p < np ? p : np - 1;  // panels past N: valid bytes, results never stored
    dma16(qs + panel_chunk_qs(K, p, kPanelRows, c) + part * 1024 + lane * 16,
          Ws + wave * 2048 + part * 1024);
  } else if (part == 2) {
    // lane l fills physical chunk l%8 of row 8g + l/8 with the logical chunk
    // that the swizzle stores there
#pragma unroll
    for (int g = (int)wave; g < 4 * MT; g += kWaves) {
      const uint32_t row = g * 8 + (lane >> 3);
      const uint32_t q = (lane & 7) ^ a_swz(row);
      uint32_t m = m0 + row;
      m = m < M ? m : M - 1;  // rows past M: valid bytes, results never stored
      dma16(A + (size_t)m * K + c * kChunkK + q * 8, As + g * 1024);
    }
  } else {
    if constexpr (MT == 1) {
      if (wave >= 4 && lane < 16) {
        const uint32_t t = (wave - 4) * 2 + (lane >> 3), q = lane & 7;
        uint32_t pp = p0 + t;
        pp = pp < np ? pp : np - 1;
        dma16(sc + panel_chunk_sc(K, pp, kPanelRows, c) + q * 8, Ss + (wave - 4) * 256);
      }
    } else {
      uint32_t p = p0 + wave;
      p = p < np ? p : np - 1;
      if (lane < 8) dma16(sc + panel_chunk_sc(K, p, kPanelRows, c) + lane * 8, Ss + wave * 128);
    }
  }
}

template <int MT>
__device__ inline void issue_stage(uint8_t *stage, const f16 *__restrict__ A,
                                   const uint8_t *__restrict__ qs, const f16 *__restrict__ sc,
                                   uint32_t M, uint32_t K, uint32_t m0, uint32_t p0, uint32_t np,
                                   uint32_t c, uint32_t wave, uint32_t lane) {
#pragma unroll
  for (int part = 0; part < 4; ++part)
    issue_part<MT>(stage, part, A, qs, sc, M, K, m0, p0, np, c, wave, lane);
}

// The MT activation fragments of k-step s from an A tile (swizzled rows).
template <int MT>
__device__ inline void load_a_frags(const uint8_t *As, int s, uint32_t h, uint32_t r,
                                    f16x8 (&bf)[MT]) {
  const uint32_t phys = ((h * 4 + s) ^ a_swz(r)) * 16;  // rows i*32 + r share (r >> 1) & 7
#pragma unroll
  for (int i = 0; i < MT; ++i)
    bf[i] = *reinterpret_cast<const f16x8 *>(As + (i * 32 + r) * 128 + phys);
}

// One 16-byte weight unit (half j of this wave's panel) of the chunk in
// `stage`, dequantised into two k-steps.
__device__ inline void dequant_unit(const uint8_t *stage, uint32_t wave, uint32_t lane, int j,
                                    f16 s, f16x8 &lo, f16x8 &hi) {
  const u32x4 u = *reinterpret_cast<const u32x4 *>(stage + wave * 2048 + j * 1024 + lane * 16);
  dequant16(u, s, lo, hi);
}

__device__ inline f16 panel_scale(const uint8_t *stage, uint32_t wave, uint32_t lane) {
  return reinterpret_cast<const f16 *>(stage + kWBytes)[wave * 64 + lane];
}

template <int MT, int EPI>
__global__ __launch_bounds__(512) void q8_gemm_kernel(const f16 *__restrict__ A,
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
  const uint32_t h = lane >> 5, r = lane & 31;
  const uint32_t m0 = tm * 32 * MT, p0 = tn * kPanelsPerTile;
  const uint32_t np = N / kPanelRows, nchunks = K / kChunkK;

  f32x16 acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = (f32x16){};

  // ---- software pipeline over a four-slot ring.  At iteration c: chunk c's
  // activation fragments feed this iteration's MFMAs (its weights were
  // dequantised during iteration c-1), chunk c+1's weights are dequantised
  // between the MFMAs, chunk c+2 is in flight and chunk c+3 is issued, a part
  // per k-step, into the slot chunk c-1 left (free once every wave passed
  // this iteration's barrier).
#pragma unroll
  for (int st = 0; st < NSTAGES - 1; ++st)
    if (st < (int)nchunks)
      issue_stage<MT>(smem + st * G::kStage, A, qs, sc, M, K, m0, p0, np, st, wave, lane);
  if (nchunks >= 3)
    wait_vmcnt<2 * G::kLoadsPerStage>();
  else
    wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();

  f16x8 wcur[4], wnext[4];
  {
    const f16 s0 = panel_scale(smem, wave, lane);
    dequant_unit(smem, wave, lane, 0, s0, wcur[0], wcur[1]);
    dequant_unit(smem, wave, lane, 1, s0, wcur[2], wcur[3]);
  }
  f16x8 bcur[MT], bnext[MT];
  load_a_frags<MT>(smem + kWBytes + kSBytes, 0, h, r, bcur);

  for (uint32_t c = 0; c < nchunks; ++c) {
    if (c + 1 < nchunks) {
      // chunk c+1 has landed once only chunk c+2's loads may be outstanding;
      // the barrier publishes every wave's part and retires slot c-1
      if (c + 2 < nchunks)
        wait_vmcnt<G::kLoadsPerStage>();
      else
        wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
    }
    const bool refill = c + 3 < nchunks;  // chunk c+3's DMA rides between the steps
    uint8_t *Rs = smem + ((c + 3) % NSTAGES) * G::kStage;
    // Branch-free compute region; on the last chunk the "next" slot holds
    // stale, in-bounds bytes whose dequantised values are never used.
    const uint8_t *As = smem + (c % NSTAGES) * G::kStage + kWBytes + kSBytes;
    const uint8_t *Wn = smem + ((c + 1) % NSTAGES) * G::kStage;
    const uint8_t *An = Wn + kWBytes + kSBytes;
    const f16 snext = panel_scale(Wn, wave, lane);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s < 3)
        load_a_frags<MT>(As, s + 1, h, r, bnext);
      else
        load_a_frags<MT>(An, 0, h, r, bnext);
      if (s == 1) dequant_unit(Wn, wave, lane, 0, snext, wnext[0], wnext[1]);
      if (s == 3) dequant_unit(Wn, wave, lane, 1, snext, wnext[2], wnext[3]);
#pragma unroll
      for (int i = 0; i < MT; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wcur[s], bcur[i], acc[i], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < MT; ++i) bcur[i] = bnext[i];
      if (refill) issue_part<MT>(Rs, s, A, qs, sc, M, K, m0, p0, np, c + 3, wave, lane);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) wcur[s] = wnext[s];
  }

  // ---- epilogue: lane holds D[n][m] for m = l%32, n = 8g + 4(l/32) + (0..3)
  const uint32_t nb = (p0 + wave) * kPanelRows;
  if (nb >= N) return;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const uint32_t m = m0 + i * 32 + r;
    if (m >= M) continue;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t n = nb + g * 8 + h * 4;
      float v[4] = {acc[i][g * 4 + 0], acc[i][g * 4 + 1], acc[i][g * 4 + 2], acc[i][g * 4 + 3]};
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

template <int MT, int EPI>
int launch_gemm(const f16 *A, const uint8_t *qs, const f16 *sc, f16 *C, const float *bias,
                uint32_t M, uint32_t N, uint32_t K) {
  const uint32_t tiles_m = (M + 32 * MT - 1) / (32 * MT);
  const uint32_t tiles_n = (N + 255) / 256;
  const uint32_t group_m = tiles_m < 6 ? tiles_m : 6;
  hipLaunchKernelGGL((q8_gemm_kernel<MT, EPI>), dim3(tiles_m * tiles_n), dim3(kWaves * 64), 0,
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
