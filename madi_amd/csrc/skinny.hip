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
// Workgroup: P weight panels (32 rows each; P = 4 for the 51866-row vocab
// matrix from 9 rows, 2 for narrow weights at prefill sizes (panel pairs),
// 1 otherwise) x one slice of 32 activation rows (the MFMA columns), KW
// waves splitting K.  Per 64-wide K chunk a wave loads each panel's two
// 16-byte units per lane (lane (h, r): row r's 32 weights of quantisation
// block h) and scale, and the slice's first XR rows (8, 16 or 32: the rows a
// batch of M <= XR has) of 64 f32 activations with coalesced loads (each
// instruction: four whole 256-byte row segments), rounds them to f16 into its
// own LDS tile and reads them back as MFMA fragments (lane (h, c): row c, the
// same 32 k; columns c >= XR are zeros without a load).  Four
// v_mfma_f32_32x32x16_f16 per panel and chunk, with the weight as the A operand
// (rows n) and the activations as B (columns m); K order of step s: k = 32h +
// 8s + e for both operands, as in the GEMM.  Activation rows past M load as
// zeros (outside the buffer resource).  The projections of a decode step are
// small (1.6 - 6.5 MB of weights), so their time is load latency: each wave
// keeps WIN chunks in flight, enough that the K range of most waves is one
// round of loads; the single-panel f32 launches load that whole first window's
// activations ahead of its weights and stage them while the weights are in
// flight.  The K partial tiles meet in LDS and four waves store one quarter
// each.
#include "common.h"

using namespace madi;

namespace {

constexpr uint32_t kSlice = 32;  // activation rows per workgroup (MFMA columns)

typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ inline rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// Per-wave constants of the loads.
template <int P>
struct Plan {
  rsrc_t wq, ws, xr;
  uint32_t K;
  uint32_t p[P], R[P];           // panels (clamped to the last one) and their row counts
  uint32_t w_voff[P], s_voff[P];  // this lane's unit / scale offsets in each panel
  uint32_t x_voff;               // this lane's activation offset (coalesced pattern)
};

// One chunk's loads for a lane: two weight units and the block scale per
// panel, and XR/4 x 16 bytes of activations in a coalesced pattern: piece i
// is row 4i + lane/16, floats 4 * (lane % 16) .. +3 of the chunk (each load
// instruction reads four whole 256-byte row segments).
//
// With f16 activations (H) and a full 32-row slice the MFMA fragments come
// straight from memory: lane (h, c) loads row c's 16 bytes of piece 4h + s for
// each k-step s.  For 8 or 16 rows most of those lanes would load rows past
// the batch (zeros, outside the activation resource), so the rows are staged
// instead, as the f32 ones: one coalesced 16-byte piece per lane and 8 rows
// (piece lane % 8 of row lane / 8), copied into the wave's LDS tile and read
// back as fragments.
template <int XR, bool H>
constexpr bool kStagedH = H && XR < 32;

template <int P, int XR, bool H = false>
struct Chunk {
  u32x4 w[P][2];
  uint32_t s[P];
  f32x4 x[H ? 1 : XR / 4];
  u32x4 xh[H ? (kStagedH<XR, H> ? XR / 8 : 4) : 1];
};

template <int P, int XR, bool H>
__device__ inline void load_weights(Chunk<P, XR, H> &b, const Plan<P> &pl, rsrc_t wq, rsrc_t ws,
                                    uint32_t c) {
#pragma unroll
  for (int t = 0; t < P; ++t) {
    const uint32_t so = (uint32_t)panel_chunk_qs(pl.K, pl.p[t], pl.R[t], c);
    b.w[t][0] = __builtin_amdgcn_raw_buffer_load_b128(wq, pl.w_voff[t], so, 0);
    b.w[t][1] = __builtin_amdgcn_raw_buffer_load_b128(wq, pl.w_voff[t] + 2 * pl.R[t] * 16, so, 0);
    b.s[t] = __builtin_amdgcn_raw_buffer_load_b16(
        ws, pl.s_voff[t], (uint32_t)panel_chunk_sc(pl.K, pl.p[t], pl.R[t], c) * 2, 0);
  }
}
template <int P, int XR, bool H>
__device__ inline void load_acts(Chunk<P, XR, H> &b, const Plan<P> &pl, rsrc_t xr, uint32_t c) {
  if constexpr (kStagedH<XR, H>) {
#pragma unroll
    for (int i = 0; i < XR / 8; ++i)
      b.xh[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, pl.x_voff + i * 8 * pl.K * 2,
                                                      c * kChunkK * 2, 0);
  } else if constexpr (H) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      b.xh[s] = __builtin_amdgcn_raw_buffer_load_b128(xr, pl.x_voff, c * kChunkK * 2 + s * 16, 0);
  } else {
#pragma unroll
    for (int i = 0; i < XR / 4; ++i)
      b.x[i] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, pl.x_voff + i * 16 * pl.K, c * kChunkK * 4, 0));
  }
}
template <int P, int XR, bool H>
__device__ inline void load_chunk(Chunk<P, XR, H> &b, const Plan<P> &pl, uint32_t c) {
  load_weights(b, pl, pl.wq, pl.ws, c);
  load_acts(b, pl, pl.xr, c);
}

// The wave's activation tile of one chunk in LDS: 32 rows x 64 f16, 128 bytes
// per row, 16-byte pieces of row c XOR-swizzled by (c >> 1) & 7 so the
// fragment reads (32 rows, one piece each) and the staging writes spread over
// all banks.
__device__ inline uint32_t x_piece(uint32_t row, uint32_t j) {
  return row * 128 + ((j ^ ((row >> 1) & 7)) * 16);
}

// f32 activations of a chunk -> f16 (round to nearest even, the kCvt32
// staging) into the wave's LDS tile, 8 bytes per piece
template <int P, int XR, bool H>
__device__ inline void stage_acts(const Chunk<P, XR, H> &b, uint8_t *xt, uint32_t lane) {
#pragma unroll
  for (int i = 0; i < XR / 4; ++i) {
    const uint32_t row = 4 * i + (lane >> 4), k4 = lane & 15;  // floats 4*k4 .. +3
    const f16x4 v = {(f16)b.x[i].x, (f16)b.x[i].y, (f16)b.x[i].z, (f16)b.x[i].w};
    *reinterpret_cast<f16x4 *>(xt + x_piece(row, k4 >> 1) + (k4 & 1) * 8) = v;
  }
}

// The four k-steps' activation fragments of a staged chunk: piece 4h + s of
// row c (zeros for columns c >= XR)
template <int XR>
__device__ inline void read_frags(const uint8_t *xt, uint32_t lane, f16x8 (&xf)[4]) {
  const uint32_t h = lane >> 5, c = lane & 31;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    xf[s] = (f16x8){};
    if (XR == 32 || c < XR) xf[s] = *reinterpret_cast<const f16x8 *>(xt + x_piece(c, 4 * h + s));
  }
}

// acc[t] += W_t(chunk) . X(chunk)^T over the four k-steps; step s uses half
// (s & 1) of weight unit s >> 1 and activation fragment s.
template <int P, int XR, bool H>
__device__ inline void mfma_chunk(const Chunk<P, XR, H> &b, const f16x8 (&xfr)[4],
                                  f32x16 (&acc)[P]) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const f16x8 xf = xfr[s];
#pragma unroll
    for (int t = 0; t < P; ++t) {
      const f16x2 s2 = {__builtin_bit_cast(f16, (uint16_t)b.s[t]),
                        __builtin_bit_cast(f16, (uint16_t)b.s[t])};
      const u32x4 u = b.w[t][s >> 1];
      const uint32_t b0 = (s & 1) ? u.z : u.x, b1 = (s & 1) ? u.w : u.y;
      const f16x2 a0 = dequant_pair(b0, kSelLo, s2), a1 = dequant_pair(b0, kSelHi, s2);
      const f16x2 a2 = dequant_pair(b1, kSelLo, s2), a3 = dequant_pair(b1, kSelHi, s2);
      const f16x8 wf = {a0.x, a0.y, a1.x, a1.y, a2.x, a2.y, a3.x, a3.y};
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf, xf, acc[t], 0, 0, 0);
    }
  }
}

// One chunk: stage (f32 activations), read the fragments, MFMAs.
template <int P, int XR, bool H>
__device__ inline void accumulate(const Chunk<P, XR, H> &b, uint8_t *xt, uint32_t lane,
                                  f32x16 (&acc)[P]) {
  f16x8 xf[4];
  if constexpr (kStagedH<XR, H>) {
#pragma unroll
    for (int i = 0; i < XR / 8; ++i)
      *reinterpret_cast<u32x4 *>(xt + x_piece(8 * i + (lane >> 3), lane & 7)) = b.xh[i];
    read_frags<XR>(xt, lane, xf);
  } else if constexpr (H) {
#pragma unroll
    for (int s = 0; s < 4; ++s) xf[s] = __builtin_bit_cast(f16x8, b.xh[s]);
  } else {
    stage_acts(b, xt, lane);
    read_frags<XR>(xt, lane, xf);
  }
  mfma_chunk(b, xf, acc);
}


// LDS: the waves' activation tiles (XR rows x 128 bytes) during the K loop,
// then the partial sums of the reduction
// The single-panel f32 launches stage their whole first window at once: one
// tile per window slot.
template <int P, int KW, bool H>
constexpr bool kStageWindow = P == 1 && KW == 8 && !H;

template <int P, int KW, int XR, int WIN, bool H>
constexpr int skinny_lds() {
  constexpr int tiles = KW * XR * 128 * (kStageWindow<P, KW, H> ? WIN : 1);
  return tiles > KW * P * 4 * 64 * 16 ? tiles : KW * P * 4 * 64 * 16;
}

// P panels per workgroup, KW waves splitting K, XR activation rows loaded per
// slice, WIN chunks in flight per wave.
//
// Grid (x, y, z) = (panel group, 32-row activation slice, K split).  The
// arguments are scalars in the order the kernel first needs them, so the
// leading ones arrive preloaded in SGPRs, and the set-up has no integer
// division: split s covers chunks [s * cper + min(s, crem), + cper + (s <
// crem)).  `x`, `out`: f32 [m][k], [m][n], or with H f16 [m][k], [m][n] (the
// sum rounded once to f16); `ws`, `cnt`: partial tiles and arrival counters
// (zero between uses) when K is split.
template <int P, int KW, int XR, int WIN, bool H = false>
__global__ __launch_bounds__(KW * 64) __attribute__((amdgpu_waves_per_eu(KW / 4 > 2 ? KW / 4 : 2))) void q8_skinny_kernel(
    const uint8_t *__restrict__ qs, const f16 *__restrict__ sc, const void *__restrict__ x,
    uint32_t M, uint32_t N, uint32_t K, uint32_t cper, uint32_t crem, uint32_t groups,
    void *__restrict__ out, f32x4 *ws, uint32_t *cnt) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[skinny_lds<P, KW, XR, WIN, H>()];

  // Consecutive workgroups go to different XCDs (round-robin, x fastest).
  // The grid's x extent is a multiple of 8, so every slice and K split of
  // panel group g runs on XCD g % 8 and shares its weights in that L2.
  const uint32_t grp = blockIdx.x, slice = blockIdx.y, split = blockIdx.z;
  if (grp >= groups) return;
  const uint32_t splits = gridDim.z;

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t h = lane >> 5, r = lane & 31;
  const uint32_t np = (N + kPanelRows - 1) / kPanelRows;
  // this workgroup's K chunks [cs, cs + nck), split KW ways over the waves
  const uint32_t cs = split * cper + (split < crem ? split : crem);
  const uint32_t nck = cper + (split < crem ? 1 : 0);
  const uint32_t c0 = cs + (wave * nck) / KW, c1 = cs + ((wave + 1) * nck) / KW;

  // Panels past N are clamped to the last one and lanes past a partial
  // panel's last row read row R-1 (in bounds; their sums are never stored).
  // The activation resource covers the slice's rows that exist, so rows past
  // M read zeros.
  Plan<P> pl;
  pl.K = K;
  pl.wq = make_rsrc(qs, N * K);
  pl.ws = make_rsrc(sc, N * (K / 32) * 2);
#pragma unroll
  for (int t = 0; t < P; ++t) {
    const uint32_t pp = grp * P + t < np ? grp * P + t : np - 1;
    pl.p[t] = pp;
    pl.R[t] = panel_rows(N, pp);
    const uint32_t rr = r < pl.R[t] ? r : pl.R[t] - 1;
    pl.w_voff[t] = (h * pl.R[t] + rr) * 16;
    pl.s_voff[t] = (h * pl.R[t] + rr) * 2;
  }
  const uint32_t m0 = slice * kSlice;
  const uint32_t rows = M - m0 < kSlice ? M - m0 : kSlice;
  constexpr uint32_t xb = H ? 2 : 4;  // bytes per activation
  pl.xr = make_rsrc(static_cast<const uint8_t *>(x) + (size_t)m0 * K * xb, rows * K * xb);
  pl.x_voff = kStagedH<XR, H> ? (lane >> 3) * K * 2 + (lane & 7) * 16
             : H                ? r * K * 2 + h * 64
                                : (lane >> 4) * K * 4 + (lane & 15) * 16;

  constexpr bool kStage = kStageWindow<P, KW, H>;
  uint8_t *xt = smem + wave * XR * 128 * (kStage ? WIN : 1);
  Chunk<P, XR, H> win[WIN];
  f32x16 acc[P];
#pragma unroll
  for (int t = 0; t < P; ++t) acc[t] = (f32x16){};
  uint32_t cfirst = c0;
  if constexpr (kStage) {
    // The first window at once: every slot's activations are loaded before
    // any weight, staged into the slot's own tile and read back as fragments
    // while the weights are still in flight, so the LDS round trip is off
    // the path from the weights' arrival to the MFMAs.  Slots past the range
    // load through zero-length resources (no memory access, zeros), which
    // keeps every load unconditional and the waits exact.
    const rsrc_t z = make_rsrc(qs, 0);
#pragma unroll
    for (int i = 0; i < WIN; ++i) load_acts(win[i], pl, c0 + i < c1 ? pl.xr : z, c0 + i);
#pragma unroll
    for (int i = 0; i < WIN; ++i)
      load_weights(win[i], pl, c0 + i < c1 ? pl.wq : z, c0 + i < c1 ? pl.ws : z, c0 + i);
    f16x8 xf[WIN][4];
#pragma unroll
    for (int i = 0; i < WIN; ++i) {
      stage_acts(win[i], xt + i * XR * 128, lane);
      read_frags<XR>(xt + i * XR * 128, lane, xf[i]);
    }
    __builtin_amdgcn_sched_barrier(0);
    // zero slots add exactly nothing (their weights and scales are zeros)
#pragma unroll
    for (int i = 0; i < WIN; ++i) {
      mfma_chunk(win[i], xf[i], acc);
      if (c0 + i + WIN < c1) load_chunk<P, XR, H>(win[i], pl, c0 + i + WIN);
    }
    cfirst = c0 + WIN;
  } else {
#pragma unroll
    for (int i = 0; i < WIN; ++i)
      if (c0 + i < c1) load_chunk<P, XR, H>(win[i], pl, c0 + i);
  }
#pragma unroll 1
  for (uint32_t c = cfirst; c < c1; c += WIN) {
#pragma unroll
    for (int i = 0; i < WIN; ++i) {
      if (c + i < c1) {
        accumulate<P, XR, H>(win[i], xt, lane, acc);
        if (c + i + WIN < c1) load_chunk<P, XR, H>(win[i], pl, c + i + WIN);
      }
    }
  }

  // Lane (h, c) holds D[n][m] of panel t for m = m0 + c and
  // n = 32 p_t + 8g + 4h + e (acc[t][4g + e]).  Wave w < 4 sums group g = w
  // of every panel over the KW K ranges.
  __syncthreads();  // every wave is done with its activation tile
  f32x4 *red = reinterpret_cast<f32x4 *>(smem);  // [wave][t][g][lane]
#pragma unroll
  for (int t = 0; t < P; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      red[((wave * P + t) * 4 + g) * 64 + lane] =
          (f32x4){acc[t][4 * g], acc[t][4 * g + 1], acc[t][4 * g + 2], acc[t][4 * g + 3]};
  __syncthreads();
  f32x4 v[P];
  if (wave < 4) {
#pragma unroll
    for (int t = 0; t < P; ++t) {
      v[t] = red[((0 * P + t) * 4 + wave) * 64 + lane];
#pragma unroll
      for (int w = 1; w < KW; ++w) v[t] += red[((w * P + t) * 4 + wave) * 64 + lane];
    }
  }
  if (splits > 1) {
    // Split K: each workgroup writes its partial tile through to memory
    // (device-scope sc1 stores) and counts itself in; the last to arrive adds
    // the splits' partials in split order and stores the rows.
    __shared__ uint32_t arrived;
    constexpr int kSc1 = 16;
    const uint32_t tile = grp * gridDim.y + slice;
    const uint32_t part = P * 4 * 64 * 16;  // bytes per partial tile
    const __amdgpu_buffer_rsrc_t wsr = make_rsrc(ws, groups * gridDim.y * splits * part);
    if (wave < 4) {
#pragma unroll
      for (int t = 0; t < P; ++t)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[t]), wsr,
                                               ((t * 4 + wave) * 64 + lane) * 16,
                                               (tile * splits + split) * part, kSc1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
      arrived = __hip_atomic_fetch_add(&cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != splits - 1) return;
    if (wave < 4) {
#pragma unroll
      for (int t = 0; t < P; ++t) {
        v[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t s2 = 0; s2 < splits; ++s2)
          v[t] += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                wsr, ((t * 4 + wave) * 64 + lane) * 16,
                                                (tile * splits + s2) * part, kSc1));
      }
    }
    if (threadIdx.x == 0)
      __hip_atomic_store(&cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const uint32_t m = m0 + r;
  if (wave >= 4 || m >= M) return;
  const uint32_t nl = wave * 8 + h * 4;  // panel-local row of v.x
#pragma unroll
  for (int t = 0; t < P; ++t) {
    if (grp * P + t >= np) break;
    const uint32_t R = pl.R[t];
    if constexpr (H) {
      f16 *o = static_cast<f16 *>(out) + (size_t)m * N + pl.p[t] * kPanelRows + nl;
      const f16x4 hv = {(f16)v[t].x, (f16)v[t].y, (f16)v[t].z, (f16)v[t].w};
      if (nl + 4 <= R) {
        // o is 8-byte aligned when N % 4 == 0 and 4-byte aligned when N is
        // even (out is 16-byte aligned and 32 p + nl is a multiple of 4)
        if (N % 4 == 0) {
          *reinterpret_cast<f16x4 *>(o) = hv;
        } else if (N % 2 == 0) {
          reinterpret_cast<f16x2 *>(o)[0] = (f16x2){hv.x, hv.y};
          reinterpret_cast<f16x2 *>(o)[1] = (f16x2){hv.z, hv.w};
        } else {
          o[0] = hv.x;
          o[1] = hv.y;
          o[2] = hv.z;
          o[3] = hv.w;
        }
      } else {
        if (nl + 0 < R) o[0] = hv.x;
        if (nl + 1 < R) o[1] = hv.y;
        if (nl + 2 < R) o[2] = hv.z;
      }
      continue;
    }
    float *o = static_cast<float *>(out) + (size_t)m * N + pl.p[t] * kPanelRows + nl;
    if (nl + 4 <= R) {
      o[0] = v[t].x;
      o[1] = v[t].y;
      o[2] = v[t].z;
      o[3] = v[t].w;
    } else {
      if (nl + 0 < R) o[0] = v[t].x;
      if (nl + 1 < R) o[1] = v[t].y;
      if (nl + 2 < R) o[2] = v[t].z;
    }
  }
}

// Launch shapes.  Single panels (decoder projections, 40 - 160 panels): eight
// waves split K, three chunks in flight each, so a K = 1280 range (2 - 3
// chunks per wave) is one round of loads.  (Sixteen waves with two chunks
// each measured slower: a workgroup's waves start up to ~0.8 us apart and the
// reduction waits for the last.)  The vocab logits (1621 panels) up to 8
// rows: one panel per workgroup and four waves splitting K, two chunks in
// flight each; 1621 workgroups spread evenly over the CUs (M = 8: 14.05 us
// against 14.92 with two panels per workgroup, cold weights).  From 9 rows
// the activations of a chunk are twice the weight bytes or more, and every
// panel's workgroup reads the whole slice, so four panels per workgroup share
// each activation load (406 workgroups, two per CU: M = 16 16.24 against
// 17.33 us with one panel, M = 32 17.2 against 19.5).
constexpr int kPanelWaves = 8, kPanelWin = 3;
constexpr int kVocabWaves = 4, kVocabWin = 2;
constexpr int kGroupWaves = 4, kGroupWin = 2;
// Panel pairs (many 32-row slices of a narrow, short weight, where a
// workgroup per panel and slice no longer fits one per CU): two panels share
// each activation load, four waves split K.
constexpr int kPairWaves = 4, kPairWin = 2;
constexpr uint32_t kMaxSplits = 4;

// One projection: out[m][n] = sum_k x[m][k] w[n][k]; x and out f32, or f16
// for the launches with H set.
struct Proj {
  void *out;
  const void *x;
  const uint8_t *qs;
  const f16 *sc;
  uint32_t m, n, k;
  const char *what;
};

template <int P, int KW, int XR, int WIN, bool H = false>
int launch_skinny(const Proj &a) {
  const uint32_t np = (a.n + kPanelRows - 1) / kPanelRows;
  const uint32_t groups = (np + P - 1) / P, slices = (a.m + kSlice - 1) / kSlice;
  const uint32_t C = a.k / kChunkK;
  // Few panels and a long K (the FFN down projection, 40 panels x 80 chunks):
  // split K over up to four workgroups per tile, >= 16 chunks each.
  uint32_t splits = 1;
  f32x4 *ws = nullptr;
  uint32_t *cnt = nullptr;
  if (P == 1 && np < 128 && C >= 32) {
    splits = C / 16 < kMaxSplits ? C / 16 : kMaxSplits;
    float *w = nullptr;
    const size_t part = (size_t)P * 4 * 64 * 16;
    if (int rc = workspace(groups * slices * splits * part, groups * slices, &w, &cnt)) return rc;
    ws = reinterpret_cast<f32x4 *>(w);
  }
  const dim3 grid((groups + 7) / 8 * 8, slices, splits);
  hipLaunchKernelGGL((q8_skinny_kernel<P, KW, XR, WIN, H>), grid, dim3(KW * 64), 0, stream(), a.qs,
                     a.sc, a.x, a.m, a.n, a.k, C / splits, C % splits, groups, a.out, ws, cnt);
  return check_launch(a.what);
}

// wide matrices (the vocab logits): one panel per workgroup up to 8 rows,
// four panels sharing each activation load for 16- and 32-row slices; narrow
// ones keep one panel per workgroup with eight waves
template <int XR, bool H = false>
int launch_rows(const Proj &a) {
  const uint32_t np = (a.n + kPanelRows - 1) / kPanelRows;
  if (np >= 1024) {
    if constexpr (XR <= 8) return launch_skinny<1, kVocabWaves, XR, kVocabWin, H>(a);
    return launch_skinny<4, kGroupWaves, XR, kGroupWin, H>(a);
  }
  return launch_skinny<1, kPanelWaves, XR, kPanelWin, H>(a);
}

}  // namespace

// Rows from which the batched projection runs as the MFMA GEMM.
#ifndef MADI_PPROJ_GEMM_ROWS
#define MADI_PPROJ_GEMM_ROWS 160
#endif
constexpr uint32_t kGemmRows = MADI_PPROJ_GEMM_ROWS;

extern "C" int madi_q8_pproj(float *out, const float *in, const void *qs, const void *scales,
                             uint32_t m, uint32_t n, uint32_t k) {
  if (!out || !in || !qs || !scales) return fail(MADI_ERR_NULL, "madi_q8_pproj: null pointer");
  if (m == 0 || n == 0 || k == 0 || k % kChunkK)
    return fail(MADI_ERR_SHAPE, "madi_q8_pproj: m=%u n=%u k=%u (need m, n > 0, k a positive multiple of 64)", m, n, k);
  // buffer offsets are 32-bit: W (n*k bytes) and one slice of activations
  // (32*k*4 bytes) must stay below 2 GiB
  if ((uint64_t)n * k >= (1ull << 31) || (uint64_t)kSlice * k * 4 >= (1ull << 31))
    return fail(MADI_ERR_SHAPE, "madi_q8_pproj: n=%u k=%u exceeds the 2 GiB operand limit", n, k);
  // the 32-row activation slices are the grid's y extent
  if ((m + kSlice - 1) / kSlice > 65535)
    return fail(MADI_ERR_SHAPE, "madi_q8_pproj: m=%u exceeds %u rows", m, 65535u * kSlice);
  if (!aligned(qs, 16) || !aligned(scales, 2) || !aligned(in, 16) || !aligned(out, 4))
    return fail(MADI_ERR_ALIGN, "madi_q8_pproj: qs and in need 16-byte alignment");
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_q8_pproj: madi_init has not succeeded");
  if (int rc = deferred_before_read(in, (size_t)m * k * 4)) return rc;
  if (int rc = deferred_before_write(out, (size_t)m * n * 4)) return rc;
  // Many rows (sequence prefill): the MFMA GEMM dequantises each weight once
  // per 32 or 64 rows of a tile that spans 128 or 256 outputs, where this
  // kernel dequantises it once per 32-row slice of a single panel.  Its tiles
  // take 7.5-11 us however few rows they hold (one K loop), so it pays from
  // 160 rows on wide or long weights (M = 320: 1280->5120 12.3 vs 27.2 us,
  // 1280->3840 12.2 vs 20.3, 5120->1280 19.0 vs 34.1; measured, cold
  // weights).  On narrower, shorter ones this kernel keeps a workgroup per
  // panel and slice while that grid fits one per CU (1280 x 1280 at M = 160
  // 4.8 us against 5.5 with panel pairs), then a workgroup per panel pair
  // while that fits (M = 224 / 288 / 320: 5.6 / 5.8 / 5.9 us against 8.0 on
  // the GEMM's 32 x 128 tiles, which leave 156 CUs idle), and only then the
  // GEMM.
  const uint64_t np = (n + kPanelRows - 1) / kPanelRows, slices = (m + kSlice - 1) / kSlice;
  const uint64_t skinny_wgs = np * slices, cus = (uint64_t)cu_count();
  if (m > kSlice && n < 2048 && k < 4096 && skinny_wgs > cus && (np + 1) / 2 * slices <= cus) {
    const Proj a{out, in, static_cast<const uint8_t *>(qs), static_cast<const f16 *>(scales), m, n,
                 k, "madi_q8_pproj"};
    return launch_skinny<2, kPairWaves, kSlice, kPairWin>(a);
  }
  if (m >= kGemmRows && (n >= 2048 || k >= 4096 || skinny_wgs > cus) &&
      n % kPanelRows == 0 && aligned(in, 16) &&
      aligned(out, 16) &&
      (uint64_t)m * k * 4 < (1ull << 31) && (uint64_t)n * 256 < (1ull << 31))
    return q8_gemm_f32io(in, qs, scales, out, m, n, k);
  const Proj a{out, in, static_cast<const uint8_t *>(qs), static_cast<const f16 *>(scales), m, n, k,
               "madi_q8_pproj"};
  // a batch of up to 8 or 16 rows loads only those activation rows
  if (m <= 8) return launch_rows<8>(a);
  if (m <= 16) return launch_rows<16>(a);
  return launch_rows<32>(a);
}

namespace madi {
// Rows from which an f16 projection on a recorded F16 copy runs the MFMA GEMM
// (madi_q8_gemm) rather than this kernel: the batched projection's rule, for
// weights whose rows fill whole 32-row panels.
bool skinny_f16_prefers_gemm(uint32_t m, uint32_t n, uint32_t k) {
  const uint64_t skinny_wgs = (uint64_t)((n + kPanelRows - 1) / kPanelRows) * ((m + kSlice - 1) / kSlice);
  return n % kPanelRows == 0 && m >= kGemmRows &&
         (n >= 2048 || k >= 4096 || skinny_wgs > (uint64_t)cu_count());
}

// out[M][N] (f16) = f16(in[M][K] (f16) . deq(W)^T), fp32 accumulation, any N
// (the vocab's 51866 rows included): matmulF16Batched on a recorded F16 copy
// of a Q8 weight (the batched decode's logits over deqW16's tok_emb copy,
// engine/metal/transcribe.zig:2391-2394).  The caller checks the pointers and
// the deferred state.
int q8_skinny_f16io(const void *in, const void *qs, const void *scales, void *out, uint32_t m,
                    uint32_t n, uint32_t k) {
  const Proj a{out, in, static_cast<const uint8_t *>(qs), static_cast<const f16 *>(scales), m, n, k,
               "madi_matmul_f16"};
  if (m <= 8) return launch_rows<8, true>(a);
  if (m <= 16) return launch_rows<16, true>(a);
  return launch_rows<32, true>(a);
}

// The f16 projection's limits: 32-bit buffer offsets (W and one 32-row slice
// of activations below 2 GiB), 65535 slices, K % 64 == 0, 16-byte aligned
// activations and output.
bool skinny_f16_ok(const void *in, const void *qs, const void *out, uint32_t m, uint32_t n,
                   uint32_t k) {
  return k % kChunkK == 0 && (uint64_t)n * k < (1ull << 31) &&
         (uint64_t)kSlice * k * 2 < (1ull << 31) && (m + kSlice - 1) / kSlice <= 65535 &&
         aligned(in, 16) && aligned(qs, 16) && aligned(out, 16);
}
}  // namespace madi
