// gemv.hip -- decoder Q8 GEMV family (M = 1), HBM-bound.
//
// Replaces gemv_q8 / _bias / _bias_gelu / _bias_res / _qkv and logit_gemv_q8
// (engine/metal/kernels/graph_helpers.metal:320-558).  The reference runs one
// 32-lane simdgroup per output row reading char4 + float4; here a workgroup
// owns one 32-row panel of the panel layout and its waves split K: four for
// the vocab matrix, sixteen for the decoder's 40 - 160-panel matrices (so a
// K = 1280 range is one round of loads).  Every wave64 load instruction moves
// one contiguous KiB (16 bytes per lane, lane (h, r) receiving 16 weights of
// row r in quantisation block h), issued as a buffer load with the
// panel/chunk offset in an SGPR.  Each wave streams its K range through a
// two-chunk window (use chunk c, refill with chunk c+2).  The four-wave
// instances keep to 62 - 71 VGPRs (seven waves per SIMD allow 72), so every workgroup
// of the 51866-row vocab matrix (1621 panels, seven per CU) is resident from
// the start; the sixteen-wave ones (four waves per SIMD) take up to 94.
//
// The activation vector is loaded next to the first weight window (before
// it for the narrow matrices, after it for the vocab), staged once per
// workgroup in LDS and read back as broadcast 128-bit LDS loads, ahead of
// the weights they meet (the narrow matrices' first window while its weights
// are in flight; the vocab's fp32 vector one 16-value unit ahead).  v_perm_b32
// turns two stored bytes u = q + 128 into the fp16 pair 1024 + u and one
// packed subtract of 1152 leaves the exact fp16 pair (q0, q1); fp16
// activations accumulate x * q with v_dot2_f32_f16 (exact products, fp32
// sums), fp32 activations with FMA.  Per quantisation block the lane
// multiplies its partial by the block's scale, the (partial * scale)
// structure of the reference's kernels; the two K-halves meet by a cross-lane
// shuffle and the four waves through LDS.  (Accumulating x * (1024 + u) and
// subtracting 1152 * sum(x) per block saves the subtract but cancels two
// large sums: an all-zero block, whose scale is 1.0, then leaks ~1e-2 of
// rounding noise into its row.)
#include "common.h"

using namespace madi;

namespace {

// Waves per workgroup (K ranges per panel): four for wide matrices (the
// vocab logits: 1621 panels, seven workgroups per CU); sixteen below
// kWidePanels, where four waves would each walk five chunks of a K = 1280
// row through the window (three rounds of memory latency) on fewer than
// half the CUs.
constexpr int kWaves = 4, kWavesNarrow = 16;
constexpr uint32_t kWidePanels = 256;
// Chunks in flight per wave, a sliding window: two keeps ~26 MB of the vocab
// matrix in flight across the GPU, enough to cover HBM latency, while the
// texture queues stay short enough that the activation vector (loaded first)
// is not stuck behind a flood of weight requests; deeper windows measured
// slower (the waves then sit blocked on issue and compute in one late burst).
constexpr int kWin = 2;
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
  // split K over `splits` workgroups per panel: partial row sums in `ws`
  // ([panel][split][32]), arrival counters in `cnt` ([panel], zero between uses)
  uint32_t splits;
  float *ws;
  uint32_t *cnt;
};

// LDS bytes: x (K elements of XT), the KW waves' partials
template <typename XT, int KW>
constexpr size_t lds_bytes(uint32_t k) {
  return (size_t)k * sizeof(XT) + KW * 32 * 4;
}

// One chunk's loads for a lane: its two 16-byte units and its block's scale.
struct ChunkW {
  u32x4 w[2];
  uint32_t s;
};

typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ inline rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// Issue chunk c of panel p (R rows) with buffer loads: the panel and chunk
// offsets are uniform (SGPR) and the lane offsets fixed, so the loads need no
// per-load address arithmetic.
__device__ inline void load_chunk(ChunkW &b, rsrc_t wq, rsrc_t ws, uint32_t K, uint32_t c,
                                  uint32_t p, uint32_t R, uint32_t w_voff, uint32_t s_voff) {
  const uint32_t so = (uint32_t)panel_chunk_qs(K, p, R, c);
  b.w[0] = __builtin_amdgcn_raw_buffer_load_b128(wq, w_voff, so, 0);
  b.w[1] = __builtin_amdgcn_raw_buffer_load_b128(wq, w_voff + 2 * R * 16, so, 0);
  b.s = __builtin_amdgcn_raw_buffer_load_b16(ws, s_voff, (uint32_t)panel_chunk_sc(K, p, R, c) * 2, 0);
}

// sum_i x[i] * q[i] over one 16-byte unit, fp16 activations: v_dot2_f32_f16
// multiplies two exact fp16 pairs (exact products) and adds them in fp32.
__device__ inline float unit_dot(const u32x4 &w, const f16 *x16, float part) {
  const f16x8 xa = *reinterpret_cast<const f16x8 *>(x16);
  const f16x8 xb = *reinterpret_cast<const f16x8 *>(x16 + 8);
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const f16x8 &xv = d < 2 ? xa : xb;
    const int e = (d & 1) * 4;
    part = __builtin_amdgcn_fdot2(q_pair(wd[d], kSelLo), (f16x2){xv[e], xv[e + 1]}, part, false);
    part = __builtin_amdgcn_fdot2(q_pair(wd[d], kSelHi), (f16x2){xv[e + 2], xv[e + 3]}, part, false);
  }
  return part;
}

// The same sum for fp32 activations: FMA of the fp32 x with the exact q.
__device__ inline float unit_dot(const u32x4 &w, const float *x32, float part) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const f32x4 xv = *reinterpret_cast<const f32x4 *>(x32 + 4 * d);
    const f16x2 q01 = q_pair(wd[d], kSelLo), q23 = q_pair(wd[d], kSelHi);
    part = __builtin_fmaf(xv.x, (float)q01.x, part);
    part = __builtin_fmaf(xv.y, (float)q01.y, part);
    part = __builtin_fmaf(xv.z, (float)q23.x, part);
    part = __builtin_fmaf(xv.w, (float)q23.y, part);
  }
  return part;
}

// One 16-weight unit's fp32 activations in registers, and its sum against
// them (the same FMA order as unit_dot).
struct XUnit {
  f32x4 v[4];
};
__device__ inline XUnit read_unit(const float *x32) {
  XUnit u;
#pragma unroll
  for (int d = 0; d < 4; ++d) u.v[d] = *reinterpret_cast<const f32x4 *>(x32 + 4 * d);
  return u;
}
__device__ inline float unit_dot(const u32x4 &w, const XUnit &x, float part) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const f16x2 q01 = q_pair(wd[d], kSelLo), q23 = q_pair(wd[d], kSelHi);
    part = __builtin_fmaf(x.v[d].x, (float)q01.x, part);
    part = __builtin_fmaf(x.v[d].y, (float)q01.y, part);
    part = __builtin_fmaf(x.v[d].z, (float)q23.x, part);
    part = __builtin_fmaf(x.v[d].w, (float)q23.y, part);
  }
  return part;
}

// acc += scale * (sum_k x[k] q[k]) over the lane's quantisation block, its
// 32 activations at xp (LDS, or registers)
template <typename XT>
__device__ inline void accumulate_x(const ChunkW &b, const XT *xp, float &acc) {
  float part = unit_dot(b.w[0], xp, 0.0f);
  part = unit_dot(b.w[1], xp + 16, part);
  acc = __builtin_fmaf(part, (float)__builtin_bit_cast(f16, (uint16_t)b.s), acc);
}
// the same over the lane's block of chunk c, x in LDS
template <typename XT>
__device__ inline void accumulate(const ChunkW &b, uint32_t c, const XT *xs, uint32_t h,
                                  float &acc) {
  accumulate_x(b, xs + c * kChunkK + h * 32, acc);
}

template <typename XT>
constexpr bool kBlockF32 = sizeof(XT) == 4;

// Narrow matrices: sixteen waves of one panel, four per SIMD, so up to 128
// VGPRs each (the first window's activations are held in registers, below).
template <int KW>
constexpr int kWavesPerEu = KW == kWavesNarrow ? 4 : 7;

template <typename XT, int MODE, int KW>
//
// Grid (x, y) = (panel, K split).  The arguments are scalars in the order the
// kernel first needs them, so the leading ones arrive preloaded in SGPRs, and
// the set-up has no integer division: split s covers chunks [s * cper +
// min(s, crem), + cper + (s < crem)).
__global__ __launch_bounds__(KW * 64) __attribute__((amdgpu_waves_per_eu(kWavesPerEu<KW>))) void q8_gemv_kernel(
    const uint8_t *qs, const f16 *sc, const void *x, uint32_t n, uint32_t k, uint32_t cper,
    uint32_t crem, float *out, const float *bias, float *wsp, uint32_t *cnt, const float *qb,
    const float *vb, float *kc, float *vc, const uint32_t *pos) {
  const GemvArgs a{out, x, qs, sc, bias, n, k, qb, vb, kc, vc, pos, gridDim.y, wsp, cnt};
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t K = a.k;
  XT *xs = reinterpret_cast<XT *>(smem);                        // [K]
  float *red = reinterpret_cast<float *>(smem + lds_bytes<XT, KW>(K) - KW * 32 * 4);  // [KW][32]

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t h = lane >> 5, r = lane & 31;
  const uint32_t p = blockIdx.x, split = blockIdx.y;
  const uint32_t R = panel_rows(a.n, p);
  const bool live = r < R;
  // this workgroup's K chunks [cs, cs + nck), split KW ways over the waves
  const uint32_t cs = split * cper + (split < crem ? split : crem);
  const uint32_t nck = cper + (split < crem ? 1 : 0);
  const uint32_t c0 = cs + (wave * nck) / KW, c1 = cs + ((wave + 1) * nck) / KW;

  // ---- x (16 bytes per thread and piece) and the first weight window.
  // Narrow matrices (sixteen waves, one or two chunks each) load x first: its
  // staging barrier, not the weights, is then the longer wait.  The vocab
  // matrix (four waves, five chunks each) issues its first weight window
  // first, so the HBM requests leave before the L2-resident vector's
  // (alternating runs in one process: 12.16 -> 11.92 us with f16 x, 12.66 ->
  // 12.35 us with f32 x; the narrow ones measured slower that way, a decoder
  // token 126 -> 134 us).  Lanes past a partial panel's last row read row R-1
  // (in bounds; their sums are never stored).
  constexpr bool kWeightsFirst = KW == kWaves;
  const uint32_t pieces = K * sizeof(XT) / 16;
  const rsrc_t xr = make_rsrc(a.x, K * sizeof(XT));
  u32x4 xv0 = {}, xv1 = {};
  const uint32_t i0 = threadIdx.x, i1 = threadIdx.x + KW * 64;
  if constexpr (!kWeightsFirst) {
    if (i0 < pieces) xv0 = __builtin_amdgcn_raw_buffer_load_b128(xr, i0 * 16, 0, 0);
    if (i1 < pieces) xv1 = __builtin_amdgcn_raw_buffer_load_b128(xr, i1 * 16, 0, 0);
  }

  const rsrc_t wq = make_rsrc(a.qs, a.n * K), ws = make_rsrc(a.sc, a.n * (K / 32) * 2);
  // chunks past the wave's range load through an empty resource: no memory
  // access, zeros returned, so their scale is 0 and they add exactly nothing.
  // Every window load is then unconditional, which keeps each window slot in
  // the same registers from trip to trip (a conditional load makes the
  // compiler copy the slot at the loop back edge, and a copy must first wait
  // for the load that was just issued, collapsing the window).
  const rsrc_t wz = make_rsrc(a.qs, 0);
  const uint32_t rr = live ? r : R - 1;
  const uint32_t w_voff = (h * R + rr) * 16, s_voff = (h * R + rr) * 2;
  // the first kWin chunks of this wave's range
  ChunkW win[kWin];
#pragma unroll
  for (int k = 0; k < kWin; ++k) {
    const bool in = c0 + k < c1;
    load_chunk(win[k], in ? wq : wz, in ? ws : wz, K, c0 + k, p, R, w_voff, s_voff);
  }
  if constexpr (kWeightsFirst) {
    if (i0 < pieces) xv0 = __builtin_amdgcn_raw_buffer_load_b128(xr, i0 * 16, 0, 0);
    if (i1 < pieces) xv1 = __builtin_amdgcn_raw_buffer_load_b128(xr, i1 * 16, 0, 0);
  }

  // The epilogue's operands (bias, residual, q/v bias, cache position) load
  // now, behind the weights, so their latency passes during the K loop
  // instead of after it.  Lanes 0..R-1 of wave 0 own the panel's rows.
  const uint32_t erow = p * kPanelRows + threadIdx.x;
  float e_bias = 0.0f, e_res = 0.0f;
  uint32_t e_pos = 0;
  if (threadIdx.x < R) {
    if constexpr (MODE == kBias || MODE == kBiasGelu) {
      e_bias = a.bias[erow];
    } else if constexpr (MODE == kBiasRes) {
      e_bias = a.bias[erow];
      e_res = a.out[erow];
    } else if constexpr (MODE == kQkv) {
      if (erow < a.k) e_bias = a.qb[erow];
      else if (erow >= 2 * a.k) e_bias = a.vb[erow - 2 * a.k];
    }
  }
  if constexpr (MODE == kQkv) e_pos = a.pos[0];

  // stage x
  for (uint32_t i = threadIdx.x; i < pieces; i += KW * 64) {
    const u32x4 v =
        i == i0 ? xv0 : (i == i1 ? xv1 : __builtin_amdgcn_raw_buffer_load_b128(xr, i * 16, 0, 0));
    reinterpret_cast<u32x4 *>(xs)[i] = v;
  }
  __syncthreads();

  // stream the range through the kWin-chunk window: use chunk c, refill its
  // registers with chunk c + kWin
  float acc = 0.0f;
  uint32_t cfirst = c0;
  if constexpr (KW == kWavesNarrow) {
    // Narrow matrices (one or two chunks per wave): the first window's
    // activations are read from LDS now, while its weights are still in
    // flight, instead of after they land, when all sixteen waves would queue
    // at the LDS at once.
    if (c0 < c1) {
      XT xf[kWin][32];
#pragma unroll
      for (int k = 0; k < kWin; ++k) {
        const uint32_t cc = c0 + k < c1 ? c0 + k : c1 - 1;
#pragma unroll
        for (int i = 0; i < 32; ++i) xf[k][i] = xs[cc * kChunkK + h * 32 + i];
      }
      // the reads stay ahead of the first wait for the weights
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < kWin; ++k) {
        accumulate_x<XT>(win[k], xf[k], acc);
        const uint32_t cn = c0 + k + kWin;
        const bool in = cn < c1;
        load_chunk(win[k], in ? wq : wz, in ? ws : wz, K, cn, p, R, w_voff, s_voff);
        __builtin_amdgcn_sched_barrier(0);
      }
      cfirst = c0 + kWin;
    }
  }
  if constexpr (KW == kWaves && kBlockF32<XT>) {
    // The vocab matrix with fp32 activations: each unit's activations are
    // read from LDS one unit ahead of their use (the next chunk's first unit
    // during this chunk's second), so the LDS latency passes under the
    // arithmetic; a whole chunk ahead would not fit the 72 VGPRs that keep
    // seven waves per SIMD.
    const float *xf = reinterpret_cast<const float *>(xs) + h * 32;
    XUnit xa = read_unit(xf + (c0 < c1 ? c0 : 0) * kChunkK);
#pragma unroll 1
    for (uint32_t c = c0; c < c1; c += kWin) {
#pragma unroll
      for (int k = 0; k < kWin; ++k) {
        const uint32_t cc = c + k < c1 ? c + k : c1 - 1;
        const uint32_t cx = c + k + 1 < c1 ? c + k + 1 : c1 - 1;  // the next slot's chunk
        // each read is issued before the arithmetic that precedes its use
        const XUnit xb = read_unit(xf + cc * kChunkK + 16);
        __builtin_amdgcn_sched_barrier(0);
        float part = unit_dot(win[k].w[0], xa, 0.0f);
        __builtin_amdgcn_sched_barrier(0);
        xa = read_unit(xf + cx * kChunkK);
        __builtin_amdgcn_sched_barrier(0);
        part = unit_dot(win[k].w[1], xb, part);
        acc = __builtin_fmaf(part, (float)__builtin_bit_cast(f16, (uint16_t)win[k].s), acc);
        const uint32_t cn = c + k + kWin;
        const bool in = cn < c1;
        load_chunk(win[k], in ? wq : wz, in ? ws : wz, K, cn, p, R, w_voff, s_voff);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    cfirst = c1;
  }
#pragma unroll 1
  for (uint32_t c = cfirst; c < c1; c += kWin) {
#pragma unroll
    for (int k = 0; k < kWin; ++k) {
      // a chunk past the range (zeros, scale 0) reads the x of the range's
      // last chunk, so its partial stays finite and 0 * partial is exact
      const uint32_t cc = c + k < c1 ? c + k : c1 - 1;
      accumulate<XT>(win[k], cc, xs, h, acc);
      const uint32_t cn = c + k + kWin;
      const bool in = cn < c1;
      load_chunk(win[k], in ? wq : wz, in ? ws : wz, K, cn, p, R, w_voff, s_voff);
      // keep the next slot's math behind this reload: interleaved, both
      // slots would have to land before either is reissued
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  acc += __shfl_xor(acc, 32);
  if (h == 0) red[wave * 32 + r] = acc;
  __syncthreads();
  const uint32_t t = threadIdx.x;
  float v = 0.0f;
  if (t < 32) {  // the waves' partials in wave order
    v = red[t];
#pragma unroll
    for (int w = 1; w < KW; ++w) v += red[w * 32 + t];
  }
  if (a.splits > 1) {
    // Split K: each workgroup writes its 32 partial row sums past its XCD's L2
    // (device-scope stores) and counts itself in with a device-scope atomic
    // (every party is a workgroup of this launch); the last to arrive adds the
    // splits' partials in split order (the same order whoever arrives last)
    // and stores the rows.
    __shared__ uint32_t arrived;
    float *mine = a.ws + ((size_t)p * a.splits + split) * 32;
    if (t < 32) __hip_atomic_store(mine + t, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t == 0)
      arrived = __hip_atomic_fetch_add(&a.cnt[p], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != a.splits - 1) return;
    if (t < 32) {
      const float *all = a.ws + (size_t)p * a.splits * 32 + t;
      v = 0.0f;
      for (uint32_t s2 = 0; s2 < a.splits; ++s2)
        v += __hip_atomic_load(all + s2 * 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (t == 0) __hip_atomic_store(&a.cnt[p], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (t >= R) return;
  const uint32_t nrow = erow;  // t == threadIdx.x
  if constexpr (MODE == kPlain) {
    a.out[nrow] = v;
  } else if constexpr (MODE == kBias) {
    a.out[nrow] = v + e_bias;
  } else if constexpr (MODE == kBiasGelu) {
    a.out[nrow] = gelu_erf(v + e_bias);
  } else if constexpr (MODE == kBiasRes) {
    a.out[nrow] = e_res + v + e_bias;
  } else {  // kQkv: a.n = 3D, a.k = D
    const uint32_t D = a.k, pos = e_pos;
    if (nrow < D)
      a.out[nrow] = v + e_bias;
    else if (nrow < 2 * D)
      a.kc[(size_t)pos * D + (nrow - D)] = v;
    else
      a.vc[(size_t)pos * D + (nrow - 2 * D)] = v + e_bias;
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
  // buffer ranges and offsets are 32-bit: the weight (n*k bytes) must stay
  // below 2 GiB, as for the GEMM and the batched projection
  if ((uint64_t)a.n * a.k >= (1ull << 31))
    return fail(MADI_ERR_SHAPE, "%s: n=%u k=%u exceeds the 2 GiB operand limit", what, a.n, a.k);
  if (!aligned(a.qs, 16) || !aligned(a.sc, 2) || !aligned(a.x, 16))
    return fail(MADI_ERR_ALIGN, "%s: qs and x need 16-byte alignment", what);
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "%s: madi_init has not succeeded", what);
  if (int rc = deferred_before_read(a.x, (size_t)a.k * sizeof(XT))) return rc;
  if (MODE == kQkv) {
    // q_out [D], and one row of each cache at a position only the device
    // knows: somewhere in the allocation from kc (vc) on, if the library
    // allocated it, else at least the first row
    const size_t row = (size_t)(a.n / 3) * 4;
    const size_t kext = alloc_extent(a.kc), vext = alloc_extent(a.vc);
    if (int rc = deferred_before_write(a.out, row)) return rc;
    if (int rc = deferred_before_write(a.kc, kext > row ? kext : row)) return rc;
    if (int rc = deferred_before_write(a.vc, vext > row ? vext : row)) return rc;
  } else if (int rc = deferred_before_write(a.out, (size_t)a.n * 4)) {
    return rc;
  }
  const uint32_t np = (a.n + kPanelRows - 1) / kPanelRows, C = a.k / kChunkK;
  // Few panels and a long K (the 5120-wide FFN down projection: 40 panels)
  // leave most CUs idle and each wave with a long chain of loads: split K
  // over up to four workgroups per panel, >= 16 chunks each.
  GemvArgs b = a;
  b.splits = 1;
  if (np < 128 && C >= 32) {
    b.splits = C / 16 < 4 ? C / 16 : 4;
    if (int rc = workspace((size_t)np * b.splits * 32 * 4, np, &b.ws, &b.cnt)) return rc;
  }
  if (np >= kWidePanels)
    hipLaunchKernelGGL((q8_gemv_kernel<XT, MODE, kWaves>), dim3(np, b.splits), dim3(kWaves * 64),
                       (lds_bytes<XT, kWaves>(a.k)), stream(), b.qs, b.sc, b.x, b.n, b.k,
                       C / b.splits, C % b.splits, b.out, b.bias, b.ws, b.cnt, b.qb, b.vb, b.kc,
                       b.vc, b.pos);
  else
    hipLaunchKernelGGL((q8_gemv_kernel<XT, MODE, kWavesNarrow>), dim3(np, b.splits),
                       dim3(kWavesNarrow * 64), (lds_bytes<XT, kWavesNarrow>(a.k)), stream(), b.qs,
                       b.sc, b.x, b.n, b.k, C / b.splits, C % b.splits, b.out, b.bias, b.ws, b.cnt,
                       b.qb, b.vb, b.kc, b.vc, b.pos);
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
