// gemm.hip -- fused Q8 GEMM for the encoder projections (M = 1500 per window).
//
// C[M][N] (f16) = epi(A[M][K] (f16) . deq(W)[N][K]^T), fp32 accumulation on
// v_mfma_f32_32x32x16_f16.  Replaces the encoder's kDeq + kM4/kM4Bias pairs
// (engine/metal/encoder.zig:262-301) and the reference's fused Q8 designs
// mul_mm_q8 (kernels/q8_gemm.metal:29-102) and m4_gemm_q8_bias_gelu
// (kernels/m4_gemm.metal:131-189).
//
// Workgroup tile: 128*PW weight rows (4*PW panels) x 32*MT activation rows,
// four waves, one per SIMD.  Wave w owns panels PW*w .. PW*w + PW-1 and all MT
// m-tiles, so per 16-wide k-step it runs PW*MT independent 32x32x16 MFMAs on
// PW dequantised weight fragments and MT activation fragments.  PW = 2 (256
// columns) by default; PW = 1 (128 columns) where it allows twice the tile
// height at the same tile count, since the dequantisation per MFMA scales as
// 1 / MT.  The weight is the MFMA A operand (rows = n) and the activations the
// B operand (columns = m).
//
// Data movement per 64-wide K chunk:
//   weights  each wave streams its own two panels straight into VGPRs
//            (buffer_load_dwordx4: one contiguous KiB per instruction; in the
//            panel layout lane (h, r) receives row r's 32 weights of
//            quantisation block h) plus one fp16 scale per lane per panel, WD
//            chunks ahead of use, into WD rotating register sets;
//   A        the 32*MT x 64 f16 activation tile is shared by the four waves
//            through an NA-stage LDS ring, written by direct-to-LDS DMA
//            (buffer_load_dwordx4 ... lds) DA chunks ahead; the 16-byte
//            chunks of row r are XOR-swizzled by (r >> 1) & 7 so each DMA
//            instruction copies 8 whole 128-byte rows and the fragment reads
//            (32 consecutive rows, one chunk each) spread over all banks.
// One barrier per two chunks (before the last k-step of each odd chunk c)
// publishes the A stages of chunks c+1 and c+2 and retires those of c-1 and
// c.
//
// Weight fragments: register w[t][s] holds panel t's k-step-s fragment.  It
// is consumed by the MFMAs of step s and refilled in place with the next
// chunk's fragment right after them (w[0][s] during step s, w[1][s] during
// step s+1), half a 16-byte unit at a time: v_perm_b32 builds the fp16
// values 1024 + (q + 128), a packed subtract makes them q exactly and a
// packed multiply by the scale rounds once, so each weight is the reference's
// half(float(q) * float(s)) (q8_gemm.metal:26) bit for bit.  Every k-step
// issues its next-step LDS reads first and then alternates one MFMA with
// three dequantisation VALU ops (fixed with sched_group_barrier), so the
// matrix pipe is never left waiting on the vector ALU.
//
// K ordering: MFMA k-slot (lane half h, slot e) of step s holds k = 32h + 8s + e
// for BOTH operands, so each lane's weight slice of a chunk lies in one
// quantisation block (one scale per lane per panel per chunk); any k
// permutation shared by both operands leaves the product unchanged.
//
// The chunk count is padded to a multiple of WD with empty chunks: their
// loads use a zero-length buffer resource, which returns zeros without
// touching memory, so they add exact zeros.  Loads are issued in the same
// pattern every chunk, which keeps every vmcnt wait a constant.
//
// Tile height: 32, 64, 96 or 128 rows (MT = 1..4), chosen per shape by the
// host so the tile count fills the CUs in one round where it can.  With one
// K split and an unpadded loop the last four chunks run m-tile by m-tile
// (tail(), below), so that the stores of finished m-tiles overlap the MFMAs
// of the others.
//
// Split K: when the tiles alone cannot fill the GPU and K is long and the
// in-workgroup K split (q8_gemm_ks_kernel, below) does not take the shape
// (700 x 5120 -> 1280: 55 tiles of 64 x 256; the batched projection's FFN
// down at M = 320: 50 tiles of 64 x 128), up to four workgroups share a tile,
// each over a contiguous K range.  Each publishes its fp32 partial tile to
// the library's workspace and counts itself in with a device-scope atomic;
// the last to arrive adds the partials in split order and runs the epilogue.
// The grid is one-dimensional over (tile, split) items, renumbered so that
// each XCD runs a contiguous share of them (the tile order, below).
//
// Epilogue: bias / GELU in fp32 registers, one rounding to f16, then the tile
// leaves through LDS one 32-row m-tile at a time (the stores of one m-tile
// overlap the conversion of the next), transposed so every global store
// writes whole row segments of the tile (256 or 512 bytes, 16 per lane).
#include "common.h"
#include "vmem.h"

using namespace madi;

namespace {

constexpr int kPanelsPerTile = 8;
constexpr int kWaves = 4;  // one wave per SIMD
constexpr int NA = 8;      // activation ring stages
constexpr int DA = 4;      // A stages are copied DA chunks ahead of use
constexpr int WD = 4;      // weight register sets (chunks of weight prefetch)
constexpr int kCStride = kPanelsPerTile * kPanelRows * 2 + 16;  // epilogue tile row pitch
constexpr uint32_t kMaxSplits = 4;  // split-K workgroups per tile
constexpr int kSplitTile = 2;       // m-tiles per tile where 128-row tiles would split K

// F32: the activations arrive as f32 (rounded to f16 on their way from LDS to
// the MFMA) and the result leaves as f32 -- the batched projection's operand
// types (the engine's f32 rows, staged to f16 for the GEMM).
template <int MT, bool F32 = false, int PW = 2>
struct Geometry {
  static constexpr int kRowBytes = F32 ? 256 : 128;  // one A row of a 64-wide chunk
  static constexpr int kStage = MT * 32 * kRowBytes;  // one A stage (32*MT rows)
  static constexpr int kRing = NA * kStage;
  static constexpr int kTilePanels = 4 * PW;  // panels (32 columns each) per tile
  static constexpr int kCPitch =
      kTilePanels * kPanelRows * (F32 ? 4 : 2) + 16;
  static constexpr int kCTile = 32 * MT * kCPitch;
  static constexpr int kLds = kRing > kCTile ? kRing : kCTile;
  // vector-memory instructions per wave per chunk, spread over the four
  // k-steps so the texture pipe never sees a burst: step 0 the first half of
  // the A DMA (LA DMAs of 1 KiB: 8 f16 rows or 4 f32 rows each), step 1 its
  // second half and weight unit (0,0), step 2 units (0,1) and (1,0), step 3
  // unit (1,1) and the scales (one panel: units (0,0), (0,1), the scale)
  static constexpr int LA = F32 ? 2 * MT : MT;
  static constexpr int LA0 = LA >= 2 ? (LA + 1) / 2 : 0;  // DMAs issued in step 0
  static constexpr int LW = 3 * PW;
  static constexpr int kPerChunk = LA + LW;
  static constexpr int kBeforeStep3 = LA + (PW == 2 ? 3 : 2);  // issued in steps 0..2
  // at the start of chunk c: the weights of chunk c+1 (the last loads of
  // chunk c+1-WD) have landed once only the loads of the WD-2 chunks after
  // them are outstanding
  static constexpr int kVmRaw = (WD - 2) * kPerChunk;
  // before step 3 of an odd chunk c, whose barrier publishes the A stages of
  // chunks c+1 and c+2: chunk c+2's stage (issued in steps 0-1 of chunk
  // c+2-DA, followed by that chunk's LW weight loads, chunk c-1's loads and
  // chunk c's first three steps) has landed
  static constexpr int kVmA = LW + (DA - 3) * kPerChunk + kBeforeStep3;
  // prologue: virtual chunks -DA..-1 issue the same pattern; chunk 0's weights
  // (virtual chunk -WD) and the A stages of chunks 0 and 1 (virtual chunks -DA
  // and 1-DA) have landed
  static constexpr int kVmPrologue = LW + (DA - 2) * kPerChunk;
  static_assert(kVmRaw < 64 && kVmA < 64 && kVmPrologue < 64, "vmcnt range");
};


// XOR swizzle of the A tile's 16-byte chunks within row `row`: 8 per f16 row,
// 16 per f32 row
__device__ inline uint32_t a_swz(uint32_t row) { return (row >> 1) & 7; }
__device__ inline uint32_t a_swz32(uint32_t row) { return row & 15; }

// One chunk's int8 weight units and scales of the wave's PW panels (two in
// 256-column tiles, one in 128-column tiles)
template <int PW = 2>
struct RawWT {
  u32x4 u[PW][2];  // [panel t][unit j]: k = 32h + 16j + 0..15 of row r
  uint32_t s[PW];  // fp16 scale bits of block h, row r (low half)
};
using RawW = RawWT<2>;

// Wait until `w`'s loads have landed: at most N later loads outstanding.  The
// registers are operands, so no use of them can be scheduled before the wait.
template <int N, int PW>
__device__ inline void wait_weights(RawWT<PW> &w) {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  if constexpr (PW == 2)
    asm volatile("s_waitcnt vmcnt(%[n])"
                 : "+v"(w.u[0][0]), "+v"(w.u[0][1]), "+v"(w.u[1][0]), "+v"(w.u[1][1]),
                   "+v"(w.s[0]), "+v"(w.s[1])
                 : [n] "n"(N));
  else
    asm volatile("s_waitcnt vmcnt(%[n])" : "+v"(w.u[0][0]), "+v"(w.u[0][1]), "+v"(w.s[0]) : [n] "n"(N));
}

// After the K loop: wait for every outstanding load, with the four weight
// register sets as operands of the wait.  The last prefetches' registers are
// dead to the compiler once the loop ends, and it would otherwise reuse them
// (for the epilogue's accumulator reads) while loads into them are still in
// flight.
template <int PW>
__device__ inline void drain(RawWT<PW> &a, RawWT<PW> &b, RawWT<PW> &c, RawWT<PW> &d) {
  if constexpr (PW == 2) {
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(a.u[0][0]), "+v"(a.u[0][1]), "+v"(a.u[1][0]), "+v"(a.u[1][1]), "+v"(a.s[0]),
                   "+v"(a.s[1]), "+v"(b.u[0][0]), "+v"(b.u[0][1]), "+v"(b.u[1][0]), "+v"(b.u[1][1]),
                   "+v"(b.s[0]), "+v"(b.s[1])::"memory");
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(c.u[0][0]), "+v"(c.u[0][1]), "+v"(c.u[1][0]), "+v"(c.u[1][1]), "+v"(c.s[0]),
                   "+v"(c.s[1]), "+v"(d.u[0][0]), "+v"(d.u[0][1]), "+v"(d.u[1][0]), "+v"(d.u[1][1]),
                   "+v"(d.s[0]), "+v"(d.s[1])::"memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(a.u[0][0]), "+v"(a.u[0][1]), "+v"(a.s[0]), "+v"(b.u[0][0]), "+v"(b.u[0][1]),
                   "+v"(b.s[0]), "+v"(c.u[0][0]), "+v"(c.u[0][1]), "+v"(c.s[0]), "+v"(d.u[0][0]),
                   "+v"(d.u[0][1]), "+v"(d.s[0])::"memory");
  }
}

// Per-wave load plan, fixed for the whole K loop.
template <int MT, bool F32, int PW = 2>
struct Plan {
  desc_t wq, ws, wa, zero;  // weights, scales, activations, empty
  uint32_t w_soff[PW];      // byte offset of panel (PW*wave + t) in the weights
  uint32_t s_voff[PW];      // per-lane byte offset of this lane's scale, panel t
  uint32_t a_voff[Geometry<MT, F32>::LA];  // per-lane activation offsets of the wave's
                            // DMAs, less each DMA's instruction offset (1024 * DMA)
  uint32_t a_lds;           // the wave's first A row within an A stage
  uint32_t nchunks;
};

// DMA I of the wave's share of one chunk's A stage.
template <int MT, bool F32, int I, int PW>
__device__ inline void dma_group(desc_t wa, const Plan<MT, F32, PW> &p, uint32_t c, uint32_t m0) {
  dma16<I * 1024, I == 0>(wa, p.a_voff[I], c * Geometry<MT, F32>::kRowBytes, m0);
}
// DMAs I .. END-1
template <int MT, bool F32, int I, int END, int PW>
__device__ inline void dma_range(desc_t wa, const Plan<MT, F32, PW> &p, uint32_t c, uint32_t m0) {
  if constexpr (I < END) {
    dma_group<MT, F32, I>(wa, p, c, m0);
    dma_range<MT, F32, I + 1, END>(wa, p, c, m0);
  }
}

// Which of a chunk's prefetches (the A stage DA chunks ahead, the weights WD
// chunks ahead) are issued.  kSel: padded chunk counts; a prefetch past the
// last chunk loads zeros through the empty descriptor (touching no memory),
// chosen at run time.  kLive: every prefetch is live.  kLast0..kLast3: the
// four chunks of the last trip of an unpadded loop, all of whose prefetches
// lie past the end: they issue nothing.  A load whose result is never used
// must not be issued at all: the compiler sees the asm write its registers at
// once and reuses them while the load is still in flight.
enum Prefetch {
  kSel = 0, kLive = 1, kLast0 = 2, kLast1 = 3, kLast2 = 4, kLast3 = 5, kLiveE = 6,
  kRamp0 = 7, kRamp1 = 8
};

// The vmcnt counts of a chunk's two waits: `raw` at its start (chunk c+1's
// weights, issued in chunk c+1-WD, have landed once only the loads issued
// after them are outstanding) and `a` before its last k-step (chunk c+1's A
// stage, issued in steps 0-1 of chunk c+2-NA).  The last trip issues fewer
// loads, so fewer remain outstanding behind each target.
// kLiveE: a chunk of the first trip of a persistent workgroup's tile, whose
// prologue loads are followed by E other vector-memory issues (the previous
// tile's epilogue) before the K loop: the waits whose targets lie in the
// prologue (chunks 0-2's weights, chunk 3's A stage) allow E more.
// kRamp0 / kRamp1: chunks 0 and 1 of a ramped start (the prologue issues
// chunks 0 and 1 only; chunk 0 issues chunks 2 and 3, chunk 1 chunks 4 and
// 5, in the same global order as the steady state): chunk 0 waits for chunk
// 1's weights with nothing issued after them, chunk 1 for chunk 2's with
// chunk 3's loads after them, and chunk 1's barrier for chunk 3's A stage
// with chunk 3's weights, chunk 4's loads and chunk 5's A stage and first
// weight unit after it.
template <int MT, bool F32, int PF, int E = 0, int PW = 2>
struct Waits {
  using G = Geometry<MT, F32, PW>;
  static constexpr int raw = PF == kLiveE ? G::kVmRaw + E
                           : PF == kLast1 ? G::kPerChunk
                           : (PF >= kLast2 && PF <= kLast3) ? 0
                           : PF == kRamp0 ? 0
                           : PF == kRamp1 ? G::kPerChunk
                                          : G::kVmRaw;
  static constexpr int a = PF == kLiveE ? G::kVmA + E
                         : PF == kLast1 ? G::LW
                         : PF == kLast3 ? 0
                         : PF == kRamp1 ? G::LW + G::kPerChunk + G::LA + 1
                                        : G::kVmA;
  static_assert(raw >= 0 && raw < 64 && a >= 0 && a < 64, "vmcnt range");
};

// The vector-memory issues of k-step s for chunk c's A stage (into `slot`) and
// chunk cw's weights (into `w`).
template <int MT, bool F32, int PF, int PW>
__device__ inline void issue_loads(int s, uint8_t *slot, uint32_t c, RawWT<PW> &w, uint32_t cw,
                                   const Plan<MT, F32, PW> &p, uint32_t lane) {
  using G = Geometry<MT, F32, PW>;
  static_assert(DA == 4 && WD == 4, "the last trip's issue plan assumes four-chunk prefetch");
  if constexpr (PF >= kLast0) return;
  desc_t wa = p.wa, wq = p.wq, ws = p.ws;
  if constexpr (PF == kSel) {
    wa = c < p.nchunks ? p.wa : p.zero;
    const bool live = cw < p.nchunks;
    wq = live ? p.wq : p.zero;
    ws = live ? p.ws : p.zero;
  }
  constexpr bool W = true;
  const uint32_t m0 = lds_addr(slot) + p.a_lds;
  if (s == 0) {
    dma_range<MT, F32, 0, G::LA0>(wa, p, c, m0);
  } else if (s == 1) {
    dma_range<MT, F32, G::LA0, G::LA>(wa, p, c, m0);
    if constexpr (W) vload16(w.u[0][0], wq, lane * 16, p.w_soff[0] + cw * 2048);
  } else if (s == 2) {
    if constexpr (W) {
      vload16<1024>(w.u[0][1], wq, lane * 16, p.w_soff[0] + cw * 2048);
      if constexpr (PW == 2) vload16(w.u[1][0], wq, lane * 16, p.w_soff[1] + cw * 2048);
    }
  } else if constexpr (W) {
    if constexpr (PW == 2) vload16<1024>(w.u[1][1], wq, lane * 16, p.w_soff[1] + cw * 2048);
    vload2(w.s[0], ws, p.s_voff[0], cw * 128);
    if constexpr (PW == 2) vload2(w.s[1], ws, p.s_voff[1], cw * 128);
  }
}

// The MT activation fragments of k-step s from an A stage (swizzled rows).
template <int MT>
__device__ inline void load_a_frags(const uint8_t *As, int s, uint32_t h, uint32_t r,
                                    f16x8 (&bf)[MT]) {
  const uint32_t phys = ((h * 4 + s) ^ a_swz(r)) * 16;  // rows i*32 + r share (r >> 1) & 7
#pragma unroll
  for (int i = 0; i < MT; ++i)
    bf[i] = *reinterpret_cast<const f16x8 *>(As + (i * 32 + r) * 128 + phys);
}

// f32 activations: a fragment's 8 values (k = 32h + 8s .. +8 of row r) are two
// 16-byte pieces of the 256-byte row, rounded to f16 once they have landed.
struct F32Frag {
  f32x4 lo, hi;
};
template <int MT>
__device__ inline void load_a_frags(const uint8_t *As, int s, uint32_t h, uint32_t r,
                                    F32Frag (&bf)[MT]) {
  const uint32_t sw = a_swz32(r);  // rows i*32 + r share r & 15
  const uint32_t p0 = ((8 * h + 2 * s) ^ sw) * 16, p1 = ((8 * h + 2 * s + 1) ^ sw) * 16;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    bf[i].lo = *reinterpret_cast<const f32x4 *>(As + (i * 32 + r) * 256 + p0);
    bf[i].hi = *reinterpret_cast<const f32x4 *>(As + (i * 32 + r) * 256 + p1);
  }
}
// round to nearest even, as the engine's f32 -> f16 staging (kCvt32)
__device__ inline f16x8 to_f16(const F32Frag &f) {
  return (f16x8){(f16)f.lo.x, (f16)f.lo.y, (f16)f.lo.z, (f16)f.lo.w,
                 (f16)f.hi.x, (f16)f.hi.y, (f16)f.hi.z, (f16)f.hi.w};
}

// What a k-step keeps of its activation fragments between their LDS read and
// the MFMAs of the next step: the f16 fragments, or the raw f32 values
template <bool F32>
struct AFrag {
  using T = f16x8;
};
template <>
struct AFrag<true> {
  using T = F32Frag;
};

// The k-step-s fragment of panel t: half (s & 1) of unit s >> 1.  The four
// pairs go through perm, subtract and multiply stage by stage (four
// independent chains), so no packed op directly follows the one it depends on
// (which would cost a wait state).
template <int PW>
__device__ inline f16x8 dequant_frag(const RawWT<PW> &w, int t, int s) {
  const u32x4 u = w.u[t][s >> 1];
  const uint32_t b0 = (s & 1) ? u.z : u.x, b1 = (s & 1) ? u.w : u.y;
  const f16 sc = __builtin_bit_cast(f16, (uint16_t)w.s[t]);
  const f16x2 s2 = {sc, sc};
  f16x2 a[4] = {q_pair(b0, kSelLo), q_pair(b0, kSelHi), q_pair(b1, kSelLo), q_pair(b1, kSelHi)};
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = a[i] * s2;
  return (f16x8){a[0].x, a[0].y, a[1].x, a[1].y, a[2].x, a[2].y, a[3].x, a[3].y};
}

// s_waitcnt lgkmcnt(0) with vmcnt and expcnt left at their maxima (gfx9
// encoding: vmcnt bits 15:14 and 3:0, expcnt 6:4, lgkmcnt 11:8)
constexpr int kLgkm0 = 0xC07F;

// Buffer cache policy sc1: the access writes through (stores) or reads past
// (loads) the XCD's own L2.
constexpr int kSc1 = 16;

// sched_group_barrier masks
constexpr int kSchedVALU = 0x002;
constexpr int kSchedMFMA = 0x008;
constexpr int kSchedVMEM = 0x020;
constexpr int kSchedDSRead = 0x100;

// Instruction order of one k-step: its LDS reads first (their latency hides
// under this step's MFMAs), then each MFMA followed by up to three VALU ops
// (the dequantisation, 24 per step) and a vector-memory issue.
template <int MT, bool F32 = false, int PW = 2>
__device__ inline void schedule_step() {
  if constexpr (F32) __builtin_amdgcn_sched_group_barrier(kSchedVALU, 4 * MT, 0);  // f32 -> f16
  __builtin_amdgcn_sched_group_barrier(kSchedDSRead, F32 ? 2 * MT : MT, 0);
#pragma unroll
  for (int i = 0; i < PW * MT; ++i) {
    __builtin_amdgcn_sched_group_barrier(kSchedMFMA, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedVALU, 12 / MT + 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedVMEM, 1, 0);
  }
}

// One chunk c.  On entry w holds chunk c's fragments except each panel's
// w[t][3] (made at step 0 from `cur`, chunk c's weights), `af` holds chunk c's step-0
// activation fragments (f32: their raw values, rounded at the step's start),
// and `nxt` receives chunk c+1's weights (loaded WD-1 chunks ago; waited for
// here).  `ld` (the same register set as `cur`, free after step 0) receives
// chunk c+WD's weights.
// The ramped start's loads for k-step s of chunk c (0 or 1): chunks 2c + 2
// and 2c + 3, the first into register set `la` and A stage 2c + 2, the
// second into `lb` and stage 2c + 3; k-steps 0-1 issue the first chunk's
// plan (A stage, then weights), k-steps 2-3 the second's.
template <int MT, bool F32, int PW>
__device__ inline void ramp_loads(int s, uint8_t *smem, uint32_t c, const Plan<MT, F32, PW> &p,
                                  uint32_t lane, RawWT<PW> &la, RawWT<PW> &lb) {
  using G = Geometry<MT, F32, PW>;
  const uint32_t c0 = 2 * c + 2, c1 = 2 * c + 3;
  if (s < 2) {
    uint8_t *slot = smem + (c0 % NA) * G::kStage;
    issue_loads<MT, F32, kLive>(2 * s, slot, c0, la, c0, p, lane);
    issue_loads<MT, F32, kLive>(2 * s + 1, slot, c0, la, c0, p, lane);
  } else {
    uint8_t *slot = smem + (c1 % NA) * G::kStage;
    issue_loads<MT, F32, kLive>(2 * (s - 2), slot, c1, lb, c1, p, lane);
    issue_loads<MT, F32, kLive>(2 * (s - 2) + 1, slot, c1, lb, c1, p, lane);
  }
}

template <int MT, bool F32, int PF, bool ODD, int E = 0, int PW = 2>
__device__ inline void chunk(uint8_t *smem, const Plan<MT, F32, PW> &p, uint32_t c, uint32_t lane,
                             uint32_t h, uint32_t r, f32x16 (&acc)[PW][MT], f16x8 (&w)[PW][4],
                             typename AFrag<F32>::T (&af)[MT], const RawWT<PW> &cur,
                             RawWT<PW> &nxt, RawWT<PW> &ld, RawWT<PW> &ld2) {
  using G = Geometry<MT, F32, PW>;
  using WT = Waits<MT, F32, PF, E, PW>;
  const uint8_t *At = smem + (c % NA) * G::kStage;
  const uint8_t *An = smem + ((c + 1) % NA) * G::kStage;
  uint8_t *Af = smem + ((c + DA) % NA) * G::kStage;
  wait_weights<WT::raw>(nxt);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    // the previous step's fragment reads (issued a whole step ago) have
    // landed: one wait here instead of one before each MFMA
    // odd chunks: the A stages of chunks c+1 and c+2 become visible, and the
    // stages of chunks c-1 and c retire (refilled from chunk c+DA-2 on); an
    // even chunk reads chunk c+1's stage, published one chunk earlier
    if (s == 3 && ODD) wait_then_barrier<WT::a>();
    __builtin_amdgcn_s_waitcnt(kLgkm0);
    f16x8 a16[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      if constexpr (F32)
        a16[i] = to_f16(af[i]);
      else
        a16[i] = af[i];
    }
    typename AFrag<F32>::T an[MT];
    if (s < 3)
      load_a_frags<MT>(At, s + 1, h, r, an);
    else
      load_a_frags<MT>(An, 0, h, r, an);
#pragma unroll
    for (int t = 0; t < PW; ++t) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
        acc[t][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w[t][s], a16[i], acc[t][i], 0, 0, 0);
      // each panel's step s-1 fragment was consumed last step, at least MT
      // MFMAs before its refill here (no read-after-write wait states): its
      // next value is chunk c's own step-3 fragment at step 0, else chunk c+1's
      w[t][(s + 3) & 3] = dequant_frag(s == 0 ? cur : nxt, t, (s + 3) & 3);
    }
    if constexpr (PF == kRamp0 || PF == kRamp1) {
      // two chunks' loads over the four k-steps, in global order (chunk 0:
      // chunks 2 and 3 into register sets `ld`, `ld2`; chunk 1: chunks 4
      // and 5)
      ramp_loads<MT, F32, PW>(s, smem, c, p, lane, ld, ld2);
    } else {
      issue_loads<MT, F32, PF == kLiveE ? kLive : PF>(s, Af, c + DA, ld, c + WD, p, lane);
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) af[i] = an[i];
    schedule_step<MT, F32, PW>();
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The bias operands of panel (2 * wave + t), 16 bytes per (t, g), loaded from
// inline asm so the compiler inserts no wait for them: its count would also
// cover the asm loads issued before or after them (weights still in flight,
// the persistent loop's next prologue), so the kernels wait with their own.
__device__ inline void load_bias(f32x4 (&b4)[2][4], const float *bias, uint32_t np, uint32_t p0,
                                 uint32_t wave, uint32_t h) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    uint32_t pb = p0 + 2 * wave + t;
    pb = pb < np ? pb : np - 1;
    const desc_t d = make_desc(bias + pb * kPanelRows, kPanelRows * 4);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x4 v;
      asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen"
                   : "=v"(v) : "v"((g * 8 + h * 4) * 4), "s"(d), "s"(sgpr(0u)));
      b4[t][g] = __builtin_bit_cast(f32x4, v);
    }
  }
#pragma clang diagnostic pop
}

template <int N>
__device__ inline void wait_bias(f32x4 (&b4)[2][4]) {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%[n])"
               : "+v"(b4[0][0]), "+v"(b4[0][1]), "+v"(b4[0][2]), "+v"(b4[0][3]), "+v"(b4[1][0]),
                 "+v"(b4[1][1]), "+v"(b4[1][2]), "+v"(b4[1][3])
               : [n] "n"(N));
}

// LDS accesses of this wave done, then meet the other waves (the C staging
// handoff of the m-tile-major tail; vector-memory stores stay in flight).
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---- m-tile-major tail (unpadded chunk count, one K split, f16 result, two
// or more m-tiles).  The last four chunks do not run chunk by chunk: m-tile 0
// runs its MFMAs over all four chunks first (the four chunks' weights
// dequantised along the way and kept in registers, 32 fragments), then m-tile
// 1 while m-tile 0 leaves -- its bias, GELU and conversion, LDS transpose and
// C stores interleaved with m-tile 1's MFMAs -- and so on: only the last
// m-tile's epilogue follows the last MFMA, and the other m-tiles' stores
// (bounded by the HBM write rate, since every workgroup writes at once)
// overlap matrix work.  Every output accumulates in the chunk loop's order
// (chunk by chunk, k-step by k-step), so the result is bit-identical to it.
//
// Entry state (the loop's last trip ended with chunk c-1, c = nchunks - 4,
// c % 4 == 0): w holds chunk c's step 0-2 fragments, r0 chunk c's weights
// (landed), r1..r3 the weights of chunks c+1..c+3 and the A stages of chunks
// c+2 and c+3 are in flight (chunk j's loads, LA DMAs then LW weight loads,
// were issued in chunk j-4), the stages of chunks c and c+1 are published,
// af holds every m-tile's step-0 fragment of chunk c.  The ring stages of
// chunks c-4 .. c-1 (four consecutive stages) are free: no DMA targets them
// and every read of them completed before the last barrier.  They hold the C
// staging, one m-tile (32 rows) per buffer.
template <int MT>
struct Tail {
  using G = Geometry<MT>;
  static constexpr int kCBuf = 32 * kCStride;
  static constexpr int kBufs = 4 * G::kStage >= 2 * kCBuf ? 2 : 1;
  static_assert(4 * G::kStage >= kCBuf, "one m-tile of C fits the free ring stages");
};

// One MFMA, then V vector-ALU ops (its shadow: one wave issues while its
// MFMA runs, so the two pipes overlap only when their instructions alternate).
template <int V>
__device__ inline void mfma_then_valu() {
  __builtin_amdgcn_sched_group_barrier(kSchedMFMA, 1, 0);
  if constexpr (V > 0) __builtin_amdgcn_sched_group_barrier(kSchedVALU, V, 0);
}
__device__ inline void mfma_then_about(int v) {
  if (v <= 0) mfma_then_valu<0>();
  else if (v <= 4) mfma_then_valu<4>();
  else if (v <= 6) mfma_then_valu<6>();
  else if (v <= 8) mfma_then_valu<8>();
  else if (v <= 12) mfma_then_valu<12>();
  else if (v <= 16) mfma_then_valu<16>();
  else if (v <= 32) mfma_then_valu<32>();
  else mfma_then_valu<64>();
}
// nm (2 or 4) MFMAs of a tail k-step, each followed by about v VALU ops
__device__ inline void schedule_tail_step(int nm, int v) {
  mfma_then_about(v);
  mfma_then_about(v);
  if (nm > 2) {
    mfma_then_about(v);
    mfma_then_about(v);
  }
}

template <int MT, int EPI>
__device__ inline void tail(uint8_t *smem, uint32_t c, uint32_t h, uint32_t r, uint32_t wave,
                            f32x16 (&acc)[2][MT], const f16x8 (&w)[2][4], const f16x8 (&af)[MT],
                            RawW &r0, RawW &r1, RawW &r2, RawW &r3, f16 *__restrict__ Cout,
                            const float *__restrict__ bias, uint32_t M, uint32_t N, uint32_t m0,
                            uint32_t p0, uint32_t np) {
  using G = Geometry<MT>;
  using TG = Tail<MT>;
  constexpr int NB = EPI != MADI_EPI_NONE ? 8 : 0;  // bias loads per lane
  const uint8_t *st[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) st[j] = smem + ((c + j) & (NA - 1)) * G::kStage;
  uint8_t *stg = smem + ((c + 4) & (NA - 1)) * G::kStage;
  uint32_t phys[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) phys[s] = ((h * 4 + s) ^ a_swz(r)) * 16;

  // chunk c+1's weights: only chunks c+2 and c+3's loads may be outstanding
  wait_weights<2 * G::kPerChunk>(r1);
  f32x4 b4[2][4];
  if constexpr (NB) load_bias(b4, bias, np, p0, wave, h);

  f16x8 W[4][2][4];  // [chunk c + j][panel][k-step]
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int s = 0; s < 3; ++s) W[0][t][s] = w[t][s];

  // C: rows past M fall outside the resource; columns past N get an offset
  // past its end (no branch around the stores)
  const uint32_t rows = M - m0 < 32 * MT ? M - m0 : 32 * MT;
  const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
      Cout + (size_t)m0 * N, 0, (int)(rows * N * 2), 0x00020000);
  const uint32_t n = p0 * kPanelRows + r * 8;
  const uint32_t col_ok = n < N ? 0u : 0x80000000u;

  // the conversion of m-tile q's register group (t, g): bias, GELU, f16, LDS
  auto epi_group = [&](int q, int t, int g) {
    uint8_t *Ct = stg + (q % TG::kBufs) * TG::kCBuf;
    const uint32_t nl = (2 * wave + t) * kPanelRows;
    float v[4] = {acc[t][q][g * 4 + 0], acc[t][q][g * 4 + 1], acc[t][q][g * 4 + 2],
                  acc[t][q][g * 4 + 3]};
    if constexpr (EPI != MADI_EPI_NONE) {
      v[0] += b4[t][g].x;
      v[1] += b4[t][g].y;
      v[2] += b4[t][g].z;
      v[3] += b4[t][g].w;
      if constexpr (EPI == MADI_EPI_BIAS_GELU) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gelu_erf_fast(v[e]);
      }
    }
    const f16x4 o = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
    *reinterpret_cast<f16x4 *>(Ct + r * kCStride + (nl + g * 8 + h * 4) * 2) = o;
  };
  // staged rows of m-tile q: lane (h, r) holds 16 bytes of row 2j + h of the
  // wave's eight, at column 8r
  u32x4 cv[4];
  auto epi_read = [&](int q) {
    const uint8_t *Ct = stg + (q % TG::kBufs) * TG::kCBuf;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      cv[j] = *reinterpret_cast<const u32x4 *>(Ct + (wave * 8 + 2 * j + h) * kCStride + r * 16);
  };
  auto epi_store = [&](int q, int j) {
    const uint32_t row = q * 32 + wave * 8 + 2 * j + h;
    // 24-bit product (rows < 2^7, N < 2^24): a 32-bit multiply-add, which
    // the compiler would otherwise form with a 64-bit addend whose unused
    // high half is an arbitrary live register
    __builtin_amdgcn_raw_buffer_store_b128(cv[j], cr, ((__umul24(row, N) + n) * 2) | col_ok, 0,
                                           kSc1);
  };

  // Passes: pass 0 runs m-tiles [0, P0) (two where there are three or more,
  // so that sixteen MFMAs per slot cover the dequantisation of the next
  // chunk), every later pass one m-tile.  Pass p >= 1 also retires the
  // m-tiles pass p-1 finished: one m-tile is converted over slots 0-1 (a
  // register group per k-step) and stored in slot 2; two are converted in
  // slots 0 and 1 (two groups per k-step) and stored in slots 1 and 2.  A
  // store slot first meets the other waves (the m-tile is staged).
  constexpr int P0 = MT >= 3 ? 2 : 1;
  constexpr int NP = MT - P0 + 1;
  static_assert(TG::kBufs == 2 || MT == 2, "a staging buffer is rewritten only after a barrier");
  auto first = [](int pp) { return pp == 0 ? 0 : P0 + pp - 1; };
  auto count = [](int pp) { return pp == 0 ? P0 : 1; };

  // A fragments of slot (p, j) = the pass's m-tiles, chunk c + j, read one slot ahead
  f16x8 fa[2][P0][4];
  auto read_frags = [&](int pp, int j, f16x8 (&dst)[P0][4]) {
#pragma unroll
    for (int mi = 0; mi < P0; ++mi) {
      if (mi < count(pp)) {
        const int i = first(pp) + mi;
#pragma unroll
        for (int s = 0; s < 4; ++s)
          dst[mi][s] = j == 0 && s == 0
                           ? af[i]
                           : *reinterpret_cast<const f16x8 *>(st[j] + (i * 32 + r) * 128 + phys[s]);
      }
    }
  };
  read_frags(0, 0, fa[0]);

#pragma unroll
  for (int pp = 0; pp < NP; ++pp) {
    const int R = pp == 0 ? 0 : count(pp - 1), q0 = pp == 0 ? 0 : first(pp - 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int cur = (pp * 4 + j) & 1;
      if (pp == 0 && j == 1) {
        // chunk c+2's A stage and weights (chunk c+3's loads and the bias may be outstanding)
        wait_then_barrier<G::kPerChunk + NB>();
        wait_weights<G::kPerChunk + NB>(r2);
      }
      if (pp == 0 && j == 2) {
        wait_then_barrier<NB>();  // chunk c+3's A stage and weights
        wait_weights<NB>(r3);
      }
      if constexpr (NB) {
        if (pp == 1 && j == 0) wait_bias<0>(b4);
      }
      // the m-tile this slot stores, if any
      const int sq = R == 1 ? (j == 2 ? q0 : -1) : R == 2 ? (j == 1 ? q0 : j == 2 ? q0 + 1 : -1) : -1;
      if (sq >= 0) lds_barrier();  // m-tile sq is staged
      if (pp * 4 + j + 1 < NP * 4) {
        const int np_ = (pp * 4 + j + 1) / 4, nj = (pp * 4 + j + 1) % 4;
        read_frags(np_, nj, fa[cur ^ 1]);
      }
      if (sq >= 0) epi_read(sq);
      __builtin_amdgcn_sched_barrier(0);
      // each k-step: the pass's MFMAs, then a share of the slot's other work
#pragma unroll
      for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int mi = 0; mi < P0; ++mi) {
          if (mi < count(pp)) {
            const int i = first(pp) + mi;
            acc[0][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(W[j][0][s], fa[cur][mi][s], acc[0][i], 0, 0, 0);
            acc[1][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(W[j][1][s], fa[cur][mi][s], acc[1][i], 0, 0, 0);
          }
        }
        if (pp == 0) {
          // the next chunk's fragments (t, u) = (s >> 1, 2 (s & 1) ..), and
          // this chunk's step-3 fragments at step 0
          if (j == 0 && s == 0) {
            W[0][0][3] = dequant_frag(r0, 0, 3);
            W[0][1][3] = dequant_frag(r0, 1, 3);
          }
          if (j < 3) {
            const RawW &src = j == 0 ? r1 : j == 1 ? r2 : r3;
            const int t = s >> 1, u = 2 * (s & 1);
            W[j + 1][t][u] = dequant_frag(src, t, u);
            W[j + 1][t][u + 1] = dequant_frag(src, t, u + 1);
          }
        }
        if (R == 1 && j < 2) {
          const int g8 = 4 * j + s;
          epi_group(q0, g8 >> 2, g8 & 3);
        }
        if (R == 2 && j < 2) {
          epi_group(q0 + j, s >> 1, 2 * (s & 1));
          epi_group(q0 + j, s >> 1, 2 * (s & 1) + 1);
        }
        if (sq >= 0) epi_store(sq, s);
        // VALU ops of the step: 12 per dequantised fragment; per converted
        // register group 6 (accumulator reads, conversions), 4 more with a
        // bias, ~44 more with GELU; 2 for a store's address
        constexpr int kGroupOps = 6 + (EPI != MADI_EPI_NONE ? 4 : 0) + (EPI == MADI_EPI_BIAS_GELU ? 44 : 0);
        const int nm = 2 * count(pp);
        const int ops = (pp == 0 ? (j < 3 ? 24 : 0) + (j == 0 && s == 0 ? 24 : 0) : 0) +
                        (R == 1 && j < 2 ? kGroupOps : 0) + (R == 2 && j < 2 ? 2 * kGroupOps : 0) +
                        (sq >= 0 ? 2 : 0);
        schedule_tail_step(nm, (ops + nm - 1) / nm);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  if (TG::kBufs == 1) lds_barrier();  // m-tile MT-2's rows are read
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) epi_group(MT - 1, t, g);
  lds_barrier();
  epi_read(MT - 1);
#pragma unroll
  for (int j = 0; j < 4; ++j) epi_store(MT - 1, j);
}


// Where a tile's outputs go: the launch's C and bias, or, when the launch
// writes several outputs (OutSeg: the encoder's q, k and v from one stacked
// weight), the segment holding the tile's columns (segments are whole tiles
// wide: the host checks), with its own pointers, row pitch and panel origin.
struct OutTile {
  void *c;
  const float *b;
  uint32_t n, p0, np;
};
__device__ inline OutTile out_tile(const OutSeg &seg, void *C, const float *bias, uint32_t N,
                                   uint32_t p0) {
  if (seg.n == 0) return {C, bias, N, p0, N / kPanelRows};
  const uint32_t n0 = p0 * kPanelRows;
  uint32_t s = 0;
#pragma unroll
  for (int i = 1; i < kMaxSegs; ++i) s += n0 >= i * seg.n ? 1u : 0u;
  return {seg.c[s], seg.b[s], seg.n, p0 - s * (seg.n / kPanelRows), seg.n / kPanelRows};
}

template <int MT, int EPI, bool PADDED, bool F32 = false, bool TAIL = false, int PW = 2>
__global__ __launch_bounds__(256) void q8_gemm_kernel(
    const void *__restrict__ A, const uint8_t *__restrict__ qs, const f16 *__restrict__ sc,
    uint32_t M, uint32_t N, uint32_t K, uint32_t tiles_m, uint32_t tiles_n, uint32_t splits,
    uint32_t cper, uint32_t crem, void *__restrict__ Cout, const float *__restrict__ bias,
    float *__restrict__ ws, uint32_t *__restrict__ cnt, const OutSeg seg) {
  using G = Geometry<MT, F32, PW>;
  static_assert(!F32 || EPI == MADI_EPI_NONE, "f32 output has no bias epilogue");
  static_assert(!TAIL || (!PADDED && !F32 && MT >= 2 && PW == 2), "the m-tile-major tail's shapes");
  static_assert(PW == 2 || !PADDED, "128-column tiles: unpadded launches");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[G::kLds];
  __shared__ uint32_t arrived;

  // ---- tile order: consecutive workgroups go to different XCDs (round-robin),
  // so the work items are renumbered to give each XCD a contiguous run.  The
  // W = T * splits items (item tile * splits + split) are cut into eight runs
  // whose lengths differ by at most one; the grid is W rounded up to a
  // multiple of 8, workgroup L runs on XCD L % 8 and takes the (L / 8)-th item
  // of that XCD's run, or exits past its end.  An XCD thus holds every K
  // split of consecutive tiles, walked in groups of `group_m` M-tiles, so its
  // tiles share A rows and W panels in its own L2.  (Measured against a
  // split-major order, where an XCD holds consecutive tiles of one K range,
  // and against the plain round-robin order: as fast or faster on every
  // shape, e.g. FFN down 5120 -> 1280 at M = 320 f32 15.3 / 15.7 / 17.8 us,
  // 24000 x 5120 -> 1280 f16 280 / 282 / 297 us.)  Split s covers chunks [s * cper + min(s, crem), + cper +
  // (s < crem)) of the tile.  The arguments the mapping needs come first and
  // arrive preloaded in SGPRs (the first 14 dwords); C, the bias and the
  // split-K workspace, needed only at the end, follow.
  const uint32_t T = tiles_m * tiles_n;
  const uint32_t W = T * splits, L = blockIdx.x, x = L & 7;
  const uint32_t first = (x * W) >> 3, run = (((x + 1) * W) >> 3) - first;
  if ((L >> 3) >= run) return;
  const uint32_t item = first + (L >> 3);
  // launches that never split K (the m-tile-major tail, the f16 128-column
  // tiles: the host checks) skip the division
  constexpr bool kUnsplit = TAIL || (PW == 1 && !F32);
  const uint32_t bid = kUnsplit ? item : item / splits, split = kUnsplit ? 0u : item - bid * splits;
  const uint32_t tile = bid;
  const uint32_t group_m = tiles_m < 6 ? tiles_m : 6;
  const uint32_t per_group = group_m * tiles_n;
  const uint32_t gi = bid / per_group, first_m = gi * group_m;
  const uint32_t gm = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
  const uint32_t tm = first_m + (bid % per_group) % gm;
  const uint32_t tn = (bid % per_group) / gm;

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t h = lane >> 5, r = lane & 31;
  const uint32_t m0 = tm * 32 * MT, p0 = tn * G::kTilePanels;
  const uint32_t np = N / kPanelRows;
  const uint32_t cb = split * cper + (split < crem ? split : crem);
  const uint32_t nchunks = cper + (split < crem ? 1 : 0);

  // ---- load plan.  Panels past N and rows past M are clamped to the last
  // valid one: their bytes are read but their results are never stored.
  Plan<MT, F32, PW> p;
  p.wq = make_desc(qs, N * K);
  p.ws = make_desc(sc, N * K / 16);
  p.wa = make_desc(A, M * K * (F32 ? 4 : 2));
  p.zero = make_desc(A, 0);
  p.nchunks = nchunks;
#pragma unroll
  for (int t = 0; t < PW; ++t) {
    uint32_t pp = p0 + PW * wave + t;
    pp = pp < np ? pp : np - 1;
    p.w_soff[t] = pp * kPanelRows * K + cb * 2048;
    p.s_voff[t] = pp * K * 2 + cb * 128 + lane * 2;  // panel pp's chunk c scales at pp*K + 64c elements
  }
#pragma unroll
  for (int i = 0; i < G::LA; ++i) {
    // wave w copies DMAs LA*w .. LA*w+LA-1 of the stage, 1 KiB each: 8 rows
    // of 64 f16 or 4 rows of 64 f32
    constexpr uint32_t kRowsPerDma = F32 ? 4 : 8;
    const uint32_t row = (G::LA * wave + i) * kRowsPerDma + (lane >> (F32 ? 4 : 3));
    const uint32_t q = F32 ? (lane & 15) ^ a_swz32(row) : (lane & 7) ^ a_swz(row);
    uint32_t m = m0 + row;
    m = m < M ? m : M - 1;
    // the DMA adds its instruction offset 1024*i to both addresses (DMA i
    // starts kRowsPerDma*i rows, at least 1024*i bytes, into A, so this cannot wrap)
    p.a_voff[i] = m * K * (F32 ? 4 : 2) + cb * G::kRowBytes + q * 16 - 1024 * i;
  }
  p.a_lds = G::LA * wave * 1024;

  f32x16 acc[PW][MT];
#pragma unroll
  for (int t = 0; t < PW; ++t)
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[t][i] = (f32x16){};

  // ---- prologue: the loads the steady state would have issued before chunk 0
  // (virtual chunks -4 .. -1), in the same order, so the loop's vmcnt waits
  // hold from the first chunk on.  Virtual chunk j loads A stage j+DA and
  // weights j+WD (stages and weights past the last chunk load zeros); register
  // set k receives chunks k, k+WD, ...
  RawWT<PW> r0, r1, r2, r3;
  static_assert(WD == 4 && DA == 4, "the loop below rotates four weight register sets");
  static_assert(NA >= DA + 2, "an A stage is refilled only after the barrier that retires it");
  // Ramped start (the m-tile-major tail's launches, at least twelve chunks:
  // the host checks): the prologue issues chunks 0 and 1 only, and chunks 0
  // and 1 issue chunks 2-5 among their MFMAs, in the steady state's global
  // order, so every later wait keeps its count.  The CU's load pipe accepts
  // ~64 bytes per cycle, so the four-chunk prologue (128 KiB per CU) held the
  // first MFMA back ~2000 cycles (per-wave stamps); waiting after two
  // chunks' loads with the rest issued before the first MFMA measured no
  // faster.
  constexpr bool kRamp = TAIL;
#pragma unroll
  for (int j = -4; j < (kRamp ? -2 : 0); ++j) {
    uint8_t *slot = smem + (uint32_t)(j + DA) * G::kStage;
    RawWT<PW> &rw = j == -4 ? r0 : j == -3 ? r1 : j == -2 ? r2 : r3;
#pragma unroll
    for (int st = 0; st < 4; ++st)
      // unpadded loops have at least eight chunks per split: all four live
      issue_loads<MT, F32, PADDED ? kSel : kLive>(st, slot, (uint32_t)(j + DA), rw,
                                                 (uint32_t)(j + WD), p, lane);
  }
  // chunk 0's weights and the A stages of chunks 0 and 1 (chunk 0 reads
  // chunk 1's stage without a barrier of its own), then chunk 0's fragments
  constexpr int kVmStart = kRamp ? G::LW : G::kVmPrologue;
  wait_then_barrier<kVmStart>();
  wait_weights<kVmStart>(r0);
  f16x8 w[PW][4];
  typename AFrag<F32>::T af[MT];
#pragma unroll
  for (int t = 0; t < PW; ++t)
#pragma unroll
    for (int s = 0; s < 3; ++s) w[t][s] = dequant_frag(r0, t, s);
  load_a_frags<MT>(smem, 0, h, r, af);

  // ---- main loop: four chunks per trip (the weight register sets rotate).
  // The loop body stays one straight-line block: extra exits let the register
  // allocator copy asm-loaded registers before their vmcnt wait.  Unpadded
  // (the chunk count a multiple of four): every trip but the last prefetches
  // only live chunks; the last trip is peeled, its prefetch targets known.
  if constexpr (PADDED) {
    const uint32_t cpad = (nchunks + WD - 1) / WD * WD;
    for (uint32_t c = 0; c < cpad; c += 4) {
      chunk<MT, F32, kSel, false>(smem, p, c + 0, lane, h, r, acc, w, af, r0, r1, r0, r0);
      chunk<MT, F32, kSel, true>(smem, p, c + 1, lane, h, r, acc, w, af, r1, r2, r1, r1);
      chunk<MT, F32, kSel, false>(smem, p, c + 2, lane, h, r, acc, w, af, r2, r3, r2, r2);
      chunk<MT, F32, kSel, true>(smem, p, c + 3, lane, h, r, acc, w, af, r3, r0, r3, r3);
    }
  } else {
    // at least two trips (the host checks): the loop is never skipped, so the
    // prologue's registers reach the last trip only through it and need no
    // copies on a path around it
    uint32_t c = 0;
    if constexpr (kRamp) {
      chunk<MT, F32, kRamp0, false>(smem, p, 0, lane, h, r, acc, w, af, r0, r1, r2, r3);
      chunk<MT, F32, kRamp1, true>(smem, p, 1, lane, h, r, acc, w, af, r1, r2, r0, r1);
      chunk<MT, F32, kLive, false>(smem, p, 2, lane, h, r, acc, w, af, r2, r3, r2, r2);
      chunk<MT, F32, kLive, true>(smem, p, 3, lane, h, r, acc, w, af, r3, r0, r3, r3);
      c = 4;
    }
    do {
      chunk<MT, F32, kLive, false>(smem, p, c + 0, lane, h, r, acc, w, af, r0, r1, r0, r0);
      chunk<MT, F32, kLive, true>(smem, p, c + 1, lane, h, r, acc, w, af, r1, r2, r1, r1);
      chunk<MT, F32, kLive, false>(smem, p, c + 2, lane, h, r, acc, w, af, r2, r3, r2, r2);
      chunk<MT, F32, kLive, true>(smem, p, c + 3, lane, h, r, acc, w, af, r3, r0, r3, r3);
      c += 4;
    } while (c + 2 * WD <= nchunks);
    if constexpr (TAIL) {
      // one K split (the host checks): the tile's epilogue is the tail's
      const OutTile ot = out_tile(seg, Cout, bias, N, p0);
      tail<MT, EPI>(smem, c, h, r, wave, acc, w, af, r0, r1, r2, r3, static_cast<f16 *>(ot.c),
                    ot.b, M, ot.n, m0, ot.p0, ot.np);
      return;
    } else {
      chunk<MT, F32, kLast0, false>(smem, p, c + 0, lane, h, r, acc, w, af, r0, r1, r0, r0);
      chunk<MT, F32, kLast1, true>(smem, p, c + 1, lane, h, r, acc, w, af, r1, r2, r1, r1);
      chunk<MT, F32, kLast2, false>(smem, p, c + 2, lane, h, r, acc, w, af, r2, r3, r2, r2);
      chunk<MT, F32, kLast3, true>(smem, p, c + 3, lane, h, r, acc, w, af, r3, r0, r3, r3);
    }
  }

  drain(r0, r1, r2, r3);

  // ---- epilogue.  Lane (h, r) holds D[n][m] for m = 32i + r and
  // n = 32(PW w + t) + 8g + 4h + e (acc[t][i][4g + e]).  Every wave must finish
  // reading the ring before it becomes the C tile.
  wait_then_barrier<0>();
  // f16 launches of 128-column tiles run unsplit (the host checks), and leave
  // the reduction's registers out of their allocation
  constexpr bool kSplits = PW == 2 || F32;
  if constexpr (kSplits) {
  if (splits > 1) {
    // Split K: every workgroup of the tile publishes its partial sums (in
    // register order, so each lane later reads back exactly what it wrote) and
    // counts itself in; the last to arrive adds the others' partials to its
    // own and finishes the tile.  The partials are written and read with
    // device-scope (sc1) buffer accesses, which write through and read past
    // the XCD's own L2, and the count is a device-scope atomic (every party is
    // a workgroup of this launch), so no L2-wide writeback or invalidate is
    // needed.
    constexpr uint32_t kPart = 4 * PW * MT * 4 * 64 * 16;  // bytes per partial tile
    const __amdgpu_buffer_rsrc_t wsr =
        __builtin_amdgcn_make_buffer_rsrc(ws, 0, (int)(T * splits * kPart), 0x00020000);
#pragma unroll
    for (int t = 0; t < PW; ++t)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(u32x4, (f32x4){acc[t][i][4 * g], acc[t][i][4 * g + 1],
                                                acc[t][i][4 * g + 2], acc[t][i][4 * g + 3]}),
              wsr, ((((wave * PW + t) * MT + i) * 4 + g) * 64 + lane) * 16,
              (tile * splits + split) * kPart, kSc1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partial has been written through
    __syncthreads();
    if (threadIdx.x == 0)
      arrived = __hip_atomic_fetch_add(&cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != splits - 1) return;
    constexpr int kGroups = PW * MT * 4;  // register groups q = (t, i, g) in order
    if (MT <= 2 && splits == 2) {
      // Two splits (fc2-like shapes at 64-row tiles): the wave's whole share
      // of the other partial (PW * MT * 4 KiB) in flight at once, one memory
      // latency; own + other is exact in either order.
      const uint32_t other = split ^ 1u;
      f32x4 o[kGroups];
#pragma unroll
      for (int q = 0; q < kGroups; ++q)
        o[q] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(wsr, ((wave * kGroups + q) * 64 + lane) * 16,
                                                         (tile * splits + other) * kPart, kSc1));
#pragma unroll
      for (int q = 0; q < kGroups; ++q) {
        const int t = q / (MT * 4), i = (q / 4) % MT, g = q % 4;
        acc[t][i][4 * g] += o[q].x;
        acc[t][i][4 * g + 1] += o[q].y;
        acc[t][i][4 * g + 2] += o[q].z;
        acc[t][i][4 * g + 3] += o[q].w;
      }
    } else {
    // Sum the splits' partials in split order, this workgroup's own from its
    // registers at its own position, so the result does not depend on which
    // workgroup arrives last.  One fully unrolled pass over the register
    // groups, each group's loads for every split issued together, keeps many
    // loads in flight (a pass per split waited out the memory latency once
    // per split).
    static_assert(kMaxSplits == 4, "the reduction below unrolls four splits");
    // every load is issued (a split past `splits`, or this workgroup's own,
    // reads zeros through an empty resource), and the own partial enters by a
    // 0/1 factor: no branches, so the loads of many groups stay in flight
    __amdgpu_buffer_rsrc_t rs[kMaxSplits];
    float mine[kMaxSplits];
    const __amdgpu_buffer_rsrc_t zr = __builtin_amdgcn_make_buffer_rsrc(ws, 0, 0, 0x00020000);
#pragma unroll
    for (uint32_t s2 = 0; s2 < kMaxSplits; ++s2) {
      rs[s2] = s2 < splits && s2 != split ? wsr : zr;
      mine[s2] = s2 == split ? 1.0f : 0.0f;
    }
    // group q + kAhead's loads are issued before group q is summed, so the
    // waits only cover old loads
    constexpr int kAhead = 6;
    auto load_group = [&](int q, f32x4 (&dst)[kMaxSplits]) {
      const uint32_t voff = ((wave * kGroups + q) * 64 + lane) * 16;
#pragma unroll
      for (uint32_t s2 = 0; s2 < kMaxSplits; ++s2)
        dst[s2] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                rs[s2], voff, (tile * splits + s2) * kPart, kSc1));
    };
    f32x4 ring[kAhead + 1][kMaxSplits];
#pragma unroll
    for (int q = 0; q < kAhead; ++q) load_group(q, ring[q]);
#pragma unroll
    for (int q = 0; q < kGroups; ++q) {
      if (q + kAhead < kGroups) load_group(q + kAhead, ring[(q + kAhead) % (kAhead + 1)]);
      const int t = q / (MT * 4), i = (q / 4) % MT, g = q % 4;
      const f32x4 own = {acc[t][i][4 * g], acc[t][i][4 * g + 1], acc[t][i][4 * g + 2],
                         acc[t][i][4 * g + 3]};
      f32x4 part[kMaxSplits];
#pragma unroll
      for (uint32_t s2 = 0; s2 < kMaxSplits; ++s2)
        part[s2] = ring[q % (kAhead + 1)][s2] + own * mine[s2];
      // splits past `splits` add exact zeros
      const f32x4 sum = ((part[0] + part[1]) + part[2]) + part[3];
      acc[t][i][4 * g] = sum.x;
      acc[t][i][4 * g + 1] = sum.y;
      acc[t][i][4 * g + 2] = sum.z;
      acc[t][i][4 * g + 3] = sum.w;
      __builtin_amdgcn_sched_barrier(0);
    }
    }
    if (threadIdx.x == 0)  // ready for the next launch
      __hip_atomic_store(&cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  }
  const OutTile ot = out_tile(seg, Cout, bias, N, p0);
  // The tile leaves through LDS one m-tile (32 rows) at a time: all waves
  // write their columns of m-tile i, meet, and each stores 8 of its rows
  // while the next m-tile is converted, so the stores (the HBM write rate
  // bounds them: every workgroup writes at once) start after a quarter of
  // the conversion instead of all of it.  A store instruction writes two
  // rows (512 B each): lane (h, r) writes 16 bytes of row 2j + h at column
  // 8r.  The stores write through the L2 (sc1), so the tile leaves no dirty
  // lines for the end-of-kernel release to write back after the last
  // workgroup; rows past M fall outside the tile's buffer resource and are
  // dropped, columns past N are skipped per lane.
  uint8_t *Ct = smem;
  const uint32_t rows = M - m0 < 32 * MT ? M - m0 : 32 * MT;
  if constexpr (F32) {
    // f32 result: a row of the tile is 32 PW lanes' 16 bytes (4 columns
    // each), a store instruction 2 / PW rows
    constexpr uint32_t kLanesPerRow = 32 * PW, kRowsPerStore = 2 / PW;
    const uint32_t col = lane % kLanesPerRow;
    const uint32_t n = ot.p0 * kPanelRows + col * 4;
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        static_cast<float *>(ot.c) + (size_t)m0 * ot.n, 0, (int)(rows * ot.n * 4), 0x00020000);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int t = 0; t < PW; ++t) {
        const uint32_t nl = (PW * wave + t) * kPanelRows;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 o = {acc[t][i][g * 4 + 0], acc[t][i][g * 4 + 1], acc[t][i][g * 4 + 2],
                           acc[t][i][g * 4 + 3]};
          *reinterpret_cast<f32x4 *>(Ct + (i * 32 + r) * G::kCPitch + (nl + g * 8 + h * 4) * 4) = o;
        }
      }
      __syncthreads();
#pragma unroll
      for (uint32_t j = 0; j < 8 / kRowsPerStore; ++j) {
        const uint32_t row = i * 32 + wave * 8 + j * kRowsPerStore + lane / kLanesPerRow;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(Ct + row * G::kCPitch + col * 16);
        if (n < ot.n) __builtin_amdgcn_raw_buffer_store_b128(v, cr, (row * ot.n + n) * 4, 0, kSc1);
      }
    }
    return;
  }
  // a row of the tile is 16 PW lanes' 16 bytes, a store instruction 4 / PW rows
  constexpr uint32_t kLanesPerRow = 16 * PW, kRowsPerStore = 4 / PW;
  const uint32_t n = ot.p0 * kPanelRows + (lane % kLanesPerRow) * 8;
  const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
      static_cast<f16 *>(ot.c) + (size_t)m0 * ot.n, 0, (int)(rows * ot.n * 2), 0x00020000);
  f32x4 b4[PW][4];
  if constexpr (EPI != MADI_EPI_NONE) {
#pragma unroll
    for (int t = 0; t < PW; ++t) {
      uint32_t pb = ot.p0 + PW * wave + t;
      pb = pb < ot.np ? pb : ot.np - 1;  // clamped panels: bias read in bounds, result never stored
#pragma unroll
      for (int g = 0; g < 4; ++g)
        b4[t][g] = *reinterpret_cast<const f32x4 *>(ot.b + pb * kPanelRows + g * 8 + h * 4);
    }
  }
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int t = 0; t < PW; ++t) {
      const uint32_t nl = (PW * wave + t) * kPanelRows;  // tile-local column of the panel
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float v[4] = {acc[t][i][g * 4 + 0], acc[t][i][g * 4 + 1], acc[t][i][g * 4 + 2],
                      acc[t][i][g * 4 + 3]};
        if constexpr (EPI != MADI_EPI_NONE) {
          v[0] += b4[t][g].x;
          v[1] += b4[t][g].y;
          v[2] += b4[t][g].z;
          v[3] += b4[t][g].w;
          if constexpr (EPI == MADI_EPI_BIAS_GELU) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gelu_erf_fast(v[e]);
          }
        }
        const f16x4 o = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
        *reinterpret_cast<f16x4 *>(Ct + (i * 32 + r) * G::kCPitch + (nl + g * 8 + h * 4) * 2) = o;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2 * PW; ++j) {
      const uint32_t row = i * 32 + wave * 8 + kRowsPerStore * j + lane / kLanesPerRow;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(Ct + row * G::kCPitch +
                                                       (lane % kLanesPerRow) * 16);
      if (n < ot.n) __builtin_amdgcn_raw_buffer_store_b128(v, cr, (row * ot.n + n) * 2, 0, kSc1);
    }
  }
}

// ---------------------------------------------------------------- persistent tile loop
// Many tiles per CU (long audio: M = 24000, 3760 fc1 tiles): each workgroup
// of a device-sized grid walks its tiles, and once a tile's K loop is done it
// issues the next tile's prologue loads (weights of chunks 0-3 into the four
// register sets, A of chunks 0-3 into ring stages 0-3) BEFORE running the
// finished tile's epilogue, so the first-chunk latency of the next tile
// passes under the conversion and stores of this one.  The epilogue stages
// the C tile two m-tiles at a time in ring stages 4-7, clear of the DMAs.
//
// Vector-memory accounting: a finished tile issues its bias loads, then the
// next tile's prologue, then its own C stores, so between a tile's prologue
// and its K loop lie kEpi = 16 stores.  The first tile issues as many empty
// DMAs (zero-length buffer, into ring stage 7, which chunk 3 refills later)
// so that every tile's first trip waits with the same counts (kLiveE, offset
// kEpi).
template <int EPI>
struct Persist {
  static constexpr int MT = 4;
  static constexpr int kStores = MT * 4;  // C stores per wave
  static constexpr int kEpi = kStores;
  static constexpr int kStage = Geometry<MT>::kStage;
  static constexpr int kCBuf = 32 * kCStride;  // one m-tile of the C tile
  static_assert(4 * kStage + 2 * kCBuf <= Geometry<MT>::kRing, "C staging fits stages 4-7");
};

template <int EPI>
__global__ __launch_bounds__(256) void q8_gemm_persist_kernel(
    const f16 *__restrict__ A, const uint8_t *__restrict__ qs, const f16 *__restrict__ sc,
    uint32_t M, uint32_t N, uint32_t K, uint32_t tiles_m, uint32_t tiles_n, uint32_t group_m,
    f16 *__restrict__ Cout, const float *__restrict__ bias) {
  using P = Persist<EPI>;
  constexpr int MT = P::MT;
  using G = Geometry<MT>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[G::kLds];

  const uint32_t T = tiles_m * tiles_n, Gd = gridDim.x;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t h = lane >> 5, r = lane & 31;
  const uint32_t np = N / kPanelRows, nchunks = K / kChunkK;
  // round j of this workgroup: tile index j * Gd + (its place in round 0);
  // workgroup x runs on XCD x % 8, and the 32 workgroups of an XCD take a
  // contiguous run of the round's tiles
  const uint32_t bx = blockIdx.x;
  uint32_t L = (bx & 7) * (Gd >> 3) + (bx >> 3);

  Plan<MT, false> p;
  p.wq = make_desc(qs, N * K);
  p.ws = make_desc(sc, N * K / 16);
  p.wa = make_desc(A, M * K * 2);
  p.zero = make_desc(A, 0);
  p.nchunks = nchunks;
  p.a_lds = MT * wave * 1024;
  uint32_t m0 = 0, p0 = 0;
  // the load plan of tile L (its m-tile row and 256-column group)
  auto plan = [&](uint32_t Lt) {
    const uint32_t per_group = group_m * tiles_n;
    const uint32_t gi = Lt / per_group, first_m = gi * group_m;
    const uint32_t gm = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
    const uint32_t tm = first_m + (Lt % per_group) % gm;
    const uint32_t tn = (Lt % per_group) / gm;
    m0 = tm * 32 * MT;
    p0 = tn * kPanelsPerTile;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t pp = p0 + 2 * wave + t;  // N % 256 == 0: every panel exists
      p.w_soff[t] = pp * kPanelRows * K;
      p.s_voff[t] = pp * K * 2 + lane * 2;
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const uint32_t row = (MT * wave + i) * 8 + (lane >> 3);
      const uint32_t q = (lane & 7) ^ a_swz(row);
      uint32_t m = m0 + row;
      m = m < M ? m : M - 1;
      p.a_voff[i] = m * K * 2 + q * 16 - 1024 * i;
    }
  };
  RawW r0, r1, r2, r3;
  auto prologue = [&]() {
#pragma unroll
    for (int j = -4; j < 0; ++j) {
      uint8_t *slot = smem + (uint32_t)(j + DA) * G::kStage;
      RawW &rw = j == -4 ? r0 : j == -3 ? r1 : j == -2 ? r2 : r3;
#pragma unroll
      for (int st = 0; st < 4; ++st)
        issue_loads<MT, false, kLive>(st, slot, (uint32_t)(j + DA), rw, (uint32_t)(j + WD), p, lane);
    }
  };

  if (L >= T) return;
  plan(L);
  prologue();
  // stand-ins for the epilogue issues a later tile finds between its prologue
  // and its K loop: empty DMAs into stage 7
#pragma unroll
  for (int e = 0; e < P::kEpi; ++e)
    dma16<0, true>(p.zero, lane * 16, 0, lds_addr(smem + 7 * G::kStage + (e & 15) * 1024));

  for (;;) {
    // the prologue's chunk 0 weights and A stages 0-1 have landed everywhere
    wait_then_barrier<G::kVmPrologue + P::kEpi>();
    wait_weights<G::kVmPrologue + P::kEpi>(r0);
    f16x8 w[2][4], af[MT];
#pragma unroll
    for (int s = 0; s < 3; ++s) w[0][s] = dequant_frag(r0, 0, s);
#pragma unroll
    for (int s = 0; s < 3; ++s) w[1][s] = dequant_frag(r0, 1, s);
    load_a_frags<MT>(smem, 0, h, r, af);
    f32x16 acc[2][MT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < MT; ++i) acc[t][i] = (f32x16){};

    // K loop: first trip (targets before it in the prologue), live trips, the
    // peeled last trip; nchunks a multiple of four and at least 12
    chunk<MT, false, kLiveE, false, P::kEpi>(smem, p, 0, lane, h, r, acc, w, af, r0, r1, r0, r0);
    chunk<MT, false, kLiveE, true, P::kEpi>(smem, p, 1, lane, h, r, acc, w, af, r1, r2, r1, r1);
    chunk<MT, false, kLiveE, false, P::kEpi>(smem, p, 2, lane, h, r, acc, w, af, r2, r3, r2, r2);
    chunk<MT, false, kLive, true>(smem, p, 3, lane, h, r, acc, w, af, r3, r0, r3, r3);
    uint32_t c = 4;
    do {
      chunk<MT, false, kLive, false>(smem, p, c + 0, lane, h, r, acc, w, af, r0, r1, r0, r0);
      chunk<MT, false, kLive, true>(smem, p, c + 1, lane, h, r, acc, w, af, r1, r2, r1, r1);
      chunk<MT, false, kLive, false>(smem, p, c + 2, lane, h, r, acc, w, af, r2, r3, r2, r2);
      chunk<MT, false, kLive, true>(smem, p, c + 3, lane, h, r, acc, w, af, r3, r0, r3, r3);
      c += 4;
    } while (c + 2 * WD <= nchunks);
    chunk<MT, false, kLast0, false>(smem, p, c + 0, lane, h, r, acc, w, af, r0, r1, r0, r0);
    chunk<MT, false, kLast1, true>(smem, p, c + 1, lane, h, r, acc, w, af, r1, r2, r1, r1);
    chunk<MT, false, kLast2, false>(smem, p, c + 2, lane, h, r, acc, w, af, r2, r3, r2, r2);
    chunk<MT, false, kLast3, true>(smem, p, c + 3, lane, h, r, acc, w, af, r3, r0, r3, r3);
    drain(r0, r1, r2, r3);
    wait_then_barrier<0>();  // every wave is done with the ring

    // the next tile's prologue, then this tile's epilogue
    const uint32_t cur_m0 = m0, cur_p0 = p0;
    const uint32_t Ln = L + Gd;
    const bool more = Ln < T;
    f32x4 b4[2][4];
    if constexpr (EPI != MADI_EPI_NONE) load_bias(b4, bias, np, cur_p0, wave, h);
    // the prologue is issued whether or not a tile follows (past the last
    // tile through the empty buffer: zeros, no memory access), so no branch
    // separates the asm-loaded registers from their waits
    plan(more ? Ln : L);
    if (!more) p.wq = p.ws = p.wa = p.zero;
    prologue();
    // the bias loads were issued before the prologue's loads
    if constexpr (EPI != MADI_EPI_NONE) wait_bias<4 * (G::LA + G::LW)>(b4);
    const uint32_t n = cur_p0 * kPanelRows + r * 8;
    const uint32_t rows = M - cur_m0 < 32 * MT ? M - cur_m0 : 32 * MT;
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        Cout + (size_t)cur_m0 * N, 0, (int)(rows * N * 2), 0x00020000);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      uint8_t *Ct = smem + 4 * P::kStage + (i & 1) * P::kCBuf;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t nl = (2 * wave + t) * kPanelRows;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float v[4] = {acc[t][i][g * 4 + 0], acc[t][i][g * 4 + 1], acc[t][i][g * 4 + 2],
                        acc[t][i][g * 4 + 3]};
          if constexpr (EPI != MADI_EPI_NONE) {
            v[0] += b4[t][g].x;
            v[1] += b4[t][g].y;
            v[2] += b4[t][g].z;
            v[3] += b4[t][g].w;
            if constexpr (EPI == MADI_EPI_BIAS_GELU) {
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = gelu_erf_fast(v[e]);
            }
          }
          const f16x4 o = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
          *reinterpret_cast<f16x4 *>(Ct + r * kCStride + (nl + g * 8 + h * 4) * 2) = o;
        }
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t row = wave * 8 + 2 * j + h;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(Ct + row * kCStride + r * 16);
        __builtin_amdgcn_raw_buffer_store_b128(v, cr, ((i * 32 + row) * N + n) * 2, 0, kSc1);
      }
    }
    if (!more) {
      // the empty prologue's loads (and DMAs into LDS) land before the
      // workgroup ends
      drain(r0, r1, r2, r3);
      break;
    }
    L = Ln;
  }
}

// ---------------------------------------------------------------- K split inside a workgroup
// For N = 1280 at M = 1500 with a long K (fc2, 5120 -> 1280) the 128 x 256
// tiles number only 60.  Here a workgroup owns a 128-row x 64-column tile
// (two panels) and its four waves split K four ways: wave w runs the K loop
// over chunks [w * cw, (w + 1) * cw) with the per-wave work of the 256-column
// kernel (two panels x four m-tiles per k-step, 32 MFMAs per chunk), its
// weights streaming into VGPRs as there and its own 128 A rows into a private
// two-stage LDS ring (the waves share nothing, so the K loop has no barrier).
// At the end the four partial tiles meet in LDS: wave w sums m-tile w in wave
// order (the result does not depend on timing) and runs the epilogue for it.
// 240 such tiles fill the GPU with no partial sums through memory.
namespace ks {
constexpr int kMT = 4;                    // m-tiles (of 32 rows) per tile
constexpr int kStage = kMT * 32 * 128;    // one chunk of A for 128 rows: 16 KiB
constexpr int kWaveRing = 2 * kStage;     // a wave's private ring
constexpr int kLds = kWaves * kWaveRing;  // 128 KiB
// Vector-memory issues per chunk: the weights of chunk c + 4 (units in steps
// 0, 1, 1, 2 and the two scales in step 2) and, in step 3, the 16 DMAs that
// copy chunk c + 2's A into the stage chunk c has just finished reading.
constexpr int kW = 6, kD = kMT * 4, kPer = kW + kD;
// Waits: `raw` at a chunk's start (chunk c + 1's weights, issued in chunk
// c - 3: after them that chunk's DMAs and two whole chunks), `a` before step
// 3 (chunk c + 1's A, the last issues of chunk c - 1: after them only chunk
// c's weight loads).  Chunk 0 follows a prologue whose first two virtual
// chunks issue no DMAs; the last trip issues no weights and DMAs only in its
// first two chunks.
enum Phase { kFirst0 = 0, kLive = 1, kLast0 = 2, kLast1 = 3, kLast2 = 4, kLast3 = 5 };
template <int PH>
struct Waits {
  static constexpr int raw = PH == kFirst0 ? 2 * kPer
                           : PH == kLast1  ? kD + kPer + kD
                           : PH == kLast2  ? 3 * kD
                           : PH == kLast3  ? 0
                                           : kD + 2 * kPer;
  static constexpr int a = PH >= kLast0 ? 0 : kW;
  static_assert(raw < 64 && a < 64, "vmcnt range");
};
constexpr int kPrologueWait = kW + kD;  // chunk 0's weights and A stage

struct Plan {
  desc_t wq, ws, wa;
  uint32_t w_soff[2];      // byte offset of panel t (chunk 0)
  uint32_t s_voff[2];      // this lane's scale of panel t, chunk 0
  uint32_t a_voff[kD];     // per-lane offsets of the 16 row groups, less their
                           // instruction offsets (1024 * (g & 3))
  uint32_t cb;             // the wave's first chunk
};

// The 16 DMAs of chunk c's A (8 rows each) into stage `slot`: four M0 values
// of four row groups each (instruction offsets 0 .. 3072).
__device__ inline void dma_chunk(const Plan &p, uint8_t *slot, uint32_t c) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t m0 = lds_addr(slot) + q * 4096;
    const uint32_t so = (p.cb + c) * 128;
    dma16<0, true>(p.wa, p.a_voff[4 * q + 0], so, m0);
    dma16<1024, false>(p.wa, p.a_voff[4 * q + 1], so, m0);
    dma16<2048, false>(p.wa, p.a_voff[4 * q + 2], so, m0);
    dma16<3072, false>(p.wa, p.a_voff[4 * q + 3], so, m0);
  }
}

__device__ inline void load_w(int s, RawW &w, uint32_t cw, const Plan &p, uint32_t lane) {
  const uint32_t c = p.cb + cw;
  if (s == 0) {
    vload16(w.u[0][0], p.wq, lane * 16, p.w_soff[0] + c * 2048);
  } else if (s == 1) {
    vload16<1024>(w.u[0][1], p.wq, lane * 16, p.w_soff[0] + c * 2048);
    vload16(w.u[1][0], p.wq, lane * 16, p.w_soff[1] + c * 2048);
  } else if (s == 2) {
    vload16<1024>(w.u[1][1], p.wq, lane * 16, p.w_soff[1] + c * 2048);
    vload2(w.s[0], p.ws, p.s_voff[0], c * 128);
    vload2(w.s[1], p.ws, p.s_voff[1], c * 128);
  }
}

template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Instruction order of a k-step: LDS reads, then MFMAs with the dequantisation
// between them, the step's weight loads, and in step 3 the A DMAs.
template <int S>
__device__ inline void schedule_step() {
  __builtin_amdgcn_sched_group_barrier(kSchedDSRead, kMT, 0);
#pragma unroll
  for (int i = 0; i < 2 * kMT; ++i) {
    __builtin_amdgcn_sched_group_barrier(kSchedMFMA, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedVALU, 24 / (2 * kMT) + 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedVMEM, S == 3 ? 2 : 1, 0);
  }
}

// One chunk c of the wave's range (cf. chunk() of the 256-column kernel).  `ld`
// receives chunk c + 4's weights and stage c & 1, read through step 2, receives
// chunk c + 2's A in step 3.
template <int PH>
__device__ inline void chunk(uint8_t *ring, const Plan &p, uint32_t c, uint32_t lane, uint32_t h,
                             uint32_t r, f32x16 (&acc)[2][kMT], f16x8 (&w)[2][4],
                             f16x8 (&af)[kMT], const RawW &cur, RawW &nxt, RawW &ld) {
  uint8_t *At = ring + (c & 1) * kStage;
  const uint8_t *An = ring + ((c + 1) & 1) * kStage;
  constexpr bool kLoadW = PH <= kLive;
  constexpr bool kDma = PH <= kLast1;
  wait_weights<Waits<PH>::raw>(nxt);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (s == 3) wait_vm<Waits<PH>::a>();  // chunk c + 1's A has landed in An
    __builtin_amdgcn_s_waitcnt(kLgkm0);
    f16x8 an[kMT];
    if (s < 3)
      load_a_frags<kMT>(At, s + 1, h, r, an);
    else
      load_a_frags<kMT>(An, 0, h, r, an);
#pragma unroll
    for (int i = 0; i < kMT; ++i)
      acc[0][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w[0][s], af[i], acc[0][i], 0, 0, 0);
    w[0][(s + 3) & 3] = dequant_frag(s == 0 ? cur : nxt, 0, (s + 3) & 3);
#pragma unroll
    for (int i = 0; i < kMT; ++i)
      acc[1][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w[1][s], af[i], acc[1][i], 0, 0, 0);
    w[1][(s + 3) & 3] = dequant_frag(s == 0 ? cur : nxt, 1, (s + 3) & 3);
    if constexpr (kLoadW) load_w(s, ld, c + WD, p, lane);
    // step 3's reads of At (issued in step 2) were waited for above
    if (s == 3 && kDma) dma_chunk(p, At, c + 2);
#pragma unroll
    for (int i = 0; i < kMT; ++i) af[i] = an[i];
    if (s == 3)
      schedule_step<3>();
    else
      schedule_step<0>();
    __builtin_amdgcn_sched_barrier(0);
  }
}
}  // namespace ks

template <int EPI>
__global__ __launch_bounds__(256) void q8_gemm_ks_kernel(
    const f16 *__restrict__ A, const uint8_t *__restrict__ qs, const f16 *__restrict__ sc,
    uint32_t M, uint32_t N, uint32_t K, uint32_t tiles_m, uint32_t tiles_n, uint32_t group_m,
    uint32_t cw, f16 *__restrict__ Cout, const float *__restrict__ bias) {
  using ks::kMT;
  using ks::kD;
  using ks::kStage;
  using ks::kWaveRing;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[ks::kLds];

  // tile order as in q8_gemm_kernel: XCD-contiguous runs walked in groups of
  // group_m M-tiles
  const uint32_t T = tiles_m * tiles_n;
  const uint32_t bid_x = blockIdx.x;
  const uint32_t remap = 0u - (uint32_t)((T & 7) == 0);
  const uint32_t bid = (((bid_x & 7) * (T >> 3) + (bid_x >> 3)) & remap) | (bid_x & ~remap);
  const uint32_t per_group = group_m * tiles_n;
  const uint32_t gi = bid / per_group, first_m = gi * group_m;
  const uint32_t gm = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
  const uint32_t tm = first_m + (bid % per_group) % gm;
  const uint32_t tn = (bid % per_group) / gm;

  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t h = lane >> 5, r = lane & 31;
  const uint32_t m0 = tm * 32 * kMT, p0 = tn * 2;

  ks::Plan p;
  p.wq = make_desc(qs, N * K);
  p.ws = make_desc(sc, N * K / 16);
  p.wa = make_desc(A, M * K * 2);
  p.cb = wave * cw;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    // N % 64 == 0: both panels exist.  The chunk (the wave's base p.cb plus
    // its own index) enters as the SGPR offset of every load.
    const uint32_t pp = p0 + t;
    p.w_soff[t] = pp * kPanelRows * K;
    p.s_voff[t] = pp * K * 2 + lane * 2;
  }
#pragma unroll
  for (int g = 0; g < kD; ++g) {
    const uint32_t row = g * 8 + (lane >> 3);
    const uint32_t q = (lane & 7) ^ a_swz(row);
    uint32_t m = m0 + row;
    m = m < M ? m : M - 1;
    // row group g starts 8g rows, at least 1024 (g & 3) bytes, into A
    p.a_voff[g] = m * K * 2 + q * 16 - 1024 * (g & 3);
  }
  uint8_t *ring = smem + wave * kWaveRing;

  f32x16 acc[2][kMT];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < kMT; ++i) acc[t][i] = (f32x16){};

  // prologue: virtual chunks -4 .. -1 issue the weights of chunks 0 .. 3, the
  // last two also the A of chunks 0 and 1 (stages 0 and 1)
  RawW r0, r1, r2, r3;
#pragma unroll
  for (int s = 0; s < 3; ++s) ks::load_w(s, r0, 0, p, lane);
#pragma unroll
  for (int s = 0; s < 3; ++s) ks::load_w(s, r1, 1, p, lane);
#pragma unroll
  for (int s = 0; s < 3; ++s) ks::load_w(s, r2, 2, p, lane);
  ks::dma_chunk(p, ring, 0);
#pragma unroll
  for (int s = 0; s < 3; ++s) ks::load_w(s, r3, 3, p, lane);
  ks::dma_chunk(p, ring + kStage, 1);
  ks::wait_vm<ks::kPrologueWait>();
  wait_weights<ks::kPrologueWait>(r0);
  f16x8 w[2][4], af[kMT];
#pragma unroll
  for (int s = 0; s < 3; ++s) w[0][s] = dequant_frag(r0, 0, s);
#pragma unroll
  for (int s = 0; s < 3; ++s) w[1][s] = dequant_frag(r0, 1, s);
  load_a_frags<kMT>(ring, 0, h, r, af);

  // first trip (chunk 0 follows the prologue), at least one live trip, last trip
  ks::chunk<ks::kFirst0>(ring, p, 0, lane, h, r, acc, w, af, r0, r1, r0);
  ks::chunk<ks::kLive>(ring, p, 1, lane, h, r, acc, w, af, r1, r2, r1);
  ks::chunk<ks::kLive>(ring, p, 2, lane, h, r, acc, w, af, r2, r3, r2);
  ks::chunk<ks::kLive>(ring, p, 3, lane, h, r, acc, w, af, r3, r0, r3);
  uint32_t c = 4;
  do {
    ks::chunk<ks::kLive>(ring, p, c + 0, lane, h, r, acc, w, af, r0, r1, r0);
    ks::chunk<ks::kLive>(ring, p, c + 1, lane, h, r, acc, w, af, r1, r2, r1);
    ks::chunk<ks::kLive>(ring, p, c + 2, lane, h, r, acc, w, af, r2, r3, r2);
    ks::chunk<ks::kLive>(ring, p, c + 3, lane, h, r, acc, w, af, r3, r0, r3);
    c += 4;
  } while (c + 2 * WD <= cw);
  ks::chunk<ks::kLast0>(ring, p, c + 0, lane, h, r, acc, w, af, r0, r1, r0);
  ks::chunk<ks::kLast1>(ring, p, c + 1, lane, h, r, acc, w, af, r1, r2, r1);
  ks::chunk<ks::kLast2>(ring, p, c + 2, lane, h, r, acc, w, af, r2, r3, r2);
  ks::chunk<ks::kLast3>(ring, p, c + 3, lane, h, r, acc, w, af, r3, r0, r3);
  drain(r0, r1, r2, r3);

  // ---- the four partial tiles meet: each wave hands the m-tiles it does not
  // own to their owners through LDS (16-byte groups in register order, so each
  // lane reads back what the same lane of the other wave wrote), then wave w
  // adds the partials of m-tile w in wave order 0..3, its own from registers.
  wait_then_barrier<0>();  // every wave is done with its ring
  float *part = reinterpret_cast<float *>(smem);
  auto slot = [&](uint32_t src, uint32_t i, int t, int g) {
    return part + ((((src * kMT + i) * 2 + t) * 4 + g) * 64 + lane) * 4;
  };
#pragma unroll
  for (int i = 0; i < kMT; ++i) {
    if ((uint32_t)i == wave) continue;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4 *>(slot(wave, i, t, g)) =
            (f32x4){acc[t][i][4 * g], acc[t][i][4 * g + 1], acc[t][i][4 * g + 2], acc[t][i][4 * g + 3]};
  }
  __syncthreads();
  f32x16 fin[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    // the wave's own m-tile is index `wave`: select it from registers
    f32x16 own = acc[t][0];
#pragma unroll
    for (int i = 1; i < kMT; ++i)
      if ((uint32_t)i == wave) own = acc[t][i];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (uint32_t src = 0; src < (uint32_t)kWaves; ++src) {
        const f32x4 o = {own[4 * g], own[4 * g + 1], own[4 * g + 2], own[4 * g + 3]};
        const f32x4 v = src == wave ? o : *reinterpret_cast<const f32x4 *>(slot(src, wave, t, g));
        sum = src == 0 ? v : sum + v;
      }
      fin[t][4 * g] = sum.x;
      fin[t][4 * g + 1] = sum.y;
      fin[t][4 * g + 2] = sum.z;
      fin[t][4 * g + 3] = sum.w;
    }
  }
  __syncthreads();  // partials read: the LDS becomes the output staging

  // ---- epilogue of m-tile `wave`: bias / GELU, one rounding to f16, the
  // 32 x 64 block transposed through the wave's own LDS region, stored as
  // 128-byte row segments (lane l: row l/8 + 8j, columns 8 (l % 8) ..)
  constexpr uint32_t kPitch = 64 * 2 + 16;
  uint8_t *Ct = smem + wave * 32 * kPitch;
  const uint32_t rows = M - m0 < 32 * kMT ? M - m0 : 32 * kMT;
  const __amdgpu_buffer_rsrc_t cr =
      __builtin_amdgcn_make_buffer_rsrc(Cout + (size_t)m0 * N, 0, (int)(rows * N * 2), 0x00020000);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float v[4] = {fin[t][4 * g], fin[t][4 * g + 1], fin[t][4 * g + 2], fin[t][4 * g + 3]};
      if constexpr (EPI != MADI_EPI_NONE) {
        const f32x4 b = *reinterpret_cast<const f32x4 *>(bias + (p0 + t) * kPanelRows + g * 8 + h * 4);
        v[0] += b.x;
        v[1] += b.y;
        v[2] += b.z;
        v[3] += b.w;
        if constexpr (EPI == MADI_EPI_BIAS_GELU) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = gelu_erf_fast(v[e]);
        }
      }
      const f16x4 o = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
      *reinterpret_cast<f16x4 *>(Ct + r * kPitch + (32 * t + g * 8 + h * 4) * 2) = o;
    }
  }
  const uint32_t n = p0 * kPanelRows + (lane & 7) * 8;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t row = (lane >> 3) + 8 * j;
    const u32x4 v = *reinterpret_cast<const u32x4 *>(Ct + row * kPitch + (lane & 7) * 16);
    __builtin_amdgcn_raw_buffer_store_b128(v, cr, ((wave * 32 + row) * N + n) * 2, 0, kSc1);
  }
}

// The persistent tile loop serves shapes with at least two rounds of 128 x 256
// tiles, whole 256-column groups and a K of 12 to 32 chunks in fours.
// Measured at M = 24000 (cold clock, first of repeated runs): fc1 337 -> 317
// us, fc1 + bias + GELU 390 -> 371 us; fc2 (K = 5120, 80 chunks per tile,
// where a tile's fixed costs are a small share) 306 -> 310 us, so long K
// keeps one workgroup per tile.
#ifndef MADI_GEMM_PERSIST
#define MADI_GEMM_PERSIST 1
#endif
bool persist_ok(uint32_t M, uint32_t N, uint32_t K) {
  const uint32_t chunks = K / kChunkK, cus = (uint32_t)cu_count();
  return MADI_GEMM_PERSIST && N % 256 == 0 && chunks % 4 == 0 && chunks >= 12 && chunks <= 32 &&
         cus >= 8 &&
         (M + 127) / 128 * (N / 256) >= 2 * cus;
}

template <int EPI>
int launch_persist(const f16 *A, const uint8_t *qs, const f16 *sc, f16 *C, const float *bias,
                   uint32_t M, uint32_t N, uint32_t K) {
  const uint32_t tiles_m = (M + 127) / 128, tiles_n = N / 256;
  const uint32_t group_m = tiles_m < 6 ? tiles_m : 6;
  const uint32_t grid = (uint32_t)cu_count() / 8 * 8;  // one workgroup per CU, a multiple of 8
  hipLaunchKernelGGL((q8_gemm_persist_kernel<EPI>), dim3(grid), dim3(kWaves * 64), 0, stream(),
                     A, qs, sc, M, N, K, tiles_m, tiles_n, group_m, C, bias);
  return check_launch("madi_q8_gemm");
}

// The per-wave chunk count of the in-workgroup K split, 0 when the shape does
// not suit it: N a multiple of 64, K a multiple of 1024 with at least 12
// chunks per wave (a first, a middle and a last trip of four), and 128 x 64
// tiles that fill at least three quarters of the CUs in one round.  Each
// wave streams its own A rows, four times the A traffic from L2 of the
// 256-column tiles, so it only pays where those would split K through
// memory: fc2 at M = 1500 (240 tiles) 29.3-29.6 -> 26.5-27.5 us with cold
// weights; two rounds (N = 2048, K = 4096: 320 tiles) were slower (42.9 vs
// 36.4 us), 160 tiles even (24.6 vs 24.7).
#ifndef MADI_GEMM_KSPLIT
#define MADI_GEMM_KSPLIT 1
#endif
uint32_t ks_chunks(uint32_t M, uint32_t N, uint32_t K) {
  if (!MADI_GEMM_KSPLIT || N % 64 || K % 1024 || K / 256 < 12) return 0;
  const uint32_t tiles = (M + 127) / 128 * (N / 64), cus = (uint32_t)cu_count();
  return tiles * 4 >= cus * 3 && tiles <= cus ? K / 256 : 0;
}

template <int EPI>
int launch_ks(const f16 *A, const uint8_t *qs, const f16 *sc, f16 *C, const float *bias,
              uint32_t M, uint32_t N, uint32_t K, uint32_t cw) {
  const uint32_t tiles_m = (M + 127) / 128, tiles_n = N / 64;
  const uint32_t group_m = tiles_m < 6 ? tiles_m : 6;
  hipLaunchKernelGGL((q8_gemm_ks_kernel<EPI>), dim3(tiles_m * tiles_n), dim3(kWaves * 64), 0,
                     stream(), A, qs, sc, M, N, K, tiles_m, tiles_n, group_m, cw, C, bias);
  return check_launch("madi_q8_gemm");
}

// Too few tiles to fill the GPU and a long K (fc2 at M = 1500 with 64-row
// tiles: 120 tiles, 80 chunks): split K over up to four workgroups per tile,
// >= 16 chunks each.  The partial sums travel through memory (about 1 us per
// MB of partials), which only pays off when each split keeps a long K range.
uint32_t split_count(uint32_t tiles, uint32_t chunks) {
  if (tiles >= 160 || chunks < 64) return 1;
  uint32_t splits = 240 / tiles;
  if (splits > kMaxSplits) splits = kMaxSplits;
  if (splits > chunks / 16) splits = chunks / 16;
  return splits < 1 ? 1 : splits;
}

// Whether a K loop of `chunks` chunks split `splits` ways needs the padded
// kernel: every split's chunk count must be a multiple of WD and at least
// 2*WD for the select-free loop (split s covers chunks / splits chunks, one
// more for the first chunks % splits splits).
bool loop_padded(uint32_t chunks, uint32_t splits) {
  const uint32_t cper = chunks / splits, crem = chunks % splits;
  for (const uint32_t n : {cper, cper + 1}) {
    if (n == cper + 1 && crem == 0) continue;
    if (n % WD || n < 2 * WD) return true;
  }
  return false;
}

uint32_t tile_count(uint32_t M, uint32_t N, uint32_t MT, uint32_t PW = 2) {
  return (M + 32 * MT - 1) / (32 * MT) * ((N + 128 * PW - 1) / (128 * PW));
}

// 128-column tiles take unpadded K loops only (a multiple of four chunks, at
// least eight); MADI_GEMM_NARROW=0 keeps 256-column tiles everywhere.
bool narrow_ok(uint32_t K) {
  const uint32_t chunks = K / kChunkK;
  const char *e = getenv("MADI_GEMM_NARROW");
  return chunks % 4 == 0 && chunks >= 8 && !(e && e[0] == '0');
}

// ---- fixed scratch for the allocation-free entry point.  A K split's
// partial sums and arrival counters live in this device array instead of
// the library's growable workspace: kScratchCounters counters (zero whenever
// no kernel is using them: every split tile's last workgroup resets its
// own), then the partials.  A split happens only below 160 tiles and only at
// 32- or 64-row tiles, and splits * tiles <= 240, so the partials of any
// split shape take at most 240 * 64 KiB = 15 MiB.
constexpr size_t kScratchBytes = size_t(16) << 20;
constexpr size_t kScratchCounters = 1024;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Device address of `scratch` per device.  In host code the array's name is
// only a host-side stand-in, so the kernels take this address instead,
// resolved with hipGetSymbolAddress once per device, with that device current.
constexpr int kMaxDevices = 64;
uint8_t *g_scratch[kMaxDevices];

__global__ void zero_counters_kernel(uint32_t *cnt, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) cnt[i] = 0;
}

// Resolves the current device's scratch address (once) and clears its
// counters.  Runs in madi_init, before any caller can be capturing a graph.
int resolve_scratch(uint8_t **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MADI_ERR_INIT, "scratch: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MADI_ERR_INIT, "scratch: device %d out of range", dev);
  if (!g_scratch[dev]) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(MADI_ERR_INIT, "scratch: hipGetSymbolAddress: %s", hipGetErrorString(e));
    hipLaunchKernelGGL(zero_counters_kernel, dim3(kScratchCounters / 256), dim3(256), 0, nullptr,
                       static_cast<uint32_t *>(ptr), (uint32_t)kScratchCounters);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess)
      return fail(MADI_ERR_INIT, "scratch: clearing the counters: %s", hipGetErrorString(e));
    g_scratch[dev] = static_cast<uint8_t *>(ptr);
  }
  *out = g_scratch[dev];
  return MADI_OK;
}

// The m-tile-major tail serves unpadded, unsplit f16 launches of two or more
// m-tiles (MADI_GEMM_TAIL=0 selects the chunk-by-chunk last trip instead).
bool use_tail(uint32_t splits, uint32_t chunks) {
  const char *e = getenv("MADI_GEMM_TAIL");
  // the ramped first trip, then at least one steady trip, then the tail
  return splits == 1 && chunks >= 12 && !(e && e[0] == '0');
}

// Where a launch keeps its split-K partials and counters.
enum Scratch { kWorkspace = 0, kStatic = 1 };

template <int MT, int EPI, bool F32 = false, int PW = 2>
int launch_gemm(const void *A, const uint8_t *qs, const f16 *sc, void *C, const float *bias,
                uint32_t M, uint32_t N, uint32_t K, Scratch where, const OutSeg &seg = OutSeg{}) {
  const uint32_t tiles_m = (M + 32 * MT - 1) / (32 * MT);
  const uint32_t tiles_n = (N + 128 * PW - 1) / (128 * PW);
  const uint32_t T = tiles_m * tiles_n, chunks = K / kChunkK;
  const uint32_t splits = split_count(T, chunks);
  // segments: unsplit launches whose tiles do not straddle a segment boundary
  if (seg.n && (splits != 1 || seg.n % (128 * PW) != 0)) return kSegUnsupported;
  float *ws = nullptr;
  uint32_t *cnt = nullptr;
  if (splits > 1) {
    const size_t part = (size_t)T * splits * (4 * PW * MT * 4 * 64 * 16);
    if (where == kStatic) {
      if (T > kScratchCounters || part > kScratchBytes - kScratchCounters * 4)
        return fail(MADI_ERR_SHAPE,
                    "madi_q8_gemm_noalloc: m=%u n=%u k=%u needs %zu bytes of split-K scratch, "
                    "more than the %zu the library holds", M, N, K,
                    part + kScratchCounters * 4, kScratchBytes);
      uint8_t *base = nullptr;
      if (int rc = resolve_scratch(&base)) return rc;
      cnt = reinterpret_cast<uint32_t *>(base);
      ws = reinterpret_cast<float *>(base + kScratchCounters * 4);
    } else {
      const int rc = workspace(part, T, &ws, &cnt);
      if (rc != MADI_OK) return rc;
    }
  }
  // split s covers cper + (s < crem) chunks
  const uint32_t cper = chunks / splits, crem = chunks % splits;
  const bool padded = loop_padded(chunks, splits);
  // one workgroup per (tile, split), the grid rounded up to a multiple of 8
  // (the kernel's XCD mapping)
  const auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3((T * splits + 7) & ~7u), dim3(kWaves * 64), 0, stream(), A, qs,
                       sc, M, N, K, tiles_m, tiles_n, splits, cper, crem, C, bias, ws, cnt, seg);
  };
  if constexpr (PW == 1) {
    // 128-column tiles: the host chooses them only for unpadded K loops, and
    // for the f16 GEMM only unsplit
    if (padded || (!F32 && splits != 1))
      return fail(MADI_ERR_SHAPE, "%s: 128-column tiles need an unpadded%s K loop",
                  F32 ? "madi_q8_pproj" : "madi_q8_gemm", F32 ? "" : ", unsplit");
    go(q8_gemm_kernel<MT, EPI, false, F32, false, 1>);
  } else if (padded)
    go(q8_gemm_kernel<MT, EPI, true, F32>);
  else if constexpr (!F32 && MT >= 2) {
    if (use_tail(splits, chunks))
      go(q8_gemm_kernel<MT, EPI, false, false, true>);
    else
      go(q8_gemm_kernel<MT, EPI, false, false>);
  } else
    go(q8_gemm_kernel<MT, EPI, false, F32>);
  return check_launch(F32 ? "madi_q8_pproj" : "madi_q8_gemm");
}

template <int MT, int PW = 2>
int dispatch_epi(int epi, const f16 *A, const uint8_t *qs, const f16 *sc, f16 *C,
                 const float *bias, uint32_t M, uint32_t N, uint32_t K, Scratch where,
                 const OutSeg &seg) {
  switch (epi) {
  case MADI_EPI_NONE:
    return launch_gemm<MT, MADI_EPI_NONE, false, PW>(A, qs, sc, C, bias, M, N, K, where, seg);
  case MADI_EPI_BIAS:
    return launch_gemm<MT, MADI_EPI_BIAS, false, PW>(A, qs, sc, C, bias, M, N, K, where, seg);
  case MADI_EPI_BIAS_GELU:
    return launch_gemm<MT, MADI_EPI_BIAS_GELU, false, PW>(A, qs, sc, C, bias, M, N, K, where, seg);
  default: return fail(MADI_ERR_ARG, "madi_q8_gemm: unknown epilogue %d", epi);
  }
}

int q8_gemm(const char *what, const void *a, const void *qs, const void *scales, void *c,
            const float *bias, uint32_t m, uint32_t n, uint32_t k, int epilogue, Scratch where,
            const OutSeg &seg = OutSeg{}) {
  if (!a || !qs || !scales || !c) return fail(MADI_ERR_NULL, "%s: null pointer", what);
  if (epilogue != MADI_EPI_NONE && !bias) return fail(MADI_ERR_NULL, "%s: null bias", what);
  if (epilogue == MADI_EPI_BIAS_RES)
    return fail(MADI_ERR_ARG, "%s: the residual epilogue exists for the GEMV only", what);
  if (m == 0 || n == 0 || k == 0 || n % kPanelRows || k % kChunkK)
    return fail(MADI_ERR_SHAPE, "%s: m=%u n=%u k=%u (need n %% 32 == 0, k %% 64 == 0)", what, m, n, k);
  // buffer offsets are 32-bit (and buffer sizes below 2 GiB): the operands
  // A (m*k*2 bytes) and W (n*k bytes) and one 128-row C tile (256*n bytes)
  // must stay below 2 GiB
  if ((uint64_t)m * k * 2 >= (1ull << 31) || (uint64_t)n * k >= (1ull << 31) ||
      (uint64_t)n * 256 >= (1ull << 31))
    return fail(MADI_ERR_SHAPE, "%s: m=%u n=%u k=%u exceeds the 2 GiB operand limit", what, m, n, k);
  if (!aligned(a, 16) || !aligned(qs, 16) || !aligned(scales, 16) || !aligned(c, 16) ||
      (bias && !aligned(bias, 16)))
    return fail(MADI_ERR_ALIGN, "%s: a/qs/scales/c/bias need 16-byte alignment", what);
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "%s: madi_init has not succeeded", what);
  if (int rc = deferred_before_read(a, (size_t)m * k * 2)) return rc;
  if (seg.n == 0) {
    if (int rc = deferred_before_write(c, (size_t)m * n * 2)) return rc;
  } else {
    for (int s = 0; s < kMaxSegs && s * seg.n < n; ++s)
      if (int rc = deferred_before_write(seg.c[s], (size_t)m * seg.n * 2)) return rc;
  }
  const f16 *A = static_cast<const f16 *>(a);
  const uint8_t *Q = static_cast<const uint8_t *>(qs);
  const f16 *S = static_cast<const f16 *>(scales);
  f16 *C = static_cast<f16 *>(c);
  if (m <= 32) return dispatch_epi<1>(epilogue, A, Q, S, C, bias, m, n, k, where, seg);
  if (m <= 64) return dispatch_epi<2>(epilogue, A, Q, S, C, bias, m, n, k, where, seg);
  // Where 128-row tiles would split K: the in-workgroup K split on 128 x 64
  // tiles where the shape suits it (fc2 at M = 1500), else 64-row tiles, which
  // halve the split count and the partial sums through memory (2 splits of
  // 40 chunks instead of 4 of 20).
  if (split_count(tile_count(m, n, 4), k / kChunkK) > 1) {
    if (seg.n) return kSegUnsupported;
    if (const uint32_t cw = ks_chunks(m, n, k)) {
      switch (epilogue) {
      case MADI_EPI_NONE: return launch_ks<MADI_EPI_NONE>(A, Q, S, C, bias, m, n, k, cw);
      case MADI_EPI_BIAS: return launch_ks<MADI_EPI_BIAS>(A, Q, S, C, bias, m, n, k, cw);
      case MADI_EPI_BIAS_GELU: return launch_ks<MADI_EPI_BIAS_GELU>(A, Q, S, C, bias, m, n, k, cw);
      default: return fail(MADI_ERR_ARG, "%s: unknown epilogue %d", what, epilogue);
      }
    }
    return dispatch_epi<kSplitTile>(epilogue, A, Q, S, C, bias, m, n, k, where, seg);
  }
  // Otherwise the lowest tiles whose count still fits one workgroup per CU:
  // a lower tile does less MFMA work per byte loaded (a 32-row tile takes
  // ~0.9x the time of a 64-row one for half the work) but spreads over more
  // CUs.  At M = 1500: out 1280->1280 60 -> 235 tiles (16.8 -> 11.3 us),
  // cross K,V 1280->2560 120 -> 240 tiles (18.2 -> 13.9 us); q,k,v
  // 1280->3840 (180 tiles) and fc1 (240) keep 128 rows.
  const uint32_t cus = (uint32_t)cu_count();
  // Where that tile would be 32 or 64 rows, a twice-as-tall tile of 128
  // columns (four waves of one panel each) keeps the tile count and halves
  // the dequantisation per MFMA (it scales as 1 / tile height): out-proj
  // 1280 -> 1280 at M = 1500 runs 64 x 128 tiles, cross K|V 1280 -> 2560
  // 128 x 128 tiles.  K loops that are padded stay with 256-column tiles.
  const bool narrow = narrow_ok(k);
  if (tile_count(m, n, 1) <= cus) {
    if (narrow && tile_count(m, n, 2, 1) <= cus)
      return dispatch_epi<2, 1>(epilogue, A, Q, S, C, bias, m, n, k, where, seg);
    return dispatch_epi<1>(epilogue, A, Q, S, C, bias, m, n, k, where, seg);
  }
  if (tile_count(m, n, 2) <= cus) {
    if (narrow && tile_count(m, n, 4, 1) <= cus)
      return dispatch_epi<4, 1>(epilogue, A, Q, S, C, bias, m, n, k, where, seg);
    return dispatch_epi<2>(epilogue, A, Q, S, C, bias, m, n, k, where, seg);
  }
  if (tile_count(m, n, 3) <= cus)
    return dispatch_epi<3>(epilogue, A, Q, S, C, bias, m, n, k, where, seg);
  if (seg.n) return kSegUnsupported;
  // at least two rounds of 128-row tiles: the persistent tile loop
  if (persist_ok(m, n, k)) {
    switch (epilogue) {
    case MADI_EPI_NONE: return launch_persist<MADI_EPI_NONE>(A, Q, S, C, bias, m, n, k);
    case MADI_EPI_BIAS: return launch_persist<MADI_EPI_BIAS>(A, Q, S, C, bias, m, n, k);
    case MADI_EPI_BIAS_GELU: return launch_persist<MADI_EPI_BIAS_GELU>(A, Q, S, C, bias, m, n, k);
    default: return fail(MADI_ERR_ARG, "%s: unknown epilogue %d", what, epilogue);
    }
  }
  return dispatch_epi<4>(epilogue, A, Q, S, C, bias, m, n, k, where, seg);
}

}  // namespace

namespace madi {
// madi_init: the current device's scratch address, resolved at set-up.
int gemm_scratch_init() {
  uint8_t *base = nullptr;
  return resolve_scratch(&base);
}

// out[M][N] (f32) = f16(in[M][K] (f32)) . deq(W)^T through the MFMA GEMM
// (the batched projection for many rows): 32- or 64-row tiles by the same
// rule as the f16 GEMM, replaced by 128-column tiles where their K loop is
// unpadded: where a 32-row tile would be chosen, 32 x 128 tiles if they fit
// one per CU (twice the workgroups, each with half the work: M = 320
// 1280 -> 2560 8.1 us against 10.1 on 64 x 128 tiles), else 64 x 128 tiles
// (the same tile count as 32 x 256, half the dequantisation per MFMA); and
// where K is split over workgroups, 64 x 128 tiles if they keep the split
// count (FFN down 5120 -> 1280 at M = 320 runs 200 workgroups instead of
// 100).  The caller has checked the shapes (N % 32 == 0, K % 64 == 0,
// 16-byte aligned in and out, operands below 2 GiB).
int q8_gemm_f32io(const float *in, const void *qs, const void *scales, float *out, uint32_t m,
                  uint32_t n, uint32_t k) {
  const uint8_t *Q = static_cast<const uint8_t *>(qs);
  const f16 *S = static_cast<const f16 *>(scales);
  const uint32_t cus = (uint32_t)cu_count();
  if (m <= 32 || (tile_count(m, n, 1) <= cus && split_count(tile_count(m, n, 4), k / kChunkK) == 1)) {
    if (narrow_ok(k) && tile_count(m, n, 1, 1) <= cus &&
        split_count(tile_count(m, n, 1, 1), k / kChunkK) == 1)
      return launch_gemm<1, MADI_EPI_NONE, true, 1>(in, Q, S, out, nullptr, m, n, k, kWorkspace);
    if (m > 32 && narrow_ok(k) && tile_count(m, n, 2, 1) <= cus &&
        split_count(tile_count(m, n, 2, 1), k / kChunkK) == 1)
      return launch_gemm<2, MADI_EPI_NONE, true, 1>(in, Q, S, out, nullptr, m, n, k, kWorkspace);
    return launch_gemm<1, MADI_EPI_NONE, true>(in, Q, S, out, nullptr, m, n, k, kWorkspace);
  }
  const uint32_t chunks = k / kChunkK, wide = tile_count(m, n, 2), narrow = tile_count(m, n, 2, 1);
  const uint32_t splits = split_count(narrow, chunks);
  if (narrow_ok(k) && splits > 1 && splits == split_count(wide, chunks) && narrow * splits <= cus &&
      !loop_padded(chunks, splits))
    return launch_gemm<2, MADI_EPI_NONE, true, 1>(in, Q, S, out, nullptr, m, n, k, kWorkspace);
  return launch_gemm<2, MADI_EPI_NONE, true>(in, Q, S, out, nullptr, m, n, k, kWorkspace);
}
}  // namespace madi

namespace madi {
int q8_gemm_seg(const void *a, const void *qs, const void *scales, const OutSeg &seg, uint32_t m,
                uint32_t n, uint32_t k, int epilogue) {
  // every segment's output and bias meets madi_q8_gemm's own checks; the
  // launch checks below are then made on segment 0's pointers
  if (seg.n == 0 || n % seg.n || n / seg.n > (uint32_t)kMaxSegs) return kSegUnsupported;
  for (uint32_t s = 0; s < n / seg.n; ++s)
    if (!seg.c[s] || !aligned(seg.c[s], 16) || (epilogue != MADI_EPI_NONE && (!seg.b[s] || !aligned(seg.b[s], 16))))
      return kSegUnsupported;
  return q8_gemm("madi_q8_gemm", a, qs, scales, seg.c[0], epilogue != MADI_EPI_NONE ? seg.b[0] : nullptr,
                 m, n, k, epilogue, kWorkspace, seg);
}
}  // namespace madi

extern "C" int madi_q8_gemm(const void *a, const void *qs, const void *scales, void *c,
                            const float *bias, uint32_t m, uint32_t n, uint32_t k, int epilogue) {
  return q8_gemm("madi_q8_gemm", a, qs, scales, c, bias, m, n, k, epilogue, kWorkspace);
}

extern "C" int madi_q8_gemm_noalloc(const void *a, const void *qs, const void *scales, void *c,
                                    const float *bias, uint32_t m, uint32_t n, uint32_t k,
                                    int epilogue) {
  return q8_gemm("madi_q8_gemm_noalloc", a, qs, scales, c, bias, m, n, k, epilogue, kStatic);
}
