// attn.hip -- encoder self-attention over the Q/K/V projections, the consumer
// of the encoder's projection GEMMs: replaces m4_flash_enc
// (engine/metal/kernels/m4_gemm.metal:268-407), which kFlash dispatches once
// per 30 s window (engine/metal/encoder.zig:138-152, called at :281-283).
//
// Arithmetic, as the reference's: S = Q K^T in f32 from f16 operands, scaled
// by 1/8; an online softmax over 64-key blocks against a running row max;
// P = f16(e); O += P V in f32; out = f16(O / (sum + 1e-6)).  Three changes
// that move only roundings: e is the hardware exp2 of s * log2(e)/8 - m'; the
// reference max m' is raised only when a block's max passes it by more than 8
// (log2 units), so e <= 256 (well inside f16, each P still rounded relative to
// its own magnitude) and O and the sum are rescaled in a few blocks instead of
// in every block; and the sum adds the rounded P (v_dot2_f32_f16, half the
// instructions of adding the f32 e), so out is a weighted mean of the V rows
// with exactly the weights the product used.
//
// Layout: q, k, v, out f16 [seq][nh*64], head hd in columns 64hd..64hd+63 (the
// projection GEMMs' output, unpadded: rows past seq are never read -- row
// indices clamp to the last row, and the keys past seq get weight 0).
//
// Workgroup: 128 query rows of one head.  A key group of 4 waves walks a
// range of the keys; wave w owns query rows 32w..32w+31 (the MFMA's 32
// columns).  KS key groups (KS waves per SIMD) split the key range and merge
// their partial (m', sum, O) in LDS at the end; the default is four, whose
// waves overlap each other's matrix and vector work.  Per 64-key block a
// wave computes
//   S^T = K Q^T: two v_mfma_f32_32x32x16_f16 tiles with the keys as rows, so
//     lane (h, r) holds query r's scores of keys 32t + 8j + 4h + i
//     (s[t][4j + i]): row max and sum are in-lane plus one exchange between
//     the lane halves;
//   O^T += V^T P^T: two tiles with d as rows; P^T comes straight from the S^T
//     registers as the B operand (k slot 8h + 4jj + i of MFMA (t, a) is key
//     32t + 16a + 8jj + 4h + i), and V^T from the untransposed V tile through
//     the LDS transpose read (ds_read_b64_tr_b16: 16 lanes pass 4 rows x 16
//     columns of f16, lane c receives column c), which gives each lane one d
//     and four consecutive keys.
// The K and V tiles of a block (64 rows x 128 bytes each) arrive by LDS DMA in
// a ring per key group, one barrier per block; the 16-byte pieces of each row
// are XOR-swizzled so that the K fragment reads (32 rows, one piece each) and
// the transpose reads (8 rows x 64 bytes) spread over all banks.  Two
// schedules: the plain one (three or four key groups: S at the start of each
// block, a 3- or 2-stage ring), and a pipelined one for one or two groups
// (the next block's S on the matrix cores during this block's softmax, the
// exponentials of each group of 8 scores feeding two P V products with two
// S products between them; a 4-stage ring, three blocks ahead).
#include "common.h"
#include "vmem.h"

using namespace madi;

namespace {

constexpr int kQRows = 128;                        // query rows per workgroup
constexpr int kTileBytes = 64 * 64 * 2;            // one K or V tile: 64 keys x 64 d
constexpr int kStageBytes = 2 * kTileBytes;        // K tile, then V tile
// Ring stages per key group: four for the pipelined schedule (blocks j+1
// and j+2 resident and j+3 in flight while block j computes), three or two
// for the plain schedule of three or four key groups (blocks j+1, j+2 or
// only j+1 in flight), which must fit 160 KiB of LDS for all groups.
template <int KS, bool PIPE>
constexpr int kStages = PIPE ? 4 : (KS >= 4 ? 2 : 3);
template <int KS, bool PIPE>
constexpr int kRingBytes = kStages<KS, PIPE> * kStageBytes;  // per key group
constexpr float kScaleLog2 = 0.125f * 1.4426950408889634f;  // 1/8 * log2(e)
constexpr float kLazy = 8.0f;  // raise the reference max when exceeded by more than this
// sched_group_barrier masks
constexpr int kSchedMFMA = 0x008;
constexpr int kSchedDSRead = 0x100;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;

// piece swizzles: K rows (fragment reads of 32 rows at one piece), V rows
// (transpose reads of 4 consecutive rows x 4 pieces per half-wave)
__device__ inline uint32_t swz_k(uint32_t row) { return (row >> 1) & 7; }
__device__ inline uint32_t swz_v(uint32_t row) { return ((row >> 1) & 1) << 2; }

__device__ inline f16x8 lds_read16(uint32_t addr) {
  return __builtin_bit_cast(f16x8, *(const lds_u32x4 *)(uintptr_t)addr);
}
__device__ inline f16x4 lds_read_tr(uint32_t addr) {
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(uintptr_t)addr));
}

// Wait for the Q fragments and every DMA issued so far, then meet the other
// waves; the fragments are operands, so no use of them is scheduled before
// the wait.
__device__ inline void wait_q_then_barrier(u32x4 (&qf)[4]) {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier"
               : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3])
               :
               : "memory");
}

// Grid: one workgroup per (head, 128-row query tile), 256 * KS threads: KS
// key groups of four waves.  PIPE: the next block's S during this block's
// softmax (two key groups, two waves per SIMD); otherwise S at the start of
// each block and the three or four waves per SIMD overlap each other.
template <int KS, bool PIPE>
__global__ __launch_bounds__(256 * KS) void flash_enc_kernel(
    f16 *__restrict__ out, const f16 *__restrict__ q, const f16 *__restrict__ k,
    const f16 *__restrict__ v, uint32_t seq, uint32_t nh, uint32_t qtiles) {
  constexpr int NS = kStages<KS, PIPE>;
  constexpr int RB = kRingBytes<KS, PIPE>;
  static_assert(KS * RB <= 160 * 1024, "LDS");
  static_assert((KS - 1) * 4 * 34 * 64 * 4 <= KS * RB, "exchange area");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[KS * RB];
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = sgpr(threadIdx.x >> 6);
  const uint32_t grp = wave >> 2, wq = wave & 3;
  const uint32_t h = lane >> 5, r = lane & 31;

  // Workgroups x and x + 8 run on the same XCD (round-robin dispatch): each
  // XCD takes a contiguous run of (head, query tile) items, heads outermost,
  // so a head's K and V rows are fetched into one or two L2s.
  const uint32_t items = nh * qtiles, b = blockIdx.x, x = b & 7;
  const uint32_t per = items >> 3, extra = items & 7;
  const uint32_t item = x * per + (x < extra ? x : extra) + (b >> 3);
  const uint32_t head = item / qtiles, qt = item - head * qtiles;

  const uint32_t rowb = nh * 128;  // bytes per sequence row
  const uint32_t bytes = seq * rowb;
  const desc_t dq = make_desc(q, bytes), dk = make_desc(k, bytes), dv = make_desc(v, bytes);

  // Q^T fragments (B operand of S^T): query row q0 + r, d = 16s + 8h .. +7
  const uint32_t q0 = qt * kQRows + wq * 32;
  const uint32_t qrow = min(q0 + r, seq - 1);
  u32x4 qf[4];
  {
    const uint32_t qv = qrow * rowb + head * 128 + h * 16;
    vload16<0>(qf[0], dq, qv, 0);
    vload16<32>(qf[1], dq, qv, 0);
    vload16<64>(qf[2], dq, qv, 0);
    vload16<96>(qf[3], dq, qv, 0);
  }

  // key blocks of this wave's group: group g takes blocks [g nb / KS,
  // (g+1) nb / KS); every group runs the same number of loop trips (one
  // barrier each), the largest group's count
  const uint32_t nb = (seq + 63) >> 6;
  const uint32_t kb0 = grp * nb / KS;
  const uint32_t nblk = (grp + 1) * nb / KS - kb0;
  const uint32_t iters = (nb + KS - 1) / KS;
  const uint32_t ring = lds_addr(smem) + grp * RB;

  // DMA plan: wave wq copies rows 16wq .. 16wq+15 of the K and V tiles, 8 rows
  // per DMA; lane -> row 16wq + 8i + lane/8, LDS piece lane%8, which holds the
  // row's logical piece (lane%8) ^ swizzle(row)
  uint32_t k_dma[2], v_dma[2], drow[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    drow[i] = 16 * wq + 8 * i + (lane >> 3);
    k_dma[i] = head * 128 + 16 * ((lane & 7) ^ swz_k(drow[i]));
    v_dma[i] = head * 128 + 16 * ((lane & 7) ^ swz_v(drow[i]));
  }
  auto issue = [&](uint32_t blk, uint32_t stage) {
    const uint32_t kv0 = (kb0 + blk) * 64;
    const uint32_t kt = ring + stage * kStageBytes + 16 * wq * 128;
    if (kv0 + 64 <= seq) {  // a whole block: the block offset is a scalar
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t row = drow[i] * rowb;
        dma16<0, true>(dk, row + k_dma[i], kv0 * rowb, kt + i * 1024);
        dma16<0, true>(dv, row + v_dma[i], kv0 * rowb, kt + kTileBytes + i * 1024);
      }
    } else {  // the last block: rows past seq repeat the last row
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t row = min(kv0 + drow[i], seq - 1) * rowb;
        dma16<0, true>(dk, row + k_dma[i], 0, kt + i * 1024);
        dma16<0, true>(dv, row + v_dma[i], 0, kt + kTileBytes + i * 1024);
      }
    }
  };
  // lane constants of the fragment reads: K row r at piece 2s + h; V^T via
  // transpose reads: lane (g = lane/16, c = lane%16) passes row 4h + c/4 of a
  // 4-row group, columns 32dd + 16(g%2) + 4(c%4) .. +3
  uint32_t k_off[4], v_off[2];
#pragma unroll
  for (int st = 0; st < 4; ++st) k_off[st] = r * 128 + 16 * ((2 * st + h) ^ swz_k(r));
  {
    const uint32_t c = lane & 15, rr = c >> 2, cc = c & 3;
    const uint32_t vrow = 4 * h + rr;
#pragma unroll
    for (int dd = 0; dd < 2; ++dd) {
      const uint32_t piece = 4 * dd + 2 * ((lane >> 4) & 1) + (cc >> 1);
      v_off[dd] = vrow * 128 + 16 * (piece ^ swz_v(vrow)) + 8 * (cc & 1);
    }
  }
  auto read_k = [&](uint32_t kt, f16x8(&kf)[2][4]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int st = 0; st < 4; ++st) kf[t][st] = lds_read16(kt + k_off[st] + t * 32 * 128);
  };
  // One block's fragments in the order the group loop consumes them: for
  // group (t, a) the two K fragments of its S products (next block) and the
  // two V^T fragments of its P V products (this block).
  auto read_frags = [&](uint32_t kt, uint32_t vt, f16x8(&kf)[2][4], f16x8(&vf)[2][2][2]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int t = g >> 1, a = g & 1;
      kf[t][2 * a] = lds_read16(kt + k_off[2 * a] + t * 32 * 128);
      kf[t][2 * a + 1] = lds_read16(kt + k_off[2 * a + 1] + t * 32 * 128);
#pragma unroll
      for (int dd = 0; dd < 2; ++dd) {
        const uint32_t at = vt + v_off[dd] + (32 * t + 16 * a) * 128;
        const f16x4 lo = lds_read_tr(at), hi = lds_read_tr(at + 8 * 128);
        vf[dd][t][a] = (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
  };

  f32x16 o[2] = {};
  float mref = -__builtin_inff(), l = 0.0f;
  const f16x2 ones = {(f16)1.0f, (f16)1.0f};
  // The last block's keys past seq take no weight; then the reference max:
  // each lane tests its own 32 scores against it, and only when some lane's
  // pass it does the wave take the two halves' common max (the two halves of
  // a query must keep one reference), so the usual block has no cross-lane
  // step ahead of its exponentials.
  auto prep = [&](uint32_t kv0, f32x16(&s)[2]) {
    if (kv0 + 64 > seq) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (kv0 + 32 * t + 8 * (e >> 2) + 4 * h + (e & 3) >= seq) s[t][e] = -__builtin_inff();
    }
    float mx = s[0][0];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = __builtin_fmaxf(mx, s[t][e]);
    if (__builtin_amdgcn_ballot_w64(mx * kScaleLog2 > mref + kLazy)) {
      mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32));
      const float mnew = mx * kScaleLog2;
      const float nref = mnew > mref + kLazy ? mnew : mref;
      const float alpha = __builtin_amdgcn_exp2f(mref - nref);  // 0 on the first block
      l *= alpha;
#pragma unroll
      for (int dd = 0; dd < 2; ++dd)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dd][e] *= alpha;
      mref = nref;
    }
  };
  // group g = (t, a) of 8 scores: exponentials and P (f16), the row sum over
  // the rounded P (so out is a weighted mean of the V rows with exactly the
  // weights the product used)
  auto exps = [&](const f32x16(&s)[2], int g) {
    const int t = g >> 1, a = g & 1;
    const float nm = -mref;
    f16x8 p;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      p[e] = (f16)__builtin_amdgcn_exp2f(__builtin_fmaf(s[t][8 * a + e], kScaleLog2, nm));
#pragma unroll
    for (int e = 0; e < 8; e += 2) l = __builtin_amdgcn_fdot2((f16x2){p[e], p[e + 1]}, ones, l, false);
    return p;
  };

  if constexpr (!PIPE) {
    // Plain schedule.  Prologue: Q and the first NS - 1 blocks resident.
#pragma unroll
    for (int i = 0; i < NS - 1; ++i)
      if (nblk > (uint32_t)i) issue(i, i);
    wait_q_then_barrier(qf);
    f16x8 qh[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) qh[st] = __builtin_bit_cast(f16x8, qf[st]);
    uint32_t stage = 0;
    for (uint32_t j = 0; j < iters; ++j) {
      if (j + NS - 1 < nblk) issue(j + NS - 1, stage == 0 ? NS - 1 : stage - 1);
      if (j < nblk) {
        const uint32_t cur = ring + stage * kStageBytes;
        f32x16 s[2];
        {
          f16x8 kf[2][4];
          read_k(cur, kf);
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            s[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[t][0], qh[0], (f32x16){}, 0, 0, 0);
#pragma unroll
            for (int st = 1; st < 4; ++st)
              s[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[t][st], qh[st], s[t], 0, 0, 0);
          }
          // the eight fragment reads issue back to back, then the MFMAs: the
          // compiler otherwise pairs each read with its MFMA behind a wait of
          // its own, and the waves, in step after the block barrier, pay the
          // LDS latency eight times (four groups: 22.05-22.35 -> 21.87-21.96 us)
          __builtin_amdgcn_sched_group_barrier(kSchedDSRead, 8, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedMFMA, 8, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        // V^T fragments of group g (t, a) for d tile dd
        auto read_v = [&](int g, int dd) {
          const uint32_t at = cur + kTileBytes + v_off[dd] + (32 * (g >> 1) + 16 * (g & 1)) * 128;
          const f16x4 lo = lds_read_tr(at), hi = lds_read_tr(at + 8 * 128);
          return (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        };
        // three groups: all sixteen fragments up front (the reads overlap the
        // max); four groups (128 VGPRs per wave): each softmax group's own
        f16x8 vf[4][2];
        if constexpr (KS < 4) {
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int dd = 0; dd < 2; ++dd) vf[g][dd] = read_v(g, dd);
        }
        prep((kb0 + j) * 64, s);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          if constexpr (KS >= 4) {
            vf[g][0] = read_v(g, 0);
            vf[g][1] = read_v(g, 1);
          }
          const f16x8 p = exps(s, g);
          o[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[g][0], p, o[0], 0, 0, 0);
          o[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[g][1], p, o[1], 0, 0, 0);
        }
      }
      // block j + 1 has landed (later blocks' DMAs may be in flight) and
      // every wave is done with block j's stage
      if constexpr (NS == 3) {
        if (j + 2 < nblk)
          wait_then_barrier<4>();
        else
          wait_then_barrier<0>();
      } else {
        wait_then_barrier<0>();
      }
      stage = stage + 1 == NS ? 0 : stage + 1;
    }
  } else {
    // Pipelined schedule.  Prologue: Q and blocks 0 and 1 resident, block 2
    // on its way, S of block 0.
  if (nblk > 0) issue(0, 0);
  if (nblk > 1) issue(1, 1);
  // one unconditional wait for Q and both first blocks: the fragments pass
  // through a single asm statement, so the compiler has no merged copy of
  // them to make before the wait
  wait_q_then_barrier(qf);
  if (nblk > 2) issue(2, 2);
  f16x8 qh[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) qh[st] = __builtin_bit_cast(f16x8, qf[st]);
  f32x16 s[2] = {};
  if (nblk > 0) {
    f16x8 kf[2][4];
    read_k(ring, kf);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int st = 0; st < 4; ++st)
        s[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[t][st], qh[st], s[t], 0, 0, 0);
  }

  // Block j: its softmax on the VALU while the matrix cores take the next
  // block's S and this block's P V, interleaved group by group.  The loop
  // keeps blocks j + 1 (its K is read here) and j + 2 resident and block j + 3
  // in flight.
  // one block: s holds its S^T, sn receives the next block's
  auto step = [&](uint32_t j, uint32_t stage, f32x16(&s)[2], f32x16(&sn)[2]) {
    if (j + 3 < nblk) issue(j + 3, (stage + 3) & 3);
    if (j < nblk) {
      const uint32_t cur = ring + stage * kStageBytes;
      // the next block's K (this block's when there is none: multiplied, unused)
      const uint32_t nxt = j + 1 < nblk ? ring + ((stage + 1) & 3) * kStageBytes : cur;
      f16x8 kf[2][4], vf[2][2][2];
      read_frags(nxt, cur + kTileBytes, kf, vf);
      prep((kb0 + j) * 64, s);
      // four groups of 8 scores (t, a): their exponentials and P, the two
      // P V products of the group, and two of the next block's S products
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int t = g >> 1, a = g & 1;
        const f16x8 p = exps(s, g);
        o[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[0][t][a], p, o[0], 0, 0, 0);
        o[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[1][t][a], p, o[1], 0, 0, 0);
        sn[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[t][2 * a], qh[2 * a],
                                                       a ? sn[t] : (f32x16){}, 0, 0, 0);
        sn[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[t][2 * a + 1], qh[2 * a + 1], sn[t], 0, 0, 0);
      }
    }
    // block j + 2 has landed (block j + 3's DMAs may be in flight) and every
    // wave is done with block j's stage and block j + 1's K
    if (j + 3 < nblk)
      wait_then_barrier<4>();
    else
      wait_then_barrier<0>();
  };
  // two blocks per trip, the S buffers trading roles, so no copy between them
  f32x16 s2[2];
  uint32_t j = 0, stage = 0;
  for (; j + 2 <= iters; j += 2, stage = (stage + 2) & 3) {
    step(j, stage, s, s2);
    step(j + 1, (stage + 1) & 3, s2, s);
  }
  if (j < iters) step(j, stage, s, s2);

  }

  // each lane summed the weights of its own 32 keys per block; the two lane
  // halves share the reference max, so their sums add
  l += __shfl_xor(l, 32);

  if constexpr (KS > 1) {
    // key groups 1 .. KS-1 hand (m', sum, O) to group 0 through LDS (the
    // ring is free: every wave passed the loop's last barrier); a group
    // without blocks hands m' = -inf, sum 0, O 0, which weigh nothing
    float *base = reinterpret_cast<float *>(smem) + wq * 34 * 64;
    constexpr int kSlot = 4 * 34 * 64;  // floats per key group
    if (grp > 0) {
      float *xch = base + (grp - 1) * kSlot;
      xch[lane] = mref;
      xch[64 + lane] = l;
#pragma unroll
      for (int dd = 0; dd < 2; ++dd)
#pragma unroll
        for (int e = 0; e < 16; ++e) xch[(2 + 16 * dd + e) * 64 + lane] = o[dd][e];
    }
    __syncthreads();
    if (grp > 0) return;
    float m = mref;
#pragma unroll
    for (int g = 1; g < KS; ++g) m = __builtin_fmaxf(m, base[(g - 1) * kSlot + lane]);
    const float fa = __builtin_amdgcn_exp2f(mref - m);
    l *= fa;
#pragma unroll
    for (int dd = 0; dd < 2; ++dd)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[dd][e] *= fa;
#pragma unroll
    for (int g = 1; g < KS; ++g) {
      const float *xch = base + (g - 1) * kSlot;
      const float fb = __builtin_amdgcn_exp2f(xch[lane] - m);
      l += xch[64 + lane] * fb;
#pragma unroll
      for (int dd = 0; dd < 2; ++dd)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dd][e] += xch[(2 + 16 * dd + e) * 64 + lane] * fb;
    }
  }

  // out row q0 + r, d = 32dd + 8g + 4h + i from o[dd][4g + i]
  const uint32_t orow = q0 + r;
  if (orow < seq) {
    const float inv = 1.0f / (l + 1e-6f);
    f16 *dst = out + (size_t)orow * nh * 64 + head * 64 + 4 * h;
#pragma unroll
    for (int dd = 0; dd < 2; ++dd)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f16x4 val = {(f16)(o[dd][4 * g] * inv), (f16)(o[dd][4 * g + 1] * inv),
                           (f16)(o[dd][4 * g + 2] * inv), (f16)(o[dd][4 * g + 3] * inv)};
        *reinterpret_cast<f16x4 *>(dst + 32 * dd + 8 * g) = val;
      }
  }
}

bool overlaps(const void *a, size_t an, const void *b, size_t bn) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + bn && y < x + an;
}

// Key groups per workgroup (waves per SIMD): four, with the plain schedule
// (measured at 1500 x 20 heads: one group 30.6 us, two pipelined 22.9, three
// 21.3, four 20.5; four also leads at 40 heads and at 3000 frames);
// MADI_FLASH_KSPLIT = 1 .. 4 picks another count.
int key_groups() {
  if (const char *e = getenv("MADI_FLASH_KSPLIT")) {
    const int ks = atoi(e);
    if (ks >= 1 && ks <= 4) return ks;
  }
  return 4;
}

template <int KS, bool PIPE>
void launch_flash(void *out, const void *q, const void *k, const void *v, uint32_t seq, uint32_t nh,
                  uint32_t qtiles) {
  flash_enc_kernel<KS, PIPE><<<nh * qtiles, 256 * KS, 0, stream()>>>(
      (f16 *)out, (const f16 *)q, (const f16 *)k, (const f16 *)v, seq, nh, qtiles);
}

}  // namespace

extern "C" int madi_flash_enc_f16(void *out, const void *q, const void *k, const void *v,
                                  uint32_t seq_len, uint32_t nh) {
  if (!out || !q || !k || !v) return fail(MADI_ERR_NULL, "madi_flash_enc_f16: null pointer");
  if (nh == 0) return fail(MADI_ERR_SHAPE, "madi_flash_enc_f16: nh must be at least 1");
  const size_t bytes = (size_t)seq_len * nh * 128;
  if (bytes > ((size_t)1 << 31))
    return fail(MADI_ERR_SHAPE, "madi_flash_enc_f16: seq_len * nh * 64 f16 = %zu bytes exceeds 2 GiB", bytes);
  if (!aligned(out, 16) || !aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16))
    return fail(MADI_ERR_ALIGN, "madi_flash_enc_f16: out, q, k and v must be 16-byte aligned");
  if (overlaps(out, bytes, k, bytes) || overlaps(out, bytes, v, bytes) ||
      (out != q && overlaps(out, bytes, q, bytes)))
    return fail(MADI_ERR_ARG, "madi_flash_enc_f16: out overlaps k or v (or q other than exactly)");
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_flash_enc_f16: madi_init has not succeeded");
  if (seq_len == 0) return MADI_OK;  // no query rows (the reference's grid is empty)
  for (const void *in : {q, k, v})
    if (int rc = deferred_before_read(in, bytes)) return rc;
  if (int rc = deferred_before_write(out, bytes)) return rc;
  const uint32_t qtiles = (seq_len + kQRows - 1) / kQRows;
  switch (key_groups()) {
  case 1: launch_flash<1, true>(out, q, k, v, seq_len, nh, qtiles); break;
  case 2: launch_flash<2, true>(out, q, k, v, seq_len, nh, qtiles); break;
  case 3: launch_flash<3, false>(out, q, k, v, seq_len, nh, qtiles); break;
  default: launch_flash<4, false>(out, q, k, v, seq_len, nh, qtiles); break;
  }
  return check_launch("madi_flash_enc_f16");
}
