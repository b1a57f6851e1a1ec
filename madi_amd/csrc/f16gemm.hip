// f16gemm.hip -- the boundary's fp16 GEMMs on pre-dequantised weights.
//
// The engine keeps F16 GEMM entry points for callers that hold an F16 weight
// (the encoder's F16 cache, the batched decode's WF16 copy): kM4 / kM4Bias
// (engine/metal/encoder.zig:125-136 -> m4_gemm_nn / m4_gemm_bias /
// m4_gemm_bias_gelu, kernels/m4_gemm.metal:19-115) and matmulF16Batched
// (metal_backend.zig:120 -> mtl_matmul_f16_enc, metal_backend.h:103).
//
// kM4 / kM4Bias on a true F16 weight run f16_nn_gemm_kernel: C[M][N] =
// A[M][K] . B[K][N], all f16 row-major, fp32 accumulation, and the
// reference's epilogue in the same kernel (the product rounded to f16, then
// the f32 bias added and GELU applied, rounded again: m4_gemm.metal:79-85,
// 108-114).  Each chunk of 64 k brings the A tile (BM rows x 128 bytes) and
// the B tile (64 rows x BN columns) into an LDS ring by LDS DMA, issued by
// four producer waves while four computing waves (one per SIMD each) read
// fragments and run the MFMAs; one barrier per chunk.  The A fragments are
// 16-byte LDS reads of a row; the B operand needs eight consecutive k of one
// column, which the row-major B tile gives through the transpose read
// (ds_read_b64_tr_b16: 16 lanes pass 4 rows x 16 columns, lane c receives
// column c's 4 values), two per fragment.  The MFMA takes the B fragment as
// its first operand, so each lane accumulates C^T (four consecutive columns
// of one row); the finished tile goes through LDS and leaves as whole rows.
// proj (decoder.zig:337-341) on a true F16 weight stages its f32 rows to f16
// and takes the same kernel with an f32 result.  Shapes the kernel does not
// take (K not a multiple of 64, N not a multiple of 128, misaligned rows),
// and matmulF16Batched with alpha != 1 or beta != 0, run rocBLAS gemm_ex with
// fp32 accumulation; its bias epilogue is then an elementwise pass.
#include <rocblas/rocblas.h>

#include "common.h"
#include "vmem.h"

namespace madi {

namespace {

// ---------------------------------------------------------------- NN GEMM
// Tile geometry: WM x WN waves, each owning TM x TN MFMA tiles of 32 x 32.
template <int TM, int TN, int WM, int WN>
struct NnGeom {
  static_assert(WM * WN == 4, "four waves");
  static constexpr int kTM = TM, kTN = TN, kWN = WN;
  static constexpr int BM = 32 * TM * WM, BN = 32 * TN * WN;
  static constexpr int kABytes = BM * 128;     // BM rows x 64 k
  static constexpr int kBBytes = 64 * BN * 2;  // 64 k rows x BN columns
  static constexpr int kStage = kABytes + kBBytes;
  static constexpr int kStages = 4 * kStage <= 160 * 1024 ? 4 : 3;
  // wave-wide 1 KiB DMAs per wave and chunk
  static constexpr int kDA = kABytes / 1024 / 4, kDB = kBBytes / 1024 / 4;
  static constexpr int kD = kDA + kDB;
  static_assert(kDA * 4096 == kABytes && kDB * 4096 == kBBytes, "whole DMAs per wave");
  static_assert(kStages * kStage <= 160 * 1024, "LDS");
  static_assert((kStages - 2) * kD < 64, "vmcnt range");
};
// NN tile shapes: 128 x 256 (one column group of 64 per wave), 128 x 128
// (2 x 2 waves of 64 x 64) and 64 x 128 (2 x 2 waves of 32 x 64).
using NnLarge = NnGeom<4, 2, 1, 4>;
using NnMid = NnGeom<2, 2, 2, 2>;
using NnSmall = NnGeom<1, 2, 2, 2>;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
__device__ inline f16x8 lds_read16(uint32_t addr) {
  return __builtin_bit_cast(f16x8, *(const lds_u32x4 *)(uintptr_t)addr);
}
__device__ inline f16x4 lds_read_tr(uint32_t addr) {
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(uintptr_t)addr));
}

// LDS layouts, 16-byte pieces XOR-swizzled so the fragment reads spread over
// all banks: A row m (128 bytes, 8 pieces) keeps logical piece p at
// p ^ ((m >> 1) & 7), so 16 consecutive rows read at one piece hit 16
// distinct 16-byte bank groups; B row k (BN columns) keeps logical piece p at
// p ^ ((k & 3) << 2), so the eight rows of a transpose read (k, k+1, k+2,
// k+3 and the same eight rows on) cover four distinct 64-byte bank groups twice.
__device__ inline uint32_t swz_a(uint32_t row) { return (row >> 1) & 7; }
// buffer cache policy sc1: a store writes through the XCD's L2
constexpr int kSc1 = 16;
__device__ inline uint32_t swz_b(uint32_t row) { return (row & 3) << 2; }

// Grid: one workgroup per tile, the grid rounded up to a multiple of 8.
// Workgroups x and x + 8 run on the same XCD (round-robin dispatch), so each
// XCD takes a contiguous run of tiles, column tiles outermost, and the B
// columns of a run are fetched into one L2.  M rows past the last are read
// as the last row (in bounds) and never stored.  Requires K % 64 == 0,
// N % BN == 0, A, B, C and bias 16-byte aligned.  F32O: C is f32 (the
// unrounded sums, no epilogue) instead of f16.
//
// Eight waves, two per SIMD: waves 0-3 compute (fragment reads and MFMAs),
// waves 4-7 only issue the LDS DMAs.  A DMA waits for room in the address
// queue at issue; in a computing wave that wait would hold back its MFMAs,
// here it holds back only the producing wave while the other wave of its
// SIMD keeps the matrix pipe busy.  Both kinds of wave meet at one barrier
// per chunk: the producers arrive once their DMAs of the chunk about to be
// computed have landed (vmcnt), the computing waves once they are done
// reading the chunk before, whose stage the producers refill right after.
template <class G, int EPI, bool F32O>
__global__ __launch_bounds__(512) void f16_nn_gemm_kernel(
    const f16 *__restrict__ A, const f16 *__restrict__ B, uint32_t M, uint32_t N, uint32_t K,
    uint32_t tiles_m, uint32_t tiles, void *__restrict__ C, const float *__restrict__ bias) {
  constexpr int S = G::kStages, BN = G::BN, TMw = G::kTM, TNw = G::kTN, WNw = G::kWN;
  static_assert(!F32O || EPI == MADI_EPI_NONE, "the f32 result takes no epilogue");
  constexpr uint32_t kOut = F32O ? 4 : 2;  // bytes per C element
  static_assert(G::BM * BN * kOut <= S * G::kStage, "the staged tile fits the ring");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[S * G::kStage];
  const uint32_t lane = threadIdx.x & 63, wave8 = sgpr(threadIdx.x >> 6);
  const uint32_t wave = wave8 & 3;
  const uint32_t h = lane >> 5, r = lane & 31;

  const uint32_t b = blockIdx.x, x = b & 7, per = tiles >> 3, extra = tiles & 7;
  const uint32_t slot = b >> 3;
  if (slot >= per + (x < extra ? 1u : 0u)) return;
  const uint32_t item = x * per + (x < extra ? x : extra) + slot;
  const uint32_t tn = item / tiles_m, tm = item - tn * tiles_m;
  const uint32_t m0 = tm * G::BM, n0 = tn * BN, nk = K / 64;
  const uint32_t ring = lds_addr(smem);
  constexpr uint32_t kPieces = BN * kOut / 16;  // 16-byte pieces per tile row

  if (wave8 >= 4) {
    // ---- producer wave `wave`.  A: DMA j copies rows 8j .. 8j+7 of the
    // tile, lane -> row 8j + lane/8 at stored piece lane%8.  B: DMA j copies
    // stored pieces 64j .. 64j+63 of the row-major tile (BN/8 per row).
    const desc_t da = make_desc(A, M * K * 2), db = make_desc(B, K * N * 2);
    const desc_t dz = make_desc(A, 0);
    uint32_t va[G::kDA], vb[G::kDB];
#pragma unroll
    for (int i = 0; i < G::kDA; ++i) {
      const uint32_t row = 8 * (wave * G::kDA + i) + (lane >> 3);
      const uint32_t gr = m0 + row < M ? m0 + row : M - 1;
      va[i] = gr * K * 2 + 16 * ((lane & 7) ^ swz_a(row));
    }
#pragma unroll
    for (int i = 0; i < G::kDB; ++i) {
      const uint32_t s = 64 * (wave * G::kDB + i) + lane;
      const uint32_t row = s / (BN / 8), q = s % (BN / 8);
      vb[i] = row * N * 2 + 2 * n0 + 16 * (q ^ swz_b(row));
    }
    // chunk c into stage st; chunks past the last load through an empty
    // descriptor (zeros into a stage no later chunk reads), so every trip
    // issues the same DMAs and one wait count serves every trip
    auto issue = [&](uint32_t c, uint32_t st) {
      const uint32_t base = ring + st * G::kStage;
      const bool real = c < nk;
      const desc_t a_ = real ? da : dz, b_ = real ? db : dz;
      const uint32_t ca = real ? c * 128 : 0, cb = real ? c * 128 * N : 0;
#pragma unroll
      for (int i = 0; i < G::kDA; ++i) dma16<0, true>(a_, va[i], ca, base + 1024 * (wave * G::kDA + i));
#pragma unroll
      for (int i = 0; i < G::kDB; ++i)
        dma16<0, true>(b_, vb[i], cb, base + G::kABytes + 1024 * (wave * G::kDB + i));
    };
#pragma unroll
    for (int s = 0; s < S - 1; ++s) issue(s, s);
    uint32_t st = 0;
#pragma unroll 1
    for (uint32_t c = 0; c < nk; ++c) {
      wait_then_barrier<(S - 2) * G::kD>();
      issue(c + S - 1, st == 0 ? S - 1 : st - 1);
      st = st == S - 1 ? 0 : st + 1;
    }
    wait_then_barrier<0>();  // every DMA has landed: the ring is free
    wait_then_barrier<0>();  // the tile is staged
  } else {
    // ---- computing wave (wm, wn): rows 32*TMw*wm .. and columns 32*TNw*wn ..
    // of the tile.  A: row 32*TMw*wm + 32*i + r at piece (2*ks + h) ^ swz_a(r).
    // B: lane (h, xh, c16) passes row 16*ks + 8*h + c16/4 (+4 for the second
    // half of the fragment), columns 32*TNw*wn + 32*j + 16*xh + 4*(c16%4) .. +3
    const uint32_t wm = wave / WNw, wn = wave % WNw;
    const uint32_t a_lane = (32 * TMw * wm + r) * 128;
    const uint32_t sa_r = swz_a(r);
    const uint32_t c16 = lane & 15, xh = (lane >> 4) & 1;
    const uint32_t b_lane = (8 * h + (c16 >> 2)) * (BN * 2) + 8 * (c16 & 1);
    const uint32_t b_p0 = 4 * TNw * wn + 2 * xh + ((c16 & 3) >> 1), b_sw = swz_b(c16 >> 2);

    f32x16 acc[TMw][TNw];
#pragma unroll
    for (int i = 0; i < TMw; ++i)
#pragma unroll
      for (int j = 0; j < TNw; ++j) acc[i][j] = (f32x16){};

    uint32_t st = 0;
#pragma unroll 1
    for (uint32_t c = 0; c < nk; ++c) {
      wait_then_barrier<0>();  // chunk c has landed; chunk c-1's stage is free
      const uint32_t sa = ring + st * G::kStage, sb = sa + G::kABytes;
      // k-step ks's fragments into slot ks & 1: read one k-step ahead of the
      // MFMAs that use them
      f16x8 af[2][TMw], bf[2][TNw];
      auto read = [&](int ks) {
#pragma unroll
        for (int i = 0; i < TMw; ++i)
          af[ks & 1][i] = lds_read16(sa + a_lane + 32 * 128 * i + 16 * ((2 * ks + h) ^ sa_r));
#pragma unroll
        for (int j = 0; j < TNw; ++j) {
          const uint32_t at = sb + 16 * ks * BN * 2 + b_lane + 16 * ((b_p0 + 4 * j) ^ b_sw);
          const f16x4 lo = lds_read_tr(at), hi = lds_read_tr(at + 4 * BN * 2);
          bf[ks & 1][j] = (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      };
      read(0);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        // the next k-step's reads stay ahead of this k-step's MFMAs
        __builtin_amdgcn_sched_barrier(0);
        if (ks < 3) read(ks + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < TMw; ++i)
#pragma unroll
          for (int j = 0; j < TNw; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[ks & 1][j], af[ks & 1][i], acc[i][j], 0, 0, 0);
      }
      st = st == S - 1 ? 0 : st + 1;
    }

    // Epilogue.  acc[i][j][4q + e] is the tile's element (row, col), row =
    // 32*TMw*wm + 32*i + r, col = 32*TNw*wn + 32*j + 8*q + 4*h + e: bias and
    // GELU in registers, then the tile through LDS (free once every DMA has
    // landed and every fragment read is done), so that C leaves as whole rows
    // of 16-byte pieces; written straight from the MFMA layout, each store
    // would touch 32 rows with 8 (f32: 16) bytes.  Row t of the staged tile
    // keeps its logical 16-byte piece p at p ^ (t & 15): the writes of 32 rows
    // at one piece, and the 16-byte reads of whole rows, spread over all banks.
    wait_then_barrier<0>();
#pragma unroll
    for (int i = 0; i < TMw; ++i) {
      const uint32_t trow = 32 * TMw * wm + 32 * i + r;
      const uint32_t rowb = ring + trow * (BN * kOut), sw = trow & 15;
#pragma unroll
      for (int j = 0; j < TNw; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t tcol = 32 * TNw * wn + 32 * j + 8 * q + 4 * h;
          if constexpr (F32O) {
            const f32x4 o = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                             acc[i][j][4 * q + 3]};
            *(lds_u32x4 *)(uintptr_t)(rowb + 16 * ((tcol >> 2) ^ sw)) = __builtin_bit_cast(u32x4, o);
          } else {
            f16x4 o;
            if constexpr (EPI == MADI_EPI_NONE) {
#pragma unroll
              for (int e = 0; e < 4; ++e) o[e] = (f16)acc[i][j][4 * q + e];
            } else {
              const f32x4 bv = *reinterpret_cast<const f32x4 *>(bias + n0 + tcol);
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                float v = (float)(f16)acc[i][j][4 * q + e] + bv[e];
                if constexpr (EPI == MADI_EPI_BIAS_GELU) v = gelu_erf_fast(v);
                o[e] = (f16)v;
              }
            }
            *(lds_u32x2 *)(uintptr_t)(rowb + 16 * ((tcol >> 3) ^ sw) + 8 * h) = __builtin_bit_cast(u32x2, o);
          }
        }
      }
    }
    wait_then_barrier<0>();
  }
  // all eight waves store: thread t takes piece (512 s + t) of the tile in
  // row-major order.  The stores write through the XCD's L2 (sc1): plain
  // write-back stores would leave the whole of C as dirty lines for the
  // release at the kernel's end to write back after the last workgroup.
  // The resource spans the tile's rows that exist (rows past M fall outside).
  const uint32_t rows = M - m0 < G::BM ? M - m0 : G::BM;
  const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
      static_cast<uint8_t *>(C) + (size_t)m0 * N * kOut, 0, (int)(rows * N * kOut), 0x00020000);
#pragma unroll
  for (uint32_t s = 0; s < G::BM * kPieces / 512; ++s) {
    const uint32_t e = 512 * s + threadIdx.x, trow = e / kPieces, p = e % kPieces;
    const u32x4 v = *(const lds_u32x4 *)(uintptr_t)(ring + trow * (BN * kOut) + 16 * (p ^ (trow & 15)));
    if (trow < rows)
      __builtin_amdgcn_raw_buffer_store_b128(v, cr, (trow * N + n0) * kOut + 16 * p, 0, kSc1);
  }
}
rocblas_handle g_blas = nullptr;

int blas(rocblas_handle *h, const char *what) {
  if (!g_blas && rocblas_create_handle(&g_blas) != rocblas_status_success) {
    g_blas = nullptr;
    return fail(MADI_ERR_INIT, "%s: rocblas_create_handle failed", what);
  }
  if (rocblas_set_stream(g_blas, stream()) != rocblas_status_success)
    return fail(MADI_ERR_DISPATCH, "%s: rocblas_set_stream failed", what);
  *h = g_blas;
  return MADI_OK;
}

// C[M][N] = alpha * A[M][K] . B[K][N] + beta * C, all row-major f16: the
// column-major product C^T = B^T A^T with the operands as stored.
int gemm_f16(const char *what, const void *a, const void *b, void *c, uint32_t m, uint32_t n,
             uint32_t k, float alpha, float beta) {
  rocblas_handle h;
  if (int rc = blas(&h, what)) return rc;
  const rocblas_status st = rocblas_gemm_ex(
      h, rocblas_operation_none, rocblas_operation_none, (rocblas_int)n, (rocblas_int)m,
      (rocblas_int)k, &alpha, b, rocblas_datatype_f16_r, (rocblas_int)n, a, rocblas_datatype_f16_r,
      (rocblas_int)k, &beta, c, rocblas_datatype_f16_r, (rocblas_int)n, c, rocblas_datatype_f16_r,
      (rocblas_int)n, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (st != rocblas_status_success)
    return fail(MADI_ERR_DISPATCH, "%s: rocblas_gemm_ex failed (%s)", what, rocblas_status_to_string(st));
  return MADI_OK;
}

// C[M][N] (f32) = A[M][K] (f16) . B[K][N] (f16), row-major, fp32 accumulation
// (rocBLAS with f16 inputs and an f32 result).
int gemm_f16_f32out(const char *what, const void *a, const void *b, float *c, uint32_t m,
                    uint32_t n, uint32_t k) {
  rocblas_handle h;
  if (int rc = blas(&h, what)) return rc;
  const float alpha = 1.0f, beta = 0.0f;
  const rocblas_status st = rocblas_gemm_ex(
      h, rocblas_operation_none, rocblas_operation_none, (rocblas_int)n, (rocblas_int)m,
      (rocblas_int)k, &alpha, b, rocblas_datatype_f16_r, (rocblas_int)n, a, rocblas_datatype_f16_r,
      (rocblas_int)k, &beta, c, rocblas_datatype_f32_r, (rocblas_int)n, c, rocblas_datatype_f32_r,
      (rocblas_int)n, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (st != rocblas_status_success)
    return fail(MADI_ERR_DISPATCH, "%s: rocblas_gemm_ex failed (%s)", what, rocblas_status_to_string(st));
  return MADI_OK;
}

// The operands the fused Q8 GEMM needs (16-byte aligned A, C and bias, whole
// 32-row panels, K a multiple of 64, and madi_q8_gemm's 32-bit buffer limits:
// A, W and one 128-row C tile below 2 GiB); otherwise a recorded weight is
// materialised and the library GEMM runs.
inline bool fusable(const void *a, const void *c, const float *bias, uint32_t m, uint32_t n,
                    uint32_t k) {
  return aligned(a, 16) && aligned(c, 16) && (!bias || aligned(bias, 16)) && n % kPanelRows == 0 &&
         k % kChunkK == 0 && (uint64_t)m * k * 2 < (1ull << 31) && (uint64_t)n * k < (1ull << 31) &&
         (uint64_t)n * 256 < (1ull << 31);
}

// dst[i] = f16(src[i]) (round to nearest even), the engine's f32 -> f16 staging
__global__ __launch_bounds__(256) void to_f16_kernel(f16 *__restrict__ dst,
                                                     const float *__restrict__ src, size_t count) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) dst[i] = (f16)src[i];
}

// c[r][col] = f16(epi(float(c[r][col]) + bias[col])), m4_gemm.metal:79-85 / 108-114
template <bool GELU>
__global__ __launch_bounds__(256) void bias_epilogue_kernel(f16 *__restrict__ c,
                                                            const float *__restrict__ bias,
                                                            uint32_t n, size_t count) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  float v = (float)c[i] + bias[i % n];
  if constexpr (GELU) v = gelu_erf_fast(v);
  c[i] = (f16)v;
}

// Whether f16_nn_gemm_kernel takes the shape: K a multiple of 64, N of 128,
// 16-byte aligned operands, A, B and one 128-row tile of C (its 32-bit
// buffer offsets) below 2 GiB.
bool nn_ok(const void *a, const void *b, const void *c, const float *bias, uint32_t m, uint32_t n,
           uint32_t k) {
  return k % 64 == 0 && n % 128 == 0 && aligned(a, 16) && aligned(b, 16) && aligned(c, 16) &&
         (!bias || aligned(bias, 16)) && (uint64_t)m * k * 2 < (1ull << 31) &&
         (uint64_t)k * n * 2 < (1ull << 31) && (uint64_t)n * 128 * 4 < (1ull << 31);
}

template <class G, int EPI, bool F32O = false>
int launch_nn(const void *a, const void *b, void *c, const float *bias, uint32_t m, uint32_t n,
              uint32_t k, const char *what) {
  const uint32_t tiles_m = (m + G::BM - 1) / G::BM, tiles = tiles_m * (n / G::BN);
  hipLaunchKernelGGL((f16_nn_gemm_kernel<G, EPI, F32O>), dim3((tiles + 7) & ~7u), dim3(512), 0,
                     stream(), static_cast<const f16 *>(a), static_cast<const f16 *>(b), m, n, k,
                     tiles_m, tiles, c, bias);
  return check_launch(what);
}

// epi: an f16 result with that epilogue; kF32Out: the f32 result
constexpr int kF32Out = -1;
template <class G>
int launch_nn_epi(int epi, const void *a, const void *b, void *c, const float *bias, uint32_t m,
                  uint32_t n, uint32_t k, const char *what) {
  switch (epi) {
    case kF32Out: return launch_nn<G, MADI_EPI_NONE, true>(a, b, c, nullptr, m, n, k, what);
    case MADI_EPI_BIAS: return launch_nn<G, MADI_EPI_BIAS>(a, b, c, bias, m, n, k, what);
    case MADI_EPI_BIAS_GELU: return launch_nn<G, MADI_EPI_BIAS_GELU>(a, b, c, bias, m, n, k, what);
    default: return launch_nn<G, MADI_EPI_NONE>(a, b, c, nullptr, m, n, k, what);
  }
}

// The NN GEMM on the largest tiles that still give most CUs a tile: 128 x 256
// (fc1 at M = 1500: 240 tiles), else 128 x 128 (cross K|V 1280 -> 2560: 240),
// else 64 x 128 (1280 -> 1280 and 5120 -> 1280: 240).
int nn_gemm(int epi, const void *a, const void *b, void *c, const float *bias, uint32_t m,
            uint32_t n, uint32_t k, const char *what) {
  const uint64_t fill = (uint64_t)cu_count() * 5 / 8;
  const uint64_t large = (uint64_t)((m + 127) / 128) * (n / 256);
  const uint64_t mid = (uint64_t)((m + 127) / 128) * (n / 128);
  if (n % 256 == 0 && large >= fill) return launch_nn_epi<NnLarge>(epi, a, b, c, bias, m, n, k, what);
  if (mid >= fill) return launch_nn_epi<NnMid>(epi, a, b, c, bias, m, n, k, what);
  return launch_nn_epi<NnSmall>(epi, a, b, c, bias, m, n, k, what);
}
}  // namespace

void f16gemm_cleanup() {
  if (g_blas) (void)rocblas_destroy_handle(g_blas);
  g_blas = nullptr;
}

}  // namespace madi

using namespace madi;

extern "C" int madi_f16_gemm(const void *a, const void *b, void *c, const float *bias, uint32_t m,
                             uint32_t n, uint32_t k, int epilogue) {
  if (!a || !b || !c) return fail(MADI_ERR_NULL, "madi_f16_gemm: null pointer");
  if (epilogue != MADI_EPI_NONE && epilogue != MADI_EPI_BIAS && epilogue != MADI_EPI_BIAS_GELU)
    return fail(MADI_ERR_ARG, "madi_f16_gemm: unknown epilogue %d", epilogue);
  if (epilogue != MADI_EPI_NONE && !bias) return fail(MADI_ERR_NULL, "madi_f16_gemm: null bias");
  if (m == 0 || n == 0 || k == 0 || m > 0x7fffffffu || n > 0x7fffffffu || k > 0x7fffffffu)
    return fail(MADI_ERR_SHAPE, "madi_f16_gemm: m=%u n=%u k=%u", m, n, k);
  if (!aligned(a, 2) || !aligned(b, 2) || !aligned(c, 2) || (bias && !aligned(bias, 4)))
    return fail(MADI_ERR_ALIGN, "madi_f16_gemm: misaligned operand");
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_f16_gemm: madi_init has not succeeded");
  // b is the F16 [K][N] that kDeq recorded for a Q8 weight [N][K]: the fused Q8
  // GEMM runs on that weight (one rounding of acc + bias, the Q8-direct
  // kernel's epilogue, m4_gemm.metal:180-186) and b is never written
  const void *qs, *sc;
  if (fusable(a, c, bias, m, n, k) && deferred_lookup(b, n, k, &qs, &sc))
    return fused_gemm(a, qs, sc, c, bias, m, n, k, epilogue);
  if (int rc = deferred_before_read(a, (size_t)m * k * 2)) return rc;
  if (int rc = deferred_before_read(b, (size_t)k * n * 2)) return rc;
  if (int rc = deferred_before_write(c, (size_t)m * n * 2)) return rc;
  if (nn_ok(a, b, c, bias, m, n, k)) return nn_gemm(epilogue, a, b, c, bias, m, n, k, "madi_f16_gemm");
  if (int rc = gemm_f16("madi_f16_gemm", a, b, c, m, n, k, 1.0f, 0.0f)) return rc;
  if (epilogue == MADI_EPI_NONE) return MADI_OK;
  const size_t count = (size_t)m * n;
  const dim3 grid((unsigned)((count + 255) / 256));
  if (epilogue == MADI_EPI_BIAS)
    hipLaunchKernelGGL(bias_epilogue_kernel<false>, grid, dim3(256), 0, stream(),
                       static_cast<f16 *>(c), bias, n, count);
  else
    hipLaunchKernelGGL(bias_epilogue_kernel<true>, grid, dim3(256), 0, stream(),
                       static_cast<f16 *>(c), bias, n, count);
  return check_launch("madi_f16_gemm(epilogue)");
}

extern "C" int madi_matmul_f16(const void *a, const void *b, void *c, int m, int n, int k,
                               float alpha, float beta) {
  if (!a || !b || !c) return fail(MADI_ERR_NULL, "madi_matmul_f16: null pointer");
  if (m <= 0 || n <= 0 || k <= 0)
    return fail(MADI_ERR_SHAPE, "madi_matmul_f16: m=%d n=%d k=%d", m, n, k);
  if (!aligned(a, 2) || !aligned(b, 2) || !aligned(c, 2))
    return fail(MADI_ERR_ALIGN, "madi_matmul_f16: misaligned operand");
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_matmul_f16: madi_init has not succeeded");
  // b is the F16 [K][N] copy deqW16 recorded for a Q8 weight [N][K]: the
  // product runs from the Q8 weight and b is never written.  Few rows (the
  // batched decode's logits, B = 8 or 16 over the vocab's 51866 rows,
  // transcribe.zig:2391-2394) take the batched projection kernel, which
  // handles any N; many rows on whole panels (the cross-attention K and V of
  // the encoder output, transcribe.zig:2440-2448) the fused GEMM.
  const void *qs, *sc;
  const uint32_t um = (uint32_t)m, un = (uint32_t)n, uk = (uint32_t)k;
  if (alpha == 1.0f && beta == 0.0f && deferred_lookup(b, un, uk, &qs, &sc)) {
    if (skinny_f16_prefers_gemm(um, un, uk) && fusable(a, c, nullptr, um, un, uk))
      return madi_q8_gemm(a, qs, sc, c, nullptr, um, un, uk, MADI_EPI_NONE);
    if (skinny_f16_ok(a, qs, c, um, un, uk)) {
      if (int rc = deferred_before_read(a, (size_t)um * uk * 2)) return rc;
      if (int rc = deferred_before_write(c, (size_t)um * un * 2)) return rc;
      return q8_skinny_f16io(a, qs, sc, c, um, un, uk);
    }
  }
  const size_t mn = (size_t)m * n * 2;
  if (int rc = deferred_before_read(a, (size_t)m * k * 2)) return rc;
  if (int rc = deferred_before_read(b, (size_t)k * n * 2)) return rc;
  if (beta != 0.0f)
    if (int rc = deferred_before_read(c, mn)) return rc;
  if (int rc = deferred_before_write(c, mn)) return rc;
  if (alpha == 1.0f && beta == 0.0f && nn_ok(a, b, c, nullptr, um, un, uk))
    return nn_gemm(MADI_EPI_NONE, a, b, c, nullptr, um, un, uk, "madi_matmul_f16");
  return gemm_f16("madi_matmul_f16", a, b, c, (uint32_t)m, (uint32_t)n, (uint32_t)k, alpha, beta);
}

extern "C" int madi_proj_f16w(float *out, const float *in, const void *w16, void *stage16,
                              uint32_t m, uint32_t n, uint32_t k) {
  if (!out || !in || !w16) return fail(MADI_ERR_NULL, "madi_proj_f16w: null pointer");
  if (m == 0 || n == 0 || k == 0 || m > 0x7fffffffu || n > 0x7fffffffu || k > 0x7fffffffu)
    return fail(MADI_ERR_SHAPE, "madi_proj_f16w: m=%u n=%u k=%u", m, n, k);
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_proj_f16w: madi_init has not succeeded");
  // w16 is a recorded F16 copy of a Q8 weight (deqW16 at decode start): the
  // batched projection runs from the Q8 weight, one kernel
  const void *qs, *sc;
  if (aligned(in, 16) && aligned(out, 4) && deferred_lookup(w16, n, k, &qs, &sc))
    return madi_q8_pproj(out, in, qs, sc, m, n, k);
  // a true F16 weight: the reference's f32 -> f16 staging, then an f16 GEMM
  // with an f32 result
  if (!stage16) return fail(MADI_ERR_NULL, "madi_proj_f16w: null staging buffer for an F16 weight");
  if (!aligned(w16, 2) || !aligned(stage16, 2) || !aligned(in, 4) || !aligned(out, 4))
    return fail(MADI_ERR_ALIGN, "madi_proj_f16w: misaligned operand");
  const size_t count = (size_t)m * k;
  if (int rc = deferred_before_read(in, count * 4)) return rc;
  if (int rc = deferred_before_read(w16, (size_t)k * n * 2)) return rc;
  if (int rc = deferred_before_write(stage16, count * 2)) return rc;
  if (int rc = deferred_before_write(out, (size_t)m * n * 4)) return rc;
  hipLaunchKernelGGL(to_f16_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream(),
                     static_cast<f16 *>(stage16), in, count);
  if (int rc = check_launch("madi_proj_f16w(stage)")) return rc;
  if (nn_ok(stage16, w16, out, nullptr, m, n, k))
    return nn_gemm(kF32Out, stage16, w16, out, nullptr, m, n, k, "madi_proj_f16w");
  return gemm_f16_f32out("madi_proj_f16w", stage16, w16, out, m, n, k);
}
