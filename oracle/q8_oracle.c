/*
 * q8_oracle.c -- CPU restatement of the reference's Q8 matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see q8_oracle.h).  Compiled with
 * -ffp-contract=off so that every `acc += a * w` is a separately rounded fp32
 * multiply and add, as in the Zig CPU loops it restates (Zig does not
 * contract float expressions by default).
 */
#include "q8_oracle.h"

#include <math.h>
#include <string.h>

/* ---- fp16 <-> fp32 (IEEE binary16, round-to-nearest-even) ------------------
 * Written from the IEEE 754 format definition.  Reference semantics: Zig
 * @floatCast(f32 -> f16) and MSL (half)float are both RNE
 * (engine/metal/transcribe.zig:206-208 h2f, engine/metal/kernels/q8_gemm.metal:26). */
float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  float f;
  if (exp == 0) {
    f = (float)man * (1.0f / 16777216.0f); /* man * 2^-24, exact */
    return sign ? -f : f;
  }
  if (exp == 31)
    bits = sign | 0x7f800000u | (man << 13);
  else
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    return (uint16_t)(sign | 0x7c00u);
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {
    /* below 2^-14: the result is a subnormal m * 2^-24 (or 2^-14 after carry) */
    float af;
    memcpy(&af, &ax, 4);
    float m = rintf(af * 16777216.0f); /* exact scaling, RNE in the default mode */
    return (uint16_t)(sign | (uint16_t)m);
  }
  uint32_t e = (ax >> 23) - 112u;
  uint32_t mant = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

void oracle_f16_to_f32_array(float *dst, const uint16_t *src, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = oracle_f16_to_f32(src[i]);
}

void oracle_f32_to_f16_array(uint16_t *dst, const float *src, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = oracle_f32_to_f16(src[i]);
}

/* ---- GELU (erf form, Abramowitz & Stegun 7.1.26) ---------------------------
 * Follows engine/metal/kernels/graph_helpers.metal:460-473 (gelu_erf32) and
 * engine/metal/kernels/m4_gemm.metal:43-56 (gelu_erf), which are identical. */
float oracle_gelu_erf(float xv) {
  float z = xv * 0.7071067811865476f;
  float az = fabsf(z);
  float sign = (z < 0.0f) ? -1.0f : 1.0f;
  float t = 1.0f / fmaf(az, 0.3275911f, 1.0f);
  float poly = fmaf(1.061405429f, t, -1.453152027f);
  poly = fmaf(poly, t, 1.421413741f);
  poly = fmaf(poly, t, -0.284496736f);
  poly = fmaf(poly, t, 0.254829592f);
  poly = poly * t;
  float ex = exp2f(fmaxf(-az * az * 1.4426950408889634f, -80.0f));
  float erf = sign * (1.0f - poly * ex);
  return 0.5f * xv * (1.0f + erf);
}

static inline float deq(const int8_t *qs, const uint16_t *scales, uint32_t k, uint32_t n_idx,
                        uint32_t k_idx) {
  /* w = f32(q) * f32(s): engine/metal/test_q8gemm.zig:65 */
  return (float)qs[(size_t)n_idx * k + k_idx] *
         oracle_f16_to_f32(scales[(size_t)n_idx * (k / 32) + k_idx / 32]);
}

/* ---- dequant_q8_f16: Q8 [N][K] -> f16 [K][N] -------------------------------
 * engine/metal/kernels/q8_gemm.metal:12-27:
 *   out[k*N + n] = half(float(qs[n*K+k]) * float(scales[n*(K/32)+k/32])) */
void oracle_dequant_q8_f16(uint16_t *out_kn, const int8_t *qs, const uint16_t *scales,
                           uint32_t n, uint32_t k) {
  for (uint32_t kk = 0; kk < k; ++kk)
    for (uint32_t nn = 0; nn < n; ++nn)
      out_kn[(size_t)kk * n + nn] = oracle_f32_to_f16(deq(qs, scales, k, nn, kk));
}

static inline float apply_epi(float acc, const float *bias, int epilogue, uint32_t col) {
  switch (epilogue) {
  case ORACLE_EPI_BIAS: return acc + bias[col];
  case ORACLE_EPI_BIAS_GELU: return oracle_gelu_erf(acc + bias[col]);
  default: return acc;
  }
}

/* ---- Q8 GEMM: C[M][N] = A[M][K] (f16) . deq(W)[N][K]^T -----------------------
 * The reference's CPU check, engine/metal/test_q8gemm.zig:59-69:
 *   acc: f32 = 0; for k: deq = f32(q)*f32(s); acc += f32(a) * deq
 * k-sequential fp32, one accumulator per output.  The bias / bias+GELU
 * epilogue follows the fused Q8 GEMM's single-rounding form
 * (engine/metal/kernels/m4_gemm.metal:180-186: v = acc + bias[n];
 * C = half(gelu ? gelu_erf(v) : v)).
 * Writes f32 results (epilogue applied, before any f16 rounding) for the rows
 * listed in `rows` (all rows when rows == NULL). */
void oracle_q8_gemm_rows(float *c_rows, const uint16_t *a, const int8_t *qs,
                         const uint16_t *scales, const float *bias, int epilogue,
                         uint32_t m, uint32_t n, uint32_t k, const uint32_t *rows,
                         uint32_t n_rows, int threads) {
  if (!rows) n_rows = m;
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
  for (uint32_t i = 0; i < n_rows; ++i) {
    uint32_t mm = rows ? rows[i] : i;
    const uint16_t *arow = a + (size_t)mm * k;
    for (uint32_t nn = 0; nn < n; ++nn) {
      float acc = 0.0f;
      for (uint32_t kk = 0; kk < k; ++kk) {
        float w = deq(qs, scales, k, nn, kk);
        acc += oracle_f16_to_f32(arow[kk]) * w;
      }
      c_rows[(size_t)i * n + nn] = apply_epi(acc, bias, epilogue, nn);
    }
  }
}

void oracle_q8_gemm_f16(uint16_t *c, const uint16_t *a, const int8_t *qs,
                        const uint16_t *scales, const float *bias, int epilogue,
                        uint32_t m, uint32_t n, uint32_t k, int threads) {
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
  for (uint32_t mm = 0; mm < m; ++mm) {
    const uint16_t *arow = a + (size_t)mm * k;
    for (uint32_t nn = 0; nn < n; ++nn) {
      float acc = 0.0f;
      for (uint32_t kk = 0; kk < k; ++kk) {
        float w = deq(qs, scales, k, nn, kk);
        acc += oracle_f16_to_f32(arow[kk]) * w;
      }
      c[(size_t)mm * n + nn] = oracle_f32_to_f16(apply_epi(acc, bias, epilogue, nn));
    }
  }
}

/* ---- Q8 GEMV: out[n] = sum_k x[k] * deq(W)[n][k] ------------------------------
 * Dequantise-then-fp32-accumulate with f32 activations, as the batched-
 * projection CPU reference does (engine/metal/test_batchproj.zig:72-78:
 * acc += xf * (f32(q) * f32(s))).  Epilogues restate the fused decoder GEMVs:
 *   BIAS       out = acc + bias[n]                 graph_helpers.metal:450
 *   BIAS_GELU  out = gelu_erf32(acc + bias[n])     graph_helpers.metal:495
 *   BIAS_RES   out = out[n] + acc + bias[n]        graph_helpers.metal:518
 *              (evaluated left to right: (out + acc) + bias) */
void oracle_q8_gemv(float *out, const float *x, const int8_t *qs, const uint16_t *scales,
                    const float *bias, int epilogue, uint32_t n, uint32_t k, int threads) {
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
  for (uint32_t nn = 0; nn < n; ++nn) {
    float acc = 0.0f;
    for (uint32_t kk = 0; kk < k; ++kk) acc += x[kk] * deq(qs, scales, k, nn, kk);
    if (epilogue == ORACLE_EPI_BIAS_RES)
      out[nn] = out[nn] + acc + bias[nn];
    else
      out[nn] = apply_epi(acc, bias, epilogue, nn);
  }
}

/* ---- fused decoder QKV GEMV + KV-cache store -----------------------------------
 * engine/metal/kernels/graph_helpers.metal:527-558 (gemv_q8_qkv):
 *   n <  D : q_out[n]            = acc + qb[n]
 *   n < 2D : kc[pos*D + (n-D)]   = acc            (k has no bias)
 *   else   : vc[pos*D + (n-2D)]  = acc + vb[n-2D]
 * over a stacked [3D][D] weight. */
void oracle_q8_gemv_qkv(float *q_out, const float *x, const int8_t *qs,
                        const uint16_t *scales, const float *qb, const float *vb,
                        float *kc, float *vc, uint32_t pos, uint32_t d) {
  for (uint32_t nn = 0; nn < 3 * d; ++nn) {
    float acc = 0.0f;
    for (uint32_t kk = 0; kk < d; ++kk) acc += x[kk] * deq(qs, scales, d, nn, kk);
    if (nn < d)
      q_out[nn] = acc + qb[nn];
    else if (nn < 2 * d)
      kc[(size_t)pos * d + (nn - d)] = acc;
    else
      vc[(size_t)pos * d + (nn - 2 * d)] = acc + vb[nn - 2 * d];
  }
}

/* ---- batched / prefill projection, f32 in -> f32 out ---------------------------
 * What decoder.zig `proj` (:337-341) and `pproj` (:427-432) compute, stated as
 * the dequantise-then-fp32-accumulate product of the f32 input rows with the
 * Q8 weight (the reference's own CPU check for these shapes,
 * engine/metal/test_batchproj.zig:72-78). */
void oracle_q8_proj(float *out, const float *in, const int8_t *qs, const uint16_t *scales,
                    uint32_t m, uint32_t n, uint32_t k, int threads) {
  if (threads < 1) threads = 1;
#pragma omp parallel for collapse(2) schedule(static) num_threads(threads)
  for (uint32_t mm = 0; mm < m; ++mm)
    for (uint32_t nn = 0; nn < n; ++nn) {
      float acc = 0.0f;
      for (uint32_t kk = 0; kk < k; ++kk)
        acc += in[(size_t)mm * k + kk] * deq(qs, scales, k, nn, kk);
      out[(size_t)mm * n + nn] = acc;
    }
}

/* ---- Q8_0 quantiser ------------------------------------------------------------
 * engine/metal/transcribe.zig:309-326 (quantInto, g_q4 off) and its offline twin
 * engine/metal/bench/quantize_q8.py:27-40.  Per 32-block of an f16 row:
 *   mx = max |w| (f32);  scale = mx > 0 ? mx / 127 : 1.0 (f32);  store f16(scale)
 *   inv = 1 / scale (f32);  q = clamp(round_half_away(w * inv), -127, 127)
 * Zig's @round rounds half away from zero, as C's roundf does. */
void oracle_quantize_q8(int8_t *qs, uint16_t *scales, const uint16_t *w_f16, uint32_t rows,
                        uint32_t dim) {
  uint32_t nb = dim / 32;
  for (uint32_t r = 0; r < rows; ++r)
    for (uint32_t b = 0; b < nb; ++b) {
      const uint16_t *blk = w_f16 + (size_t)r * dim + (size_t)b * 32;
      float mx = 0.0f;
      for (int i = 0; i < 32; ++i) {
        float w = fabsf(oracle_f16_to_f32(blk[i]));
        if (w > mx) mx = w;
      }
      float scale = mx > 0.0f ? mx / 127.0f : 1.0f;
      scales[(size_t)r * nb + b] = oracle_f32_to_f16(scale);
      float inv = 1.0f / scale;
      for (int i = 0; i < 32; ++i) {
        float q = roundf(oracle_f16_to_f32(blk[i]) * inv);
        if (q < -127.0f) q = -127.0f;
        if (q > 127.0f) q = 127.0f;
        qs[(size_t)r * dim + (size_t)b * 32 + i] = (int8_t)q;
      }
    }
}

/* ---- FNV-1a 64 (WHASH weight identity) -----------------------------------------
 * engine/metal/transcribe.zig:129-140: x ^= b; x *%= 0x100000001b3, over qs
 * bytes then the scales' little-endian bytes; seed 0xcbf29ce484222325
 * (:1225). */
uint64_t oracle_fnv1a64(uint64_t seed, const uint8_t *bytes, size_t n) {
  uint64_t x = seed;
  for (size_t i = 0; i < n; ++i) {
    x ^= bytes[i];
    x *= 0x100000001b3ull;
  }
  return x;
}

uint64_t oracle_fnv_q8(uint64_t seed, const int8_t *qs, size_t nq, const uint16_t *scales,
                       size_t nsc) {
  uint64_t x = oracle_fnv1a64(seed, (const uint8_t *)qs, nq);
  return oracle_fnv1a64(x, (const uint8_t *)scales, nsc * 2);
}

/* ---- Q8 embedding row ----------------------------------------------------------
 * engine/metal/kernels/graph_helpers.metal:370-383 (gpu_emb_lookup_q8):
 *   out[d] = float(qs[tok*dim + d]) * float(scales[tok*(dim/32) + d/32]) */
void oracle_emb_row_q8(float *out, const int8_t *qs, const uint16_t *scales, uint32_t tok,
                       uint32_t dim) {
  for (uint32_t d = 0; d < dim; ++d) out[d] = deq(qs, scales, dim, tok, d);
}

/* ---- Q8 embedding rows plus positions (sequence prefill) ------------------------
 * engine/metal/kernels/decoder_ops.metal:614-633 (emb_pe_rows_q8):
 *   out[m*dim + d] = float(qs[tokens[m]*dim + d]) * float(scales[tokens[m]*(dim/32) + d/32])
 *                    + pe[(pos0 + m)*dim + d] */
void oracle_emb_pe_rows_q8(float *out, const int8_t *qs, const uint16_t *scales,
                           const uint32_t *tokens, const float *pe, uint32_t dim, uint32_t pos0,
                           uint32_t m) {
  for (uint32_t r = 0; r < m; ++r)
    for (uint32_t d = 0; d < dim; ++d) {
      const float e = deq(qs, scales, dim, tokens[r], d);
      out[(size_t)r * dim + d] = e + pe[(size_t)(pos0 + r) * dim + d];
    }
}

/* ---- f16 GEMM on pre-dequantised weights ---------------------------------------
 * The MPS op behind mtl_matmul_f16_enc (engine/metal/metal_backend.h:103):
 * C[M][N] = alpha * A[M][K] . B[K][N] + beta * C, all f16 row-major.  MPS does not
 * document its accumulation precision; this restatement accumulates in fp32,
 * k-sequential, and rounds once to f16. */
void oracle_gemm_f16(uint16_t *c, const uint16_t *a, const uint16_t *b, uint32_t m,
                     uint32_t n, uint32_t k, float alpha, float beta, int threads) {
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
  for (uint32_t mm = 0; mm < m; ++mm)
    for (uint32_t nn = 0; nn < n; ++nn) {
      float acc = 0.0f;
      for (uint32_t kk = 0; kk < k; ++kk)
        acc += oracle_f16_to_f32(a[(size_t)mm * k + kk]) *
               oracle_f16_to_f32(b[(size_t)kk * n + nn]);
      float r = alpha * acc;
      if (beta != 0.0f) r = r + beta * oracle_f16_to_f32(c[(size_t)mm * n + nn]);
      c[(size_t)mm * n + nn] = oracle_f32_to_f16(r);
    }
}

/* ---- encoder self-attention over the projections ---------------------------------
 * m4_flash_enc (engine/metal/kernels/m4_gemm.metal:268-407), dispatched by kFlash
 * (engine/metal/encoder.zig:138-152).  q, k, v, out: f16 [seq][nh*64], head hd in
 * columns hd*64 .. hd*64+63.  Per head and 64-row query tile, over 64-key blocks
 * (:325-400): S = Q.K^T in f32 (:327-336), v = S * 0.125 with keys >= seq at -inf
 * (:342-356), the row max over the block's two 32-column halves and the running
 * max m (:357-360), alpha = exp(m_old - m_new), 0 while m_old is -inf (:361),
 * e = exp(v - m_new), masked keys 0 (:363-374), P = f16(e) (:375), per-half sums
 * of the unrounded e folded as sum = sum * alpha + half0 + half1 (:377-382),
 * O = O * alpha + P.V in f32 (:384-394); out = f16(O / (sum + 1e-6)) for rows
 * < seq (:396-406).  Rows past seq and keys past seq are never read. */
void oracle_flash_enc_f16(uint16_t *out, const uint16_t *q, const uint16_t *k,
                          const uint16_t *v, uint32_t seq, uint32_t nh, int threads) {
  if (threads < 1) threads = 1;
  const uint32_t tiles = (seq + 63) / 64;
  const size_t ld = (size_t)nh * 64;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
  for (uint32_t job = 0; job < nh * tiles; ++job) {
    const uint32_t hd = job / tiles, q0 = (job % tiles) * 64;
    const uint32_t rows = seq - q0 < 64 ? seq - q0 : 64;
    float qf[64][64], o[64][64], s[64][64], m[64], sum[64];
    uint16_t p[64][64];
    for (uint32_t i = 0; i < rows; ++i) {
      for (uint32_t d = 0; d < 64; ++d) {
        qf[i][d] = oracle_f16_to_f32(q[(q0 + i) * ld + hd * 64 + d]);
        o[i][d] = 0.0f;
      }
      m[i] = -INFINITY;
      sum[i] = 0.0f;
    }
    for (uint32_t kv0 = 0; kv0 < seq; kv0 += 64) {
      const uint32_t kcur = seq - kv0 < 64 ? seq - kv0 : 64;
      for (uint32_t j = 0; j < kcur; ++j) {
        float kr[64];
        for (uint32_t d = 0; d < 64; ++d) kr[d] = oracle_f16_to_f32(k[(kv0 + j) * ld + hd * 64 + d]);
        for (uint32_t i = 0; i < rows; ++i) {
          float acc = 0.0f;
          for (uint32_t d = 0; d < 64; ++d) acc += qf[i][d] * kr[d];
          s[i][j] = acc;
        }
      }
      for (uint32_t i = 0; i < rows; ++i) {
        float half_max[2] = {-INFINITY, -INFINITY}, half_sum[2] = {0.0f, 0.0f};
        for (uint32_t j = 0; j < kcur; ++j) {
          const float x = s[i][j] * 0.125f;
          if (x > half_max[j / 32]) half_max[j / 32] = x;
        }
        float m_new = m[i];
        if (half_max[0] > m_new) m_new = half_max[0];
        if (half_max[1] > m_new) m_new = half_max[1];
        const float alpha = (m[i] == -INFINITY) ? 0.0f : expf(m[i] - m_new);
        for (uint32_t hf = 0; hf < 2; ++hf)
          for (uint32_t j4 = 32 * hf; j4 < 32 * hf + 32; j4 += 4) {
            float e4[4];
            for (uint32_t c = 0; c < 4; ++c) {
              const uint32_t j = j4 + c;
              e4[c] = j < kcur ? expf(s[i][j] * 0.125f - m_new) : 0.0f;
              p[i][j] = oracle_f32_to_f16(e4[c]);
            }
            half_sum[hf] += e4[0] + e4[1] + e4[2] + e4[3];
          }
        m[i] = m_new;
        sum[i] = sum[i] * alpha + half_sum[0] + half_sum[1];
        for (uint32_t d = 0; d < 64; ++d) o[i][d] *= alpha;
      }
      for (uint32_t j = 0; j < kcur; ++j) {
        float vr[64];
        for (uint32_t d = 0; d < 64; ++d) vr[d] = oracle_f16_to_f32(v[(kv0 + j) * ld + hd * 64 + d]);
        for (uint32_t i = 0; i < rows; ++i) {
          const float pij = oracle_f16_to_f32(p[i][j]);
          for (uint32_t d = 0; d < 64; ++d) o[i][d] += pij * vr[d];
        }
      }
    }
    for (uint32_t i = 0; i < rows; ++i)
      for (uint32_t d = 0; d < 64; ++d)
        out[(q0 + i) * ld + hd * 64 + d] = oracle_f32_to_f16(o[i][d] / (sum[i] + 1e-6f));
  }
}
