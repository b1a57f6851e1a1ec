// boundary.hip -- the engine-facing half of the C ABI: kernel handles by name,
// the wrappers that take them, and the deferred dequantisation that lets the
// engine's unchanged call sequences reach the fused Q8 kernels.
//
// The engine resolves its kernels by name once (mtl.getFunction,
// engine/metal/metal_backend.zig:61-65; encoder.zig:41-51, decoder.zig:64-81)
// and passes the handle to wrappers such as kM4 / kM4Bias (encoder.zig:125-136)
// and kGemvQ8BiasEpi (decoder.zig:176-181).  madi_get_function hands out
// handles for the names of this path, and madi_m4_gemm / madi_q8_gemv_epi take
// them, so those wrappers keep their `f: mtl.Function` parameter.
//
// The encoder's forward pass (encoder.zig:262-301) dequantises each Q8 weight
// into a shared F16 scratch (kDeq -> wdq) and multiplies by it on the next
// line (kM4 / kM4Bias(f, x, wdq, ...)); the batched decoder does the same with
// its per-decode F16 copies (deqW16 -> WF16, then proj / matmulF16Batched).
// Here madi_q8_dequant_f16 records the pair (wdq -> Q8 weight) instead of
// writing wdq, and an F16 GEMM whose weight operand is exactly a recorded wdq
// with the recorded shape runs the fused Q8 kernel on the Q8 weight.  The
// dequantisation is carried out ("materialised") only when something else
// could observe wdq: a library op that reads it any other way, a download of
// it, a write or free of the Q8 source, or an explicit madi_q8_materialize.  A
// write into wdq (another dequant, an op's output, an upload) or its free
// retires the record.  Reads and writes of wdq or of its Q8 source by code
// outside this library are not visible here: such a caller calls
// madi_q8_materialize before a read and madi_q8_forget before a write, or
// turns the deferral off (madi_set_deferred_dequant(0)).
#include <string.h>

#include <vector>

#include "common.h"

namespace madi {

namespace {

// Kernel handles: the reference's kernel names on this path.
enum Fn {
  kFnNone = 0,
  kFnDeq,
  kFnM4,
  kFnM4Bias,
  kFnM4BiasGelu,
  kFnGemv,
  kFnGemvBias,
  kFnGemvBiasGelu,
  kFnGemvBiasRes,
  kFnQkv,
  kFnLogit,
  kFnEmbLookup,
  kFnEmbIndirect,
  kFnEmbPeRows,
  kFnMulMmQ8,
  kFnFlashEnc,
};

struct FnName {
  const char *name;
  Fn id;
};
// kernels/q8_gemm.metal:12, 29; m4_gemm.metal:19, 60, 88, 268; graph_helpers.metal:320,
// 354, 370, 390, 424, 475, 498, 527; decoder_ops.metal:614; encoder_ops.metal:398
constexpr FnName kFunctions[] = {
    {"dequant_q8_f16", kFnDeq},          {"m4_gemm_nn", kFnM4},
    {"m4_gemm_bias", kFnM4Bias},         {"m4_gemm_bias_gelu", kFnM4BiasGelu},
    {"gemv_q8", kFnGemv},                {"gemv_q8_bias", kFnGemvBias},
    {"gemv_q8_bias_gelu", kFnGemvBiasGelu}, {"gemv_q8_bias_res", kFnGemvBiasRes},
    {"gemv_q8_qkv", kFnQkv},             {"logit_gemv_q8", kFnLogit},
    {"gpu_emb_lookup_q8", kFnEmbLookup}, {"emb_lookup_indirect_q8", kFnEmbIndirect},
    {"emb_pe_rows_q8", kFnEmbPeRows},    {"mul_mm_q8", kFnMulMmQ8},
    {"m4_flash_enc", kFnFlashEnc},       {"flash_attention_enc_f16", kFnFlashEnc},
};

// One recorded kDeq.  [lo, hi) is the byte range of wdq still owed the
// dequantised weights: all of it when recorded; a later write by this library
// that covers one end of the range (the encoder's next, smaller kDeq into the
// same scratch, encoder.zig:262-265 after :297) moves that end instead of
// writing the weights out first.  A record whose range is no longer all of
// wdq serves no fused GEMM; it is only carried out (over its range) if
// something observes that range.
struct Deferred {
  uintptr_t wdq;        // F16 [K][N] destination, 2*n*k bytes
  const void *qs, *sc;  // panel-layout Q8 source
  uint32_t n, k;
  bool pending;   // the range not written yet
  size_t lo, hi;  // byte range of wdq owed the weights
};
std::vector<Deferred> g_def;
bool g_defer = true;

bool overlaps(uintptr_t a, size_t an, uintptr_t b, size_t bn) { return a < b + bn && b < a + an; }

size_t wdq_bytes(const Deferred &d) { return (size_t)d.n * d.k * 2; }
bool whole(const Deferred &d) { return d.lo == 0 && d.hi == wdq_bytes(d); }
bool range_overlaps(const Deferred &d, uintptr_t p, size_t bytes) {
  return overlaps(d.wdq + d.lo, d.hi - d.lo, p, bytes);
}

bool source_overlaps(const Deferred &d, uintptr_t p, size_t bytes) {
  return overlaps(reinterpret_cast<uintptr_t>(d.qs), (size_t)d.n * d.k, p, bytes) ||
         overlaps(reinterpret_cast<uintptr_t>(d.sc), (size_t)d.n * (d.k / 32) * 2, p, bytes);
}

int materialize(Deferred &d) {
  if (!d.pending) return MADI_OK;
  // lo and hi are even (element boundaries) by construction
  if (int rc = dequant_launch(reinterpret_cast<void *>(d.wdq), d.qs, d.sc, d.n, d.k, d.lo / 2,
                              d.hi / 2))
    return rc;
  d.pending = false;
  return MADI_OK;
}

}  // namespace

static void retire(size_t i) {
  g_def[i] = g_def.back();
  g_def.pop_back();
}

int deferred_before_write(const void *ptr, size_t bytes) {
  if (g_def.empty() || !ptr) return MADI_OK;
  const uintptr_t p = reinterpret_cast<uintptr_t>(ptr);
  for (size_t i = 0; i < g_def.size();) {
    Deferred &d = g_def[i];
    const bool src = source_overlaps(d, p, bytes);
    const bool dst = range_overlaps(d, p, bytes);
    if (!src && !dst) {
      ++i;
      continue;
    }
    if (!src) {
      // Part of the owed range is about to be overwritten.  A write over all
      // of it makes the record moot; one over either end (at an element
      // boundary) shortens the range; one inside it leaves two pieces, which
      // are written out now (the write then lands on top).
      const uintptr_t a = d.wdq + d.lo, b = d.wdq + d.hi;
      const bool head = p <= a, tail = p + bytes >= b;
      if (head && tail) {
        retire(i);
        continue;
      }
      if (head && (p + bytes - d.wdq) % 2 == 0) {
        d.lo = p + bytes - d.wdq;
        ++i;
        continue;
      }
      if (tail && (p - d.wdq) % 2 == 0) {
        d.hi = p - d.wdq;
        ++i;
        continue;
      }
    }
    // The Q8 source is about to change, or the write splits the range:
    // wdq gets its weights now.
    if (int rc = materialize(d)) return rc;
    retire(i);
  }
  return MADI_OK;
}

int deferred_before_free(const void *ptr, size_t bytes) {
  if (g_def.empty() || !ptr) return MADI_OK;
  const uintptr_t p = reinterpret_cast<uintptr_t>(ptr);
  int launched = 0;
  for (size_t i = 0; i < g_def.size();) {
    Deferred &d = g_def[i];
    const bool dst = range_overlaps(d, p, bytes);
    const bool src = source_overlaps(d, p, bytes);
    if (!src && !dst) {
      ++i;
      continue;
    }
    // a Q8 source about to be freed: its wdq (if it survives) is written now
    if (src && !dst && d.pending) {
      if (int rc = materialize(d)) return rc;
      launched = 1;
    }
    retire(i);
  }
  return launched;
}

int deferred_before_read(const void *ptr, size_t bytes) {
  if (g_def.empty() || !ptr) return MADI_OK;
  const uintptr_t p = reinterpret_cast<uintptr_t>(ptr);
  for (Deferred &d : g_def)
    if (d.pending && range_overlaps(d, p, bytes))
      if (int rc = materialize(d)) return rc;
  return MADI_OK;
}

bool deferred_lookup(const void *wdq, uint32_t n, uint32_t k, const void **qs, const void **sc) {
  const uintptr_t p = reinterpret_cast<uintptr_t>(wdq);
  for (const Deferred &d : g_def)
    if (d.wdq == p && d.n == n && d.k == k && whole(d)) {
      *qs = d.qs;
      *sc = d.sc;
      return true;
    }
  return false;
}

int deferred_record(void *wdq, const void *qs, const void *sc, uint32_t n, uint32_t k) {
  // wdq is overwritten either way: records that name it (or whose source it
  // overlaps) are retired first
  if (int rc = deferred_before_write(wdq, (size_t)n * k * 2)) return rc;
  if (!g_defer) return 0;
  g_def.push_back({reinterpret_cast<uintptr_t>(wdq), qs, sc, n, k, true, 0, (size_t)n * k * 2});
  return 1;
}

int deferred_flush_all() {
  for (Deferred &d : g_def)
    if (int rc = materialize(d)) return rc;
  g_def.clear();
  return MADI_OK;
}

}  // namespace madi

using namespace madi;

extern "C" int madi_get_function(const char *name, int *out_id) {
  if (!name || !out_id) return fail(MADI_ERR_NULL, "madi_get_function: null pointer");
  for (const FnName &f : kFunctions)
    if (strcmp(f.name, name) == 0) {
      *out_id = (int)f.id;
      return MADI_OK;
    }
  return fail(MADI_ERR_ARG, "madi_get_function: no kernel named '%s' on the Q8 path", name);
}

extern "C" int madi_q8_materialize(void *wdq) {
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_q8_materialize: madi_init has not succeeded");
  if (!wdq) {
    for (Deferred &d : g_def)
      if (int rc = materialize(d)) return rc;
    return MADI_OK;
  }
  // every record naming wdq (a shortened one and the later kDeq that
  // shortened it own disjoint ranges)
  for (Deferred &d : g_def)
    if (d.wdq == reinterpret_cast<uintptr_t>(wdq))
      if (int rc = materialize(d)) return rc;
  return MADI_OK;
}

extern "C" int madi_q8_forget(void *ptr, size_t bytes) {
  if (!ptr || bytes == 0) return MADI_OK;
  if (!initialized()) return fail(MADI_ERR_NOT_INIT, "madi_q8_forget: madi_init has not succeeded");
  // the same bookkeeping as a write by this library: a recorded wdq that the
  // write covers entirely is dropped, one it covers in part, or whose Q8
  // source it touches, is written first
  return deferred_before_write(ptr, bytes);
}

extern "C" int madi_set_deferred_dequant(int on) {
  if (!on && initialized())
    for (Deferred &d : g_def)
      if (int rc = materialize(d)) return rc;
  g_defer = on != 0;
  return MADI_OK;
}

extern "C" int madi_m4_gemm(int func, const void *a, const void *b, void *c, const float *bias,
                            uint32_t m, uint32_t n, uint32_t k) {
  int epi;
  switch (func) {
  case kFnM4: epi = MADI_EPI_NONE; break;
  case kFnM4Bias: epi = MADI_EPI_BIAS; break;
  case kFnM4BiasGelu: epi = MADI_EPI_BIAS_GELU; break;
  default: return fail(MADI_ERR_ARG, "madi_m4_gemm: handle %d is not m4_gemm_nn/_bias/_bias_gelu", func);
  }
  return madi_f16_gemm(a, b, c, epi == MADI_EPI_NONE ? nullptr : bias, m, n, k, epi);
}

extern "C" int madi_q8_gemv_epi(int func, float *out, const float *x, const void *qs,
                                const void *scales, const float *bias, uint32_t n, uint32_t k) {
  switch (func) {
  case kFnGemvBias: return madi_q8_gemv_bias(out, x, qs, scales, bias, n, k);
  case kFnGemvBiasGelu: return madi_q8_gemv_bias_gelu(out, x, qs, scales, bias, n, k);
  case kFnGemvBiasRes: return madi_q8_gemv_bias_res(out, x, qs, scales, bias, n, k);
  default:
    return fail(MADI_ERR_ARG, "madi_q8_gemv_epi: handle %d is not gemv_q8_bias/_bias_gelu/_bias_res", func);
  }
}
