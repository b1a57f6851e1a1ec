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

// ---- q|k|v as one launch.  The encoder computes q, k and v as three GEMMs
// on the same activations (encoder.zig:262-267): kDeq of a 1280-row slice of
// the stacked q|k|v weight, then kM4Bias into its own output, three times.
// A fused GEMM whose weight is the first slice of a stacked weight (a
// madi_alloc allocation holding at least three such slices) is held back;
// the next fused GEMMs with the same activations, shape and epilogue on the
// following slices join it, and the group runs as one launch of the stacked
// GEMM with three outputs once its last slice (the allocation's end, or the
// third) arrives.  Anything else that touches the group's memory -- a read
// of an output, a write of any operand -- or a sync, commit or stream change
// launches the group first.  Code outside this library that reads q or k
// before the v GEMM has been issued must call madi_sync (or
// madi_set_gemm_grouping(0)); the engine reads them only in kFlash, after v.
struct PendingGemm {
  const void *a, *qs, *sc;
  void *c;
  const float *bias;
  uint32_t m, n, k;
  int epi;
};
PendingGemm g_grp[kMaxSegs];
int g_ngrp = 0;
bool g_grouping = true;

bool group_touches(uintptr_t p, size_t bytes, bool write) {
  for (int i = 0; i < g_ngrp; ++i) {
    const PendingGemm &g = g_grp[i];
    if (overlaps(reinterpret_cast<uintptr_t>(g.c), (size_t)g.m * g.n * 2, p, bytes)) return true;
    if (!write) continue;
    if (overlaps(reinterpret_cast<uintptr_t>(g.a), (size_t)g.m * g.k * 2, p, bytes) ||
        overlaps(reinterpret_cast<uintptr_t>(g.qs), (size_t)g.n * g.k, p, bytes) ||
        overlaps(reinterpret_cast<uintptr_t>(g.sc), (size_t)g.n * (g.k / 32) * 2, p, bytes) ||
        (g.bias && overlaps(reinterpret_cast<uintptr_t>(g.bias), (size_t)g.n * 4, p, bytes)))
      return true;
  }
  return false;
}

}  // namespace

// Launches the held q|k|v group (as one GEMM with an output per slice where
// the shape's kernel allows it, else one GEMM per slice).
int group_flush() {
  if (g_ngrp == 0) return MADI_OK;
  PendingGemm g[kMaxSegs];
  const int cnt = g_ngrp;
  for (int i = 0; i < cnt; ++i) g[i] = g_grp[i];
  g_ngrp = 0;  // the launches below check their operands against no group
  if (cnt > 1) {
    OutSeg seg{};
    seg.n = g[0].n;
    for (int i = 0; i < cnt; ++i) {
      seg.c[i] = g[i].c;
      seg.b[i] = g[i].bias;
    }
    const int rc = q8_gemm_seg(g[0].a, g[0].qs, g[0].sc, seg, g[0].m, g[0].n * cnt, g[0].k, g[0].epi);
    if (rc != kSegUnsupported) return rc;
  }
  for (int i = 0; i < cnt; ++i)
    if (int rc = madi_q8_gemm(g[i].a, g[i].qs, g[i].sc, g[i].c, g[i].bias, g[i].m, g[i].n, g[i].k,
                              g[i].epi))
      return rc;
  return MADI_OK;
}

// The fused route of the F16 GEMM entry points (a recorded wdq as the weight):
// joins, holds or launches, as described above.
int fused_gemm(const void *a, const void *qs, const void *sc, void *c, const float *bias, uint32_t m,
               uint32_t n, uint32_t k, int epi) {
  const uintptr_t ua = reinterpret_cast<uintptr_t>(a), uc = reinterpret_cast<uintptr_t>(c);
  const size_t abytes = (size_t)m * k * 2, cbytes = (size_t)m * n * 2;
  const size_t qbytes = (size_t)n * k, sbytes = (size_t)n * (k / 32) * 2;
  if (g_ngrp > 0) {
    const PendingGemm &f = g_grp[0], &l = g_grp[g_ngrp - 1];
    bool join = g_grouping && g_ngrp < kMaxSegs && a == f.a && m == f.m && n == f.n && k == f.k &&
                epi == f.epi &&
                qs == static_cast<const uint8_t *>(l.qs) + qbytes &&
                sc == static_cast<const uint8_t *>(l.sc) + sbytes && !overlaps(uc, cbytes, ua, abytes);
    for (int i = 0; join && i < g_ngrp; ++i)
      join = !overlaps(uc, cbytes, reinterpret_cast<uintptr_t>(g_grp[i].c), cbytes);
    if (join) {
      if (int rc = deferred_before_write(c, cbytes)) return rc;
      // (that write could touch the group's weights or bias and launch it;
      // then this GEMM is no longer part of a group)
      if (g_ngrp > 0) {
        g_grp[g_ngrp++] = {a, qs, sc, c, bias, m, n, k, epi};
        if (g_ngrp == kMaxSegs || alloc_extent(qs) < 2 * qbytes) return group_flush();
        return MADI_OK;
      }
    } else if (int rc = group_flush()) {
      return rc;
    }
  }
  if (g_grouping && alloc_extent(qs) >= 3 * qbytes && alloc_extent(sc) >= 3 * sbytes &&
      !overlaps(uc, cbytes, ua, abytes)) {
    if (int rc = deferred_before_read(a, abytes)) return rc;
    if (int rc = deferred_before_write(c, cbytes)) return rc;
    g_grp[0] = {a, qs, sc, c, bias, m, n, k, epi};
    g_ngrp = 1;
    return MADI_OK;
  }
  return madi_q8_gemm(a, qs, sc, c, bias, m, n, k, epi);
}

static void retire(size_t i) {
  g_def[i] = g_def.back();
  g_def.pop_back();
}

int deferred_before_write(const void *ptr, size_t bytes) {
  if (g_ngrp && ptr && group_touches(reinterpret_cast<uintptr_t>(ptr), bytes, true))
    if (int rc = group_flush()) return rc;
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
  int launched = 0;
  if (g_ngrp && ptr && group_touches(reinterpret_cast<uintptr_t>(ptr), bytes, true)) {
    if (int rc = group_flush()) return rc;
    launched = 1;
  }
  if (g_def.empty() || !ptr) return launched;
  const uintptr_t p = reinterpret_cast<uintptr_t>(ptr);
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
  if (g_ngrp && ptr && group_touches(reinterpret_cast<uintptr_t>(ptr), bytes, false))
    if (int rc = group_flush()) return rc;
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
  if (int rc = group_flush()) return rc;
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
  if (int rc = group_flush()) return rc;
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

extern "C" int madi_set_gemm_grouping(int on) {
  if (!on && initialized())
    if (int rc = group_flush()) return rc;
  g_grouping = on != 0;
  return MADI_OK;
}

extern "C" int madi_set_deferred_dequant(int on) {
  if (initialized())
    if (int rc = group_flush()) return rc;
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
