/*
 * madi_q8.h -- C ABI of the MI355X (gfx950) Q8 matmul path.
 *
 * Drop-in for the Whisper large-v3-turbo engine's Q8 matmul operators.  The
 * engine's Zig operator wrappers keep their signatures and lower to these
 * entry points instead of the Metal bridge (engine/metal/metal_backend.h).
 * Every entry point takes plain pointers and sizes, returns 0 on success or a
 * negative MADI_ERR_* code, and records a message for madi_last_error().
 *
 * Memory: madi_alloc returns DEVICE memory (HBM).  Unlike Metal's unified
 * buffers it is not host-addressable: the host fills it with madi_upload and
 * reads it with madi_download.  All op pointers are device pointers.
 *
 * Ordering: every op is enqueued on one HIP stream (the null stream unless
 * madi_set_stream chose another) and runs in call order; nothing blocks until
 * madi_sync.  Like the Metal bridge, the library keeps one global queue and
 * expects calls from one host thread at a time.
 *
 * ---------------------------------------------------------------------------
 * Q8 weights.  A Q8_0 weight W[N][K] (K % 32 == 0) is int8 quants plus one
 * fp16 scale per 32-element K block: w[n][k] = q[n][k] * s[n][k/32]
 * (engine/metal/encoder.zig:21, decoder.zig:22).  The reference stores them
 * row-major ("natural": qs[n*K+k], scales[n*(K/32)+k/32]).
 *
 * The loader repacks them once (madi_q8_repack / madi_q8_repack_host) into
 * the CDNA4 PANEL layout that every op below reads.  Requires K % 64 == 0.
 *   panel p      = rows [32p, 32p+R), R = min(32, N-32p)
 *   qs   bytes   : panel p starts at byte 32*p*K (same offset as natural), then
 *                  chunk c (k in [64c, 64c+64)) at c*R*64, then the 16-byte
 *                  unit (j, h, r) at ((2j+h)*R + r)*16 holding
 *                  q[32p+r][64c+32h+16j+i] + 128 (uint8), i = 0..15
 *   scales fp16  : panel p starts at element 32*p*(K/32) (same offset as
 *                  natural), chunk c at c*2R, element (h, r) at h*R + r holding
 *                  s[32p+r][2c+h]
 * Buffer sizes are unchanged (N*K bytes, N*K/32 scales) and every panel keeps
 * its natural offset, so the engine's row slicing of stacked weights
 * (qs + D*D, scales + D*(D/32); engine/metal/encoder.zig:263-267) stays valid
 * at any row offset that is a multiple of 32.  For a full panel the 1 KiB
 * half-chunk j is exactly one wave64 load of 16 bytes per lane, lane = 32h+r,
 * and lane (h, r) holds the 32 weights of ONE quantisation block.
 * ---------------------------------------------------------------------------
 */
#ifndef MADI_Q8_H
#define MADI_Q8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes.  The reference bridge returns 0 / -1 (metal_backend.h:14-46)
 * and the Zig wrapper maps failures to error{InitFailed, LibraryLoadFailed,
 * FunctionNotFound, AllocFailed, DispatchFailed, SyncFailed}
 * (engine/metal/metal_backend.zig:34-41); the codes below refine -1. */
#define MADI_OK 0
#define MADI_ERR_INIT (-1)      /* InitFailed: no gfx950 device / HIP init error   */
#define MADI_ERR_ALLOC (-2)     /* AllocFailed                                      */
#define MADI_ERR_DISPATCH (-3)  /* DispatchFailed: kernel launch failed             */
#define MADI_ERR_SYNC (-4)      /* SyncFailed: stream sync reported an error        */
#define MADI_ERR_SHAPE (-5)     /* unsupported shape (K % 64, zero sizes, ...)      */
#define MADI_ERR_NULL (-6)      /* required pointer is NULL                         */
#define MADI_ERR_ALIGN (-7)     /* pointer not aligned as the op requires           */
#define MADI_ERR_NOT_INIT (-8)  /* madi_init has not succeeded                      */
#define MADI_ERR_ARG (-9)       /* bad enum / argument value                        */

/* Epilogues of the fused GEMM / GEMV ops. */
#define MADI_EPI_NONE 0      /* out = acc                                          */
#define MADI_EPI_BIAS 1      /* out = acc + bias[n]                                */
#define MADI_EPI_BIAS_GELU 2 /* out = gelu_erf(acc + bias[n])                      */
#define MADI_EPI_BIAS_RES 3  /* out[n] = out[n] + acc + bias[n]  (GEMV only)       */

/* ---- runtime ------------------------------------------------------------ */
/* replaces mtl_init (metal_backend.h:15): selects device 0, checks gfx950. */
int madi_init(void);
/* replaces mtl_cleanup (metal_backend.h:16). */
void madi_cleanup(void);
/* replaces mtl_alloc (metal_backend.h:21): device memory, 256-byte aligned,
 * NULL on failure. */
void *madi_alloc(size_t size);
/* replaces mtl_free (metal_backend.h:22). */
void madi_free(void *ptr);
/* replace mtl_upload / mtl_download (metal_backend.h:29-30): blocking copies
 * host <-> device, ordered after previously enqueued ops. */
int madi_upload(void *dst_device, const void *src_host, size_t size);
int madi_download(void *dst_host, const void *src_device, size_t size);
/* replace mtl_begin_command_buffer / mtl_commit_command_buffer / mtl_sync
 * (metal_backend.h:62-69).  HIP launches are already queued asynchronously, so
 * begin and commit only check state; sync waits for the stream. */
int madi_begin_command_buffer(void);
int madi_commit_command_buffer(void);
int madi_sync(void);
/* No reference counterpart: lets a host that owns a HIP stream (hipStream_t
 * passed as void*) order this library's launches on it.  NULL = null stream.
 * The new stream first waits (on the device, the host does not block) for
 * the work already issued on the old one, so the library's launches stay in
 * call order across the switch.  Where either stream is under graph capture
 * no such wait is added (a capture may not wait on outside work): the caller
 * orders the two streams, e.g. synchronises before capturing. */
int madi_set_stream(void *hip_stream);
/* Message of the last failure on the calling thread ("" if none). */
const char *madi_last_error(void);
/* Number of compute units of the current device (0 before madi_init). */
int madi_device_cu_count(void);

/* ---- Q8 layout (load time) ------------------------------------------------ */
/* Natural -> panel layout, host memory to host memory.  Replaces nothing in
 * the reference directly: it runs where the loader has just produced or read
 * the Q8 rows (transcribe.zig:235-263 upVecQ8, :309-341 quantInto/readQ8,
 * :377-410 upMatQ8/upQKVQ8enc, :434-465 upQKVQ8).  Needs no GPU. */
int madi_q8_repack_host(void *dst_qs, void *dst_scales, const void *qs,
                        const void *scales, uint32_t n, uint32_t k);
/* Panel -> natural layout, host to host (inverse of madi_q8_repack_host). */
int madi_q8_unpack_host(void *dst_qs, void *dst_scales, const void *tiled_qs,
                        const void *tiled_scales, uint32_t n, uint32_t k);
/* Natural -> panel layout, device to device (src and dst must not overlap). */
int madi_q8_repack(void *dst_qs, void *dst_scales, const void *qs, const void *scales,
                   uint32_t n, uint32_t k);

/* F16 [N][K] (natural, device) -> panel-layout Q8 (device), the loader's
 * quantisation done on the GPU: per 32-block scale = max|w| / 127 (1.0 for an
 * all-zero block) stored as f16, q = clamp(round_half_away(w * (1 / scale)), +-127),
 * bit-identical to quantInto (transcribe.zig:309-326) followed by the repack.
 * w must be 16-byte aligned. */
int madi_q8_quantize(void *dst_qs, void *dst_scales, const void *w_f16, uint32_t n, uint32_t k);
/* The WHASH weight identity: fnvQ8 (transcribe.zig:131-140), FNV-1a 64 over a
 * NATURAL-layout weight's qs bytes (nq of them) then its nsc fp16 scales'
 * bytes, continuing from `seed` (0xcbf29ce484222325 to start).  Host memory. */
uint64_t madi_q8_fnv(uint64_t seed, const void *qs, size_t nq, const void *scales, size_t nsc);

/* ---- ops (device pointers, panel-layout weights) ---------------------------- */
/* Q8 -> F16 [K][N] transposed dequant, bit-exact fp16_rne(q * s).  Replaces
 * kDeq (engine/metal/encoder.zig:154-159) and deqW16 (transcribe.zig:4387-4393),
 * kernel dequant_q8_f16 (engine/metal/kernels/q8_gemm.metal:12-27).  Deferred
 * by default: see "Deferred dequantisation" below. */
int madi_q8_dequant_f16(void *wdq, const void *qs, const void *scales, uint32_t n,
                        uint32_t k);

/* Fused Q8 GEMM: C[M][N] (f16) = epi(A[M][K] (f16) . deq(W)^T), fp32 accumulate.
 * Argument order of m4_gemm_q8_bias_gelu (engine/metal/kernels/m4_gemm.metal:131-141);
 * replaces the encoder's kDeq + kM4 / kM4Bias pairs (encoder.zig:125-136,
 * 262-301) and mul_mm_q8 (q8_gemm.metal:29-102).  epilogue: NONE, BIAS or
 * BIAS_GELU (bias may be NULL for NONE).  Requires N % 32 == 0, K % 64 == 0,
 * 16-byte aligned A and C. */
int madi_q8_gemm(const void *a, const void *qs, const void *scales, void *c,
                 const float *bias, uint32_t m, uint32_t n, uint32_t k, int epilogue);

/* No counterpart in the reference: madi_q8_gemm for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * madi_q8_gemm, bit for bit; where a shape splits K over workgroups, the
 * partial sums and arrival counters live in a fixed 16 MiB device array of
 * the library (MADI_Q8_GEMM_NOALLOC_SCRATCH bytes per GPU, held until the
 * process ends) instead of the growable workspace, so the call allocates
 * nothing.  Every split shape of madi_q8_gemm fits (at most 15 MiB of
 * partials); a larger need fails with MADI_ERR_SHAPE.  All calls on one GPU
 * share that GPU's array: calls that overlap on one GPU (several streams or
 * host threads) race and must not. */
#define MADI_Q8_GEMM_NOALLOC_SCRATCH (16u << 20)
int madi_q8_gemm_noalloc(const void *a, const void *qs, const void *scales, void *c,
                         const float *bias, uint32_t m, uint32_t n, uint32_t k, int epilogue);

/* Decoder GEMVs, x f32 [K] -> out f32 [N] (M = 1).  Argument order of the Zig
 * wrappers (engine/metal/decoder.zig:155-181) with the Q8w struct spelled out as
 * (qs, scales):
 *   madi_q8_gemv            kGemvQ8          -> gemv_q8            graph_helpers.metal:390-419
 *   madi_q8_gemv_bias       kGemvQ8Bias      -> gemv_q8_bias       graph_helpers.metal:424-451
 *   madi_q8_gemv_bias_gelu  kGemvQ8BiasEpi   -> gemv_q8_bias_gelu  graph_helpers.metal:475-496
 *   madi_q8_gemv_bias_res   kGemvQ8BiasEpi   -> gemv_q8_bias_res   graph_helpers.metal:498-519
 * x must be 16-byte aligned; out may not alias x. */
int madi_q8_gemv(float *out, const float *x, const void *qs, const void *scales,
                 uint32_t n, uint32_t k);
int madi_q8_gemv_bias(float *out, const float *x, const void *qs, const void *scales,
                      const float *bias, uint32_t n, uint32_t k);
int madi_q8_gemv_bias_gelu(float *out, const float *x, const void *qs, const void *scales,
                           const float *bias, uint32_t n, uint32_t k);
int madi_q8_gemv_bias_res(float *out, const float *x, const void *qs, const void *scales,
                          const float *bias, uint32_t n, uint32_t k);
/* Fused self-attention QKV: stacked [3D][D] weight, q_out = acc + qb, k -> kc[pos],
 * v + vb -> vc[pos] with pos read on the device from *pos.  Replaces kQkv
 * (decoder.zig:169-174) -> gemv_q8_qkv (graph_helpers.metal:527-558). */
int madi_q8_gemv_qkv(float *q_out, const float *x, const void *qs, const void *scales,
                     const float *qb, const float *vb, float *kc, float *vc,
                     const uint32_t *pos, uint32_t d);
/* Vocab logits over the tied Q8 embedding.  Replaces kLogitGemv
 * (transcribe.zig:4369-4374) -> logit_gemv_q8 (graph_helpers.metal:320-351). */
int madi_q8_logit_gemv(float *logits, const void *qs, const void *scales, const float *x,
                       uint32_t vocab, uint32_t dim);
/* GEMV with fp16 activations x [K] (the measured configuration: fp16 A,
 * fp32 out).  epilogue: NONE, BIAS, BIAS_GELU or BIAS_RES.  No reference
 * counterpart with this dtype; same arithmetic as madi_q8_gemv. */
int madi_q8_gemv_f16x(float *out, const void *x_f16, const void *qs, const void *scales,
                      const float *bias, uint32_t n, uint32_t k, int epilogue);

/* Batched / skinny projection: out[M][N] (f32) = in[M][K] (f32) . deq(W)^T for
 * any M: a few token rows (the batched-decode GEMV, 32 rows per pass over W)
 * or, from 160 rows on weights 2048 or more wide or 4096 or more long, or
 * where the row count would need more workgroups than CUs, the MFMA GEMM with
 * f32 operands (sequence prefill); the same arithmetic either way.
 * Replaces pproj (engine/metal/decoder.zig:427-432: kDeq + kCvt32 +
 * matmulF16Batched + kCvt16) and the per-slot proj calls of the batched
 * decode (decoder.zig:337-341) with one fused kernel: activations rounded to
 * f16 and weights to fp16_rne(q * s) as that pipeline does, fp32
 * accumulation, f32 result (the pipeline's f16 output staging is not
 * repeated).  in must be 16-byte aligned; out may not alias in. */
int madi_q8_pproj(float *out, const float *in, const void *qs, const void *scales,
                  uint32_t m, uint32_t n, uint32_t k);

/* ---- kernel handles and the engine's handle-taking wrappers ---------------- */
/* Handle for one of this path's kernel names (replaces mtl_get_function,
 * metal_backend.h:46, behind mtl.getFunction, metal_backend.zig:61-65):
 * "dequant_q8_f16", "m4_gemm_nn", "m4_gemm_bias", "m4_gemm_bias_gelu",
 * "gemv_q8", "gemv_q8_bias", "gemv_q8_bias_gelu", "gemv_q8_bias_res",
 * "gemv_q8_qkv", "logit_gemv_q8", "gpu_emb_lookup_q8",
 * "emb_lookup_indirect_q8", "emb_pe_rows_q8", "mul_mm_q8", and the
 * encoder attention kernels "m4_flash_enc" and "flash_attention_enc_f16"
 * (both run madi_flash_enc_f16).  Another name fails with MADI_ERR_ARG
 * (FunctionNotFound).  Needs no device. */
int madi_get_function(const char *name, int *out_id);
/* kM4 / kM4Bias (engine/metal/encoder.zig:125-136) with the handle the engine
 * resolved: m4_gemm_nn (bias ignored), m4_gemm_bias or m4_gemm_bias_gelu, on
 * an F16 weight b [K][N]; same as madi_f16_gemm with that epilogue. */
int madi_m4_gemm(int func, const void *a, const void *b, void *c, const float *bias, uint32_t m,
                 uint32_t n, uint32_t k);
/* kGemvQ8BiasEpi (engine/metal/decoder.zig:176-181) with its handle:
 * gemv_q8_bias_gelu or gemv_q8_bias_res (or gemv_q8_bias). */
int madi_q8_gemv_epi(int func, float *out, const float *x, const void *qs, const void *scales,
                     const float *bias, uint32_t n, uint32_t k);
/* proj (engine/metal/decoder.zig:337-341): out[B][N] (f32) = in[B][K] (f32)
 * . w16, w16 the F16 [K][N] copy deqW16 made of a Q8 weight.  A recorded
 * copy (below) runs madi_q8_pproj on the Q8 weight; a true F16 weight is
 * staged to f16 in stage16 ([B][K] f16, the BScratch in16 buffer) and
 * multiplied by the NN f16 GEMM with an f32 result (rocBLAS for shapes it
 * does not take). */
int madi_proj_f16w(float *out, const float *in, const void *w16, void *stage16, uint32_t m,
                   uint32_t n, uint32_t k);

/* Deferred dequantisation.  madi_q8_dequant_f16 (kDeq, deqW16) records
 * (wdq -> Q8 weight) instead of writing wdq.  madi_f16_gemm, madi_m4_gemm,
 * madi_matmul_f16 (alpha 1, beta 0) and madi_proj_f16w whose F16 weight is
 * exactly a recorded wdq of the recorded shape run the fused Q8 kernels on
 * the Q8 weight, so the encoder's kDeq + kM4 / kM4Bias pairs
 * (encoder.zig:262-301) and the batched decoder's deqW16 + proj need no
 * change to run them.  wdq is written ("materialised") before anything in
 * this library could observe it: another op reading it, madi_download of it,
 * a write into or madi_free of the Q8 source, a partial overwrite of wdq; a
 * full overwrite or madi_free of wdq drops the record.  Kernels outside this
 * library that read wdq need madi_q8_materialize(wdq) first (NULL: every
 * record).  Code outside this library that WRITES into a recorded wdq or into
 * its Q8 source (an engine kernel, hipMemcpy, a torch copy) calls
 * madi_q8_forget(ptr, bytes) on the range first: a record whose wdq the range
 * covers entirely is dropped, one whose wdq it covers in part or whose Q8
 * source it touches is materialised (so wdq keeps the weights it was made
 * from).  Without that call a later F16 GEMM on wdq would run the fused kernel
 * on the recorded Q8 weight and a later materialisation would read the
 * changed source.  madi_set_deferred_dequant(0) materialises every record and
 * makes madi_q8_dequant_f16 write wdq at once (the default is 1).  No
 * counterpart in the reference (Metal's kDeq writes wdq at once). */
int madi_q8_materialize(void *wdq);
int madi_q8_forget(void *ptr, size_t bytes);
int madi_set_deferred_dequant(int on);

/* q|k|v grouping.  The encoder computes q, k and v as three F16 GEMMs on the
 * same activations, each on a kDeq of the next 1280-row slice of the stacked
 * q|k|v weight (encoder.zig:262-267).  With grouping on (the default), an
 * F16 GEMM that runs the fused Q8 kernel on the FIRST slice of a stacked
 * weight (its Q8 source at the start of a madi_alloc allocation holding at
 * least three such slices) is held; the GEMMs on the following slices with
 * the same activations, shape and epilogue join it, and the three run as one
 * launch of the stacked GEMM writing the three outputs once the last slice
 * arrives (the allocation's end or the third).  Any library call that reads
 * a held output or writes a held operand, madi_sync, madi_commit_command_buffer,
 * madi_set_stream and madi_q8_materialize launch a held group first.  Code
 * outside this library that reads q or k before the v GEMM has been issued
 * calls madi_sync first, or turns grouping off with madi_set_gemm_grouping(0)
 * (which launches a held group).  No counterpart in the reference. */
int madi_set_gemm_grouping(int on);

/* ---- fp16 GEMMs (pre-dequantised F16 weights) ------------------------------ */
/* C[M][N] (f16) = epi(A[M][K] (f16) . B[K][N] (f16)), all row-major, fp32
 * accumulation.  Replaces kM4 / kM4Bias (engine/metal/encoder.zig:125-136) ->
 * m4_gemm_nn / m4_gemm_bias / m4_gemm_bias_gelu (kernels/m4_gemm.metal:19-115)
 * for callers that hold an F16 weight in the [K][N] layout kDeq produces.
 * Epilogues round like the reference: c = f16(A.B), then f16(c + bias[n]) and
 * for BIAS_GELU f16(gelu(c + bias[n])).  K a multiple of 64, N of 128 and
 * 16-byte aligned a, b, c and bias run the library's NN f16 GEMM (epilogue in
 * the kernel); other shapes run rocBLAS and an elementwise epilogue pass. */
int madi_f16_gemm(const void *a, const void *b, void *c, const float *bias, uint32_t m,
                  uint32_t n, uint32_t k, int epilogue);
/* C = alpha * A . B + beta * C, f16 row-major [M][K] . [K][N] -> [M][N], fp32
 * accumulation.  Replaces mtl_matmul_f16_enc (engine/metal/metal_backend.h:103),
 * behind matmulF16Batched (metal_backend.zig:120).  alpha 1 and beta 0 on the
 * shapes madi_f16_gemm's kernel takes run it; the rest run rocBLAS. */
int madi_matmul_f16(const void *a, const void *b, void *c, int m, int n, int k, float alpha,
                    float beta);

/* Q8 embedding rows from the panel layout (the tied tok_emb the logit GEMV
 * reads): out[d] = f32(q) * f32(s) for row *tok_ptr (gpu_emb_lookup_q8,
 * graph_helpers.metal:370-383) or row tokens[*pos_ptr]
 * (emb_lookup_indirect_q8, graph_helpers.metal:354-367).  The panel layout
 * needs the table's row count (`vocab`) to place its last, partial panel; a
 * token >= vocab writes nothing. */
int madi_q8_emb_lookup(float *out, const void *qs, const void *scales,
                       const uint32_t *tok_ptr, uint32_t vocab, uint32_t dim);
int madi_q8_emb_lookup_indirect(float *out, const void *qs, const void *scales,
                                const uint32_t *tokens, const uint32_t *pos_ptr,
                                uint32_t vocab, uint32_t dim);
/* Sequence prefill's embedding rows from the panel layout: out[m][d] =
 * f32(q) * f32(s) of row tokens[m] + pe[(pos0 + m) * dim + d] for m < M
 * (f32 out [M][dim], one rounding: the add).  Replaces emb_pe_rows_q8
 * (engine/metal/kernels/decoder_ops.metal:614-633) behind prefillEmbed
 * (engine/metal/decoder.zig:460-467), which reads the tied tok_emb.  pe must
 * hold rows up to pos0 + M - 1 (the caller's bound, as in the reference); a
 * token >= vocab leaves its row untouched.  out and pe 16-byte aligned. */
int madi_q8_emb_pe_rows(float *out, const void *qs, const void *scales, const uint32_t *tokens,
                        const float *pe, uint32_t dim, uint32_t pos0, uint32_t m, uint32_t vocab);

/* ---- encoder self-attention over the projections ------------------------------ */
/* m4_flash_enc (engine/metal/kernels/m4_gemm.metal:268-407; buffers 0-5 in this
 * order), which kFlash (engine/metal/encoder.zig:138-152) dispatches once per
 * window on the Q, K, V projections: bidirectional attention with head dim 64,
 * out = softmax(q k^T / 8) v per head, in the reference's arithmetic (f32
 * scores, an online softmax over 64-key blocks, f16 P, f32 sums, out =
 * f16(O / (sum + 1e-6))).  q, k, v, out: f16 [seq_len][nh*64], head h in
 * columns 64h..64h+63.  Unlike the reference kernel, q/k/v need no padding
 * rows past seq_len.  All four 16-byte aligned; out must not overlap k or v
 * (out == q is allowed: each query row is read before its output is
 * written); seq_len = 0 does nothing; seq_len * nh * 128 <= 2 GiB. */
int madi_flash_enc_f16(void *out, const void *q, const void *k, const void *v, uint32_t seq_len,
                       uint32_t nh);

#ifdef __cplusplus
}
#endif
#endif /* MADI_Q8_H */
