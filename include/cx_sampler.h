/*
 * cx_sampler.h -- C-ABI of the MI355X (gfx950) token-sampling library.
 *
 * The reference exposes these operations as Python methods only; each entry
 * point below names the reference code it replaces.  Plain pointers and
 * sizes, no framework types.  Device entry points take device pointers and
 * a hipStream_t (passed as void*), never synchronise and never allocate;
 * the "_host" variants take host memory, run on an internal stream and
 * return when the results are on the host.
 *
 * Return value: 0 on success; CX_EINVAL (-1) for bad arguments, CX_EHIP (-2)
 * for a HIP runtime error, CX_ENOSPACE (-3) when the workspace is too small.
 * cx_last_error() gives a thread-local message for the last failure.
 *
 * Per-row outcomes are reported in row_status (CX_ROW_*), mirroring the
 * reference's control flow: which rows consumed their uniform, which fell
 * back to argmax, and which would have raised ValueError in numpy.
 */
#ifndef CX_SAMPLER_H
#define CX_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CX_OK        0
#define CX_EINVAL   (-1)
#define CX_EHIP     (-2)
#define CX_ENOSPACE (-3)

/* row_status low byte: outcome */
#define CX_ROW_OK          0  /* stochastic draw; consumed its uniform          (sampler.py:127) */
#define CX_ROW_GREEDY      1  /* T == 0: argmax of penalised logits              (sampler.py:114-115) */
#define CX_ROW_ARGMAX      2  /* filtered mass <= 0: argmax of penalised logits  (sampler.py:123-125) */
#define CX_ROW_ERROR       3  /* reference raises ValueError (NaN probabilities in choice) */
#define CX_ROW_UNSUPPORTED 4  /* input outside the library's limits (history window) */
/* row_status high bits: how the row was computed (informational) */
#define CX_ROW_FLAG_SLOW   0x100  /* resolved by the exact multi-pass row path */
#define CX_ROW_FLAG_DEEP   0x400  /* with CX_ROW_FLAG_SLOW: by its three-pass deep-nucleus variant */
#define CX_ROW_FLAG_EXACT  0x200  /* normaliser recomputed in fp64 for a near-threshold decision */

/* Per-row sampling parameters, 64 bytes.  Mirrors SamplingParams
 * (sampler.py:23-35) plus presence/frequency penalties, which the reference
 * lacks (0 = off; with both 0 the result is the reference's).  The doubles
 * are Python floats: they must not be rounded to fp32. */
typedef struct cx_row_params {
  double temperature;        /* 0 => greedy                                   */
  double top_p;              /* 1 => off                                      */
  double min_p;              /* 0 => off                                      */
  double typical_p;          /* 1 => off                                      */
  double repetition_penalty; /* 1 => off                                      */
  double presence_penalty;   /* 0 => off; subtracted once per id seen         */
  double frequency_penalty;  /* 0 => off; subtracted once per occurrence      */
  int32_t top_k;             /* 0 => off                                      */
  int32_t n_keep;            /* >0: penalty window = last max(64, n_keep) ids */
} cx_row_params;

/*
 * Sampler.sample for a batch of rows (sampler.py:108-127, with
 * apply_penalties :63-73 and _truncate :75-106).  Replaces a per-row loop of
 * `Sampler.sample(logits[b], params[b], generated_ids[b])` (engine.py:165,
 * speculative.py:126,171, scheduler.py:61).
 *
 *  logits    [B, ld] fp32 (cx_sample_f32) or bf16 bit patterns (cx_sample_bf16);
 *            row b holds V logits.  Never written.
 *  hist      [B, ldh] int32 token ids (generated_ids); hist_len[b] of them are
 *            used; ids outside [0, V) are ignored (sampler.py:68).  May be
 *            NULL when ldh == 0.
 *  prm       [B] cx_row_params
 *  u         [B] fp64 uniforms in [0, 1): the variate numpy's
 *            Generator.choice would draw (rows that do not draw ignore it).
 *  out_id    [B] int32 sampled ids
 *  row_status[B] int32 CX_ROW_* outcome | flags
 *  out_probs [B, V] fp32 post-filter normalised probabilities, or NULL.
 *            Costs one extra write of the batch; for verification.
 *  workspace device scratch of cx_sample_workspace_bytes(B, V, ldh) bytes;
 *            needs no initial contents (every call writes what it reads
 *            there before reading it).  One workspace per stream.
 */
int cx_sample_f32(const float* logits, int64_t ld, int32_t B, int32_t V,
                  const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                  const cx_row_params* prm, const double* u,
                  int32_t* out_id, int32_t* row_status, float* out_probs,
                  void* workspace, size_t ws_bytes, void* stream);

int cx_sample_bf16(const uint16_t* logits, int64_t ld, int32_t B, int32_t V,
                   const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                   const cx_row_params* prm, const double* u,
                   int32_t* out_id, int32_t* row_status, float* out_probs,
                   void* workspace, size_t ws_bytes, void* stream);

/* fp64 logits (the reference's Sampler.sample takes any float row; its model
 * produces fp32).  Same contract as cx_sample_f32; every row runs the exact
 * multi-pass fp64 path (slower than the fused fp32 / bf16 kernel). */
int cx_sample_f64(const double* logits, int64_t ld, int32_t B, int32_t V,
                  const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                  const cx_row_params* prm, const double* u,
                  int32_t* out_id, int32_t* row_status, float* out_probs,
                  void* workspace, size_t ws_bytes, void* stream);

size_t cx_sample_workspace_bytes(int32_t B, int32_t V, int64_t ldh);

/*
 * cx_sample_f32 without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference, which
 * has no device code.  It allocates nothing: its workspace is a static
 * device array of 64 MiB (CX_NOALLOC_SCRATCH_BYTES) that each GPU the
 * library runs on holds until the process ends.  Inputs, outputs, results
 * and errors are cx_sample_f32's; a batch whose workspace
 * (cx_sample_workspace_bytes) exceeds the scratch returns CX_EINVAL before
 * any device work.  Every call on one GPU shares that GPU's scratch: calls
 * that overlap on one GPU (on different streams or threads) race and must
 * be serialised by the caller.  No state carries from one call to the next.
 */
#define CX_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int cx_sample_f32_noalloc(const float* logits, int64_t ld, int32_t B, int32_t V,
                          const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                          const cx_row_params* prm, const double* u,
                          int32_t* out_id, int32_t* row_status, float* out_probs,
                          void* stream);


/* Host-memory variants: same arguments on host memory; allocate, copy,
 * launch, copy back and synchronise.  dtype: 0 = fp32, 1 = bf16, 2 = fp64. */
int cx_sample_host(const void* logits, int32_t dtype, int64_t ld, int32_t B, int32_t V,
                   const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                   const cx_row_params* prm, const double* u,
                   int32_t* out_id, int32_t* row_status, float* out_probs);

/*
 * Sampler.apply_penalties (sampler.py:63-73) for a batch of rows: out[b] is
 * float64(logits[b]) with the repetition penalty (x / rp if x > 0 else
 * x * rp, once per distinct in-range id of the window) and then the
 * presence / frequency penalties applied.  The window and id filtering are
 * those of cx_sample_f32.  Never writes the logits.
 *
 *  logits     [B, ld] of dtype 0 = fp32, 1 = bf16 bit patterns, 2 = fp64
 *  out        [B, ldo] fp64
 *  row_status [B] CX_ROW_OK, or CX_ROW_UNSUPPORTED when the row's window is
 *             longer than 4095 ids (out[b] is then not written)
 * No workspace; stream-ordered, never synchronises.
 */
int cx_apply_penalties(const void* logits, int32_t dtype, int64_t ld, int32_t B, int32_t V,
                       const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                       const cx_row_params* prm, double* out, int64_t ldo,
                       int32_t* row_status, void* stream);

int cx_apply_penalties_host(const void* logits, int32_t dtype, int64_t ld, int32_t B, int32_t V,
                            const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                            const cx_row_params* prm, double* out, int32_t* row_status);

/*
 * Sampler._truncate (sampler.py:75-106) for a batch of rows of fp64
 * probabilities: top-k (ties kept), top-p, min-p and typical-p on the
 * values as given (not renormalised, as the reference does), in that order.
 * out[b, i] = probs[b, i] where kept, else 0.  Equal values are ordered by
 * ascending id in the top-p and typical orders (numpy's argsort leaves that
 * order unspecified).  Uses temperature-independent fields of prm only.
 *
 *  row_status [B] CX_ROW_OK, or CX_ROW_ERROR for a row holding NaN or a
 *             negative value (out[b] is then not written)
 * No workspace; stream-ordered, never synchronises.
 */
int cx_truncate_f64(const double* probs, int64_t ld, int32_t B, int32_t V,
                    const cx_row_params* prm, double* out, int64_t ldo,
                    int32_t* row_status, void* stream);

int cx_truncate_host(const double* probs, int64_t ld, int32_t B, int32_t V,
                     const cx_row_params* prm, double* out, int32_t* row_status);

/*
 * Speculative-decoding verify step (speculative.py:145-171, with _softmax
 * :67-69) for B sequences at once.  Replaces the inline loop of
 * SpeculativeDecoder.generate.  All gamma positions are evaluated in parallel;
 * the result is what the reference's serial loop returns.
 *
 *  target     [B, gamma+1, V] fp32 target logits (row gamma = bonus row)
 *  draft      [B, gamma, V] fp32 draft logits (q rows); may be NULL if every
 *             temperature is 0
 *  draft_ids  [B, gamma] int32 proposed tokens
 *  u          [B, gamma+1] fp64: the verify generator's next gamma+1 variates
 *  temperature[B] fp32 (0 = greedy); the reference divides the fp32 row by
 *             fp32(T)
 *  accepted   [B] int32 accepted draft tokens
 *  next_tok   [B] int32 correction token, argmax of the bonus row (greedy),
 *             or -1 when every draft token was accepted in stochastic mode
 *             (the caller samples row gamma with the full sampler, :171)
 *  used       [B] int32 number of uniforms the reference would have consumed
 *  row_status [B] int32 CX_ROW_* flags
 *  workspace  device scratch of cx_spec_verify_workspace_bytes(B, gamma, V)
 *             bytes; any contents (every call writes what it reads).  One
 *             workspace per stream.
 */
int cx_spec_verify_f32(const float* target, const float* draft, const int32_t* draft_ids,
                       const double* u, const float* temperature,
                       int32_t B, int32_t gamma, int32_t V,
                       int32_t* accepted, int32_t* next_tok, int32_t* used,
                       int32_t* row_status, void* workspace, size_t ws_bytes, void* stream);

size_t cx_spec_verify_workspace_bytes(int32_t B, int32_t gamma, int32_t V);

int cx_spec_verify_host(const float* target, const float* draft, const int32_t* draft_ids,
                        const double* u, const float* temperature,
                        int32_t B, int32_t gamma, int32_t V,
                        int32_t* accepted, int32_t* next_tok, int32_t* used,
                        int32_t* row_status);

/*
 * LM-head projection with the greedy draw fused (transformer.py:102-104,
 * logits = h @ out_w.T, then sampler.py:114-115, argmax of the row, for a
 * greedy request with no penalty): the [B, V] logits never reach HBM.
 * bf16 operands, fp32 accumulation on MFMA.
 *
 *  hidden     [B, ldh] bf16 bits: the final-normed hidden states
 *  weight     [V, ldw] bf16 bits: the head weights (out_w, or the tied
 *             token embedding)
 *  D          hidden size, a multiple of 128; rows 16-byte aligned
 *  out_id     [B] int32: the first index of the row maximum, or of the
 *             first NaN (numpy's argmax)
 *  out_max    nullable [B] fp32: that logit
 *  out_logits nullable [B, V] fp32: every logit (verification only; this
 *             write is what the fusion saves)
 *  workspace  device scratch of cx_lmhead_workspace_bytes(B, V) bytes; any
 *             contents.
 * Device pointers, stream-ordered, no synchronisation, no allocation.
 */
int cx_lmhead_argmax_bf16(const uint16_t* hidden, int64_t ldh, const uint16_t* weight,
                          int64_t ldw, int32_t B, int32_t D, int32_t V, int32_t* out_id,
                          float* out_max, float* out_logits, void* workspace, size_t ws_bytes,
                          void* stream);

size_t cx_lmhead_workspace_bytes(int32_t B, int32_t V);

/* Kernel timing (measurement only).  While enabled, every library kernel is
 * dispatched with a start / stop event pair recorded by the dispatch itself
 * (hipExtLaunchKernel): the kernel's execution interval on its stream.
 * cx_timing_read waits for the recorded events, returns the summed
 * milliseconds and launch count of one kernel kind and forgets its records.
 * No counterpart in the reference (which has no device code); callers are
 * benchmarks and profilers. */
#define CX_KERNEL_SAMPLE        0  /* fused sampler kernel            */
#define CX_KERNEL_SAMPLE_SLOW   1  /* region finisher / exact row kernel */
#define CX_KERNEL_VERIFY_STATS  2  /* verify: stats over all rows     */
#define CX_KERNEL_VERIFY_REST   3  /* verify: decide + residual draw  */
#define CX_KERNEL_SAMPLE_FINISH 4  /* reserved: no longer launched (the region
                                      finisher runs in CX_KERNEL_SAMPLE_SLOW) */
#define CX_KERNEL_PENALTIES     5  /* apply_penalties                 */
#define CX_KERNEL_TRUNCATE      6  /* _truncate                       */
#define CX_KERNEL_LMHEAD        7  /* LM head: projection tiles + argmax keys */
#define CX_KERNEL_LMHEAD_MERGE  8  /* LM head: per-row merge of the keys */
#define CX_KERNEL_KINDS         9
int cx_timing_enable(int on);
int cx_timing_read(int32_t kernel, double* total_ms, int64_t* launches);

/* Thread-local description of the last failure ("" if none). */
const char* cx_last_error(void);

/* Library version string. */
const char* cx_version(void);

#ifdef __cplusplus
}
#endif
#endif /* CX_SAMPLER_H */
