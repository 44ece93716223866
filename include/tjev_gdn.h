/* C ABI of the MI355X (gfx950) Gated DeltaNet megakernel library, libtjev_gdn.so.
 *
 * Drop-in for the two Pallas calls behind tjev's `gdn_megakernel`
 * (src/tjev/kernels/gated_delta_rule/pallas_tpu_mega.py:585-639): the forward kernel
 * `gdn_mega2_fwd` (:429-468) and the backward kernel `gdn_mega2_bwd` (:471-524) with the XLA
 * sums of `_core_bwd` (:554-572). The caller (a jax.ffi handler, ctypes, torch) passes plain
 * device pointers and the stream; every entry point is asynchronous on that stream, validates
 * its arguments before any launch and returns 0 or a nonzero tjev_gdn_status
 * (tjev_gdn_last_error() then describes it). No torch or HIP types appear here.
 *
 * Layouts (row-major, as the reference's arrays):
 *   qkv        [B, T, 2*Hk*Dk + H*Dv]  io_dtype   raw in_proj_qkv output (taps > 0, mega2)
 *                                                 or the post-conv activations (taps == 0, mega1)
 *   a, b       [B, T, H]               gate_dtype raw gate projections
 *   a_log      [H] fp32, dt_bias [H] fp32
 *   conv_w     [K, 2*Hk*Dk + H*Dv]     fp32       (K = taps; ignored when taps == 0)
 *   seg        [B, T] int32            segment ids, 0 = padding
 *   out        [B, T, H, Dv]           io_dtype
 *   residuals  tjev_gdn_residual_bytes(p) bytes, the forward's output for the backward,
 *              each part 256-byte aligned, in this order:
 *                states [B, H, ceil(T/C), Dk, Dv]  the state before each chunk (gdn_states):
 *                                                   fp32, or bf16 under TJEV_GDN_MIXED and
 *                                                   TJEV_GDN_ONE_PASS_BF16 (the reference's
 *                                                   _state_dtypes, pallas_tpu_mega.py:425-426)
 *                tinv   [B, H, ceil(T/C), C, C]    (I + L)^-1 of each chunk (gdn_tinv), fp32 (bf16
 *                                                   under TJEV_GDN_ONE_PASS_BF16), when
 *                                                   residuals >= TJEV_GDN_SAVE_TINV
 *                v_new  [B, H, ceil(T/C)*C, Dv]    fp32 u - w S of each token, when
 *                                                   residuals == TJEV_GDN_SAVE_ALL
 *              (C: the chunk the kernels run, min(max(chunk, 16), 128): chunk 8 runs the
 *              16-token kernels, chunks above 128 the 128-token ones)
 * T need not be a multiple of the chunk: the kernels pad the tail with zero q, k, v and beta,
 * g = 0 and the last token's segment id (xla.py:198-204), so the padding changes no output
 * (pallas_tpu_mega.py:616-621 pads with segment 0: the same outputs) and carries the state after
 * token T-1 unchanged to the end of the last chunk.
 */
#ifndef TJEV_GDN_H
#define TJEV_GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum tjev_gdn_dtype { TJEV_GDN_F32 = 0, TJEV_GDN_BF16 = 1 };

/* the reference's `precision` (xla.py:23): highest = fp32 products; high = bf16x3; bf16 = one
 * bf16 pass; mixed = bf16x3 intra-chunk products, one bf16 pass for products with the state */
enum tjev_gdn_precision {
  TJEV_GDN_HIGHEST = 0,
  TJEV_GDN_HIGH = 1,
  TJEV_GDN_ONE_PASS_BF16 = 2,
  TJEV_GDN_MIXED = 3
};

/* the reference's `inverse` (pallas_tpu_v2.py:141-193): (I + L)^-1 of each chunk by the pure
 * doubling from T = I, every level's products at the intra-chunk precision, or with its 16 x 16
 * diagonal blocks inverted exactly (forward substitution in fp32) before the doubling levels */
enum tjev_gdn_inverse { TJEV_GDN_DOUBLING = 0, TJEV_GDN_BLOCKED = 1 };

/* what the forward keeps for the backward (the reference's remat residual contract names
 * gdn_tinv and gdn_states, pallas_tpu_mega.py:543-548): the states only (the backward rebuilds
 * T and v_new: least memory), states and T (the reference's residuals: the backward rebuilds
 * v_new from T), or states, T and v_new (the backward rebuilds neither) */
enum tjev_gdn_residuals { TJEV_GDN_SAVE_STATES = 0, TJEV_GDN_SAVE_TINV = 1, TJEV_GDN_SAVE_ALL = 2 };

enum tjev_gdn_status {
  TJEV_GDN_OK = 0,
  TJEV_GDN_EINVAL = 1,       /* bad shape or parameter (the reference raises ValueError) */
  TJEV_GDN_EUNSUPPORTED = 2, /* valid for the reference, no kernel instantiated for it here */
  TJEV_GDN_EWORKSPACE = 3,   /* workspace missing or too small */
  TJEV_GDN_EHIP = 4          /* a HIP launch or runtime error */
};

typedef struct tjev_gdn_params {
  int32_t batch;          /* B */
  int32_t length;         /* T */
  int32_t key_heads;      /* Hk */
  int32_t key_dim;        /* Dk */
  int32_t value_heads;    /* H (a multiple of Hk) */
  int32_t value_dim;      /* Dv */
  int32_t taps;           /* conv taps K in 1..5 (mega2), 0 for mega1 (conv_weight=None) */
  int32_t chunk;          /* C, a power of two >= 8 */
  int32_t io_dtype;       /* tjev_gdn_dtype of qkv, out, d_out, d_qkv */
  int32_t gate_dtype;     /* tjev_gdn_dtype of a, b, d_a, d_b */
  int32_t precision;      /* tjev_gdn_precision */
  int32_t inverse;        /* tjev_gdn_inverse */
  int32_t heads_per_step; /* accepted for the reference's signature (0 = default) */
  int32_t residuals;      /* tjev_gdn_residuals */
  int32_t qk_dtype;       /* tjev_gdn_dtype of q, k, d_q, d_k (the v2 entry points only) */
} tjev_gdn_params;

/* 0 if the library has kernels for these parameters, else a status (and the message). */
int tjev_gdn_check(const tjev_gdn_params* p);

/* bytes of the states part of the residuals, of all the residuals p->residuals keeps, and of
 * the scratch the forward / backward need */
size_t tjev_gdn_states_bytes(const tjev_gdn_params* p);
size_t tjev_gdn_residual_bytes(const tjev_gdn_params* p);
size_t tjev_gdn_workspace_bytes(const tjev_gdn_params* p, int backward);

/* forward: replaces pallas_call "gdn_mega2_fwd" (pallas_tpu_mega.py:429-468), whose outputs are
 * out, tinv and states (:444-449); writes out and the residuals. `stream` is a hipStream_t. */
int tjev_gdn_mega2_fwd(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a,
                       const void* b, const float* a_log, const float* dt_bias,
                       const float* conv_w, const int32_t* seg, void* out, float* residuals,
                       void* workspace, size_t workspace_bytes);

/* the forward plus the state a decode step continues from (the serving prefill; no
 * counterpart in the megakernel, whose XLA sibling returns the final state,
 * xla.py:170-262): final_state [B, H, Dk, Dv] fp32, the recurrent state after token T-1
 * (xla.py:141-167 run to the last token: restarted where the segment id changes), and
 * conv_state [B, K-1, W] io_dtype, the raw rows T-K+1 .. T-1 (oldest first), zero before the
 * row or outside token T-1's segment. Either may be null; a conv of 0 or 1 taps has no history:
 * a non-null conv_state then returns TJEV_GDN_EINVAL. */
int tjev_gdn_mega2_fwd_state(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a,
                             const void* b, const float* a_log, const float* dt_bias,
                             const float* conv_w, const int32_t* seg, void* out, float* residuals,
                             float* final_state, void* conv_state, void* workspace,
                             size_t workspace_bytes);

/* A sequence continued from an earlier call (a long prompt prefilled in pieces, a prefill that
 * resumes a cached state): the chunked rule with an initial state (xla.py:170-262,
 * `initial_state`; test_gated_delta_rule.py:61-73), and the conv over the rows before token 0.
 * initial_state [B, H, Dk, Dv] fp32: the state before token 0, read by chunk 0's tokens of token
 * 0's segment (chunk 0's "token before" is token 0's id instead of -2, xla.py:214-216);
 * initial_conv [B, K-1, W] io_dtype: the raw rows before token 0, oldest first, read by the
 * conv of token 0's segment (as conv_state below returns them). Either may be null (a fresh
 * start: state 0; no rows before the row). final_state and conv_state as for
 * tjev_gdn_mega2_fwd_state (null: not written). With both inputs null this is
 * tjev_gdn_mega2_fwd_state. No counterpart in the megakernel, which starts every row fresh. */
int tjev_gdn_mega2_fwd_cont(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a,
                            const void* b, const float* a_log, const float* dt_bias,
                            const float* conv_w, const int32_t* seg, const float* initial_state,
                            const void* initial_conv, void* out, float* residuals,
                            float* final_state, void* conv_state, void* workspace,
                            size_t workspace_bytes);

/* tjev_gdn_mega2_fwd_cont followed by the gated RMSNorm of its output, replacing the pair of
 * calls GatedDeltaNet.__call__ makes (src/tjev/model/gdn.py:126-164: core_mega, then
 * GatedRMSNorm, src/tjev/model/norms.py:36-62) with the norm in the output kernel's epilogue:
 * y [B, T, H, Dv] io_dtype = weight * round(x rsqrt(mean x^2 + eps)) * silu(gate), x = out as
 * stored, 0 on padding tokens (seg <= 0) -- what tjev_gdn_gated_rmsnorm_fwd(out, gate, weight,
 * seg) writes, up to the summation order of mean x^2 (a rare last-bit difference). out is still
 * written (the norm's backward, tjev_gdn_gated_rmsnorm_bwd, reads it). gate [B, T, H, Dv]
 * io_dtype and y are 16-byte aligned; norm_weight [Dv] fp32; eps >= 0. */
int tjev_gdn_mega2_fwd_normed(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a,
                              const void* b, const float* a_log, const float* dt_bias,
                              const float* conv_w, const int32_t* seg, const float* initial_state,
                              const void* initial_conv, const void* gate, const float* norm_weight,
                              float eps, void* out, void* y, float* residuals, float* final_state,
                              void* conv_state, void* workspace, size_t workspace_bytes);

/* The backward of tjev_gdn_mega2_fwd_cont: initial_state and initial_conv as given to the forward
 * (initial_state's values are in the residuals; only whether it is null matters here);
 * d_final_state [B, H, Dk, Dv] fp32, the gradient of the forward's final_state (null: 0; any
 * length: the padded tail carries the state unchanged). Writes, beside
 * tjev_gdn_mega2_bwd's outputs, d_initial_state [B, H, Dk, Dv] fp32 and d_initial_conv
 * [B, K-1, W] io_dtype when not null (each needs its input). The gradient of the forward's
 * conv_state is that of rows of qkv or initial_conv: the caller adds it there. */
int tjev_gdn_mega2_bwd_cont(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a,
                            const void* b, const float* a_log, const float* dt_bias,
                            const float* conv_w, const int32_t* seg, const float* initial_state,
                            const void* initial_conv, const float* residuals, const void* d_out,
                            const float* d_final_state, void* d_qkv, void* d_a, void* d_b,
                            float* d_a_log, float* d_dt_bias, float* d_conv_w,
                            float* d_initial_state, void* d_initial_conv, void* workspace,
                            size_t workspace_bytes);

/* The backward of tjev_gdn_mega2_fwd_normed: the gated RMSNorm's backward (what
 * tjev_gdn_gated_rmsnorm_bwd computes from out, gate, norm_weight, seg and d_y: d out, d_gate and,
 * when not null, d_norm_weight [Dv] fp32), then tjev_gdn_mega2_bwd_cont's from that d out, in one
 * call on the caller's stream (the backward of GatedDeltaNet.__call__'s core and norm,
 * src/tjev/model/gdn.py:157-160). d out lives in the workspace, of
 * tjev_gdn_workspace_bytes_normed(p, d_norm_weight != null) bytes. out, gate, d_y and d_gate
 * [B, T, H, Dv] io_dtype, 16-byte aligned. */
size_t tjev_gdn_workspace_bytes_normed(const tjev_gdn_params* p, int norm_weight_grad);
int tjev_gdn_mega2_bwd_normed(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a,
                              const void* b, const float* a_log, const float* dt_bias,
                              const float* conv_w, const int32_t* seg, const float* initial_state,
                              const void* initial_conv, const float* residuals, const void* out,
                              const void* gate, const float* norm_weight, float eps,
                              const void* d_y, const float* d_final_state, void* d_qkv, void* d_a,
                              void* d_b, float* d_a_log, float* d_dt_bias, float* d_conv_w,
                              float* d_initial_state, void* d_initial_conv, void* d_gate,
                              float* d_norm_weight, void* workspace, size_t workspace_bytes);

/* tjev_gdn_mega2_fwd_cont without a workspace argument and without any allocation: no
 * counterpart in the reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops that prefill prompt pieces, harnesses that forbid hipMalloc). The
 * workspace is a static device array of TJEV_GDN_SCRATCH_BYTES on each GPU the library runs on,
 * held until the process ends: a problem whose forward workspace (tjev_gdn_workspace_bytes(p, 0))
 * exceeds it gets TJEV_GDN_EWORKSPACE (at the 0.8B head shape, 16 key and value heads of 128,
 * that is about 3,900 tokens per call in bf16, 2,700 in fp32). Nothing in it needs to start at zero. Every call on one
 * GPU uses that GPU's one array: calls that overlap on a GPU (other streams, other threads)
 * race, so order them on one stream. */
#define TJEV_GDN_SCRATCH_BYTES (128u << 20)
int tjev_gdn_mega2_fwd_cont_noalloc(const tjev_gdn_params* p, void* stream, const void* qkv,
                                    const void* a, const void* b, const float* a_log,
                                    const float* dt_bias, const float* conv_w, const int32_t* seg,
                                    const float* initial_state, const void* initial_conv, void* out,
                                    float* residuals, float* final_state, void* conv_state);

/* One decode step, T = 1 token per row (p->length == 1; chunk and residuals are ignored):
 * the reference's token recurrence (xla.py:141-167, its "T=1 decode step") on the
 * megakernel's inputs, with the conv over the kept rows (HF causal_conv1d_update). qkv [B, W]
 * (raw; post-conv when taps == 0), a, b [B, H]; conv_state [B, K-1, W] io_dtype read, and
 * conv_state_out the same history shifted by the new row (must not alias conv_state); state
 * [B, H, Dk, Dv] fp32 read and state_out written (may alias state); out [B, H, Dv] io_dtype.
 * qkv, conv_state, conv_state_out, state and state_out are 16-byte aligned. The step
 * continues the segment the state belongs to (no reset). */
int tjev_gdn_decode_step(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a,
                         const void* b, const float* a_log, const float* dt_bias,
                         const float* conv_w, const void* conv_state, const float* state,
                         void* out, void* conv_state_out, float* state_out);

/* The v2 operator (tjev's chunk_gated_delta_rule_v2, pallas_tpu_v2.py:541-582, behind
 * gdn_impl=pallas_tpu_v2): the same chunked delta rule on given q, k [B, T, Hk, Dk] (qk_dtype;
 * used as given: the model passes l2norm(q) * Dk^-1/2 and l2norm(k)), v [B, T, H, Dv]
 * (io_dtype), g (log decay) and beta [B, T, H] (gate_dtype); out [B, T, H, Dv] in io_dtype.
 * taps must be 0. The residuals and workspace are as for the megakernel. The backward writes
 * d_q, d_k (qk_dtype), d_v (io_dtype), d_g and d_beta (gate_dtype). */
int tjev_gdn_v2_fwd(const tjev_gdn_params* p, void* stream, const void* q, const void* k, const void* v,
                    const void* g, const void* beta, const int32_t* seg, void* out, float* residuals,
                    void* workspace, size_t workspace_bytes);
int tjev_gdn_v2_bwd(const tjev_gdn_params* p, void* stream, const void* q, const void* k, const void* v,
                    const void* g, const void* beta, const int32_t* seg, const float* residuals,
                    const void* d_out, void* d_q, void* d_k, void* d_v, void* d_g, void* d_beta,
                    void* workspace, size_t workspace_bytes);

/* The v2 operator with a state in and out: the reference's chunked rule
 * chunk_gated_delta_rule(q, k, v, g, beta, segment_ids, initial_state) -> (out, final_state)
 * (xla.py:170-262) on the v2 operator's inputs. initial_state [B, H, Dk, Dv] fp32 or null (as
 * for tjev_gdn_mega2_fwd_cont); final_state [B, H, Dk, Dv] fp32 or null: the state after token
 * T-1. The backward takes initial_state as given to the forward, d_final_state (null: 0; any
 * length) and writes d_initial_state when not null. */
int tjev_gdn_v2_fwd_cont(const tjev_gdn_params* p, void* stream, const void* q, const void* k,
                         const void* v, const void* g, const void* beta, const int32_t* seg,
                         const float* initial_state, void* out, float* residuals,
                         float* final_state, void* workspace, size_t workspace_bytes);
int tjev_gdn_v2_bwd_cont(const tjev_gdn_params* p, void* stream, const void* q, const void* k,
                         const void* v, const void* g, const void* beta, const int32_t* seg,
                         const float* initial_state, const float* residuals, const void* d_out,
                         const float* d_final_state, void* d_q, void* d_k, void* d_v, void* d_g,
                         void* d_beta, float* d_initial_state, void* workspace,
                         size_t workspace_bytes);

/* backward: replaces pallas_call "gdn_mega2_bwd" (pallas_tpu_mega.py:471-524) plus the XLA sums
 * of _core_bwd (:563-571): d_qkv (io_dtype), d_a, d_b (gate_dtype), d_a_log and d_dt_bias ([H] fp32), and,
 * when d_conv_w is not null, the conv weight's gradient [K, W] fp32 (the reference's
 * gdn_mega2_bwd_dw variant, computed only when requested). */
int tjev_gdn_mega2_bwd(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a,
                       const void* b, const float* a_log, const float* dt_bias,
                       const float* conv_w, const int32_t* seg, const float* residuals,
                       const void* d_out, void* d_qkv, void* d_a, void* d_b, float* d_a_log,
                       float* d_dt_bias, float* d_conv_w, void* workspace,
                       size_t workspace_bytes);

/* The gated RMSNorm of the GDN output, replacing tjev's GatedRMSNorm (src/tjev/model/norms.py:
 * 13-15, 36-40; its .flat form :42-62 is the same arithmetic on the same memory) and the padding
 * select after it (src/tjev/model/gdn.py:157-163):
 *   y = w * cast(x * rsqrt(mean_D(x^2) + eps)) * silu(gate), in fp32, stored in `dtype`
 * where cast rounds to `dtype` and back (a no-op for fp32). x, gate, y [tokens, heads, dim];
 * w [dim] fp32; seg [tokens] int32 or null: when given, y = 0 (and the incoming gradient is
 * taken as 0) on tokens whose segment id is <= 0. */
typedef struct tjev_gdn_norm_params {
  int64_t tokens; /* B*T */
  int32_t heads;  /* H */
  int32_t dim;    /* D, the normalized axis: 16, 32, 64, 128 or 256 */
  int32_t dtype;  /* tjev_gdn_dtype of x, gate, y, d_y, d_x, d_gate */
  float eps;      /* rms_norm_eps (1e-6 in Qwen3.5) */
} tjev_gdn_norm_params;

/* scratch of the backward's weight gradient (0 if d_weight will be null) */
size_t tjev_gdn_norm_workspace_bytes(const tjev_gdn_norm_params* p, int weight_grad);

int tjev_gdn_gated_rmsnorm_fwd(const tjev_gdn_norm_params* p, void* stream, const void* x,
                               const void* gate, const float* weight, const int32_t* seg,
                               void* y);

/* d_x and d_gate in `dtype`, as the reference's autodiff gives them (the cotangent of the
 * rounding cast is itself rounded to `dtype`); d_weight [dim] fp32, summed over tokens and
 * heads in a fixed order, only when not null (the reference's weight is frozen). */
int tjev_gdn_gated_rmsnorm_bwd(const tjev_gdn_norm_params* p, void* stream, const void* x,
                               const void* gate, const float* weight, const int32_t* seg,
                               const void* d_y, void* d_x, void* d_gate, float* d_weight,
                               void* workspace, size_t workspace_bytes);

/* Per-kernel timing (no counterpart in the reference, whose kernels are timed by xprof):
 * between tjev_gdn_profile_begin() and tjev_gdn_profile_end(), every launch of the megakernel
 * and norm calls is bracketed by a hipEvent pair on the call's stream. _end synchronizes those events
 * and writes, for kernel ids 0..n-1, the summed milliseconds and the launch count.
 * TJEV_GDN_KERNELS is the number of ids; tjev_gdn_kernel_name(id) names them. Not thread-safe:
 * profile from one host thread. */
#define TJEV_GDN_KERNELS 16
int tjev_gdn_profile_begin(void);
int tjev_gdn_profile_end(float* ms, int* launches, int n);
const char* tjev_gdn_kernel_name(int kernel);

/* message of the last nonzero status on this thread */
const char* tjev_gdn_last_error(void);

/* (major << 16) | minor */
int tjev_gdn_version(void);

/* 1 in the LDS-poison debug build (libtjev_gdn_lds_poison.so: every kernel fills its LDS with NaN
 * bytes before its own code runs, the counterpart of the reference's interpret-mode run with
 * uninitialized_memory="nan", tests/kernels/test_gdn_mega.py:161-178), 0 in the library */
int tjev_gdn_lds_poison(void);

#ifdef __cplusplus
}
#endif

#endif /* TJEV_GDN_H */
