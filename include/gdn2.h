/*
 * gdn2.h -- C ABI of libgdn2_amd.so, the MI355X (gfx950) GDN-2 scan.
 *
 * The library is the drop-in replacement for delta-block-lm's GDN-2 scan
 * operator.  Each entry point below names the reference interface it stands
 * in for.  Plain pointers and sizes only: device pointers come from the
 * caller's allocator (PyTorch, a Rust FFI crate, ...); the library itself
 * never allocates device memory and never synchronises the stream.
 *
 * Layouts (reference crates/mixers/src/chunk.rs:126):
 *   sequences  [batch, time, head, channel]     masks [batch, time] (f32 0/1)
 *   states     [batch, head, key, value]        scores [batch, time, head]
 * Inputs are strided views (element strides, any sign-free layout, stride 0
 * allowed for broadcast gates).  Outputs and gradients are dense row-major.
 *
 * Semantics (reference crates/mixers/src/reference.rs:41-257, per valid token):
 *   bar   = diag(alpha) S            (S zeroed first when reset[t] != 0)
 *   delta = write .* v - (erase .* k)^T bar
 *   S'    = bar + k delta^T,  out = S'^T q,  score = ||k|| * ||delta||
 * Padding tokens (valid == 0) emit zero output and score and keep the state.
 * At a zero edit the score takes the zero subgradient.
 *
 * Errors: every entry point validates before launching.  On failure it
 * returns a nonzero status, launches nothing, and gdn2_last_error() (per
 * calling thread) describes the failure.  There is no CPU fallback.
 * Calls are asynchronous on `stream` (a hipStream_t; NULL = default stream).
 */
#ifndef GDN2_AMD_H
#define GDN2_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) || defined(__clang__)
#define GDN2_API __attribute__((visibility("default")))
#else
#define GDN2_API
#endif

enum gdn2_dtype { GDN2_F32 = 0, GDN2_BF16 = 1, GDN2_I32 = 2 /* document limits only */ };

enum gdn2_status {
    GDN2_OK = 0,
    GDN2_ERR_ARGUMENT = 1,  /* null pointer, bad enum, bad chunk */
    GDN2_ERR_SHAPE = 2,     /* empty axis or unsupported key/value width */
    GDN2_ERR_DTYPE = 3,     /* unsupported or mismatched dtypes */
    GDN2_ERR_WORKSPACE = 4, /* checkpoint/workspace buffer too small */
    GDN2_ERR_LAUNCH = 5     /* HIP launch error */
};

/* Logical problem size.  keys = d_k, values = d_v (each 1..128). */
typedef struct gdn2_shape {
    int64_t batch, time, heads, keys, values;
} gdn2_shape;

/* Strided read-only device view.  For sequence tensors the strides are those
 * of [batch, time, head, channel]; for states [batch, head, key, value]; for
 * masks [batch, time] (stride[2], stride[3] unused); for per-head scalars
 * [batch, time, head] (stride[3] unused).  Strides are in elements. */
typedef struct gdn2_view {
    const void *data;
    int32_t dtype; /* enum gdn2_dtype */
    int32_t reserved;
    int64_t stride[4];
} gdn2_view;

/* Version of this ABI (major * 100 + minor). */
GDN2_API int gdn2_abi_version(void);

/* Message of the last failure on the calling thread ("" after success). */
GDN2_API const char *gdn2_last_error(void);

/* ---- Channel-wise GDN-2 training scan ------------------------------------ */
/* Replaces GdnTrainingOps::gdn_training_scan / gdn_training_backward
 * (reference crates/kernels/src/gdn_training_ops.rs:27-68) and their CubeCL
 * launches run_scan / run_backward (crates/kernels/src/gdn_training.rs:344-487).
 * The reference packs [output ; final_state ; scores] into one f32 buffer
 * (gdn_training_ops.rs:300-332); passing output = packed, final_state =
 * packed + B*T*H*V, scores = packed + B*T*H*V + B*H*K*V with an f32 output
 * reproduces that packing exactly.  The reference's private `checkpoint` and
 * `auxiliary` tensors are replaced by one opaque checkpoint buffer written by
 * the forward and read by the backward.
 *
 * q, k, v: F32 or BF16 (same dtype); alpha, erase, write, valid, reset,
 * initial: F32.  initial.data may be NULL (zero state).  chunk: 1..64, the
 * checkpoint interval of the reference (1..16, gdn_training.rs:370-373; up to
 * 64 accepted here); results do not depend on it.  bf16 q/k/v with keys =
 * values = 64, unit channel stride and 16-byte aligned token rows run the
 * 16-token chunk-WY MFMA kernels; every other shape (keys, values <= 128, f32
 * or bf16, any strides) runs the 16-token f32 chunk kernels, which read bf16
 * inputs as their exact f32 values.  The bf16 MFMA kernels need alpha >= 0 on
 * valid tokens: a negative alpha gives NaN outputs, state and gradients for
 * its sequence (the f32 chunk kernels accept any alpha).  alpha = 0 and tiny
 * alphas get their exact gradient on both.  On the MFMA kernels d_output must
 * have aligned rows too.  checkpoint (and the backward's workspace) must be
 * 16-byte aligned. */
GDN2_API size_t gdn2_training_checkpoint_bytes(const gdn2_shape *shape, int chunk);

GDN2_API int gdn2_training_scan(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                       const gdn2_view *k, const gdn2_view *v, const gdn2_view *alpha,
                       const gdn2_view *erase, const gdn2_view *write,
                       const gdn2_view *valid, const gdn2_view *reset,
                       const gdn2_view *initial, void *output, int32_t output_dtype,
                       float *final_state, float *scores, void *checkpoint,
                       size_t checkpoint_bytes, void *stream);

/* Scratch the backward needs beyond the checkpoint. */
GDN2_API size_t gdn2_training_workspace_bytes(const gdn2_shape *shape, int chunk);

/* d_output ([B,T,H,V], F32 or BF16, strided), d_final_state ([B,H,K,V] F32,
 * contiguous) and d_scores ([B,T,H] F32, contiguous) may each be NULL (zero
 * adjoint).  Gradients are written densely: dq, dk, dv in the dtype of q/k/v;
 * dalpha, derase, dwrite, d_initial in F32.  Any gradient pointer may be NULL
 * (not wanted) except that the kernel still computes it internally. */
GDN2_API int gdn2_training_backward(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                           const gdn2_view *k, const gdn2_view *v, const gdn2_view *alpha,
                           const gdn2_view *erase, const gdn2_view *write,
                           const gdn2_view *valid, const gdn2_view *reset,
                           const void *checkpoint, size_t checkpoint_bytes,
                           const gdn2_view *d_output, const float *d_final_state,
                           const float *d_scores, void *dq, void *dk, void *dv,
                           float *dalpha, float *derase, float *dwrite, float *d_initial,
                           void *workspace, size_t workspace_bytes, void *stream);

/* ---- Document-limit GDN-2 scan -------------------------------------------- */
/* Replaces Gdn2Ops::gdn2_scan / gdn2_backward (reference
 * crates/kernels/src/ops.rs:17-276, CubeCL launches crates/kernels/src/gdn2.rs);
 * forward semantics of the f64 oracle crates/mixers/src/gdn2_reference.rs:51-103.
 * Packed documents are described per token by inclusive int32 limits
 * doc_start[b,t], doc_end[b,t] (I32 views, strides [batch, time]):
 *   end < start      padding: zero output, state kept
 *   start == t       the state is zeroed before the token's update
 * The backward is the exact VJP of that forward, as the reference's chunked
 * kernels compute it (gdn2.rs:24-65 decay products that vanish across a
 * reset, :288-490): the state adjoint never crosses a reset and passes
 * unchanged through padding.  The reference's f64 oracle
 * (gdn2_reference.rs:107-226) instead clears the adjoint at tokens with
 * end == t; the two agree whenever each reset follows a document end (the
 * limits every packed batch carries) and differ only for limits where a reset
 * has no preceding end or an end no following reset.  Zero initial state; no
 * final state or score outputs.  q, k, v: F32 or BF16 (same dtype); alpha,
 * erase, write: F32.  bf16 q/k/v with keys = values = 64 and 16-byte aligned
 * rows run the 16-token chunk-WY MFMA kernels, every other shape (keys, values
 * <= 128) the 16-token f32 chunk kernels.  The MFMA kernels need alpha >= 0 on
 * live tokens (a negative alpha gives NaN results for its sequence); the f32
 * chunk kernels accept any alpha.  The checkpoint (opaque, 16-byte aligned, as
 * is the backward's workspace) replaces the reference's [B, H, T/16, 48, 64]
 * checkpoint tensor. */
GDN2_API size_t gdn2_scan_checkpoint_bytes(const gdn2_shape *shape);

GDN2_API int gdn2_scan(const gdn2_shape *shape, const gdn2_view *q, const gdn2_view *k,
                       const gdn2_view *v, const gdn2_view *alpha, const gdn2_view *erase,
                       const gdn2_view *write, const gdn2_view *doc_start,
                       const gdn2_view *doc_end, void *output, int32_t output_dtype,
                       void *checkpoint, size_t checkpoint_bytes, void *stream);

GDN2_API size_t gdn2_scan_workspace_bytes(const gdn2_shape *shape);

/* d_output: [B,T,H,V] in q's dtype (strided).  Gradients dense: dq, dk, dv in
 * q's dtype, dalpha, derase, dwrite F32; any may be NULL (not wanted). */
GDN2_API int gdn2_backward(const gdn2_shape *shape, const gdn2_view *q, const gdn2_view *k,
                           const gdn2_view *v, const gdn2_view *alpha, const gdn2_view *erase,
                           const gdn2_view *write, const gdn2_view *doc_start,
                           const gdn2_view *doc_end, const void *checkpoint,
                           size_t checkpoint_bytes, const gdn2_view *d_output, void *dq, void *dk,
                           void *dv, float *dalpha, float *derase, float *dwrite, void *workspace,
                           size_t workspace_bytes, void *stream);

/* ---- Scalar-gate gated delta rule (chunked, MFMA) ------------------------ */
/* The scalar special case of the same recurrence: alpha[i] = exp(g),
 * erase[i] = write[j] = beta for every channel.  beta and g are [B,T,H] F32
 * (g is the log decay, finite).  No counterpart entry exists in the reference
 * (it reaches this case only through the channel-wise op with broadcast
 * gates); this is the chunk-WY fast path the north-star benchmark measures.
 * The chunk-WY MFMA kernels run when chunk == 64, d_k == d_v (64 or 128) and
 * q, k, v are BF16 with unit channel stride, 16-byte aligned data and every
 * other stride a multiple of 8 elements; any other call takes the
 * token-sequential kernels.  On the chunk-WY path d_output must satisfy the
 * same row rule (a stride-0 broadcast upstream is rejected with
 * GDN2_ERR_ARGUMENT: pass a dense copy). */
GDN2_API size_t gdn_scalar_checkpoint_bytes(const gdn2_shape *shape, int chunk);

GDN2_API int gdn_scalar_scan(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                    const gdn2_view *k, const gdn2_view *v, const gdn2_view *beta,
                    const gdn2_view *g, const gdn2_view *valid, const gdn2_view *reset,
                    const gdn2_view *initial, void *output, int32_t output_dtype,
                    float *final_state, float *scores, void *checkpoint,
                    size_t checkpoint_bytes, void *stream);

GDN2_API size_t gdn_scalar_workspace_bytes(const gdn2_shape *shape, int chunk);

GDN2_API int gdn_scalar_backward(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                        const gdn2_view *k, const gdn2_view *v, const gdn2_view *beta,
                        const gdn2_view *g, const gdn2_view *valid, const gdn2_view *reset,
                        const void *checkpoint, size_t checkpoint_bytes,
                        const gdn2_view *d_output, const float *d_final_state,
                        const float *d_scores, void *dq, void *dk, void *dv, float *dbeta,
                        float *dg, float *d_initial, void *workspace, size_t workspace_bytes,
                        void *stream);

/* The same backward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  It
 * calls no allocating routine: its scratch is a fixed device array of
 * GDN2_NOALLOC_SCRATCH_BYTES inside the library (one per device, held until
 * the process ends), and a shape whose gdn_scalar_workspace_bytes exceeds
 * that size is rejected with GDN2_ERR_WORKSPACE.  Every call on a device
 * shares that device's array, so calls that overlap in time on one device
 * (other streams, other threads) race; calls in order on one stream do not.
 * Arguments and results are those of gdn_scalar_backward. */
#define GDN2_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

GDN2_API int gdn_scalar_backward_noalloc(const gdn2_shape *shape, int chunk, const gdn2_view *q,
                        const gdn2_view *k, const gdn2_view *v, const gdn2_view *beta,
                        const gdn2_view *g, const gdn2_view *valid, const gdn2_view *reset,
                        const void *checkpoint, size_t checkpoint_bytes,
                        const gdn2_view *d_output, const float *d_final_state,
                        const float *d_scores, void *dq, void *dk, void *dv, float *dbeta,
                        float *dg, float *d_initial, void *stream);

/* ---- Decode step on a carried state -------------------------------------- */
/* One token per sequence (time == 1) applied in place to state [B,H,K,V] F32.
 * Equivalent to gdn2_training_scan with time = 1, initial = final_state =
 * state; the reference reaches it as the T=1 scans of Mixer::prepare_sbd's
 * noisy path (crates/mixers/src/sbd.rs:270-283).  valid/reset may have
 * data == NULL (all valid, no reset). */
GDN2_API int gdn2_decode_step(const gdn2_shape *shape, const gdn2_view *q, const gdn2_view *k,
                     const gdn2_view *v, const gdn2_view *alpha, const gdn2_view *erase,
                     const gdn2_view *write, const gdn2_view *valid, const gdn2_view *reset,
                     float *state, void *output, int32_t output_dtype, float *scores,
                     void *stream);

/* ---- Mixer prologue / epilogue operators --------------------------------- */
/* The elementwise and row-local operators around the scan in the reference's
 * GDN mixer (crates/mixers/src/lib.rs:456-525, :667-688), as the reference's
 * custom ops expose them (crates/kernels/src/conv.rs, norm.rs, decay.rs).  All
 * tensors are F32; inputs are strided views, outputs and gradients are dense.
 * Parameter gradients are reduced deterministically through a caller-provided
 * workspace (its size from the *_workspace_bytes query). */

/* Rows of a [batch, time, heads, width] tensor (width = channels of one row). */
typedef struct gdn2_rows_shape {
    int64_t batch, time, heads, width;
} gdn2_rows_shape;

/* Depthwise causal convolution with `taps` lags over [batch, time, channels]
 * (reference crates/kernels/src/conv.rs:22-45 forward, :47-104 VJP; the
 * mixer's causal_conv, crates/mixers/src/lib.rs:696-725):
 *   y[b,t,c] = sum_{l < taps, l <= t} x[b,t-l,c] w[l,c] m(b, t-l, t),
 *   m(b,s,d) = valid[b,s] valid[b,d] [docs[b,s] == docs[b,d]]
 * (a lag never crosses a document boundary or an invalid token).  x views
 * [batch, time, channels] (stride[3] unused), w views [taps, channels],
 * valid/docs [batch, time].  activation 1 applies SiLU to y in the same pass
 * (the mixer applies it right after the convolution, lib.rs:463-466);
 * activation 0 is the reference operator itself.  taps 1..8. */
typedef struct gdn2_conv_shape {
    int64_t batch, time, channels, taps;
} gdn2_conv_shape;

GDN2_API int gdn2_conv_forward(const gdn2_conv_shape *shape, const gdn2_view *x,
                               const gdn2_view *w, const gdn2_view *valid, const gdn2_view *docs,
                               int activation, float *y, void *stream);
GDN2_API size_t gdn2_conv_workspace_bytes(const gdn2_conv_shape *shape);
/* dy: [batch, time, channels] view.  dx dense [batch, time, channels], dw dense
 * [taps, channels]; either may be NULL (not wanted). */
GDN2_API int gdn2_conv_backward(const gdn2_conv_shape *shape, const gdn2_view *x,
                                const gdn2_view *w, const gdn2_view *valid, const gdn2_view *docs,
                                int activation, const gdn2_view *dy, float *dx, float *dw,
                                void *workspace, size_t workspace_bytes, void *stream);

/* Row normalization (reference crates/kernels/src/norm.rs:22-72 forward,
 * :74-164 VJPs), rows of width <= 1024:
 *   mode 0 (L2):        y = x / sqrt(sum x^2 + eps)
 *   mode 1 (RMS):       y = w x / sqrt(mean x^2 + eps)
 *   mode 2 (gated RMS): z = x sigmoid(gate), y = w z / sqrt(mean z^2 + eps)
 * weight [width] (modes 1, 2; view stride[0]) and gate (mode 2, same shape as
 * x) may otherwise be NULL.  inverse [rows] receives 1/sqrt(...) for the
 * backward. */
GDN2_API int gdn2_norm_forward(const gdn2_rows_shape *shape, int mode, float epsilon,
                               const gdn2_view *x, const gdn2_view *weight, const gdn2_view *gate,
                               float *y, float *inverse, void *stream);
GDN2_API size_t gdn2_norm_workspace_bytes(const gdn2_rows_shape *shape);
/* dx (and dgate for mode 2) dense like x; dweight [width] (modes 1, 2).  Any
 * gradient pointer may be NULL. */
GDN2_API int gdn2_norm_backward(const gdn2_rows_shape *shape, int mode, const gdn2_view *x,
                                const gdn2_view *weight, const gdn2_view *gate,
                                const float *inverse, const gdn2_view *dy, float *dx, float *dgate,
                                float *dweight, void *workspace, size_t workspace_bytes,
                                void *stream);

/* Decay gate (reference crates/kernels/src/decay.rs): with z = x + bias[h,k],
 * softplus(z) = z for z > 20 else log1p(exp(z)),
 *   alpha = exp(-exp(scale[h]) softplus(z)).
 * x [batch, time, heads, width], bias [heads * width], scale [heads] (views use
 * stride[0]).  Backward: dx, dbias [heads * width], dscale [heads]. */
GDN2_API int gdn2_decay_forward(const gdn2_rows_shape *shape, const gdn2_view *x,
                                const gdn2_view *bias, const gdn2_view *scale, float *y,
                                void *stream);
GDN2_API size_t gdn2_decay_workspace_bytes(const gdn2_rows_shape *shape);
GDN2_API int gdn2_decay_backward(const gdn2_rows_shape *shape, const gdn2_view *x,
                                 const gdn2_view *bias, const gdn2_view *scale,
                                 const gdn2_view *dy, float *dx, float *dbias, float *dscale,
                                 void *workspace, size_t workspace_bytes, void *stream);

/* ---- Training-step operators ---------------------------------------------- */

/* Row cross entropy (reference crates/kernels/src/cross_entropy.rs:7-60 forward,
 * :62-83 backward; op cross_entropy_rows, cross_entropy_ops.rs:108-117):
 *   m = max_c x[r,c],  s = ln sum_c exp(x[r,c] - m)
 *   loss[r] = (m - x[r, target[r]]) + s,   stats[2r] = m, stats[2r+1] = s
 *   dx[r,c] = (exp(x[r,c] - m - s) - [c == target[r]]) * upstream[r]
 * x: [rows, width] F32 or BF16 (stride[0] between rows, stride[1] between
 * columns).  target: int64 class ids, target[r * target_stride] (the reference
 * passes integral f32 labels); an id outside [0, width) gives loss NaN and no
 * one-hot term.  upstream: f32, upstream[r * upstream_stride].  dx: contiguous
 * [rows, width] in x's dtype. */
GDN2_API int gdn2_cross_entropy_forward(int64_t rows, int64_t width, const gdn2_view *x,
                                        const int64_t *target, int64_t target_stride,
                                        float *loss, float *stats, void *stream);
GDN2_API int gdn2_cross_entropy_backward(int64_t rows, int64_t width, const gdn2_view *x,
                                         const int64_t *target, int64_t target_stride,
                                         const float *stats, const float *upstream,
                                         int64_t upstream_stride, void *dx, void *stream);
/* Forward and gradient in one pass over the rows, for a loss whose upstream
 * gradient per row is the constant `scale` (a mean over rows: 1 / rows):
 * loss[r] as above and dx[r,c] = (exp(x[r,c] - m - s) - [c == target[r]]) * scale.
 * dx may be x's own storage (x contiguous): the logits are then replaced by
 * their gradient.  No counterpart in the reference, which runs the two kernels
 * above; it serves training steps that need the logits only for this loss. */
GDN2_API int gdn2_cross_entropy_fused(int64_t rows, int64_t width, const gdn2_view *x,
                                      const int64_t *target, int64_t target_stride, float scale,
                                      float *loss, void *dx, void *stream);

/* AdamW with per-parameter gradient clipping (reference
 * crates/kernels/src/update.rs:46-82 adam_kernel and :116-199 adam; op
 * adamw_update, update_ops.rs:90-117; caller FusedAdamW,
 * crates/experiment/src/update.rs:43-96).  For each tensor, with its own
 * gradient norm n = sqrt(sum g^2):
 *   g' = g * min(clip / (n + FLT_MIN), 1)
 *   m  = g' (1 - 0.9)        [+ 0.9 m_prev   when initialized]
 *   v  = g'^2 (1 - 0.999)    [+ 0.999 v_prev when initialized]
 *   param = param * (1 - lr weight_decay) - lr (m / c1) / (sqrt(v / c2) + 1e-5)
 * with c1 = 1 - 0.9^time and c2 = 1 - 0.999^time in f32, every operation
 * rounded in this order (no fused multiply-adds).  param, first and second are
 * updated in place; all f32 and contiguous. */
typedef struct gdn2_adamw_tensor {
    float *param;
    const float *grad;
    float *first;  /* first moment (read only when initialized) */
    float *second; /* second moment */
    int64_t numel;
} gdn2_adamw_tensor;

/* One launch pair for a whole parameter set: the descriptor table and the
 * per-chunk squared-norm partials live in the workspace.  With reuse_table
 * nonzero the workspace must still hold the table that a previous call wrote
 * for the same tensors; the call then skips rewriting it.  The norms are
 * reduced in a fixed order: results do not depend on the launch. */
GDN2_API size_t gdn2_adamw_workspace_bytes(int32_t count, const gdn2_adamw_tensor *tensors);
GDN2_API int gdn2_adamw_update(int32_t count, const gdn2_adamw_tensor *tensors, int initialized,
                               int64_t time, double lr, float weight_decay, float clip,
                               int reuse_table, void *workspace, size_t workspace_bytes,
                               void *stream);

/* ---- Fused operators of the lm512 training step ------------------------------ */
/* No counterpart in the reference, whose model composes the f32 operators
 * above one by one (crates/mixers/src/lib.rs:456-525; block
 * crates/experiment/src/model.rs:300-364).  They serve a bf16 training step of
 * that model: each folds the casts, slices, residual adds and pointwise ops
 * around a GEMM into one pass, computing in f32 and rounding to bf16 exactly
 * where the unfused bf16 composition rounds.  All tensors are dense and
 * row-major; "bf16" arguments point to bfloat16 storage.  Parameter gradients
 * are reduced deterministically through the workspace. */

/* RMSNorm with the residual add in front, rows of `width` (128, or a multiple
 * of 256 up to 1024):  u = x + residual (bf16; NULL: u = x),
 *   y = bf16(weight * u / sqrt(mean u^2 + epsilon)),  inverse[r] = 1/sqrt(...).
 * u (f32, may be NULL) receives the sum.  x, u, weight 16-byte aligned. */
GDN2_API int gdn2_lm_norm_forward(int64_t rows, int64_t width, float epsilon, const float *x,
                                  const void *residual, const float *weight, float *u, void *y,
                                  float *inverse, void *stream);
GDN2_API size_t gdn2_lm_norm_workspace_bytes(int64_t rows, int64_t width);
/* VJP with the residual gradient added: dx = dres + J^T dy (dy bf16; dres f32
 * or NULL).  dx (f32) and dx_bf16 (bf16 copy, may be NULL); dweight [width]. */
GDN2_API int gdn2_lm_norm_backward(int64_t rows, int64_t width, const float *x,
                                   const float *weight, const float *inverse, const void *dy,
                                   const float *dres, float *dx, void *dx_bf16, float *dweight,
                                   void *workspace, size_t workspace_bytes, void *stream);

/* The GDN mixer around the scalar-gate scan.  z is the packed input
 * projection, bf16 [batch, time, z_stride], per token
 *   [q (H K) | k (H K) | v (H V) | gate (H V) | beta (H) | decay (H)]
 * with keys = values = 64, heads a power of two up to 32, taps 1..8. */
typedef struct gdn2_lm_mixer_shape {
    int64_t batch, time, heads, keys, values, taps, z_stride;
} gdn2_lm_mixer_shape;

/* qkv bf16 [batch, time, 3 H 64] = per-head L2 (q, k; epsilon 1e-6) of
 * silu(causal_conv(z[..., :3 H 64], conv_w)) (conv_w f32 [taps, 3 H 64]; the
 * masks as for gdn2_conv_forward); beta, g f32 [batch, time, H]:
 *   beta = sigmoid(z_beta),  g = -exp(decay_scale[h]) softplus(z_decay + decay_bias[h]). */
GDN2_API int gdn2_lm_mixer_in_forward(const gdn2_lm_mixer_shape *shape, const void *z,
                                      const float *conv_w, const float *valid, const float *docs,
                                      const float *decay_scale, const float *decay_bias,
                                      void *qkv, float *beta, float *g, void *stream);
GDN2_API size_t gdn2_lm_mixer_in_workspace_bytes(const gdn2_lm_mixer_shape *shape);
/* From the scan's gradients (dq, dk, dv bf16 [batch, time, H, 64]; dbeta, dg
 * f32 [batch, time, H]): the q, k, v, beta and decay columns of dz (bf16, z's
 * layout; the gate columns are left to gdn2_lm_mixer_out_backward), dconv_w
 * [taps, 3 H 64], ddecay_scale [H], ddecay_bias [H]. */
GDN2_API int gdn2_lm_mixer_in_backward(const gdn2_lm_mixer_shape *shape, const void *z,
                                       const float *conv_w, const float *valid, const float *docs,
                                       const float *decay_scale, const float *decay_bias,
                                       const void *dq, const void *dk, const void *dv,
                                       const float *dbeta, const float *dg, void *dz,
                                       float *dconv_w, float *ddecay_scale, float *ddecay_bias,
                                       void *workspace, size_t workspace_bytes, void *stream);

/* Output gate: y bf16 [batch, time, H 64] = rms_norm(o, norm_w) * silu(gate)
 * per head (o bf16 [batch, time, H, 64], the scan output; gate from z);
 * inverse [batch time H]. */
GDN2_API int gdn2_lm_mixer_out_forward(const gdn2_lm_mixer_shape *shape, const void *o,
                                       const void *z, const float *norm_w, float epsilon, void *y,
                                       float *inverse, void *stream);
GDN2_API size_t gdn2_lm_mixer_out_workspace_bytes(const gdn2_lm_mixer_shape *shape);
/* d_o bf16 (the scan's output gradient), the gate columns of dz, dnorm_w [64]. */
GDN2_API int gdn2_lm_mixer_out_backward(const gdn2_lm_mixer_shape *shape, const void *o,
                                        const void *z, const float *norm_w, const float *inverse,
                                        const void *dy, void *d_o, void *dz, float *dnorm_w,
                                        void *workspace, size_t workspace_bytes, void *stream);

/* SwiGLU: h bf16 [rows, 2 width] = [gate | up] ->
 *   a bf16 [rows, width] = bf16(bf16(silu(gate)) * up);
 * the VJP writes both halves of dh.  width a multiple of 8, 16-byte aligned. */
GDN2_API int gdn2_lm_swiglu_forward(int64_t rows, int64_t width, const void *h, void *a,
                                    void *stream);
GDN2_API int gdn2_lm_swiglu_backward(int64_t rows, int64_t width, const void *h, const void *da,
                                     void *dh, void *stream);

/* ---- HOLA exact-memory cache read (the consumer of the scan's scores) ------- */
/* Replaces HolaOps::hola_schedule / hola_read / hola_backward (reference
 * crates/kernels/src/hola_ops.rs:17-425, kernels crates/kernels/src/hola.rs;
 * semantics of the scalar oracle crates/mixers/src/hola_checks.rs:294-391).
 * Per (batch, head), chunks of `chunk` tokens in order:
 *   * every valid query t attends with softmax, scale 1/sqrt(keys), to the
 *     cache kept before its chunk plus tokens first..t of its chunk, restricted
 *     to valid tokens of its own document, next to a learned sink logit
 *     sink[h] whose value is zero; invalid queries output zero;
 *   * after the chunk the cache keeps, of cache + chunk, the valid tokens whose
 *     document equals that of the chunk's last physical slot (padding
 *     included), the `capacity` highest by score (recency: by position),
 *     ties to the earlier position.
 * Scores choose membership only: they take no gradient.  q, k: [B,T,H,keys],
 * v: [B,T,H,values], scores [B,T,H] (stride[3] unused), valid and documents
 * [B,T], sink [H] (stride[0]); all F32 views.  keys, values 1..128, capacity
 * 1..64, chunk 1..16 (the reference's chunk limit). */
typedef struct gdn2_hola_shape {
    int64_t batch, time, heads, keys, values;
    int32_t capacity, chunk;
} gdn2_hola_shape;

/* Positions only (hola_ops.rs:358-385): schedule [B, H, ceil(T/chunk) + 1,
 * capacity] F32, the cache before the first chunk and after each chunk, -1 for
 * an empty slot. */
GDN2_API int gdn2_hola_schedule(const gdn2_hola_shape *shape, int recency,
                                const gdn2_view *scores, const gdn2_view *valid,
                                const gdn2_view *documents, float *schedule, void *stream);

/* Read (hola_ops.rs:387-425): output [B,T,H,values] F32 dense, and optionally
 * the final cache positions [B,H,capacity].  The checkpoint (opaque, sized by
 * gdn2_hola_checkpoint_bytes) keeps the schedule, per-key visibility ends and
 * the softmax statistics for the backward. */
GDN2_API size_t gdn2_hola_checkpoint_bytes(const gdn2_hola_shape *shape);
GDN2_API int gdn2_hola_read(const gdn2_hola_shape *shape, int recency, const gdn2_view *q,
                            const gdn2_view *k, const gdn2_view *v, const gdn2_view *scores,
                            const gdn2_view *valid, const gdn2_view *documents,
                            const gdn2_view *sink, float *output, float *final_positions,
                            void *checkpoint, size_t checkpoint_bytes, void *stream);

/* VJP of sum(output * d_output) in q, k, v (dense [B,T,H,*] F32) and sink
 * [H]; `output` is the read's own output.  d_output may be NULL (zero). */
GDN2_API size_t gdn2_hola_workspace_bytes(const gdn2_hola_shape *shape);
GDN2_API int gdn2_hola_backward(const gdn2_hola_shape *shape, const gdn2_view *q,
                                const gdn2_view *k, const gdn2_view *v, const gdn2_view *valid,
                                const gdn2_view *documents, const gdn2_view *sink,
                                const void *checkpoint, size_t checkpoint_bytes,
                                const float *output, const gdn2_view *d_output, float *dq,
                                float *dk, float *dv, float *dsink, void *workspace,
                                size_t workspace_bytes, void *stream);

/* Measurement hook.  No counterpart in the reference: it serves benchmarks
 * that need the duration of each kernel of the chunk-WY path, measured on the
 * stream the kernels run on.  After gdn2_stage_timing(1), every chunk-path
 * call of gdn_scalar_scan / gdn_scalar_backward records a pair of HIP events
 * around each of its kernels on the call's stream; gdn2_stage_ms(i) returns
 * the duration of stage i in the most recent call that ran it (the caller
 * synchronises the stream first), or a negative value if stage i has not run
 * since timing was enabled.  Stages: 0 prep, 1 state scan, 2 output
 * (forward); 3 backward prep, 4 adjoint scan, 5 gradients (backward).
 * Process-wide state for the current device, not thread safe: enable it only
 * in single-threaded measurement runs.  A call whose stream is being captured
 * into a graph records no events (the stage then keeps its last duration).
 * Returns GDN2_OK or an error. */
GDN2_API int gdn2_stage_timing(int enable);
GDN2_API int gdn2_stage_count(void);
GDN2_API const char *gdn2_stage_name(int stage);
GDN2_API float gdn2_stage_ms(int stage);

#ifdef __cplusplus
}
#endif

#endif /* GDN2_AMD_H */
