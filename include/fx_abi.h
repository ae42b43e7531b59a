/*
 * fx_abi.h -- C ABI of libfxforge.so, the gfx950 (MI355X, CDNA4) kernels behind
 * the fxlm / fxgpu Python surface.
 *
 * Conventions
 *   - Every pointer is HIP device memory unless the comment says "host".
 *   - bf16 tensors are passed as uint16_t* holding IEEE bfloat16 bit patterns.
 *   - `stream` is a hipStream_t passed as void* (torch.cuda.current_stream().cuda_stream).
 *   - Every entry point only enqueues work on `stream`; none synchronises and none
 *     allocates device memory.  Workspace buffers are owned by the caller, except for
 *     fx_adamw_step_noalloc, whose workspace is a fixed buffer inside the library.
 *   - Return value: 0 on success, FX_EINVAL when an argument check fails, otherwise
 *     the hipError_t of the failed HIP call.  fx_last_error() gives a message.
 *
 * Each entry point names the reference interface it replaces
 * (berattunca21-byte/radeon-igpu-forge, paths relative to the repo root).
 */
#ifndef FX_ABI_H
#define FX_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FX_EINVAL (-1)
#define FX_ABI_VERSION 5

/* ---- library ------------------------------------------------------------ */

/* ABI version (FX_ABI_VERSION).  No reference counterpart (the reference has no
 * prebuilt library; its loader is ml/fxgpu/hip_kernel.py:50-145). */
int fx_abi_version(void);

/* Message for the last non-zero return on the calling host thread. */
const char* fx_last_error(void);

/* Loader smoke kernel: p[i] = value for i < n.
 * Replaces the fill42 smoke of ml/fxgpu/hip_kernel.py:148-163. */
int fx_fill_f32(float* p, int64_t n, float value, void* stream);

/* ---- RMSNorm ------------------------------------------------------------ */

/* y = x * rstd * w, rstd[r] = 1/sqrt(mean_d(x[r,d]^2) + eps) (fp32, one per row).
 * x, y: (N, D) bf16 contiguous; w: (D,) bf16; D % 8 == 0, 8 <= D <= 8192.
 * Replaces _RMSNorm.forward + rms_norm_fwd
 * (ml/fxlm/norm.py:47-62, ml/fxlm/kernels/norm.hip:32-59). */
int fx_rms_norm_fwd(const uint16_t* x, const uint16_t* w, uint16_t* y, float* rstd,
                    int64_t N, int32_t D, float eps, void* stream);

/* Bytes of fp32 workspace fx_rms_norm_bwd needs for (N, D). */
int64_t fx_rms_norm_bwd_workspace(int64_t N, int32_t D);

/* dx = rstd*w*dy - x*(rstd^3 * sum_d(x*w*dy) / D)   (bf16, (N, D))
 * dw = sum_rows x*rstd*dy                             (fp32 dw_f32 and bf16 dw, (D,))
 * One pass over x and dy: dx and per-block dw partials in one kernel, then a column
 * reduction of the partials.  `work` holds fx_rms_norm_bwd_workspace(N, D) bytes.
 * dw (bf16) may be NULL.  dw_f32 and work are 16-byte aligned, dw 8-byte aligned.
 * Replaces _RMSNorm.backward + rms_norm_bwd_dx + rms_norm_bwd_dw + part.sum(0)
 * (ml/fxlm/norm.py:64-85, ml/fxlm/kernels/norm.hip:63-127). */
int fx_rms_norm_bwd(const uint16_t* x, const uint16_t* dy, const uint16_t* w,
                    const float* rstd, uint16_t* dx, float* dw_f32, uint16_t* dw,
                    float* work, int64_t N, int32_t D, void* stream);

/* fx_rms_norm_bwd with dx += dres ((N, D) bf16, 16-byte aligned) in the same pass: the
 * gradient of a pre-norm residual block's input, dres arriving along the residual path
 * and dy through the norm.  No counterpart in the reference: it fuses the sum that
 * autograd forms for ml/fxlm/model.py:69,71 (x = x + proj(attn(norm(x))), x = x + mlp(norm(x))),
 * one bf16 add kernel per norm in the backward. */
int fx_rms_norm_bwd_add(const uint16_t* x, const uint16_t* dy, const uint16_t* dres,
                        const uint16_t* w, const float* rstd, uint16_t* dx, float* dw_f32,
                        uint16_t* dw, float* work, int64_t N, int32_t D, void* stream);

/* xsum = x + r (fp32 sum rounded to bf16, as a bf16 tensor add rounds it) and
 * fx_rms_norm_fwd of xsum, in one pass: (N, D) bf16 x, r, xsum, y, 16-byte aligned;
 * y and rstd are bit for bit those of the add followed by fx_rms_norm_fwd.  No
 * counterpart in the reference: it fuses the residual sums of ml/fxlm/model.py:69,71
 * (x = x + proj(...), x = x + fc2(...)) into the next norm that reads them. */
int fx_rms_norm_fwd_add(const uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* xsum,
                        uint16_t* y, float* rstd, int64_t N, int32_t D, float eps, void* stream);

/* ---- softmax cross-entropy ---------------------------------------------- */

/* inv_n = 1/count(target != ignore_index) (0 when the count is 0);
 * mul = inv_n * (grad_scale ? *grad_scale : grad_scale_value).
 * Out-of-range targets count here (they are ignored by fx_ce_fwd_grad), exactly as
 * _inv_nvalid does.  Replaces _inv_nvalid and the `mul = inv_n * gs_t` line
 * (ml/fxlm/cross_entropy.py:41-44, :117-121). */
int fx_ce_inv_nvalid(const int64_t* target, int64_t N, int64_t ignore_index,
                     const float* grad_scale, float grad_scale_value,
                     float* inv_n, float* mul, void* stream);

/* Argument block of the fused CE kernel; mirrors CEArgs
 * (ml/fxlm/kernels/ce.hip:10-19, ml/fxlm/cross_entropy.py:23-30) with bf16 logits
 * and a per-row loss vector instead of one atomically accumulated scalar. */
typedef struct fxCEArgs {
    const uint16_t* logits;   /* (N, V) bf16, row stride ld (elements) */
    const int64_t* target;    /* (N,) int64 */
    uint16_t* grad;           /* (N, V) bf16 row stride ldg, or NULL (loss only) */
    float* row_loss;          /* (N,) fp32: lse - x_t for valid rows, 0 otherwise */
    const float* mul;         /* () fp32 grad multiplier (grad_scale / n_valid) */
    int64_t N;
    int64_t V;
    int64_t ld;               /* logits row stride, elements */
    int64_t ldg;              /* grad row stride, elements */
    int64_t ignore_index;
} fxCEArgs;

/* Per row r: m, Z = max and sum(exp(x - m)) of logits[r]; valid = (t != ignore_index
 * && 0 <= t < V); row_loss[r] = valid ? m + log Z - x[t] : 0;
 * grad[r, :] = valid ? (softmax - onehot(t)) * (*mul) : 0.
 * Replaces _ce_rows + ce_fwd_grad (ml/fxlm/cross_entropy.py:47-59,
 * ml/fxlm/kernels/ce.hip:32-116). */
int fx_ce_fwd_grad(const fxCEArgs* args, void* stream);

/* loss = (sum_r row_loss[r]) * (*inv_n), summed in a fixed order (deterministic).
 * Replaces `loss_sum * inv_n` (ml/fxlm/cross_entropy.py:88, :139, :183). */
int fx_ce_loss_finalize(const float* row_loss, int64_t N, const float* inv_n,
                        float* loss, void* stream);

/* grad *= (*g) / applied[src]; applied[1 - src] = *g.  `applied` holds two floats
 * (the multiplier already in grad lives in slot src; the caller flips src after each
 * call), so no block reads the slot that is written.  src == -1: grad holds multiplier
 * 1 (applied is not read) and *g goes to applied[1].  Exits at once when the ratio is
 * 1, so the usual loss.backward() (g == 1) costs one tiny launch and no pass over grad.
 * Replaces _FusedCE.backward's `grad * g` (ml/fxlm/cross_entropy.py:90-93). */
int fx_ce_scale_grad(uint16_t* grad, int64_t numel, const float* g, float* applied,
                     int32_t src, void* stream);

/* s = (*g) * (gs ? 1 / *gs : inv_value); dw_out = bf16(dw * s) for the fp32 (nw,) weight
 * gradient and dx_out = bf16(dx * bf16(s)) for the bf16 (nx,) input gradient, in one pass; all
 * four buffers 16-byte aligned.  Replaces _LinearCE.backward's reciprocal, products and
 * cast (ml/fxlm/cross_entropy.py:141-148: gx = dx * (g * inv), gw = (dW * (g * inv)).to(dtype)),
 * with the same fp32 roundings. */
int fx_ce_lin_grad_scale(const float* dw, int64_t nw, const uint16_t* dx, int64_t nx, const float* g,
                         const float* gs, float inv_value, uint16_t* dw_out, uint16_t* dx_out,
                         void* stream);

/* fx_ce_lin_grad_scale for a bf16 dw: the weight gradient of a single-chunk linear-CE,
 * the one bf16 product, which fp32 represents exactly, so the result is bit for bit that
 * of converting dw to fp32 first (ml/fxlm/cross_entropy.py:135, 160-161) without the
 * fp32 copy. */
int fx_ce_lin_grad_scale_bf16w(const uint16_t* dw, int64_t nw, const uint16_t* dx, int64_t nx, const float* g,
                               const float* gs, float inv_value, uint16_t* dw_out, uint16_t* dx_out,
                               void* stream);

/* fx_ce_lin_grad_scale_bf16w in place: dw = bf16(dw * s), dx = bf16(dx * bf16(s)), the same
 * roundings (dw bf16 (nw,), dx bf16 (nx,), 16-byte aligned).  When s == 1 no value changes
 * (the products are exact), and the kernel returns without a pass over either buffer: the
 * usual training step, where the incoming gradient is the loss scale the head's gradients
 * were formed with.  Replaces the first backward's gx = dx * (g * inv), gw = (dW * (g * inv))
 * .to(dtype) of _LinearCE (ml/fxlm/cross_entropy.py:141-148), on the saved gradients. */
int fx_ce_lin_grad_scale_inplace(uint16_t* dw, int64_t nw, uint16_t* dx, int64_t nx, const float* g,
                                 const float* gs, float inv_value, void* stream);

/* ---- FlatAdamW ---------------------------------------------------------- */

#define FX_ADAMW_MAX_TENSORS 64

/* By-value tensor list; mirrors TensorList (ml/fxlm/kernels/optim.hip:15-21,
 * ml/fxlm/optim.py:28-35).  Gradients are bf16, contiguous, 16-byte aligned;
 * off[] are element offsets into the flat buffers (multiples of 8). */
typedef struct fxTensorList {
    const uint16_t* g[FX_ADAMW_MAX_TENSORS];
    int64_t off[FX_ADAMW_MAX_TENSORS];
    int64_t n[FX_ADAMW_MAX_TENSORS];
    int32_t wd[FX_ADAMW_MAX_TENSORS];
    int32_t count;
} fxTensorList;

/* Flat optimiser state and hyper-parameters. */
typedef struct fxAdamWState {
    float* master;            /* fp32 flat master weights */
    float* m;                 /* fp32 first moment */
    float* v;                 /* fp32 second moment */
    uint16_t* p16;            /* bf16 flat params (model parameters are views of it) */
    int32_t* step;            /* () step counter, incremented before bias correction */
    float* found_inf;         /* () 1.0 when any gradient is non-finite, else 0.0 */
    float* grad_norm;         /* () sqrt(sum g^2) / scale */
    float* scale;             /* () dynamic loss scale, updated in place */
    int32_t* growth;          /* () clean steps since the last scale change */
    float* work;              /* fx_adamw_workspace(...) bytes, 16-byte aligned */
    float lr, beta1, beta2, eps, weight_decay, max_grad_norm;
    float growth_factor;      /* 2.0 in the reference */
    float backoff_factor;     /* 0.5 in the reference */
    int32_t growth_interval;
} fxAdamWState;

/* Bytes of workspace fx_adamw_step needs for these tensor lists. */
int64_t fx_adamw_workspace(const fxTensorList* lists, int32_t nlists);

/* One optimiser step, fully on the device (no host synchronisation):
 *   sumsq = sum g^2 over all lists, bad = any non-finite g or non-finite sumsq;
 *   found_inf = bad; grad_norm = sqrt(sumsq)/scale; clip = bad ? 0 : min(1, max/(norm+1e-6));
 *   if !bad: step += 1 and, per element, g' = g*clip/scale;
 *            w -= lr*wd*w (wd flag); m = b1 m + (1-b1) g'; v = b2 v + (1-b2) g'^2;
 *            w -= lr*(m/(1-b1^step)) / (sqrt(v/(1-b2^step)) + eps); p16 = bf16(w);
 *   then the loss-scale update of torch._amp_update_scale_ (backoff on bad, growth
 *   after growth_interval clean steps).
 * Replaces FlatAdamW.step: adamw_sumsq + adamw_final + adamw_update +
 * torch._amp_update_scale_ (ml/fxlm/optim.py:136-173,
 * ml/fxlm/kernels/optim.hip:25-162). */
int fx_adamw_step(const fxAdamWState* state, const fxTensorList* lists, int32_t nlists,
                  void* stream);

/* Bytes of the buffer inside the library that fx_adamw_step_noalloc uses as its workspace:
 * 16 bytes of header plus 4 bytes per 8192-element chunk, so at most
 * (FX_ADAMW_NOALLOC_SCRATCH_BYTES / 4 - 4) * 8192 = 2,147,450,880 parameters per call. */
#define FX_ADAMW_NOALLOC_SCRATCH_BYTES (1 << 20)

/* fx_adamw_step with no workspace argument and no allocation: state->work is ignored and
 * the step's partial sums live in a device buffer inside the library, one per GPU (held
 * until the process ends; FX_ADAMW_NOALLOC_SCRATCH_BYTES).  Lists needing more return
 * FX_EINVAL before any launch.  Calls that overlap on one GPU (concurrent streams or host
 * threads) share that buffer and race; calls in stream order do not.  The buffer's device
 * address is looked up on the first call on each device.
 * No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, allocation-free harnesses).  This build does
 * not support or verify capturing a whole training step in a HIP graph; the step runs eagerly. */
int fx_adamw_step_noalloc(const fxAdamWState* state, const fxTensorList* lists, int32_t nlists,
                          void* stream);

/* ---- flash attention ------------------------------------------------------ */

/* Argument block of the attention kernels; mirrors AttnArgs
 * (ml/fxlm/kernels/attention.hip:35-47, ml/fxlm/attention.py:22-38) with bf16 tensors,
 * the head dimension as a field and one Delta workspace.
 * q, k, v, dq, dk, dv: (B, T, H, D) with unit stride along D and the element strides
 * below along b, t, h (views of a fused (B, T, 3, H, D) buffer are fine);
 * o, dout: (B, T, H, D) contiguous; lse, delta: (B, H, T) fp32.  Every bf16 tensor is
 * 16-byte aligned and its strides are multiples of 8 elements. */
typedef struct fxAttnArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const uint16_t* o;        /* forward output, read by the backward */
    const uint16_t* dout;     /* upstream gradient */
    uint16_t* o_out;          /* forward output */
    uint16_t* dq;
    uint16_t* dk;
    uint16_t* dv;
    const float* lse;         /* logsumexp from the forward, read by the backward */
    float* lse_out;           /* logsumexp written by the forward */
    float* delta;             /* backward workspace: rowsum(dout * o) */
    int64_t qsb, qst, qsh, ksb, kst, ksh, vsb, vst, vsh;
    int64_t dqb, dqt, dqh, dkb, dkt, dkh, dvb, dvt, dvh;
    int32_t B, T, H, D;       /* D in {64, 128} */
    float scale;              /* > 0 and finite (1/sqrt(D) in fxlm) */
    int32_t causal;
} fxAttnArgs;

/* O = softmax(Q K^T * scale [causal: key <= query]) V, lse = max + log(sum exp)
 * (-inf and O = 0 for a row with no visible key).  bf16 MFMA, fp32 online softmax.
 * Replaces _fwd + attn_fwd (ml/fxlm/attention.py:87-104,
 * ml/fxlm/kernels/attention.hip:103-224). */
int fx_attn_fwd(const fxAttnArgs* args, void* stream);

/* Delta = rowsum(dout * o); P = exp(S*scale - lse); dS = P * (dP - Delta) * scale;
 * dQ = dS K, dK = dS^T Q, dV = P^T dout (dP = dout V^T).  Two kernels: per query
 * tile (Delta and dQ), then per key tile (dK and dV).  No atomics: deterministic.
 * Replaces _bwd + attn_bwd_prep/_dkv/_dq (ml/fxlm/attention.py:107-134,
 * ml/fxlm/kernels/attention.hip:228-534). */
int fx_attn_bwd(const fxAttnArgs* args, void* stream);

/* ---- decode attention (KV cache) ------------------------------------------- */

/* One new query per (sequence, head) against the first lens[b] cached keys:
 * o[b, h] = softmax(scale q[b, h] . K[b, :lens[b], h]^T) V[b, :lens[b], h].
 * q element (b, h, d) at q[b*qsb + h*qsh + d]; cache element (b, t, h, d) at
 * k[b*ksb + t*kst + h*ksh + d] (same for v); o (B, H, D) contiguous; lse (B, H) or NULL;
 * work: fx_attn_decode_workspace(B, H, Tmax, D) bytes of fp32 (NULL when that is 0). */
typedef struct fxAttnDecodeArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const int32_t* lens;      /* (B,) device array, 0 <= lens[b] <= Tmax */
    uint16_t* o;
    float* lse;
    float* work;
    int64_t qsb, qsh, ksb, kst, ksh, vsb, vst, vsh;
    int32_t B, H, Tmax, D;    /* D in {64, 128} */
    float scale;              /* > 0 and finite */
    /* Optional (both or neither): the new token's key and value, knew[b*knb + h*knh + d]
     * (vnew likewise).  Key lens[b] - 1 is then taken from them and written into the
     * caches at that row in the same pass (no separate cache write).  NULL: every key
     * comes from the caches. */
    const uint16_t* knew;
    const uint16_t* vnew;
    int64_t knb, knh, vnb, vnh;
} fxAttnDecodeArgs;

int64_t fx_attn_decode_workspace(int32_t B, int32_t H, int32_t Tmax, int32_t D);

/* No counterpart in the reference, whose sampler re-runs the whole context through the
 * model for every new token (ml/fxlm/sample.py:62-73); this is the attention of a
 * KV-cache decoding step (bf16 in and out, fp32 softmax).  All
 * vectors 16-byte aligned, strides multiples of 8 elements. */
int fx_attn_decode(const fxAttnDecodeArgs* args, void* stream);

/* ---- fused (gather) linear ------------------------------------------------- */

/* Y = act(A W^T + bias), A (M, K): dense rows (A row m = X + m*ldx) when idx is NULL,
 * otherwise gathered windows A[m, w*F + f] = X[idx[m] + w, f] of X (R, F) (K = W*F,
 * F % 8 == 0; a window outside X reads as zeros).  W (N, K) bf16 contiguous, bias (N,)
 * or NULL, Y (M, N).  act: 0 identity, 1 GELU (tanh approximation), 2 GELU with H
 * receiving its derivative.  H (M, N), when not NULL, receives the pre-activation h
 * (act 0 and 1) or gelu_tanh'(h) (act 2: computed from the same exponential as the GELU,
 * for the backward's fx_linear_dgrad_gate / fx_gelu_bwd_gate); Xg (M, K), when not NULL,
 * the gathered A.
 * bf16 MFMA, fp32 accumulation.  K % 8 == 0.
 * Replaces FusedGatherLinear.forward + gather_gemm (ml/fxgpu/fused_linear.py:35-88,
 * ml/fxgpu/gather_gemm.hip:16-180) and the fc -> gelu_tanh of the GPT MLP
 * (ml/fxlm/model.py:71). */
int fx_linear_fwd(const uint16_t* X, int64_t ldx, const int32_t* idx, int64_t F, int64_t R,
                  const uint16_t* W, const uint16_t* bias, uint16_t* Y, uint16_t* H,
                  uint16_t* Xg, int64_t M, int64_t N, int64_t K, int32_t act, void* stream);

/* Dense-row form of fx_linear_fwd with two fusions for inference:
 *   Y = act(norm(X) W^T + bias) + res
 * norm(X) = X * rsqrt(mean(X^2, row) + eps) * norm_w, rounded to bf16 as the RMSNorm
 * forward writes it, when norm_w (K,) is given (M <= 64 rows: the few-row kernel
 * computes the rows' rstd itself); res (M, N) row stride ldres, when given, is added
 * after the activation.  X (M, K) row stride ldx, W (N, K) contiguous, bias (N,) or
 * NULL, Y (M, N) contiguous, H (M, N) or NULL receives the pre-activation (before the
 * residual).  X, W and norm_w 16-byte aligned, K % 8 == 0.
 * No counterpart in the reference: it folds the RMSNorm before a block's qkv / fc and
 * the residual sum after its proj / fc2 (ml/fxlm/model.py:60-71) into the projection,
 * for decoding steps whose few rows make every extra kernel launch count. */
typedef struct fxLinearArgs {
    const uint16_t* X;
    int64_t ldx;
    const uint16_t* W;
    const uint16_t* bias;
    const uint16_t* res;
    int64_t ldres;
    const uint16_t* norm_w;
    uint16_t* Y;
    uint16_t* H;
    int64_t M, N, K;
    float eps;
    int32_t act;
} fxLinearArgs;

int fx_linear_fwd_ex(const fxLinearArgs* args, void* stream);

/* dh = dy * gelu_tanh'(h), elementwise over n bf16 values (16-byte aligned buffers).
 * The activation half of the fused linear's backward (the reference's torch autograd
 * of F.gelu(approximate="tanh"), ml/fxlm/model.py:71). */
int fx_gelu_bwd(const uint16_t* dy, const uint16_t* h, uint16_t* dh, int64_t n, void* stream);

/* dh = dy * g, elementwise over n bf16 values (16-byte aligned buffers), g = gelu_tanh'(h)
 * as fx_linear_fwd with act 2 stores it.  The same backward as fx_gelu_bwd (the reference's
 * autograd of F.gelu(approximate="tanh"), ml/fxlm/model.py:71) with the derivative taken
 * in the forward, from the fp32 pre-activation, and saved in place of it. */
int fx_gelu_bwd_gate(const uint16_t* dy, const uint16_t* g, uint16_t* dh, int64_t n, void* stream);

/* Bytes of workspace fx_embedding_bwd needs for n positions, a V-row table and rows of D
 * values (0 when n, V or D is not positive). */
int64_t fx_embedding_bwd_workspace(int64_t n, int64_t V, int64_t D);

/* Token-embedding gradient: grad (V, D) bf16, row-major, = for every row v the sum of dy[t]
 * over the positions t with idx[t] == v; rows no position selects are zero and ids outside
 * [0, V) select nothing.  The positions are sorted by (id, t) into slots 0.. (stable), cut
 * into segments of 32 slots; an id's rows are summed in fp32 in increasing t within each
 * segment, its segments' sums are added in segment order, and the total is rounded once to
 * bf16.  idx int64 (n,), dy (n, D) with row stride ldy (16-byte aligned rows, D a multiple of
 * 8), work of fx_embedding_bwd_workspace(n, V, D) bytes (16-byte aligned).  Deterministic (a
 * stable counting sort, no atomics), with launch sizes that depend on n and V only, and no
 * wave summing more than 32 rows whatever the ids.  Replaces torch's nn.Embedding backward
 * behind the reference's tok_emb(idx) (ml/fxlm/model.py:82,118). */
int fx_embedding_bwd(const int64_t* idx, int64_t n, const uint16_t* dy, int64_t ldy, uint16_t* grad, int64_t V,
                     int64_t D, void* work, void* stream);

/* Bytes of fp32 workspace fx_linear_wgrad needs for an (M, N) weight gradient over K
 * tokens (0: none; the K split depends on the device's CU count). */
int64_t fx_linear_wgrad_workspace(int64_t M, int64_t N, int64_t K);

/* Weight gradient dW (M, N) = dY^T X, dY (K, M) with row stride ldy, X (K, N) with row
 * stride ldx, dW row stride ldw; bf16 in and out, fp32 accumulation, the K (token)
 * dimension split over workgroups and the fp32 partials (in `work`) summed in a fixed
 * order.  M, N, ldy, ldx, ldw multiples of 8; 16-byte aligned buffers.
 * Replaces the rocBLAS dW = g^T Xg of FusedGatherLinear.backward
 * (ml/fxgpu/fused_linear.py:90-101) and the dense layers' weight gradients of the GPT
 * (ml/fxlm/model.py:22-130, torch autograd of nn.Linear). */
int fx_linear_wgrad(const uint16_t* dY, int64_t ldy, const uint16_t* X, int64_t ldx, uint16_t* dW,
                    int64_t ldw, float* work, int64_t M, int64_t N, int64_t K, void* stream);

/* Input gradient dX (M, N) = dY (M, K) W (K, N), W the layer's (out, in) weight with row
 * stride ldw, dY row stride ldy, dX (and H) row stride ldx; bf16 in and out, fp32
 * accumulation.  With H non-null (the pre-activation of a GELU(tanh) layer feeding this
 * one, (M, N)): dX = bf16(bf16(dY W) gelu'(H)), the GELU backward of fx_gelu_bwd folded
 * into the product's epilogue, bit for bit the unfused pair.  Whole tiles only: M % 256 == 0,
 * N % 256 == 0 or N % 192 == 0, K % 32 == 0 and K >= 128, row strides multiples of 8,
 * 16-byte aligned buffers; other shapes return FX_EINVAL before any launch.
 * Replaces the dense layers' input gradients of the GPT (ml/fxlm/model.py:22-130, torch
 * autograd of nn.Linear: dY W) and, with H, the F.gelu backward between fc and fc2
 * (ml/fxlm/model.py:71). */
int fx_linear_dgrad(const uint16_t* dY, int64_t ldy, const uint16_t* W, int64_t ldw, const uint16_t* H,
                    uint16_t* dX, int64_t ldx, int64_t M, int64_t N, int64_t K, void* stream);

/* fx_linear_dgrad with G (M, N) the GELU derivative at this product's output columns, as
 * fx_linear_fwd with act 2 stores it: dX = bf16(bf16(dY W) G), bit for bit fx_linear_dgrad
 * without H followed by fx_gelu_bwd_gate; the epilogue multiplies instead of evaluating the
 * derivative.  Same shapes, strides and alignment as fx_linear_dgrad; G row stride ldx.
 * Replaces the GPT MLP's fc2 input gradient and the F.gelu backward after it
 * (ml/fxlm/model.py:71, torch autograd of nn.Linear and F.gelu(approximate="tanh")). */
int fx_linear_dgrad_gate(const uint16_t* dY, int64_t ldy, const uint16_t* W, int64_t ldw, const uint16_t* G,
                         uint16_t* dX, int64_t ldx, int64_t M, int64_t N, int64_t K, void* stream);

/* ---- fused linear cross-entropy ------------------------------------------- */

/* Bytes of workspace fx_lce_fwd needs for M rows of an (V, K) head, or 0 when the fused
 * kernels do not take the shape (they need V % 256 == 0 or V % 192 == 0, K % 32 == 0 and
 * K >= 128); such heads stay on the mm + fx_ce_fwd_grad chunk loop. */
int64_t fx_lce_workspace(int64_t M, int64_t V, int64_t K);

/* Loss half of a linear cross-entropy with the logits never stored: logits = X E^T
 * (X (M, K) bf16 with row stride ldx, E (V, K) bf16 contiguous) are formed tile by tile in
 * MFMA accumulators, rounded to bf16 as a stored logit is, and reduced on the spot to a
 * (max, sum exp(x - max)) pair per row and tile plus the target's logit; a second kernel
 * merges the pairs in a fixed order into stat[r] = (M_r, Z_r) (fp32 pairs) and writes
 * row_loss[r] = M_r + log Z_r - x_t (0 for rows whose target is ignore_index or outside
 * [0, V)).  work: fx_lce_workspace bytes, 16-byte aligned.  Replaces the chunk loop's
 * torch.mm + ce_fwd_grad loss pass (ml/fxlm/cross_entropy.py:127-130, :170-183). */
int fx_lce_fwd(const uint16_t* X, int64_t ldx, const uint16_t* E, const int64_t* target, int64_t ignore_index,
               void* work, float* stat, float* row_loss, int64_t M, int64_t V, int64_t K, void* stream);

/* Gradient half: the same product again, and dl = exp(x - M_r) (mul / Z_r) - mul [c == t]
 * written as bf16 (row stride ldd, zero rows for ignored targets), given fx_lce_fwd's stat
 * and the device scalar mul (grad_scale / n_valid): the dlogits of fx_ce_fwd_grad without
 * the logits in memory.  Replaces the chunk loop's torch.mm + ce_fwd_grad gradient pass
 * (ml/fxlm/cross_entropy.py:127-130). */
int fx_lce_grad(const uint16_t* X, int64_t ldx, const uint16_t* E, const int64_t* target, int64_t ignore_index,
                const float* stat, const float* mul, uint16_t* dl, int64_t ldd, int64_t M, int64_t V, int64_t K,
                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FX_ABI_H */
