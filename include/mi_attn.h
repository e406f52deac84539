/*
 * mi_attn.h — C ABI of the MI355X (gfx950) attention hot path.
 *
 * Causal / non-causal flash attention (forward with saved log-sum-exp, backward
 * producing dQ, dK, dV) and the interleaved-pair rotary position embedding, plus
 * the train step's fused vocabulary cross entropy, RMSNorm, SwiGLU and AdamW
 * step.
 * Every entry point takes plain device pointers, element strides and sizes, and
 * enqueues its kernels on the given HIP stream (a `hipStream_t`, passed as
 * `void*`; NULL means the null stream).  Nothing here allocates, frees or
 * synchronises: the caller owns every output and workspace buffer.
 *
 * Tensor conventions
 *   - attention tensors are logically [B, H, S, D]; `*_strides` holds the four
 *     element strides in that order (batch, head, seq, dim).  The dim stride
 *     must be 1 (other strides are free).
 *   - lse is dense fp32 [B, H, S] (natural-log log-sum-exp of the scaled,
 *     masked scores); the backward workspace is dense fp32 [2, B, H, S]
 *     (delta = rowsum(dO * O), then lse * log2(e); see mi_attn_bwd).
 *   - rope tensors are logically [S, B, H, D] (the layout the model hands to
 *     RoPE); the cos/sin tables are [S, D/2] with two element strides.
 *   - dtypes: MI_F32, MI_F16, MI_BF16.  Attention runs on bf16/f16 MFMA when
 *     every row is 16-byte aligned, for D = 16, 32, 64 or 128 and any S (16
 *     and 32 in the D = 64 kernels' layout, the padding staged as zeros; no
 *     row at or past S is read or written); every other supported case runs
 *     on an exact-fp32 VALU kernel.  Arithmetic is fp32 in all kernels.
 *
 * Errors: a non-zero mi_status; mi_last_error() gives a message for the
 * calling thread.  Arguments are validated before anything is launched.
 */
#ifndef MI_ATTN_H
#define MI_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The enums are int-sized in C; in C++ they get int as a fixed underlying type
 * (same size and values), so that any int a C caller passes is a valid value
 * for the implementation to reject. */
#ifdef __cplusplus
#define MI_ENUM_INT : int
#else
#define MI_ENUM_INT
#endif

typedef enum MI_ENUM_INT {
  MI_OK = 0,
  MI_ERR_INVALID_ARGUMENT = 1, /* bad shape, stride, pointer or dtype */
  MI_ERR_UNSUPPORTED = 2,      /* valid request that no kernel here covers */
  MI_ERR_LAUNCH = 3            /* the HIP runtime refused a launch */
} mi_status;

typedef enum MI_ENUM_INT { MI_F32 = 0, MI_F16 = 1, MI_BF16 = 2 } mi_dtype;

/* Library version, (major << 16) | minor. */
int mi_version(void);

/* Static text for a status code. */
const char* mi_status_str(mi_status status);

/* Message describing the last failure on the calling thread ("" if none). */
const char* mi_last_error(void);

/*
 * Flash-attention forward: O = softmax(Q K^T * scale + mask) V, and
 * lse[b,h,i] = log sum_j exp(scale * q_i . k_j) over unmasked j.
 * Replaces the launch of `_attn_fwd` inside FlashAttn.forward,
 * core/myFlashAttn.py:198-285 (grid :234-236, launch :249-277, M alloc :240).
 */
mi_status mi_attn_fwd(mi_dtype dtype, int B, int H, int S, int D, int causal,
                      float scale,
                      const void* q, const int64_t q_strides[4],
                      const void* k, const int64_t k_strides[4],
                      const void* v, const int64_t v_strides[4],
                      void* o, const int64_t o_strides[4],
                      float* lse, void* stream);

/*
 * Backward workspace `ws`: 2*B*H*S fp32 values, caller-allocated, written by
 * mi_attn_bwd_preprocess and read by the gradient launches:
 *   ws[0 .. B*H*S)          delta[b,h,s] = rowsum(dO * O)  (the reference's D)
 *   ws[B*H*S .. 2*B*H*S)    lse[b,h,s] * log2(e)           (exp2 argument scale)
 * both indexed (b*H + h)*S + s.
 *
 * Flash-attention backward: the workspace, then dQ, dK, dV.  lse is the
 * forward's output (natural log).
 * Replaces FlashAttn.backward's three launches, core/myFlashAttn.py:288-441
 * (`_attn_bwd_precompute` :330, `_attn_bwd_LoopQ` :365, `_attn_bwd_LoopKV` :409).
 */
mi_status mi_attn_bwd(mi_dtype dtype, int B, int H, int S, int D, int causal,
                      float scale,
                      const void* q, const int64_t q_strides[4],
                      const void* k, const int64_t k_strides[4],
                      const void* v, const int64_t v_strides[4],
                      const void* o, const int64_t o_strides[4],
                      const void* dout, const int64_t dout_strides[4],
                      const float* lse, float* ws,
                      void* dq, const int64_t dq_strides[4],
                      void* dk, const int64_t dk_strides[4],
                      void* dv, const int64_t dv_strides[4],
                      void* stream);

/*
 * mi_attn_bwd for attention on rotated q, k whose gradients are wanted with
 * respect to the unrotated ones: dQ and dK leave inverse-rotated by the RoPE
 * tables (interleaved pairs, the rotation of mi_rope with inverse = 1,
 * evaluated on dQ and dK rounded to `dtype` first, so the result equals
 * mi_attn_bwd followed by mi_rope_qk(inverse = 1) on dq, dk in place, bit for
 * bit).  On the matrix-core path at D = 64 or 128 with 16-bit tables whose
 * angles are contiguous and whose row starts are 4-angle aligned (the
 * model's), the rotation is applied as the kernels store dQ and dK, saving the
 * separate read and write of both; otherwise the two run one after the other
 * (a shape past the separate pass's launch limit, 2^31 angle pairs, is then
 * refused with MI_ERR_UNSUPPORTED before anything is enqueued).  cos / sin:
 * [>= S rows, D/2 angles], strides in elements, dtype tab_dtype.  Replaces the attention block's backward pair,
 * FlashAttn.backward (core/myFlashAttn.py:288-441) then TritonRoPE.backward
 * on dq and dk (core/rope_triton.py:50-72), as driven by the autograd of
 * core/transformer_layer.py:42-61.
 */
mi_status mi_attn_bwd_rope(mi_dtype dtype, int B, int H, int S, int D, int causal,
                           float scale,
                           const void* q, const int64_t q_strides[4],
                           const void* k, const int64_t k_strides[4],
                           const void* v, const int64_t v_strides[4],
                           const void* o, const int64_t o_strides[4],
                           const void* dout, const int64_t dout_strides[4],
                           const float* lse, float* ws,
                           void* dq, const int64_t dq_strides[4],
                           void* dk, const int64_t dk_strides[4],
                           void* dv, const int64_t dv_strides[4],
                           mi_dtype tab_dtype,
                           const void* cos_tab, const int64_t cos_strides[2],
                           const void* sin_tab, const int64_t sin_strides[2],
                           void* stream);

/*
 * mi_attn_bwd is mi_attn_bwd_preprocess followed by mi_attn_bwd_grads.  The
 * latter produces dQ, dK and dV in one launch where the matrix-core path
 * applies (dK/dV and dQ work interleaved in one grid) and otherwise runs
 * mi_attn_bwd_dkdv then mi_attn_bwd_dq.  The four are exposed separately, one
 * per kernel of the reference's backward, for callers that schedule them.
 */
mi_status mi_attn_bwd_grads(mi_dtype dtype, int B, int H, int S, int D, int causal,
                            float scale,
                            const void* q, const int64_t q_strides[4],
                            const void* k, const int64_t k_strides[4],
                            const void* v, const int64_t v_strides[4],
                            const void* dout, const int64_t dout_strides[4],
                            const float* lse, const float* ws,
                            void* dq, const int64_t dq_strides[4],
                            void* dk, const int64_t dk_strides[4],
                            void* dv, const int64_t dv_strides[4],
                            void* stream);

/*
 * The backward workspace: delta = rowsum(dO * O) (fp32) and lse * log2(e).
 * Replaces the `_attn_bwd_precompute` launch, core/myFlashAttn.py:323-346.
 */
mi_status mi_attn_bwd_preprocess(mi_dtype dtype, int B, int H, int S, int D,
                                 const void* o, const int64_t o_strides[4],
                                 const void* dout, const int64_t dout_strides[4],
                                 const float* lse, float* ws, void* stream);

/*
 * dK and dV: per key tile, loop over query tiles (needs lse and the workspace).
 * Replaces the `_attn_bwd_LoopQ` launch, core/myFlashAttn.py:349-396.
 */
mi_status mi_attn_bwd_dkdv(mi_dtype dtype, int B, int H, int S, int D, int causal,
                           float scale,
                           const void* q, const int64_t q_strides[4],
                           const void* k, const int64_t k_strides[4],
                           const void* v, const int64_t v_strides[4],
                           const void* dout, const int64_t dout_strides[4],
                           const float* lse, const float* ws,
                           void* dk, const int64_t dk_strides[4],
                           void* dv, const int64_t dv_strides[4],
                           void* stream);

/*
 * dQ: per query tile, loop over key tiles (needs lse and the workspace).
 * Replaces the `_attn_bwd_LoopKV` launch, core/myFlashAttn.py:398-439.
 */
mi_status mi_attn_bwd_dq(mi_dtype dtype, int B, int H, int S, int D, int causal,
                         float scale,
                         const void* q, const int64_t q_strides[4],
                         const void* k, const int64_t k_strides[4],
                         const void* v, const int64_t v_strides[4],
                         const void* dout, const int64_t dout_strides[4],
                         const float* lse, const float* ws,
                         void* dq, const int64_t dq_strides[4],
                         void* stream);

/*
 * Rotary embedding on one tensor x [S,B,H,D] with interleaved pairs (2i, 2i+1):
 *   forward (inverse = 0): (e, o) -> (e*c - o*s, e*s + o*c)
 *   inverse (inverse = 1): (e, o) -> (e*c + o*s, o*c - e*s)   (rotation by -theta)
 * with c = cos[s, i], s = sin[s, i].  x_dtype and tab_dtype are independent.
 * The tables must hold at least S rows of D/2 angles (their extent is not
 * passed, so it is the caller's to check).
 * In place: `out` may be `x` itself with the same strides (every element is
 * read and then written by the same lane); any other overlap of out with x is
 * undefined.
 * Replaces `_rope_kernel` launches in TritonRoPE.forward / .backward,
 * core/rope_triton.py:10-72 (launch :33-40 and :63-70, kernel :74-141).
 */
mi_status mi_rope(mi_dtype x_dtype, mi_dtype tab_dtype, int S, int B, int H, int D,
                  int inverse,
                  const void* x, const int64_t x_strides[4],
                  const void* cos_tab, const int64_t cos_strides[2],
                  const void* sin_tab, const int64_t sin_strides[2],
                  void* out, const int64_t out_strides[4],
                  void* stream);

/*
 * The same rotation applied to q and k (same shape, dtype and tables) in one
 * launch.  In place as for mi_rope: q_out may be q and k_out may be k (same
 * pointers and strides); the outputs must not otherwise overlap either input.
 * Replaces the two TritonRoPE.apply calls of apply_rope_qk,
 * core/rope_triton.py:147-148, and their two backward launches.
 */
mi_status mi_rope_qk(mi_dtype x_dtype, mi_dtype tab_dtype, int S, int B, int H, int D,
                     int inverse,
                     const void* q, const int64_t q_strides[4],
                     const void* k, const int64_t k_strides[4],
                     const void* cos_tab, const int64_t cos_strides[2],
                     const void* sin_tab, const int64_t sin_strides[2],
                     void* q_out, const int64_t q_out_strides[4],
                     void* k_out, const int64_t k_out_strides[4],
                     void* stream);

/*
 * Copy of two [S, B, H, D] tensors (q and k views, any 16-byte aligned row
 * strides) into outputs of any 16-byte aligned row strides: the relayout that
 * FlashAttn.forward's .contiguous() calls perform (core/myFlashAttn.py:206-208),
 * run with mi_rope_qk's launch (the same items, grid and memory accesses,
 * without the rotation and the tables), so it is also the streaming ceiling
 * of that launch.  Requires unit dim strides, D a multiple of 16 bytes and
 * 16-byte aligned bases and row strides (MI_ERR_UNSUPPORTED otherwise).
 */
mi_status mi_copy_qk(mi_dtype dtype, int S, int B, int H, int D,
                     const void* q, const int64_t q_strides[4],
                     const void* k, const int64_t k_strides[4],
                     void* q_out, const int64_t q_out_strides[4],
                     void* k_out, const int64_t k_out_strides[4],
                     void* stream);

/*
 * Softmax cross entropy of each logits row against an integer target, at one
 * tensor-parallel rank (the whole vocabulary on this GPU).  Replaces the
 * forward of _VocabParallelCrossEntropy, core/tensor_parallel/loss.py:9-57:
 *   loss[r] = log sum_j exp(z_rj - m_r) - (z_r,t - m_r),  m_r = max_j z_rj,
 * where a target outside [0, vocab) is masked: its shifted logit counts as 0
 * (:33-41).  Instead of the normalised softmax (:54-56) it saves
 * lse[r] = m_r + log sum_j exp(z_rj - m_r), fp32, for mi_xent_bwd.
 * logits: rows of `vocab` elements, `row_stride` elements apart (any alignment);
 * target: int64 [rows]; loss: [rows] in the logits dtype.  Row statistics are
 * fp32.
 */
mi_status mi_xent_fwd(mi_dtype dtype, int64_t rows, int64_t vocab, const void* logits,
                      int64_t row_stride, const int64_t* target, void* loss, float* lse,
                      void* stream);

/*
 * Gradient of mi_xent_fwd: grad[r, j] = (exp(z_rj - lse[r]) - [j == t_r]) *
 * grad_loss[r], with no -1 for a masked target.  Replaces
 * _VocabParallelCrossEntropy.backward, core/tensor_parallel/loss.py:59-72.
 * grad_logits may be the logits buffer itself (same row stride): each element
 * is read before it is overwritten.  Any other overlap is undefined.
 */
mi_status mi_xent_bwd(mi_dtype dtype, int64_t rows, int64_t vocab, const void* logits,
                      int64_t row_stride, const int64_t* target, const float* lse,
                      const void* grad_loss, void* grad_logits, int64_t grad_row_stride,
                      void* stream);

/*
 * RMSNorm forward over `rows` rows of `hidden` elements.  Replaces
 * RMSNorm.forward, core/normalization.py:13-25:
 *   r = rsqrt(mean(x^2) + eps)   (fp32),   y = round_x(x * r) * weight
 * where round_x rounds to x's dtype (:23) and the product is taken in the
 * promotion of x's and weight's dtypes (:24).  weight ([hidden]) has x's dtype
 * or is fp32; y has weight's dtype if that is fp32, else x's.  rstd ([rows],
 * fp32) receives r for mi_rmsnorm_bwd.  Row strides are in elements.
 */
mi_status mi_rmsnorm_fwd(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                         float eps, const void* x, int64_t x_row_stride, const void* weight,
                         void* y, int64_t y_row_stride, float* rstd, void* stream);

/* fp32 elements of workspace mi_rmsnorm_bwd needs for this shape (0 if invalid). */
int64_t mi_rmsnorm_bwd_workspace(int64_t rows, int64_t hidden);

/*
 * RMSNorm backward: dx (x's dtype) and dweight (weight's dtype) from dy (y's
 * dtype), x, weight and the forward's rstd -- the gradients autograd derives
 * for core/normalization.py:13-25, computed in fp32:
 *   dn = dy * weight;  dx = r dn - x r^3 mean(dn * x);
 *   dweight = sum over rows of dy * round_x(x r).
 * dweight is reduced through `workspace` in a fixed order (deterministic, and
 * the same on every device).  dx may alias dy when both have the same dtype
 * and row stride.
 */
mi_status mi_rmsnorm_bwd(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                         const void* x, int64_t x_row_stride, const void* weight,
                         const float* rstd, const void* dy, int64_t dy_row_stride, void* dx,
                         int64_t dx_row_stride, void* dweight, float* workspace,
                         int64_t workspace_elems, void* stream);

/*
 * RMSNorm with the residual add in front: the `residual + branch` of
 * TransformerLayer.forward (core/transformer_layer.py:96, :102) followed by the
 * RMSNorm that reads the sum (the next post_attention_norm / input_norm, or the
 * final norm), core/normalization.py:13-25.  Writes
 *   sum = round_x(x + res)          (x's dtype: torch's add of two such tensors)
 * and y, rstd of mi_rmsnorm_fwd over sum.  x (the residual stream), res (the
 * branch output) and sum have x's dtype; sum may alias x or res (each row is
 * read whole before any of it is written).
 */
mi_status mi_rmsnorm_add_fwd(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                             float eps, const void* x, int64_t x_row_stride, const void* res,
                             int64_t res_row_stride, const void* weight, void* sum,
                             int64_t sum_row_stride, void* y, int64_t y_row_stride, float* rstd,
                             void* stream);

/*
 * Backward of mi_rmsnorm_add_fwd: mi_rmsnorm_bwd over `sum` (the forward's
 * output, in place of x) with the gradient `dsum` that reaches the sum from its
 * other use added to dx:
 *   dx = round_x(round_x(r dn - sum r^3 mean(dn * sum)) + dsum),
 * the two roundings of autograd's norm backward and gradient accumulation.
 * dx is the gradient of both x and res.  dx may alias dsum, or dy under the
 * condition of mi_rmsnorm_bwd.  workspace as mi_rmsnorm_bwd.
 */
mi_status mi_rmsnorm_add_bwd(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                             const void* sum, int64_t sum_row_stride, const void* weight,
                             const float* rstd, const void* dy, int64_t dy_row_stride,
                             const void* dsum, int64_t dsum_row_stride, void* dx,
                             int64_t dx_row_stride, void* dweight, float* workspace,
                             int64_t workspace_elems, void* stream);

/*
 * mi_rmsnorm_bwd and mi_rmsnorm_add_bwd with dweight accumulated instead of
 * written: dweight[j] = round_w(dweight[j] + round_w(sum over rows)), the
 * gradient the norm's backward returns followed by autograd's accumulation of
 * it into an existing weight gradient (AccumulateGrad, for the weight of
 * core/normalization.py:8-11 whose .grad is the optimizer's flat buffer view,
 * core/optimizer.py:39-70), bitwise as the two steps round, without the
 * separate [hidden] gradient and the extra launch.  Other arguments and
 * conditions as those two.
 */
mi_status mi_rmsnorm_bwd_acc(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                             const void* x, int64_t x_row_stride, const void* weight,
                             const float* rstd, const void* dy, int64_t dy_row_stride, void* dx,
                             int64_t dx_row_stride, void* dweight, float* workspace,
                             int64_t workspace_elems, void* stream);
mi_status mi_rmsnorm_add_bwd_acc(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows,
                                 int64_t hidden, const void* sum, int64_t sum_row_stride,
                                 const void* weight, const float* rstd, const void* dy,
                                 int64_t dy_row_stride, const void* dsum, int64_t dsum_row_stride,
                                 void* dx, int64_t dx_row_stride, void* dweight, float* workspace,
                                 int64_t workspace_elems, void* stream);

/*
 * SwiGLU on the fused gate_up projection: rows of 2*inter elements, gate in
 * columns [0, inter), up in [inter, 2*inter).  Replaces
 * `gate, up = gate_up.chunk(2, dim=-1); x = F.silu(gate) * up`,
 * core/mlp.py:25-28:  h = round(round(silu(gate)) * up), each product rounded to
 * the dtype as torch's two ops do; h has rows of inter elements.
 */
mi_status mi_swiglu_fwd(mi_dtype dtype, int64_t rows, int64_t inter, const void* gate_up,
                        int64_t gate_up_row_stride, void* out, int64_t out_row_stride,
                        void* stream);

/*
 * Gradient of mi_swiglu_fwd as autograd evaluates the reference's ops (mul,
 * silu_backward, then the chunk's concatenation): dgate_up rows of 2*inter
 * elements, d_gate = round(round(dout*up) * silu'(gate)), d_up = round(dout *
 * round(silu(gate))), written in place of the concatenation.
 */
mi_status mi_swiglu_bwd(mi_dtype dtype, int64_t rows, int64_t inter, const void* gate_up,
                        int64_t gate_up_row_stride, const void* dout, int64_t dout_row_stride,
                        void* dgate_up, int64_t dgate_up_row_stride, void* stream);

/* fp32 elements of workspace mi_grad_sumsq needs (result in element 0). */
int64_t mi_adamw_workspace(void);

/*
 * workspace[0] = sum of grad^2 over n elements in fp32, reduced in a fixed
 * order (deterministic).  Replaces the local norm of
 * DistributedOptimizer._clip_grad_norm, core/optimizer.py:100, at one rank.
 */
mi_status mi_grad_sumsq(mi_dtype grad_dtype, int64_t n, const void* grad, float* workspace,
                        int64_t workspace_elems, void* stream);

/*
 * One AdamW step over flat buffers, with gradient clipping and the copy into
 * the model's parameter buffer.  Replaces DistributedOptimizer.step at one rank,
 * core/optimizer.py:79-104, with torch.optim.AdamW (train.py:130-138):
 *   if clip > 0 and norm = sqrt(*grad_sumsq) > clip:
 *       g = round_grad(g * clip / (norm + 1e-6))               (:102-104)
 *   p = p * weight_decay_factor                 (weight_decay_factor = 1 - lr*wd)
 *   m = m + lerp_weight * (g - m)               (lerp_weight = 1 - beta1)
 *   v = v * beta2 + one_minus_beta2 * g * g
 *   p = p - step_size * m / (sqrt(v) / bias_correction2_sqrt + eps)
 *       (step_size = lr / (1 - beta1^t), bias_correction2_sqrt = sqrt(1 - beta2^t))
 *   param = round_param(p)                      (the all-gather into the bf16 buffer, :95)
 * master, exp_avg, exp_avg_sq are fp32 [n], updated in place; param may be
 * NULL.  grad_sumsq is a device pointer (workspace of mi_grad_sumsq): nothing
 * is read back to the host.
 */
mi_status mi_adamw_step(mi_dtype grad_dtype, mi_dtype param_dtype, int64_t n, const void* grad,
                        float* master, float* exp_avg, float* exp_avg_sq, void* param,
                        float weight_decay_factor, float lerp_weight, float beta2,
                        float one_minus_beta2, float step_size, float bias_correction2_sqrt,
                        float eps, float clip, const float* grad_sumsq, void* stream);

/*
 * mi_attn_bwd without the workspace argument, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  It has no counterpart in the reference.
 * The workspace lives in a library-owned static device array of
 * 2 * MI_ATTN_NOALLOC_MAX_ROWS floats (8 MiB) on each GPU the library runs on,
 * held until the process ends; its address is looked up once per device on
 * the first call there (hipGetSymbolAddress, with that device made current
 * for the lookup).  Make that first call on each device outside stream
 * capture; later calls only enqueue kernels and may be captured into a HIP
 * graph and replayed.  B*H*S must not exceed MI_ATTN_NOALLOC_MAX_ROWS
 * (MI_ERR_INVALID_ARGUMENT otherwise, before anything is enqueued).  The call
 * allocates nothing.  Every call on one GPU shares that array: calls that
 * overlap on one GPU (other streams, other threads) race and must be
 * serialised by the caller.  Results are those of mi_attn_bwd (same kernels).
 */
#define MI_ATTN_NOALLOC_MAX_ROWS (1 << 20)
mi_status mi_attn_bwd_noalloc(mi_dtype dtype, int B, int H, int S, int D, int causal,
                              float scale,
                              const void* q, const int64_t q_strides[4],
                              const void* k, const int64_t k_strides[4],
                              const void* v, const int64_t v_strides[4],
                              const void* o, const int64_t o_strides[4],
                              const void* dout, const int64_t dout_strides[4],
                              const float* lse,
                              void* dq, const int64_t dq_strides[4],
                              void* dk, const int64_t dk_strides[4],
                              void* dv, const int64_t dv_strides[4],
                              void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI_ATTN_H */
