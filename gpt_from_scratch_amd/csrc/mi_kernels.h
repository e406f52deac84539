// mi_kernels.h — argument blocks and host launchers shared between the kernel
// translation units and the C ABI (capi.hip).  Internal to the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi {

// One attention tensor: base pointer and element strides (batch, head, seq);
// the dim stride is 1 by contract.
struct TensorArg {
  const void* ptr;
  int64_t sb, sh, ss;
};

// Rotary tables for an inverse rotation fused into the attention backward's
// dQ / dK stores: cos / sin [>= S rows, D/2 angles], element strides, table
// dtype (mi_dtype values).  cos == nullptr: no rotation.
struct RopeTab {
  const void* cos;
  const void* sin;
  int64_t cs_s, cs_i, ss_s, ss_i;
  int tdt;
};

struct AttnArgs {
  TensorArg q, k, v, o, dout, dq, dk, dv;
  float* lse;
  float* delta;        // backward workspace [2, B, H, S]: delta, then lse2
  const float* lse2;   // lse * log2(e) (= delta + B*H*S), written by the preprocess
  int B, H, S, D;
  float scale;       // softmax scale (1/sqrt(D) in the model)
  float scale_log2;  // scale * log2(e)
  int causal;
  RopeTab rope;        // backward only: dQ and dK stored inverse-rotated
};

// Kernel-family launchers.  Each returns hipSuccess or the launch error.
// `dtype` uses mi_dtype values (0 f32, 1 f16, 2 bf16).
hipError_t launch_attn_fwd_mfma(int dtype, const AttnArgs& a, hipStream_t st);
hipError_t launch_attn_bwd_dkdv_mfma(int dtype, const AttnArgs& a, hipStream_t st);
// dK/dV and dQ in one launch (same results as the two launches above).
hipError_t launch_attn_bwd_mfma(int dtype, const AttnArgs& a, hipStream_t st);
hipError_t launch_attn_bwd_dq_mfma(int dtype, const AttnArgs& a, hipStream_t st);
hipError_t launch_attn_fwd_valu(int dtype, const AttnArgs& a, hipStream_t st);
hipError_t launch_attn_bwd_dkdv_valu(int dtype, const AttnArgs& a, hipStream_t st);
hipError_t launch_attn_bwd_dq_valu(int dtype, const AttnArgs& a, hipStream_t st);
hipError_t launch_attn_delta(int dtype, const AttnArgs& a, hipStream_t st);

// Which D values each family is instantiated for.
bool mfma_supports(int dtype, int D, int S);
bool valu_supports(int D);

struct RopeTensor {
  const void* in;
  void* out;
  int64_t is_s, is_b, is_h, is_d;  // input strides
  int64_t os_s, os_b, os_h, os_d;  // output strides
};

struct RopeArgs {
  RopeTensor t[2];
  int ntensors;
  const void* cos_tab;
  const void* sin_tab;
  int64_t cs_s, cs_i, ss_s, ss_i;  // table strides (position, pair index)
  int S, B, H, D;
  int inverse;
};

hipError_t launch_rope(int x_dtype, int tab_dtype, const RopeArgs& a, bool vector_ok,
                       hipStream_t st);
// mi_copy_qk: two tensors copied with the RoPE vector path's launch (its
// layout requirements checked by the caller).
hipError_t launch_copy_qk(int x_dtype, const RopeArgs& a, hipStream_t st);

// Softmax cross entropy over the vocabulary (model_ops.hip).  One row per
// token; logits / grad rows are `row_stride` / `grad_row_stride` elements apart.
struct XentArgs {
  const void* logits;
  int64_t rows, vocab, row_stride;
  const int64_t* target;
  void* loss;           // [rows], logits dtype (forward)
  float* lse;           // [rows] fp32, written by forward, read by backward
  const void* grad_loss;  // [rows], logits dtype (backward)
  void* grad;           // backward output
  int64_t grad_row_stride;
};

hipError_t launch_xent_fwd(int dtype, const XentArgs& a, hipStream_t st);
hipError_t launch_xent_bwd(int dtype, const XentArgs& a, hipStream_t st);

// RMSNorm over rows of `hidden` elements (model_ops.hip).
struct RmsArgs {
  int64_t rows, hidden;
  float eps;
  const void* x;
  int64_t x_stride;
  const void* w;  // [hidden], x's dtype or fp32
  void* y;        // forward output, the promoted dtype
  int64_t y_stride;
  float* rstd;    // [rows] fp32, written by forward, read by backward
  const void* dy;
  int64_t dy_stride;
  void* dx;
  int64_t dx_stride;
  void* dw;        // [hidden], w's dtype
  float* partial;  // [parts, hidden] fp32 workspace of the backward
  int parts;
  int dw_acc = 0;  // backward: dw += round_w(reduction) instead of dw = ...
  int vec16 = 0;   // forward: 16-byte accesses (bf16 x, H % 8 == 0, 16-byte aligned rows)
  // Residual add fused in front (all null otherwise).  Forward: x is the
  // residual stream, res the branch output; sum = round_x(x + res) is written
  // and normalised.  Backward: x is that sum and dsum the gradient reaching
  // the sum from its other use; dx = round_x(round_x(norm's dx) + dsum).
  const void* res;
  int64_t res_stride;
  void* sum;
  int64_t sum_stride;
  const void* dsum;
  int64_t dsum_stride;
};

// Number of dw partial rows the backward uses for `rows` rows (<= 256).
int64_t rmsnorm_parts(int64_t rows);
hipError_t launch_rmsnorm_fwd(int x_dtype, int w_dtype, const RmsArgs& a, bool vec,
                              hipStream_t st);
hipError_t launch_rmsnorm_bwd(int x_dtype, int w_dtype, const RmsArgs& a, bool vec,
                              hipStream_t st);

// SwiGLU on the fused [rows, 2 * inter] gate_up projection (model_ops.hip):
// forward writes h [rows, inter]; backward (bwd = true) reads dh and writes the
// [rows, 2 * inter] gradient.
hipError_t launch_swiglu(bool bwd, int dtype, int64_t rows, int64_t inter, const void* gu,
                         int64_t gu_stride, const void* dh, int64_t dh_stride, void* out,
                         int64_t out_stride, bool vec, hipStream_t st);

// The optimizer step (model_ops.hip).  Squared gradient norm into out[0] via
// adam_parts() partial sums; the AdamW step over the flat buffers with
// hp = {1 - lr*wd, 1 - beta1, beta2, 1 - beta2, lr / (1 - beta1^t),
//       sqrt(1 - beta2^t), eps, clip}.
int64_t adam_parts();
hipError_t launch_grad_sumsq(int g_dtype, int64_t n, const void* grad, bool vec, float* out,
                             float* partial, hipStream_t st);
hipError_t launch_adamw_step(int g_dtype, int p_dtype, int64_t n, const void* grad, float* master,
                             float* m, float* v, void* param, const float (&hp)[8],
                             const float* sumsq, bool vec, hipStream_t st);

}  // namespace mi
