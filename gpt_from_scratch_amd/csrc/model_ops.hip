// model_ops.hip — the train step's bandwidth-bound operators around the
// attention path, fused into single passes over HBM.
//
// Softmax cross entropy over the vocabulary (`_VocabParallelCrossEntropy` at one
// tensor-parallel rank, core/tensor_parallel/loss.py:8-72):
//   forward:  loss[r] = log sum_j exp(z_rj - m_r) - (z_r,t - m_r), m_r = max_j z_rj
//             (:13-43; a target outside [0, vocab) is masked: its logit counts as
//             0 after the shift, :29-35); the log-sum-exp lse_r = m_r + log(sum)
//             is kept for the backward instead of the whole softmax (:47-50);
//   backward: dz_rj = (exp(z_rj - lse_r) - [j == t_r]) * dloss_r   (:58-72).
// One workgroup per row.  The reference computes in the logits' dtype; here the
// row statistics and the softmax are fp32 and only the outputs are rounded.
//
// Logits rows of a vocabulary of odd length are not 16-byte aligned, so each
// row is split into a scalar head up to the first 16-byte boundary, a body of
// 16-byte vectors and a scalar tail.
#include "mi_device.h"
#include "mi_kernels.h"

namespace mi {

namespace {

constexpr int XT = 256;  // threads per workgroup

template <int DT>
struct Vec16 {
  static constexpr int N = DT == 0 ? 4 : 8;  // elements per 16 bytes
};

template <int DT>
__device__ __forceinline__ float elem(const u32x4& v, int e) {
  if constexpr (DT == 0) return __uint_as_float(v[e]);
  else {
    const uint32_t w = v[e >> 1];
    const uint32_t h = (e & 1) ? (w >> 16) : (w & 0xffffu);
    if constexpr (DT == 2) return __uint_as_float(h << 16);
    else return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
}

// Running (max, sum of exp(x - max)) of one thread, fed a group of values.
struct MaxSum {
  float m = -INFINITY, s = 0.f;
  __device__ __forceinline__ void add_group(const float* x, int n) {
    float mx = x[0];
    for (int e = 1; e < n; ++e) mx = fmaxf(mx, x[e]);
    if (mx > m) {
      s *= fast_exp2((m - mx) * kLog2e);  // exp(-inf) = 0 on the first group
      m = mx;
    }
    for (int e = 0; e < n; ++e) s += fast_exp2((x[e] - m) * kLog2e);
  }
  __device__ __forceinline__ void merge(float m2, float s2) {
    if (m2 == -INFINITY) return;
    if (m == -INFINITY) { m = m2; s = s2; return; }
    const float M = fmaxf(m, m2);
    s = s * fast_exp2((m - M) * kLog2e) + s2 * fast_exp2((m2 - M) * kLog2e);
    m = M;
  }
};

// Elements [0, head) and [tail0, vocab) go scalar; [head, tail0) as 16-byte
// vectors.  head = elements to the first 16-byte boundary of `row`.
template <int DT>
__device__ __forceinline__ void row_split(const void* row, int64_t vocab, int64_t& head,
                                          int64_t& nvec, int64_t& tail0) {
  constexpr int esz = DT == 0 ? 4 : 2;
  const uintptr_t a = (uintptr_t)row;
  head = (int64_t)(((16 - (a & 15)) & 15) / esz);
  if (head > vocab) head = vocab;
  nvec = (vocab - head) / Vec16<DT>::N;
  tail0 = head + nvec * Vec16<DT>::N;
}

template <int DT>
__global__ __launch_bounds__(XT) void xent_fwd_kernel(const void* logits, int64_t row_stride,
                                                      int64_t vocab, const int64_t* target,
                                                      void* loss, float* lse_out) {
  typedef typename Store<DT>::type T;
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const T* z = (const T*)logits + r * row_stride;
  int64_t head, nvec, tail0;
  row_split<DT>(z, vocab, head, nvec, tail0);
  MaxSum ms;
  for (int64_t i = tid; i < head; i += XT) {
    const float x = Store<DT>::ld(z, i);
    ms.add_group(&x, 1);
  }
  for (int64_t i = tail0 + tid; i < vocab; i += XT) {
    const float x = Store<DT>::ld(z, i);
    ms.add_group(&x, 1);
  }
  const u32x4* zv = (const u32x4*)(z + head);
  constexpr int N = Vec16<DT>::N;
  // U vectors per thread in flight; the last partial round is guarded
  constexpr int U = 4;
  for (int64_t i0 = tid; i0 < nvec; i0 += U * XT) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u * XT < nvec) v[u] = __builtin_nontemporal_load(zv + i0 + u * XT);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (i0 + u * XT < nvec) {
        float x[N];
#pragma unroll
        for (int e = 0; e < N; ++e) x[e] = elem<DT>(v[u], e);
        ms.add_group(x, N);
      }
    }
  }
  // workgroup reduction of (max, sum)
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
    ms.merge(__shfl_xor(ms.m, off, 64), __shfl_xor(ms.s, off, 64));
  __shared__ float sm[XT / 64], ss[XT / 64];
  if ((tid & 63) == 0) {
    sm[tid >> 6] = ms.m;
    ss[tid >> 6] = ms.s;
  }
  __syncthreads();
  if (tid == 0) {
    MaxSum t;
    for (int w = 0; w < XT / 64; ++w) t.merge(sm[w], ss[w]);
    const int64_t tg = target[r];
    const float zt = (tg >= 0 && tg < vocab) ? Store<DT>::ld(z, tg) - t.m : 0.f;
    const float logs = __logf(t.s);
    Store<DT>::st((T*)loss, r, logs - zt);
    lse_out[r] = t.m + logs;
  }
}

template <int DT>
__global__ __launch_bounds__(XT) void xent_bwd_kernel(const void* logits, int64_t row_stride,
                                                      int64_t vocab, const int64_t* target,
                                                      const float* lse, const void* grad_loss,
                                                      void* grad, int64_t grad_row_stride,
                                                      int vec_ok) {
  typedef typename Store<DT>::type T;
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const T* z = (const T*)logits + r * row_stride;
  T* gz = (T*)grad + r * grad_row_stride;
  const float l2 = lse[r] * kLog2e;
  const float gl = Store<DT>::ld((const T*)grad_loss, r);
  const int64_t tg = target[r];
  auto value = [&](float x, int64_t j) __attribute__((always_inline)) {
    const float p = fast_exp2(__builtin_fmaf(x, kLog2e, -l2));
    return (j == tg ? p - 1.f : p) * gl;
  };
  int64_t head, nvec, tail0;
  if (vec_ok) {
    row_split<DT>(z, vocab, head, nvec, tail0);
  } else {
    head = vocab;
    nvec = 0;
    tail0 = vocab;
  }
  for (int64_t i = tid; i < head; i += XT) Store<DT>::st(gz, i, value(Store<DT>::ld(z, i), i));
  for (int64_t i = tail0 + tid; i < vocab; i += XT)
    Store<DT>::st(gz, i, value(Store<DT>::ld(z, i), i));
  const u32x4* zv = (const u32x4*)(z + head);
  u32x4* gv = (u32x4*)(gz + head);
  constexpr int N = Vec16<DT>::N;
  constexpr int U = 4;
  for (int64_t i0 = tid; i0 < nvec; i0 += U * XT) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u * XT < nvec) v[u] = __builtin_nontemporal_load(zv + i0 + u * XT);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + u * XT;
      if (i < nvec) {
        // position of the target inside this vector, or outside [0, N)
        const int64_t rel = tg - (head + i * N);
        const int te = (rel >= 0 && rel < N) ? (int)rel : -1;
        float y[N];
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const float p = fast_exp2(__builtin_fmaf(elem<DT>(v[u], e), kLog2e, -l2));
          y[e] = (e == te ? p - 1.f : p) * gl;
        }
        u32x4 o;
        if constexpr (DT == 0) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = __float_as_uint(y[e]);
        } else if constexpr (DT == 2) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = BF16::pack2(y[2 * e], y[2 * e + 1]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = F16::pack2(y[2 * e], y[2 * e + 1]);
        }
        __builtin_nontemporal_store(o, gv + i);
      }
    }
  }
}

}  // namespace

hipError_t launch_xent_fwd(int dtype, const XentArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)a.rows), block(XT);
  if (dtype == 0)
    hipLaunchKernelGGL(xent_fwd_kernel<0>, grid, block, 0, st, a.logits, a.row_stride, a.vocab,
                       a.target, a.loss, a.lse);
  else if (dtype == 1)
    hipLaunchKernelGGL(xent_fwd_kernel<1>, grid, block, 0, st, a.logits, a.row_stride, a.vocab,
                       a.target, a.loss, a.lse);
  else
    hipLaunchKernelGGL(xent_fwd_kernel<2>, grid, block, 0, st, a.logits, a.row_stride, a.vocab,
                       a.target, a.loss, a.lse);
  return hipGetLastError();
}

hipError_t launch_xent_bwd(int dtype, const XentArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)a.rows), block(XT);
  // The vector body needs the logits and gradient rows at the same offset from
  // a 16-byte boundary in every row.
  const int esz = dtype == 0 ? 4 : 2;
  const int vec_ok = ((uintptr_t)a.logits % 16 == (uintptr_t)a.grad % 16) &&
                     ((a.row_stride * esz) % 16 == (a.grad_row_stride * esz) % 16);
  if (dtype == 0)
    hipLaunchKernelGGL(xent_bwd_kernel<0>, grid, block, 0, st, a.logits, a.row_stride, a.vocab,
                       a.target, a.lse, a.grad_loss, a.grad, a.grad_row_stride, vec_ok);
  else if (dtype == 1)
    hipLaunchKernelGGL(xent_bwd_kernel<1>, grid, block, 0, st, a.logits, a.row_stride, a.vocab,
                       a.target, a.lse, a.grad_loss, a.grad, a.grad_row_stride, vec_ok);
  else
    hipLaunchKernelGGL(xent_bwd_kernel<2>, grid, block, 0, st, a.logits, a.row_stride, a.vocab,
                       a.target, a.lse, a.grad_loss, a.grad, a.grad_row_stride, vec_ok);
  return hipGetLastError();
}

}  // namespace mi
