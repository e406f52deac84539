// model_ops.hip — the train step's bandwidth-bound operators around the
// attention path, each fused into the fewest passes over HBM.
//
// Softmax cross entropy over the vocabulary (`_VocabParallelCrossEntropy` at one
// tensor-parallel rank, core/tensor_parallel/loss.py:9-72):
//   forward:  loss[r] = log sum_j exp(z_rj - m_r) - (z_r,t - m_r), m_r = max_j z_rj
//             (:14-50; a target outside [0, vocab) is masked: its logit counts as
//             0 after the shift, :33-41); the log-sum-exp lse_r = m_r + log(sum)
//             is kept for the backward instead of the whole softmax (:54-56);
//   backward: dz_rj = (exp(z_rj - lse_r) - [j == t_r]) * dloss_r   (:59-72).
// The forward runs one workgroup per row; the backward too, except for dense
// rows (below), which it streams as one flat run of vectors.  The reference
// computes in the logits' dtype; here the row statistics and the softmax are
// fp32 and only the outputs are rounded.
//
// Logits rows of a vocabulary of odd length are not 16-byte aligned, so each
// row is split into a scalar head up to the first 16-byte boundary, a body of
// 16-byte vectors and a scalar tail.
//
// RMSNorm (core/normalization.py:13-25): further below.
#include "mi_device.h"
#include "mi_kernels.h"

namespace mi {

namespace {

constexpr int XT = 256;  // threads per workgroup (backward)
// Forward: XFT threads per row, XFU 16-byte vectors per thread in flight.  At
// config 5's [8192, 50257] bf16, timed right after a backward pass, 512 x 4 (or
// x 2) took ~124 us, against 131 for 256 x 4 or x 8, 138 for 128 x 8 and 144
// for 1024 x 2.
constexpr int XFT = 512;
constexpr int XFU = 4;

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
    // an all -inf group adds exp(-inf) = 0; skipping it also keeps the first
    // group's x - m away from -inf - (-inf) = NaN
    if (mx == -INFINITY) return;
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
__global__ __launch_bounds__(XFT) void xent_fwd_kernel(const void* logits, int64_t row_stride,
                                                      int64_t vocab, const int64_t* target,
                                                      void* loss, float* lse_out) {
  typedef typename Store<DT>::type T;
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const T* z = (const T*)logits + r * row_stride;
  int64_t head, nvec, tail0;
  row_split<DT>(z, vocab, head, nvec, tail0);
  MaxSum ms;
  for (int64_t i = tid; i < head; i += XFT) {
    const float x = Store<DT>::ld(z, i);
    ms.add_group(&x, 1);
  }
  for (int64_t i = tail0 + tid; i < vocab; i += XFT) {
    const float x = Store<DT>::ld(z, i);
    ms.add_group(&x, 1);
  }
  const u32x4* zv = (const u32x4*)(z + head);
  constexpr int N = Vec16<DT>::N;
  // XFU vectors per thread in flight; the last partial round is guarded
  for (int64_t i0 = tid; i0 < nvec; i0 += XFU * XFT) {
    u32x4 v[XFU];
#pragma unroll
    for (int u = 0; u < XFU; ++u)
      if (i0 + u * XFT < nvec) v[u] = __builtin_nontemporal_load(zv + i0 + u * XFT);
#pragma unroll
    for (int u = 0; u < XFU; ++u) {
      if (i0 + u * XFT < nvec) {
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
  __shared__ float sm[XFT / 64], ss[XFT / 64];
  if ((tid & 63) == 0) {
    sm[tid >> 6] = ms.m;
    ss[tid >> 6] = ms.s;
  }
  __syncthreads();
  if (tid == 0) {
    MaxSum t;
    for (int w = 0; w < XFT / 64; ++w) t.merge(sm[w], ss[w]);
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
  constexpr int U = 8;  // 16-byte vectors in flight per thread (4: 1.5% slower)
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

// Dense rows (both row strides == vocab, both buffers 16-byte aligned, fewer
// than 2^31 elements): the [rows, vocab] matrix as one run of 16-byte vectors,
// consecutive across the grid on every pass -- the access pattern a plain copy
// streams at -- instead of one row per workgroup (thousands of separate
// read and write streams at once).  With vocab >= 64 * 8 + 8 a wave's 64
// consecutive vectors touch at most two rows, A and A + 1; their statistics
// are wave-uniform scalar loads, and a lane picks one set for its vector,
// per element only for the one vector that straddles the row boundary.
// At config 5's [8192, 50257] bf16: 308-324 us (~5.3 TB/s) against 356 us for
// the per-row kernel; 1024 workgroups (one vector per lane) 473 us, 2048 with
// one 330-340, with four 312-328, 8192 with one 318-330.
constexpr int XENT_FLAT_GRID = 2048;
constexpr int XENT_FLAT_U = 2;
constexpr int64_t XENT_FLAT_MIN_VOCAB = 1024;

template <int DT>
__global__ __launch_bounds__(XT) void xent_bwd_flat_kernel(const void* logits, uint32_t n,
                                                           uint32_t rows, FastDiv vocab,
                                                           const int64_t* target,
                                                           const float* lse,
                                                           const void* grad_loss, void* grad) {
  typedef typename Store<DT>::type T;
  constexpr int N = Vec16<DT>::N;
  const uint32_t V = vocab.d;
  // statistics of row r: lse in exp2 units, dloss, flat index of the target
  // (-1 for a masked target, which no element matches)
  auto stats = [&](uint32_t r, float& l2, float& gl, int64_t& tf) __attribute__((always_inline)) {
    l2 = lse[r] * kLog2e;
    gl = Store<DT>::ld((const T*)grad_loss, r);
    const int64_t t = target[r];
    tf = (t >= 0 && t < (int64_t)V) ? (int64_t)r * V + t : -1;
  };
  auto value = [&](float x, int64_t f, float l2, float gl, int64_t tf) __attribute__((always_inline)) {
    const float p = fast_exp2(__builtin_fmaf(x, kLog2e, -l2));
    return (f == tf ? p - 1.f : p) * gl;
  };
  const uint32_t nv = n / N;
  const uint32_t stride = gridDim.x * XT;
  const u32x4* zv = (const u32x4*)logits;
  u32x4* gv = (u32x4*)grad;
  // XENT_FLAT_U vectors per lane in flight, a grid apart
  for (uint32_t q0 = blockIdx.x * XT + threadIdx.x; q0 - threadIdx.x % 64 < nv;
       q0 += XENT_FLAT_U * stride) {
    u32x4 v[XENT_FLAT_U];
#pragma unroll
    for (int u = 0; u < XENT_FLAT_U; ++u)
      if (q0 + u * stride < nv) v[u] = __builtin_nontemporal_load(zv + q0 + u * stride);
#pragma unroll
    for (int u = 0; u < XENT_FLAT_U; ++u) {
      const uint32_t q = q0 + u * stride;
      // rows of this wave's first vector (A) and the next one (B)
      const uint32_t f0 = __builtin_amdgcn_readfirstlane(q * N);
      if (f0 >= n) break;  // wave-uniform
      const uint32_t ra = fdiv(f0, vocab);
      const uint32_t rb = min(ra + 1, rows - 1);
      float l2a, gla, l2b, glb;
      int64_t tfa, tfb;
      stats(ra, l2a, gla, tfa);
      stats(rb, l2b, glb, tfb);
      if (q >= nv) continue;
      const uint32_t f = q * N;
      const uint32_t bnd = (ra + 1) * V;  // first element of row A + 1
      float y[N];
      if (f + N <= bnd || f >= bnd) {
        const bool b = f >= bnd;
        const float l2 = b ? l2b : l2a, gl = b ? glb : gla;
        const int64_t tf = b ? tfb : tfa;
#pragma unroll
        for (int e = 0; e < N; ++e) y[e] = value(elem<DT>(v[u], e), (int64_t)f + e, l2, gl, tf);
      } else {
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const bool b = f + e >= bnd;
          y[e] = value(elem<DT>(v[u], e), (int64_t)f + e, b ? l2b : l2a, b ? glb : gla,
                       b ? tfb : tfa);
        }
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
      __builtin_nontemporal_store(o, gv + q);
    }
  }
  // the last n % N elements, one per lane of the first workgroup
  if (blockIdx.x == 0 && threadIdx.x < n - nv * N) {
    const uint32_t fl = nv * N + threadIdx.x;
    const uint32_t r = fdiv(fl, vocab);
    float l2, gl;
    int64_t tf;
    stats(r, l2, gl, tf);
    Store<DT>::st((T*)grad, fl, value(Store<DT>::ld((const T*)logits, fl), fl, l2, gl, tf));
  }
}

}  // namespace

hipError_t launch_xent_fwd(int dtype, const XentArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)a.rows), block(XFT);
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
  const int64_t n = a.rows * a.vocab;
  if (a.row_stride == a.vocab && a.grad_row_stride == a.vocab && (uintptr_t)a.logits % 16 == 0 &&
      (uintptr_t)a.grad % 16 == 0 && a.vocab >= XENT_FLAT_MIN_VOCAB && n < (int64_t)1 << 31) {
    const FastDiv fv = make_fastdiv((uint32_t)a.vocab);
    const int N = 16 / esz;
    const int64_t want = (n / N + XT - 1) / XT;
    const dim3 fgrid((unsigned)(want < XENT_FLAT_GRID ? (want > 0 ? want : 1) : XENT_FLAT_GRID));
    const uint32_t un = (uint32_t)n, ur = (uint32_t)a.rows;
    if (dtype == 0)
      hipLaunchKernelGGL(xent_bwd_flat_kernel<0>, fgrid, block, 0, st, a.logits, un, ur, fv,
                         a.target, a.lse, a.grad_loss, a.grad);
    else if (dtype == 1)
      hipLaunchKernelGGL(xent_bwd_flat_kernel<1>, fgrid, block, 0, st, a.logits, un, ur, fv,
                         a.target, a.lse, a.grad_loss, a.grad);
    else
      hipLaunchKernelGGL(xent_bwd_flat_kernel<2>, fgrid, block, 0, st, a.logits, un, ur, fv,
                         a.target, a.lse, a.grad_loss, a.grad);
    return hipGetLastError();
  }
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

// ---------------------------------------------------------------------------
// RMSNorm over the last dim (RMSNorm.forward, core/normalization.py:13-25):
//   r_i = rsqrt(mean_j x_ij^2 + eps)              fp32 (:15-21)
//   y_ij = round_x(x_ij * r_i) * w_j              rounded to x's dtype (:23), then
//                                                 multiplied in the promoted dtype (:24)
// The forward saves r (fp32, one per row) for the backward:
//   dn_ij = dy_ij * w_j
//   dx_ij = r_i dn_ij - x_ij r_i^3 (sum_j dn_ij x_ij) / H
//   dw_j  = sum_i dy_ij * round_x(x_ij r_i)
// dw is reduced deterministically: each backward workgroup writes the partial
// sum of its rows to a [parts, H] fp32 workspace, and a second kernel sums the
// parts of each column in a fixed order.  `parts` depends only on the row
// count, so results are bitwise reproducible across devices.
//
// With the residual add fused in front (the two `residual + branch` adds of
// TransformerLayer.forward, core/transformer_layer.py:91-105, each followed by
// the next RMSNorm): the forward also reads the branch output, writes the sum
// round_x(x + res) and normalises it; the backward adds the sum's other
// gradient to dx, each rounded to x's dtype as autograd's two ops round.
//
// Fast path: H % 4 == 0, rows 4-element aligned, H <= 4096 (forward) or 2048
// (backward).  One wave per row,
// 4 consecutive elements per lane and chunk (8-byte loads for 16-bit types),
// the row cached in registers.  Anything else takes the scalar path.
// ---------------------------------------------------------------------------
namespace {

template <int DT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (DT == 0) return v;
  else if constexpr (DT == 2) return __uint_as_float(((uint32_t)f32_to_bf16(v)) << 16);
  else return f16_to_f32(f32_to_f16(v));
}

// 4 consecutive elements as loaded (packed for 16-bit types): 2 registers for
// bf16/fp16, 4 for fp32
template <int DT>
struct Packed4 {
  typedef u32x2 type;
};
template <>
struct Packed4<0> {
  typedef f32x4 type;
};

// NT: non-temporal access (data that this kernel touches once)
template <int DT, bool NT = false>
__device__ __forceinline__ typename Packed4<DT>::type ld4_packed(const void* row, int64_t i) {
  typedef typename Packed4<DT>::type P;
  const P* p = (const P*)((const char*)row + i * (DT == 0 ? 4 : 2));
  return NT ? __builtin_nontemporal_load(p) : *p;
}

template <int DT>
__device__ __forceinline__ void unpack4(const typename Packed4<DT>::type& q, float (&v)[4]) {
  if constexpr (DT == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = q[e];
  } else {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      if constexpr (DT == 2) {
        v[2 * e] = __uint_as_float(q[e] << 16);
        v[2 * e + 1] = __uint_as_float(q[e] & 0xffff0000u);
      } else {
        v[2 * e] = f16_to_f32((uint16_t)(q[e] & 0xffffu));
        v[2 * e + 1] = f16_to_f32((uint16_t)(q[e] >> 16));
      }
    }
  }
}

template <int DT, bool NT = false>
__device__ __forceinline__ void ld4(const void* row, int64_t i, float (&v)[4]) {
  unpack4<DT>(ld4_packed<DT, NT>(row, i), v);
}

template <int DT, bool NT = false>
__device__ __forceinline__ void st4(void* row, int64_t i, const float (&v)[4]) {
  if constexpr (DT == 0) {
    f32x4 q;
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = v[e];
    if constexpr (NT) __builtin_nontemporal_store(q, (f32x4*)((float*)row + i));
    else *(f32x4*)((float*)row + i) = q;
  } else {
    u32x2 q;
    if constexpr (DT == 2) {
      q[0] = BF16::pack2(v[0], v[1]);
      q[1] = BF16::pack2(v[2], v[3]);
    } else {
      q[0] = F16::pack2(v[0], v[1]);
      q[1] = F16::pack2(v[2], v[3]);
    }
    if constexpr (NT) __builtin_nontemporal_store(q, (u32x2*)((uint16_t*)row + i));
    else *(u32x2*)((uint16_t*)row + i) = q;
  }
}

// 8 consecutive elements: one 16-byte access for 16-bit types, two for fp32.
template <int DT, bool NT = false>
__device__ __forceinline__ void ld8(const void* row, int64_t i, float (&v)[8]) {
  if constexpr (DT == 0) {
    float h[2][4];
    ld4<0, NT>(row, i, h[0]);
    ld4<0, NT>(row, i + 4, h[1]);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = h[e >> 2][e & 3];
  } else {
    const u32x4* p = (const u32x4*)((const uint16_t*)row + i);
    const u32x4 q = NT ? __builtin_nontemporal_load(p) : *p;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (DT == 2) {
        v[2 * e] = __uint_as_float(q[e] << 16);
        v[2 * e + 1] = __uint_as_float(q[e] & 0xffff0000u);
      } else {
        v[2 * e] = f16_to_f32((uint16_t)(q[e] & 0xffffu));
        v[2 * e + 1] = f16_to_f32((uint16_t)(q[e] >> 16));
      }
    }
  }
}

template <int DT, bool NT = false>
__device__ __forceinline__ void st8(void* row, int64_t i, const float (&v)[8]) {
  if constexpr (DT == 0) {
    float h[2][4];
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e >> 2][e & 3] = v[e];
    st4<0, NT>(row, i, h[0]);
    st4<0, NT>(row, i + 4, h[1]);
  } else {
    u32x4 q;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      q[e] = DT == 2 ? BF16::pack2(v[2 * e], v[2 * e + 1]) : F16::pack2(v[2 * e], v[2 * e + 1]);
    if constexpr (NT) __builtin_nontemporal_store(q, (u32x4*)((uint16_t*)row + i));
    else *(u32x4*)((uint16_t*)row + i) = q;
  }
}

template <int DT>
__device__ __forceinline__ const void* row_ptr(const void* base, int64_t row, int64_t stride) {
  return (const char*)base + row * stride * (DT == 0 ? 4 : 2);
}
template <int DT>
__device__ __forceinline__ void* row_ptr(void* base, int64_t row, int64_t stride) {
  return (char*)base + row * stride * (DT == 0 ? 4 : 2);
}

// Sum over the 64 lanes, the same bits in every lane: DPP butterflies within
// each row of 16 lanes (xor 1, xor 2, mirror within 8, mirror within 16), then
// the row pairs (lane ^ 16) and the halves (lane ^ 32) by permlane swaps.
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  return sum_halves(v);
}

// The same sum as wave_sum over 64 lanes whose lane l held p0 (l even) or p1
// (l odd) of lane l/2 here, computed by each half-wave (lanes 0-31 and 32-63
// separately): lane i of the 64-lane tree maps to lane i/2 of a half, so each
// step of the tree is the step that pairs the same groups here, and every add
// sees the operands wave_sum's add sees (the same bits in every lane).
__device__ __forceinline__ float half_wave_sum2(float p0, float p1) {
  float v = p0 + p1;        // wave_sum's quad_perm [1,0,3,2]
  v = dpp_add<0xB1>(v);     // its quad_perm [2,3,0,1]
  v = dpp_add<0x4E>(v);     // its row_half_mirror
  v = dpp_add<0x141>(v);    // its row_mirror
  v = dpp_add<0x140>(v);    // its permlane16 swap
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);  // its permlane32 swap
}

// y dtype: the promotion of x's dtype and w's dtype (w is x's dtype or fp32)
template <int DT, int WDT>
struct RmsTypes {
  static constexpr int YDT = WDT == 0 ? 0 : DT;
};

// Waves per backward workgroup: 16 while the row, w and the dw partial fit in
// 128 registers (C <= 4 chunks), else 8 with w re-read from cache per row.
constexpr int RMS_PARTS_ROWS = 16;  // rows per dw partial at most, before the cap
template <int C>
struct RmsBwdCfg {
  static constexpr int W = C <= 4 ? 16 : 8;
  static constexpr bool CACHE_W = C <= 4;
};

// The vector kernels read and write each row once: non-temporal loads and
// stores.  At config 5's [8192, 768] bf16 from HBM: forward 8.2 -> 7.7 us,
// with the residual add 12.6 -> 10.4 us, backward (with the dw reduction)
// 14.5 -> 13.5 us, with the add 16.8 -> 14.8 us; outputs unchanged.  (Stores
// alone give most of it; SwiGLU's kernels, measured the same way, gain nothing.)
constexpr bool kRmsNtLoad = true, kRmsNtStore = true;

template <int DT, int WDT, int C, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_fwd_vec_kernel(RmsArgs a) {
  constexpr int YDT = RmsTypes<DT, WDT>::YDT;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // whole waves only; the kernel has no barrier
  const int nq = (int)(a.hidden / 4);
  const void* xr = row_ptr<DT>(a.x, row, a.x_stride);
  const void* rr = ADD ? row_ptr<DT>(a.res, row, a.res_stride) : nullptr;
  float v[C][4], w[C][4], rv[ADD ? C : 1][4];
  float ss = 0.f;
  // x (and the branch) and w requested together: one memory round trip
  // before the reduction; the whole row is read before any of it is written
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int q = c * 64 + lane;
    if (q < nq) {
      ld4<DT, kRmsNtLoad>(xr, 4 * q, v[c]);
      if constexpr (ADD) ld4<DT, kRmsNtLoad>(rr, 4 * q, rv[c]);
      ld4<WDT>(a.w, 4 * q, w[c]);
    }
  }
  void* sr = ADD ? row_ptr<DT>(a.sum, row, a.sum_stride) : nullptr;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int q = c * 64 + lane;
    if (q < nq) {
      if constexpr (ADD) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[c][e] = round_to<DT>(v[c][e] + rv[c][e]);
        st4<DT, kRmsNtStore>(sr, 4 * q, v[c]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) ss = __builtin_fmaf(v[c][e], v[c][e], ss);
    }
  }
  ss = wave_sum(ss);
  const float r = __builtin_amdgcn_rsqf(ss / (float)a.hidden + a.eps);
  void* yr = row_ptr<YDT>(a.y, row, a.y_stride);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int q = c * 64 + lane;
    if (q < nq) {
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = round_to<DT>(v[c][e] * r) * w[c][e];
      st4<YDT, kRmsNtStore>(yr, 4 * q, y);
    }
  }
  if (lane == 0) a.rstd[row] = r;
}

// Forward with 16-byte accesses (bf16 x, H % 8 == 0, 16-byte aligned rows):
// each half-wave takes RPH rows, C chunks of 8 elements per lane and row, and
// issues every load of its rows before the first reduction.  At config 5's
// [8192, 768] from HBM: 5.8 us against 7.7 for rmsnorm_fwd_vec_kernel (and 6.7
// for torch's copy of the same bytes), with the residual add 9.0 against 10.2;
// two rows per half-wave measured 7.3 and 10.5.  Rows past the end
// are computed on zeros and not stored (the half-wave reduction needs every
// lane of the half).  Lane l's 8 elements of chunk c are the 4 + 4 that lanes
// 2l and 2l + 1 of rmsnorm_fwd_vec_kernel hold in its chunk c; summed as two
// partials in that kernel's order and reduced by half_wave_sum2, the sum of
// squares, and so every output, is bitwise that kernel's.
constexpr int RMS_V16_RPH = 1;
template <int DT, int WDT, int C, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_fwd_v16_kernel(RmsArgs a) {
  constexpr int YDT = RmsTypes<DT, WDT>::YDT;
  constexpr int RPH = RMS_V16_RPH;
  const int lane = threadIdx.x & 63, hl = lane & 31;
  const int64_t row0 = ((int64_t)blockIdx.x * 8 + (threadIdx.x >> 5)) * RPH;
  const int nq = (int)(a.hidden / 8);
  float w[C][8], v[RPH][C][8], rv[ADD ? RPH : 1][ADD ? C : 1][8];
#pragma unroll
  for (int r = 0; r < RPH; ++r) {
    const int64_t row = row0 + r;
    const bool ok = row < a.rows;
    const void* xr = row_ptr<DT>(a.x, ok ? row : 0, a.x_stride);
    const void* rr = ADD ? row_ptr<DT>(a.res, ok ? row : 0, a.res_stride) : nullptr;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int q = c * 32 + hl;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[r][c][e] = 0.f;
      if (ok && q < nq) {
        ld8<DT, kRmsNtLoad>(xr, 8 * q, v[r][c]);
        if constexpr (ADD) ld8<DT, kRmsNtLoad>(rr, 8 * q, rv[r][c]);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int q = c * 32 + hl;
    if (q < nq) ld8<WDT>(a.w, 8 * q, w[c]);
  }
#pragma unroll
  for (int r = 0; r < RPH; ++r) {
    const int64_t row = row0 + r;
    const bool ok = row < a.rows;
    float ss0 = 0.f, ss1 = 0.f;
    void* sr = ADD ? row_ptr<DT>(a.sum, ok ? row : 0, a.sum_stride) : nullptr;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int q = c * 32 + hl;
      if (q < nq) {
        if constexpr (ADD) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[r][c][e] = round_to<DT>(v[r][c][e] + rv[r][c][e]);
          if (ok) st8<DT, kRmsNtStore>(sr, 8 * q, v[r][c]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ss0 = __builtin_fmaf(v[r][c][e], v[r][c][e], ss0);
          ss1 = __builtin_fmaf(v[r][c][4 + e], v[r][c][4 + e], ss1);
        }
      }
    }
    const float ss = half_wave_sum2(ss0, ss1);
    const float rs = __builtin_amdgcn_rsqf(ss / (float)a.hidden + a.eps);
    if (!ok) continue;
    void* yr = row_ptr<YDT>(a.y, row, a.y_stride);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int q = c * 32 + hl;
      if (q < nq) {
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = round_to<DT>(v[r][c][e] * rs) * w[c][e];
        st8<YDT, kRmsNtStore>(yr, 8 * q, y);
      }
    }
    if (hl == 0) a.rstd[row] = rs;
  }
}

template <int DT, int WDT, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_fwd_scalar_kernel(RmsArgs a) {
  constexpr int YDT = RmsTypes<DT, WDT>::YDT;
  typedef typename Store<DT>::type T;
  typedef typename Store<WDT>::type TW;
  typedef typename Store<YDT>::type TY;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  // with ADD, the sum is written in the first pass (each element read, then
  // written, by one lane) and the second pass reads it back
  const T* xr = ADD ? (const T*)a.sum + row * a.sum_stride : (const T*)a.x + row * a.x_stride;
  float ss = 0.f;
  for (int64_t j = lane; j < a.hidden; j += 64) {
    float v;
    if constexpr (ADD) {
      v = round_to<DT>(Store<DT>::ld((const T*)a.x + row * a.x_stride, j) +
                       Store<DT>::ld((const T*)a.res + row * a.res_stride, j));
      Store<DT>::st((T*)a.sum + row * a.sum_stride, j, v);
    } else {
      v = Store<DT>::ld(xr, j);
    }
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  const float r = __builtin_amdgcn_rsqf(ss / (float)a.hidden + a.eps);
  TY* yr = (TY*)a.y + row * a.y_stride;
  for (int64_t j = lane; j < a.hidden; j += 64)
    Store<YDT>::st(yr, j, round_to<DT>(Store<DT>::ld(xr, j) * r) * Store<WDT>::ld((const TW*)a.w, j));
  if (lane == 0) a.rstd[row] = r;
}

// dx for every row, and this workgroup's partial dw into partial[blockIdx.x].
template <int DT, int WDT, int C, bool ADD>
__global__ __launch_bounds__(64 * RmsBwdCfg<C>::W) void rmsnorm_bwd_vec_kernel(RmsArgs a) {
  constexpr int YDT = RmsTypes<DT, WDT>::YDT;
  constexpr int W = RmsBwdCfg<C>::W;
  constexpr bool CACHE_W = RmsBwdCfg<C>::CACHE_W;
  constexpr int CS = C < 8 ? C : 8;  // chunks per LDS reduction slice
  __shared__ float red[W][CS * 256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nq = (int)(a.hidden / 4);
  const float inv_h = 1.f / (float)a.hidden;
  float w[CACHE_W ? C : 1][4], acc[C][4];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int q = c * 64 + lane;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[c][e] = 0.f;
    if constexpr (CACHE_W) {
#pragma unroll
      for (int e = 0; e < 4; ++e) w[c][e] = 0.f;
      if (q < nq) ld4<WDT>(a.w, 4 * q, w[c]);
    }
  }
  typedef typename Packed4<DT>::type PX;
  typedef typename Packed4<YDT>::type PY;
  // a row's x, dy (and dsum) as loaded, packed: elements 4q .. 4q + 3 of
  // chunk c = q / 64 in lane q % 64; zeros past the row's end
  auto load = [&](int64_t row, PX (&xq)[C], PY (&dq)[C], PX (&sq)[ADD ? C : 1]) {
    const void* xr = row_ptr<DT>(a.x, row, a.x_stride);
    const void* dyr = row_ptr<YDT>(a.dy, row, a.dy_stride);
    const void* dsr = ADD ? row_ptr<DT>(a.dsum, row, a.dsum_stride) : nullptr;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int q = c * 64 + lane;
      xq[c] = PX{};
      dq[c] = PY{};
      if constexpr (ADD) sq[c] = PX{};
      if (q < nq) {
        xq[c] = ld4_packed<DT, kRmsNtLoad>(xr, 4 * q);
        dq[c] = ld4_packed<YDT, kRmsNtLoad>(dyr, 4 * q);
        if constexpr (ADD) sq[c] = ld4_packed<DT, kRmsNtLoad>(dsr, 4 * q);
      }
    }
  };
  // dx of one row, and its terms added to this wave's dw columns
  auto finish = [&](int64_t row, float r, const PX (&xq)[C], const PY (&dq)[C],
                    const PX (&sq)[ADD ? C : 1]) {
    float x[C][4], dn[C][4], ds[ADD ? C : 1][4];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      unpack4<DT>(xq[c], x[c]);
      unpack4<YDT>(dq[c], dn[c]);
      if constexpr (ADD) unpack4<DT>(sq[c], ds[c]);
    }
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float dy = dn[c][e];
        acc[c][e] = __builtin_fmaf(dy, round_to<DT>(x[c][e] * r), acc[c][e]);
        float wv;
        if constexpr (CACHE_W) {
          wv = w[c][e];
        } else {
          const int64_t j = 4 * (c * 64 + lane) + e;
          wv = j < a.hidden ? Store<WDT>::ld((const typename Store<WDT>::type*)a.w, j) : 0.f;
        }
        dn[c][e] = dy * wv;
        s = __builtin_fmaf(dn[c][e], x[c][e], s);
      }
    s = wave_sum(s);
    const float k = r * r * r * s * inv_h;
    void* dxr = row_ptr<DT>(a.dx, row, a.dx_stride);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int q = c * 64 + lane;
      if (q < nq) {
        float d[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          d[e] = __builtin_fmaf(r, dn[c][e], -x[c][e] * k);
          if constexpr (ADD) d[e] = round_to<DT>(d[e]) + ds[c][e];
        }
        st4<DT, kRmsNtStore>(dxr, 4 * q, d);
      }
    }
  };
  // Two rows in flight per wave: the loads of rows `row` and `row + stride`
  // are issued before the first one's arithmetic, and the second row stays
  // packed (2 registers per 4 16-bit elements) until its turn.  dw adds the
  // rows in the order one row at a time would (row, row + stride, ...), so
  // every output is bitwise that order's.  Config 5 from HBM, one build per
  // process, interleaved: 12.7-12.8 -> 12.3-12.4 us with the dw reduction.
  // Where the second row would not fit the register budget (fp32 x or dy, or
  // 4 chunks at 16 waves) the rows go one at a time.
  constexpr bool PAIR = DT != 0 && YDT != 0 && (W == 8 || C <= 3);
  const int64_t stride = (int64_t)gridDim.x * W;
  for (int64_t row = (int64_t)blockIdx.x * W + wave; row < a.rows;
       row += (PAIR ? 2 : 1) * stride) {
    const int64_t row2 = row + stride;
    PX xq[C], xq2[C], sq[ADD ? C : 1], sq2[ADD ? C : 1];
    PY dq[C], dq2[C];
    load(row, xq, dq, sq);
    const float r = a.rstd[row];
    if (PAIR && row2 < a.rows) {
      load(row2, xq2, dq2, sq2);
      const float r2 = a.rstd[row2];
      finish(row, r, xq, dq, sq);
      finish(row2, r2, xq2, dq2, sq2);
    } else {
      finish(row, r, xq, dq, sq);
    }
  }
  // partial dw of this workgroup: sum the waves in a fixed order
  float* part = a.partial + (int64_t)blockIdx.x * a.hidden;
#pragma unroll
  for (int s0 = 0; s0 < C; s0 += CS) {
#pragma unroll
    for (int c = s0; c < s0 + CS && c < C; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave][4 * ((c - s0) * 64 + lane) + e] = acc[c][e];
    __syncthreads();
    for (int j = threadIdx.x; j < CS * 256; j += 64 * W) {
      const int64_t col = (int64_t)s0 * 256 + j;
      if (col < a.hidden) {
        float t = 0.f;
#pragma unroll
        for (int v = 0; v < W; ++v) t += red[v][j];
        part[col] = t;
      }
    }
    __syncthreads();
  }
}

template <int DT, int WDT, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_bwd_dx_scalar_kernel(RmsArgs a) {
  constexpr int YDT = RmsTypes<DT, WDT>::YDT;
  typedef typename Store<DT>::type T;
  typedef typename Store<WDT>::type TW;
  typedef typename Store<YDT>::type TY;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const T* xr = (const T*)a.x + row * a.x_stride;
  const TY* dyr = (const TY*)a.dy + row * a.dy_stride;
  const TW* wr = (const TW*)a.w;
  const float r = a.rstd[row];
  float s = 0.f;
  for (int64_t j = lane; j < a.hidden; j += 64)
    s = __builtin_fmaf(Store<YDT>::ld(dyr, j) * Store<WDT>::ld(wr, j), Store<DT>::ld(xr, j), s);
  s = wave_sum(s);
  const float k = r * r * r * s / (float)a.hidden;
  T* dxr = (T*)a.dx + row * a.dx_stride;
  // every element of the row is read above before any is written below, so
  // dx may alias dy (same stride); dsum is read by the lane that then writes
  // the element, so dx may alias it too
  for (int64_t j = lane; j < a.hidden; j += 64) {
    const float dn = Store<YDT>::ld(dyr, j) * Store<WDT>::ld(wr, j);
    float d = __builtin_fmaf(r, dn, -Store<DT>::ld(xr, j) * k);
    if constexpr (ADD) d = round_to<DT>(d) + Store<DT>::ld((const T*)a.dsum + row * a.dsum_stride, j);
    Store<DT>::st(dxr, j, d);
  }
}

// partial[p][col] = sum over rows [p*rpp, (p+1)*rpp) of dy * round_x(x r)
template <int DT, int WDT>
__global__ __launch_bounds__(256) void rmsnorm_dw_partial_scalar_kernel(RmsArgs a, int64_t rpp) {
  constexpr int YDT = RmsTypes<DT, WDT>::YDT;
  typedef typename Store<DT>::type T;
  typedef typename Store<YDT>::type TY;
  const int64_t col = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (col >= a.hidden) return;
  const int64_t r0 = (int64_t)blockIdx.y * rpp;
  const int64_t r1 = min(r0 + rpp, a.rows);
  float t = 0.f;
  for (int64_t row = r0; row < r1; ++row) {
    const float n = round_to<DT>(Store<DT>::ld((const T*)a.x + row * a.x_stride, col) * a.rstd[row]);
    t = __builtin_fmaf(Store<YDT>::ld((const TY*)a.dy + row * a.dy_stride, col), n, t);
  }
  a.partial[(int64_t)blockIdx.y * a.hidden + col] = t;
}

// Columns per workgroup of the dw reduction (16 partial groups each): 16
// puts H / 16 workgroups on the [parts, H] partials (48 at H = 768), ~0.5 us
// faster per backward at config 5 than 64 columns (12 workgroups); 8 and 32
// measured between the two.  The summation order does not depend on it.
constexpr int DW_COLS = 16;

// dw[col] = sum_p partial[p][col], p in increasing order within 16 strided
// groups, then the 16 group sums in order.  With dw_acc the sum, rounded to w's
// dtype, is added to dw[col] (rounded again): autograd's accumulation of a
// weight gradient into an existing .grad, two roundings included.
template <int WDT>
__global__ __launch_bounds__(16 * DW_COLS) void rmsnorm_dw_reduce_kernel(RmsArgs a) {
  typedef typename Store<WDT>::type TW;
  __shared__ float red[16][DW_COLS + 1];
  const int cl = threadIdx.x % DW_COLS, g = threadIdx.x / DW_COLS;
  const int64_t col = (int64_t)blockIdx.x * DW_COLS + cl;
  float t = 0.f;
  if (col < a.hidden) {
#pragma unroll 16
    for (int p = g; p < a.parts; p += 16) t += a.partial[(int64_t)p * a.hidden + col];
  }
  red[g][cl] = t;
  __syncthreads();
  if (g == 0 && col < a.hidden) {
    float u = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) u += red[k][cl];
    if (a.dw_acc) u = Store<WDT>::ld((const TW*)a.dw, col) + round_to<WDT>(u);
    Store<WDT>::st((TW*)a.dw, col, u);
  }
}

// The forward's vector path covers H <= 64 * 4 * 16; the backward's, which also
// holds dy and the dw partial in registers, H <= 64 * 4 * 8 (beyond, it spills).
constexpr int64_t RMS_VEC_FWD_MAX = 4096, RMS_VEC_BWD_MAX = 2048;

template <int DT, int WDT, int C, bool ADD>
void launch_rms_vec(bool fwd, const RmsArgs& a, hipStream_t st) {
  if (fwd)
    hipLaunchKernelGGL((rmsnorm_fwd_vec_kernel<DT, WDT, C, ADD>),
                       dim3((unsigned)((a.rows + 3) / 4)), dim3(256), 0, st, a);
  else if constexpr (C <= 8)
    hipLaunchKernelGGL((rmsnorm_bwd_vec_kernel<DT, WDT, C, ADD>), dim3((unsigned)a.parts),
                       dim3(64 * RmsBwdCfg<C>::W), 0, st, a);
}

template <int DT, int WDT, bool ADD>
hipError_t launch_rms_dt(bool fwd, const RmsArgs& a, bool vec, hipStream_t st) {
  const int64_t nq = a.hidden / 4;
  if (a.hidden > (fwd ? RMS_VEC_FWD_MAX : RMS_VEC_BWD_MAX)) vec = false;
  // bf16 only: for fp16 the backend fuses some of a row's x * r products with
  // their conversion into one v_fma_mixlo_f16 (a single rounding of the exact
  // product), and which ones depends on the kernel's code, so the two kernels
  // could round a rare element differently; bf16 has no such fusion
  if constexpr (DT == 2) {
    if (fwd && vec && a.vec16) {
      const int64_t n8 = a.hidden / 8;
      const dim3 grid((unsigned)((a.rows + 8 * RMS_V16_RPH - 1) / (8 * RMS_V16_RPH)));
      if (n8 <= 32) hipLaunchKernelGGL((rmsnorm_fwd_v16_kernel<DT, WDT, 1, ADD>), grid, dim3(256), 0, st, a);
      else if (n8 <= 64) hipLaunchKernelGGL((rmsnorm_fwd_v16_kernel<DT, WDT, 2, ADD>), grid, dim3(256), 0, st, a);
      else if (n8 <= 96) hipLaunchKernelGGL((rmsnorm_fwd_v16_kernel<DT, WDT, 3, ADD>), grid, dim3(256), 0, st, a);
      else if (n8 <= 128) hipLaunchKernelGGL((rmsnorm_fwd_v16_kernel<DT, WDT, 4, ADD>), grid, dim3(256), 0, st, a);
      else if (n8 <= 192) hipLaunchKernelGGL((rmsnorm_fwd_v16_kernel<DT, WDT, 6, ADD>), grid, dim3(256), 0, st, a);
      else if (n8 <= 256) hipLaunchKernelGGL((rmsnorm_fwd_v16_kernel<DT, WDT, 8, ADD>), grid, dim3(256), 0, st, a);
      else if (n8 <= 384) hipLaunchKernelGGL((rmsnorm_fwd_v16_kernel<DT, WDT, 12, ADD>), grid, dim3(256), 0, st, a);
      else hipLaunchKernelGGL((rmsnorm_fwd_v16_kernel<DT, WDT, 16, ADD>), grid, dim3(256), 0, st, a);
      return hipGetLastError();
    }
  }
  if (vec) {
    // smallest instantiated chunk count covering the row
    if (nq <= 64) launch_rms_vec<DT, WDT, 1, ADD>(fwd, a, st);
    else if (nq <= 128) launch_rms_vec<DT, WDT, 2, ADD>(fwd, a, st);
    else if (nq <= 192) launch_rms_vec<DT, WDT, 3, ADD>(fwd, a, st);
    else if (nq <= 256) launch_rms_vec<DT, WDT, 4, ADD>(fwd, a, st);
    else if (nq <= 384) launch_rms_vec<DT, WDT, 6, ADD>(fwd, a, st);
    else if (nq <= 512) launch_rms_vec<DT, WDT, 8, ADD>(fwd, a, st);
    else if (nq <= 768) launch_rms_vec<DT, WDT, 12, ADD>(fwd, a, st);
    else launch_rms_vec<DT, WDT, 16, ADD>(fwd, a, st);
  } else if (fwd) {
    hipLaunchKernelGGL((rmsnorm_fwd_scalar_kernel<DT, WDT, ADD>),
                       dim3((unsigned)((a.rows + 3) / 4)), dim3(256), 0, st, a);
  } else {
    // dw partials first: dx may overwrite dy
    const int64_t rpp = (a.rows + a.parts - 1) / a.parts;
    hipLaunchKernelGGL((rmsnorm_dw_partial_scalar_kernel<DT, WDT>),
                       dim3((unsigned)((a.hidden + 255) / 256), (unsigned)a.parts), dim3(256), 0,
                       st, a, rpp);
    hipLaunchKernelGGL((rmsnorm_bwd_dx_scalar_kernel<DT, WDT, ADD>),
                       dim3((unsigned)((a.rows + 3) / 4)), dim3(256), 0, st, a);
  }
  if (!fwd)
    hipLaunchKernelGGL((rmsnorm_dw_reduce_kernel<WDT>),
                       dim3((unsigned)((a.hidden + DW_COLS - 1) / DW_COLS)),
                       dim3(16 * DW_COLS), 0, st, a);
  return hipGetLastError();
}

template <bool ADD>
hipError_t launch_rms_add(bool fwd, int x_dtype, int w_dtype, const RmsArgs& a, bool vec,
                          hipStream_t st) {
  if (x_dtype == 2 && w_dtype == 2) return launch_rms_dt<2, 2, ADD>(fwd, a, vec, st);
  if (x_dtype == 2 && w_dtype == 0) return launch_rms_dt<2, 0, ADD>(fwd, a, vec, st);
  if (x_dtype == 1 && w_dtype == 1) return launch_rms_dt<1, 1, ADD>(fwd, a, vec, st);
  if (x_dtype == 1 && w_dtype == 0) return launch_rms_dt<1, 0, ADD>(fwd, a, vec, st);
  return launch_rms_dt<0, 0, ADD>(fwd, a, vec, st);
}

hipError_t launch_rms(bool fwd, int x_dtype, int w_dtype, const RmsArgs& a, bool vec,
                      hipStream_t st) {
  const bool add = fwd ? a.res != nullptr : a.dsum != nullptr;
  return add ? launch_rms_add<true>(fwd, x_dtype, w_dtype, a, vec, st)
             : launch_rms_add<false>(fwd, x_dtype, w_dtype, a, vec, st);
}

}  // namespace

int64_t rmsnorm_parts(int64_t rows) {
  const int64_t p = (rows + RMS_PARTS_ROWS - 1) / RMS_PARTS_ROWS;
  return p < 1 ? 1 : (p > 256 ? 256 : p);
}

hipError_t launch_rmsnorm_fwd(int x_dtype, int w_dtype, const RmsArgs& a, bool vec,
                              hipStream_t st) {
  return launch_rms(true, x_dtype, w_dtype, a, vec, st);
}

hipError_t launch_rmsnorm_bwd(int x_dtype, int w_dtype, const RmsArgs& a, bool vec,
                              hipStream_t st) {
  return launch_rms(false, x_dtype, w_dtype, a, vec, st);
}

// ---------------------------------------------------------------------------
// SwiGLU activation (ParallelMLP.forward, core/mlp.py:24-28) on the fused
// gate_up projection [N, 2I]: gate = columns [0, I), up = columns [I, 2I).
//   s = round(silu(g)),  h = round(s * u)        (F.silu then the product, each
//                                                  rounded to the tensor dtype)
// Backward, as autograd evaluates it (mul, then silu_backward, then the chunk's
// concatenation), written straight into the [N, 2I] gradient:
//   d_up = round(dh * s),  d_s = round(dh * u),
//   d_g  = round(d_s * sig * (1 + g (1 - sig))),  sig = 1 / (1 + exp(-g)).
// 8 elements (16 bytes of 16-bit data) per lane and step when rows are 8-element
// aligned, scalar otherwise.
// ---------------------------------------------------------------------------
namespace {

struct SwigluArgs {
  int64_t rows, inter;
  const void* gu;
  int64_t gu_stride;
  const void* dh;
  int64_t dh_stride;
  void* out;  // h (forward) or dgate_up (backward)
  int64_t out_stride;
};

template <int DT>
__device__ __forceinline__ void swiglu_fwd_elem(float g, float u, float& h) {
  const float s = round_to<DT>(g / (1.f + __expf(-g)));
  h = s * u;
}

template <int DT>
__device__ __forceinline__ void swiglu_bwd_elem(float g, float u, float dh, float& dg, float& du) {
  const float e = __expf(-g);
  const float s = round_to<DT>(g / (1.f + e));
  du = dh * s;
  const float ds = round_to<DT>(dh * u);
  const float sig = 1.f / (1.f + e);
  dg = ds * (sig * (1.f + g * (1.f - sig)));
}


// Grid: x covers the row's chunks (SW_T lanes per workgroup), y the rows with
// a stride loop; no per-element division.
constexpr int SW_T = 128;

template <int DT, bool BWD>
__global__ __launch_bounds__(SW_T) void swiglu_vec_kernel(SwigluArgs a) {
  const int64_t c = (int64_t)blockIdx.x * SW_T + threadIdx.x;
  if (c >= a.inter / 8) return;  // no barrier in this kernel
  const int64_t i = 8 * c;
  for (int64_t row = blockIdx.y; row < a.rows; row += gridDim.y) {
    const void* gr = row_ptr<DT>(a.gu, row, a.gu_stride);
    float g[8], u[8];
    ld8<DT>(gr, i, g);
    ld8<DT>(gr, a.inter + i, u);
    if constexpr (!BWD) {
      float h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) swiglu_fwd_elem<DT>(g[e], u[e], h[e]);
      st8<DT>(row_ptr<DT>(a.out, row, a.out_stride), i, h);
    } else {
      float d[8], dg[8], du[8];
      ld8<DT>(row_ptr<DT>(a.dh, row, a.dh_stride), i, d);
#pragma unroll
      for (int e = 0; e < 8; ++e) swiglu_bwd_elem<DT>(g[e], u[e], d[e], dg[e], du[e]);
      void* orow = row_ptr<DT>(a.out, row, a.out_stride);
      st8<DT>(orow, i, dg);
      st8<DT>(orow, a.inter + i, du);
    }
  }
}

template <int DT, bool BWD>
__global__ __launch_bounds__(SW_T) void swiglu_scalar_kernel(SwigluArgs a) {
  typedef typename Store<DT>::type T;
  const int64_t j = (int64_t)blockIdx.x * SW_T + threadIdx.x;
  if (j >= a.inter) return;
  for (int64_t row = blockIdx.y; row < a.rows; row += gridDim.y) {
    const T* gr = (const T*)a.gu + row * a.gu_stride;
    const float g = Store<DT>::ld(gr, j), u = Store<DT>::ld(gr, a.inter + j);
    T* orow = (T*)a.out + row * a.out_stride;
    if constexpr (!BWD) {
      float h;
      swiglu_fwd_elem<DT>(g, u, h);
      Store<DT>::st(orow, j, h);
    } else {
      float dg, du;
      swiglu_bwd_elem<DT>(g, u, Store<DT>::ld((const T*)a.dh + row * a.dh_stride, j), dg, du);
      Store<DT>::st(orow, j, dg);
      Store<DT>::st(orow, a.inter + j, du);
    }
  }
}

template <int DT>
hipError_t launch_swiglu_dt(bool bwd, const SwigluArgs& a, bool vec, hipStream_t st) {
  const int64_t per_row = vec ? a.inter / 8 : a.inter;
  const dim3 grid((unsigned)((per_row + SW_T - 1) / SW_T),
                  (unsigned)(a.rows < 65535 ? a.rows : 65535));
  if (vec) {
    if (bwd) hipLaunchKernelGGL((swiglu_vec_kernel<DT, true>), grid, dim3(SW_T), 0, st, a);
    else hipLaunchKernelGGL((swiglu_vec_kernel<DT, false>), grid, dim3(SW_T), 0, st, a);
  } else {
    if (bwd) hipLaunchKernelGGL((swiglu_scalar_kernel<DT, true>), grid, dim3(SW_T), 0, st, a);
    else hipLaunchKernelGGL((swiglu_scalar_kernel<DT, false>), grid, dim3(SW_T), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_swiglu(bool bwd, int dtype, int64_t rows, int64_t inter, const void* gu,
                         int64_t gu_stride, const void* dh, int64_t dh_stride, void* out,
                         int64_t out_stride, bool vec, hipStream_t st) {
  SwigluArgs a{rows, inter, gu, gu_stride, dh, dh_stride, out, out_stride};
  if (dtype == 2) return launch_swiglu_dt<2>(bwd, a, vec, st);
  if (dtype == 1) return launch_swiglu_dt<1>(bwd, a, vec, st);
  return launch_swiglu_dt<0>(bwd, a, vec, st);
}

// ---------------------------------------------------------------------------
// The optimizer step of DistributedOptimizer.step at one data-parallel rank
// (core/optimizer.py:79-104) with torch.optim.AdamW (train.py:130-138), over
// the flat gradient / fp32 master / moment buffers:
//   clip (:98-104):   norm = sqrt(sum g^2) (fp32); if norm > clip:
//                     g <- round_g(g * clip / (norm + 1e-6))   (the bf16 buffer is
//                     scaled in place in the reference, so the scaled gradient is
//                     rounded to its dtype)
//   AdamW (torch's multi-tensor form, fp32):
//     p <- p * (1 - lr wd);  m <- m + (1 - b1)(g - m);  v <- v b2 + (1 - b2) g g
//     p <- p - step_size * m / (sqrt(v) / sqrt(1 - b2^t) + eps),
//     step_size = lr / (1 - b1^t)     (bias corrections computed by the host)
//   and the model's copy param <- round_p(p) (the all-gather into the bf16
//   parameter buffer, :95).
// The squared norm is reduced deterministically: ADAM_PARTS workgroups with a
// fixed grid-stride partition write partial sums, then one workgroup sums them
// in order.  The step
// kernel reads the norm from device memory, so nothing waits for the host.
// ---------------------------------------------------------------------------
namespace {

constexpr int ADAM_PARTS = 4096;  // workgroups of the norm pass = partial sums
constexpr int ADAM_T = 256;
// Two workgroups per CU: at config 5's 190 M parameters 978 us, against 1115
// at 1024 workgroups, 1183 at 2048, 1010 at 384 and 1030 at 768 (its eight
// streams of 16-byte vectors keep fewer DRAM pages open with fewer waves).
// One vector per lane and iteration: two consecutive vectors per lane took
// 2190 us (each load instruction spans 2 KB), two grid-strided ones 1040 us.
constexpr int ADAM_STEP_GRID = 512;

// 16 bytes of the gradient as floats (8 16-bit or 4 fp32 elements)
template <int GT>
__device__ __forceinline__ float sumsq16(const u32x4& v) {
  float s = 0.f;
  if constexpr (GT == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float g = __uint_as_float(v[e]);
      s = __builtin_fmaf(g, g, s);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float g = elem<GT>(v, e);
      s = __builtin_fmaf(g, g, s);
    }
  }
  return s;
}

// Grid-stride over 16-byte vectors (one per lane per iteration, consecutive
// across the grid: the streaming pattern that reads fastest), then the
// elements after the last whole vector.  Block b's partial sum goes to
// partial[b]; the grid size is fixed, so the summation order is too.
template <int GT>
__global__ __launch_bounds__(ADAM_T) void grad_sumsq_partial_kernel(const void* grad, int64_t n,
                                                                    bool vec, float* partial) {
  constexpr int EPV = GT == 0 ? 4 : 8;  // elements per 16-byte vector
  const int64_t nv = vec ? n / EPV : 0;
  const int64_t stride = (int64_t)gridDim.x * ADAM_T;
  const int64_t t = (int64_t)blockIdx.x * ADAM_T + threadIdx.x;
  float s = 0.f;
  const u32x4* gv = (const u32x4*)grad;
  for (int64_t q = t; q < nv; q += stride) s += sumsq16<GT>(__builtin_nontemporal_load(gv + q));
  typedef typename Store<GT>::type T;
  for (int64_t k = nv * EPV + t; k < n; k += stride) {
    const float g = Store<GT>::ld((const T*)grad, k);
    s = __builtin_fmaf(g, g, s);
  }
  s = wave_sum(s);
  __shared__ float ws[ADAM_T / 64];
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float u = 0.f;
#pragma unroll
    for (int w = 0; w < ADAM_T / 64; ++w) u += ws[w];
    partial[blockIdx.x] = u;
  }
}

// out[0] = sum of partial[0 .. ADAM_PARTS) in a fixed order (one workgroup)
__global__ __launch_bounds__(1024) void grad_sumsq_final_kernel(const float* partial,
                                                                float* out) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < ADAM_PARTS / 1024; ++k) s += partial[k * 1024 + threadIdx.x];
  s = wave_sum(s);
  __shared__ float ws[16];
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < 16; ++w) t += ws[w];
    out[0] = t;
  }
}

struct AdamArgs {
  int64_t n;
  const void* grad;
  float *master, *m, *v;
  void* param;  // may be null
  float decay, lerp_w, beta2, one_m_beta2, step_size, bc2_sqrt, eps, clip;
  const float* sumsq;  // device scalar; read when clip > 0
};

__device__ __forceinline__ float clip_coef(const AdamArgs& a, bool& clipping) {
  clipping = false;
  if (!(a.clip > 0.f)) return 1.f;
  const float norm = sqrtf(*a.sumsq);
  if (!(norm > a.clip)) return 1.f;
  clipping = true;
  return a.clip / (norm + 1e-6f);
}

__device__ __forceinline__ void adam_elem(const AdamArgs& a, float g, float& p, float& m,
                                          float& v) {
  p = p * a.decay;
  m = m + a.lerp_w * (g - m);
  v = v * a.beta2;
  v = v + a.one_m_beta2 * (g * g);
  const float denom = sqrtf(v) / a.bc2_sqrt + a.eps;
  p = p + (-a.step_size) * (m / denom);
}

template <int GT, int PT>
__global__ __launch_bounds__(ADAM_T) void adamw_step_kernel(AdamArgs a, bool vec) {
  bool clipping;
  const float coef = clip_coef(a, clipping);
  const int64_t nv = vec ? a.n / 4 : 0;
  const int64_t gstride = (int64_t)gridDim.x * ADAM_T;
  for (int64_t q = (int64_t)blockIdx.x * ADAM_T + threadIdx.x; q < nv; q += gstride) {
    const int64_t i = 4 * q;
    float g[4];
    ld4<GT>(a.grad, i, g);
    f32x4 p = __builtin_nontemporal_load((const f32x4*)(a.master + i));
    f32x4 m = __builtin_nontemporal_load((const f32x4*)(a.m + i));
    f32x4 v = __builtin_nontemporal_load((const f32x4*)(a.v + i));
    float po[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float ge = clipping ? round_to<GT>(g[e] * coef) : g[e];
      float pe = p[e], me = m[e], ve = v[e];
      adam_elem(a, ge, pe, me, ve);
      p[e] = pe;
      m[e] = me;
      v[e] = ve;
      po[e] = pe;
    }
    __builtin_nontemporal_store(p, (f32x4*)(a.master + i));
    __builtin_nontemporal_store(m, (f32x4*)(a.m + i));
    __builtin_nontemporal_store(v, (f32x4*)(a.v + i));
    if (a.param) st4<PT>(a.param, i, po);
  }
  // elements after the last full vector (all of them when !vec)
  typedef typename Store<GT>::type TG;
  typedef typename Store<PT>::type TP;
  for (int64_t i = 4 * nv + (int64_t)blockIdx.x * ADAM_T + threadIdx.x; i < a.n; i += gstride) {
    float g = Store<GT>::ld((const TG*)a.grad, i);
    if (clipping) g = round_to<GT>(g * coef);
    float p = a.master[i], m = a.m[i], v = a.v[i];
    adam_elem(a, g, p, m, v);
    a.master[i] = p;
    a.m[i] = m;
    a.v[i] = v;
    if (a.param) Store<PT>::st((TP*)a.param, i, p);
  }
}

template <int GT>
hipError_t launch_adamw_g(int p_dtype, const AdamArgs& a, bool vec, hipStream_t st) {
  const int64_t work = vec ? a.n / 4 : a.n;
  const int64_t want = (work + ADAM_T - 1) / ADAM_T;
  const dim3 grid((unsigned)(want < ADAM_STEP_GRID ? (want > 0 ? want : 1) : ADAM_STEP_GRID));
  if (p_dtype == 2) hipLaunchKernelGGL((adamw_step_kernel<GT, 2>), grid, dim3(ADAM_T), 0, st, a, vec);
  else if (p_dtype == 1) hipLaunchKernelGGL((adamw_step_kernel<GT, 1>), grid, dim3(ADAM_T), 0, st, a, vec);
  else hipLaunchKernelGGL((adamw_step_kernel<GT, 0>), grid, dim3(ADAM_T), 0, st, a, vec);
  return hipGetLastError();
}

}  // namespace

int64_t adam_parts() { return ADAM_PARTS; }

hipError_t launch_grad_sumsq(int g_dtype, int64_t n, const void* grad, bool vec, float* out,
                             float* partial, hipStream_t st) {
  if (g_dtype == 2)
    hipLaunchKernelGGL(grad_sumsq_partial_kernel<2>, dim3(ADAM_PARTS), dim3(ADAM_T), 0, st, grad,
                       n, vec, partial);
  else if (g_dtype == 1)
    hipLaunchKernelGGL(grad_sumsq_partial_kernel<1>, dim3(ADAM_PARTS), dim3(ADAM_T), 0, st, grad,
                       n, vec, partial);
  else
    hipLaunchKernelGGL(grad_sumsq_partial_kernel<0>, dim3(ADAM_PARTS), dim3(ADAM_T), 0, st, grad,
                       n, vec, partial);
  hipLaunchKernelGGL(grad_sumsq_final_kernel, dim3(1), dim3(1024), 0, st, partial, out);
  return hipGetLastError();
}

hipError_t launch_adamw_step(int g_dtype, int p_dtype, int64_t n, const void* grad, float* master,
                             float* m, float* v, void* param, const float (&hp)[8],
                             const float* sumsq, bool vec, hipStream_t st) {
  AdamArgs a;
  a.n = n;
  a.grad = grad;
  a.master = master;
  a.m = m;
  a.v = v;
  a.param = param;
  a.decay = hp[0];
  a.lerp_w = hp[1];
  a.beta2 = hp[2];
  a.one_m_beta2 = hp[3];
  a.step_size = hp[4];
  a.bc2_sqrt = hp[5];
  a.eps = hp[6];
  a.clip = hp[7];
  a.sumsq = sumsq;
  if (g_dtype == 2) return launch_adamw_g<2>(p_dtype, a, vec, st);
  if (g_dtype == 1) return launch_adamw_g<1>(p_dtype, a, vec, st);
  return launch_adamw_g<0>(p_dtype, a, vec, st);
}

}  // namespace mi
