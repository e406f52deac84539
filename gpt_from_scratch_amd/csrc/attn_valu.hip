// attn_valu.hip — exact-fp32 flash attention on the vector ALUs.
//
// Same algorithm as the MFMA kernels (online-softmax forward with saved
// log-sum-exp, FlashAttention-2 backward), one lane per query row (forward,
// dQ) or per key row (dK/dV), with 64-row K/V (or Q/dO) tiles staged in LDS as
// fp32.  Used for fp32 tensors (no rounding anywhere: fp32 in, fp32 math,
// fp32 out), for any S (tails are masked) and for head dims / strides the MFMA
// kernels do not cover.  Counterparts: `_attn_fwd` (core/myFlashAttn.py:447-728),
// `_attn_bwd_LoopKV` (:1069-1317) and `_attn_bwd_LoopQ` (:795-1066).
#include "mi_device.h"
#include "mi_kernels.h"

namespace mi {

namespace {

constexpr int VT = 64;  // rows per tile and lanes per workgroup

template <int DT, int D>
__device__ __forceinline__ void stage_rows(float (*dst)[D], const typename Store<DT>::type* base,
                                           int64_t ss, int row0, int S) {
  // 64 lanes copy a 64 x D tile; rows past S are zero-filled.
  for (int e = threadIdx.x; e < VT * D; e += VT) {
    const int r = e / D, d = e % D;
    const int row = row0 + r;
    dst[r][d] = row < S ? Store<DT>::ld(base, (int64_t)row * ss + d) : 0.f;
  }
}

template <int DT, int D, bool CAUSAL>
__global__ __launch_bounds__(64) void attn_fwd_valu_kernel(AttnArgs a) {
  typedef typename Store<DT>::type T;
  __shared__ float Kt[VT][D];
  __shared__ float Vt[VT][D];
  const int bh = blockIdx.y;
  const int b = bh / a.H, h = bh % a.H;
  const int S = a.S;
  const int q0 = blockIdx.x * VT;
  const int qi = q0 + threadIdx.x;
  const bool valid = qi < S;
  const int qc = valid ? qi : S - 1;

  const T* qp = (const T*)a.q.ptr + b * a.q.sb + h * a.q.sh;
  const T* kp = (const T*)a.k.ptr + b * a.k.sb + h * a.k.sh;
  const T* vp = (const T*)a.v.ptr + b * a.v.sb + h * a.v.sh;

  constexpr int SUNROLL = D <= 64 ? VT : 4;
  float q[D], o[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    q[d] = Store<DT>::ld(qp, (int64_t)qc * a.q.ss + d);
    o[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const float c = a.scale_log2;
  const int kv_end = CAUSAL ? min(q0 + VT, S) : S;

  for (int kv0 = 0; kv0 < kv_end; kv0 += VT) {
    __syncthreads();
    stage_rows<DT, D>(Kt, kp, a.k.ss, kv0, S);
    stage_rows<DT, D>(Vt, vp, a.v.ss, kv0, S);
    __syncthreads();
    // Scores of the tile in registers: the j loops unroll fully up to D = 64
    // (a partially unrolled loop indexes s[] at run time and puts it in
    // scratch memory); at D = 128, q and o alone fill the register file.
    float s[VT];
    float mx = -INFINITY;
#pragma unroll SUNROLL
    for (int j = 0; j < VT; ++j) {
      const int kv = kv0 + j;
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) acc = __builtin_fmaf(q[d], Kt[j][d], acc);
      const bool ok = kv < S && (!CAUSAL || kv <= qc);
      s[j] = ok ? acc * c : -INFINITY;
      mx = fmaxf(mx, s[j]);
    }
    const float m_new = fmaxf(m, mx);
    if (m_new == -INFINITY) continue;  // nothing visible yet
    const float alpha = exp2f(m - m_new);
    l *= alpha;
#pragma unroll
    for (int d = 0; d < D; ++d) o[d] *= alpha;
#pragma unroll SUNROLL
    for (int j = 0; j < VT; ++j) {
      const float p = exp2f(s[j] - m_new);
      l += p;
#pragma unroll
      for (int d = 0; d < D; ++d) o[d] = __builtin_fmaf(p, Vt[j][d], o[d]);
    }
    m = m_new;
  }
  if (!valid) return;
  T* op = (T*)a.o.ptr + b * a.o.sb + h * a.o.sh + (int64_t)qi * a.o.ss;
  const float inv = 1.f / l;
#pragma unroll
  for (int d = 0; d < D; ++d) Store<DT>::st(op, d, o[d] * inv);
  a.lse[(int64_t)bh * S + qi] = (m + log2f(l)) * kLn2;
}

template <int DT, int D, bool CAUSAL>
__global__ __launch_bounds__(64) void attn_bwd_dq_valu_kernel(AttnArgs a) {
  typedef typename Store<DT>::type T;
  __shared__ float Kt[VT][D];
  __shared__ float Vt[VT][D];
  const int bh = blockIdx.y;
  const int b = bh / a.H, h = bh % a.H;
  const int S = a.S;
  const int q0 = blockIdx.x * VT;
  const int qi = q0 + threadIdx.x;
  const bool valid = qi < S;
  const int qc = valid ? qi : S - 1;

  const T* qp = (const T*)a.q.ptr + b * a.q.sb + h * a.q.sh;
  const T* kp = (const T*)a.k.ptr + b * a.k.sb + h * a.k.sh;
  const T* vp = (const T*)a.v.ptr + b * a.v.sb + h * a.v.sh;
  const T* dp = (const T*)a.dout.ptr + b * a.dout.sb + h * a.dout.sh;

  float q[D], dov[D], dq[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    q[d] = Store<DT>::ld(qp, (int64_t)qc * a.q.ss + d);
    dov[d] = Store<DT>::ld(dp, (int64_t)qc * a.dout.ss + d);
    dq[d] = 0.f;
  }
  const float lse2 = a.lse[(int64_t)bh * S + qc] * kLog2e;
  const float dl = a.delta[(int64_t)bh * S + qc];
  const float c = a.scale_log2;
  const int kv_end = CAUSAL ? min(q0 + VT, S) : S;

  for (int kv0 = 0; kv0 < kv_end; kv0 += VT) {
    __syncthreads();
    stage_rows<DT, D>(Kt, kp, a.k.ss, kv0, S);
    stage_rows<DT, D>(Vt, vp, a.v.ss, kv0, S);
    __syncthreads();
    for (int j = 0; j < VT; ++j) {
      const int kv = kv0 + j;
      if (kv >= S || (CAUSAL && kv > qc)) continue;
      float sd = 0.f, pd = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        sd = __builtin_fmaf(q[d], Kt[j][d], sd);
        pd = __builtin_fmaf(dov[d], Vt[j][d], pd);
      }
      const float p = exp2f(sd * c - lse2);
      const float ds = p * (pd - dl);
#pragma unroll
      for (int d = 0; d < D; ++d) dq[d] = __builtin_fmaf(ds, Kt[j][d], dq[d]);
    }
  }
  if (!valid) return;
  T* out = (T*)a.dq.ptr + b * a.dq.sb + h * a.dq.sh + (int64_t)qi * a.dq.ss;
#pragma unroll
  for (int d = 0; d < D; ++d) Store<DT>::st(out, d, dq[d] * a.scale);
}

template <int DT, int D, bool CAUSAL>
__global__ __launch_bounds__(64) void attn_bwd_dkdv_valu_kernel(AttnArgs a) {
  typedef typename Store<DT>::type T;
  __shared__ float Qt[VT][D];
  __shared__ float Dt[VT][D];
  __shared__ float Lt[VT], Et[VT];
  const int bh = blockIdx.y;
  const int b = bh / a.H, h = bh % a.H;
  const int S = a.S;
  const int k0 = blockIdx.x * VT;
  const int ki = k0 + threadIdx.x;
  const bool valid = ki < S;
  const int kc = valid ? ki : S - 1;

  const T* qp = (const T*)a.q.ptr + b * a.q.sb + h * a.q.sh;
  const T* kp = (const T*)a.k.ptr + b * a.k.sb + h * a.k.sh;
  const T* vp = (const T*)a.v.ptr + b * a.v.sb + h * a.v.sh;
  const T* dp = (const T*)a.dout.ptr + b * a.dout.sb + h * a.dout.sh;
  const float* lsep = a.lse + (int64_t)bh * S;
  const float* delp = a.delta + (int64_t)bh * S;

  float k[D], v[D], dk[D], dv[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    k[d] = Store<DT>::ld(kp, (int64_t)kc * a.k.ss + d);
    v[d] = Store<DT>::ld(vp, (int64_t)kc * a.v.ss + d);
    dk[d] = 0.f;
    dv[d] = 0.f;
  }
  const float c = a.scale_log2;
  const int q_begin = CAUSAL ? k0 : 0;

  for (int qt0 = q_begin; qt0 < S; qt0 += VT) {
    __syncthreads();
    stage_rows<DT, D>(Qt, qp, a.q.ss, qt0, S);
    stage_rows<DT, D>(Dt, dp, a.dout.ss, qt0, S);
    {
      const int r = qt0 + threadIdx.x;
      Lt[threadIdx.x] = r < S ? lsep[r] * kLog2e : 0.f;
      Et[threadIdx.x] = r < S ? delp[r] : 0.f;
    }
    __syncthreads();
    for (int j = 0; j < VT; ++j) {
      const int qi = qt0 + j;
      if (qi >= S || (CAUSAL && qi < kc)) continue;
      float sd = 0.f, pd = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        sd = __builtin_fmaf(Qt[j][d], k[d], sd);
        pd = __builtin_fmaf(Dt[j][d], v[d], pd);
      }
      const float p = exp2f(sd * c - Lt[j]);
      const float ds = p * (pd - Et[j]);
#pragma unroll
      for (int d = 0; d < D; ++d) {
        dv[d] = __builtin_fmaf(p, Dt[j][d], dv[d]);
        dk[d] = __builtin_fmaf(ds, Qt[j][d], dk[d]);
      }
    }
  }
  if (!valid) return;
  T* dko = (T*)a.dk.ptr + b * a.dk.sb + h * a.dk.sh + (int64_t)ki * a.dk.ss;
  T* dvo = (T*)a.dv.ptr + b * a.dv.sb + h * a.dv.sh + (int64_t)ki * a.dv.ss;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    Store<DT>::st(dko, d, dk[d] * a.scale);
    Store<DT>::st(dvo, d, dv[d]);
  }
}

template <int DT, int D>
hipError_t fwd_d(const AttnArgs& a, hipStream_t st) {
  dim3 grid((a.S + VT - 1) / VT, a.B * a.H), block(VT);
  if (a.causal)
    hipLaunchKernelGGL((attn_fwd_valu_kernel<DT, D, true>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((attn_fwd_valu_kernel<DT, D, false>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <int DT, int D>
hipError_t dkdv_d(const AttnArgs& a, hipStream_t st) {
  dim3 grid((a.S + VT - 1) / VT, a.B * a.H), block(VT);
  if (a.causal)
    hipLaunchKernelGGL((attn_bwd_dkdv_valu_kernel<DT, D, true>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((attn_bwd_dkdv_valu_kernel<DT, D, false>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <int DT, int D>
hipError_t dq_d(const AttnArgs& a, hipStream_t st) {
  dim3 grid((a.S + VT - 1) / VT, a.B * a.H), block(VT);
  if (a.causal)
    hipLaunchKernelGGL((attn_bwd_dq_valu_kernel<DT, D, true>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((attn_bwd_dq_valu_kernel<DT, D, false>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <int DT>
hipError_t fwd_t(const AttnArgs& a, hipStream_t st) {
  switch (a.D) {
    case 16: return fwd_d<DT, 16>(a, st);
    case 32: return fwd_d<DT, 32>(a, st);
    case 64: return fwd_d<DT, 64>(a, st);
    default: return fwd_d<DT, 128>(a, st);
  }
}

template <int DT>
hipError_t dkdv_t(const AttnArgs& a, hipStream_t st) {
  switch (a.D) {
    case 16: return dkdv_d<DT, 16>(a, st);
    case 32: return dkdv_d<DT, 32>(a, st);
    case 64: return dkdv_d<DT, 64>(a, st);
    default: return dkdv_d<DT, 128>(a, st);
  }
}

template <int DT>
hipError_t dq_t(const AttnArgs& a, hipStream_t st) {
  switch (a.D) {
    case 16: return dq_d<DT, 16>(a, st);
    case 32: return dq_d<DT, 32>(a, st);
    case 64: return dq_d<DT, 64>(a, st);
    default: return dq_d<DT, 128>(a, st);
  }
}

}  // namespace

bool valu_supports(int D) { return D == 16 || D == 32 || D == 64 || D == 128; }

hipError_t launch_attn_fwd_valu(int dtype, const AttnArgs& a, hipStream_t st) {
  if (dtype == 0) return fwd_t<0>(a, st);
  if (dtype == 1) return fwd_t<1>(a, st);
  return fwd_t<2>(a, st);
}

hipError_t launch_attn_bwd_dkdv_valu(int dtype, const AttnArgs& a, hipStream_t st) {
  if (dtype == 0) return dkdv_t<0>(a, st);
  if (dtype == 1) return dkdv_t<1>(a, st);
  return dkdv_t<2>(a, st);
}

hipError_t launch_attn_bwd_dq_valu(int dtype, const AttnArgs& a, hipStream_t st) {
  if (dtype == 0) return dq_t<0>(a, st);
  if (dtype == 1) return dq_t<1>(a, st);
  return dq_t<2>(a, st);
}

}  // namespace mi
