// attn_valu.hip — exact-fp32 flash attention on the vector ALUs.
//
// Same algorithm as the MFMA kernels (online-softmax forward with saved
// log-sum-exp, FlashAttention-2 backward), 8 lanes (4 at D = 16) per query row
// (forward, dQ) or per key row (dK/dV), with 64-row K/V (or Q/dO) tiles staged
// in LDS as fp32.  Used for fp32 tensors (no rounding anywhere: fp32 in, fp32
// math, fp32 out), for any S (tails are masked) and for head dims / strides the
// MFMA kernels do not cover.  Counterparts: `_attn_fwd` (core/myFlashAttn.py:447-728),
// `_attn_bwd_LoopKV` (:1069-1317) and `_attn_bwd_LoopQ` (:795-1066).
#include "mi_device.h"
#include "mi_kernels.h"

namespace mi {

namespace {

constexpr int VT = 64;  // rows per staged tile

// Forward: LPQ lanes per query row (8; 4 at D = 16), each holding D / LPQ of
// the row's dimensions as 4-float chunks part, part + LPQ, ... (part = lane %
// LPQ), so a key row's chunks are read from LDS by LPQ adjacent lanes at once
// and every query row of the wave reads the same key row (broadcast).  A
// score is the lanes' partial dot products summed by an xor butterfly, which
// gives every lane of the row the same bits, so the row's running max and sum
// stay identical across its lanes.  A workgroup of 4 waves owns 4 * 64 / LPQ
// query rows and stages each 64-key tile once for all of them.
template <int D>
struct FvCfg {
  static constexpr int LPQ = D >= 32 ? 8 : 4;
  static constexpr int CH = D / 4 / LPQ;  // 4-float chunks per lane
  static constexpr int QPW = 64 / LPQ;    // query rows per wave
  static constexpr int QWG = 4 * QPW;     // query rows per workgroup
  static constexpr int NT = 256;
};

template <int DT, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_fwd_valu_kernel(AttnArgs a) {
  typedef typename Store<DT>::type T;
  using C = FvCfg<D>;
  __shared__ __attribute__((aligned(16))) float Kt[VT][D];
  __shared__ __attribute__((aligned(16))) float Vt[VT][D];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int part = lane % C::LPQ;
  const int bh = blockIdx.y;
  const int b = bh / a.H, h = bh % a.H;
  const int S = a.S;
  const int q0 = blockIdx.x * C::QWG;
  const int qi = q0 + wave * C::QPW + lane / C::LPQ;
  const bool valid = qi < S;
  const int qc = valid ? qi : S - 1;

  const T* qp = (const T*)a.q.ptr + b * a.q.sb + h * a.q.sh;
  const T* kp = (const T*)a.k.ptr + b * a.k.sb + h * a.k.sh;
  const T* vp = (const T*)a.v.ptr + b * a.v.sb + h * a.v.sh;

  float q[C::CH][4], o[C::CH][4];
#pragma unroll
  for (int ch = 0; ch < C::CH; ++ch)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      q[ch][e] = Store<DT>::ld(qp, (int64_t)qc * a.q.ss + 4 * (part + ch * C::LPQ) + e);
      o[ch][e] = 0.f;
    }
  float m = -INFINITY, l = 0.f;
  const float c = a.scale_log2;
  const int kv_end = CAUSAL ? min(q0 + C::QWG, S) : S;

  for (int kv0 = 0; kv0 < kv_end; kv0 += VT) {
    __syncthreads();
    // 256 threads copy the 64 x D tiles (rows past S as zeros)
    for (int e = threadIdx.x; e < VT * D; e += C::NT) {
      const int r = e / D, d = e % D;
      const int row = kv0 + r;
      Kt[r][d] = row < S ? Store<DT>::ld(kp, (int64_t)row * a.k.ss + d) : 0.f;
      Vt[r][d] = row < S ? Store<DT>::ld(vp, (int64_t)row * a.v.ss + d) : 0.f;
    }
    __syncthreads();
    float s[VT];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < VT; ++j) {
      const int kv = kv0 + j;
      float acc = 0.f;
#pragma unroll
      for (int ch = 0; ch < C::CH; ++ch) {
        const f32x4 k4 = *(const f32x4*)&Kt[j][4 * (part + ch * C::LPQ)];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_fmaf(q[ch][e], k4[e], acc);
      }
      acc = group_sum<C::LPQ>(acc);
      const bool ok = kv < S && (!CAUSAL || kv <= qc);
      s[j] = ok ? acc * c : -INFINITY;
      mx = fmaxf(mx, s[j]);
    }
    const float m_new = fmaxf(m, mx);
    if (m_new == -INFINITY) continue;  // nothing visible yet (uniform per row)
    const float alpha = exp2f(m - m_new);
    l *= alpha;
#pragma unroll
    for (int ch = 0; ch < C::CH; ++ch)
#pragma unroll
      for (int e = 0; e < 4; ++e) o[ch][e] *= alpha;
#pragma unroll
    for (int j = 0; j < VT; ++j) {
      const float p = exp2f(s[j] - m_new);
      l += p;
#pragma unroll
      for (int ch = 0; ch < C::CH; ++ch) {
        const f32x4 v4 = *(const f32x4*)&Vt[j][4 * (part + ch * C::LPQ)];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[ch][e] = __builtin_fmaf(p, v4[e], o[ch][e]);
      }
    }
    m = m_new;
  }
  if (!valid) return;
  T* op = (T*)a.o.ptr + b * a.o.sb + h * a.o.sh + (int64_t)qi * a.o.ss;
  const float inv = 1.f / l;
#pragma unroll
  for (int ch = 0; ch < C::CH; ++ch)
#pragma unroll
    for (int e = 0; e < 4; ++e) Store<DT>::st(op, 4 * (part + ch * C::LPQ) + e, o[ch][e] * inv);
  if (part == 0) a.lse[(int64_t)bh * S + qi] = (m + log2f(l)) * kLn2;
}

// Backward: the forward's layout, LPQ lanes per query row (dQ) or key row
// (dK/dV), 4 * 64 / LPQ rows per workgroup, 64-row tiles of the other side
// staged in LDS.  Both dot products of a (query, key) pair are the lanes'
// partial sums added by the same butterfly, so every lane of a row holds the
// same P and dS; masked pairs take P = 0, which adds exact zeros.
template <int DT, int D>
__device__ __forceinline__ void stage_tile_pair(float (*t0)[D], float (*t1)[D],
                                                const typename Store<DT>::type* p0, int64_t ss0,
                                                const typename Store<DT>::type* p1, int64_t ss1,
                                                int row0, int S) {
  for (int e = threadIdx.x; e < VT * D; e += FvCfg<D>::NT) {
    const int r = e / D, d = e % D;
    const int row = row0 + r;
    t0[r][d] = row < S ? Store<DT>::ld(p0, (int64_t)row * ss0 + d) : 0.f;
    t1[r][d] = row < S ? Store<DT>::ld(p1, (int64_t)row * ss1 + d) : 0.f;
  }
}

template <int DT, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dq_valu_kernel(AttnArgs a) {
  typedef typename Store<DT>::type T;
  using C = FvCfg<D>;
  __shared__ __attribute__((aligned(16))) float Kt[VT][D];
  __shared__ __attribute__((aligned(16))) float Vt[VT][D];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int part = lane % C::LPQ;
  const int bh = blockIdx.y;
  const int b = bh / a.H, h = bh % a.H;
  const int S = a.S;
  const int q0 = blockIdx.x * C::QWG;
  const int qi = q0 + wave * C::QPW + lane / C::LPQ;
  const bool valid = qi < S;
  const int qc = valid ? qi : S - 1;

  const T* qp = (const T*)a.q.ptr + b * a.q.sb + h * a.q.sh;
  const T* kp = (const T*)a.k.ptr + b * a.k.sb + h * a.k.sh;
  const T* vp = (const T*)a.v.ptr + b * a.v.sb + h * a.v.sh;
  const T* dp = (const T*)a.dout.ptr + b * a.dout.sb + h * a.dout.sh;

  float q[C::CH][4], dov[C::CH][4], dq[C::CH][4];
#pragma unroll
  for (int ch = 0; ch < C::CH; ++ch)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = 4 * (part + ch * C::LPQ) + e;
      q[ch][e] = Store<DT>::ld(qp, (int64_t)qc * a.q.ss + d);
      dov[ch][e] = Store<DT>::ld(dp, (int64_t)qc * a.dout.ss + d);
      dq[ch][e] = 0.f;
    }
  const float lse2 = a.lse[(int64_t)bh * S + qc] * kLog2e;
  const float dl = a.delta[(int64_t)bh * S + qc];
  const float c = a.scale_log2;
  const int kv_end = CAUSAL ? min(q0 + C::QWG, S) : S;

  for (int kv0 = 0; kv0 < kv_end; kv0 += VT) {
    __syncthreads();
    stage_tile_pair<DT, D>(Kt, Vt, kp, a.k.ss, vp, a.v.ss, kv0, S);
    __syncthreads();
#pragma unroll 8
    for (int j = 0; j < VT; ++j) {
      const int kv = kv0 + j;
      float sd = 0.f, pd = 0.f;
#pragma unroll
      for (int ch = 0; ch < C::CH; ++ch) {
        const f32x4 k4 = *(const f32x4*)&Kt[j][4 * (part + ch * C::LPQ)];
        const f32x4 v4 = *(const f32x4*)&Vt[j][4 * (part + ch * C::LPQ)];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sd = __builtin_fmaf(q[ch][e], k4[e], sd);
          pd = __builtin_fmaf(dov[ch][e], v4[e], pd);
        }
      }
      sd = group_sum<C::LPQ>(sd);
      pd = group_sum<C::LPQ>(pd);
      const bool ok = kv < S && (!CAUSAL || kv <= qc);
      const float p = ok ? exp2f(sd * c - lse2) : 0.f;
      const float ds = p * (pd - dl);
#pragma unroll
      for (int ch = 0; ch < C::CH; ++ch) {
        const f32x4 k4 = *(const f32x4*)&Kt[j][4 * (part + ch * C::LPQ)];
#pragma unroll
        for (int e = 0; e < 4; ++e) dq[ch][e] = __builtin_fmaf(ds, k4[e], dq[ch][e]);
      }
    }
  }
  if (!valid) return;
  T* out = (T*)a.dq.ptr + b * a.dq.sb + h * a.dq.sh + (int64_t)qi * a.dq.ss;
#pragma unroll
  for (int ch = 0; ch < C::CH; ++ch)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      Store<DT>::st(out, 4 * (part + ch * C::LPQ) + e, dq[ch][e] * a.scale);
}

template <int DT, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_valu_kernel(AttnArgs a) {
  typedef typename Store<DT>::type T;
  using C = FvCfg<D>;
  __shared__ __attribute__((aligned(16))) float Qt[VT][D];
  __shared__ __attribute__((aligned(16))) float Dt[VT][D];
  __shared__ float Lt[VT], Et[VT];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int part = lane % C::LPQ;
  const int bh = blockIdx.y;
  const int b = bh / a.H, h = bh % a.H;
  const int S = a.S;
  const int k0 = blockIdx.x * C::QWG;
  const int ki = k0 + wave * C::QPW + lane / C::LPQ;
  const bool valid = ki < S;
  const int kc = valid ? ki : S - 1;

  const T* qp = (const T*)a.q.ptr + b * a.q.sb + h * a.q.sh;
  const T* kp = (const T*)a.k.ptr + b * a.k.sb + h * a.k.sh;
  const T* vp = (const T*)a.v.ptr + b * a.v.sb + h * a.v.sh;
  const T* dp = (const T*)a.dout.ptr + b * a.dout.sb + h * a.dout.sh;
  const float* lsep = a.lse + (int64_t)bh * S;
  const float* delp = a.delta + (int64_t)bh * S;

  float k[C::CH][4], v[C::CH][4], dk[C::CH][4], dv[C::CH][4];
#pragma unroll
  for (int ch = 0; ch < C::CH; ++ch)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = 4 * (part + ch * C::LPQ) + e;
      k[ch][e] = Store<DT>::ld(kp, (int64_t)kc * a.k.ss + d);
      v[ch][e] = Store<DT>::ld(vp, (int64_t)kc * a.v.ss + d);
      dk[ch][e] = 0.f;
      dv[ch][e] = 0.f;
    }
  const float c = a.scale_log2;
  const int q_begin = CAUSAL ? k0 : 0;

  for (int qt0 = q_begin; qt0 < S; qt0 += VT) {
    __syncthreads();
    stage_tile_pair<DT, D>(Qt, Dt, qp, a.q.ss, dp, a.dout.ss, qt0, S);
    if (threadIdx.x < VT) {
      const int r = qt0 + threadIdx.x;
      Lt[threadIdx.x] = r < S ? lsep[r] * kLog2e : 0.f;
      Et[threadIdx.x] = r < S ? delp[r] : 0.f;
    }
    __syncthreads();
#pragma unroll 8
    for (int j = 0; j < VT; ++j) {
      const int qi = qt0 + j;
      float sd = 0.f, pd = 0.f;
#pragma unroll
      for (int ch = 0; ch < C::CH; ++ch) {
        const f32x4 q4 = *(const f32x4*)&Qt[j][4 * (part + ch * C::LPQ)];
        const f32x4 d4 = *(const f32x4*)&Dt[j][4 * (part + ch * C::LPQ)];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sd = __builtin_fmaf(q4[e], k[ch][e], sd);
          pd = __builtin_fmaf(d4[e], v[ch][e], pd);
        }
      }
      sd = group_sum<C::LPQ>(sd);
      pd = group_sum<C::LPQ>(pd);
      const bool ok = qi < S && (!CAUSAL || qi >= kc);
      const float p = ok ? exp2f(sd * c - Lt[j]) : 0.f;
      const float ds = p * (pd - Et[j]);
#pragma unroll
      for (int ch = 0; ch < C::CH; ++ch) {
        const f32x4 q4 = *(const f32x4*)&Qt[j][4 * (part + ch * C::LPQ)];
        const f32x4 d4 = *(const f32x4*)&Dt[j][4 * (part + ch * C::LPQ)];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dv[ch][e] = __builtin_fmaf(p, d4[e], dv[ch][e]);
          dk[ch][e] = __builtin_fmaf(ds, q4[e], dk[ch][e]);
        }
      }
    }
  }
  if (!valid) return;
  T* dko = (T*)a.dk.ptr + b * a.dk.sb + h * a.dk.sh + (int64_t)ki * a.dk.ss;
  T* dvo = (T*)a.dv.ptr + b * a.dv.sb + h * a.dv.sh + (int64_t)ki * a.dv.ss;
#pragma unroll
  for (int ch = 0; ch < C::CH; ++ch)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = 4 * (part + ch * C::LPQ) + e;
      Store<DT>::st(dko, d, dk[ch][e] * a.scale);
      Store<DT>::st(dvo, d, dv[ch][e]);
    }
}

template <int DT, int D>
hipError_t fwd_d(const AttnArgs& a, hipStream_t st) {
  dim3 grid((a.S + FvCfg<D>::QWG - 1) / FvCfg<D>::QWG, a.B * a.H), block(FvCfg<D>::NT);
  if (a.causal)
    hipLaunchKernelGGL((attn_fwd_valu_kernel<DT, D, true>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((attn_fwd_valu_kernel<DT, D, false>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <int DT, int D>
hipError_t dkdv_d(const AttnArgs& a, hipStream_t st) {
  dim3 grid((a.S + FvCfg<D>::QWG - 1) / FvCfg<D>::QWG, a.B * a.H), block(FvCfg<D>::NT);
  if (a.causal)
    hipLaunchKernelGGL((attn_bwd_dkdv_valu_kernel<DT, D, true>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((attn_bwd_dkdv_valu_kernel<DT, D, false>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <int DT, int D>
hipError_t dq_d(const AttnArgs& a, hipStream_t st) {
  dim3 grid((a.S + FvCfg<D>::QWG - 1) / FvCfg<D>::QWG, a.B * a.H), block(FvCfg<D>::NT);
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
