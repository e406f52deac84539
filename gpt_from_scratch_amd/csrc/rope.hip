// rope.hip — rotary position embedding, interleaved pairs, bandwidth-bound.
//
// Counterpart of `_rope_kernel` (core/rope_triton.py:74-141): x is [S,B,H,D]
// with arbitrary strides, pairs are adjacent elements (2i, 2i+1) (:112-115),
// angles come from cos/sin tables [S, D/2] (:118-123), and
//   forward: (e, o) -> (e*c - o*s, e*s + o*c)             (:131-133)
//   inverse: (e, o) -> (e*c + o*s, o*c - e*s)             (:128-130)
// computed in fp32 (rope_rotate, explicit fused multiply-adds) and rounded
// once to the output type.
//
// One launch covers q and k (apply_rope_qk, :147-148).  The vector path gives
// each lane the same 16 bytes (8 bf16/f16 or 4 fp32 values = 4 or 2 pairs) of
// q and of k, so a wave reads whole 1 KiB segments of both, the angles of
// those pairs come in with one vector load per table and serve both tensors,
// and the index decomposition (multiply-high division by the run-time
// sizes) is done once.  Every lane takes four items and issues all their
// loads before the first store.  Results are written with non-temporal
// stores (the output is not read again by this kernel; measured ~15% faster
// than plain stores at the model's shapes).  A scalar path (one pair per lane, any
// strides) covers layouts the vector path cannot.
#include "mi_device.h"
#include "mi_kernels.h"

namespace mi {

namespace {

struct RopeDivs {
  FastDiv C, H, B, S;
};

template <int DT>
__device__ __forceinline__ float ldx(const void* p, int64_t i) {
  return Store<DT>::ld((const typename Store<DT>::type*)p, i);
}


// NP consecutive table entries (one vector load: 8 or 16 bytes for 4 pairs,
// 4 or 8 bytes for 2 pairs).
template <int TDT, int NP>
__device__ __forceinline__ void load_angles(const void* tab, int64_t i, float (&v)[NP]) {
  if constexpr (TDT == 0) {
    if constexpr (NP == 4) {
      const f32x4 w = *(const f32x4*)((const float*)tab + i);
#pragma unroll
      for (int p = 0; p < 4; ++p) v[p] = w[p];
    } else {
      const f32x2 w = *(const f32x2*)((const float*)tab + i);
      v[0] = w[0];
      v[1] = w[1];
    }
  } else {
    uint32_t w[NP / 2];
    if constexpr (NP == 4) {
      const u32x2 q = *(const u32x2*)((const uint16_t*)tab + i);
      w[0] = q[0];
      w[1] = q[1];
    } else {
      w[0] = *(const uint32_t*)((const uint16_t*)tab + i);
    }
#pragma unroll
    for (int k = 0; k < NP / 2; ++k) {
      if constexpr (TDT == 2) {
        v[2 * k] = __uint_as_float(w[k] << 16);
        v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
      } else {
        v[2 * k] = F16::to_f32((uint16_t)(w[k] & 0xffffu));
        v[2 * k + 1] = F16::to_f32((uint16_t)(w[k] >> 16));
      }
    }
  }
}

// 16-byte vector path: requires unit dim strides, D % VEC == 0, 16-byte
// aligned rows, unit pair stride in the tables and table rows (and bases)
// aligned to the angle vector.  NTEN tensors (q, or q and k) per lane.  A
// workgroup covers U * ROPE_T consecutive items, lane i items i, i + ROPE_T, ...
// (each pass of its lanes reads whole 1 KiB segments); every lane issues all
// its loads (tables and the U chunks of both tensors) before its first store,
// so U * NTEN 16-byte loads per lane are in flight at once.
// Threads per workgroup of the vector path: at config 2 from HBM 9.2 us,
// against 9.5-9.8 us with 128, 512 or 1024 threads.
constexpr uint32_t ROPE_T = 256;

template <int XDT, int TDT, int NTEN, int U>
__global__ __launch_bounds__(ROPE_T) void rope_vec_kernel(RopeArgs a, RopeDivs dv, uint32_t total) {
  constexpr int VEC = (XDT == 0) ? 4 : 8;  // elements per lane and tensor
  constexpr int NP = VEC / 2;               // pairs per lane
  const uint32_t first = blockIdx.x * (ROPE_T * U) + threadIdx.x;
  u32x4 x[U][NTEN];
  float cs[U][NP], sn[U][NP];
  int64_t out_off[U][NTEN];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t item = first + ROPE_T * u;
    if (item >= total) continue;
    uint32_t r = fdiv(item, dv.C);
    const uint32_t cidx = item - r * dv.C.d;
    const uint32_t r2 = fdiv(r, dv.H);
    const uint32_t h = r - r2 * dv.H.d;
    const uint32_t s = fdiv(r2, dv.B);
    const uint32_t b = r2 - s * dv.B.d;
    const int pair0 = cidx * NP;
    load_angles<TDT, NP>(a.cos_tab, s * a.cs_s + pair0, cs[u]);
    load_angles<TDT, NP>(a.sin_tab, s * a.ss_s + pair0, sn[u]);
#pragma unroll
    for (int t = 0; t < NTEN; ++t) {
      const RopeTensor& T = a.t[t];
      const int64_t in_off = s * T.is_s + b * T.is_b + h * T.is_h + (int64_t)cidx * VEC;
      out_off[u][t] = s * T.os_s + b * T.os_b + h * T.os_h + (int64_t)cidx * VEC;
      // read once: non-temporal (9.3 against 9.45 us for the C2 q/k pair from HBM)
      x[u][t] = (XDT == 0)
                    ? __builtin_nontemporal_load((const u32x4*)((const float*)T.in + in_off))
                    : __builtin_nontemporal_load((const u32x4*)((const uint16_t*)T.in + in_off));
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (first + ROPE_T * u >= total) continue;
#pragma unroll
    for (int t = 0; t < NTEN; ++t) {
      u32x4 y;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        float e, o;
        if constexpr (XDT == 0) {
          e = __uint_as_float(x[u][t][2 * p]);
          o = __uint_as_float(x[u][t][2 * p + 1]);
        } else if constexpr (XDT == 2) {
          e = __uint_as_float(x[u][t][p] << 16);
          o = __uint_as_float(x[u][t][p] & 0xffff0000u);
        } else {
          e = F16::to_f32((uint16_t)(x[u][t][p] & 0xffffu));
          o = F16::to_f32((uint16_t)(x[u][t][p] >> 16));
        }
        float re, ro;
        rope_rotate(e, o, cs[u][p], sn[u][p], a.inverse != 0, re, ro);
        if constexpr (XDT == 0) {
          y[2 * p] = __float_as_uint(re);
          y[2 * p + 1] = __float_as_uint(ro);
        } else {
          y[p] = (XDT == 2) ? BF16::pack2(re, ro) : F16::pack2(re, ro);
        }
      }
      const RopeTensor& T = a.t[t];
      if constexpr (XDT == 0)
        __builtin_nontemporal_store(y, (u32x4*)((float*)T.out + out_off[u][t]));
      else
        __builtin_nontemporal_store(y, (u32x4*)((uint16_t*)T.out + out_off[u][t]));
    }
  }
}

// mi_copy_qk: the vector path's items, grid and accesses without the rotation
// (and without the tables): each lane copies the same 16 bytes of q and of k
// for U items, all loads before the first store.
template <int U>
__global__ __launch_bounds__(ROPE_T) void copy_qk_vec_kernel(RopeArgs a, RopeDivs dv,
                                                             uint32_t total) {
  const uint32_t first = blockIdx.x * (ROPE_T * U) + threadIdx.x;
  const int64_t ebytes = 16 / (a.D / (int)dv.C.d);  // bytes per element (D/C per 16-byte chunk)
  u32x4 x[U][2];
  int64_t out_off[U][2];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t item = first + ROPE_T * u;
    if (item >= total) continue;
    uint32_t r = fdiv(item, dv.C);
    const uint32_t cidx = item - r * dv.C.d;
    const uint32_t r2 = fdiv(r, dv.H);
    const uint32_t h = r - r2 * dv.H.d;
    const uint32_t s = fdiv(r2, dv.B);
    const uint32_t b = r2 - s * dv.B.d;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const RopeTensor& T = a.t[t];
      // byte offsets (the strides count elements)
      const int64_t in_off = (s * T.is_s + b * T.is_b + h * T.is_h) * ebytes + (int64_t)cidx * 16;
      out_off[u][t] = (s * T.os_s + b * T.os_b + h * T.os_h) * ebytes + (int64_t)cidx * 16;
      x[u][t] = __builtin_nontemporal_load((const u32x4*)((const char*)T.in + in_off));
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (first + ROPE_T * u >= total) continue;
#pragma unroll
    for (int t = 0; t < 2; ++t)
      __builtin_nontemporal_store(x[u][t], (u32x4*)((char*)a.t[t].out + out_off[u][t]));
  }
}

// Scalar path: one pair per lane, any strides.
template <int XDT, int TDT>
__global__ __launch_bounds__(256) void rope_pair_kernel(RopeArgs a, RopeDivs dv, uint32_t total) {
  typedef typename Store<XDT>::type T_;
  const uint32_t item = blockIdx.x * 256u + threadIdx.x;
  if (item >= total) return;
  uint32_t r = fdiv(item, dv.C);
  const uint32_t i = item - r * dv.C.d;
  uint32_t r2 = fdiv(r, dv.H);
  const uint32_t h = r - r2 * dv.H.d;
  r = fdiv(r2, dv.B);
  const uint32_t b = r2 - r * dv.B.d;
  r2 = fdiv(r, dv.S);
  const uint32_t s = r - r2 * dv.S.d;
  const uint32_t t = r2;

  const RopeTensor& T = a.t[t];
  const T_* in = (const T_*)T.in + s * T.is_s + b * T.is_b + h * T.is_h;
  T_* out = (T_*)T.out + s * T.os_s + b * T.os_b + h * T.os_h;
  const float e = Store<XDT>::ld(in, (int64_t)(2 * i) * T.is_d);
  const float o = Store<XDT>::ld(in, (int64_t)(2 * i + 1) * T.is_d);
  const float cs = ldx<TDT>(a.cos_tab, s * a.cs_s + (int64_t)i * a.cs_i);
  const float sn = ldx<TDT>(a.sin_tab, s * a.ss_s + (int64_t)i * a.ss_i);
  float re, ro;
  rope_rotate(e, o, cs, sn, a.inverse != 0, re, ro);
  Store<XDT>::st(out, (int64_t)(2 * i) * T.os_d, re);
  Store<XDT>::st(out, (int64_t)(2 * i + 1) * T.os_d, ro);
}

template <int XDT, int TDT>
hipError_t rope_launch(const RopeArgs& a, bool vec, hipStream_t st) {
  const int vecn = (XDT == 0) ? 4 : 8;
  const int C = vec ? a.D / vecn : a.D / 2;
  RopeDivs dv;
  dv.C = make_fastdiv(C);
  dv.H = make_fastdiv(a.H);
  dv.B = make_fastdiv(a.B);
  dv.S = make_fastdiv(a.S);
  if (vec) {
    // one lane per (s, b, h, 16-byte chunk), all tensors
    const uint64_t total = (uint64_t)a.S * a.B * a.H * C;
    // three items per lane (C2: 1024 workgroups, four per CU, every load of
    // the launch in flight at once): 9.04-9.09 us from HBM against 9.17-9.18
    // for four items (768 workgroups) and 9.9-10.1 for five, interleaved on one
    // box; earlier, 10.7 us for a grid-stride loop over 2048 workgroups, two
    // items 10.6, six 10.2, eight 12.2
    constexpr int U = 3;
    const dim3 grid((uint32_t)((total + ROPE_T * U - 1) / (ROPE_T * U))), block(ROPE_T);
    if (a.ntensors == 2)
      hipLaunchKernelGGL((rope_vec_kernel<XDT, TDT, 2, U>), grid, block, 0, st, a, dv, (uint32_t)total);
    else
      hipLaunchKernelGGL((rope_vec_kernel<XDT, TDT, 1, U>), grid, block, 0, st, a, dv, (uint32_t)total);
  } else {
    const uint64_t total = (uint64_t)a.ntensors * a.S * a.B * a.H * C;
    const dim3 grid((uint32_t)((total + 255) / 256)), block(256);
    hipLaunchKernelGGL((rope_pair_kernel<XDT, TDT>), grid, block, 0, st, a, dv, (uint32_t)total);
  }
  return hipGetLastError();
}

template <int XDT>
hipError_t rope_x(int tab_dtype, const RopeArgs& a, bool vec, hipStream_t st) {
  if (tab_dtype == 0) return rope_launch<XDT, 0>(a, vec, st);
  if (tab_dtype == 1) return rope_launch<XDT, 1>(a, vec, st);
  return rope_launch<XDT, 2>(a, vec, st);
}

}  // namespace

hipError_t launch_copy_qk(int x_dtype, const RopeArgs& a, hipStream_t st) {
  const int vecn = (x_dtype == 0) ? 4 : 8;
  const int C = a.D / vecn;
  RopeDivs dv;
  dv.C = make_fastdiv(C);
  dv.H = make_fastdiv(a.H);
  dv.B = make_fastdiv(a.B);
  dv.S = make_fastdiv(a.S);
  const uint64_t total = (uint64_t)a.S * a.B * a.H * C;
  constexpr int U = 3;  // as the RoPE vector path
  const dim3 grid((uint32_t)((total + ROPE_T * U - 1) / (ROPE_T * U))), block(ROPE_T);
  hipLaunchKernelGGL((copy_qk_vec_kernel<U>), grid, block, 0, st, a, dv, (uint32_t)total);
  return hipGetLastError();
}

hipError_t launch_rope(int x_dtype, int tab_dtype, const RopeArgs& a, bool vector_ok,
                       hipStream_t st) {
  if (x_dtype == 0) return rope_x<0>(tab_dtype, a, vector_ok, st);
  if (x_dtype == 1) return rope_x<1>(tab_dtype, a, vector_ok, st);
  return rope_x<2>(tab_dtype, a, vector_ok, st);
}

}  // namespace mi
