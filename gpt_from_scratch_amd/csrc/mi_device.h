// mi_device.h — device-side building blocks shared by the gfx950 kernels.
//
// Everything here is written for CDNA4 (gfx950, wave64).  The MFMA helpers wrap
// the 32x32x16 bf16 / f16 matrix-core instructions; the operand layout they
// assume is the hardware's:
//   A (32 x 16): lane l holds A[l % 32][k-slot 0..7 of half l / 32]
//   B (16 x 32): lane l holds B[k-slot 0..7 of half l / 32][l % 32]
//   C (32 x 32): lane l, register r holds C[8*(r/4) + 4*(l/32) + r%4][l % 32]
// The k-slot -> k mapping is the same for A and B, so any assignment of the 16
// k indices to (half, slot) pairs gives the same product as long as A and B use
// the same one.  The kernels rely on that to feed a C-layout accumulator
// (softmax probabilities) straight back in as a B operand.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// 16-bit element types: storage is raw uint16_t, arithmetic is fp32.
// ---------------------------------------------------------------------------
struct BF16 {
  typedef bf16x8 vec8;
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return __uint_as_float(((uint32_t)x) << 16);
  }
  // Two floats -> packed pair (round to nearest even, v_cvt_pk_bf16_f32).
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
    bf16x2 v;
    v[0] = (__bf16)a;
    v[1] = (__bf16)b;
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // acc + lo + hi of a packed pair (v_dot2c_f32_bf16 against (1, 1)).
  static __device__ __forceinline__ float sum2(uint32_t pair, float acc) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), one, acc, false);
  }
};

struct F16 {
  typedef f16x8 vec8;
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return (float)__builtin_bit_cast(_Float16, x);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
    f16x2 v;
    v[0] = (_Float16)a;
    v[1] = (_Float16)b;
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float sum2(uint32_t pair, float acc) {
    typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pair), one, acc, false);
  }
};

__device__ __forceinline__ float bf16_to_f32(uint16_t x) { return BF16::to_f32(x); }
__device__ __forceinline__ float f16_to_f32(uint16_t x) { return F16::to_f32(x); }
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  return (uint16_t)(BF16::pack2(x, 0.f) & 0xffffu);
}
__device__ __forceinline__ uint16_t f32_to_f16(float x) {
  return (uint16_t)(F16::pack2(x, 0.f) & 0xffffu);
}

// Rotary rotation of one interleaved pair (core/rope_triton.py:128-133) in
// fp32 with explicit fused multiply-adds, so that every kernel applying it
// (RoPE itself, and the attention backward's dQ/dK stores) rounds the same:
//   forward: (e, o) -> (e c - o s, e s + o c)
//   inverse: (e, o) -> (e c + o s, o c - e s)
__device__ __forceinline__ void rope_rotate(float e, float o, float c, float s, bool inverse,
                                            float& re, float& ro) {
  if (inverse) {
    re = __builtin_fmaf(e, c, o * s);
    ro = __builtin_fmaf(o, c, -(e * s));
  } else {
    re = __builtin_fmaf(e, c, -(o * s));
    ro = __builtin_fmaf(e, s, o * c);
  }
}

// Storage-type traits for kernels that are generic over fp32 / f16 / bf16.
template <int DT> struct Store;  // DT: 0 = f32, 1 = f16, 2 = bf16 (mi_dtype values)
template <> struct Store<0> {
  typedef float type;
  static __device__ __forceinline__ float ld(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void st(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Store<1> {
  typedef uint16_t type;
  static __device__ __forceinline__ float ld(const uint16_t* p, int64_t i) { return f16_to_f32(p[i]); }
  static __device__ __forceinline__ void st(uint16_t* p, int64_t i, float v) { p[i] = f32_to_f16(v); }
};
template <> struct Store<2> {
  typedef uint16_t type;
  static __device__ __forceinline__ float ld(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
  static __device__ __forceinline__ void st(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
};

// ---------------------------------------------------------------------------
// Wave-level helpers.
// ---------------------------------------------------------------------------
// IEEE 754-2019 maximum (NaN-propagating); lowers to v_maximum3_f32 chains.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Reductions over lanes l and l ^ 32 (the two halves of a wave), one
// v_permlane32_swap each: the swap exchanges the upper half of its first
// operand with the lower half of its second, so swapping x with itself puts
// x[l ^ 32] into one of the two results for every lane.
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// v plus the value of the lane that DPP control CTRL selects (quad_perm,
// row_half_mirror, row_mirror, ...), in every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF,
                                                        false));
}

// Sum over each aligned group of N (2, 4 or 8) lanes by xor butterflies
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror): IEEE addition
// commutes, so every lane of a group gets the same bits.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(N == 2 || N == 4 || N == 8, "group size");
  v = dpp_add<0xB1>(v);
  if constexpr (N >= 4) v = dpp_add<0x4E>(v);
  if constexpr (N >= 8) v = dpp_add<0x141>(v);
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// ---------------------------------------------------------------------------
// Buffer resource for raw buffer loads based at `p` (wave-uniform pointer, so
// the descriptor lives in SGPRs and per-tile rebasing is scalar arithmetic),
// covering `bytes` bytes from p: a load at or past that extent returns zeros
// (and a direct-to-LDS load writes zeros) instead of reading whatever memory
// follows.  Word 3 = 0x00020000: 32-bit data format, no swizzle, no stride
// (gfx9 family).
// ---------------------------------------------------------------------------
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           0x00020000);
}

// Bytes spanned by `rows` rows of `cols` 16-bit elements, `ss` elements apart
// (0 for no rows).
__device__ __forceinline__ uint32_t rows_extent(int rows, int64_t ss, int cols) {
  return rows <= 0 ? 0u : (uint32_t)(((int64_t)(rows - 1) * ss + cols) * 2);
}

// A byte offset past every extent above: the host admits a tensor to the
// matrix-core kernels only when 256 of its rows span less than 2^31 bytes,
// so a load at this offset returns zeros (writes zeros to LDS) and touches
// no memory.  Head dims below 64 staged in the D = 64 layout fetch their
// padding chunks with it.
constexpr uint32_t kOobOffset = 0x80000000u;

// ---------------------------------------------------------------------------
// Division by a run-time invariant (Granlund-Montgomery): n / d for n < 2^31.
// ---------------------------------------------------------------------------
struct FastDiv {
  uint32_t d, m, s;
};

__host__ inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  f.s = s;
  f.m = (uint32_t)((((1ull << 32) * ((1ull << s) - d)) / d) + 1);
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.m) + n) >> f.s;
}

// ---------------------------------------------------------------------------
// Transposition of a 4-row x 2-column block of 16-bit values held as one
// 32-bit word per row: returns the two columns, each packed as 2 words
// (rows 0,1 | rows 2,3).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void transpose4x2(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3,
                                             u32x2& c0, u32x2& c1) {
  c0[0] = __builtin_amdgcn_perm(r1, r0, 0x05040100u);
  c0[1] = __builtin_amdgcn_perm(r3, r2, 0x05040100u);
  c1[0] = __builtin_amdgcn_perm(r1, r0, 0x07060302u);
  c1[1] = __builtin_amdgcn_perm(r3, r2, 0x07060302u);
}

// ---------------------------------------------------------------------------
// Transposed MFMA A operand straight from a row-major LDS tile.
//
// ds_read_b64_tr_b16 works on groups of 16 lanes: lane j of a group supplies
// the address of 4 consecutive 16-bit elements (chunk j) and lane i receives
// element i%4 of chunks i/4, 4 + i/4, 8 + i/4 and 12 + i/4.
//
// For a tile T[k][m] (row stride ld elements) the 32x32x16 A operand wants
// lane l to hold column m = l%32 at eight k values.  With every lane pointing
// at row tr_row(l) = 4*(l/32) + (l%16)/4 and column tr_col(l) = 16*((l/16)%2)
// + 4*(l%4) of a 16-row window, one read gives lane l the column l%32 at rows
// 4*(l/32) + {0,1,2,3}, and a second read 8 rows further down the rows
// 8 + 4*(l/32) + {0,1,2,3}: the k-slot order of a B operand taken from a
// 32x32 accumulator (registers 8h .. 8h+7 hold rows 16h + 4*(l/32) + {0..3}
// and 16h + 8 + 4*(l/32) + {0..3}).
// ---------------------------------------------------------------------------

// 16 bytes per lane from a buffer straight into LDS (no VGPRs): lane i's data
// lands at lds + 16*i bytes; `lds` must be wave-uniform.  Completion is
// counted by vmcnt.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rs, uint32_t voffset,
                                                  uint16_t* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(lds), 16,
                                           voffset, 0, 0, 0);
}

// The same with 4 bytes per lane (lane i's word lands at lds + 4*i bytes).
__device__ __forceinline__ void buffer_load_lds4(__amdgpu_buffer_rsrc_t rs, uint32_t voffset,
                                                 float* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(lds), 4,
                                           voffset, 0, 0, 0);
}

// x unchanged, in a VGPR, through an empty volatile asm: the compiler can no
// longer treat x as loop-invariant where this runs inside a loop body.
__device__ __forceinline__ void opaque(int& x) { asm volatile("" : "+v"(x)); }

__device__ __forceinline__ u32x2 ds_read_tr16(const uint16_t* p) {
  typedef __attribute__((ext_vector_type(4))) short s16x4;
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (s16x4 __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// A operand for rows [m0, m0+32) of T^T and k rows [k0, k0+16) of T, where
// `p` = tile + k0*ld + m0 + tr_row(l)*ld + tr_col(l) (the window offsets
// above; the kernels fold their LDS swizzle into them).
__device__ __forceinline__ u32x4 tr_operand(const uint16_t* p, int ld) {
  const u32x2 lo = ds_read_tr16(p);
  const u32x2 hi = ds_read_tr16(p + 8 * ld);
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// Stores one wave's 32 x D output block, held transposed in 32x32 MFMA
// accumulators (block db covers columns [32db, 32db+32); lane l holds row l%32
// and, per register group jj, columns 32db + 8jj + 4(l/32) + {0..3}), times a
// per-lane (per-row) factor `sc`, rounded to E.  Written straight out, every
// store instruction would touch 32 rows with 8 bytes each; staged through the
// wave's own LDS region `lds` (32*D elements, idle at this point) each lane
// stores 16 contiguous bytes and one instruction covers 64/(D/8) whole rows.
// The stores are non-temporal: whole 16-byte row segments need no write
// combining in L2, and the kernel's outputs are not read again by it (config
// 2: forward 19.2 -> 18.4 us, backward 50.3 -> 49.9 us, the HBM-cold step
// 96.6 -> 93.3 us; outputs identical).
// `grow` points at row 0 of the block, `ss` is the row stride in elements.
// Row r of the staging keeps 16-byte chunk c at position c ^ (r & 7).
// DP < D (head dims 16 and 32 run in the D = 64 layout): only the first DP
// columns are stored; the accumulators of the others are never read.  Only
// rows below nrows are stored (sequence tails).
template <typename E, int D, int DP = D>
__device__ __forceinline__ void store_block_rows(const f32x16 (&acc)[D / 32], float sc,
                                                 uint16_t* lds, uint16_t* grow, int64_t ss,
                                                 int nrows = 32) {
  static_assert(DP % 16 == 0 && DP <= D, "stored columns");
  constexpr int CPR = D / 8;     // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;  // rows per store instruction
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int c = 4 * db + jj;
      if (c >= DP / 8) continue;
      u32x2 w;
      w[0] = E::pack2(acc[db][4 * jj + 0] * sc, acc[db][4 * jj + 1] * sc);
      w[1] = E::pack2(acc[db][4 * jj + 2] * sc, acc[db][4 * jj + 3] * sc);
      *(u32x2*)(lds + l32 * D + ((c ^ (l32 & 7)) << 3) + 4 * g) = w;
    }
#pragma unroll
  for (int p = 0; p < 32 / RPI; ++p) {
    const int r = p * RPI + lane / CPR;
    const int c = lane % CPR;
    if ((DP < D && c >= DP / 8) || r >= nrows) continue;
    const u32x4 v = *(const u32x4*)(lds + r * D + ((c ^ (r & 7)) << 3));
    __builtin_nontemporal_store(v, (u32x4*)(grow + (int64_t)r * ss + 8 * c));
  }
}

}  // namespace mi
