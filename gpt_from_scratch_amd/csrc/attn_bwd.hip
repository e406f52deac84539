// attn_bwd.hip — flash-attention backward on gfx950 bf16/f16 matrix cores.
//
// Counterpart of FlashAttn.backward's three kernels (core/myFlashAttn.py:288-441):
//   delta  = rowsum(dO * O) in fp32                     (`_attn_bwd_precompute` :731-790)
//   dK, dV : per key tile, loop over query tiles         (`_attn_bwd_LoopQ` :795-1066)
//            P = exp(S*scale - lse), dV += P^T dO, dP = dO V^T,
//            dS = P * (dP - delta), dK += dS^T Q * scale
//   dQ     : per query tile, loop over key tiles         (`_attn_bwd_LoopKV` :1069-1317)
//            dQ += dS K * scale
// The formulas are the ones stated in the reference's docstring (:289-315).
//
// Layout choices (wave64, 32x32x16 MFMA; see mi_device.h for operand layouts):
//   * dK/dV kernel: a workgroup owns 128 keys (wave w: keys [32w, 32w+32)); the
//     wave's K and V rows live in registers as B operands for the whole loop.
//     S = Q K^T and dP = dO V^T are computed with keys along the lane index, so
//     P and dS come out of the accumulators already in B-operand form for
//     dV^T = dO^T P and dK^T = Q^T dS.  Q and dO tiles are staged row-major in
//     LDS (double-buffered): the A operands of S and dP are plain 16-byte
//     reads, those of dV^T and dK^T come from the same tiles through the
//     transposing LDS read (ds_read_b64_tr_b16).
//   * dQ kernel: a workgroup owns 128 queries; Q and dO rows live in registers;
//     S^T = K Q^T and dP^T = V dO^T put queries along the lane index so that
//     lse and delta are per-lane scalars and dS^T feeds dQ^T = K^T dS^T directly
//     (K^T read transposed from the row-major K tile).
//   * causal: key tiles only visit query tiles at or after the diagonal, query
//     tiles only key tiles at or before it; 32-row blocks entirely above the
//     diagonal are skipped per wave, blocks that straddle it are masked.
//   * head dims 16 and 32 run the D = 64 kernels with DP valid columns, and
//     sequence lengths that are not a multiple of 64 run the RAG
//     instantiations (rows past S staged as zeros and not stored); both are
//     template parameters, so the other instantiations are unaffected.
#include <type_traits>

#include "mi_device.h"
#include "mi_kernels.h"

namespace mi {

namespace {

// ---------------------------------------------------------------------------
// delta[b,h,s] = sum_d dO[b,h,s,d] * O[b,h,s,d]   (fp32 accumulation), and
// the second half of the workspace: lse * log2(e), the form the dK/dV loop
// subtracts inside exp2 (one multiply per row here instead of one per score
// there).  Eight lanes per row; each lane takes every 8th chunk of VEC elements.
// ---------------------------------------------------------------------------
template <int DT, int VEC>
__global__ __launch_bounds__(256) void attn_delta_kernel(AttnArgs a, FastDiv divS, FastDiv divH,
                                                         uint32_t nrows) {
  typedef typename Store<DT>::type T;
  // 32 rows per workgroup; nrows < 2^31, so the row index fits 32 bits
  const uint32_t row = blockIdx.x * 32u + (threadIdx.x >> 3);
  const int sub = threadIdx.x & 7;
  float acc = 0.f;
  if (row < nrows) {
    const uint32_t bh = fdiv(row, divS);
    const uint32_t s = row - bh * divS.d;
    const uint32_t b = fdiv(bh, divH);
    const uint32_t h = bh - b * divH.d;
    const T* o = (const T*)a.o.ptr + b * a.o.sb + h * a.o.sh + s * a.o.ss;
    const T* d = (const T*)a.dout.ptr + b * a.dout.sb + h * a.dout.sh + s * a.dout.ss;
    for (int c = sub * VEC; c < a.D; c += 8 * VEC) {
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        acc += Store<DT>::ld(o, c + e) * Store<DT>::ld(d, c + e);
    }
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  acc += __shfl_xor(acc, 4, 64);
  if (row < nrows && sub == 0) {
    a.delta[row] = acc;
    a.delta[nrows + row] = a.lse[row] * kLog2e;
  }
}

// One 16-bit value (bf16 or fp16, per DT) held in the low bits of x, as fp32.
template <int DT>
__device__ __forceinline__ float half_f32(uint32_t x) {
  if constexpr (DT == 2) return __uint_as_float(x << 16);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)x);
}

// The same for 16-bit O and dO with 16-byte aligned rows and D = 8 * LPR *
// NCH: lane l of a group of LPR (8; 4 at D = 32, 2 at D = 16) loads bytes
// [16(l%LPR), 16(l%LPR)+16) of each 16*LPR-byte chunk, so one wave
// instruction reads 64/LPR whole rows; every lane takes R rows (256/LPR
// apart) and issues all its loads before the first use.
template <int DT, int NCH, int R, int LPR = 8>
__global__ __launch_bounds__(256) void attn_delta_v16_kernel(AttnArgs a, FastDiv divS,
                                                             FastDiv divH, uint32_t nrows) {
  constexpr int RPW = 256 / LPR;  // rows per workgroup and pass
  const int sub = threadIdx.x & (LPR - 1);
  const uint32_t rbase = blockIdx.x * (RPW * R) + (threadIdx.x / LPR);
  u32x4 ov[R][NCH], dv[R][NCH];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t row = rbase + RPW * r;
    if (row < nrows) {
      const uint32_t bh = fdiv(row, divS);
      const uint32_t s = row - bh * divS.d;
      const uint32_t b = fdiv(bh, divH);
      const uint32_t h = bh - b * divH.d;
      const uint16_t* o = (const uint16_t*)a.o.ptr + b * a.o.sb + h * a.o.sh + s * a.o.ss;
      const uint16_t* d = (const uint16_t*)a.dout.ptr + b * a.dout.sb + h * a.dout.sh + s * a.dout.ss;
#pragma unroll
      for (int k = 0; k < NCH; ++k) {
        ov[r][k] = *(const u32x4*)(o + 8 * LPR * k + 8 * sub);
        dv[r][k] = *(const u32x4*)(d + 8 * LPR * k + 8 * sub);
      }
    } else {
#pragma unroll
      for (int k = 0; k < NCH; ++k) ov[r][k] = dv[r][k] = u32x4{0, 0, 0, 0};
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < NCH; ++k)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t x = ov[r][k][w], y = dv[r][k][w];
        acc += half_f32<DT>(x & 0xffffu) * half_f32<DT>(y & 0xffffu);
        acc += half_f32<DT>(x >> 16) * half_f32<DT>(y >> 16);
      }
    acc = group_sum<LPR>(acc);  // the xor-1, xor-2, xor-4 tree, by DPP
    const uint32_t row = rbase + RPW * r;
    if (row < nrows && sub == 0) {
      a.delta[row] = acc;
      a.delta[nrows + row] = a.lse[row] * kLog2e;
    }
  }
}

// ---------------------------------------------------------------------------
// Work items.  The gradients are produced by items of two kinds:
//   kind 0 (dK/dV, `_attn_bwd_LoopQ`): OWN keys of one head; the item loops
//          over query tiles, with K and V rows of its keys in registers;
//   kind 1 (dQ, `_attn_bwd_LoopKV`):   OWN queries of one head; the item loops
//          over key tiles, with Q and dO rows of its queries in registers.
// Both stream TILE-row tiles of the other two tensors into LDS with direct
// global -> LDS loads (double buffered, no registers, no LDS store
// instructions) and keep the same register layout (two resident row sets,
// the B operands), so one launch can run both kinds.
// ---------------------------------------------------------------------------
template <int D>
struct BwdCfg {
  static constexpr int OWN = 128;                   // rows owned by an item
  static constexpr int TILE = (D == 64) ? 64 : 32;  // rows of a streamed tile
  static constexpr int NT = 256;
  static constexpr int KS = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int TB = TILE / 32;             // 32-row blocks per streamed tile
  static constexpr int ELEMS = TILE * D;           // elements of one streamed tile
  static constexpr int CPR = D / 8;                // 16-byte chunks per row
  static constexpr int RPS = 64 / CPR;             // rows per 1 KB slice (one wave instruction)
  static constexpr int SPW = ELEMS * 2 / 1024 / 4; // slices per wave per tile
  static_assert(SPW >= 1 && TILE <= 64, "tile layout");
  static_assert(ELEMS >= 32 * D, "a tile buffer stages one wave's 32 output rows");
};

// LDS layout of a streamed tile: TILE rows of D elements, no padding; the
// 16-byte chunk c of row r sits at chunk position c ^ swz(r), with
//   swz(r) = 2*(r & 3) + ((r >> 2) & 1)        (D = 128)
//   swz(r) = that ^ 2*((r >> 3) & 1)           (D = 64)
// The tiles are read two ways: 16-byte row reads (16 consecutive rows per LDS
// cycle, one chunk each) and transposing reads (four consecutive rows and two
// adjacent chunks per 16 lanes: swz >> 1 takes four distinct values there).
// The gfx950 LDS has 64 four-byte banks and serves a 16-byte read for 16 lanes
// per cycle.  At D = 64 a 256-byte bank line holds two rows, so the row reads
// of rows r..r+15 are conflict-free when swz takes eight distinct values on
// the eight rows of each parity: the term in bit 3 of r gives that (without
// it rows r and r + 8 collide, a 2-way conflict), at the price of a second
// offset for the transposing read 8 rows on.  At D = 128 a row fills a bank
// line, so 16 rows need 16 positions: SW16 adds bit 3 of r as bit 3 of the
// swizzle (the dQ kind; the dK/dV kind, at its register limit, cannot hold the
// extra offsets, keeps the 3-bit swizzle repeating every 8 rows and its 2-way
// conflict).  Each kind writes and reads its own staged tiles, so the two may
// differ.
template <int D, bool SW16 = false>
__device__ __forceinline__ int bwd_swz(int r) {
  const int s = ((r & 3) << 1) | ((r >> 2) & 1);
  if constexpr (D == 64) return s ^ (((r >> 3) & 1) << 1);
  else if constexpr (SW16) return s | (((r >> 3) & 1) << 3);
  else return s;
}

// Per-lane LDS byte offsets of the two tile reads: 16-byte row reads (row
// l%32, chunk 2ks + l/32) and transposing reads (rows 4(l/32) + (l%16)/4 and,
// for the operand's second half, those + 8; column 32db + 16((l/16)%2) +
// 4(l%4)).  A 3-bit swz only changes the low three bits of a chunk index, so
// chunk c + 8 sits 128 bytes after chunk c, and swz repeats every 16 rows:
// four row offsets and two (D = 128: the second half is 8 rows on, same
// swizzle) or four transposing offsets, plus immediates, cover every read.
// With SW16 bit 3 of the position is bit 3 of the chunk XOR bit 3 of the row:
// eight row offsets; the transposing reads' first half (rows < 8) is as
// without, the second half flips bit 3 (+128 bytes for chunks < 8, -128 above).
// The offsets hold the lane part only: every read adds its tile buffer and
// block as a constant, which the LDS instruction takes as its immediate
// offset.  refresh() at the top of each step keeps the compiler from
// hoisting "buffer + offset" sums out of the step loop, which would hold one
// register per buffer, parity and offset (34 in the dK/dV loop, 24 in the dQ
// loop) instead of one per offset.
template <int D, bool SW16 = false>
struct LdsOffsets {
  static constexpr bool R8 = D == 128 && SW16;
  int r4[R8 ? 8 : 4], t2[2], t2h[D == 64 || R8 ? 2 : 1];
  __device__ __forceinline__ int row(int ks) const {
    if constexpr (R8) return r4[ks];
    else return r4[ks & 3] + 128 * (ks >> 2);
  }
  __device__ __forceinline__ int tr(int db) const { return t2[db & 1] + 128 * (db >> 1); }
  __device__ __forceinline__ int tr_hi(int db) const {
    if constexpr (D == 64) return t2h[db & 1] + 128 * (db >> 1);
    else if constexpr (R8) return t2h[db & 1] + 128 * (1 - (db >> 1));
    else return tr(db) + 16 * D;
  }
  __device__ __forceinline__ void refresh() {
#pragma unroll
    for (int i = 0; i < (R8 ? 8 : 4); ++i) opaque(r4[i]);
#pragma unroll
    for (int i = 0; i < 2; ++i) opaque(t2[i]);
#pragma unroll
    for (int i = 0; i < (D == 64 || R8 ? 2 : 1); ++i) opaque(t2h[i]);
  }
};

template <int D, bool SW16 = false>
__device__ __forceinline__ LdsOffsets<D, SW16> lds_offsets(int lane) {
  const int l32 = lane & 31;
  const int g = lane >> 5;
  LdsOffsets<D, SW16> o;
  if constexpr (LdsOffsets<D, SW16>::R8) {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      o.r4[ks] = 2 * (l32 * D + (((2 * ks + g) ^ bwd_swz<D, SW16>(l32)) << 3));
  } else {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      o.r4[ks] = 2 * (l32 * D + (((2 * ks + g) ^ bwd_swz<D, SW16>(l32)) << 3));
  }
#pragma unroll
  for (int db = 0; db < 2; ++db) {
    const int r = 4 * g + ((lane & 15) >> 2);
    const int ch = 4 * db + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    o.t2[db] = 2 * (r * D + ((ch ^ bwd_swz<D, SW16>(r)) << 3) + 4 * (lane & 1));
    if constexpr (D == 64)
      o.t2h[db] = 2 * ((r + 8) * D + ((ch ^ bwd_swz<D>(r + 8)) << 3) + 4 * (lane & 1));
    else if constexpr (LdsOffsets<D, SW16>::R8)
      // rows r + 8 (< 16): low three bits as row r, bit 3 of the chunk
      // flipped; the +128 / -128 bytes of that flip is tr_hi's immediate
      o.t2h[db] = 2 * ((r + 8) * D + ((ch ^ (bwd_swz<D, SW16>(r + 8) & 7)) << 3) + 4 * (lane & 1));
  }
  return o;
}

// The element of type T at `bytes` bytes past an LDS buffer.
template <typename T>
__device__ __forceinline__ const T* lds_at(const void* base, int bytes) {
  return (const T*)((const char*)base + bytes);
}

// The transposed A operand from its two halves (rows k0..k0+7 and k0+8..+15).
__device__ __forceinline__ u32x4 tr_operand2(const uint16_t* lo, const uint16_t* hi) {
  const u32x2 a = ds_read_tr16(lo);
  const u32x2 b = ds_read_tr16(hi);
  return u32x4{a[0], a[1], b[0], b[1]};
}

// The four angles i0 .. i0+3 of table row `pos` (contiguous angles, dtype
// TDT: 0 fp32, 1 fp16, 2 bf16) with one vector load, kept packed until used.
template <int TDT>
struct Tab4 {
  typedef typename std::conditional<TDT == 0, f32x4, u32x2>::type type;
  static __device__ __forceinline__ type load(const void* tab, int64_t row_stride, int64_t pos,
                                              int i0) {
    if constexpr (TDT == 0)
      return *(const f32x4*)((const float*)tab + pos * row_stride + i0);
    else
      return *(const u32x2*)((const uint16_t*)tab + pos * row_stride + i0);
  }
  static __device__ __forceinline__ float get(const type& q, int k) {
    if constexpr (TDT == 0) {
      return q[k];
    } else {
      const uint16_t h = (uint16_t)(q[k >> 1] >> (16 * (k & 1)));
      return TDT == 2 ? BF16::to_f32(h) : F16::to_f32(h);
    }
  }
};

// store_block_rows with the inverse rotary rotation applied on the way out.
// The block is staged in LDS rounded to E, exactly as an unfused dQ / dK is
// stored; on the read back each lane holds 8 consecutive elements of row r,
// i.e. the interleaved pairs (2i, 2i+1), i = 4c .. 4c+3, at sequence position
// pos0 + r, and reads their angles with one vector load per table, rotates
// them with rope_rotate (the RoPE kernel's arithmetic) and rounds again -- the
// values the separate inverse RoPE pass over the stored gradient would write.
// Tables: 16-bit, contiguous angles, rows 4-angle aligned (checked by the
// host).
// TAIL: rows at or past nrows (sequence tails) are not stored, and read the
// angles of row nrows - 1.
template <typename E, int D, int TDT, bool TAIL>
__device__ __forceinline__ void store_block_rows_rope_t(const f32x16 (&acc)[D / 32], float sc,
                                                        uint16_t* lds, uint16_t* grow,
                                                        int64_t ss, const RopeTab& t, int pos0,
                                                        int nrows) {
  constexpr int CPR = D / 8;
  constexpr int RPI = 64 / CPR;
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int c = 4 * db + jj;
      u32x2 w;
      w[0] = E::pack2(acc[db][4 * jj + 0] * sc, acc[db][4 * jj + 1] * sc);
      w[1] = E::pack2(acc[db][4 * jj + 2] * sc, acc[db][4 * jj + 3] * sc);
      *(u32x2*)(lds + l32 * D + ((c ^ (l32 & 7)) << 3) + 4 * g) = w;
    }
  // the angles after the accumulators are staged (and dead): loading them
  // earlier would hold both at once.  Groups of PCH store instructions load
  // their angles together (all eight at D = 64; four at a time at D = 128,
  // whose dK/dV kernel sits at its register limit).
  __builtin_amdgcn_sched_barrier(0);
  constexpr int NP = 32 / RPI;
  constexpr int PCH = D == 128 ? 4 : NP;
#pragma unroll
  for (int p0 = 0; p0 < NP; p0 += PCH) {
    typename Tab4<TDT>::type cs[PCH], sn[PCH];
#pragma unroll
    for (int i = 0; i < PCH; ++i) {
      const int r0 = (p0 + i) * RPI + lane / CPR;
      const int r = TAIL ? min(r0, nrows - 1) : r0;
      const int c = lane % CPR;
      cs[i] = Tab4<TDT>::load(t.cos, t.cs_s, pos0 + r, 4 * c);
      sn[i] = Tab4<TDT>::load(t.sin, t.ss_s, pos0 + r, 4 * c);
    }
#pragma unroll
    for (int i = 0; i < PCH; ++i) {
      const int r = (p0 + i) * RPI + lane / CPR;
      const int c = lane % CPR;
      const u32x4 v = *(const u32x4*)(lds + r * D + ((c ^ (r & 7)) << 3));
      u32x4 o;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float re, ro;
        rope_rotate(E::to_f32((uint16_t)(v[k] & 0xffffu)), E::to_f32((uint16_t)(v[k] >> 16)),
                    Tab4<TDT>::get(cs[i], k), Tab4<TDT>::get(sn[i], k), true, re, ro);
        o[k] = E::pack2(re, ro);
      }
      if (!TAIL || r < nrows) __builtin_nontemporal_store(o, (u32x4*)(grow + (int64_t)r * ss + 8 * c));
    }
  }
}

template <typename E, int D, bool TAIL = false>
__device__ __forceinline__ void store_block_rows_rope(const f32x16 (&acc)[D / 32], float sc,
                                                      uint16_t* lds, uint16_t* grow, int64_t ss,
                                                      const RopeTab& t, int pos0,
                                                      int nrows = 32) {
  // 16-bit tables only (the host runs fp32 tables as a separate pass)
  if (t.tdt == 2)
    store_block_rows_rope_t<E, D, 2, TAIL>(acc, sc, lds, grow, ss, t, pos0, nrows);
  else
    store_block_rows_rope_t<E, D, 1, TAIL>(acc, sc, lds, grow, ss, t, pos0, nrows);
}

struct BwdItem {
  int kind;  // 0: dK/dV, 1: dQ
  int tile;  // key tile (kind 0) or query tile (kind 1), OWN rows each
  int bh;
};

template <int D>
struct Resident {
  u32x4 r[2][D / 16];  // kind 0: K, -V rows; kind 1: Q, dO rows (lane: row l%32, 8 columns)
  float lse2, dl;      // kind 1: lse*log2e and delta of this lane's query row
};

// One LDS staging buffer: the two streamed tiles and, for the dK/dV kind,
// lse * log2(e) and delta of the tile's query rows (as in the workspace).
struct BwdBuf {
  uint16_t* t0;
  uint16_t* t1;
  float* sl;
};

// Tile buffer w of the four (ELEMS elements each, at least 32*D): the output
// staging area of wave w once the steps are over.
__device__ __forceinline__ uint16_t* wave_stage_buf(const BwdBuf (&bufs)[2], int wave) {
  // selects, not an index: a runtime index would put `bufs` in scratch memory
  uint16_t* const b0 = (wave & 1) ? bufs[0].t1 : bufs[0].t0;
  uint16_t* const b1 = (wave & 1) ? bufs[1].t1 : bufs[1].t0;
  return (wave & 2) ? b1 : b0;
}

// Where an item's streamed tiles come from: head bases and strides, and this
// lane's byte offsets inside a tile for its slices (buffer loads, so that
// advancing a tile is scalar arithmetic).
template <int D>
struct StageSrc {
  const uint16_t* p0;
  const uint16_t* p1;
  int64_t ss0, ss1;
  uint32_t off0[BwdCfg<D>::SPW], off1[BwdCfg<D>::SPW];
  const float* lse;    // lse * log2(e) rows of this head
  const float* delta;
};

__device__ __forceinline__ const uint16_t* head_ptr(const TensorArg& t, int b, int h) {
  return (const uint16_t*)t.ptr + b * t.sb + h * t.sh;
}

template <int D, bool CAUSAL>
__device__ __forceinline__ int first_row(const BwdItem& it) {
  return (CAUSAL && it.kind == 0) ? it.tile * BwdCfg<D>::OWN : 0;
}

// SKIP0: leave res.r[0] unloaded (the D = 128 dK/dV kind keeps K in LDS).
// DP < D: rows of DP columns; the registers of columns past DP are zeros.
// RAG: the descriptors end at row S (rows past it load as zeros, lse and
// delta as 0).
template <int D, bool SKIP0 = false, int DP = D, bool RAG = false>
__device__ __forceinline__ void load_resident(const AttnArgs& a, const BwdItem& it,
                                              Resident<D>& res) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = it.bh / a.H;
  const int h = it.bh % a.H;
  const TensorArg& t0 = it.kind ? a.q : a.k;
  const TensorArg& t1 = it.kind ? a.dout : a.v;
  const int w0 = it.tile * BwdCfg<D>::OWN + 32 * wave;  // first row of this wave (SGPR)
  if (w0 < a.S) {
    // wave base in the descriptor, lane offset (row l%32, 8 columns) in one VGPR
    const int nr = RAG ? min(32, a.S - w0) : 32;
    const auto r0 = tile_rsrc(head_ptr(t0, b, h) + (int64_t)w0 * t0.ss, rows_extent(nr, t0.ss, DP));
    const auto r1 = tile_rsrc(head_ptr(t1, b, h) + (int64_t)w0 * t1.ss, rows_extent(nr, t1.ss, DP));
    const uint32_t o0 = (uint32_t)(((lane & 31) * t0.ss + 8 * (lane >> 5)) * 2);
    const uint32_t o1 = (uint32_t)(((lane & 31) * t1.ss + 8 * (lane >> 5)) * 2);
    // kind 0 keeps V negated (sign bits of both 16-bit halves flipped)
    const uint32_t neg = it.kind ? 0u : 0x80008000u;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      if (ks >= DP / 16) {
        res.r[0][ks] = u32x4{0, 0, 0, 0};
        res.r[1][ks] = u32x4{0, 0, 0, 0};
        continue;
      }
      if (!SKIP0) res.r[0][ks] = __builtin_amdgcn_raw_buffer_load_b128(r0, o0 + 32 * ks, 0, 0);
      res.r[1][ks] = __builtin_amdgcn_raw_buffer_load_b128(r1, o1 + 32 * ks, 0, 0) ^ neg;
    }
    if (it.kind) {
      const int64_t o = (int64_t)it.bh * a.S + w0;
      res.lse2 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                     tile_rsrc(a.lse2 + o, nr * 4), (lane & 31) * 4, 0, 0));
      res.dl = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                   tile_rsrc(a.delta + o, nr * 4), (lane & 31) * 4, 0, 0));
    }
  } else {
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      res.r[0][ks] = u32x4{0, 0, 0, 0};
      res.r[1][ks] = u32x4{0, 0, 0, 0};
    }
    res.lse2 = 0.f;
    res.dl = 0.f;
  }
}

// DP < D: chunks past DP (padding) take the out-of-range offset and stage as
// zeros.
template <int D, bool SW16 = false, int DP = D>
__device__ __forceinline__ StageSrc<D> stage_src(const AttnArgs& a, const BwdItem& it) {
  using C = BwdCfg<D>;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = it.bh / a.H;
  const int h = it.bh % a.H;
  const TensorArg& t0 = it.kind ? a.k : a.q;
  const TensorArg& t1 = it.kind ? a.v : a.dout;
  StageSrc<D> s;
  s.p0 = head_ptr(t0, b, h);
  s.p1 = head_ptr(t1, b, h);
  s.ss0 = t0.ss;
  s.ss1 = t1.ss;
  // Slice m of this wave covers rows (wave + 4m)*RPS ..; lane i writes chunk
  // position i%CPR of row (wave + 4m)*RPS + i/CPR, i.e. fetches chunk
  // (i%CPR) ^ swz(row).
#pragma unroll
  for (int m = 0; m < C::SPW; ++m) {
    const int r = (wave + 4 * m) * C::RPS + lane / C::CPR;
    const int ch = (lane % C::CPR) ^ bwd_swz<D, SW16>(r);
    const bool pad = DP < D && ch >= DP / 8;
    s.off0[m] = pad ? kOobOffset : (uint32_t)((r * t0.ss + (ch << 3)) * 2);
    s.off1[m] = pad ? kOobOffset : (uint32_t)((r * t1.ss + (ch << 3)) * 2);
  }
  s.lse = a.lse2 + (int64_t)it.bh * a.S;
  s.delta = a.delta + (int64_t)it.bh * a.S;
  return s;
}

// Streamed tile starting at row `row0` straight into LDS buffer `dst`;
// completion is tracked by vmcnt and the barrier that ends the step.
// RAG: the descriptors end at row S (rows past it stage as zeros, their lse
// and delta as 0).
template <int D, int DP = D, bool RAG = false>
__device__ __forceinline__ void dma_stage(const StageSrc<D>& s, int kind, int row0,
                                          const BwdBuf& dst, int S = 0) {
  using C = BwdCfg<D>;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nr = RAG ? min(C::TILE, S - row0) : C::TILE;
  const auto r0 = tile_rsrc(s.p0 + (int64_t)row0 * s.ss0, rows_extent(nr, s.ss0, DP));
  const auto r1 = tile_rsrc(s.p1 + (int64_t)row0 * s.ss1, rows_extent(nr, s.ss1, DP));
#pragma unroll
  for (int m = 0; m < C::SPW; ++m) {
    buffer_load_lds16(r0, s.off0[m], dst.t0 + (wave + 4 * m) * 512);
    buffer_load_lds16(r1, s.off1[m], dst.t1 + (wave + 4 * m) * 512);
  }
  if (kind == 0 && wave >= 2 && lane < C::TILE) {
    // waves 2 and 3: lse and delta of the tile's query rows (4 bytes per lane)
    const float* src = (wave == 2 ? s.lse : s.delta) + row0;
    buffer_load_lds4(tile_rsrc(src, nr * 4), lane * 4, dst.sl + (wave - 2) * C::TILE);
  }
}

// ---------------------------------------------------------------------------
// dK / dV item.  Wave w owns keys [kv0 + 32w, +32).  S = Q K^T and
// dP = dO V^T are computed with keys along the lane index, so P and dS leave
// the accumulators in B-operand form for dV^T = dO^T P and dK^T = Q^T dS; the
// dO^T and Q^T A operands are read transposed from the same tiles.
// The dP accumulators start at +delta and the V rows are negated once per
// item, so they hold delta - dO V^T and dS = -P * acc.
// At D = 128 the wave's 32 K rows live in LDS (its own 8 KB region, in the
// tiles' swizzle) rather than in registers: K, -V and the dK and dV
// accumulators together need ~290 VGPRs, and holding all of them spilled
// ~390 bytes per lane.  The region then stages the wave's dK and dV stores.
// ---------------------------------------------------------------------------
template <typename E, int D, bool CAUSAL, bool ROPE, int DP, bool RAG>
__device__ __forceinline__ void dkdv_item(const AttnArgs& a, const BwdItem& it,
                                          const BwdBuf (&bufs)[2]) {
  using C = BwdCfg<D>;
  constexpr int KSP = DP / 16;         // k-steps over the valid columns
  constexpr int DBP = (DP + 31) / 32;  // accumulator blocks holding valid columns
  constexpr bool PREFETCH = D == 64;  // operands a block ahead (D = 128 has no registers for it)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int S = a.S;

  const int kv0 = it.tile * C::OWN;
  const int kw = kv0 + 32 * wave;
  const bool wave_valid = kw < S;
  const int b = it.bh / a.H;
  const int h = it.bh % a.H;
  constexpr bool K_IN_LDS = (D == 128);
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[K_IN_LDS ? C::OWN * D : 8];
  uint16_t* const kw_lds = k_lds + (K_IN_LDS ? wave * 32 * D : 0);

  // per-lane LDS byte offsets: 16-byte row reads (row l32, chunk 2ks + g) and
  // transposing reads (row 4g + (lane%16)/4, column 32db + 16((lane/16)%2) + 4(lane%4)),
  // and the lane's part of the lse / delta reads (query rows 4g + i of each group of 8)
  LdsOffsets<D> lo = lds_offsets<D>(lane);
  int slo = 16 * g;

  const int q_begin = first_row<D, CAUSAL>(it);
  const int nq = RAG ? (S - q_begin + C::TILE - 1) / C::TILE : (S - q_begin) / C::TILE;
  const StageSrc<D> src = stage_src<D, false, DP>(a, it);

  f32x16 dk[C::DB], dv[C::DB];
#pragma unroll
  for (int i = 0; i < C::DB; ++i) {
    dk[i] = f32x16{};
    dv[i] = f32x16{};
  }
  const float c = a.scale_log2;

  // First tile's loads before the resident rows: one memory round trip for
  // both (the V negation waits for its rows, not for the tile).
  dma_stage<D, DP, RAG>(src, 0, q_begin, bufs[0], S);
  if constexpr (K_IN_LDS) {
    // the wave's 32 K rows: 8 one-KB slices of 4 rows, lane i writing chunk
    // position i%16 of row 4m + i/16, i.e. fetching chunk (i%16) ^ swz(row)
    if (wave_valid) {
      const auto rk = tile_rsrc(head_ptr(a.k, b, h) + (int64_t)kw * a.k.ss,
                                rows_extent(RAG ? min(32, S - kw) : 32, a.k.ss, D));
#pragma unroll
      for (int m = 0; m < 32 * D * 2 / 1024; ++m) {
        const int r = m * C::RPS + lane / C::CPR;
        const int col = ((lane % C::CPR) ^ bwd_swz<D>(r)) << 3;
        buffer_load_lds16(rk, (uint32_t)((r * a.k.ss + col) * 2), kw_lds + m * 512);
      }
    }
  }
  Resident<D> res;
  load_resident<D, K_IN_LDS, DP, RAG>(a, it, res);
  const u32x4(&kf)[C::KS] = res.r[0];
  const u32x4(&vn)[C::KS] = res.r[1];  // -V
  __syncthreads();

  // Query tile j in buffer P = j & 1 (a compile-time tag); the next tile goes
  // into the other buffer.  MASKED steps are the ones that straddle this
  // item's keys (causal only): there a 32-row block entirely before a wave's
  // keys is skipped and the block on the wave's diagonal (qbs == kw,
  // everything is 32-aligned) is masked with the fixed triangle key > query.
  auto step = [&](int j, auto masked_tag, auto last_tag, auto parity) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool LAST = decltype(last_tag)::value;
    constexpr int P = decltype(parity)::value;
    const int q0 = q_begin + j * C::TILE;
    // (at D = 128 the last step is not peeled: a uniform branch skips its load)
    if (!LAST && (D == 64 || j + 1 < nq))
      dma_stage<D, DP, RAG>(src, 0, q0 + C::TILE, bufs[P ^ 1], S);

    lo.refresh();
    opaque(slo);
    if (wave_valid && (!MASKED || q0 + C::TILE - 1 >= kw)) {
      const uint16_t* Qs = bufs[P].t0;
      const uint16_t* dOs = bufs[P].t1;
      const float* sl = bufs[P].sl;
      u32x4 pb[C::TB][2], sb[C::TB][2];
      bool live[C::TB];
      // Each block's A operands and delta rows are requested before its first
      // product: block 0's at the top of the step, block 1's right after
      // block 0's products are issued (one LDS round trip per block instead
      // of one per product).  The scheduling barriers keep the compiler from
      // sinking the reads back next to their uses.
      u32x4 qa[KSP], da[KSP];
      f32x16 sacc[C::TB], dpacc[C::TB];
      auto read_ops = [&](int qb) __attribute__((always_inline)) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const f32x4 d4 = *lds_at<f32x4>(sl, slo + 4 * (C::TILE + 32 * qb + 8 * jj));
#pragma unroll
          for (int i = 0; i < 4; ++i) dpacc[qb][4 * jj + i] = d4[i];
        }
#pragma unroll
        for (int ks = 0; ks < KSP; ++ks) {
          qa[ks] = *lds_at<u32x4>(Qs, 64 * qb * D + lo.row(ks));
          da[ks] = *lds_at<u32x4>(dOs, 64 * qb * D + lo.row(ks));
        }
      };
      if constexpr (PREFETCH) {
        read_ops(0);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int qb = 0; qb < C::TB; ++qb) {
        const int qbs = q0 + 32 * qb;
        live[qb] = !MASKED || (qbs + 31 >= kw);
        if constexpr (!PREFETCH) read_ops(qb);
        if (live[qb]) {
          sacc[qb] = f32x16{};
#pragma unroll
          for (int ks = 0; ks < KSP; ++ks) {
            if constexpr (K_IN_LDS)
              sacc[qb] = E::mfma(qa[ks], *lds_at<u32x4>(kw_lds, lo.row(ks)), sacc[qb]);
            else
              sacc[qb] = E::mfma(qa[ks], kf[ks], sacc[qb]);
          }
#pragma unroll
          for (int ks = 0; ks < KSP; ++ks) dpacc[qb] = E::mfma(da[ks], vn[ks], dpacc[qb]);
        }
        if constexpr (PREFETCH) {
          if (qb + 1 < C::TB) {
            read_ops(qb + 1);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
#pragma unroll
      for (int qb = 0; qb < C::TB; ++qb) {
        if (!live[qb]) continue;
        const int qbs = q0 + 32 * qb;
        f32x16& s = sacc[qb];
        f32x16& dp = dpacc[qb];
        const bool diag = MASKED && qbs == kw;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const f32x4 l4 = *lds_at<f32x4>(sl, slo + 4 * (32 * qb + 8 * jj));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 4 * jj + i;
            float p = fast_exp2(__builtin_fmaf(s[r], c, -l4[i]));
            // (key row l32 against query column 8jj + 4g + i, as l32 - 4g against
            // a constant: one register instead of one per element)
            if (MASKED && diag && l32 - 4 * g > 8 * jj + i) p = 0.f;
            s[r] = p;
            dp[r] = -(p * dp[r]);
          }
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            pb[qb][hh][w] = E::pack2(s[8 * hh + 2 * w], s[8 * hh + 2 * w + 1]);
            sb[qb][hh][w] = E::pack2(dp[8 * hh + 2 * w], dp[8 * hh + 2 * w + 1]);
          }
      }
#pragma unroll
      for (int qb = 0; qb < C::TB; ++qb) {
        if (!live[qb]) continue;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int db = 0; db < DBP; ++db) {
            const int off = 2 * (32 * qb + 16 * hh) * D;  // bytes
            dv[db] = E::mfma(tr_operand2(lds_at<uint16_t>(dOs, off + lo.tr(db)),
                                         lds_at<uint16_t>(dOs, off + lo.tr_hi(db))),
                             pb[qb][hh], dv[db]);
            dk[db] = E::mfma(tr_operand2(lds_at<uint16_t>(Qs, off + lo.tr(db)),
                                         lds_at<uint16_t>(Qs, off + lo.tr_hi(db))),
                             sb[qb][hh], dk[db]);
          }
        }
      }
    }
    __syncthreads();
  };

  // Steps [j, j_end) with the buffer parity fixed per call site.
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  int j = 0;
  auto run = [&](int j_end, auto masked_tag) __attribute__((always_inline)) {
    if ((j & 1) && j < j_end) step(j++, masked_tag, std::false_type{}, P1{});
    for (; j + 1 < j_end; j += 2) {
      step(j, masked_tag, std::false_type{}, P0{});
      step(j + 1, masked_tag, std::false_type{}, P1{});
    }
    if (j < j_end) step(j++, masked_tag, std::false_type{}, P0{});
  };
  // nq >= 1 (S > q_begin)
  if constexpr (D == 128) {
    // Peeled last steps (four more copies of the step) raised the register
    // pressure of the whole item past 256 and spilled; here the loop runs to
    // nq and the step skips the load past the end.
    if constexpr (CAUSAL) run(min(nq, C::OWN / C::TILE), std::true_type{});
    run(nq, std::false_type{});
  } else {
    const int n_diag = CAUSAL ? min(nq - 1, C::OWN / C::TILE) : 0;
    if constexpr (CAUSAL) run(n_diag, std::true_type{});
    run(nq - 1, std::false_type{});
    const bool last_masked = CAUSAL && nq - 1 < C::OWN / C::TILE;
    if (last_masked) {
      if (j & 1) step(j, std::true_type{}, std::true_type{}, P1{});
      else step(j, std::true_type{}, std::true_type{}, P0{});
    } else {
      if (j & 1) step(j, std::false_type{}, std::true_type{}, P1{});
      else step(j, std::false_type{}, std::true_type{}, P0{});
    }
  }

  if (!wave_valid) return;
  const int nrows = RAG ? min(32, S - kw) : 32;  // keys of this wave below S
  uint16_t* const dk_rows = (uint16_t*)a.dk.ptr + b * a.dk.sb + h * a.dk.sh + (int64_t)kw * a.dk.ss;
  uint16_t* const dv_rows = (uint16_t*)a.dv.ptr + b * a.dv.sb + h * a.dv.sh + (int64_t)kw * a.dv.ss;
  if constexpr (D == 64) {
    // The staging buffers are idle after the last step's barrier: wave w
    // stages its rows (dK, then dV) through tile buffer w.
    uint16_t* stage = wave_stage_buf(bufs, wave);
    // dV first: its accumulators are dead before dK's rotation needs registers
    store_block_rows<E, D, DP>(dv, 1.f, stage, dv_rows, a.dv.ss, nrows);
    if (ROPE && a.rope.cos)
      store_block_rows_rope<E, D, RAG>(dk, a.scale, stage, dk_rows, a.dk.ss, a.rope, kw, nrows);
    else
      store_block_rows<E, D, DP>(dk, a.scale, stage, dk_rows, a.dk.ss, nrows);
  } else {
    // D = 128: the wave's K region (32 x D, its own) is idle after the last
    // step.  (Written straight from the accumulators instead, 8 bytes per lane
    // and row, the launch measured the same at configs 3 and 4 and 2% slower
    // at B8 S1024.)
    store_block_rows<E, D>(dv, 1.f, kw_lds, dv_rows, a.dv.ss, nrows);
    if (ROPE && a.rope.cos)
      store_block_rows_rope<E, D, RAG>(dk, a.scale, kw_lds, dk_rows, a.dk.ss, a.rope, kw, nrows);
    else
      store_block_rows<E, D>(dk, a.scale, kw_lds, dk_rows, a.dk.ss, nrows);
  }
}

// ---------------------------------------------------------------------------
// dQ item.  Wave w owns queries [q0 + 32w, +32).  S^T = K Q^T and
// dP^T = V dO^T put queries along the lane index, so lse and delta are
// per-lane scalars and dS^T feeds dQ^T = K^T dS^T directly (K^T read
// transposed from the K tile).
// ---------------------------------------------------------------------------
template <typename E, int D, bool CAUSAL, bool ROPE, int DP, bool RAG>
__device__ __forceinline__ void dq_item(const AttnArgs& a, const BwdItem& it,
                                        const BwdBuf (&bufs)[2]) {
  using C = BwdCfg<D>;
  constexpr int KSP = DP / 16;         // k-steps over the valid columns
  constexpr int DBP = (DP + 31) / 32;  // accumulator blocks holding valid columns
  static_assert(D == 64 || D == 128, "head dim of the item layout");
  constexpr bool PREFETCH = D == 64;  // operands a block ahead (D = 128: one block per tile, below)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int S = a.S;

  const int q0 = it.tile * C::OWN;
  const int qw = q0 + 32 * wave;
  const bool wave_valid = qw < S;

  // D = 128: the 4-bit swizzle (conflict-free row reads), see bwd_swz
  LdsOffsets<D, D == 128> lo = lds_offsets<D, D == 128>(lane);

  const int kv_end = CAUSAL ? min(q0 + C::OWN, S) : S;
  const int nkv = RAG ? (kv_end + C::TILE - 1) / C::TILE : kv_end / C::TILE;
  const StageSrc<D> src = stage_src<D, D == 128, DP>(a, it);

  f32x16 acc[C::DB];
#pragma unroll
  for (int i = 0; i < C::DB; ++i) acc[i] = f32x16{};
  const float c = a.scale_log2;

  // First tile's loads before the resident rows (one round trip for both).
  dma_stage<D, DP, RAG>(src, 1, 0, bufs[0], S);
  Resident<D> res;
  load_resident<D, false, DP, RAG>(a, it, res);
  const u32x4(&qf)[C::KS] = res.r[0];
  const u32x4(&df)[C::KS] = res.r[1];
  const float lse2 = res.lse2;
  const float dl = res.dl;
  // The dP^T accumulators start at -delta (a per-lane constant here), so they
  // end at dP - delta and dS = P * acc is one multiply.
  f32x16 ndl;
#pragma unroll
  for (int r = 0; r < 16; ++r) ndl[r] = -dl;
  __syncthreads();

  // Key tile j in buffer P = j & 1.  MASKED steps are the causal ones that
  // straddle this item's queries: a 32-key block after a wave's queries is
  // skipped and the block on the wave's diagonal (kvb == qw) gets the fixed
  // triangle mask.  Earlier tiles are visible to every query.
  auto step = [&](int j, auto masked_tag, auto last_tag, auto parity) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool LAST = decltype(last_tag)::value;
    constexpr int P = decltype(parity)::value;
    const int kv0 = j * C::TILE;
    if (!LAST) dma_stage<D, DP, RAG>(src, 1, kv0 + C::TILE, bufs[P ^ 1], S);

    lo.refresh();
    if (wave_valid && (!MASKED || kv0 <= qw + 31)) {
      const uint16_t* Ks = bufs[P].t0;
      const uint16_t* Vs = bufs[P].t1;
      u32x4 sb[C::TB][2];
      bool live[C::TB];
      // Each block's A operands requested before its first product (block
      // 0's at the top of the step, block 1's once block 0's products are
      // issued), as in the dK/dV item.
      u32x4 ka[KSP], va[KSP];
      f32x16 sacc[C::TB], dpacc[C::TB];
      auto read_ops = [&](int kb) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < KSP; ++ks) {
          ka[ks] = *lds_at<u32x4>(Ks, 64 * kb * D + lo.row(ks));
          va[ks] = *lds_at<u32x4>(Vs, 64 * kb * D + lo.row(ks));
        }
      };
      if constexpr (PREFETCH) {
        read_ops(0);
        __builtin_amdgcn_sched_barrier(0);
      } else if constexpr (D == 128) {
        // one block per tile: its K operands up front, its V operands while
        // the S^T products run (one LDS round trip before each chain)
#pragma unroll
        for (int ks = 0; ks < KSP; ++ks) ka[ks] = *lds_at<u32x4>(Ks, lo.row(ks));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < KSP; ++ks) va[ks] = *lds_at<u32x4>(Vs, lo.row(ks));
      }
#pragma unroll
      for (int kb = 0; kb < C::TB; ++kb) {
        const int kvb = kv0 + 32 * kb;
        live[kb] = !MASKED || (kvb <= qw + 31);
        if (live[kb]) {
          sacc[kb] = f32x16{};
          dpacc[kb] = ndl;
#pragma unroll
          for (int ks = 0; ks < KSP; ++ks) sacc[kb] = E::mfma(ka[ks], qf[ks], sacc[kb]);
          if constexpr (D == 128) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int ks = 0; ks < KSP; ++ks) dpacc[kb] = E::mfma(va[ks], df[ks], dpacc[kb]);
        }
        if constexpr (PREFETCH) {
          if (kb + 1 < C::TB) {
            read_ops(kb + 1);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
#pragma unroll
      for (int kb = 0; kb < C::TB; ++kb) {
        if (!live[kb]) continue;
        const int kvb = kv0 + 32 * kb;
        f32x16& s = sacc[kb];
        f32x16& dp = dpacc[kb];
        const bool diag = MASKED && kvb == qw;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = fast_exp2(__builtin_fmaf(s[r], c, -lse2));
          if (MASKED && diag && 8 * (r >> 2) + (r & 3) > l32 - 4 * g) p = 0.f;
          // RAG, non-causal: the last tile's keys at or past S (zero rows,
          // whose P = exp2(-lse) need not be finite) take P = 0; causal
          // masking already covers them
          if (RAG && !CAUSAL && LAST && 8 * (r >> 2) + (r & 3) >= S - kvb - 4 * g) p = 0.f;
          dp[r] = p * dp[r];
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int w = 0; w < 4; ++w)
            sb[kb][hh][w] = E::pack2(dp[8 * hh + 2 * w], dp[8 * hh + 2 * w + 1]);
      }
#pragma unroll
      for (int kb = 0; kb < C::TB; ++kb) {
        if (!live[kb]) continue;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int db = 0; db < DBP; ++db) {
            const int off = 2 * (32 * kb + 16 * hh) * D;  // bytes
            acc[db] = E::mfma(tr_operand2(lds_at<uint16_t>(Ks, off + lo.tr(db)),
                                          lds_at<uint16_t>(Ks, off + lo.tr_hi(db))),
                              sb[kb][hh], acc[db]);
          }
        }
      }
    }
    __syncthreads();
  };

  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  int j = 0;
  auto run = [&](int j_end, auto masked_tag) __attribute__((always_inline)) {
    if ((j & 1) && j < j_end) step(j++, masked_tag, std::false_type{}, P1{});
    for (; j + 1 < j_end; j += 2) {
      step(j, masked_tag, std::false_type{}, P0{});
      step(j + 1, masked_tag, std::false_type{}, P1{});
    }
    if (j < j_end) step(j++, masked_tag, std::false_type{}, P0{});
  };
  // nkv >= 1 (kv_end > 0)
  const int n_main = CAUSAL ? max(0, nkv - C::OWN / C::TILE) : nkv;
  run(min(n_main, nkv - 1), std::false_type{});
  if constexpr (CAUSAL) run(nkv - 1, std::true_type{});
  const bool last_masked = CAUSAL && nkv - 1 >= n_main;
  if (last_masked) {
    if (j & 1) step(j, std::true_type{}, std::true_type{}, P1{});
    else step(j, std::true_type{}, std::true_type{}, P0{});
  } else {
    if (j & 1) step(j, std::false_type{}, std::true_type{}, P1{});
    else step(j, std::false_type{}, std::true_type{}, P0{});
  }

  if (!wave_valid) return;
  const int b = it.bh / a.H;
  const int h = it.bh % a.H;
  uint16_t* const dq_rows =
      (uint16_t*)a.dq.ptr + b * a.dq.sb + h * a.dq.sh + (int64_t)qw * a.dq.ss;
  const int nrows = RAG ? min(32, S - qw) : 32;  // queries of this wave below S
  if (ROPE && a.rope.cos)
    store_block_rows_rope<E, D, RAG>(acc, a.scale, wave_stage_buf(bufs, wave), dq_rows, a.dq.ss,
                                a.rope, qw, nrows);
  else
    store_block_rows<E, D, DP>(acc, a.scale, wave_stage_buf(bufs, wave), dq_rows, a.dq.ss,
                               nrows);
}

// One item per workgroup.  One LDS array per buffer and tensor, so that the
// compiler can see that a direct load into one buffer never aliases the
// reads of the other.
template <typename E, int D, bool CAUSAL, bool ROPE, int DP = D, bool RAG = false>
__device__ __forceinline__ void run_item(const AttnArgs& a, const BwdItem it) {
  using C = BwdCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t A0[C::ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t A1[C::ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t B0[C::ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t B1[C::ELEMS];
  __shared__ __attribute__((aligned(16))) float SA[2 * C::TILE];
  __shared__ __attribute__((aligned(16))) float SB[2 * C::TILE];
  const BwdBuf bufs[2] = {{A0, A1, SA}, {B0, B1, SB}};
  if (it.kind)
    dq_item<E, D, CAUSAL, ROPE, DP, RAG>(a, it, bufs);
  else
    dkdv_item<E, D, CAUSAL, ROPE, DP, RAG>(a, it, bufs);
}

// ROPE (every kernel below): the kernel carries the rotating stores, and dQ
// and dK leave inverse-rotated by the tables in a.rope when a.rope.cos is set;
// without it the kernel has no rotation code.
template <typename E, int D, bool CAUSAL, bool ROPE, bool RAG = false>
__global__ __launch_bounds__(256, 2) void attn_bwd_dkdv_kernel(AttnArgs a) {
  // key tile 0 sees the most query tiles: dispatched first
  const int BH = a.B * a.H;
  run_item<E, D, CAUSAL, ROPE, D, RAG>(a, BwdItem{0, (int)(blockIdx.x / BH),
                                                  (int)(blockIdx.x % BH)});
}

template <typename E, int D, bool CAUSAL, bool ROPE, bool RAG = false>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_kernel(AttnArgs a, int n_qtiles) {
  const int BH = a.B * a.H;
  run_item<E, D, CAUSAL, ROPE, D, RAG>(
      a, BwdItem{1, n_qtiles - 1 - (int)(blockIdx.x / BH), (int)(blockIdx.x % BH)});
}

// dK/dV and dQ in one launch.  Workgroups are ordered heaviest-first with the
// two kinds alternating (rank r: kind r & 1; key tile r/2, or query tile
// n_tiles-1-r/2, the tiles that see the most of the sequence under causal
// masking), so the short tails of both kinds overlap the long heads of the
// other and the launch keeps the whole chip busy.  only_kind 0 or 1 runs the
// items of that kind alone (rank r: tile r of it, heaviest first): the D = 64
// separate launches use this kernel, whose compiled item bodies have no
// scratch (standalone instantiations of the dK/dV item spilled 8-28 bytes).
// DP: head columns of the tensors.  Head dims 16 and 32 run in the D = 64
// layout: the padding chunks of the staged tiles and resident rows load as
// zeros, the products over the head dim stop at DP, accumulator blocks past
// DP are not formed and only DP columns are stored (no rotating stores).
// RAG: S not a multiple of 64 (rows past S load as zeros and are not
// stored; padded query rows add exact zeros to dK and dV, padded key rows
// exact zeros to dQ, the non-causal last tile's padded keys take P = 0).
template <typename E, int D, bool CAUSAL, bool ROPE, int DP = D, bool RAG = false>
__global__ __launch_bounds__(256, 2) void attn_bwd_kernel(AttnArgs a, int n_tiles,
                                                          int only_kind) {
  static_assert(DP == D || (D == 64 && !ROPE && (DP == 16 || DP == 32)), "head dim");
  const int BH = a.B * a.H;
  const int rank = blockIdx.x / BH;
  const int kind = only_kind < 0 ? rank & 1 : only_kind;
  const int r = only_kind < 0 ? rank >> 1 : rank;
  run_item<E, D, CAUSAL, ROPE, DP, RAG>(
      a, BwdItem{kind, kind ? n_tiles - 1 - r : r, (int)(blockIdx.x % BH)});
}

template <typename E, int D, bool ROPE, bool RAG = false>
hipError_t launch_dkdv_dr(const AttnArgs& a, hipStream_t st) {
  const int BH = a.B * a.H;
  const int nkt = (a.S + BwdCfg<D>::OWN - 1) / BwdCfg<D>::OWN;
  if (a.causal)
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<E, D, true, ROPE, RAG>), dim3(nkt * BH), dim3(256),
                       0, st, a);
  else
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<E, D, false, ROPE, RAG>), dim3(nkt * BH), dim3(256),
                       0, st, a);
  return hipGetLastError();
}

template <typename E, int D, bool ROPE, bool RAG = false>
hipError_t launch_dq_dr(const AttnArgs& a, hipStream_t st) {
  const int BH = a.B * a.H;
  const int nqt = (a.S + BwdCfg<D>::OWN - 1) / BwdCfg<D>::OWN;
  if (a.causal)
    hipLaunchKernelGGL((attn_bwd_dq_kernel<E, D, true, ROPE, RAG>), dim3(nqt * BH), dim3(256), 0,
                       st, a, nqt);
  else
    hipLaunchKernelGGL((attn_bwd_dq_kernel<E, D, false, ROPE, RAG>), dim3(nqt * BH), dim3(256),
                       0, st, a, nqt);
  return hipGetLastError();
}

// (One instantiation with the rotation applied at run time: compiled without
// the rotating stores, the causal kernel's registers spilled 12 bytes.)
// only_kind: -1 both kinds interleaved, else that kind alone.
// Head dims 16 and 32 (DP < D) have no rotating stores: the host runs their
// inverse RoPE as a separate pass.
template <typename E, int D, bool CAUSAL, int DP = D, bool RAG = false>
hipError_t launch_both_dc(const AttnArgs& a, int only_kind, hipStream_t st) {
  const int BH = a.B * a.H;
  const int n = (a.S + BwdCfg<D>::OWN - 1) / BwdCfg<D>::OWN;
  hipLaunchKernelGGL((attn_bwd_kernel<E, D, CAUSAL, DP == D, DP, RAG>),
                     dim3((only_kind < 0 ? 2 : 1) * n * BH), dim3(256), 0, st, a, n, only_kind);
  return hipGetLastError();
}

template <typename E, int D, int DP = D, bool RAG = false>
hipError_t launch_both_d(const AttnArgs& a, hipStream_t st, int only_kind = -1) {
  return a.causal ? launch_both_dc<E, D, true, DP, RAG>(a, only_kind, st)
                  : launch_both_dc<E, D, false, DP, RAG>(a, only_kind, st);
}

// Head dims 16 and 32: the combined D = 64 kernel with DP columns, restricted
// to one kind (0 or 1) or both (-1).
template <typename E>
hipError_t launch_small_d(const AttnArgs& a, hipStream_t st, int only_kind) {
  if (a.S % 64) {
    if (a.D == 16) return launch_both_d<E, 64, 16, true>(a, st, only_kind);
    return launch_both_d<E, 64, 32, true>(a, st, only_kind);
  }
  if (a.D == 16) return launch_both_d<E, 64, 16>(a, st, only_kind);
  return launch_both_d<E, 64, 32>(a, st, only_kind);
}

// The separate launches: at D = 64 the combined kernel restricted to one kind
// (it rotates only when a.rope.cos is set, which these entry points leave
// unset); at D = 128 the kernels of one kind, rotating when a.rope.cos is set.
template <typename E, int D, bool RAG = false>
hipError_t launch_dkdv_d(const AttnArgs& a, hipStream_t st) {
  if constexpr (D == 64) {
    return launch_both_d<E, D, D, RAG>(a, st, 0);
  } else {
    if (a.rope.cos) return launch_dkdv_dr<E, D, true, RAG>(a, st);
    return launch_dkdv_dr<E, D, false, RAG>(a, st);
  }
}

template <typename E, int D, bool RAG = false>
hipError_t launch_dq_d(const AttnArgs& a, hipStream_t st) {
  if constexpr (D == 64) {
    return launch_both_d<E, D, D, RAG>(a, st, 1);
  } else {
    if (a.rope.cos) return launch_dq_dr<E, D, true, RAG>(a, st);
    return launch_dq_dr<E, D, false, RAG>(a, st);
  }
}

// Sequence lengths that are not a multiple of 64 (head dims 64 and 128) run
// the RAG instantiations.
template <typename E>
hipError_t launch_dkdv_e(const AttnArgs& a, hipStream_t st) {
  if (a.D < 64) return launch_small_d<E>(a, st, 0);
  const bool rag = a.S % 64 != 0;
  if (a.D == 64) return rag ? launch_dkdv_d<E, 64, true>(a, st) : launch_dkdv_d<E, 64>(a, st);
  return rag ? launch_dkdv_d<E, 128, true>(a, st) : launch_dkdv_d<E, 128>(a, st);
}

template <typename E>
hipError_t launch_dq_e(const AttnArgs& a, hipStream_t st) {
  if (a.D < 64) return launch_small_d<E>(a, st, 1);
  const bool rag = a.S % 64 != 0;
  if (a.D == 64) return rag ? launch_dq_d<E, 64, true>(a, st) : launch_dq_d<E, 64>(a, st);
  return rag ? launch_dq_d<E, 128, true>(a, st) : launch_dq_d<E, 128>(a, st);
}

// D = 128: two launches.  Both kinds sit at the 256-register limit of two waves
// per SIMD there, and one combined launch measured 10-15% slower than the two
// (when the dK/dV kind still held K in registers and spilled).
template <typename E>
hipError_t launch_both_e(const AttnArgs& a, hipStream_t st) {
  if (a.D < 64) return launch_small_d<E>(a, st, -1);
  const bool rag = a.S % 64 != 0;
  if (a.D == 64)
    return rag ? launch_both_d<E, 64, 64, true>(a, st) : launch_both_d<E, 64>(a, st);
  hipError_t e = rag ? launch_dkdv_d<E, 128, true>(a, st) : launch_dkdv_d<E, 128>(a, st);
  if (e != hipSuccess) return e;
  return rag ? launch_dq_d<E, 128, true>(a, st) : launch_dq_d<E, 128>(a, st);
}

template <int DT>
hipError_t launch_delta_t(const AttnArgs& a, hipStream_t st) {
  const uint32_t nrows = (uint32_t)a.B * a.H * a.S;
  const FastDiv dS = make_fastdiv(a.S), dH = make_fastdiv(a.H);
  const dim3 grid((uint32_t)(((uint64_t)nrows + 31) / 32));
  constexpr int V16 = (DT == 0) ? 4 : 8;
  if constexpr (DT != 0) {
    auto a16 = [](const TensorArg& t) {
      return ((uintptr_t)t.ptr % 16 == 0) && t.sb % 8 == 0 && t.sh % 8 == 0 && t.ss % 8 == 0;
    };
    // rows per lane: 2 (1536 workgroups at config 2) measured ~0.3 us per step
    // faster than 1, 4 or 8 inside the fwd+bwd sequence
    constexpr int R = 2;
    const dim3 g4((nrows + 32 * R - 1) / (32 * R));
    if (a16(a.o) && a16(a.dout) && (a.D == 64 || a.D == 128)) {
      if (a.D == 64)
        hipLaunchKernelGGL((attn_delta_v16_kernel<DT, 1, R>), g4, dim3(256), 0, st, a, dS, dH, nrows);
      else
        hipLaunchKernelGGL((attn_delta_v16_kernel<DT, 2, R>), g4, dim3(256), 0, st, a, dS, dH, nrows);
      return hipGetLastError();
    }
    // D = 32 and 16: four and two lanes per row (64 and 128 rows per
    // workgroup and pass)
    if (a16(a.o) && a16(a.dout) && (a.D == 32 || a.D == 16)) {
      if (a.D == 32)
        hipLaunchKernelGGL((attn_delta_v16_kernel<DT, 1, R, 4>),
                           dim3((nrows + 64 * R - 1) / (64 * R)), dim3(256), 0, st, a, dS, dH,
                           nrows);
      else
        hipLaunchKernelGGL((attn_delta_v16_kernel<DT, 1, R, 2>),
                           dim3((nrows + 128 * R - 1) / (128 * R)), dim3(256), 0, st, a, dS, dH,
                           nrows);
      return hipGetLastError();
    }
  }
  if (a.D % (8 * V16) == 0)
    hipLaunchKernelGGL((attn_delta_kernel<DT, V16>), grid, dim3(256), 0, st, a, dS, dH, nrows);
  else
    hipLaunchKernelGGL((attn_delta_kernel<DT, 1>), grid, dim3(256), 0, st, a, dS, dH, nrows);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_delta(int dtype, const AttnArgs& a, hipStream_t st) {
  if (dtype == 0) return launch_delta_t<0>(a, st);
  if (dtype == 1) return launch_delta_t<1>(a, st);
  return launch_delta_t<2>(a, st);
}

hipError_t launch_attn_bwd_dkdv_mfma(int dtype, const AttnArgs& a, hipStream_t st) {
  if (dtype == 2) return launch_dkdv_e<BF16>(a, st);
  return launch_dkdv_e<F16>(a, st);
}

hipError_t launch_attn_bwd_dq_mfma(int dtype, const AttnArgs& a, hipStream_t st) {
  if (dtype == 2) return launch_dq_e<BF16>(a, st);
  return launch_dq_e<F16>(a, st);
}

hipError_t launch_attn_bwd_mfma(int dtype, const AttnArgs& a, hipStream_t st) {
  if (dtype == 2) return launch_both_e<BF16>(a, st);
  return launch_both_e<F16>(a, st);
}

}  // namespace mi
