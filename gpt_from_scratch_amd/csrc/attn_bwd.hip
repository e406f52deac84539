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
#include <type_traits>

#include "mi_device.h"
#include "mi_kernels.h"

namespace mi {

namespace {

// ---------------------------------------------------------------------------
// delta[b,h,s] = sum_d dO[b,h,s,d] * O[b,h,s,d]   (fp32 accumulation)
// Eight lanes per row; each lane takes every 8th chunk of VEC elements.
// ---------------------------------------------------------------------------
template <int DT, int VEC>
__global__ __launch_bounds__(256) void attn_delta_kernel(AttnArgs a, FastDiv divS, FastDiv divH,
                                                         uint32_t nrows) {
  typedef typename Store<DT>::type T;
  const uint32_t t = blockIdx.x * 256 + threadIdx.x;
  const uint32_t row = t >> 3;
  const int sub = t & 7;
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
  if (row < nrows && sub == 0) a.delta[row] = acc;
}

// ---------------------------------------------------------------------------
// Work items.  The gradients are produced by items of two kinds:
//   kind 0 (dK/dV, `_attn_bwd_LoopQ`): OWN keys of one head; the item loops
//          over query tiles, with K and V rows of its keys in registers;
//   kind 1 (dQ, `_attn_bwd_LoopKV`):   OWN queries of one head; the item loops
//          over key tiles, with Q and dO rows of its queries in registers.
// Both stream TILE-row tiles of the other two tensors through LDS (double
// buffered) and keep the same register layout: two resident row sets (B
// operands) and one staged tile, so one launch can run both kinds.
// ---------------------------------------------------------------------------
template <int D>
struct BwdCfg {
  static constexpr int OWN = 128;                   // rows owned by an item
  static constexpr int TILE = (D == 64) ? 64 : 32;  // rows of a streamed tile
  static constexpr int NT = 256;
  static constexpr int RLD = D + 8;  // row stride of the row-major LDS tiles (elements)
  static constexpr int KS = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int TB = TILE / 32;  // 32-row blocks per streamed tile
  static constexpr int CG = D / 4;      // loader column groups (4 columns each)
  static constexpr int RG = TILE / 4;   // loader row groups (4 rows each)
  static_assert(CG * RG == NT, "loader covers the tile with 4x4 blocks");
  static constexpr int BUF = 2 * TILE * RLD;  // uint16 per LDS buffer: both streamed tensors
  // two buffers, then lse*log2e and -delta of each buffer's query rows (dK/dV kind)
  static constexpr int LDS_BYTES = 2 * BUF * 2 + 2 * 2 * TILE * 4;
};

struct BwdItem {
  int kind;  // 0: dK/dV, 1: dQ
  int tile;  // key tile (kind 0) or query tile (kind 1), OWN rows each
  int bh;
};

template <int D>
struct Resident {
  u32x4 r[2][D / 16];  // kind 0: K, V rows; kind 1: Q, dO rows (lane: row l%32, 8 columns)
  float lse2, dl;      // kind 1: lse*log2e and delta of this lane's query row
};

struct Staged {
  u32x2 t[2][4];  // one streamed tile: 4 rows x 4 columns of each tensor per thread
  float s0, s1;   // kind 0: lse*log2e and -delta of query row `tid` (tid < TILE)
};

// Where an item's streamed tiles come from: head bases, strides and this
// thread's fixed byte offset inside a tile (buffer loads, so that advancing
// a tile is scalar arithmetic).
struct StageSrc {
  const uint16_t* p0;
  const uint16_t* p1;
  int64_t ss0, ss1;
  uint32_t off0, off1;
  const float* lse;
  const float* delta;
};

__device__ __forceinline__ const uint16_t* head_ptr(const TensorArg& t, int b, int h) {
  return (const uint16_t*)t.ptr + b * t.sb + h * t.sh;
}

template <int D, bool CAUSAL>
__device__ __forceinline__ int first_row(const BwdItem& it) {
  return (CAUSAL && it.kind == 0) ? it.tile * BwdCfg<D>::OWN : 0;
}

template <int D>
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
    const auto r0 = tile_rsrc(head_ptr(t0, b, h) + (int64_t)w0 * t0.ss);
    const auto r1 = tile_rsrc(head_ptr(t1, b, h) + (int64_t)w0 * t1.ss);
    const uint32_t o0 = (uint32_t)(((lane & 31) * t0.ss + 8 * (lane >> 5)) * 2);
    const uint32_t o1 = (uint32_t)(((lane & 31) * t1.ss + 8 * (lane >> 5)) * 2);
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      res.r[0][ks] = __builtin_amdgcn_raw_buffer_load_b128(r0, o0 + 32 * ks, 0, 0);
      res.r[1][ks] = __builtin_amdgcn_raw_buffer_load_b128(r1, o1 + 32 * ks, 0, 0);
    }
    if (it.kind) {
      const int64_t o = (int64_t)it.bh * a.S + w0;
      res.lse2 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                     tile_rsrc(a.lse + o), (lane & 31) * 4, 0, 0)) * kLog2e;
      res.dl = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                   tile_rsrc(a.delta + o), (lane & 31) * 4, 0, 0));
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

template <int D>
__device__ __forceinline__ StageSrc stage_src(const AttnArgs& a, const BwdItem& it) {
  using C = BwdCfg<D>;
  const int tid = threadIdx.x;
  const int rg = tid / C::CG;
  const int cg = tid % C::CG;
  const int b = it.bh / a.H;
  const int h = it.bh % a.H;
  const TensorArg& t0 = it.kind ? a.k : a.q;
  const TensorArg& t1 = it.kind ? a.v : a.dout;
  StageSrc s;
  s.p0 = head_ptr(t0, b, h);
  s.p1 = head_ptr(t1, b, h);
  s.ss0 = t0.ss;
  s.ss1 = t1.ss;
  s.off0 = (uint32_t)((4 * rg * t0.ss + 4 * cg) * 2);
  s.off1 = (uint32_t)((4 * rg * t1.ss + 4 * cg) * 2);
  s.lse = a.lse + (int64_t)it.bh * a.S;
  s.delta = a.delta + (int64_t)it.bh * a.S;
  return s;
}

// Streamed tile starting at row `row0` into registers.
template <int D>
__device__ __forceinline__ void load_stage(const StageSrc& s, int kind, int row0, Staged& st) {
  const auto r0 = tile_rsrc(s.p0 + (int64_t)row0 * s.ss0);
  const auto r1 = tile_rsrc(s.p1 + (int64_t)row0 * s.ss1);
  const uint32_t rb0 = (uint32_t)(s.ss0 * 2), rb1 = (uint32_t)(s.ss1 * 2);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    st.t[0][r] = __builtin_amdgcn_raw_buffer_load_b64(r0, s.off0, r * rb0, 0);
    st.t[1][r] = __builtin_amdgcn_raw_buffer_load_b64(r1, s.off1, r * rb1, 0);
  }
  const int tid = threadIdx.x;
  if (kind == 0 && tid < BwdCfg<D>::TILE) {
    const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b32(tile_rsrc(s.lse + row0), tid * 4, 0, 0);
    const uint32_t dl = __builtin_amdgcn_raw_buffer_load_b32(tile_rsrc(s.delta + row0), tid * 4, 0, 0);
    st.s0 = __builtin_bit_cast(float, lo) * kLog2e;
    st.s1 = -__builtin_bit_cast(float, dl);  // dP accumulators start at -delta
  }
}

// Staged tile into one LDS buffer (row-major, both tensors) and, for the
// dK/dV kind, its query rows' lse and -delta.
template <int D>
__device__ __forceinline__ void store_stage(const Staged& st, int kind, uint16_t* buf, float* slb) {
  using C = BwdCfg<D>;
  const int tid = threadIdx.x;
  const int rg = tid / C::CG;
  const int cg = tid % C::CG;
  uint16_t* t1 = buf + C::TILE * C::RLD;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    *(u32x2*)(&buf[(4 * rg + r) * C::RLD + 4 * cg]) = st.t[0][r];
    *(u32x2*)(&t1[(4 * rg + r) * C::RLD + 4 * cg]) = st.t[1][r];
  }
  if (kind == 0 && tid < C::TILE) {
    slb[tid] = st.s0;
    slb[C::TILE + tid] = st.s1;
  }
}

// ---------------------------------------------------------------------------
// dK / dV item.  Wave w owns keys [kv0 + 32w, +32).  S = Q K^T and
// dP = dO V^T are computed with keys along the lane index, so P and dS leave
// the accumulators in B-operand form for dV^T = dO^T P and dK^T = Q^T dS; the
// dO^T and Q^T A operands are read transposed from the row-major tiles.
// `stg` holds the item's first query tile on entry.
// ---------------------------------------------------------------------------
template <typename E, int D, bool CAUSAL>
__device__ __forceinline__ void dkdv_item(const AttnArgs& a, const BwdItem& it,
                                          const Resident<D>& res, Staged& stg,
                                          uint16_t (*smem)[BwdCfg<D>::BUF],
                                          float (*sl)[2 * BwdCfg<D>::TILE]) {
  using C = BwdCfg<D>;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int S = a.S;

  const int kv0 = it.tile * C::OWN;
  const int kw = kv0 + 32 * wave;
  const bool wave_valid = kw < S;
  const int krow = kw + l32;
  const int tro = tr_lane_offset(lane, C::RLD);
  const u32x4(&kf)[C::KS] = res.r[0];
  const u32x4(&vf)[C::KS] = res.r[1];

  const int q_begin = first_row<D, CAUSAL>(it);
  const int nq = (S - q_begin) / C::TILE;
  const StageSrc src = stage_src<D>(a, it);

  f32x16 dk[C::DB], dv[C::DB];
#pragma unroll
  for (int i = 0; i < C::DB; ++i) {
    dk[i] = f32x16{};
    dv[i] = f32x16{};
  }
  const float c = a.scale_log2;

  store_stage<D>(stg, 0, smem[0], sl[0]);
  __syncthreads();

  // Query tile j.  MASKED steps are the ones that straddle this item's keys
  // (causal only): there a 32-row block entirely before a wave's keys is
  // skipped and the block on the wave's diagonal (qbs == kw, everything is
  // 32-aligned) is masked with the fixed triangle key > query.  All later
  // tiles see every key of the item and run the branch-free body.
  auto step = [&](int j, auto masked_tag, auto last_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool LAST = decltype(last_tag)::value;
    const int buf = j & 1;
    const int q0 = q_begin + j * C::TILE;
    if (!LAST) load_stage<D>(src, 0, q0 + C::TILE, stg);

    const bool active = wave_valid && (!MASKED || q0 + C::TILE - 1 >= kw);
    const uint16_t* Qs = smem[buf];
    const uint16_t* dOs = Qs + C::TILE * C::RLD;
    u32x4 pb[C::TB][2], sb[C::TB][2];
    bool live[C::TB];
    if (active) {
#pragma unroll
      for (int qb = 0; qb < C::TB; ++qb) {
        const int qbs = q0 + 32 * qb;
        live[qb] = !MASKED || (qbs + 31 >= kw);
        if (!live[qb]) continue;
        // dP starts at -delta (row = query), so the MFMAs leave dP - delta.
        f32x16 s = f32x16{}, dp;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const f32x4 d4 = *(const f32x4*)(&sl[buf][C::TILE + 32 * qb + 8 * jj + 4 * g]);
#pragma unroll
          for (int i = 0; i < 4; ++i) dp[4 * jj + i] = d4[i];
        }
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) {
          const u32x4 qa = *(const u32x4*)(&Qs[(32 * qb + l32) * C::RLD + 16 * ks + 8 * g]);
          s = E::mfma(qa, kf[ks], s);
        }
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) {
          const u32x4 da = *(const u32x4*)(&dOs[(32 * qb + l32) * C::RLD + 16 * ks + 8 * g]);
          dp = E::mfma(da, vf[ks], dp);
        }
        const bool diag = MASKED && qbs == kw;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const f32x4 l4 = *(const f32x4*)(&sl[buf][32 * qb + 8 * jj + 4 * g]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 4 * jj + i;
            float p = fast_exp2(__builtin_fmaf(s[r], c, -l4[i]));
            if (MASKED && diag && l32 > 8 * jj + 4 * g + i) p = 0.f;
            s[r] = p;
            dp[r] = p * dp[r];
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
    }
    if (active) {
#pragma unroll
      for (int qb = 0; qb < C::TB; ++qb) {
        if (!live[qb]) continue;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int db = 0; db < C::DB; ++db) {
            const int off = (32 * qb + 16 * hh) * C::RLD + 32 * db + tro;
            dv[db] = E::mfma(tr_operand(&dOs[off], C::RLD), pb[qb][hh], dv[db]);
            dk[db] = E::mfma(tr_operand(&Qs[off], C::RLD), sb[qb][hh], dk[db]);
          }
        }
      }
    }

    if (!LAST) store_stage<D>(stg, 0, smem[buf ^ 1], sl[buf ^ 1]);
    __syncthreads();
  };

  // nq >= 1: the matrix-core path needs S % 64 == 0.
  const int n_diag = CAUSAL ? min(nq, C::OWN / C::TILE) : 0;
  int j = 0;
  if constexpr (CAUSAL)
    for (; j < n_diag && j + 1 < nq; ++j) step(j, std::true_type{}, std::false_type{});
  for (; j + 1 < nq; ++j) step(j, std::false_type{}, std::false_type{});
  if (CAUSAL && j < n_diag)
    step(j, std::true_type{}, std::true_type{});
  else
    step(j, std::false_type{}, std::true_type{});

  if (!wave_valid) return;
  const int b = it.bh / a.H;
  const int h = it.bh % a.H;
  uint16_t* dkrow = (uint16_t*)a.dk.ptr + b * a.dk.sb + h * a.dk.sh + (int64_t)krow * a.dk.ss;
  uint16_t* dvrow = (uint16_t*)a.dv.ptr + b * a.dv.sb + h * a.dv.sh + (int64_t)krow * a.dv.ss;
  const float sc = a.scale;
#pragma unroll
  for (int db = 0; db < C::DB; ++db) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      u32x2 wk, wv;
      wk[0] = E::pack2(dk[db][4 * jj + 0] * sc, dk[db][4 * jj + 1] * sc);
      wk[1] = E::pack2(dk[db][4 * jj + 2] * sc, dk[db][4 * jj + 3] * sc);
      wv[0] = E::pack2(dv[db][4 * jj + 0], dv[db][4 * jj + 1]);
      wv[1] = E::pack2(dv[db][4 * jj + 2], dv[db][4 * jj + 3]);
      *(u32x2*)(dkrow + 32 * db + 8 * jj + 4 * g) = wk;
      *(u32x2*)(dvrow + 32 * db + 8 * jj + 4 * g) = wv;
    }
  }
}

// ---------------------------------------------------------------------------
// dQ item.  Wave w owns queries [q0 + 32w, +32).  S^T = K Q^T and
// dP^T = V dO^T put queries along the lane index, so lse and delta are
// per-lane scalars and dS^T feeds dQ^T = K^T dS^T directly (K^T read
// transposed from the row-major K tile).
// ---------------------------------------------------------------------------
template <typename E, int D, bool CAUSAL>
__device__ __forceinline__ void dq_item(const AttnArgs& a, const BwdItem& it,
                                        const Resident<D>& res, Staged& stg,
                                        uint16_t (*smem)[BwdCfg<D>::BUF]) {
  using C = BwdCfg<D>;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int S = a.S;

  const int q0 = it.tile * C::OWN;
  const int qw = q0 + 32 * wave;
  const bool wave_valid = qw < S;
  const int qrow = qw + l32;
  const int tro = tr_lane_offset(lane, C::RLD);
  const u32x4(&qf)[C::KS] = res.r[0];
  const u32x4(&df)[C::KS] = res.r[1];
  const float lse2 = res.lse2;
  const float dl = res.dl;

  const int kv_end = CAUSAL ? min(q0 + C::OWN, S) : S;
  const int nkv = kv_end / C::TILE;
  const StageSrc src = stage_src<D>(a, it);

  f32x16 acc[C::DB];
#pragma unroll
  for (int i = 0; i < C::DB; ++i) acc[i] = f32x16{};
  const float c = a.scale_log2;

  store_stage<D>(stg, 1, smem[0], nullptr);
  __syncthreads();

  // Key tile j.  MASKED steps are the causal ones that straddle this item's
  // queries: a 32-key block after a wave's queries is skipped and the block on
  // the wave's diagonal (kvb == qw) gets the fixed triangle mask.  Earlier
  // tiles are visible to every query and run the branch-free body.
  auto step = [&](int j, auto masked_tag, auto last_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool LAST = decltype(last_tag)::value;
    const int buf = j & 1;
    const int kv0 = j * C::TILE;
    if (!LAST) load_stage<D>(src, 1, kv0 + C::TILE, stg);

    const bool active = wave_valid && (!MASKED || kv0 <= qw + 31);
    const uint16_t* Ks = smem[buf];
    const uint16_t* Vs = Ks + C::TILE * C::RLD;
    u32x4 sb[C::TB][2];
    bool live[C::TB];
    if (active) {
#pragma unroll
      for (int kb = 0; kb < C::TB; ++kb) {
        const int kvb = kv0 + 32 * kb;
        live[kb] = !MASKED || (kvb <= qw + 31);
        if (!live[kb]) continue;
        f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) {
          const u32x4 ka = *(const u32x4*)(&Ks[(32 * kb + l32) * C::RLD + 16 * ks + 8 * g]);
          s = E::mfma(ka, qf[ks], s);
        }
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) {
          const u32x4 va = *(const u32x4*)(&Vs[(32 * kb + l32) * C::RLD + 16 * ks + 8 * g]);
          dp = E::mfma(va, df[ks], dp);
        }
        const bool diag = MASKED && kvb == qw;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = fast_exp2(__builtin_fmaf(s[r], c, -lse2));
          if (MASKED && diag && 8 * (r >> 2) + 4 * g + (r & 3) > l32) p = 0.f;
          dp[r] = p * (dp[r] - dl);
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int w = 0; w < 4; ++w)
            sb[kb][hh][w] = E::pack2(dp[8 * hh + 2 * w], dp[8 * hh + 2 * w + 1]);
      }
    }
    if (active) {
#pragma unroll
      for (int kb = 0; kb < C::TB; ++kb) {
        if (!live[kb]) continue;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int db = 0; db < C::DB; ++db) {
            const int off = (32 * kb + 16 * hh) * C::RLD + 32 * db + tro;
            acc[db] = E::mfma(tr_operand(&Ks[off], C::RLD), sb[kb][hh], acc[db]);
          }
        }
      }
    }

    if (!LAST) store_stage<D>(stg, 1, smem[buf ^ 1], nullptr);
    __syncthreads();
  };

  // nkv >= 1: the matrix-core path needs S % 64 == 0.
  const int n_main = CAUSAL ? max(0, nkv - C::OWN / C::TILE) : nkv;
  int j = 0;
  for (; j < n_main && j + 1 < nkv; ++j) step(j, std::false_type{}, std::false_type{});
  if constexpr (CAUSAL)
    for (; j + 1 < nkv; ++j) step(j, std::true_type{}, std::false_type{});
  if (!CAUSAL || j < n_main)
    step(j, std::false_type{}, std::true_type{});
  else
    step(j, std::true_type{}, std::true_type{});

  if (!wave_valid) return;
  const int b = it.bh / a.H;
  const int h = it.bh % a.H;
  uint16_t* dqrow = (uint16_t*)a.dq.ptr + b * a.dq.sb + h * a.dq.sh + (int64_t)qrow * a.dq.ss;
  const float sc = a.scale;
#pragma unroll
  for (int db = 0; db < C::DB; ++db) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      u32x2 w;
      w[0] = E::pack2(acc[db][4 * jj + 0] * sc, acc[db][4 * jj + 1] * sc);
      w[1] = E::pack2(acc[db][4 * jj + 2] * sc, acc[db][4 * jj + 3] * sc);
      *(u32x2*)(dqrow + 32 * db + 8 * jj + 4 * g) = w;
    }
  }
}

// One item per workgroup.
template <typename E, int D, bool CAUSAL>
__device__ __forceinline__ void run_item(const AttnArgs& a, const BwdItem it) {
  using C = BwdCfg<D>;
  __shared__ __attribute__((aligned(16))) unsigned char lds[C::LDS_BYTES];
  auto smem = (uint16_t(*)[C::BUF])lds;
  auto sl = (float(*)[2 * C::TILE])(lds + 2 * C::BUF * 2);
  Resident<D> res;
  Staged stg;
  load_resident<D>(a, it, res);
  load_stage<D>(stage_src<D>(a, it), it.kind, first_row<D, CAUSAL>(it), stg);
  if (it.kind)
    dq_item<E, D, CAUSAL>(a, it, res, stg, smem);
  else
    dkdv_item<E, D, CAUSAL>(a, it, res, stg, smem, sl);
}

template <typename E, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(AttnArgs a) {
  // key tile 0 sees the most query tiles: dispatched first
  const int BH = a.B * a.H;
  run_item<E, D, CAUSAL>(a, BwdItem{0, (int)(blockIdx.x / BH), (int)(blockIdx.x % BH)});
}

template <typename E, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnArgs a, int n_qtiles) {
  const int BH = a.B * a.H;
  run_item<E, D, CAUSAL>(
      a, BwdItem{1, n_qtiles - 1 - (int)(blockIdx.x / BH), (int)(blockIdx.x % BH)});
}

// dK/dV and dQ in one launch.  Workgroups are ordered heaviest-first with the
// two kinds alternating (rank r: kind r & 1; key tile r/2, or query tile
// n_tiles-1-r/2, the tiles that see the most of the sequence under causal
// masking), so the short tails of both kinds overlap the long heads of the
// other and the launch keeps the whole chip busy.
template <typename E, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_kernel(AttnArgs a, int n_tiles) {
  const int BH = a.B * a.H;
  const int rank = blockIdx.x / BH;
  const int kind = rank & 1;
  run_item<E, D, CAUSAL>(
      a, BwdItem{kind, kind ? n_tiles - 1 - (rank >> 1) : (rank >> 1), (int)(blockIdx.x % BH)});
}

template <typename E, int D>
hipError_t launch_dkdv_d(const AttnArgs& a, hipStream_t st) {
  const int BH = a.B * a.H;
  const int nkt = (a.S + BwdCfg<D>::OWN - 1) / BwdCfg<D>::OWN;
  if (a.causal)
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<E, D, true>), dim3(nkt * BH), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<E, D, false>), dim3(nkt * BH), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <typename E, int D>
hipError_t launch_dq_d(const AttnArgs& a, hipStream_t st) {
  const int BH = a.B * a.H;
  const int nqt = (a.S + BwdCfg<D>::OWN - 1) / BwdCfg<D>::OWN;
  if (a.causal)
    hipLaunchKernelGGL((attn_bwd_dq_kernel<E, D, true>), dim3(nqt * BH), dim3(256), 0, st, a, nqt);
  else
    hipLaunchKernelGGL((attn_bwd_dq_kernel<E, D, false>), dim3(nqt * BH), dim3(256), 0, st, a, nqt);
  return hipGetLastError();
}

template <typename E, int D, bool CAUSAL>
hipError_t launch_both_dc(const AttnArgs& a, hipStream_t st) {
  const int BH = a.B * a.H;
  const int n = (a.S + BwdCfg<D>::OWN - 1) / BwdCfg<D>::OWN;
  hipLaunchKernelGGL((attn_bwd_kernel<E, D, CAUSAL>), dim3(2 * n * BH), dim3(256), 0, st, a, n);
  return hipGetLastError();
}

template <typename E, int D>
hipError_t launch_both_d(const AttnArgs& a, hipStream_t st) {
  return a.causal ? launch_both_dc<E, D, true>(a, st) : launch_both_dc<E, D, false>(a, st);
}

template <typename E>
hipError_t launch_dkdv_e(const AttnArgs& a, hipStream_t st) {
  if (a.D == 64) return launch_dkdv_d<E, 64>(a, st);
  return launch_dkdv_d<E, 128>(a, st);
}

template <typename E>
hipError_t launch_dq_e(const AttnArgs& a, hipStream_t st) {
  if (a.D == 64) return launch_dq_d<E, 64>(a, st);
  return launch_dq_d<E, 128>(a, st);
}

// D = 128: the two kinds need different register budgets (the dK/dV kind
// alone runs at 1 wave/SIMD), so they stay separate launches.
template <typename E>
hipError_t launch_both_e(const AttnArgs& a, hipStream_t st) {
  if (a.D == 64) return launch_both_d<E, 64>(a, st);
  hipError_t e = launch_dkdv_d<E, 128>(a, st);
  if (e != hipSuccess) return e;
  return launch_dq_d<E, 128>(a, st);
}

template <int DT>
hipError_t launch_delta_t(const AttnArgs& a, hipStream_t st) {
  const uint32_t nrows = (uint32_t)a.B * a.H * a.S;
  const FastDiv dS = make_fastdiv(a.S), dH = make_fastdiv(a.H);
  const dim3 grid((nrows * 8 + 255) / 256);
  constexpr int V16 = (DT == 0) ? 4 : 8;
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
