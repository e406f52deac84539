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
// dK / dV
// ---------------------------------------------------------------------------
template <int D>
struct DkvCfg {
  static constexpr int BKV = 128;
  static constexpr int BQ = (D == 64) ? 64 : 32;
  static constexpr int NT = 256;
  static constexpr int RLD = D + 8;   // row-major Q / dO tile stride (elements)
  static constexpr int KS = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int QB = BQ / 32;
  static constexpr int CG = D / 4;    // loader column groups (4 columns each)
  static constexpr int RG = BQ / 4;   // loader row groups (4 rows each)
  static_assert(CG * RG == NT, "loader covers the tile with 4x4 blocks");
  static constexpr int BUF = 2 * BQ * RLD;  // uint16 per buffer: Q and dO tiles
};

// One key tile `kt` of head `bh`.  smem: 2 staging buffers; sl: lse*log2e and
// delta of the staged query tiles.
template <typename E, int D, bool CAUSAL>
__device__ __forceinline__ void dkdv_body(const AttnArgs& a, const int kt, const int bh,
                                          uint16_t (*smem)[DkvCfg<D>::BUF],
                                          float (*sl)[2 * DkvCfg<D>::BQ]) {
  using C = DkvCfg<D>;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31;
  const int g = lane >> 5;

  const int b = bh / a.H;
  const int h = bh % a.H;
  const int S = a.S;

  const uint16_t* qp = (const uint16_t*)a.q.ptr + b * a.q.sb + h * a.q.sh;
  const uint16_t* kp = (const uint16_t*)a.k.ptr + b * a.k.sb + h * a.k.sh;
  const uint16_t* vp = (const uint16_t*)a.v.ptr + b * a.v.sb + h * a.v.sh;
  const uint16_t* dop = (const uint16_t*)a.dout.ptr + b * a.dout.sb + h * a.dout.sh;
  const float* lsep = a.lse + (int64_t)bh * S;
  const float* delp = a.delta + (int64_t)bh * S;

  const int kv0 = kt * C::BKV;
  const int kw = kv0 + 32 * wave;
  const bool wave_valid = kw < S;
  const int krow = kw + l32;
  const int tro = tr_lane_offset(lane, C::RLD);

  u32x4 kf[C::KS], vf[C::KS];
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) {
    if (wave_valid) {
      kf[ks] = *(const u32x4*)(kp + (int64_t)krow * a.k.ss + 16 * ks + 8 * g);
      vf[ks] = *(const u32x4*)(vp + (int64_t)krow * a.v.ss + 16 * ks + 8 * g);
    } else {
      kf[ks] = u32x4{0, 0, 0, 0};
      vf[ks] = u32x4{0, 0, 0, 0};
    }
  }

  const int q_begin = CAUSAL ? kv0 : 0;
  const int nq = (S - q_begin) / C::BQ;

  // staging registers
  const int rg = tid / C::CG;
  const int cg = tid % C::CG;
  u32x2 qreg[4], dreg[4];
  float lreg = 0.f, dlreg = 0.f;

  // Buffer loads: one descriptor per tile, a fixed per-lane byte offset and
  // the row step as a scalar offset, so no per-lane address arithmetic.
  const uint32_t qoff = (uint32_t)((4 * rg * a.q.ss + 4 * cg) * 2);
  const uint32_t doff = (uint32_t)((4 * rg * a.dout.ss + 4 * cg) * 2);
  const uint32_t qrow_b = (uint32_t)(a.q.ss * 2), drow_b = (uint32_t)(a.dout.ss * 2);
  auto load_tile = [&](int q0) {
    const auto rq = tile_rsrc(qp + (int64_t)q0 * a.q.ss);
    const auto rd = tile_rsrc(dop + (int64_t)q0 * a.dout.ss);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      qreg[r] = __builtin_amdgcn_raw_buffer_load_b64(rq, qoff, r * qrow_b, 0);
      dreg[r] = __builtin_amdgcn_raw_buffer_load_b64(rd, doff, r * drow_b, 0);
    }
    if (tid < C::BQ) {
      const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b32(tile_rsrc(lsep + q0), tid * 4, 0, 0);
      const uint32_t dl = __builtin_amdgcn_raw_buffer_load_b32(tile_rsrc(delp + q0), tid * 4, 0, 0);
      lreg = __builtin_bit_cast(float, lo) * kLog2e;
      dlreg = -__builtin_bit_cast(float, dl);  // dP accumulators start at -delta
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* Qs = smem[buf];
    uint16_t* dOs = Qs + C::BQ * C::RLD;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      *(u32x2*)(&Qs[(4 * rg + r) * C::RLD + 4 * cg]) = qreg[r];
      *(u32x2*)(&dOs[(4 * rg + r) * C::RLD + 4 * cg]) = dreg[r];
    }
    if (tid < C::BQ) {
      sl[buf][tid] = lreg;
      sl[buf][C::BQ + tid] = dlreg;
    }
  };

  f32x16 dk[C::DB], dv[C::DB];
#pragma unroll
  for (int i = 0; i < C::DB; ++i) {
    dk[i] = f32x16{};
    dv[i] = f32x16{};
  }
  const float c = a.scale_log2;

  if (nq > 0) {
    load_tile(q_begin);
    store_tile(0);
  }
  __syncthreads();

  // Query tile j.  MASKED steps are the ones that straddle this workgroup's
  // keys (causal only): there a 32-row block entirely before a wave's keys is
  // skipped and the block on the wave's diagonal (qbs == kw, everything is
  // 32-aligned) is masked with the fixed triangle key > query.  All later
  // tiles see every key of the workgroup and run the branch-free body.
  auto step = [&](int j, auto masked_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    const int buf = j & 1;
    const int q0 = q_begin + j * C::BQ;
    if (j + 1 < nq) load_tile(q0 + C::BQ);

    if (wave_valid && (!MASKED || q0 + C::BQ - 1 >= kw)) {
      const uint16_t* Qs = smem[buf];
      const uint16_t* dOs = Qs + C::BQ * C::RLD;
      u32x4 pb[C::QB][2], sb[C::QB][2];
      bool live[C::QB];
#pragma unroll
      for (int qb = 0; qb < C::QB; ++qb) {
        const int qbs = q0 + 32 * qb;
        live[qb] = !MASKED || (qbs + 31 >= kw);
        if (!live[qb]) continue;
        // dP starts at -delta (row = query), so the MFMAs leave dP - delta.
        f32x16 s = f32x16{}, dp;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const f32x4 d4 = *(const f32x4*)(&sl[buf][C::BQ + 32 * qb + 8 * jj + 4 * g]);
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
#pragma unroll
      for (int qb = 0; qb < C::QB; ++qb) {
        if (!live[qb]) continue;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int db = 0; db < C::DB; ++db) {
            // dO^T and Q^T operands read transposed from the row-major tiles.
            const int off = (32 * qb + 16 * hh) * C::RLD + 32 * db + tro;
            dv[db] = E::mfma(tr_operand(&dOs[off], C::RLD), pb[qb][hh], dv[db]);
            dk[db] = E::mfma(tr_operand(&Qs[off], C::RLD), sb[qb][hh], dk[db]);
          }
        }
      }
    }

    if (j + 1 < nq) store_tile(buf ^ 1);
    __syncthreads();
  };

  const int n_diag = CAUSAL ? min(nq, C::BKV / C::BQ) : 0;
  int j = 0;
  if constexpr (CAUSAL)
    for (; j < n_diag; ++j) step(j, std::true_type{});
  for (; j < nq; ++j) step(j, std::false_type{});

  if (!wave_valid) return;
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
// dQ
// ---------------------------------------------------------------------------
template <int D>
struct DqCfg {
  static constexpr int BQ = 128;
  static constexpr int BKV = (D == 64) ? 64 : 32;
  static constexpr int NKB = BKV / 32;
  static constexpr int NT = 256;
  static constexpr int RLD = D + 8;    // row-major K / V tile stride
  static constexpr int KS = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int CG = D / 4;
  static constexpr int RG = BKV / 4;
  static_assert(CG * RG == NT, "loader covers the tile with 4x4 blocks");
  static constexpr int BUF = 2 * BKV * RLD;  // uint16 per buffer: K and V tiles
};

// One query tile `qt` of head `bh`.  smem: 2 staging buffers.
template <typename E, int D, bool CAUSAL>
__device__ __forceinline__ void dq_body(const AttnArgs& a, const int qt, const int bh,
                                        uint16_t (*smem)[DqCfg<D>::BUF]) {
  using C = DqCfg<D>;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31;
  const int g = lane >> 5;

  const int b = bh / a.H;
  const int h = bh % a.H;
  const int S = a.S;

  const uint16_t* qp = (const uint16_t*)a.q.ptr + b * a.q.sb + h * a.q.sh;
  const uint16_t* kp = (const uint16_t*)a.k.ptr + b * a.k.sb + h * a.k.sh;
  const uint16_t* vp = (const uint16_t*)a.v.ptr + b * a.v.sb + h * a.v.sh;
  const uint16_t* dop = (const uint16_t*)a.dout.ptr + b * a.dout.sb + h * a.dout.sh;

  const int q0 = qt * C::BQ;
  const int qw = q0 + 32 * wave;
  const bool wave_valid = qw < S;
  const int qrow = qw + l32;
  const int tro = tr_lane_offset(lane, C::RLD);

  u32x4 qf[C::KS], df[C::KS];
  float lse2 = 0.f, dl = 0.f;
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) {
    if (wave_valid) {
      qf[ks] = *(const u32x4*)(qp + (int64_t)qrow * a.q.ss + 16 * ks + 8 * g);
      df[ks] = *(const u32x4*)(dop + (int64_t)qrow * a.dout.ss + 16 * ks + 8 * g);
    } else {
      qf[ks] = u32x4{0, 0, 0, 0};
      df[ks] = u32x4{0, 0, 0, 0};
    }
  }
  if (wave_valid) {
    lse2 = a.lse[(int64_t)bh * S + qrow] * kLog2e;
    dl = a.delta[(int64_t)bh * S + qrow];
  }

  const int kv_end = CAUSAL ? min(q0 + C::BQ, S) : S;
  const int nkv = kv_end / C::BKV;

  const int rg = tid / C::CG;
  const int cg = tid % C::CG;
  u32x2 kreg[4], vreg[4];

  const uint32_t koff = (uint32_t)((4 * rg * a.k.ss + 4 * cg) * 2);
  const uint32_t voff = (uint32_t)((4 * rg * a.v.ss + 4 * cg) * 2);
  const uint32_t krow_b = (uint32_t)(a.k.ss * 2), vrow_b = (uint32_t)(a.v.ss * 2);
  auto load_tile = [&](int kv0) {
    const auto rk = tile_rsrc(kp + (int64_t)kv0 * a.k.ss);
    const auto rv = tile_rsrc(vp + (int64_t)kv0 * a.v.ss);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      kreg[r] = __builtin_amdgcn_raw_buffer_load_b64(rk, koff, r * krow_b, 0);
      vreg[r] = __builtin_amdgcn_raw_buffer_load_b64(rv, voff, r * vrow_b, 0);
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* Ks = smem[buf];
    uint16_t* Vs = Ks + C::BKV * C::RLD;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      *(u32x2*)(&Ks[(4 * rg + r) * C::RLD + 4 * cg]) = kreg[r];
      *(u32x2*)(&Vs[(4 * rg + r) * C::RLD + 4 * cg]) = vreg[r];
    }
  };

  f32x16 acc[C::DB];
#pragma unroll
  for (int i = 0; i < C::DB; ++i) acc[i] = f32x16{};
  const float c = a.scale_log2;

  load_tile(0);
  store_tile(0);
  __syncthreads();

  // Key tile j.  MASKED steps are the causal ones that straddle this
  // workgroup's queries: a 32-key block after a wave's queries is skipped and
  // the block on the wave's diagonal (kvb == qw) gets the fixed triangle mask.
  // Earlier tiles are visible to every query and run the branch-free body.
  auto step = [&](int j, auto masked_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    const int buf = j & 1;
    const int kv0 = j * C::BKV;
    if (j + 1 < nkv) load_tile(kv0 + C::BKV);

    if (wave_valid && (!MASKED || kv0 <= qw + 31)) {
      const uint16_t* Ks = smem[buf];
      const uint16_t* Vs = Ks + C::BKV * C::RLD;
      u32x4 sb[C::NKB][2];
      bool live[C::NKB];
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb) {
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
#pragma unroll
      for (int kb = 0; kb < C::NKB; ++kb) {
        if (!live[kb]) continue;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int db = 0; db < C::DB; ++db) {
            // K^T operand read transposed from the row-major K tile.
            const int off = (32 * kb + 16 * hh) * C::RLD + 32 * db + tro;
            acc[db] = E::mfma(tr_operand(&Ks[off], C::RLD), sb[kb][hh], acc[db]);
          }
        }
      }
    }

    if (j + 1 < nkv) store_tile(buf ^ 1);
    __syncthreads();
  };

  const int n_main = CAUSAL ? max(0, nkv - C::BQ / C::BKV) : nkv;
  int j = 0;
  for (; j < n_main; ++j) step(j, std::false_type{});
  if constexpr (CAUSAL)
    for (; j < nkv; ++j) step(j, std::true_type{});

  if (!wave_valid) return;
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

template <typename E, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[2][DkvCfg<D>::BUF];
  __shared__ __attribute__((aligned(16))) float sl[2][2 * DkvCfg<D>::BQ];
  const int BH = a.B * a.H;
  // key tile 0 sees the most query tiles: dispatched first
  dkdv_body<E, D, CAUSAL>(a, blockIdx.x / BH, blockIdx.x % BH, smem, sl);
}

template <typename E, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnArgs a, int n_qtiles) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[2][DqCfg<D>::BUF];
  const int BH = a.B * a.H;
  dq_body<E, D, CAUSAL>(a, n_qtiles - 1 - (int)(blockIdx.x / BH), blockIdx.x % BH, smem);
}

// dK/dV and dQ in one launch.  The two workgroup kinds alternate in dispatch
// order, each heaviest-first (key tile 0 and the last query tile see the most
// tiles under causal masking), so the short tails of both kinds overlap the
// long heads of the other and the launch keeps the whole chip busy.  They
// share one LDS allocation.
template <int D>
struct BwdLds {
  static constexpr int DKV = 2 * DkvCfg<D>::BUF * 2 + 2 * 2 * DkvCfg<D>::BQ * 4;
  static constexpr int DQ = 2 * DqCfg<D>::BUF * 2;
  static constexpr int BYTES = DKV > DQ ? DKV : DQ;
};

template <typename E, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_bwd_kernel(AttnArgs a, int n_tiles) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[BwdLds<D>::BYTES];
  const int BH = a.B * a.H;
  const int rank = blockIdx.x / BH;
  const int bh = blockIdx.x % BH;
  if (rank & 1) {
    dq_body<E, D, CAUSAL>(a, n_tiles - 1 - (rank >> 1), bh, (uint16_t(*)[DqCfg<D>::BUF])lds);
  } else {
    dkdv_body<E, D, CAUSAL>(a, rank >> 1, bh, (uint16_t(*)[DkvCfg<D>::BUF])lds,
                            (float(*)[2 * DkvCfg<D>::BQ])(lds + 2 * DkvCfg<D>::BUF * 2));
  }
}

template <typename E, int D>
hipError_t launch_dkdv_d(const AttnArgs& a, hipStream_t st) {
  const int BH = a.B * a.H;
  const int nkt = (a.S + DkvCfg<D>::BKV - 1) / DkvCfg<D>::BKV;
  if (a.causal)
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<E, D, true>), dim3(nkt * BH), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<E, D, false>), dim3(nkt * BH), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <typename E, int D>
hipError_t launch_dq_d(const AttnArgs& a, hipStream_t st) {
  const int BH = a.B * a.H;
  const int nqt = (a.S + DqCfg<D>::BQ - 1) / DqCfg<D>::BQ;
  if (a.causal)
    hipLaunchKernelGGL((attn_bwd_dq_kernel<E, D, true>), dim3(nqt * BH), dim3(256), 0, st, a, nqt);
  else
    hipLaunchKernelGGL((attn_bwd_dq_kernel<E, D, false>), dim3(nqt * BH), dim3(256), 0, st, a, nqt);
  return hipGetLastError();
}

template <typename E, int D>
hipError_t launch_both_d(const AttnArgs& a, hipStream_t st) {
  static_assert(DkvCfg<D>::BKV == DqCfg<D>::BQ, "both kinds tile the sequence alike");
  const int BH = a.B * a.H;
  const int n = (a.S + DqCfg<D>::BQ - 1) / DqCfg<D>::BQ;
  if (a.causal)
    hipLaunchKernelGGL((attn_bwd_kernel<E, D, true>), dim3(2 * n * BH), dim3(256), 0, st, a, n);
  else
    hipLaunchKernelGGL((attn_bwd_kernel<E, D, false>), dim3(2 * n * BH), dim3(256), 0, st, a, n);
  return hipGetLastError();
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
