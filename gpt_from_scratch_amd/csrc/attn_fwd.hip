// attn_fwd.hip — flash-attention forward on gfx950 bf16/f16 matrix cores.
//
// Counterpart of `_attn_fwd` + `_attn_fwd_inner` (core/myFlashAttn.py:447-728):
// per Q tile, stream K/V tiles, online softmax in fp32 with the running max m
// and running sum l, O = O*alpha + P V, finally O /= l and
// lse = m + ln(l) (:640-649).  Causal tiles above the diagonal are never
// visited (:670-674); only tiles that straddle the diagonal are masked.
//
// Work decomposition:
//   * a workgroup (4 waves) owns BQ = 128 query rows of one (batch, head);
//     wave w owns rows [32w, 32w + 32);
//   * everything is computed transposed, S^T = K Q^T and O^T = V^T P^T, so that
//     in the 32x32 accumulator layout each lane holds one query column: the row
//     statistics are per-lane scalars (one v_permlane32_swap for the max) and
//     the probabilities feed the P V product as a B operand without any
//     register shuffle;
//   * K/V tiles of BKV = 64 keys are staged row-major through LDS; the K
//     operand is a contiguous 16-byte read, the V^T operand of P V comes from
//     the same row-major V tile through the transposing LDS read
//     (ds_read_b64_tr_b16);
//   * software pipeline: while the VALU runs the softmax of tile j, the matrix
//     cores already compute S for tile j+1, then P V for tile j.  K is staged
//     two tiles ahead and V one tile ahead (double buffers for each), so one
//     barrier per tile suffices;
//   * key tiles below the diagonal run a branch-free body; the diagonal tiles
//     run a masked body that also skips tiles a wave cannot see;
//   * the running max is only moved (and O, l rescaled) when a new score
//     exceeds it by more than 2^8 in exp2 units; otherwise probabilities are
//     taken against the stale max, which keeps them <= 256 and the result
//     exact (O and l share the same reference point);
//   * the grid is linearised heaviest-first: the Q tiles nearest the end of the
//     sequence (which see the most keys under causal masking) are dispatched
//     first, and all tiles of one head land on the same XCD (workgroups go
//     round-robin over the 8 XCDs and the index stride between tiles of one
//     head is B*H).
#include <type_traits>

#include "mi_device.h"
#include "mi_kernels.h"

namespace mi {

namespace {

template <int D>
struct FwdCfg {
  static constexpr int BQ = 128;
  static constexpr int BKV = 64;
  static constexpr int NT = 256;                     // 4 waves x 32 query rows
  static constexpr int KS = D / 16;                  // MFMA k-steps of K Q^T
  static constexpr int DB = D / 32;                  // 32-row blocks of O^T
  static constexpr int TILE = BKV * D;               // elements of a staged K or V tile
  static constexpr int CPR = D / 8;                  // 16-byte chunks per row
  static constexpr int RPS = 64 / CPR;               // rows per 1 KB slice (one wave instruction)
  static constexpr int SPW = TILE * 2 / 1024 / 4;    // slices per wave per tile
  // LDS buffers per tensor.  Steps run in phases of NBUF/2 tiles with one
  // barrier per phase; D = 128 tiles are twice as large, so two buffers.
  static constexpr int NBUF = (D == 64) ? 4 : 2;
  static constexpr int L = NBUF / 2;  // tiles per phase
};

// LDS layout of a staged tile: BKV rows of D elements, no padding; the
// 16-byte chunk c of row r sits at chunk position c ^ swz(r).
//   K: swz = r & 7        the A-operand reads of K Q^T (each lane a 16-byte
//                         chunk, eight consecutive rows per LDS cycle) land
//                         on eight different chunk positions;
//   V: swz = 2 * (r & 3)  the transposing reads of V^T (16-lane groups over
//                         four consecutive rows and two adjacent chunks)
//                         likewise.
__device__ __forceinline__ int swz_k(int r) { return r & 7; }
__device__ __forceinline__ int swz_v(int r) { return (r & 3) << 1; }

constexpr float kRescaleSlack = 8.f;  // log2 units: probabilities stay <= 2^8

template <typename E, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_fwd_mfma_kernel(AttnArgs a, int n_qtiles) {
  using C = FwdCfg<D>;
  // One array per buffer, so that the compiler can see that a direct load
  // into one buffer never aliases the reads of another.
  constexpr int T23 = C::NBUF == 4 ? C::TILE : 8;
  __shared__ __attribute__((aligned(16))) uint16_t K0[C::TILE];
  __shared__ __attribute__((aligned(16))) uint16_t K1[C::TILE];
  __shared__ __attribute__((aligned(16))) uint16_t K2[T23];
  __shared__ __attribute__((aligned(16))) uint16_t K3[T23];
  __shared__ __attribute__((aligned(16))) uint16_t V0[C::TILE];
  __shared__ __attribute__((aligned(16))) uint16_t V1[C::TILE];
  __shared__ __attribute__((aligned(16))) uint16_t V2[T23];
  __shared__ __attribute__((aligned(16))) uint16_t V3[T23];
  auto kbuf = [&](auto i) __attribute__((always_inline)) -> uint16_t* {
    constexpr int I = decltype(i)::value;
    if constexpr (I == 0) return K0;
    else if constexpr (I == 1) return K1;
    else if constexpr (I == 2) return K2;
    else return K3;
  };
  auto vbuf = [&](auto i) __attribute__((always_inline)) -> uint16_t* {
    constexpr int I = decltype(i)::value;
    if constexpr (I == 0) return V0;
    else if constexpr (I == 1) return V1;
    else if constexpr (I == 2) return V2;
    else return V3;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  const int qt = n_qtiles - 1 - bid / BH;
  const int bh = bid % BH;
  const int b = bh / a.H;
  const int h = bh % a.H;
  const int S = a.S;

  const uint16_t* qp = (const uint16_t*)a.q.ptr + b * a.q.sb + h * a.q.sh;
  const uint16_t* kp = (const uint16_t*)a.k.ptr + b * a.k.sb + h * a.k.sh;
  const uint16_t* vp = (const uint16_t*)a.v.ptr + b * a.v.sb + h * a.v.sh;
  uint16_t* op = (uint16_t*)a.o.ptr + b * a.o.sb + h * a.o.sh;

  const int q0 = qt * C::BQ;
  const int qw = q0 + 32 * wave;       // first query row of this wave (SGPR)
  const bool wave_valid = qw < S;      // S % 64 == 0: 32-row blocks are all-or-nothing
  const int qrow = qw + l32;

  u32x4 qf[C::KS];
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks)
    qf[ks] = wave_valid ? *(const u32x4*)(qp + (int64_t)qrow * a.q.ss + 16 * ks + 8 * g)
                        : u32x4{0, 0, 0, 0};

  const int kv_end = CAUSAL ? min(q0 + C::BQ, S) : S;
  const int nkv = kv_end / C::BKV;

  // ---- staging: direct global -> LDS loads ----
  // A tile is 1 KB slices; wave w fills slices w, w + 4, ...  Lane i of slice
  // s writes the 16 bytes at row s*RPS + i/CPR, chunk position i%CPR, so it
  // fetches chunk (i%CPR) ^ swz(row) of that row.  One buffer descriptor per
  // tile, fixed per-lane byte offsets; completion is tracked by vmcnt and the
  // barrier that ends each step.
  uint32_t kdo[C::SPW], vdo[C::SPW];
#pragma unroll
  for (int m = 0; m < C::SPW; ++m) {
    const int r = (wave + 4 * m) * C::RPS + lane / C::CPR;
    const int pos = lane % C::CPR;
    kdo[m] = (uint32_t)((r * a.k.ss + ((pos ^ swz_k(r)) << 3)) * 2);
    vdo[m] = (uint32_t)((r * a.v.ss + ((pos ^ swz_v(r)) << 3)) * 2);
  }
  auto dma = [&](const uint16_t* base, int64_t ss, const uint32_t(&off)[C::SPW], int t,
                 uint16_t* tile) __attribute__((always_inline)) {
    const auto rs = tile_rsrc(base + (int64_t)t * C::BKV * ss);
#pragma unroll
    for (int m = 0; m < C::SPW; ++m)
      buffer_load_lds16(rs, off[m], tile + (wave + 4 * m) * 512);
  };

  // Per-lane LDS offsets of the MFMA operands.
  //   K Q^T A operand, k-step ks: row l32 (+32 per key block), chunk 2ks + g;
  //   V^T operand of P V (transposing read), O^T block db: row 4g + (lane%16)/4
  //   (+16 per half-block, +8 for the second read), column 32db +
  //   16((lane/16)%2) + 4(lane%4).
  int kro[C::KS], vro[C::DB];
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) kro[ks] = l32 * D + (((2 * ks + g) ^ swz_k(l32)) << 3);
#pragma unroll
  for (int db = 0; db < C::DB; ++db) {
    const int r = 4 * g + ((lane & 15) >> 2);
    const int ch = 4 * db + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    vro[db] = r * D + ((ch ^ swz_v(r)) << 3) + 4 * (lane & 1);
  }

  // ---- per-wave compute pieces ----
  f32x16 acc[C::DB];
#pragma unroll
  for (int i = 0; i < C::DB; ++i) acc[i] = f32x16{};
  float m_run = -INFINITY;  // running reference max (exp2 units)
  float l_run = 0.f;        // running sum over this lane's half of the keys
  const float c = a.scale_log2;

  // S^T for one key tile (two 32-key blocks).
  auto qk = [&](const uint16_t* kt, f32x16(&s)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4 kf = *(const u32x4*)(&kt[32 * kb * D + kro[ks]]);
        s[kb] = E::mfma(kf, qf[ks], ks == 0 ? f32x16{} : s[kb]);
      }
    }
  };
  // Softmax of S^T in place, probabilities packed into pb; key tile starts at kv0.
  auto softmax = [&](f32x16(&s)[2], u32x4(&pb)[2][2], int kv0, bool masked) __attribute__((always_inline)) {
    if (masked) {
      const int rel = qrow - kv0 - 4 * g;  // visible iff (kv - kv0 - 4g) <= rel
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (32 * kb + 8 * (r >> 2) + (r & 3) > rel) s[kb][r] = -INFINITY;
    }
    // NaN-propagating maximum: v_maximum3_f32 chains without input
    // canonicalisation (2 scores per instruction).
    float mx = vmax(s[0][0], s[0][1]);
#pragma unroll
    for (int i = 2; i < 32; i += 2) mx = vmax(vmax(mx, s[i >> 4][i & 15]), s[i >> 4][(i & 15) + 1]);
    mx = max_halves(mx) * c;
    if (__any(mx > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) acc[db] *= alpha;
    }
    const float mref = m_run;
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(__builtin_fmaf(s[kb][r], c, -mref));
        s[kb][r] = p;
        psum += p;
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int w = 0; w < 4; ++w)
          pb[kb][hh][w] = E::pack2(s[kb][8 * hh + 2 * w], s[kb][8 * hh + 2 * w + 1]);
    }
    l_run += psum;
  };
  // O^T += V^T P^T.
  auto pv = [&](const uint16_t* vt, const u32x4(&pb)[2][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int db = 0; db < C::DB; ++db)
          acc[db] = E::mfma(tr_operand(&vt[(32 * kb + 16 * hh) * D + vro[db]], D), pb[kb][hh],
                            acc[db]);
  };

  // Mask-free tile with the matrix-core work woven into the softmax.  The 32
  // scores per lane form 4 groups of 8 (one B operand of P V each).  Group g
  // issues 1/4 of the next tile's K Q^T MFMAs, turns its 8 scores into
  // probabilities, and issues the P V MFMAs of group g-1, so that every MFMA
  // has ~7 VALU instructions behind it to overlap with.  sched_barrier keeps
  // the compiler from clustering the MFMAs back together.
  auto hot = [&](const uint16_t* kt, const uint16_t* vt, f32x16(&s)[2], f32x16(&sn)[2]) __attribute__((always_inline)) {
    constexpr int KPG = C::KS / 4;  // k-steps of the next tile's S per group
    // K fragments of group g+1 are read while group g computes.
    u32x4 kf[2][KPG][2];
    auto read_k = [&](int grp, u32x4(&dst)[KPG][2]) __attribute__((always_inline)) {
#pragma unroll
      for (int kk = 0; kk < KPG; ++kk)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          dst[kk][nb] = *(const u32x4*)(&kt[32 * nb * D + kro[KPG * grp + kk]]);
    };
    read_k(0, kf[0]);

    float mx = vmax(s[0][0], s[0][1]);
#pragma unroll
    for (int i = 2; i < 32; i += 2) mx = vmax(vmax(mx, s[i >> 4][i & 15]), s[i >> 4][(i & 15) + 1]);
    mx = max_halves(mx) * c;
    if (__any(mx > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) acc[db] *= alpha;
    }
    const float mref = m_run;
    float psum = 0.f;
    u32x4 pb[4];
    auto pv_group = [&](int grp) __attribute__((always_inline)) {
      const int kb = grp >> 1, hh = grp & 1;
#pragma unroll
      for (int db = 0; db < C::DB; ++db)
        acc[db] = E::mfma(tr_operand(&vt[(32 * kb + 16 * hh) * D + vro[db]], D), pb[grp],
                          acc[db]);
    };
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      __builtin_amdgcn_sched_barrier(0);
      const int kb = grp >> 1, hh = grp & 1;
      if (grp < 3) read_k(grp + 1, kf[(grp + 1) & 1]);
#pragma unroll
      for (int kk = 0; kk < KPG; ++kk) {
        const int ks = KPG * grp + kk;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          sn[nb] = E::mfma(kf[grp & 1][kk][nb], qf[ks], ks == 0 ? f32x16{} : sn[nb]);
      }
      float p[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        p[i] = fast_exp2(__builtin_fmaf(s[kb][8 * hh + i], c, -mref));
        psum += p[i];
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) pb[grp][w] = E::pack2(p[2 * w], p[2 * w + 1]);
      if (grp > 0) pv_group(grp - 1);
      // 2*KPG + DB MFMAs against ~28 VALU ops: one MFMA, then a run of VALU.
#pragma unroll
      for (int m = 0; m < 2 * KPG + (grp > 0 ? C::DB : 0); ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    pv_group(3);
    l_run += psum;
  };

  // ---- prologue: K_0..K_L and V_0..V_{L-1} into LDS; S for tile 0 ----
  using I0_ = std::integral_constant<int, 0>;
  using I1_ = std::integral_constant<int, 1>;
  using I2_ = std::integral_constant<int, 2>;
  dma(kp, a.k.ss, kdo, 0, K0);
  dma(vp, a.v.ss, vdo, 0, V0);
  if (nkv > 1) dma(kp, a.k.ss, kdo, 1, K1);
  if constexpr (C::L == 2) {
    if (nkv > 1) dma(vp, a.v.ss, vdo, 1, V1);
    if (nkv > 2) dma(kp, a.k.ss, kdo, 2, K2);
  }
  __syncthreads();

  f32x16 sA[2], sB[2];
  if (wave_valid) qk(K0, sA);
  // The first phase loads a tile into K0: every wave must be done reading it.
  __syncthreads();

  // Tile j in buffer slot I = j % NBUF (a compile-time tag): S_{j+1} from K
  // slot I+1 runs on the matrix cores while the VALU turns S_j into P_j; then
  // O += P_j V_j from V slot I.
  auto step = [&](int j, f32x16(&scur)[2], f32x16(&snext)[2], auto masked_tag, auto slot) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr int I = decltype(slot)::value;
    const uint16_t* const knext = kbuf(std::integral_constant<int, (I + 1) % C::NBUF>{});
    const uint16_t* const vcur = vbuf(std::integral_constant<int, I>{});
    const int kv0 = j * C::BKV;
    u32x4 pb[2][2];
    if (!MASKED) {
      hot(knext, vcur, scur, snext);
    } else if (wave_valid) {
      if (j + 1 < nkv && (!CAUSAL || (j + 1) * C::BKV <= qw + 31)) qk(knext, snext);
      if (!CAUSAL || kv0 <= qw + 31) {
        softmax(scur, pb, kv0, CAUSAL && kv0 + C::BKV - 1 > qw);
        pv(vcur, pb);
      }
    }
  };
  // Phase starting at tile j (slot I0 = j % NBUF): loads K_{j+L+1..j+2L} and
  // V_{j+L..j+2L-1} into the slots the previous phase finished reading, runs
  // its L tiles and ends with the one barrier, by which the loads have landed.
  auto phase = [&](int j, auto masked_tag, auto slot0) __attribute__((always_inline)) {
    constexpr int I0 = decltype(slot0)::value;
    if (j + C::L + 1 < nkv)
      dma(kp, a.k.ss, kdo, j + C::L + 1, kbuf(std::integral_constant<int, (I0 + C::L + 1) % C::NBUF>{}));
    if (j + C::L < nkv)
      dma(vp, a.v.ss, vdo, j + C::L, vbuf(std::integral_constant<int, (I0 + C::L) % C::NBUF>{}));
    if constexpr (C::L == 2) {
      if (j + 4 < nkv) dma(kp, a.k.ss, kdo, j + 4, kbuf(std::integral_constant<int, I0>{}));
      if (j + 3 < nkv) dma(vp, a.v.ss, vdo, j + 3, vbuf(std::integral_constant<int, (I0 + 3) % 4>{}));
      step(j, sA, sB, masked_tag, std::integral_constant<int, I0>{});
      if (j + 1 < nkv) step(j + 1, sB, sA, masked_tag, std::integral_constant<int, I0 + 1>{});
    } else {
      // one tile per phase: scur alternates with the slot
      if constexpr (I0 == 0)
        step(j, sA, sB, masked_tag, I0_{});
      else
        step(j, sB, sA, masked_tag, I1_{});
    }
    __syncthreads();
  };

  // Branch-free body: tile j lies below the diagonal for every wave of the
  // workgroup and tile j+1 exists and is visible to every wave.  Phases hold
  // two tiles each (an even count keeps S_j in sA for even j).
  const int n_main =
      (wave_valid ? (CAUSAL ? min(q0 / C::BKV, nkv - 1) : nkv - 1) : 0) & ~1;
  int j = 0;
  auto run = [&](int j_end, auto masked_tag) __attribute__((always_inline)) {
    // phases over [j, j_end) with j even; slot pattern repeats every NBUF tiles
    if constexpr (C::L == 2) {
      if ((j & 3) == 2 && j < j_end) {
        phase(j, masked_tag, I2_{});
        j += 2;
      }
      for (; j + 2 < j_end; j += 4) {
        phase(j, masked_tag, I0_{});
        phase(j + 2, masked_tag, I2_{});
      }
      if (j < j_end) {
        phase(j, masked_tag, I0_{});
        j += 2;
      }
    } else {
      for (; j + 1 < j_end; j += 2) {
        phase(j, masked_tag, I0_{});
        phase(j + 1, masked_tag, I1_{});
      }
      if (j < j_end) {
        phase(j, masked_tag, I0_{});
        ++j;
      }
    }
  };
  run(n_main, std::false_type{});
  run(nkv, std::true_type{});

  if (!wave_valid) return;
  const float l_tot = sum_halves(l_run);
  const float inv_l = 1.f / l_tot;
  uint16_t* orow = op + (int64_t)qrow * a.o.ss;
#pragma unroll
  for (int db = 0; db < C::DB; ++db) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      u32x2 w;
      w[0] = E::pack2(acc[db][4 * jj + 0] * inv_l, acc[db][4 * jj + 1] * inv_l);
      w[1] = E::pack2(acc[db][4 * jj + 2] * inv_l, acc[db][4 * jj + 3] * inv_l);
      *(u32x2*)(orow + 32 * db + 8 * jj + 4 * g) = w;
    }
  }
  if (g == 0) a.lse[(int64_t)bh * S + qrow] = (m_run + fast_log2(l_tot)) * kLn2;
}

template <typename E, int D>
hipError_t launch_fwd_d(const AttnArgs& a, hipStream_t st) {
  const int n_qtiles = (a.S + FwdCfg<D>::BQ - 1) / FwdCfg<D>::BQ;
  dim3 grid(n_qtiles * a.B * a.H), block(FwdCfg<D>::NT);
  if (a.causal)
    hipLaunchKernelGGL((attn_fwd_mfma_kernel<E, D, true>), grid, block, 0, st, a, n_qtiles);
  else
    hipLaunchKernelGGL((attn_fwd_mfma_kernel<E, D, false>), grid, block, 0, st, a, n_qtiles);
  return hipGetLastError();
}

template <typename E>
hipError_t launch_fwd_e(const AttnArgs& a, hipStream_t st) {
  if (a.D == 64) return launch_fwd_d<E, 64>(a, st);
  return launch_fwd_d<E, 128>(a, st);
}

}  // namespace

bool mfma_supports(int dtype, int D, int S) {
  return (dtype == 1 || dtype == 2) && (D == 64 || D == 128) && S > 0 && S % 64 == 0;
}

hipError_t launch_attn_fwd_mfma(int dtype, const AttnArgs& a, hipStream_t st) {
  if (dtype == 2) return launch_fwd_e<BF16>(a, st);
  return launch_fwd_e<F16>(a, st);
}

}  // namespace mi
