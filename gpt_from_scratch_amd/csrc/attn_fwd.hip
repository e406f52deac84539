// attn_fwd.hip — flash-attention forward on gfx950 bf16/f16 matrix cores.
//
// Counterpart of `_attn_fwd` + `_attn_fwd_inner` (core/myFlashAttn.py:447-728):
// per Q tile, stream K/V tiles, online softmax in fp32 with the running max m
// and running sum l, O = O*alpha + P V, finally O /= l and
// lse = m + ln(l) (:640-649).  Causal tiles above the diagonal are never
// visited (:670-674); only tiles that straddle the diagonal are masked.
//
// Work decomposition (one workgroup = 4 waves = 256 threads):
//   * a workgroup owns BQ = 128 query rows of one (batch, head); wave w owns
//     rows [32w, 32w + 32);
//   * K/V tiles of BKV = 64 keys are staged through LDS, double-buffered: the
//     next tile is fetched into registers while the current one is consumed;
//   * everything is computed transposed, S^T = K Q^T and O^T = V^T P^T, so that
//     in the 32x32 accumulator layout each lane holds one query column: the row
//     statistics are per-lane scalars (one cross-half exchange for the max) and
//     the probabilities feed the P V product as a B operand without any
//     register shuffle.  V is transposed once per tile while it is written to
//     LDS (4x4 blocks through v_perm), so every MFMA operand read from LDS is a
//     contiguous 8- or 16-byte access.
//   * the grid is linearised heaviest-first: the Q tiles nearest the end of the
//     sequence (which see the most keys under causal masking) are dispatched
//     first, and all tiles of one head are dispatched to the same XCD
//     (consecutive workgroups go round-robin over the 8 XCDs, and the index
//     stride between tiles of one head is B*H).
#include "mi_device.h"
#include "mi_kernels.h"

namespace mi {

namespace {

template <int D>
struct FwdCfg {
  static constexpr int BQ = 128;
  static constexpr int BKV = 64;
  static constexpr int NT = 256;
  static constexpr int KLD = D + 8;       // row stride of the K tile in LDS (elements)
  static constexpr int VLD = BKV + 4;     // row stride of the V^T tile in LDS
  static constexpr int KS = D / 16;       // MFMA k-steps of Q K^T
  static constexpr int DB = D / 32;       // 32-row blocks of O^T
  static constexpr int KCH = BKV * D / 8 / NT;  // 16-byte K chunks per thread
  static constexpr int VCPT = BKV * D / (NT * 4);  // V columns per thread (4 rows each)
  static constexpr int VCG = D / VCPT;    // V column groups
};

template <typename E, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void attn_fwd_mfma_kernel(AttnArgs a, int n_qtiles) {
  using C = FwdCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][C::BKV * C::KLD];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][D * C::VLD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
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
  const int qw = q0 + 32 * wave;          // first query row of this wave
  const bool wave_valid = qw < S;
  const int qrow = qw + l32;              // the query row this lane carries

  // Q^T operand fragments (B operand of S^T = K Q^T), kept for the whole loop.
  u32x4 qf[C::KS];
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) {
    if (wave_valid)
      qf[ks] = *(const u32x4*)(qp + (int64_t)qrow * a.q.ss + 16 * ks + 8 * g);
    else
      qf[ks] = u32x4{0, 0, 0, 0};
  }

  const int kv_end = CAUSAL ? min(q0 + C::BQ, S) : S;
  const int nkv = kv_end / C::BKV;

  // Per-thread staging registers for one K and one V tile.
  u32x4 kreg[C::KCH];
  typedef __attribute__((ext_vector_type(C::VCPT / 2))) uint32_t vrow_t;
  vrow_t vreg[4];

  const int v_rg = tid / C::VCG;  // V row group (4 rows)
  const int v_cg = tid % C::VCG;  // V column group (VCPT columns)

  auto load_tile = [&](int kv0) {
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) {
      const int ci = tid + C::NT * i;
      const int row = ci / (D / 8);
      const int col = (ci % (D / 8)) * 8;
      kreg[i] = *(const u32x4*)(kp + (int64_t)(kv0 + row) * a.k.ss + col);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      vreg[r] = *(const vrow_t*)(vp + (int64_t)(kv0 + 4 * v_rg + r) * a.v.ss + C::VCPT * v_cg);
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) {
      const int ci = tid + C::NT * i;
      const int row = ci / (D / 8);
      const int col = (ci % (D / 8)) * 8;
      *(u32x4*)(&Ks[buf][row * C::KLD + col]) = kreg[i];
    }
#pragma unroll
    for (int w = 0; w < C::VCPT / 2; ++w) {
      u32x2 c0, c1;
      transpose4x2(vreg[0][w], vreg[1][w], vreg[2][w], vreg[3][w], c0, c1);
      const int d = C::VCPT * v_cg + 2 * w;
      *(u32x2*)(&Vt[buf][d * C::VLD + 4 * v_rg]) = c0;
      *(u32x2*)(&Vt[buf][(d + 1) * C::VLD + 4 * v_rg]) = c1;
    }
  };

  f32x16 acc[C::DB];
#pragma unroll
  for (int i = 0; i < C::DB; ++i) acc[i] = f32x16{};
  float m_run = -INFINITY;  // running max of scaled scores (log2 units)
  float l_run = 0.f;        // running sum, this lane's half of the keys only
  const float c = a.scale_log2;

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int j = 0; j < nkv; ++j) {
    const int buf = j & 1;
    const int kv0 = j * C::BKV;
    if (j + 1 < nkv) load_tile(kv0 + C::BKV);

    if (wave_valid && (!CAUSAL || kv0 <= qw + 31)) {
      f32x16 s[2];
      bool live[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        live[kb] = !CAUSAL || (kv0 + 32 * kb <= qw + 31);
        s[kb] = f32x16{};
        if (live[kb]) {
#pragma unroll
          for (int ks = 0; ks < C::KS; ++ks) {
            const u32x4 kf = *(const u32x4*)(&Ks[buf][(32 * kb + l32) * C::KLD + 16 * ks + 8 * g]);
            s[kb] = E::mfma(kf, qf[ks], s[kb]);
          }
        }
      }
      // Causal mask on blocks that straddle the diagonal; fully masked blocks
      // are dropped below.
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        if (!live[kb]) continue;
        if (CAUSAL && kv0 + 32 * kb + 31 > qw) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kv = kv0 + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3);
            if (kv > qrow) s[kb][r] = -INFINITY;
          }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      }
      mx = fmaxf(mx, xor_shfl(mx, 32));
      const float m_new = fmaxf(m_run, mx * c);
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      float psum = 0.f;
      u32x4 pb[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = live[kb] ? fast_exp2(__builtin_fmaf(s[kb][r], c, -m_new)) : 0.f;
          s[kb][r] = p;
          psum += p;
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int w = 0; w < 4; ++w)
            pb[kb][hh][w] = E::pack2(s[kb][8 * hh + 2 * w], s[kb][8 * hh + 2 * w + 1]);
      }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) acc[db] *= alpha;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        if (!live[kb]) continue;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int db = 0; db < C::DB; ++db) {
            const uint16_t* vrow = &Vt[buf][(32 * db + l32) * C::VLD + 32 * kb + 16 * hh + 4 * g];
            const u32x2 lo = *(const u32x2*)vrow;
            const u32x2 hi = *(const u32x2*)(vrow + 8);
            const u32x4 vf = u32x4{lo[0], lo[1], hi[0], hi[1]};
            acc[db] = E::mfma(vf, pb[kb][hh], acc[db]);
          }
        }
      }
    }

    if (j + 1 < nkv) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (!wave_valid) return;
  const float l_tot = l_run + xor_shfl(l_run, 32);
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
  dim3 grid(n_qtiles * a.B * a.H), block(256);
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
