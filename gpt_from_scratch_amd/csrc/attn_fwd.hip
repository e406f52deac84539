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
//   * K/V tiles of BKV = 64 keys are staged row-major through LDS by direct
//     global->LDS loads; the K operand is a contiguous 16-byte read, the V^T
//     operand of P V comes from the same row-major V tile through the
//     transposing LDS read (ds_read_b64_tr_b16);
//   * one tile per step (S, softmax, P V) with double buffers: the loads of
//     tile j+1 run under step j, one barrier per step.  Only one S tile is live,
//     so D = 64 fits a three-waves-per-SIMD register budget (three workgroups
//     per CU at once), which hides the step's latency better than pipelining
//     S_{j+1} under softmax_j inside a wave at half the occupancy;
//   * key tiles below the diagonal run a branch-free body; the diagonal tiles
//     run a masked body that also skips tiles a wave cannot see;
//   * the running max is only moved (and O, l rescaled) when a new score
//     exceeds it by more than 2^8 in exp2 units; otherwise probabilities are
//     taken against the stale max, which keeps the result exact (O and l share
//     the same reference point).  At D = 64 a step does not even compute its
//     tile's max: it takes the probabilities against the stale max and checks
//     their sum, and only a sum past a bound (a probability possibly above
//     2^8, or the first tile, which has no reference yet) recomputes the tile's
//     scores and takes the exact step;
//   * at D = 64, l sums the probabilities as rounded for P V (v_dot2 over the
//     packed pairs), so O / l normalises exactly the weights P V applied;
//   * the grid is linearised heaviest-first: the Q tiles nearest the end of the
//     sequence (which see the most keys under causal masking) are dispatched
//     first, and all tiles of one head land on the same XCD (workgroups go
//     round-robin over the 8 XCDs and the index stride between tiles of one
//     head is B*H).  Workgroups w and w + #CU share a CU, so every odd round
//     of #CU workgroups is taken in reverse (XCD kept): a CU's co-resident
//     tiles pair heavy with light.
//   * head dims 16 and 32 run the D = 64 kernel with DP valid columns, and
//     sequence lengths that are not a multiple of 64 the RAG instantiation
//     (rows past S staged as zeros, the last key tile's keys past S masked,
//     rows past S not stored); both are template parameters.
#include <atomic>
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
  // Waves per SIMD the register budget is held to.  D = 64 fits 128 VGPRs
  // (four waves) with an 8-byte spill and the operand reads issued just in
  // time; at three waves (up to 168 VGPRs, ~149 used) it runs 2-3% faster at
  // configs B8 S1024 and B4 S2048 (both 768 workgroups, three per CU anyway).
  static constexpr int WAVES_PER_EU = D == 64 ? 3 : 2;
};

// LDS layout of a staged tile: BKV rows of D elements, no padding; the
// 16-byte chunk c of row r sits at chunk position c ^ swz(r).  The gfx950 LDS
// has 64 four-byte banks: one 256-byte bank line holds two rows at D = 64 and
// one row at D = 128, and a 16-byte read serves 16 lanes per cycle.
//   K: the A-operand reads of K Q^T (each lane one 16-byte chunk, 16
//      consecutive rows per cycle) must land on 16 different 16-byte bank
//      groups: at D = 64 the two rows of a bank line differ in bit 0, so the
//      8 chunk positions are spread over rows r and r + 8 by (r & 7) ^ bit 3;
//      at D = 128 by r & 15.  (r & 7 alone at D = 64 measured half the read
//      rate of a conflict-free pattern in a probe of this access.)
//   V: the transposing reads of V^T cover four consecutive rows and four
//      adjacent chunks per 32 lanes: 2 * (r & 3) at D = 64 (rows of one bank
//      line differ in bit 0 already), 4 * (r & 3) at D = 128.
// Both swizzles repeat within 16 rows, and the V swizzle within 8, which the
// operand reads assume (K block offsets are multiples of 32 rows; the second
// transposing read of an operand is 8 rows on).
template <int D>
__device__ __forceinline__ int swz_k(int r) { return D == 64 ? ((r & 7) ^ ((r >> 3) & 1)) : (r & 15); }
template <int D>
__device__ __forceinline__ int swz_v(int r) { return D == 64 ? ((r & 3) << 1) : ((r & 3) << 2); }

constexpr float kRescaleSlack = 8.f;  // log2 units: exact-max probabilities stay <= 2^8

// Largest probability sum of one lane and tile taken without the tile's max
// (D = 64): 2^64 for bf16 P (fp32 O and l have room for it at any length),
// 2^14 for fp16 P (whose largest finite value is 65504).  A sum past it means
// a probability above 2^8, i.e. a max more than kRescaleSlack above the
// reference, so the exact step that follows moves the reference.
template <typename E>
__device__ __forceinline__ constexpr float kProbLimit() {
  return std::is_same<E, BF16>::value ? 0x1p64f : 0x1p14f;
}

// DP: head columns of the tensors.  Head dims 16 and 32 run in the D = 64
// layout: the padding chunks of the staged tiles load as zeros, the K Q^T
// products stop at DP, O^T blocks past DP are not accumulated and only DP
// columns are stored.
// RAG: S not a multiple of 64.  Rows at or past S load as zeros (the Q row
// loads are guarded, the tile descriptors end at row S), keys at or past S
// are masked in the last key tile, which takes the masked step, and rows at
// or past S are not stored.
template <typename E, int D, bool CAUSAL, int DP = D, bool RAG = false>
__global__ __launch_bounds__(256, FwdCfg<D>::WAVES_PER_EU) void attn_fwd_mfma_kernel(AttnArgs a, int n_qtiles, int n_cu) {
  using C = FwdCfg<D>;
  static_assert(DP == D || (D == 64 && (DP == 16 || DP == 32)), "head dim");
  constexpr int KSP = DP / 16;         // k-steps of K Q^T over the valid columns
  constexpr int DBP = (DP + 31) / 32;  // O^T blocks holding valid columns
  // One array per buffer, so that the compiler can see that a direct load
  // into one buffer never aliases the reads of another.
  __shared__ __attribute__((aligned(16))) uint16_t K0[C::TILE];
  __shared__ __attribute__((aligned(16))) uint16_t K1[C::TILE];
  __shared__ __attribute__((aligned(16))) uint16_t V0[C::TILE];
  __shared__ __attribute__((aligned(16))) uint16_t V1[C::TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  const int BH = a.B * a.H;
  int bid = blockIdx.x;
  {
    // Heaviest query tiles first; odd rounds of #CU workgroups reversed
    // (within each XCD), so a CU's co-resident tiles pair heavy with light.
    const int R = bid / n_cu, c = bid % n_cu;
    const int cnt = min(n_cu, (int)gridDim.x - R * n_cu);
    if ((R & 1) && cnt % 8 == 0) bid = R * n_cu + 8 * (cnt / 8 - 1 - c / 8) + (c & 7);
  }
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
  const bool wave_valid = qw < S;      // without RAG, 32-row blocks are all-or-nothing
  const int qrow = qw + l32;

  u32x4 qf[C::KS];
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks)
    qf[ks] = (wave_valid && ks < KSP && (!RAG || qrow < S))
                 ? *(const u32x4*)(qp + (int64_t)qrow * a.q.ss + 16 * ks + 8 * g)
                 : u32x4{0, 0, 0, 0};

  const int kv_end = CAUSAL ? min(q0 + C::BQ, S) : S;
  const int nkv = RAG ? (kv_end + C::BKV - 1) / C::BKV : kv_end / C::BKV;
  // first tile that may need a mask (RAG: the last one holds keys past S)
  const int jdiag = CAUSAL ? q0 / C::BKV : (RAG ? nkv - 1 : nkv);

  // ---- staging: direct global -> LDS loads ----
  // A tile is 1 KB slices; wave w fills slices w, w + 4, ...
  // Lane i of slice s writes the 16 bytes at row s*RPS + i/CPR, chunk position
  // i%CPR, so it fetches chunk (i%CPR) ^ swz(row) of that row.  One buffer
  // descriptor per tile, fixed per-lane byte offsets; completion is tracked by
  // vmcnt and the barrier that ends each step.  Chunks past DP (padding) take
  // the out-of-range offset and stage as zeros.
  uint32_t kdo[C::SPW], vdo[C::SPW];
#pragma unroll
  for (int m = 0; m < C::SPW; ++m) {
    const int r = (wave + 4 * m) * C::RPS + lane / C::CPR;
    const int pos = lane % C::CPR;
    const int kc = pos ^ swz_k<D>(r), vc = pos ^ swz_v<D>(r);
    kdo[m] = (DP < D && kc >= DP / 8) ? kOobOffset : (uint32_t)((r * a.k.ss + (kc << 3)) * 2);
    vdo[m] = (DP < D && vc >= DP / 8) ? kOobOffset : (uint32_t)((r * a.v.ss + (vc << 3)) * 2);
  }
  auto dma = [&](const uint16_t* base, int64_t ss, const uint32_t(&off)[C::SPW], int t,
                 uint16_t* tile) __attribute__((always_inline)) {
    const int rows = RAG ? min(C::BKV, S - t * C::BKV) : C::BKV;
    const auto rs = tile_rsrc(base + (int64_t)t * C::BKV * ss, rows_extent(rows, ss, DP));
#pragma unroll
    for (int m = 0; m < C::SPW; ++m)
      buffer_load_lds16(rs, off[m], tile + (wave + 4 * m) * 512);
  };

  // Per-lane LDS offsets of the MFMA operands.
  //   K Q^T A operand, k-step ks: row l32 (+32 per key block), chunk 2ks + g;
  //   V^T operand of P V (transposing read), O^T block db: row 4g + (lane%16)/4
  //   (+16 per half-block, +8 for the second read), column 32db +
  //   16((lane/16)%2) + 4(lane%4).
  // Byte offsets, the lane part only: each read adds its tile buffer and block
  // as a constant that the LDS instruction takes as its immediate.  They are
  // refreshed (opaque) at the top of every step, so the compiler cannot hoist
  // one "buffer + offset" register per buffer out of the step loop.
  int kro[C::KS], vro[C::DB];
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) kro[ks] = 2 * (l32 * D + (((2 * ks + g) ^ swz_k<D>(l32)) << 3));
#pragma unroll
  for (int db = 0; db < C::DB; ++db) {
    const int r = 4 * g + ((lane & 15) >> 2);
    const int ch = 4 * db + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    vro[db] = 2 * (r * D + ((ch ^ swz_v<D>(r)) << 3) + 4 * (lane & 1));
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
    for (int ks = 0; ks < KSP; ++ks) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4 kf = *(const u32x4*)((const char*)kt + 64 * kb * D + kro[ks]);
        s[kb] = E::mfma(kf, qf[ks], ks == 0 ? f32x16{} : s[kb]);
      }
    }
  };
  // Triangle mask of a diagonal tile (key tile starting at kv0).
  auto mask = [&](f32x16(&s)[2], int kv0) __attribute__((always_inline)) {
    const int rel = qrow - kv0 - 4 * g;  // visible iff (kv - kv0 - 4g) <= rel
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (32 * kb + 8 * (r >> 2) + (r & 3) > rel) s[kb][r] = -INFINITY;
  };
  // RAG: keys at or past S of the tile starting at kv0 masked.
  auto mask_tail = [&](f32x16(&s)[2], int kv0) __attribute__((always_inline)) {
    const int lim = S - kv0 - 4 * g;  // visible iff (kv - kv0 - 4g) < lim
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (32 * kb + 8 * (r >> 2) + (r & 3) >= lim) s[kb][r] = -INFINITY;
  };
  // Probabilities against the reference mref, in place, packed into pb; returns
  // their sum.  D = 64 sums the packed (rounded) values, the ones P V
  // multiplies, with one v_dot2 per pair; D = 128 (where that measured ~1%
  // slower) sums the fp32 values.
  auto probs = [&](f32x16(&s)[2], u32x4(&pb)[2][2], float mref) __attribute__((always_inline)) {
    float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[kb][r] = fast_exp2(__builtin_fmaf(s[kb][r], c, -mref));
        if constexpr (D != 64) ps[r & 3] += s[kb][r];
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          pb[kb][hh][w] = E::pack2(s[kb][8 * hh + 2 * w], s[kb][8 * hh + 2 * w + 1]);
          if constexpr (D == 64) ps[w] = E::sum2(pb[kb][hh][w], ps[w]);
        }
    }
    return (ps[0] + ps[1]) + (ps[2] + ps[3]);
  };
  // Exact reference: the running max moved to this tile's max (O and l
  // rescaled) when that exceeds it by more than kRescaleSlack; otherwise the
  // probabilities stay against the stale max, <= 2^8, and exact (O and l share
  // the reference point).
  auto to_max = [&](f32x16(&s)[2]) __attribute__((always_inline)) {
    // NaN-propagating maximum: v_maximum3_f32 chains without input
    // canonicalisation (2 scores per instruction).
    float mx = vmax(s[0][0], s[0][1]);
#pragma unroll
    for (int i = 2; i < 32; i += 2) mx = vmax(vmax(mx, s[i >> 4][i & 15]), s[i >> 4][(i & 15) + 1]);
    mx = max_halves(mx) * c;
    if (__any(mx > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) acc[db] *= alpha;
      m_run = m_new;
    }
  };
  // O^T += V^T P^T.
  auto pv = [&](const uint16_t* vt, const u32x4(&pb)[2][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int db = 0; db < DBP; ++db)
          acc[db] = E::mfma(tr_operand((const uint16_t*)((const char*)vt +
                                                         2 * (32 * kb + 16 * hh) * D + vro[db]),
                                       D),
                            pb[kb][hh], acc[db]);
  };

  // ---- steps over key tiles [0, nkv) ----
  // Step j works on tile j from buffer j & 1 while the direct loads of tile
  // j + 1 fill the other buffer; the barrier that ends step j also ends those
  // loads (vmcnt) and every read of buffer j & 1.
  dma(kp, a.k.ss, kdo, 0, K0);
  dma(vp, a.v.ss, vdo, 0, V0);
  __syncthreads();
  auto step = [&](int j, auto masked_tag, auto slot) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr int I = decltype(slot)::value;
    const uint16_t* kt = I ? K1 : K0;
    const uint16_t* vt = I ? V1 : V0;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) opaque(kro[ks]);
#pragma unroll
    for (int db = 0; db < C::DB; ++db) opaque(vro[db]);
    if (j + 1 < nkv) {
      dma(kp, a.k.ss, kdo, j + 1, I ? K0 : K1);
      dma(vp, a.v.ss, vdo, j + 1, I ? V0 : V1);
    }
    const int kv0 = j * C::BKV;
    if (wave_valid && (!MASKED || !CAUSAL || kv0 <= qw + 31)) {
      const bool msk = MASKED && CAUSAL && kv0 + C::BKV - 1 > qw;
      const bool tmsk = RAG && MASKED && kv0 + C::BKV > S;
      f32x16 s[2];
      qk(kt, s);
      if (msk) mask(s, kv0);
      if (tmsk) mask_tail(s, kv0);
      u32x4 pb[2][2];
      // D = 64: probabilities against the running reference m_run without
      // this tile's max, exact as long as their sum stays within kProbLimit
      // (O and l share the reference).  The first tile (no reference yet) and
      // a tile whose sum says a probability may have passed the limit
      // recompute S from the staged K tile and take the exact step.  D = 128
      // takes the exact step every time (the skip's extra code spills there).
      float psum = 0.f;
      bool exact = D != 64 || j == 0;
      if (!exact) {
        psum = probs(s, pb, m_run);
        if (__any(!(psum <= kProbLimit<E>()))) {
          exact = true;
          qk(kt, s);
          if (msk) mask(s, kv0);
          if (tmsk) mask_tail(s, kv0);
        }
      }
      if (exact) {
        to_max(s);
        psum = probs(s, pb, m_run);
      }
      l_run += psum;
      pv(vt, pb);
    }
    __syncthreads();
  };
  using I0_ = std::integral_constant<int, 0>;
  using I1_ = std::integral_constant<int, 1>;
  // Branch-free pairs below the diagonal, then masked steps.
  const int n_main = wave_valid ? (min(jdiag, nkv) & ~1) : 0;
  int j = 0;
  for (; j < n_main; j += 2) {
    step(j, std::false_type{}, I0_{});
    step(j + 1, std::false_type{}, I1_{});
  }
  for (; j + 1 < nkv; j += 2) {
    step(j, std::true_type{}, I0_{});
    step(j + 1, std::true_type{}, I1_{});
  }
  if (j < nkv) step(j, std::true_type{}, I0_{});

  if (!wave_valid) return;
  const float l_tot = sum_halves(l_run);
  // Every buffer is idle after the last step's barrier: wave w stages its O
  // rows through buffer w.
  uint16_t* stage = wave == 0 ? K0 : wave == 1 ? K1 : wave == 2 ? V0 : V1;
  store_block_rows<E, D, DP>(acc, 1.f / l_tot, stage, op + (int64_t)qw * a.o.ss, a.o.ss,
                             RAG ? min(32, S - qw) : 32);
  if (g == 0 && (!RAG || qrow < S)) a.lse[(int64_t)bh * S + qrow] = (m_run + fast_log2(l_tot)) * kLn2;
}

// Compute units of the device `st` launches on (cached per device), the size
// of one dispatch round of the grid ordering; 0 when unknown or not a multiple
// of the 8 XCDs.  Calls may come from several host threads at once (the
// forward from the caller's, the backward from autograd's): the cache entries
// are atomics, and a race only makes two threads store the same value.
int cu_count(hipStream_t st) {
  static std::atomic<int> cache[64];
  int dev = -1;
  if (hipStreamGetDevice(st, &dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      cus = 0;
    n = (cus > 0 && cus % 8 == 0) ? cus : -1;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n > 0 ? n : 0;
}

template <typename E, int D, int DP = D, bool RAG = false>
hipError_t launch_fwd_d(const AttnArgs& a, hipStream_t st) {
  const int n_qtiles = (a.S + FwdCfg<D>::BQ - 1) / FwdCfg<D>::BQ;
  int n_cu = cu_count(st);
  if (n_cu == 0) n_cu = 1 << 30;  // one round: no reversal
  dim3 grid(n_qtiles * a.B * a.H), block(FwdCfg<D>::NT);
  if (a.causal)
    hipLaunchKernelGGL((attn_fwd_mfma_kernel<E, D, true, DP, RAG>), grid, block, 0, st, a,
                       n_qtiles, n_cu);
  else
    hipLaunchKernelGGL((attn_fwd_mfma_kernel<E, D, false, DP, RAG>), grid, block, 0, st, a,
                       n_qtiles, n_cu);
  return hipGetLastError();
}

template <typename E>
hipError_t launch_fwd_e(const AttnArgs& a, hipStream_t st) {
  if (a.S % 64) {
    if (a.D == 16) return launch_fwd_d<E, 64, 16, true>(a, st);
    if (a.D == 32) return launch_fwd_d<E, 64, 32, true>(a, st);
    if (a.D == 64) return launch_fwd_d<E, 64, 64, true>(a, st);
    return launch_fwd_d<E, 128, 128, true>(a, st);
  }
  if (a.D == 16) return launch_fwd_d<E, 64, 16>(a, st);
  if (a.D == 32) return launch_fwd_d<E, 64, 32>(a, st);
  if (a.D == 64) return launch_fwd_d<E, 64>(a, st);
  return launch_fwd_d<E, 128>(a, st);
}

}  // namespace

bool mfma_supports(int dtype, int D, int S) {
  return (dtype == 1 || dtype == 2) && S > 0 && (D == 16 || D == 32 || D == 64 || D == 128);
}

hipError_t launch_attn_fwd_mfma(int dtype, const AttnArgs& a, hipStream_t st) {
  if (dtype == 2) return launch_fwd_e<BF16>(a, st);
  return launch_fwd_e<F16>(a, st);
}

}  // namespace mi
