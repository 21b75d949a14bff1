// Causal attention backward over transformed operands for gfx950 (the closed form of
// tests/test_fpope.py:1571-1602 evaluated blockwise; P is recomputed from the forward's LSE):
//   P = exp(scale q~k~^T - lse), dV = P^T dO, dP = dO V^T, Di = rowsum(dO o O),
//   dS = P o (dP - Di), dq~ = scale dS k~, dk~ = scale dS^T q~.
// Two kernels, no atomics (results are bitwise reproducible):
//   dkdv_kernel: a workgroup owns NW*32 keys of one kv head (k~, v rows in registers) and walks
//                every query block of every query head in its GQA group; S and dP come out with the
//                key axis across lanes, so P^T / dS^T are A operands as they sit; dO and q~ are read
//                from LDS with the transpose load for dV and dk~.
//   dq_kernel:   a workgroup owns NW*32 queries (q~, dO rows in registers) and walks key blocks;
//                S^T and dP^T come out with queries across lanes, dS is the A operand of dq~ = dS k~,
//                k~ is read with the transpose load.
#include "pe_common.h"
#include "pe_internal.h"

namespace pe {

// The fp32 kernels recompute P in natural units, exp(fma(s, scale, -lse)): the one rounding of the
// exponent is at the size of s * scale - lse, which is small exactly where P is large, as in the
// reference's fp32 softmax.  The log2-unit form exp2(s * (scale log2 e) - lse log2 e) rounds at the
// size of the raw score (tens), and its P carried about three times the reference's error into dV
// and dK.  The bf16 kernels keep the log2 form (their error is set by the bf16 roundings).
// lse of query row q of (b, h) in natural units, +inf for rows past Sq and rows without keys (so
// their P is 0)
__device__ __forceinline__ float lse_nat(const CoreArgs& a, int bh, int q) {
  if (q >= a.Sq) return INFINITY;
  const float x = a.lse_in[(int64_t)bh * a.Sq + q];
  return x > -INFINITY ? x : INFINITY;
}
template <int DT> __device__ __forceinline__ float prob(float s, float scale, float sl2, float l) {
  if constexpr (DT == 1) return exp2f(__builtin_fmaf(s, scale, -l) * LOG2E);
  else return exp2f(s * sl2 - l);
}

// P with the explicit mask's log2-unit term ml2 (mask_l2) added to the score
template <int DT> __device__ __forceinline__ float prob_m(float s, float scale, float sl2, float l, float ml2) {
  if constexpr (DT == 1) return exp2f(__builtin_fmaf(s, scale, -l) * LOG2E + ml2);
  else return exp2f(s * sl2 + ml2 - l);
}

// MB (here and in dq_kernel): the explicit-mask instantiation, for any operand type.
template <int DT, int DQK, int DV, int BMQ, int NW, bool MB>
__global__ __launch_bounds__(NW * 64, 1) void dkdv_kernel(CoreArgs a) {
  using E = typename Elem<DT>::T;
  using M = MT<DT>;
  constexpr int KC = M::KC, EPL = M::EPL, ESZ = M::ESZ;
  constexpr int BNK = NW * 32, NT = NW * 64;
  constexpr int NCQ = DQK * ESZ / 16, NCO = DV * ESZ / 16;
  constexpr int NKF = DQK / KC, NVF = DV / KC, NQT = BMQ / 32, NPF = BMQ / KC, SPT = 32 / KC;
  constexpr int NDK = DQK / 32, NDV = DV / 32;
  constexpr int SQ_BYTES = BMQ * NCQ * 16, SO_BYTES = BMQ * NCO * 16;
  __shared__ __attribute__((aligned(16))) char smem[SQ_BYTES + SO_BYTES + 2 * BMQ * 4];
  char* sQ = smem;
  char* sO = smem + SQ_BYTES;
  float* sL = (float*)(smem + SQ_BYTES + SO_BYTES);
  float* sD = sL + BMQ;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int nkb = (a.Sk + BNK - 1) / BNK;
  int kb, bh;
  map_block(blockIdx.x, nkb, a.nbh, false, kb, bh);
  bh += a.bh0;  // the head group's units
  const int b = bh / a.Hkv, hk = bh % a.Hkv, grp = a.Hq / a.Hkv;
  const int k0 = kb * BNK, kw0 = k0 + w * 32, myk = kw0 + l32;
  const int off = a.causal_off;

  u32x4 kf[NKF], vf[NVF];
  {
    const int kr = myk < a.Sk ? myk : 0;
    const E* krow = (const E*)a.k + ((int64_t)(b * a.Hkv + hk) * a.Sk + kr) * DQK;
    const E* vrow = (const E*)a.v + b * a.v_sb + hk * a.v_sh + (int64_t)kr * a.v_ss;
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int kk = 0; kk < NKF; ++kk) kf[kk] = myk < a.Sk ? *(const u32x4*)(krow + kk * KC + g * EPL) : z;
#pragma unroll
    for (int kk = 0; kk < NVF; ++kk) vf[kk] = myk < a.Sk ? *(const u32x4*)(vrow + kk * KC + g * EPL) : z;
  }
  f32x16 dk[NDK], dv[NDV];
#pragma unroll
  for (int t = 0; t < NDK; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) dk[t][j] = 0.f;
#pragma unroll
  for (int t = 0; t < NDV; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) dv[t][j] = 0.f;

  const int nqb = (a.Sq + BMQ - 1) / BMQ;
  int qb0 = 0;
  if (a.causal) qb0 = max(0, k0 - off) / BMQ;
  if (qb0 > nqb) qb0 = nqb;
  const int nper = nqb - qb0;
  const int niter = nper * grp;
  const float sl2 = a.scale * LOG2E;
  const int64_t qrs = (int64_t)DQK * ESZ, ors = (int64_t)DV * ESZ;

  TileStage<BMQ, NCQ, NT> stQ;
  TileStage<BMQ, NCO, NT> stO;
  auto src_q = [&](int it, int& h, int& q0) {
    h = hk * grp + it / nper;
    q0 = (qb0 + it % nper) * BMQ;
  };
  if (niter > 0) {
    int h, q0;
    src_q(0, h, q0);
    const int64_t r0 = (int64_t)(b * a.Hq + h) * a.Sq + q0;
    stQ.load((const char*)a.q + r0 * qrs, qrs, a.Sq - q0, tid);
    stO.load((const char*)a.dO + r0 * ors, ors, a.Sq - q0, tid);
  }
  for (int it = 0; it < niter; ++it) {
    int h, q0;
    src_q(it, h, q0);
    const int64_t r0 = (int64_t)(b * a.Hq + h) * a.Sq + q0;
    __syncthreads();
    stQ.store(sQ, tid);
    stO.store(sO, tid);
    if (tid < BMQ) {
      const int64_t p0 = (int64_t)(b * a.Hq + h) * a.sq_pad + q0;
      if constexpr (DT == 1) sL[tid] = lse_nat(a, b * a.Hq + h, q0 + tid);
      else sL[tid] = a.L2[p0 + tid];
      sD[tid] = a.Di[p0 + tid];
    }
    __syncthreads();
    if (it + 1 < niter) {
      int h2, q2;
      src_q(it + 1, h2, q2);
      const int64_t r2 = (int64_t)(b * a.Hq + h2) * a.Sq + q2;
      stQ.load((const char*)a.q + r2 * qrs, qrs, a.Sq - q2, tid);
      stO.load((const char*)a.dO + r2 * ors, ors, a.Sq - q2, tid);
    }
    if (a.causal && kw0 > q0 + BMQ - 1 + off) continue;  // every key of this wave is after every query
    const bool edge = a.causal && (kw0 + 31 > q0 + off);

    u32x4 pf[NPF], dsf[NPF];
#pragma unroll
    for (int mt = 0; mt < NQT; ++mt) {
      f32x16 s, dp;
#pragma unroll
      for (int j = 0; j < 16; ++j) { s[j] = 0.f; dp[j] = 0.f; }
      const int row = mt * 32 + perm_row<DT>(l32);
#pragma unroll
      for (int kk = 0; kk < NKF; ++kk) s = M::mma(lds_row_frag<NCQ>(sQ, row, 2 * kk + g), kf[kk], s);
#pragma unroll
      for (int kk = 0; kk < NVF; ++kk) dp = M::mma(lds_row_frag<NCO>(sO, row, 2 * kk + g), vf[kk], dp);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int qi = mt * 32 + c_logical<DT>(j, g);
        float p;
        if constexpr (MB) p = prob_m<DT>(s[j], a.scale, sl2, sL[qi], mask_l2(a, b, h, q0 + qi, myk));
        else p = prob<DT>(s[j], a.scale, sl2, sL[qi]);
        if (edge && myk > q0 + qi + off) p = 0.f;
        s[j] = p;
        dp[j] = p * (dp[j] - sD[qi]);
      }
#pragma unroll
      for (int si = 0; si < SPT; ++si) {
        pf[mt * SPT + si] = M::pack(s, si * EPL);
        dsf[mt * SPT + si] = M::pack(dp, si * EPL);
      }
    }
    // two-level sums: each tile's products go into a zeroed accumulator that is then added to the
    // running one, so the running sums (|dv| reaches ~8 on early keys) are rounded once per tile
    // rather than once per product; chained over a whole sequence they carried about three times
    // the error of the reference's blocked fp32 products
#pragma unroll
    for (int t = 0; t < NDV; ++t) {
      f32x16 acc = {};
#pragma unroll
      for (int ks = 0; ks < NPF; ++ks) acc = M::mma(pf[ks], lds_col_frag<DT, NCO>(sO, ks * KC, t * 32, lane), acc);
      dv[t] += acc;
    }
#pragma unroll
    for (int t = 0; t < NDK; ++t) {
      f32x16 acc = {};
#pragma unroll
      for (int ks = 0; ks < NPF; ++ks) acc = M::mma(dsf[ks], lds_col_frag<DT, NCQ>(sQ, ks * KC, t * 32, lane), acc);
      dk[t] += acc;
    }
  }

  // epilogue: C rows = keys (kw0 + c_row), cols = feature / value column t*32 + l32
  float* dkb = a.dk_t + (int64_t)(b * a.Hkv + hk) * a.Sk * DQK;
#pragma unroll
  for (int t = 0; t < NDK; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int key = kw0 + c_row(j, g);
      if (key < a.Sk) dkb[(int64_t)key * DQK + t * 32 + l32] = dk[t][j] * a.scale;
    }
#pragma unroll
  for (int t = 0; t < NDV; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int key = kw0 + c_row(j, g), col = t * 32 + l32;
      if (key < a.Sk && col < a.dv_real)
        store_from_float(a.dv, b * a.dv_sb + hk * a.dv_sh + (int64_t)key * a.dv_ss + col, a.dv_dtype, dv[t][j]);
    }
}

template <int DT, int DQK, int DV, int BN, int NW, bool MB>
__global__ __launch_bounds__(NW * 64, 1) void dq_kernel(CoreArgs a) {
  using E = typename Elem<DT>::T;
  using M = MT<DT>;
  constexpr int KC = M::KC, EPL = M::EPL, ESZ = M::ESZ;
  constexpr int BM = NW * 32, NT = NW * 64;
  constexpr int NCK = DQK * ESZ / 16, NCV = DV * ESZ / 16;
  constexpr int NQF = DQK / KC, NVF = DV / KC, NKT = BN / 32, NPF = BN / KC, SPT = 32 / KC;
  constexpr int NDQ = DQK / 32;
  constexpr int SK_BYTES = BN * NCK * 16, SV_BYTES = BN * NCV * 16;
  __shared__ __attribute__((aligned(16))) char smem[SK_BYTES + SV_BYTES];
  char* sK = smem;
  char* sV = smem + SK_BYTES;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int nqb = (a.Sq + BM - 1) / BM;
  int qb, bh;
  map_block(blockIdx.x, nqb, a.nbh * (a.Hq / a.Hkv), a.causal != 0, qb, bh);
  bh += a.bh0 * (a.Hq / a.Hkv);  // the head group's query heads
  const int b = bh / a.Hq, h = bh % a.Hq, hk = h / (a.Hq / a.Hkv);
  const int q0 = qb * BM, qw = q0 + w * 32, myq = qw + l32;
  const int off = a.causal_off;
  const int64_t rowq = (int64_t)(b * a.Hq + h) * a.Sq + (myq < a.Sq ? myq : 0);

  u32x4 qf[NQF], of[NVF];
  {
    const E* qrow = (const E*)a.q + rowq * DQK;
    const E* orow = (const E*)a.dO + rowq * DV;
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int kk = 0; kk < NQF; ++kk) qf[kk] = myq < a.Sq ? *(const u32x4*)(qrow + kk * KC + g * EPL) : z;
#pragma unroll
    for (int kk = 0; kk < NVF; ++kk) of[kk] = myq < a.Sq ? *(const u32x4*)(orow + kk * KC + g * EPL) : z;
  }
  const int64_t prow = (int64_t)(b * a.Hq + h) * a.sq_pad + myq;
  const float lse2 = DT == 1 ? lse_nat(a, b * a.Hq + h, myq) : a.L2[prow], Dq = a.Di[prow];
  f32x16 dq[NDQ];
#pragma unroll
  for (int t = 0; t < NDQ; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) dq[t][j] = 0.f;

  int kend = a.Sk;
  if (a.causal) kend = min(a.Sk, q0 + BM + off);
  const int nkb = kend > 0 ? (kend + BN - 1) / BN : 0;
  const char* kbase = (const char*)((const E*)a.k + (int64_t)(b * a.Hkv + hk) * a.Sk * DQK);
  const char* vbase = (const char*)((const E*)a.v + b * a.v_sb + hk * a.v_sh);
  const int64_t krs = (int64_t)DQK * ESZ, vrs = a.v_ss * ESZ;
  const float sl2 = a.scale * LOG2E;

  TileStage<BN, NCK, NT> stK;
  TileStage<BN, NCV, NT> stV;
  if (nkb > 0) {
    stK.load(kbase, krs, a.Sk, tid);
    stV.load(vbase, vrs, a.Sk, tid);
  }
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * BN;
    __syncthreads();
    stK.store(sK, tid);
    stV.store(sV, tid);
    __syncthreads();
    if (kb + 1 < nkb) {
      stK.load(kbase + (int64_t)(k0 + BN) * krs, krs, a.Sk - k0 - BN, tid);
      stV.load(vbase + (int64_t)(k0 + BN) * vrs, vrs, a.Sk - k0 - BN, tid);
    }
    if (a.causal && k0 > qw + 31 + off) continue;
    const bool edge = (a.causal && k0 + BN - 1 > qw + off) || (k0 + BN > a.Sk);

    u32x4 dsf[NPF];
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt) {
      f32x16 s, dp;
#pragma unroll
      for (int j = 0; j < 16; ++j) { s[j] = 0.f; dp[j] = 0.f; }
      const int row = nt * 32 + perm_row<DT>(l32);
#pragma unroll
      for (int kk = 0; kk < NQF; ++kk) s = M::mma(lds_row_frag<NCK>(sK, row, 2 * kk + g), qf[kk], s);
#pragma unroll
      for (int kk = 0; kk < NVF; ++kk) dp = M::mma(lds_row_frag<NCV>(sV, row, 2 * kk + g), of[kk], dp);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float p;
        if constexpr (MB) p = prob_m<DT>(s[j], a.scale, sl2, lse2, mask_l2(a, b, h, myq, k0 + nt * 32 + c_logical<DT>(j, g)));
        else p = prob<DT>(s[j], a.scale, sl2, lse2);
        if (edge) {
          const int key = k0 + nt * 32 + c_logical<DT>(j, g);
          if (key >= a.Sk || (a.causal && key > myq + off)) p = 0.f;
        }
        dp[j] = p * (dp[j] - Dq);
      }
#pragma unroll
      for (int si = 0; si < SPT; ++si) dsf[nt * SPT + si] = M::pack(dp, si * EPL);
    }
#pragma unroll
    for (int t = 0; t < NDQ; ++t) {  // two-level sums, as in dkdv_kernel
      f32x16 acc = {};
#pragma unroll
      for (int ks = 0; ks < NPF; ++ks) acc = M::mma(dsf[ks], lds_col_frag<DT, NCK>(sK, ks * KC, t * 32, lane), acc);
      dq[t] += acc;
    }
  }

  float* dqb = a.dq_t + (int64_t)(b * a.Hq + h) * a.Sq * DQK;
#pragma unroll
  for (int t = 0; t < NDQ; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int q = qw + c_row(j, g);
      if (q < a.Sq) dqb[(int64_t)q * DQK + t * 32 + l32] = dq[t][j] * a.scale;
    }
}

// ---------------------------------------------------------------------------------------------
// bf16 kernels tuned for gfx950.  Both keep one wave per SIMD (the 32-row fp32 accumulators for a
// 256-wide dk~/dq~ take 128 registers) and stream 64-row tiles through an LDS ring filled by
// direct global->LDS loads (one barrier per tile, no prefetch registers).  A tile is consumed as
// two 32-row halves, software-pipelined inside each wave: the VALU work that turns the scores of
// half h into packed bf16 P / dS overlaps the MFMAs that consume half h-1, so the matrix core is
// not idle while the exponentials run (a single wave per SIMD has no other wave to hide them).
// ---------------------------------------------------------------------------------------------

// Causal mask for value j of a 32x32 score tile whose lanes are keys (key = lane) and whose
// values are rows of c_logical(j, g): the key is visible to the row iff key - off <= row.
// `kd` = key - off - (first row of the tile) - 8*g; returns true where the key is masked.
__device__ __forceinline__ bool masked_row(int kd, int j) { return kd > ((j >> 3) << 4) + (j & 7); }

// Fused RoPE / no-PE gradient (CoreArgs::rope_fuse) of NR rows, sequence indices base .. base + NR - 1
// (valid below nidx) of head h of batch b.  `stage` leaves the scaled dq~ or dk~ rows in st as fp32
// [NR][64] (barriers included).  8 of the NT threads per row, thread t taking the chunk of pairs
// 4t .. 4t + 3, with the stand-alone inv_rope_vec_kernel's arithmetic (inv_rope_chunk), so dq / dk
// are bitwise its results.  (Loading every row's x chunk before `stage`, so that the load latency is
// paid once, made the dK/dV kernel 4 % slower.)
template <int HT, int NT, int NR, typename Stage>
__device__ __forceinline__ void rope_epi_rows(const CoreArgs& a, const EpiPoPE& e, const float* st, int tid, int base,
                                              int nidx, int b, int h, Stage&& stage) {
  stage();
  const int t = tid & 7;
  float fr4[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) fr4[k] = a.rope_mode == 1 ? a.freqs[4 * t + k] : 0.f;
  const int64_t xb = b * e.x_s[0] + h * e.x_s[1] + t * 8, db = b * e.dx_s[0] + h * e.dx_s[1] + t * 8;
  for (int r = tid >> 3; r < NR; r += NT / 8) {
    const int idx = base + r;
    if (idx >= nidx) break;  // the same for the row's 8 threads
    float x[8], gv[8], dx[8];
    load8t<HT>(e.x, xb + (int64_t)idx * e.x_s[2], e.x_dtype, x);
    const f32x4 g0 = *(const f32x4*)(st + r * 64 + t * 8), g1 = *(const f32x4*)(st + r * 64 + t * 8 + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      gv[j] = g0[j];
      gv[j + 4] = g1[j];
    }
    inv_rope_chunk(a.rope_mode, a.rope_l2 != 0, fr4, pe_pos(e.start_pos + idx, e.pos_round), a.rope_ms, 8, x, gv, dx);
    store8t<HT>(e.dx, db + (int64_t)idx * e.dx_s[2], e.dx_dtype, dx);
  }
}

// dK~/dV: a workgroup owns 32*NW keys of one kv head; wave w keeps k~ and v of its 32 keys as MFMA
// B operands in registers and walks every visible 64-query tile of every query head of its GQA
// group.  LDS ring of 3 stages (q~ 64 x DQK, dO 64 x DV, the rows' log2 lse and Di): the tile being
// loaded, the tile being consumed and the previous tile, whose last half's dV / dK products run
// during the first half of the current one.
template <int HT, int DQK, int DV, int NW>
__global__ __launch_bounds__(NW * 64, 1) void dkdv_bf16_kernel(CoreArgs a) {
  using M = MT<HT>;  // HT: the 16-bit operand type, bf16 (0) or fp16 (2)
  constexpr int BMQ = 64, BNK = NW * 32;
  constexpr int NCQ = DQK / 8, NCO = DV / 8;
  constexpr int NKF = DQK / 16, NVF = DV / 16, NDK = DQK / 32, NDV = DV / 32;
  constexpr int SQ_BYTES = BMQ * NCQ * 16, SO_BYTES = BMQ * NCO * 16;
  constexpr int STAGE = SQ_BYTES + SO_BYTES + 2 * BMQ * 4;
  constexpr int NSTAGE = 3;
  __shared__ __attribute__((aligned(1024))) char smem[NSTAGE * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int nkb = (a.Sk + BNK - 1) / BNK;
  int kb, bh;
  map_block(blockIdx.x, nkb, a.nbh, false, kb, bh);
  bh += a.bh0;  // the head group's units
  const int b = bh / a.Hkv, hk = bh % a.Hkv, grp = a.Hq / a.Hkv;
  const int k0 = kb * BNK, kw0 = k0 + w * 32, myk = kw0 + l32;
  const int off = a.causal_off;

  u32x4 kf[NKF], vf[NVF];
  {
    const int kr = myk < a.Sk ? myk : a.Sk - 1;
    const uint16_t* krow = (const uint16_t*)a.k + ((int64_t)(b * a.Hkv + hk) * a.Sk + kr) * DQK;
    const uint16_t* vrow = (const uint16_t*)a.v + b * a.v_sb + hk * a.v_sh + (int64_t)kr * a.v_ss;
#pragma unroll
    for (int kk = 0; kk < NKF; ++kk) kf[kk] = *(const u32x4*)(krow + kk * 16 + g * 8);
#pragma unroll
    for (int kk = 0; kk < NVF; ++kk) vf[kk] = *(const u32x4*)(vrow + kk * 16 + g * 8);
  }
  f32x16 dk[NDK], dv[NDV];
#pragma unroll
  for (int t = 0; t < NDK; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) dk[t][j] = 0.f;
#pragma unroll
  for (int t = 0; t < NDV; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) dv[t][j] = 0.f;

  const int nqb = (a.Sq + BMQ - 1) / BMQ;
  int qb0 = 0;
  if (a.causal) qb0 = max(0, k0 - off) / BMQ;
  if (qb0 > nqb) qb0 = nqb;
  const int nper = nqb - qb0;
  const int niter = nper * grp;
  const float sl2 = a.scale * LOG2E;
  const int64_t qrs = (int64_t)DQK * 2;

  auto issue = [&](int it, char* st) {
    // lane-derived DMA offsets are recomputed per tile from an opaque copy of the lane id: held
    // across the loop they would be spilled, and a scratch reload waits for every load in flight
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int h = hk * grp + it / nper;
    const int q0 = (qb0 + it % nper) * BMQ;
    const int64_t r0 = (int64_t)(b * a.Hq + h) * a.Sq + q0;
    dma_tile<BMQ, NCQ, NW>(st, (const char*)a.q + r0 * qrs, qrs, a.Sq - q0, w, ln);
    dma_tile<BMQ, NCO, NW>(st + SQ_BYTES,
                           (const char*)a.dO + (b * a.do_sb + h * a.do_sh + (int64_t)q0 * a.do_ss) * 2,
                           a.do_ss * 2, a.Sq - q0, w, ln);
    if (w == 0) {
      const int64_t p0 = (int64_t)(b * a.Hq + h) * a.sq_pad + q0;
      const float* src = (lane < 16 ? a.L2 : a.Di) + p0 + (lane & 15) * 4;
      if (lane < 32)
        dma16(src, lds_addr(st + SQ_BYTES + SO_BYTES));
    }
  };

  // One loop step per 32-query half h (two halves per tile t = h / 2, stage t % 3):
  //   A. P / dS of half h from its scores (VALU), interleaved with the MFMAs of half h-1's
  //      products dV += P^T dO and dK~ += dS^T q~ (B operands by the transpose load);
  //   B. at a tile boundary: wait for the tile's loads, barrier, start loading tile t + 2's
  //      stage predecessor (the ring holds the previous, current and next tile);
  //   C. scores S = q~ k~^T and dP = dO v^T of half h + 1.
  const int nhalf = 2 * niter;
  u32x4 ppf[2], pdsf[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    ppf[i] = u32x4{0u, 0u, 0u, 0u};
    pdsf[i] = u32x4{0u, 0u, 0u, 0u};
  }
  int pbase = 0;  // byte offset of the pending half's stage within smem; its first row = prow
  int prow = 0;
  f32x16 s, dp;
#pragma unroll
  for (int j = 0; j < 16; ++j) { s[j] = 0.f; dp[j] = 0.f; }

  // Fragment reads run FD products ahead of the matrix core through fenced register rings (left to
  // itself the scheduler waits on every read right before its product); per-lane XOR bases, shared
  // by the q~ and dO tiles, make every fragment address a row pointer plus base plus immediate.
  constexpr int FD = 3;  // 3 and 4 measured equal; 3 leaves fewer registers to spill
  const RowX<NCQ> rq(perm_row<0>(l32), g);  // q~ / dO rows mt*32 + perm_row(l32)
  const RowX<NCO> ro(perm_row<0>(l32), g);
  const ColX<NCQ> cq(lane);                 // q~ / dO transpose fragments
  const ColX<NCO> co(lane);
  const uint32_t rrq = (uint32_t)perm_row<0>(l32) * NCQ * 16, rro = (uint32_t)perm_row<0>(l32) * NCO * 16;
  const uint32_t crq = ColX<NCQ>::row_term(lane), cro = ColX<NCO>::row_term(lane);

  auto scores = [&](int hh) {  // S / dP of half hh into s / dp
    const int t = hh >> 1, mt = hh & 1;
    const char* sq = smem + (t % NSTAGE) * STAGE + mt * 32 * NCQ * 16 + rrq;
    const char* so = smem + (t % NSTAGE) * STAGE + SQ_BYTES + mt * 32 * NCO * 16 + rro;
#pragma unroll
    for (int j = 0; j < 16; ++j) { s[j] = 0.f; dp[j] = 0.f; }
    constexpr int NS = NKF + NVF;
    auto rd = [&](int i) -> u32x4 { return i < NKF ? rq.read(sq, 0, i) : ro.read(so, 0, i - NKF); };
    u32x4 ring[FD];
#pragma unroll
    for (int i = 0; i < FD; ++i) ring[i] = rd(i);
    // fences for MFMA / LDS reads only (0x416 lets VALU, SALU, transcendental and global memory
    // instructions cross; the ALU bit 0x1 would let MFMAs cross as well, and under register pressure
    // the scheduler then pulls each product up to its own read, which leaves no read-ahead), so the
    // next tile's DMA issue, which precedes the scores at a tile boundary, can be spread between the
    // products
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      __builtin_amdgcn_sched_barrier(0x416);
      const u32x4 cur = ring[i % FD];
      if (i + FD < NS) ring[i % FD] = rd(i + FD);
      __builtin_amdgcn_sched_barrier(0x416);
      if (i < NKF) s = M::mma(cur, kf[i], s);
      else dp = M::mma(cur, vf[i - NKF], dp);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // products of the pending half (dV += P^T dO, dK~ += dS^T q~): NP products, ks-major so the two
  // products of one accumulator are NDV + NDK apart
  constexpr int NP = 2 * (NDV + NDK);
  auto rdp = [&](const char* pq, const char* po, int i) -> u32x4 {
    const int ks = i / (NDV + NDK), u = i % (NDV + NDK);
    return u < NDV ? co.read(po, ks * 16, u * 32) : cq.read(pq, ks * 16, (u - NDV) * 32);
  };
  auto prod = [&](int i, const u32x4& fr) {
    const int ks = i / (NDV + NDK), u = i % (NDV + NDK);
    if (u < NDV) dv[u] = M::mma(ppf[ks], fr, dv[u]);
    else dk[u - NDV] = M::mma(pdsf[ks], fr, dk[u - NDV]);
  };

  if (niter > 0) {
    issue(0, smem);
    dma_wait();
    __syncthreads();
    if (niter > 1) issue(1, smem + STAGE);
    scores(0);
  }
  for (int hh = 0; hh < nhalf; ++hh) {
    const int t = hh >> 1, mt = hh & 1;
    const int sb = (t % NSTAGE) * STAGE;
    const int q0 = (qb0 + t % nper) * BMQ;
    const float* sL = (const float*)(smem + sb + SQ_BYTES + SO_BYTES);
    const float* sD = sL + BMQ;
    __builtin_amdgcn_sched_barrier(0);
    // A. P = exp2(S*scale*log2e - L2) (rows past Sq carry L2 = +inf -> 0), dS = P (dP - Di), one
    //    element per product region of the pending half's products, so the VALU work interleaves
    //    with the matrix core
    // causal limit folded into kd (non-causal: never masked), so masking is one compare + select
    const int kd = a.causal ? myk - off - (q0 + mt * 32) - g * 8 : -(1 << 30);
    // L2 / Di of the lane's 16 rows: element j is row mt*32 + (j/8)*16 + g*8 + j%8; groups of 4
    // elements are read two product regions ahead into a double buffer
    f32x4 lg[2], dg[2];
    auto load_ld = [&](int G) {
      const int qi0 = mt * 32 + (G >> 1) * 16 + g * 8 + (G & 1) * 4;
      lg[G & 1] = *(const f32x4*)(sL + qi0);
      dg[G & 1] = *(const f32x4*)(sD + qi0);
    };
    load_ld(0);
    load_ld(1);
    const char* pq = smem + pbase + prow * NCQ * 16 + crq;
    const char* po = smem + pbase + SQ_BYTES + prow * NCO * 16 + cro;
    // the causal mask only where the half straddles the diagonal (wave-uniform branch): masked
    // scores become -inf, so exp2 gives P = 0; tiles wholly below the diagonal, almost all of
    // them, skip the compare and select
    if (__builtin_amdgcn_readfirstlane(a.causal && kw0 + 31 - off - (q0 + mt * 32) > 0)) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[i] = masked_row(kd, i) ? -INFINITY : s[i];
    }
    u32x4 ring[FD];
#pragma unroll
    for (int i = 0; i < FD; ++i) ring[i] = rdp(pq, po, i);
    float pprev = 0.f, dprev = 0.f;  // even element of the pair being packed
    u32x4 cpf[2], cdsf[2];
    // max(NP, 16) regions: every one of the 16 softmax elements gets a region even when the
    // pending half has fewer products (small head widths)
    constexpr int NR = NP > 16 ? NP : 16;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      // fence for MFMA / LDS reads only (mask 0x406 lets VALU, SALU and transcendental
      // instructions cross, but not MFMAs), so the softmax chains of consecutive elements overlap
      __builtin_amdgcn_sched_barrier(0x406);
      const u32x4 cur = ring[i % FD];
      if (i + FD < NP) ring[i % FD] = rdp(pq, po, i + FD);
      if (i % 4 == 2 && i + 2 < 16) load_ld((i + 2) / 4);
      if (i < 16) {
        const float lv = lg[(i / 4) & 1][i % 4], dd = dg[(i / 4) & 1][i % 4];
        const float p = fast_exp2(s[i] * sl2 - lv);
        const float ds = p * (dp[i] - dd);
        if (i & 1) {  // element pairs are packed as soon as they are complete
          cpf[i / 8][(i % 8) / 2] = pack2<HT>(pprev, p);
          cdsf[i / 8][(i % 8) / 2] = pack2<HT>(dprev, ds);
        } else {
          pprev = p;
          dprev = ds;
        }
      }
      if (i < NP) prod(i, cur);
    }
    __builtin_amdgcn_sched_barrier(0);
    // dS of this half in fragment order for the dQ GEMM: the wave's two 1 KiB chunks rows are
    // contiguous (block (key/32, q0/64), chunks (mt*2 + h2)*64 + lane); rows past Sk are padding
    {
      const int h = hk * grp + t / nper;
      char* blk = (char*)a.dS + ((int64_t)(b * a.Hq + h - a.bh0 * grp) * a.ds_head + ds_row_base(kw0 >> 5, a.ds_e, a.ds_nqt, a.causal) +
                                 (q0 >> 6) - ds_first(kb, a.ds_e, a.causal)) * 4096;
      __builtin_nontemporal_store(cdsf[0], (u32x4*)(blk + ((mt * 2 + 0) * 64 + lane) * 16));  // read once
      __builtin_nontemporal_store(cdsf[1], (u32x4*)(blk + ((mt * 2 + 1) * 64 + lane) * 16));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      ppf[i] = cpf[i];
      pdsf[i] = cdsf[i];
    }
    pbase = sb;
    prow = mt * 32;
    // B. tile boundary
    if (hh + 1 < nhalf) {
      if (mt == 1) {
        // the next tile's loads were issued before this tile's four dS stores; vector memory
        // counts retire in issue order, so allowing four outstanding waits for the loads only
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        __syncthreads();
        if (t + 2 < niter) issue(t + 2, smem + ((t + 2) % NSTAGE) * STAGE);
      }
      // C. scores of the next half
      scores(hh + 1);
    }
  }
  if (niter > 0) {
    const char* pq = smem + pbase + prow * NCQ * 16 + crq;
    const char* po = smem + pbase + SQ_BYTES + prow * NCO * 16 + cro;
    u32x4 ring[FD];
#pragma unroll
    for (int i = 0; i < FD; ++i) ring[i] = rdp(pq, po, i);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      __builtin_amdgcn_sched_barrier(0);
      const u32x4 cur = ring[i % FD];
      if (i + FD < NP) ring[i % FD] = rdp(pq, po, i + FD);
      __builtin_amdgcn_sched_barrier(0);
      prod(i, cur);
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  if (DQK == 64 && a.rope_fuse) {
    if constexpr (DQK == 64) {
      // RoPE / no-PE gradient: the scaled dk~ rows of the block's keys go through LDS (the ring is
      // free once every wave has passed the barrier), 8 threads per row
      static_assert(NSTAGE * STAGE >= BNK * 64 * 4, "staged dk~ rows fit the ring");
      float* st = (float*)smem;  // [BNK keys][64]
      rope_epi_rows<HT, NW * 64, BNK>(a, a.ek, st, tid, k0, a.Sk, b, hk, [&] {
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NDK; ++t)
#pragma unroll
          for (int j = 0; j < 16; ++j) st[(w * 32 + c_row(j, g)) * DQK + t * 32 + l32] = dk[t][j] * a.scale;
        __syncthreads();
      });
    }
  } else if (a.fuse_inv) {
    // inverse PoPE transform: the scaled dk~ rows go through LDS (the ring is free now) so that
    // one plain loop applies the transform, a fixed dim c per thread; dk is written through the
    // caller's view and dphi / pos*dphi are summed per block in a fixed order
    const EpiPoPE& e = a.ek;
    const int Dr = DQK / 2;
    float* st = (float*)smem;  // [BNK keys][DQK]
    const int c = tid % Dr;
    // EU rows per trip, software-pipelined: the x loads of trip i+1 are in flight while trip i
    // computes (one wave per SIMD has nothing else to hide their latency behind)
    constexpr int EU = 8;
    const int rstep = NW * 64 / Dr;
    const int64_t xb = b * e.x_s[0] + hk * e.x_s[1] + c * e.x_s[3];
    auto load_trip = [&](int r0, float (&xv)[EU]) {
#pragma unroll
      for (int u = 0; u < EU; ++u) {
        const int r = r0 + u * rstep, key = k0 + r;
        xv[u] = (r < BNK && key < a.Sk) ? load_as_float_t<HT>(e.x, xb + (int64_t)key * e.x_s[2], e.x_dtype) : 0.f;
      }
    };
    float xv[EU], xn[EU];
    load_trip(tid / Dr, xv);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NDK; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) st[(w * 32 + c_row(j, g)) * DQK + t * 32 + l32] = dk[t][j] * a.scale;
    __syncthreads();
    const float fr = a.freqs[c];
    const float dl = a.delta ? a.delta[hk * a.delta_hs + c] : 0.f;
    float sd = 0.f, sf = 0.f;
#pragma unroll 1
    for (int r0 = tid / Dr; r0 < BNK; r0 += EU * rstep) {
      load_trip(r0 + EU * rstep, xn);
#pragma unroll
      for (int u = 0; u < EU; ++u) {
        const int r = r0 + u * rstep, key = k0 + r;
        if (r < BNK && key < a.Sk) {
          const float pos = pe_pos(e.start_pos + key, e.pos_round);
          float dx;
          const float dph = inv_pope_elem(xv[u], pos, fr, dl, a.delta != nullptr, st[r * DQK + c],
                                          st[r * DQK + Dr + c], dx);
          store_from_float_t<HT>(e.dx, b * e.dx_s[0] + hk * e.dx_s[1] + (int64_t)key * e.dx_s[2] + c * e.dx_s[3],
                           e.dx_dtype, dx);
          sd += dph;
          sf += pos * dph;
        }
      }
#pragma unroll
      for (int u = 0; u < EU; ++u) xv[u] = xn[u];
    }
    if (e.part_delta || e.part_freq) {
      __syncthreads();
      float* red = st;  // [2][NW*64/Dr][Dr]
      const int nt = NW * 64 / Dr;  // threads per dim
      red[(0 * nt + tid / Dr) * Dr + c] = sd;
      red[(1 * nt + tid / Dr) * Dr + c] = sf;
      __syncthreads();
      const int64_t blk = (int64_t)bh * nkb + kb;
      if (tid < Dr) {
        float d0 = 0.f, f0 = 0.f;
        for (int i = 0; i < nt; ++i) {
          d0 += red[(0 * nt + i) * Dr + tid];
          f0 += red[(1 * nt + i) * Dr + tid];
        }
        if (e.part_delta) e.part_delta[blk * Dr + tid] = d0;
        if (e.part_freq) e.part_freq[blk * Dr + tid] = f0;
      }
    }
  } else {
    float* dkb = a.dk_t + (int64_t)(b * a.Hkv + hk) * a.Sk * DQK;
#pragma unroll
    for (int t = 0; t < NDK; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int key = kw0 + c_row(j, g);
        if (key < a.Sk) dkb[(int64_t)key * DQK + t * 32 + l32] = dk[t][j] * a.scale;
      }
  }
#pragma unroll
  for (int t = 0; t < NDV; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int key = kw0 + c_row(j, g), col = t * 32 + l32;
      if (key < a.Sk && col < a.dv_real)
        store_from_float_t<HT>(a.dv, b * a.dv_sb + hk * a.dv_sh + (int64_t)key * a.dv_ss + col, a.dv_dtype, dv[t][j]);
    }
}

// Vectorised form of the fused inverse PoPE epilogue.  It needs x and dx (and, with a content part,
// dxc) with a unit dim stride and every row 16-byte aligned (true of the projections'
// (B, S, H, D) views).
__device__ __forceinline__ bool epi_vec_ok(const EpiPoPE& e, int dc) {
  const int64_t xe = e.x_dtype == 1 ? 4 : 2, de = e.dx_dtype == 1 ? 4 : 2, ce = e.dxc_dtype == 1 ? 4 : 2;
  const bool c_ok = dc == 0 || (e.dxc_s[3] == 1 && (uintptr_t)e.dxc % 16 == 0 && (e.dxc_s[0] * ce) % 16 == 0 &&
                                (e.dxc_s[1] * ce) % 16 == 0 && (e.dxc_s[2] * ce) % 16 == 0);
  return c_ok && e.x_s[3] == 1 && e.dx_s[3] == 1 && (uintptr_t)e.x % 16 == 0 && (uintptr_t)e.dx % 16 == 0 &&
         (e.x_s[0] * xe) % 16 == 0 && (e.x_s[1] * xe) % 16 == 0 && (e.x_s[2] * xe) % 16 == 0 &&
         (e.dx_s[0] * de) % 16 == 0 && (e.dx_s[1] * de) % 16 == 0 && (e.dx_s[2] * de) % 16 == 0;
}
// Inverse transform of NR staged rows (st: fp32 [NR][DQK]; each row's gradient is the content part
// [0, DC), then the cos half [DC, DC + DR) and the sin half [DC + DR, DQK), DR = (DQK - DC) / 2).
// Thread (cg, rr) of the NT threads takes dims 8cg .. 8cg+7 of rows rr + RPP*i, with
// RPP = NT / (DR/8): it loads all its x rows first (16 or 32 bytes each), so their latency is paid
// once, then reads the two gradient halves as 16-byte LDS vectors and stores 8 dx at a time.  Row r
// is sequence index base + r (valid below nidx).  With key set, dl (8 values) is the key phase
// bias; sdl / sf accumulate sum(dphi) and sum(pos * dphi) per dim over the thread's rows.  With TAB
// (query side) the sin / cos of each row's phases come from launch_phase_table's [S][2][DR] table,
// indexed by the row's sequence index, instead of being evaluated.
template <int HT, int DQK, int DC, int NT, int NR, bool TAB>
__device__ __forceinline__ void inv_pope_rows(const EpiPoPE& e, const float* st, int tid, int64_t xb,
                                              int64_t dxb, int base, int nidx, const float (&fr)[8],
                                              const float (&dl)[8], bool key, const float* tab,
                                              float (&sdl)[8], float (&sf)[8]) {
  constexpr int Dr = (DQK - DC) / 2, CG = Dr / 8, RPP = NT / CG, NI = NR / RPP;
  static_assert(NT % CG == 0 && NR % RPP == 0, "whole rows per thread");
  const int c0 = (tid % CG) * 8, rr = tid / CG;
  float xv[NI][8];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int idx = base + rr + RPP * i;
    if (idx < nidx) {
      load8t<HT>(e.x, xb + (int64_t)idx * e.x_s[2] + c0, e.x_dtype, xv[i]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[i][j] = 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int r = rr + RPP * i, idx = base + r;
    if (idx < nidx) {
      const float* gr = st + r * DQK + DC;
      const f32x4 c_lo = *(const f32x4*)(gr + c0), c_hi = *(const f32x4*)(gr + c0 + 4);
      const f32x4 s_lo = *(const f32x4*)(gr + Dr + c0), s_hi = *(const f32x4*)(gr + Dr + c0 + 4);
      const float pos = pe_pos(e.start_pos + idx, e.pos_round);
      float dx[8];
      if constexpr (TAB) {
        const float* tr = tab + (int64_t)idx * (2 * Dr) + c0;
        const f32x4 tc0 = *(const f32x4*)tr, tc1 = *(const f32x4*)(tr + 4);
        const f32x4 ts0 = *(const f32x4*)(tr + Dr), ts1 = *(const f32x4*)(tr + Dr + 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float gc = j < 4 ? c_lo[j] : c_hi[j - 4], gs = j < 4 ? s_lo[j] : s_hi[j - 4];
          const float cs = j < 4 ? tc0[j] : tc1[j - 4], sn = j < 4 ? ts0[j] : ts1[j - 4];
          const float dph = inv_pope_elem_cs(xv[i][j], sn, cs, gc, gs, dx[j]);
          sdl[j] += dph;
          sf[j] += pos * dph;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float gc = j < 4 ? c_lo[j] : c_hi[j - 4], gs = j < 4 ? s_lo[j] : s_hi[j - 4];
          const float dph = inv_pope_elem(xv[i][j], pos, fr[j], dl[j], key, gc, gs, dx[j]);
          sdl[j] += dph;
          sf[j] += pos * dph;
        }
      }
      store8t<HT>(e.dx, dxb + (int64_t)idx * e.dx_s[2] + c0, e.dx_dtype, dx);
    }
  }
}
// The content part [0, DC) of NR staged rows, copied to dxc 8 dims at a time (no transform: the
// content dims enter the scores unchanged, so their gradient is the staged one).
template <int HT, int DQK, int DC, int NT, int NR>
__device__ __forceinline__ void content_rows(const EpiPoPE& e, const float* st, int tid, int64_t dxcb, int base,
                                             int nidx) {
  constexpr int CG = DC / 8, RPP = NT / CG;
  static_assert(DC % 8 == 0 && NT % CG == 0 && NR % RPP == 0, "whole rows per thread");
  const int c0 = (tid % CG) * 8, rr = tid / CG;
#pragma unroll
  for (int i = 0; i < NR / RPP; ++i) {
    const int r = rr + RPP * i, idx = base + r;
    if (idx < nidx) {
      const f32x4 lo = *(const f32x4*)(st + r * DQK + c0), hi = *(const f32x4*)(st + r * DQK + c0 + 4);
      const float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      store8t<HT>(e.dxc, dxcb + (int64_t)idx * e.dxc_s[2] + c0, e.dxc_dtype, v);
    }
  }
}

// The dK~ epilogue of the pair kernel and of dkdv_combine, 512 threads: the inverse PoPE
// transform of the staged rows st_epi[128 keys][DQK] (fp32, scaled) of key block kb of (b, hk)
// into dk (and the content part's copy into dk_c), plus the block's phase-gradient partials at
// index bh * nkb + kb.  Only with a.fuse_inv set.
template <int HT, int DQK>
__device__ __forceinline__ void dk_epilogue(const CoreArgs& a, float* st_epi, int tid, int b, int hk, int kb,
                                            int bh, int nkb) {
  constexpr int NW = 8, BNK = 128;
  const int k0 = kb * BNK;
  // DC is the content width, 0, or DQK / 2 at DQK = 128 (the host fuses no other split)
  auto epi_vec = [&](auto dc_tag) {
    constexpr int DC = decltype(dc_tag)::value;
    const EpiPoPE& e = a.ek;
    constexpr int Dr = (DQK - DC) / 2, CG = Dr / 8, RPP = NW * 64 / CG;
    const int c0 = (tid % CG) * 8, rr = tid / CG;
    float fr[8], dl[8], sdl[8], sf[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      fr[j] = a.freqs[c0 + j];
      dl[j] = a.delta ? a.delta[hk * a.delta_hs + c0 + j] : 0.f;
      sdl[j] = sf[j] = 0.f;
    }
    __syncthreads();  // every dk~ row staged
    if constexpr (DC > 0)
      content_rows<HT, DQK, DC, NW * 64, BNK>(e, st_epi, tid, b * e.dxc_s[0] + hk * e.dxc_s[1], k0, a.Sk);
    inv_pope_rows<HT, DQK, DC, NW * 64, BNK, false>(e, st_epi, tid, b * e.x_s[0] + hk * e.x_s[1],
                                                b * e.dx_s[0] + hk * e.dx_s[1], k0, a.Sk, fr, dl,
                                                a.delta != nullptr, nullptr, sdl, sf);
    if (e.part_delta || e.part_freq) {  // fixed-order sums over the RPP row groups of each dim
      __syncthreads();
      float* red = st_epi;  // [2][RPP][Dr]
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        red[(0 * RPP + rr) * Dr + c0 + j] = sdl[j];
        red[(1 * RPP + rr) * Dr + c0 + j] = sf[j];
      }
      __syncthreads();
      const int64_t blk = (int64_t)bh * nkb + kb;
      if (tid < Dr) {
        float d0 = 0.f, f0 = 0.f;
        for (int i = 0; i < RPP; ++i) {
          d0 += red[(0 * RPP + i) * Dr + tid];
          f0 += red[(1 * RPP + i) * Dr + tid];
        }
        if (e.part_delta) e.part_delta[blk * Dr + tid] = d0;
        if (e.part_freq) e.part_freq[blk * Dr + tid] = f0;
      }
    }
  };
  if (DQK == 128 && a.fuse_inv && a.Dc == DQK / 2) {  // split form: fused only at width 128, vector views
    if constexpr (DQK == 128) epi_vec(std::integral_constant<int, DQK / 2>{});
  } else if (a.fuse_inv && epi_vec_ok(a.ek, 0)) {
    epi_vec(std::integral_constant<int, 0>{});
  } else if (a.fuse_inv) {  // the same, element by element, for strided x / dx
    const EpiPoPE& e = a.ek;
    const int Dr = DQK / 2;
    float* st = st_epi;
    const int c = tid % Dr;
    constexpr int EU = 4;
    const int rstep = NW * 64 / Dr;
    const int64_t xb = b * e.x_s[0] + hk * e.x_s[1] + c * e.x_s[3];
    auto load_trip = [&](int r0, float (&xv)[EU]) {
#pragma unroll
      for (int u = 0; u < EU; ++u) {
        const int r = r0 + u * rstep, key = k0 + r;
        xv[u] = (r < BNK && key < a.Sk) ? load_as_float_t<HT>(e.x, xb + (int64_t)key * e.x_s[2], e.x_dtype) : 0.f;
      }
    };
    float xv[EU], xn[EU];
    load_trip(tid / Dr, xv);
    __syncthreads();
    const float fr = a.freqs[c];
    const float dl = a.delta ? a.delta[hk * a.delta_hs + c] : 0.f;
    float sdl = 0.f, sf = 0.f;
#pragma unroll 1
    for (int r0 = tid / Dr; r0 < BNK; r0 += EU * rstep) {
      load_trip(r0 + EU * rstep, xn);
#pragma unroll
      for (int u = 0; u < EU; ++u) {
        const int r = r0 + u * rstep, key = k0 + r;
        if (r < BNK && key < a.Sk) {
          const float pos = pe_pos(e.start_pos + key, e.pos_round);
          float dx;
          const float dph = inv_pope_elem(xv[u], pos, fr, dl, a.delta != nullptr, st[r * DQK + c],
                                          st[r * DQK + Dr + c], dx);
          store_from_float_t<HT>(e.dx, b * e.dx_s[0] + hk * e.dx_s[1] + (int64_t)key * e.dx_s[2] + c * e.dx_s[3],
                           e.dx_dtype, dx);
          sdl += dph;
          sf += pos * dph;
        }
      }
#pragma unroll
      for (int u = 0; u < EU; ++u) xv[u] = xn[u];
    }
    if (e.part_delta || e.part_freq) {
      __syncthreads();
      float* red = st;  // [2][NW*64/Dr][Dr]
      const int nt = NW * 64 / Dr;
      red[(0 * nt + tid / Dr) * Dr + c] = sdl;
      red[(1 * nt + tid / Dr) * Dr + c] = sf;
      __syncthreads();
      const int64_t blk = (int64_t)bh * nkb + kb;
      if (tid < Dr) {
        float d0 = 0.f, f0 = 0.f;
        for (int i = 0; i < nt; ++i) {
          d0 += red[(0 * nt + i) * Dr + tid];
          f0 += red[(1 * nt + i) * Dr + tid];
        }
        if (e.part_delta) e.part_delta[blk * Dr + tid] = d0;
        if (e.part_freq) e.part_freq[blk * Dr + tid] = f0;
      }
    }
  }
}

// dK~/dV with two waves per SIMD.  A workgroup of 8 waves owns 128 keys of one kv head; the 32
// keys of pair p are shared by wave p (role A: scores S, P = softmax numerator, dV += P^T dO) and
// wave p + 4 (role B: dP = dO v^T, dS = P (dP - Di), the dS store, dK~ += dS^T q~), which land on
// the same SIMD, so each SIMD interleaves two instruction streams of 24 products per 32-query tile
// and neither wave's exponentials, loads or waits leave the matrix core idle.  B gets the P it
// needs through an LDS exchange buffer in fp16 (11 significant bits, 2 KiB per wave per tile): dS
// = P (dP - Di) is rounded to bf16 (8 bits) right after, so the hand-off adds about an eighth of
// dS's own rounding error, where a bf16 hand-off would double it.  On fp16 operands dS itself keeps
// 11 bits, so there P goes over in fp32 (4 KiB per wave per 32-query sub-tile), as the fused SDPA
// backward forms dS from fp32 P; an fp16 hand-off made dQ's and dK's mean error 1.25 times that
// path's.  Each loop step t runs A's S of
// tile t, the loads of tile t+2, P of tile t and dV of tile t-1 (so A starts the step on products
// while B forms dS), and B's dS / dK~ of tile t-1 and dP of tile t, then one barrier; the 32-query
// tiles stream through a ring of 4 LDS stages (q~ 32 x DQK, dO 32 x DV, the rows' log2 lse and Di)
// loaded two steps ahead.
// (pack_h2 / unpack_h2, pe_common.h: two floats <-> one dword of fp16, round-to-nearest-even)
// MB: the explicit-mask instantiation; role A adds mask_l2 to the scaled scores before its
// exponentials, so P, the handed-over P and the stored dS carry the mask.
template <int HT, int DQK, int DV, int QT, bool QS, bool MB = false>
__global__ __launch_bounds__(512, 1) void dkdv_pair_kernel(CoreArgs a) {
  using M = MT<HT>;  // HT: the 16-bit operand type, bf16 (0) or fp16 (2)
  constexpr int NW = 8, BMQ = 32 * QT, BNK = 128, NSTG = 4;
  constexpr int NCQ = DQK / 8, NCO = DV / 8;
  constexpr int NKF = DQK / 16, NVF = DV / 16, NDK = DQK / 32, NDV = DV / 32;
  constexpr int SQ_BYTES = BMQ * NCQ * 16, SO_BYTES = BMQ * NCO * 16;
  constexpr int STAGE = SQ_BYTES + SO_BYTES + 2 * BMQ * 4;
  constexpr bool P32 = HT == 2;           // fp32 hand-off on fp16 operands
  // one pair's P of a step: fp16 [sub-tile][half][lane] 8 values, fp32 [sub-tile][quarter][lane] 4
  constexpr int XBP = (P32 ? 4096 : 2048) * QT;
  constexpr int XB_BYTES = 2 * 4 * XBP;   // P exchange: [step parity][pair]
  constexpr int RING = NSTG * STAGE + XB_BYTES;
  constexpr int EPI = BNK * DQK * 4;
  constexpr int SMEM = RING > EPI ? RING : EPI;
  // the four role-A waves issue all tile loads (issued by role B too, in place of its idle time at
  // the barrier, the kernel measured 1-2 % slower): DMA instructions per A wave per tile for q~,
  // dO and, from wave 0 only, one for the floats of L2 / Di
  constexpr int NA = 4;
  constexpr int PER = BMQ * NCQ / (64 * NA) + BMQ * NCO / (64 * NA) + 1;  // with the L2 / Di load
  static_assert(BMQ * NCQ % (64 * NA) == 0 && BMQ * NCO % (64 * NA) == 0, "whole wave instructions");
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];
  char* xbuf = smem + NSTG * STAGE;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int pw = w & 3;
  const bool roleB = __builtin_amdgcn_readfirstlane(w >> 2) != 0;
  const bool l2w = __builtin_amdgcn_readfirstlane(w) == 0;  // the wave that loads each tile's L2 / Di
  const int nkb = (a.Sk + BNK - 1) / BNK;
  int kb, bh;
  // QS (launched with a.qsplit > 1): workgroup jq of a key block takes query heads jq * hpw .. of
  // its group and leaves fp32 partial dK~ / dV for dkdv_combine (run by the dQ launch).  A separate
  // instantiation, so the unsplit kernel carries none of its registers.
  const int nblk = nkb * a.nbh, jq = QS ? (int)blockIdx.x / nblk : 0;
  map_block(blockIdx.x - jq * nblk, nkb, a.nbh, false, kb, bh);
  bh += a.bh0;  // the head group's units
  const int b = bh / a.Hkv, hk = bh % a.Hkv, grp = a.Hq / a.Hkv;
  const int hpw = QS ? grp / a.qsplit : grp, h_first = hk * grp + jq * hpw;
  const int k0 = kb * BNK, kw0 = k0 + pw * 32, myk = kw0 + l32;
  const int off = a.causal_off;

  const int nqt = (a.Sq + BMQ - 1) / BMQ;
  int qb0 = 0;
  if (a.causal) qb0 = max(0, k0 - off) / BMQ;
  if (qb0 > nqt) qb0 = nqt;
  const int nper = nqt - qb0;
  const int niter = nper * hpw;
  const float sl2 = a.scale * LOG2E;
  const int64_t qrs = (int64_t)DQK * 2;

  // tiles are issued in loop order: query tile qt of query head h advances qt, then h
  constexpr int SZ = 1;  // swizzle kind of the q~ and dO tiles (both take transpose reads)
  const DmaPlan<BMQ, NCQ, NA, SZ> plan_q(pw, lane, (uint32_t)qrs);
  const DmaPlan<BMQ, NCO, NA, SZ> plan_o(pw, lane, (uint32_t)(a.do_ss * 2));
  const uint32_t smem_l = lds_addr(smem);
  int iss_h = h_first, iss_qt = qb0;
  auto issue = [&](int it) {
    char* st = smem + (it % NSTG) * STAGE;
    const uint32_t stl = smem_l + (uint32_t)((it % NSTG) * STAGE);
    const int h = iss_h, q0 = iss_qt * BMQ;
    const char* qsrc = (const char*)a.q + ((int64_t)(b * a.Hq + h) * a.Sq + q0) * qrs;
    const char* osrc = (const char*)a.dO + (b * a.do_sb + h * a.do_sh + (int64_t)q0 * a.do_ss) * 2;
    if (a.Sq - q0 >= BMQ) {
      plan_q.full(qsrc, stl, pw, (uint32_t)qrs);
      plan_o.full(osrc, stl + SQ_BYTES, pw, (uint32_t)(a.do_ss * 2));
    } else {
      dma_tile<BMQ, NCQ, NA, SZ>(st, qsrc, qrs, a.Sq - q0, pw, lane);
      dma_tile<BMQ, NCO, NA, SZ>(st + SQ_BYTES, osrc, a.do_ss * 2, a.Sq - q0, pw, lane);
    }
    // the first A wave alone loads the tile's L2 (lanes 0 .. NL-1) and Di (lanes NL .. 2 NL-1),
    // NL = BMQ / 4 lanes of 4 floats each (when every A wave issued it, dK/dV was 0.5 % slower)
    constexpr int NL = BMQ / 4;
    const int64_t p0 = (int64_t)(b * a.Hq + h) * a.sq_pad + q0;
    if (l2w && lane < 2 * NL) dma16((lane < NL ? a.L2 : a.Di) + p0 + (lane % NL) * 4, stl + SQ_BYTES + SO_BYTES);
    if (++iss_qt == nqt) {
      iss_qt = qb0;
      ++iss_h;
    }
  };

  // fragment read-ahead depth: fragment i + FD is read while product i runs.  The fences below
  // (masks 0x416 / 0x406) pin LDS reads and MFMAs in program order and let vector, scalar and
  // transcendental work cross; with the ALU bit 0x1 MFMAs may cross too, and role B (at the register
  // limit) then had each product scheduled right after its own read.  Depths 3 and 4 with the ring
  // intact measured alike.
  constexpr int FD = 3;
  const RowX<NCQ, SZ> rq(perm_row<0>(l32), g);
  const RowX<NCO, SZ> ro(perm_row<0>(l32), g);
  const ColX<NCQ, SZ> cq(lane);
  const ColX<NCO, SZ> co(lane);
  const uint32_t rrq = (uint32_t)perm_row<0>(l32) * NCQ * 16, rro = (uint32_t)perm_row<0>(l32) * NCO * 16;
  const uint32_t crq = ColX<NCQ>::row_term(lane), cro = ColX<NCO>::row_term(lane);

  // A: S of the tile's QT 32-query sub-tiles into s[m] (the q~ rows of sub-tile m against the
  // wave's k~; fragment r of the read order is k-step r / QT of sub-tile r % QT)
  constexpr int NSS = NKF * QT;
  auto scores_s = [&](const char* sq, const u32x4 (&kf)[NKF], f32x16 (&s)[QT]) {
#pragma unroll
    for (int m = 0; m < QT; ++m)
#pragma unroll
      for (int j = 0; j < 16; ++j) s[m][j] = 0.f;
    u32x4 ring[FD];
#pragma unroll
    for (int i = 0; i < FD; ++i) ring[i] = rq.read(sq, (i % QT) * 32, i / QT);
#pragma unroll
    for (int i = 0; i < NSS; ++i) {
      __builtin_amdgcn_sched_barrier(0x416);
      const u32x4 cur = ring[i % FD];
      if (i + FD < NSS) ring[i % FD] = rq.read(sq, ((i + FD) % QT) * 32, (i + FD) / QT);
      __builtin_amdgcn_sched_barrier(0x416);
      s[i % QT] = M::mma(cur, kf[i / QT], s[i % QT]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // B: dP of the tile's sub-tiles into dp[m]
  constexpr int NSP = NVF * QT;
  auto scores_dp = [&](const char* so, const u32x4 (&vf)[NVF], f32x16 (&dp)[QT]) {
#pragma unroll
    for (int m = 0; m < QT; ++m)
#pragma unroll
      for (int j = 0; j < 16; ++j) dp[m][j] = 0.f;
    u32x4 ring[FD];
#pragma unroll
    for (int i = 0; i < FD; ++i) ring[i] = ro.read(so, (i % QT) * 32, i / QT);
#pragma unroll
    for (int i = 0; i < NSP; ++i) {
      __builtin_amdgcn_sched_barrier(0x416);
      const u32x4 cur = ring[i % FD];
      if (i + FD < NSP) ring[i % FD] = ro.read(so, ((i + FD) % QT) * 32, (i + FD) / QT);
      __builtin_amdgcn_sched_barrier(0x416);
      dp[i % QT] = M::mma(cur, vf[i / QT], dp[i % QT]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // products of one tile: NPR = 2 * QT * NT MFMAs over accumulators acc[0..NT), B operands by the
  // transpose load from the tile at `base` (k-step major, so the products of one accumulator are
  // NT apart; k-step ks covers query rows 16 ks .. 16 ks + 15)
  auto products = [&](auto& acc, const u32x4 (&af)[2 * QT], const char* base, const auto& cx) {
    constexpr int NT = sizeof(acc) / sizeof(acc[0]);
    constexpr int NPR = 2 * QT * NT;
    u32x4 ring[FD];
#pragma unroll
    for (int i = 0; i < FD; ++i) ring[i] = cx.read(base, (i / NT) * 16, (i % NT) * 32);
#pragma unroll
    for (int i = 0; i < NPR; ++i) {
      __builtin_amdgcn_sched_barrier(0x406);
      const u32x4 cur = ring[i % FD];
      if (i + FD < NPR) ring[i % FD] = cx.read(base, ((i + FD) / NT) * 16, ((i + FD) % NT) * 32);
      __builtin_amdgcn_sched_barrier(0x406);
      acc[i % NT] = M::mma(af[i / NT], cur, acc[i % NT]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };


  const int kr = myk < a.Sk ? myk : a.Sk - 1;
  const int64_t mkofs = MB ? (int64_t)kr * a.m_sk : 0;  // this lane's key in the mask view
  // MB, a mask constant over the query rows and heads (key padding, (B, 1, 1, Sk)): this lane's value
  // for the whole kernel.  Its loop then reads no mask and issues its tile loads where the unmasked
  // kernel does.
  const bool kinv = MB && a.m_sq == 0 && a.m_sh == 0;
  const float kmask = kinv ? mask_elem_l2(a, b * a.m_sb + mkofs) : 0.f;
  if (!roleB) {
    if (niter > 0) issue(0);
    if (niter > 1) issue(1);
    if (niter > 1) {
      if (l2w) wait_vmcnt<PER>();
      else wait_vmcnt<PER - 1>();
    } else {
      wait_vmcnt<0>();
    }
  }
  __syncthreads();
  float* st_epi = (float*)smem;  // [BNK keys][DQK] fp32 dk~ for the fused inverse transform
  // The two roles run separate loops with the same number of barriers (one per step), so each
  // role's registers (A: k~ and the dV accumulators, B: v and the dK~ accumulators) are live only
  // in its own branch.
  if (!roleB) {
    u32x4 kf[NKF];
    {
      const uint16_t* krow = (const uint16_t*)a.k + ((int64_t)(b * a.Hkv + hk) * a.Sk + kr) * DQK;
#pragma unroll
      for (int kk = 0; kk < NKF; ++kk) kf[kk] = *(const u32x4*)(krow + kk * 16 + g * 8);
      // a wait the compiler sees (the inline-asm waits for the tile loads are opaque to it):
      // without it these loads stay pending in its accounting, and it inserts vmcnt(15) .. vmcnt(0)
      // into the score products of every step, which also drains the tile loads issued a step
      // earlier.  Here it costs one wait for tile 1's loads.
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
    }
    f32x16 dv[NDV];
#pragma unroll
    for (int t = 0; t < NDV; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) dv[t][j] = 0.f;
    u32x4 pa0[2 * QT], pa1[2 * QT];  // bf16 P, alternating tiles
#pragma unroll
    for (int i = 0; i < 2 * QT; ++i) pa0[i] = pa1[i] = u32x4{0u, 0u, 0u, 0u};
    f32x16 s[QT];
    int cur_qt = qb0;  // query tile of step t
    // step t: S of tile t (products right after the barrier), the loads of tile t + 2, P of tile t,
    // then dV of tile t - 1 from the other P buffer
    auto astep = [&](int t, u32x4 (&pn)[2 * QT], u32x4 (&pp)[2 * QT]) {
      if (t < niter) {
        const char* st = smem + (t % NSTG) * STAGE;
        // S and P of tile t are the step's critical path (role B's next step needs P): role A runs
        // them above role B's priority and drops to the lowest for its dV products (dK/dV 1.5 %
        // faster than with A always below B; A above B throughout measured in between)
        __builtin_amdgcn_s_setprio(3);
        // MB: the mask of this lane's key at the 16 query rows of each sub-tile (rows past Sq, in the
        // last tile only, read row Sq - 1), loaded at the start of the step.  The compiler's wait for
        // them also drains every DMA issued before its use (it cannot see those), so the tile loads of
        // this step are issued after the exponentials instead, and that wait covers only tile t + 1,
        // which the step needs landed by its end anyway.
        float mlv[MB ? QT : 1][16];
        if constexpr (MB) {
          const int hq = h_first + (t / nper), q0 = (qb0 + t % nper) * BMQ;
          const int64_t rb = b * a.m_sb + hq * a.m_sh + mkofs;
          if (kinv) {  // one value per lane for the whole kernel, read before the loop
#pragma unroll
            for (int m = 0; m < QT; ++m)
#pragma unroll
              for (int i = 0; i < 16; ++i) mlv[m][i] = kmask;
          } else if (a.m_sq == 0) {  // a mask that does not vary with the query row: one read per step
            const float v = mask_elem_l2(a, rb);
#pragma unroll
            for (int m = 0; m < QT; ++m)
#pragma unroll
              for (int i = 0; i < 16; ++i) mlv[m][i] = v;
          } else {
#pragma unroll
            for (int m = 0; m < QT; ++m) {
              const int qm = q0 + 32 * m + g * 8;
              if (q0 + 32 * m + 31 < a.Sq) {  // every row inside: a per-lane base plus uniform row offsets
                const int64_t lb = rb + (int64_t)qm * a.m_sq;
#pragma unroll
                for (int G = 0; G < 4; ++G)
#pragma unroll
                  for (int e = 0; e < 4; ++e)
                    mlv[m][4 * G + e] = mask_elem_l2(a, lb + (int64_t)((G >> 1) * 16 + (G & 1) * 4 + e) * a.m_sq);
              } else {
#pragma unroll
                for (int G = 0; G < 4; ++G)
#pragma unroll
                  for (int e = 0; e < 4; ++e) {
                    const int q = qm + (G >> 1) * 16 + (G & 1) * 4 + e;
                    mlv[m][4 * G + e] = mask_elem_l2(a, rb + (int64_t)min(q, a.Sq - 1) * a.m_sq);
                  }
              }
            }
          }
        }
        // the rows' log2 lse, read ahead of the score products so that the exponentials do not wait
        // on them (0.5 % faster)
        const float* sL = (const float*)(st + SQ_BYTES + SO_BYTES);
        f32x4 lvp[QT][4];
#pragma unroll
        for (int m = 0; m < QT; ++m)
#pragma unroll
          for (int G = 0; G < 4; ++G) lvp[m][G] = *(const f32x4*)(sL + m * 32 + (G >> 1) * 16 + g * 8 + (G & 1) * 4);
        scores_s(st + rrq, kf, s);
        // the loads of tile t + 2 (its stage held tile t - 2, released by the last barrier) go out
        // between the score products and the exponentials: 1.4 % faster than after the P hand-off,
        // and every earlier point, inside the score products' chain, measured slower
        if ((!MB || kinv) && t + 2 < niter) issue(t + 2);
        const int q0 = cur_qt * BMQ;
        if (++cur_qt == nqt) cur_qt = qb0;
#pragma unroll
        for (int m = 0; m < QT; ++m) {
          const int q0m = q0 + 32 * m;
          if (__builtin_amdgcn_readfirstlane(a.causal && kw0 + 31 - off - q0m > 0)) {
            const int kd = myk - off - q0m - g * 8;
#pragma unroll
            for (int i = 0; i < 16; ++i) s[m][i] = masked_row(kd, i) ? -INFINITY : s[m][i];
          }
        }
        char* xb = xbuf + ((t & 1) * 4 + pw) * XBP;
#pragma unroll
        for (int m = 0; m < QT; ++m) {
          u32x4 ph[2];
#pragma unroll
          for (int G = 0; G < 4; ++G) {
            const f32x4 lv = lvp[m][G];
            f32x4 p;
            if constexpr (MB) {
#pragma unroll
              for (int e = 0; e < 4; ++e) p[e] = fast_exp2(fmaf(s[m][4 * G + e], sl2, mlv[m][4 * G + e]) - lv[e]);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) p[e] = fast_exp2(s[m][4 * G + e] * sl2 - lv[e]);
            }
            if constexpr (P32) {
              *(f32x4*)(xb + ((4 * m + G) * 64 + lane) * 16) = p;
            } else {
              ph[G >> 1][(G & 1) * 2] = pack_h2(p[0], p[1]);
              ph[G >> 1][(G & 1) * 2 + 1] = pack_h2(p[2], p[3]);
            }
            pn[2 * m + (G >> 1)][(G & 1) * 2] = pack2<HT>(p[0], p[1]);
            pn[2 * m + (G >> 1)][(G & 1) * 2 + 1] = pack2<HT>(p[2], p[3]);
          }
          if constexpr (!P32) {
            *(u32x4*)(xb + ((2 * m + 0) * 64 + lane) * 16) = ph[0];
            *(u32x4*)(xb + ((2 * m + 1) * 64 + lane) * 16) = ph[1];
          }
        }
        if (MB && !kinv && t + 2 < niter) issue(t + 2);
        __builtin_amdgcn_s_setprio(0);
      }
      if (t >= 1) products(dv, pp, smem + ((t - 1) % NSTG) * STAGE + SQ_BYTES + cro, co);
      if (t + 1 < niter) {  // tile t + 1 has landed: only tile t + 2's loads may be outstanding
        if (t + 2 < niter) {
          if (l2w) wait_vmcnt<PER>();
          else wait_vmcnt<PER - 1>();
        } else {
          wait_vmcnt<0>();
        }
      }
      __syncthreads();
    };
    for (int t = 0; t <= niter; t += 2) {
      astep(t, pa0, pa1);
      if (t + 1 <= niter) astep(t + 1, pa1, pa0);
    }
    if constexpr (QS) {
      float* dvp = a.dv_part + ((int64_t)jq * a.B * a.Hkv + bh) * a.Sk * DV;
#pragma unroll
      for (int t = 0; t < NDV; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = kw0 + c_row(j, g);
          if (key < a.Sk) dvp[(int64_t)key * DV + t * 32 + l32] = dv[t][j];
        }
    } else {
#pragma unroll
      for (int t = 0; t < NDV; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = kw0 + c_row(j, g), col = t * 32 + l32;
          if (key < a.Sk && col < a.dv_real)
            store_from_float_t<HT>(a.dv, b * a.dv_sb + hk * a.dv_sh + (int64_t)key * a.dv_ss + col, a.dv_dtype,
                                   dv[t][j]);
        }
    }
  } else {
    u32x4 vf[NVF];
    {
      const uint16_t* vrow = (const uint16_t*)a.v + b * a.v_sb + hk * a.v_sh + (int64_t)kr * a.v_ss;
#pragma unroll
      for (int kk = 0; kk < NVF; ++kk) vf[kk] = *(const u32x4*)(vrow + kk * 16 + g * 8);
    }
    f32x16 dk[NDK];
#pragma unroll
    for (int t = 0; t < NDK; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) dk[t][j] = 0.f;
    f32x16 dp[QT];
    int prev_h = h_first, prev_qt = qb0;  // head and query tile of step t - 1
    // the wave's key row in the packed dS (pe_internal.h), less its first stored 64-query block
    const int64_t ds_row = ds_row_base(kw0 >> 5, a.ds_e, a.ds_nqt, a.causal) - ds_first(kb, a.ds_e, a.causal);
    // role B's instructions go first when both waves of a SIMD are ready to issue, except while
    // role A forms S and P (priority 3 there, 0 elsewhere)
    __builtin_amdgcn_s_setprio(2);
    for (int t = 0; t <= niter; ++t) {
      if (t >= 1) {  // dS of tile t - 1 from A's P; store it; dK~ += dS^T q~
        const char* st = smem + ((t - 1) % NSTG) * STAGE;
        const float* sD = (const float*)(st + SQ_BYTES + SO_BYTES) + BMQ;
        const char* xb = xbuf + (((t - 1) & 1) * 4 + pw) * XBP;
        u32x4 dsf[2 * QT];
#pragma unroll
        for (int m = 0; m < QT; ++m) {
          u32x4 ph[2];
          if constexpr (!P32) {
            ph[0] = *(const u32x4*)(xb + ((2 * m + 0) * 64 + lane) * 16);
            ph[1] = *(const u32x4*)(xb + ((2 * m + 1) * 64 + lane) * 16);
          }
#pragma unroll
          for (int G = 0; G < 4; ++G) {
            f32x4 p;
            if constexpr (P32) {
              p = *(const f32x4*)(xb + ((4 * m + G) * 64 + lane) * 16);
            } else {
              float p0, p1, p2, p3;
              unpack_h2(ph[G >> 1][(G & 1) * 2], p0, p1);
              unpack_h2(ph[G >> 1][(G & 1) * 2 + 1], p2, p3);
              p = f32x4{p0, p1, p2, p3};
            }
            const f32x4 dd = *(const f32x4*)(sD + m * 32 + (G >> 1) * 16 + g * 8 + (G & 1) * 4);
            float ds[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) ds[e] = p[e] * (dp[m][4 * G + e] - dd[e]);
            dsf[2 * m + (G >> 1)][(G & 1) * 2] = pack2<HT>(ds[0], ds[1]);
            dsf[2 * m + (G >> 1)][(G & 1) * 2 + 1] = pack2<HT>(ds[2], ds[3]);
          }
        }
        const int h = prev_h, q0 = prev_qt * BMQ;
        if (++prev_qt == nqt) {
          prev_qt = qb0;
          ++prev_h;
        }
        char* blk = (char*)a.dS + ((int64_t)(b * a.Hq + h - a.bh0 * grp) * a.ds_head + ds_row + (q0 >> 6)) * 4096;
        const int mt = (q0 >> 5) & 1;  // 0 for 64-query tiles, which fill their block
        // dS is read once, by the dQ GEMM after this kernel: non-temporal stores keep it from
        // displacing the q~ / dO tiles that the other key blocks re-read (4 % of this kernel's
        // time; non-temporal loads of it in the dQ GEMM measured 35 % slower there)
#pragma unroll
        for (int i = 0; i < 2 * QT; ++i)
          __builtin_nontemporal_store(dsf[i], (u32x4*)(blk + ((mt * 2 + i) * 64 + lane) * 16));
        products(dk, dsf, st + crq, cq);
      }
      if (t < niter) scores_dp(smem + (t % NSTG) * STAGE + SQ_BYTES + rro, vf, dp);
      __syncthreads();  // role A waited for tile t + 1's loads before this barrier
    }
    if (a.fuse_inv && !QS) {
#pragma unroll
      for (int t = 0; t < NDK; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) st_epi[(pw * 32 + c_row(j, g)) * DQK + t * 32 + l32] = dk[t][j] * a.scale;
    } else {  // dk_t, or partial jq of it
      float* dkb = a.dk_t + ((int64_t)jq * a.B * a.Hkv + bh) * a.Sk * DQK;
#pragma unroll
      for (int t = 0; t < NDK; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = kw0 + c_row(j, g);
          if (key < a.Sk) dkb[(int64_t)key * DQK + t * 32 + l32] = dk[t][j] * a.scale;
        }
    }
  }

  if constexpr (!QS) dk_epilogue<HT, DQK>(a, st_epi, tid, b, hk, kb, bh, nkb);
}

// The query-head split of the pair kernel (a.qsplit > 1, grids with fewer key blocks than compute
// units): one workgroup of 512 threads per key block of (b, hk) adds the qsplit fp32 partials of
// dV and dK~ in slice order, stores dV in dv's dtype, and either runs the dK~ epilogue
// (a.fuse_inv) or leaves the sum in slice 0 of dk_t for the stand-alone inverse-transform kernels.
// Both paths see the same sums, so the fused and unfused gradients stay bitwise equal.  It runs as
// extra workgroups of the dQ GEMM's launch (the two are independent), on the compute units that a
// small dQ grid leaves idle.  st_epi: 128 x DQK floats of LDS.
template <int HT, int DQK, int DV>
__device__ __forceinline__ void dkdv_combine(const CoreArgs& a, int blk_id, float* st_epi) {
  constexpr int BNK = 128, NT = 512;
  const int tid = threadIdx.x;
  const int nkb = (a.Sk + BNK - 1) / BNK;
  int kb, bh;
  map_block(blk_id, nkb, a.nbh, false, kb, bh);
  bh += a.bh0;
  const int b = bh / a.Hkv, hk = bh % a.Hkv, k0 = kb * BNK;
  const int64_t units = (int64_t)a.B * a.Hkv;
  for (int i = tid; i < BNK * (DV / 4); i += NT) {
    const int r = i / (DV / 4), c = (i % (DV / 4)) * 4, key = k0 + r;
    if (key >= a.Sk) continue;
    f32x4 sum = *(const f32x4*)(a.dv_part + ((int64_t)bh * a.Sk + key) * DV + c);
    for (int j = 1; j < a.qsplit; ++j) sum += *(const f32x4*)(a.dv_part + ((j * units + bh) * a.Sk + key) * DV + c);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (c + e < a.dv_real)
        store_from_float_t<HT>(a.dv, b * a.dv_sb + hk * a.dv_sh + (int64_t)key * a.dv_ss + c + e, a.dv_dtype, sum[e]);
  }
  for (int i = tid; i < BNK * (DQK / 4); i += NT) {
    const int r = i / (DQK / 4), c = (i % (DQK / 4)) * 4, key = k0 + r;
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
    if (key < a.Sk) {
      float* d0 = a.dk_t + ((int64_t)bh * a.Sk + key) * DQK + c;
      sum = *(const f32x4*)d0;
      for (int j = 1; j < a.qsplit; ++j) sum += *(const f32x4*)(a.dk_t + ((j * units + bh) * a.Sk + key) * DQK + c);
      if (!a.fuse_inv) *(f32x4*)d0 = sum;
    }
    if (a.fuse_inv) *(f32x4*)(st_epi + r * DQK + c) = sum;
  }
  if (a.fuse_inv) dk_epilogue<HT, DQK>(a, st_epi, tid, b, hk, kb, bh, nkb);
}

// dQ~ = dS k~ as a GEMM over the dS^T rows the dK/dV kernel stored (no score recompute).  A
// workgroup owns 256 queries of one head; its 8 waves split them into 4 pairs of 32-query tiles x
// 2 halves of the dq~ columns, so every fragment read from LDS feeds two MFMAs (A: dS for 32
// queries x 16 keys, shared by the wave's column tiles; B: k~ for 16 keys x 32 columns, shared by
// its two query tiles) and the 128 accumulators per wave leave room for two waves per SIMD.  (Four
// waves of 128 queries x 128 columns in AGPRs at one wave per SIMD read one fragment per MFMA
// instead of 1.5, but measured 25 % slower, as each wave then waits on its own LDS reads and
// loads; that variant is not built.)  Each BK-key step stages dS^T (BK keys x 256 queries) and k~ (BK x DQK) in one slot of an NSTAGE ring,
// NSTAGE - 1 steps ahead: dS is read once from HBM, so the kernel streams it and needs several
// tiles in flight to cover the memory latency.  Both operands are read with the transpose load.
// Keys past a query's causal limit or past Sk hold no valid dS (never written), so on those tiles
// the A fragments are masked to zero.
__device__ __forceinline__ uint32_t keep_bf2(uint32_t v, bool lo, bool hi) {
  return (lo ? (v & 0xffffu) : 0u) | (hi ? (v & 0xffff0000u) : 0u);
}

// CDV > 0: the launch also carries the key blocks' dkdv_combine (value width CDV) as workgroups
// past the dQ grid
template <int HT, int DQK, int NW, int BK, int NSTAGE, int CDV>
__global__ __launch_bounds__(NW * 64, 1) void dq_gemm_kernel(CoreArgs a) {
  using M = MT<HT>;  // HT: the 16-bit operand type, bf16 (0) or fp16 (2)
  static_assert(NW == 8, "4 query groups x 2 column halves");
  constexpr int SZ = 1;  // tile swizzle kind (both tiles are only read with the transpose load)
  constexpr int NQG = NW / 2, QT = 8 / NQG;  // query groups; 32-query tiles per wave
  static_assert(NSTAGE >= 2 && NSTAGE <= 4, "ring depth");
  constexpr int BQ = 256;
  constexpr int NCK = DQK / 8, NCS = BQ / 8;
  constexpr int NTH = DQK / 64;  // 32-column tiles per wave
  // column tile of a wave's t-th accumulator: with an even count, wave dh takes cos tiles
  // dh*NTH/2 .. +NTH/2-1 and the matching sin tiles (+ DQK/64), so the inverse transform of a
  // column needs no exchange between waves
  auto ctile = [&](int t, int dhv) -> int {
    if constexpr (NTH % 2 == 0) {
      constexpr int H2 = NTH / 2;
      return t < H2 ? dhv * H2 + t : NTH + dhv * H2 + (t - H2);
    } else {
      return dhv * NTH + t;
    }
  };
  constexpr int SK_BYTES = BK * NCK * 16, SS_BYTES = BK * NCS * 16, STAGE = SK_BYTES + SS_BYTES;
  // DMA instructions one wave issues per step (k~ tile + dS tile)
  constexpr int PER = BK * NCK / (64 * NW) + BK * NCS / (64 * NW);
  static_assert(BK * NCS % (64 * NW) == 0, "dS tile must split into whole wave instructions");
  constexpr int EPI_BYTES = NTH % 2 == 0 ? 128 * DQK * 4 : 0;  // fused epilogue staging
  constexpr int SMEM = NSTAGE * STAGE > EPI_BYTES ? NSTAGE * STAGE : EPI_BYTES;
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int nqb = (a.Sq + BQ - 1) / BQ;
  if constexpr (CDV > 0) {
    static_assert(NW == 8 && SMEM >= 128 * DQK * 4, "the combine takes 512 threads and 128 x DQK floats");
    const int ndq = nqb * a.nbh * (a.Hq / a.Hkv);
    if ((int)blockIdx.x >= ndq) {
      dkdv_combine<HT, DQK, CDV>(a, (int)blockIdx.x - ndq, (float*)smem);
      return;
    }
  }
  int qb, bh;
  map_block(blockIdx.x, nqb, a.nbh * (a.Hq / a.Hkv), a.causal != 0, qb, bh);
  bh += a.bh0 * (a.Hq / a.Hkv);  // the head group's query heads
  const int b = bh / a.Hq, h = bh % a.Hq, hk = h / (a.Hq / a.Hkv);
  const int q0 = qb * BQ;
  const int qp = w % NQG, dh = w / NQG;
  const int qw = q0 + qp * QT * 32;  // this wave's QT*32 queries: tiles qw + 32 i
  const int off = a.causal_off;

  f32x16 acc[QT][NTH];
#pragma unroll
  for (int i = 0; i < QT; ++i)
#pragma unroll
    for (int t = 0; t < NTH; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[i][t][j] = 0.f;

  // per-lane fragment bases: the wave's two dS query tiles and its NTH k~ column tiles
  ColBase<NCS, SZ> cA[QT];
#pragma unroll
  for (int i = 0; i < QT; ++i) cA[i] = ColBase<NCS, SZ>(lane, qp * QT * 32 + i * 32);
  ColBase<NCK, SZ> cB[NTH];
#pragma unroll
  for (int t = 0; t < NTH; ++t) cB[t] = ColBase<NCK, SZ>(lane, ctile(t, dh) * 32);
  int kend = a.Sk;
  if (a.causal) kend = min(a.Sk, q0 + BQ + off);
  const int nkb = kend > 0 ? (kend + BK - 1) / BK : 0;
  const char* kbase = (const char*)((const uint16_t*)a.k + (int64_t)(b * a.Hkv + hk) * a.Sk * DQK);
  // the packed dS of this (b, h) (pe_internal.h): key row r of the block's 64-query blocks
  // j0 .. j0 + 3 (j0 = q0 / 64) starts at block ds_row_base(r) + j0 - ds_first(r / 4)
  const int j0 = q0 >> 6;
  const char* sbase = (const char*)a.dS + ((int64_t)(b * a.Hq + h - a.bh0 * (a.Hq / a.Hkv)) * a.ds_head + j0) * 4096;
  const int64_t krs = (int64_t)DQK * 2;
  // dS window for keys k0 .. k0+BK-1 and this block's 256 queries: LDS slot (row kl, physical chunk
  // pc) holds query chunk lc = pc ^ swz(kl) of key k0 + kl; its source is key row r = (k0 + kl) / 32
  // at 64-query block j0 + lc/8, chunk ((q>>1)*64 + (q&1)*32 + kl%32), q = lc % 8.  A DMA
  // instruction covers 64 / (BK / 8) = 256 / BK key rows of one 32-key row, so per instruction the
  // row base is wave-uniform (computed per step) and a lane's offset (lc/8) * 4096 + chunk is a
  // per-lane constant, computed once
  constexpr int NDS = BK * NCS / (64 * NW);
  uint32_t ds_off[NDS];
#pragma unroll
  for (int i = 0; i < NDS; ++i) {
    const int slot = (i * NW + w) * 64 + lane;
    const int kl = slot / NCS, pc = slot % NCS;
    const int lc = pc ^ swz<NCS, SZ>(kl);
    const int q = lc & 7;
    ds_off[i] = (uint32_t)((lc >> 3) * 4096 + ((q >> 1) * 64 + (q & 1) * 32 + (kl & 31)) * 16);
  }
  // key row (within the step) of DMA instruction i: slots (i * NW + w) * 64 .. +63 hold key rows
  // kl = slot / NCS of one 32-row group, (i * NW + w) * 64 / NCS / 32, the same for every wave when
  // NW * 64 / NCS divides 32
  static_assert((NW * 64 / NCS) <= 32 && 32 % (NW * 64 / NCS) == 0, "one 32-key row per DMA instruction");
  const DmaPlan<BK, NCK, NW, SZ> plan_k(w, lane, (uint32_t)krs);
  const uint32_t smem_l = lds_addr(smem);
  // tiles are issued in key order, so the packed row start ds_row_base(r) - ds_first(r / 4) of the
  // next tile's first key row is carried forward: row r + 1 starts nqt - ds_first((r + 1) / 4)
  // blocks after row r
  int iss_r = 0;
  int64_t iss_rs = 0;
  auto next_rs = [&](int r, int64_t rs) -> int64_t { return rs + a.ds_nqt - ds_first((r + 1) >> 2, a.ds_e, a.causal); };
  auto issue = [&](int kb) {
    char* st = smem + (kb % NSTAGE) * STAGE;
    const uint32_t stl = smem_l + (uint32_t)((kb % NSTAGE) * STAGE);
    const char* ksrc = kbase + (int64_t)kb * BK * krs;
    if (a.Sk - kb * BK >= BK) plan_k.full(ksrc, stl, w, (uint32_t)krs);
    else dma_tile<BK, NCK, NW, SZ>(st, ksrc, krs, a.Sk - kb * BK, w, lane);
    int64_t rs[BK / 32];  // row starts of the step's key rows iss_r .. iss_r + BK/32 - 1 (= kb * BK / 32 ..)
    rs[0] = iss_rs;
#pragma unroll
    for (int j = 1; j < BK / 32; ++j) rs[j] = next_rs(iss_r + j - 1, rs[j - 1]);
#pragma unroll
    for (int i = 0; i < NDS; ++i) {
      const int rr = ((i * NW + w) * 64 / NCS) / 32;  // key row of instruction i within the step
      dma16s(ds_off[i], sbase + rs[rr] * 4096, stl + SK_BYTES + (uint32_t)((i * NW + w) * 64 * 16));
    }
    iss_rs = next_rs(iss_r + BK / 32 - 1, rs[BK / 32 - 1]);
    iss_r += BK / 32;
  };
#pragma unroll
  for (int i = 0; i < NSTAGE - 1; ++i)
    if (i < nkb) issue(i);
  // One BK-key step.  Steps in which no key passes a query's causal limit or Sk (every step but the
  // last few of a causal block) run without masking; the rest (EDGE) mask every A fragment and,
  // for a wave whose queries all end before the step, multiply zeros.  Both loop bodies are
  // straight-line code, so the accumulators stay in place across iterations.
  auto step = [&](int kb, auto edge_tag) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    const int k0 = kb * BK;
    const char* sK = smem + (kb % NSTAGE) * STAGE;
    const char* sS = sK + SK_BYTES;
    // tile kb has landed once at most (steps issued after it) * PER loads are outstanding
    const int after = min(NSTAGE - 2, nkb - 1 - kb);
    if (after >= 2) wait_vmcnt<2 * PER>();
    else if (after == 1) wait_vmcnt<PER>();
    else wait_vmcnt<0>();
    __syncthreads();  // tile kb visible; every wave is done with slot (kb - 1) % NSTAGE
    // Fenced double buffer over the 16-key slices: region ks issues every read of slice ks + 1 and
    // then the products of slice ks, whose fragments were read one region earlier (left to itself
    // the scheduler waits on each read right before its product).
    u32x4 fa[2][QT], fb[2][NTH];
    auto read_slice = [&](int ks, u32x4 (&ra)[QT], u32x4 (&rb)[NTH]) {
#pragma unroll
      for (int i = 0; i < QT; ++i) ra[i] = cA[i].read(sS, ks * 16);
#pragma unroll
      for (int t = 0; t < NTH; ++t) rb[t] = cB[t].read(sK, ks * 16);
    };
    read_slice(0, fa[0], fb[0]);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      __builtin_amdgcn_sched_barrier(0);
      if (ks + 1 < BK / 16) read_slice(ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);  // the reads go out before this slice's products
      u32x4 af[QT];
#pragma unroll
      for (int i = 0; i < QT; ++i) af[i] = fa[ks & 1][i];
      if constexpr (EDGE) {
#pragma unroll
        for (int i = 0; i < QT; ++i) {
          // element e of lane (l32, g) is key k0 + ks*16 + g*8 + e of query qw + i*32 + l32
          const int kmax = a.causal ? min(qw + i * 32 + l32 + off, a.Sk - 1) : a.Sk - 1;
          const int lim = kmax - (k0 + ks * 16 + g * 8);
#pragma unroll
          for (int c = 0; c < 4; ++c) af[i][c] = keep_bf2(af[i][c], 2 * c <= lim, 2 * c + 1 <= lim);
        }
      }
#pragma unroll
      for (int t = 0; t < NTH; ++t)
#pragma unroll
        for (int i = 0; i < QT; ++i) acc[i][t] = M::mma(af[i], fb[ks & 1][t], acc[i][t]);
      if (ks == 0) {
        // the next tile's copies into slot (kb - 1) % NSTAGE (free since the barrier) go out
        // behind the first slice's products rather than straight after the barrier, where every
        // wave would issue them at once ahead of its first LDS reads (measured: dQ 6% faster),
        // at raised priority (another 1.5 %; priorities 2 and 3 measured no better)
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
        if (kb + NSTAGE - 1 < nkb) issue(kb + NSTAGE - 1);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // steps whose keys all lie at or below the causal limit of the block's first query and below Sk
  const int kfull = a.causal ? min(a.Sk, q0 + off + 1) : a.Sk;
  const int nfull = min(nkb, max(kfull, 0) / BK);
  int kb = 0;
  for (; kb < nfull; ++kb) step(kb, std::false_type{});
  for (; kb < nkb; ++kb) step(kb, std::true_type{});

  if constexpr (NTH % 2 == 0) {
    if (a.fuse_inv) {
      // inverse PoPE transform (no phase bias on queries): the scaled dq~ rows of two query pairs
      // at a time go through LDS, then one plain loop with a fixed dim c per thread
      const EpiPoPE& e = a.eq;
      const int Dr = DQK / 2;
      constexpr int Dr_c = DQK / 2;
      float* st = (float*)smem;  // [128 queries][DQK], one half of the block's rows at a time
      const int c = tid % Dr;
      // EU rows per trip, pipelined as in the dK epilogue but with shorter trips and no loads across
      // a staging barrier: the waves whose half is staged second still hold their accumulators
      constexpr int EU = 4;
      const int rstep = NW * 64 / Dr, ntrip = 256 / (EU * rstep);
      const int64_t xb = b * e.x_s[0] + h * e.x_s[1] + c * e.x_s[3];
      auto load_trip = [&](int R0, float (&xv)[EU]) {
#pragma unroll
        for (int u = 0; u < EU; ++u) {
          const int q = q0 + R0 + u * rstep;
          xv[u] = q < a.Sq ? load_as_float_t<HT>(e.x, xb + (int64_t)q * e.x_s[2], e.x_dtype) : 0.f;
        }
      };
      auto stage = [&](int half) {
        __syncthreads();
        if (((qp * QT * 32) >> 7) == half) {  // waves whose query rows lie in this half
#pragma unroll
          for (int i = 0; i < QT; ++i)
#pragma unroll
            for (int t = 0; t < NTH; ++t)
#pragma unroll
              for (int j = 0; j < 16; ++j)
                st[(((qp * QT * 32) & 127) + i * 32 + c_row(j, g)) * DQK + ctile(t, dh) * 32 + l32] = acc[i][t][j] * a.scale;
        }
        __syncthreads();
      };
      // vectorised rows; DC is the content width, 0, or DQK / 2 at DQK = 128 (the host fuses no other
      // split, and the split form only with vector views)
      auto epi_vec = [&](auto dc_tag) {
        constexpr int DC = decltype(dc_tag)::value;
        constexpr int Drv = (DQK - DC) / 2, CG = Drv / 8, RPP = NW * 64 / CG;
        const int c0 = (tid % CG) * 8, rr = tid / CG;
        float fr8[8], dl8[8], sdl8[8], sf8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          fr8[j] = a.freqs[c0 + j];
          dl8[j] = sdl8[j] = sf8[j] = 0.f;
        }
        for (int half = 0; half < 2; ++half) {
          stage(half);
          if constexpr (DC > 0)
            content_rows<HT, DQK, DC, NW * 64, 128>(e, st, tid, b * e.dxc_s[0] + h * e.dxc_s[1], q0 + half * 128, a.Sq);
          inv_pope_rows<HT, DQK, DC, NW * 64, 128, true>(e, st, tid, b * e.x_s[0] + h * e.x_s[1],
                                                     b * e.dx_s[0] + h * e.dx_s[1], q0 + half * 128, a.Sq, fr8,
                                                     dl8, false, a.qtab, sdl8, sf8);
        }
        if (e.part_freq) {  // fixed-order sums over the RPP row groups of each dim
          __syncthreads();
          float* red = st;
#pragma unroll
          for (int j = 0; j < 8; ++j) red[rr * Drv + c0 + j] = sf8[j];
          __syncthreads();
          const int64_t blk = (int64_t)bh * nqb + qb;
          if (tid < Drv) {
            float f0 = 0.f;
            for (int i = 0; i < RPP; ++i) f0 += red[i * Drv + tid];
            e.part_freq[blk * Drv + tid] = f0;
          }
        }
      };
      if constexpr (DQK == 128) {  // split form: fused only at width 128, with vector views
        if (a.qtab && a.Dc == DQK / 2) {
          epi_vec(std::integral_constant<int, DQK / 2>{});
          return;
        }
      }
      if (epi_vec_ok(e, 0) && a.qtab) {  // the host provides the query phase table with the fused form
        epi_vec(std::integral_constant<int, 0>{});
        return;
      }
      float xv[EU], xn[EU];
      const float fr = a.freqs[c];
      float sf = 0.f;
#pragma unroll 1
      for (int it = 0; it < ntrip; ++it) {
        const int R0 = tid / Dr + it * EU * rstep;
        if (it % (ntrip / 2) == 0) {
          stage(it / (ntrip / 2));
          load_trip(R0, xv);
        }
        if ((it + 1) % (ntrip / 2) != 0) load_trip(R0 + EU * rstep, xn);
#pragma unroll
        for (int u = 0; u < EU; ++u) {
          const int R = R0 + u * rstep, q = q0 + R;
          if (q < a.Sq) {
            const int r = R & 127;
            const float pos = pe_pos(e.start_pos + q, e.pos_round);
            float dx;
            const float dph = inv_pope_elem(xv[u], pos, fr, 0.f, false, st[r * DQK + c], st[r * DQK + Dr + c], dx);
            store_from_float_t<HT>(e.dx, b * e.dx_s[0] + h * e.dx_s[1] + (int64_t)q * e.dx_s[2] + c * e.dx_s[3],
                             e.dx_dtype, dx);
            sf += pos * dph;
          }
        }
#pragma unroll
        for (int u = 0; u < EU; ++u) xv[u] = xn[u];
      }
      if (e.part_freq) {
        __syncthreads();
        float* red = st;
        const int nt = NW * 64 / Dr;
        red[(tid / Dr) * Dr + c] = sf;
        __syncthreads();
        const int64_t blk = (int64_t)bh * nqb + qb;
        if (tid < Dr) {
          float f0 = 0.f;
          for (int i = 0; i < nt; ++i) f0 += red[i * Dr + tid];
          e.part_freq[blk * Dr + tid] = f0;
        }
      }
      return;
    }
  }
  if constexpr (DQK == 64) {
    if (a.rope_fuse) {
      // RoPE / no-PE gradient: the scaled dq~ rows of the block's 256 queries go through LDS (the
      // ring is free once every wave has passed the barrier), 8 threads per row
      static_assert(SMEM >= 256 * 64 * 4, "staged dq~ rows fit the ring");
      float* st = (float*)smem;  // [256 queries][64]
      rope_epi_rows<HT, NW * 64, 256>(a, a.eq, st, tid, q0, a.Sq, b, h, [&] {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < QT; ++i)
#pragma unroll
          for (int t = 0; t < NTH; ++t)
#pragma unroll
            for (int j = 0; j < 16; ++j)
              st[(qp * QT * 32 + i * 32 + c_row(j, g)) * DQK + ctile(t, dh) * 32 + l32] = acc[i][t][j] * a.scale;
        __syncthreads();
      });
      return;
    }
  }
  float* dqb = a.dq_t + (int64_t)(b * a.Hq + h) * a.Sq * DQK;
#pragma unroll
  for (int i = 0; i < QT; ++i)
#pragma unroll
    for (int t = 0; t < NTH; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int q = qw + i * 32 + c_row(j, g);
        if (q < a.Sq) dqb[(int64_t)q * DQK + ctile(t, dh) * 32 + l32] = acc[i][t][j] * a.scale;
      }
}

// the generic kernels: fp32 operands, and the explicit-mask instantiations (MB) of fp32 and of the
// 16-bit widths outside the pair kernel's
template <int DT, int DQK, int DV, bool MB>
static int run_bwd_generic(int which, const CoreArgs& a, hipStream_t s) {
  constexpr int NW = 4, BMQ = 32, BN = 32;
  if (which == 0) {
    const int nkb = (a.Sk + NW * 32 - 1) / (NW * 32);
    hipLaunchKernelGGL((dkdv_kernel<DT, DQK, DV, BMQ, NW, MB>), dim3(nkb * a.nbh), dim3(NW * 64), 0, s, a);
  } else {
    const int nqb = (a.Sq + NW * 32 - 1) / (NW * 32);
    hipLaunchKernelGGL((dq_kernel<DT, DQK, DV, BN, NW, MB>), dim3(nqb * a.nbh * (a.Hq / a.Hkv)), dim3(NW * 64), 0, s, a);
  }
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

template <int DT, int DQK, int DV>
static int run_bwd(int which, const CoreArgs& a, hipStream_t s) {
  constexpr int NW = 4;
  constexpr bool PAIR = DT != 1 && (DQK == 128 || DQK == 256) && (DV == 128 || DV == 64);
  if constexpr (PAIR) {
    if (a.mask) {  // explicit mask: the pair kernel's mask instantiation (no query-head split), then the dQ GEMM
      if (which == 0) {
        constexpr int QT = DQK == 128 && DV == 64 && DT != 2 ? 2 : 1;
        const int nkb = (a.Sk + NW * 32 - 1) / (NW * 32);
        hipLaunchKernelGGL((dkdv_pair_kernel<DT, DQK, DV, QT, false, true>), dim3(nkb * a.nbh), dim3(512), 0, s, a);
      } else {
        const int nqb = (a.Sq + 255) / 256;
        hipLaunchKernelGGL((dq_gemm_kernel<DT, DQK, 8, 32, 4, 0>), dim3(nqb * a.nbh * (a.Hq / a.Hkv)), dim3(8 * 64), 0, s, a);
      }
      return hipGetLastError() == hipSuccess ? 0 : -7;
    }
  } else {
    if (a.mask) return run_bwd_generic<DT, DQK, DV, true>(which, a, s);
  }
  if constexpr (DT != 1) {
    if (which == 0) {
      const int nkb = (a.Sk + NW * 32 - 1) / (NW * 32);
      if constexpr ((DQK == 128 || DQK == 256) && (DV == 128 || DV == 64)) {
        // two waves per SIMD (role-split pairs); the one-wave kernel serves the other widths (at QK
        // width 64 / V width 64 the pair kernel with 64-query tiles measured 2 % slower)
        // 64-query tiles where they fit the LDS (QK width 128, V width 64: the ~125M GPT shape and the
        // split training form), which halves the per-step barriers and waits per product; on fp16
        // operands the fp32 P exchange of 64-query tiles would not fit (162 KiB), so 32-query tiles
        constexpr int QT = DQK == 128 && DV == 64 && DT != 2 ? 2 : 1;
        if (a.qsplit > 1)
          hipLaunchKernelGGL((dkdv_pair_kernel<DT, DQK, DV, QT, true>), dim3(nkb * a.nbh * a.qsplit), dim3(512), 0, s, a);
        else
          hipLaunchKernelGGL((dkdv_pair_kernel<DT, DQK, DV, QT, false>), dim3(nkb * a.nbh), dim3(512), 0, s, a);
      } else {
        hipLaunchKernelGGL((dkdv_bf16_kernel<DT, DQK, DV, NW>), dim3(nkb * a.nbh), dim3(NW * 64), 0, s, a);
      }
    } else {
      const int nqb = (a.Sq + 255) / 256;
      // wide operands: 32-key steps in a 4-deep ring (three steps of loads in flight) measured
      // 4 % faster than 64-key steps double-buffered or a 3-deep ring of 32-key steps; the narrow
      // 64-wide k~ (a 32-key tile of it is less than one DMA instruction per wave) keeps 64-key
      // steps double-buffered
      constexpr bool TW = DQK == 256 || DQK == 128;
      const int ndq = nqb * a.nbh * (a.Hq / a.Hkv);
      if constexpr ((DQK == 128 || DQK == 256) && (DV == 128 || DV == 64)) {
        if (a.qsplit > 1) {  // with the pair kernel's partials to combine, one workgroup per key block
          const int nkb = (a.Sk + 127) / 128;
          hipLaunchKernelGGL((dq_gemm_kernel<DT, DQK, 8, 32, 4, DV>), dim3(ndq + nkb * a.nbh), dim3(8 * 64), 0, s, a);
          return hipGetLastError() == hipSuccess ? 0 : -7;
        }
      }
      hipLaunchKernelGGL((dq_gemm_kernel<DT, DQK, 8, (TW ? 32 : 64), (TW ? 4 : 2), 0>), dim3(ndq), dim3(8 * 64), 0, s, a);
    }
    return hipGetLastError() == hipSuccess ? 0 : -7;
  } else {
    return run_bwd_generic<DT, DQK, DV, false>(which, a, s);
  }
}

template <int DT>
static int bwd_dt(int which, int dqk, int dv, const CoreArgs& a, hipStream_t s) {
  if (dqk == 64 && dv == 64) return run_bwd<DT, 64, 64>(which, a, s);
  if (dqk == 64 && dv == 128) return run_bwd<DT, 64, 128>(which, a, s);
  if (dqk == 128 && dv == 64) return run_bwd<DT, 128, 64>(which, a, s);
  if (dqk == 128 && dv == 128) return run_bwd<DT, 128, 128>(which, a, s);
  if (dqk == 256 && dv == 64) return run_bwd<DT, 256, 64>(which, a, s);
  if (dqk == 256 && dv == 128) return run_bwd<DT, 256, 128>(which, a, s);
  return -3;
}

// dt: 0 bf16, 1 fp32, 2 fp16 operands
int launch_bwd_dkdv(int dt, int dqk, int dv, const CoreArgs& a, hipStream_t s) {
  if (dt == 0) return bwd_dt<0>(0, dqk, dv, a, s);
  if (dt == 2) return bwd_dt<2>(0, dqk, dv, a, s);
  return bwd_dt<1>(0, dqk, dv, a, s);
}

int launch_bwd_dq(int dt, int dqk, int dv, const CoreArgs& a, hipStream_t s) {
  if (dt == 0) return bwd_dt<0>(1, dqk, dv, a, s);
  if (dt == 2) return bwd_dt<2>(1, dqk, dv, a, s);
  return bwd_dt<1>(1, dqk, dv, a, s);
}

}  // namespace pe
