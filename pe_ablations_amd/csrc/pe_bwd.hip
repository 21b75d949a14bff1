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

template <int DT, int DQK, int DV, int BMQ, int NW>
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
  map_block(blockIdx.x, nkb, a.B * a.Hkv, false, kb, bh);
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
      sL[tid] = a.L2[p0 + tid];
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
        float p = exp2f(s[j] * sl2 - sL[qi]);
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
#pragma unroll
    for (int t = 0; t < NDV; ++t)
#pragma unroll
      for (int ks = 0; ks < NPF; ++ks)
        dv[t] = M::mma(pf[ks], lds_col_frag<DT, NCO>(sO, ks * KC, t * 32, lane), dv[t]);
#pragma unroll
    for (int t = 0; t < NDK; ++t)
#pragma unroll
      for (int ks = 0; ks < NPF; ++ks)
        dk[t] = M::mma(dsf[ks], lds_col_frag<DT, NCQ>(sQ, ks * KC, t * 32, lane), dk[t]);
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

template <int DT, int DQK, int DV, int BN, int NW>
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
  map_block(blockIdx.x, nqb, a.B * a.Hq, a.causal != 0, qb, bh);
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
  const float lse2 = a.L2[prow], Dq = a.Di[prow];
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
        float p = exp2f(s[j] * sl2 - lse2);
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
    for (int t = 0; t < NDQ; ++t)
#pragma unroll
      for (int ks = 0; ks < NPF; ++ks)
        dq[t] = M::mma(dsf[ks], lds_col_frag<DT, NCK>(sK, ks * KC, t * 32, lane), dq[t]);
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
// 256-wide dk~/dq~ take 128 registers) and stream 64-row tiles through LDS with direct
// global->LDS loads into a double buffer (one barrier per tile, no prefetch registers).  A tile
// is consumed as two 32-row halves so that only one 32x32 score tile and its packed bf16 copy are
// live at a time.
// ---------------------------------------------------------------------------------------------

// dK~/dV: a workgroup owns 32*NW keys of one kv head; wave w keeps k~ and v of its 32 keys as MFMA
// B operands in registers and walks every visible 64-query block of every query head of its GQA
// group.  Per tile the LDS stage holds q~ (64 x DQK), dO (64 x DV) and the rows' lse / Di.
template <int DQK, int DV, int NW>
__global__ __launch_bounds__(NW * 64, 1) void dkdv_bf16_kernel(CoreArgs a) {
  using M = MT<0>;
  constexpr int BMQ = 64, BNK = NW * 32;
  constexpr int NCQ = DQK / 8, NCO = DV / 8;
  constexpr int NKF = DQK / 16, NVF = DV / 16, NDK = DQK / 32, NDV = DV / 32;
  constexpr int SQ_BYTES = BMQ * NCQ * 16, SO_BYTES = BMQ * NCO * 16;
  constexpr int STAGE = SQ_BYTES + SO_BYTES + 2 * BMQ * 4;
  __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int nkb = (a.Sk + BNK - 1) / BNK;
  int kb, bh;
  map_block(blockIdx.x, nkb, a.B * a.Hkv, false, kb, bh);
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
  const int64_t qrs = (int64_t)DQK * 2, ors = (int64_t)DV * 2;

  // stage one (head, query block) tile: q~ and dO rows (swizzled), then the rows' log2-scaled
  // lse and Di from the padded per-row arrays (lanes 0-15 and 16-31 of wave 0, one chunk each)
  auto issue = [&](int it, char* st) {
    const int h = hk * grp + it / nper;
    const int q0 = (qb0 + it % nper) * BMQ;
    const int64_t r0 = (int64_t)(b * a.Hq + h) * a.Sq + q0;
    dma_tile<BMQ, NCQ, NW>(st, (const char*)a.q + r0 * qrs, qrs, a.Sq - q0, w, lane);
    dma_tile<BMQ, NCO, NW>(st + SQ_BYTES, (const char*)a.dO + r0 * ors, ors, a.Sq - q0, w, lane);
    if (w == 0) {
      const int64_t p0 = (int64_t)(b * a.Hq + h) * a.sq_pad + q0;
      const float* src = (lane < 16 ? a.L2 : a.Di) + p0 + (lane & 15) * 4;
      if (lane < 32)
        __builtin_amdgcn_global_load_lds((const void*)src,
                                         (__attribute__((address_space(3))) void*)(st + SQ_BYTES + SO_BYTES), 16, 0, 0);
    }
  };

  if (niter > 0) issue(0, smem);
  for (int it = 0; it < niter; ++it) {
    char* st = smem + (it & 1) * STAGE;
    const int q0 = (qb0 + it % nper) * BMQ;
    dma_wait();
    __syncthreads();
    if (it + 1 < niter) issue(it + 1, smem + ((it + 1) & 1) * STAGE);
    if (a.causal && kw0 > q0 + BMQ - 1 + off) continue;  // every key of this wave is after every query
    const char* sQ = st;
    const char* sO = st + SQ_BYTES;
    const float* sL = (const float*)(st + SQ_BYTES + SO_BYTES);
    const float* sD = sL + BMQ;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int qm = q0 + mt * 32;
      if (a.causal && kw0 > qm + 31 + off) continue;
      if (qm >= a.Sq) continue;
      f32x16 s, dp;
#pragma unroll
      for (int j = 0; j < 16; ++j) { s[j] = 0.f; dp[j] = 0.f; }
      const int row = mt * 32 + perm_row<0>(l32);
#pragma unroll
      for (int kk = 0; kk < NKF; ++kk) s = M::mma(lds_row_frag<NCQ>(sQ, row, 2 * kk + g), kf[kk], s);
#pragma unroll
      for (int kk = 0; kk < NVF; ++kk) dp = M::mma(lds_row_frag<NCO>(sO, row, 2 * kk + g), vf[kk], dp);
      // query rows of value j: mt*32 + c_logical(j, g) = mt*32 + (j/8)*16 + g*8 + j%8
      const bool edge = a.causal && kw0 + 31 > qm + off;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int qi0 = mt * 32 + hh * 16 + g * 8;
        const f32x4 l0 = *(const f32x4*)(sL + qi0), l1 = *(const f32x4*)(sL + qi0 + 4);
        const f32x4 d0 = *(const f32x4*)(sD + qi0), d1 = *(const f32x4*)(sD + qi0 + 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = hh * 8 + e;
          const float lv = e < 4 ? l0[e] : l1[e - 4];
          const float dd = e < 4 ? d0[e] : d1[e - 4];
          // rows past Sq carry lse = +inf, so p = 0 there without a test
          float p = fast_exp2(s[j] * sl2 - lv);
          if (edge && myk > q0 + qi0 + e + off) p = 0.f;
          s[j] = p;
          dp[j] = p * (dp[j] - dd);
        }
      }
      u32x4 pf[2], dsf[2];
#pragma unroll
      for (int si = 0; si < 2; ++si) {
        pf[si] = M::pack(s, si * 8);
        dsf[si] = M::pack(dp, si * 8);
      }
#pragma unroll
      for (int t = 0; t < NDV; ++t)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          dv[t] = M::mma(pf[ks], lds_col_frag<0, NCO>(sO, mt * 32 + ks * 16, t * 32, lane), dv[t]);
#pragma unroll
      for (int t = 0; t < NDK; ++t)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          dk[t] = M::mma(dsf[ks], lds_col_frag<0, NCQ>(sQ, mt * 32 + ks * 16, t * 32, lane), dk[t]);
    }
  }

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
// dQ~: a workgroup owns 32*NW queries of one head; wave w keeps q~ and dO of its 32 queries as MFMA
// B operands and walks the visible 64-key tiles of k~ and v.  S^T and dP^T come out with queries
// across lanes, so each lane's lse / Di are scalars; dS is the A operand of dq~ = dS k~ with k~
// read by the transpose load.
template <int DQK, int DV, int NW>
__global__ __launch_bounds__(NW * 64, 1) void dq_bf16_kernel(CoreArgs a) {
  using M = MT<0>;
  constexpr int BN = 64, BM = NW * 32;
  constexpr int NCK = DQK / 8, NCV = DV / 8;
  constexpr int NQF = DQK / 16, NVF = DV / 16, NDQ = DQK / 32;
  constexpr int SK_BYTES = BN * NCK * 16, SV_BYTES = BN * NCV * 16, STAGE = SK_BYTES + SV_BYTES;
  __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int nqb = (a.Sq + BM - 1) / BM;
  int qb, bh;
  map_block(blockIdx.x, nqb, a.B * a.Hq, a.causal != 0, qb, bh);
  const int b = bh / a.Hq, h = bh % a.Hq, hk = h / (a.Hq / a.Hkv);
  const int q0 = qb * BM, qw = q0 + w * 32, myq = qw + l32;
  const int off = a.causal_off;

  u32x4 qf[NQF], of[NVF];
  {
    const int64_t rowq = (int64_t)(b * a.Hq + h) * a.Sq + (myq < a.Sq ? myq : a.Sq - 1);
    const uint16_t* qrow = (const uint16_t*)a.q + rowq * DQK;
    const uint16_t* orow = (const uint16_t*)a.dO + rowq * DV;
#pragma unroll
    for (int kk = 0; kk < NQF; ++kk) qf[kk] = *(const u32x4*)(qrow + kk * 16 + g * 8);
#pragma unroll
    for (int kk = 0; kk < NVF; ++kk) of[kk] = *(const u32x4*)(orow + kk * 16 + g * 8);
  }
  const int64_t prow = (int64_t)(b * a.Hq + h) * a.sq_pad + myq;
  const float lse2 = a.L2[prow], Dq = a.Di[prow];
  f32x16 dq[NDQ];
#pragma unroll
  for (int t = 0; t < NDQ; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) dq[t][j] = 0.f;

  int kend = a.Sk;
  if (a.causal) kend = min(a.Sk, q0 + BM + off);
  const int nkb = kend > 0 ? (kend + BN - 1) / BN : 0;
  const char* kbase = (const char*)((const uint16_t*)a.k + (int64_t)(b * a.Hkv + hk) * a.Sk * DQK);
  const char* vbase = (const char*)((const uint16_t*)a.v + b * a.v_sb + hk * a.v_sh);
  const int64_t krs = (int64_t)DQK * 2, vrs = a.v_ss * 2;
  const float sl2 = a.scale * LOG2E;

  if (nkb > 0) {
    dma_tile<BN, NCK, NW>(smem, kbase, krs, a.Sk, w, lane);
    dma_tile<BN, NCV, NW>(smem + SK_BYTES, vbase, vrs, a.Sk, w, lane);
  }
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * BN;
    const char* sK = smem + (kb & 1) * STAGE;
    const char* sV = sK + SK_BYTES;
    dma_wait();
    __syncthreads();
    if (kb + 1 < nkb) {
      char* nK = smem + ((kb + 1) & 1) * STAGE;
      dma_tile<BN, NCK, NW>(nK, kbase + (int64_t)(k0 + BN) * krs, krs, a.Sk - k0 - BN, w, lane);
      dma_tile<BN, NCV, NW>(nK + SK_BYTES, vbase + (int64_t)(k0 + BN) * vrs, vrs, a.Sk - k0 - BN, w, lane);
    }
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int kn = k0 + nt * 32;
      if (a.causal && kn > qw + 31 + off) continue;
      if (kn >= a.Sk) continue;
      f32x16 s, dp;
#pragma unroll
      for (int j = 0; j < 16; ++j) { s[j] = 0.f; dp[j] = 0.f; }
      const int row = nt * 32 + perm_row<0>(l32);
#pragma unroll
      for (int kk = 0; kk < NQF; ++kk) s = M::mma(lds_row_frag<NCK>(sK, row, 2 * kk + g), qf[kk], s);
#pragma unroll
      for (int kk = 0; kk < NVF; ++kk) dp = M::mma(lds_row_frag<NCV>(sV, row, 2 * kk + g), of[kk], dp);
      const bool edge = (a.causal && kn + 31 > qw + off) || (kn + 32 > a.Sk);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float p = fast_exp2(s[j] * sl2 - lse2);
        if (edge) {
          const int key = kn + c_logical<0>(j, g);
          if (key >= a.Sk || (a.causal && key > myq + off)) p = 0.f;
        }
        dp[j] = p * (dp[j] - Dq);
      }
      u32x4 dsf[2];
#pragma unroll
      for (int si = 0; si < 2; ++si) dsf[si] = M::pack(dp, si * 8);
#pragma unroll
      for (int t = 0; t < NDQ; ++t)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          dq[t] = M::mma(dsf[ks], lds_col_frag<0, NCK>(sK, nt * 32 + ks * 16, t * 32, lane), dq[t]);
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

template <int DT, int DQK, int DV>
static int run_bwd(int which, const CoreArgs& a, hipStream_t s) {
  constexpr int NW = 4;
  if constexpr (DT == 0) {
    if (which == 0) {
      const int nkb = (a.Sk + NW * 32 - 1) / (NW * 32);
      hipLaunchKernelGGL((dkdv_bf16_kernel<DQK, DV, NW>), dim3(nkb * a.B * a.Hkv), dim3(NW * 64), 0, s, a);
    } else {
      const int nqb = (a.Sq + NW * 32 - 1) / (NW * 32);
      hipLaunchKernelGGL((dq_bf16_kernel<DQK, DV, NW>), dim3(nqb * a.B * a.Hq), dim3(NW * 64), 0, s, a);
    }
    return hipGetLastError() == hipSuccess ? 0 : -7;
  }
  constexpr int BMQ = (DT == 0 && DQK <= 128) ? 64 : 32;
  constexpr int BN = DT == 0 ? 64 : 32;
  if (which == 0) {
    const int nkb = (a.Sk + NW * 32 - 1) / (NW * 32);
    hipLaunchKernelGGL((dkdv_kernel<DT, DQK, DV, BMQ, NW>), dim3(nkb * a.B * a.Hkv), dim3(NW * 64), 0, s, a);
  } else {
    const int nqb = (a.Sq + NW * 32 - 1) / (NW * 32);
    hipLaunchKernelGGL((dq_kernel<DT, DQK, DV, BN, NW>), dim3(nqb * a.B * a.Hq), dim3(NW * 64), 0, s, a);
  }
  return hipGetLastError() == hipSuccess ? 0 : -7;
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

int launch_bwd_dkdv(int dt, int dqk, int dv, const CoreArgs& a, hipStream_t s) {
  return dt == 0 ? bwd_dt<0>(0, dqk, dv, a, s) : bwd_dt<1>(0, dqk, dv, a, s);
}

int launch_bwd_dq(int dt, int dqk, int dv, const CoreArgs& a, hipStream_t s) {
  return dt == 0 ? bwd_dt<0>(1, dqk, dv, a, s) : bwd_dt<1>(1, dqk, dv, a, s);
}

}  // namespace pe
