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
      const bool ok = q0 + tid < a.Sq;
      const float lv = ok ? a.lse_in[r0 + tid] : INFINITY;
      sL[tid] = lv == -INFINITY ? INFINITY : lv * LOG2E;
      sD[tid] = ok ? a.Di[r0 + tid] : 0.f;
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
  float lse2 = INFINITY, Dq = 0.f;
  if (myq < a.Sq) {
    const float lv = a.lse_in[rowq];
    lse2 = lv == -INFINITY ? INFINITY : lv * LOG2E;
    Dq = a.Di[rowq];
  }
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

template <int DT, int DQK, int DV>
static int run_bwd(int which, const CoreArgs& a, hipStream_t s) {
  constexpr int NW = 4;
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
