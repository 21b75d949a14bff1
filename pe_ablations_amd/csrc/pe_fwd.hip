// Causal attention forward over transformed operands (q~, k~ of width DQK; v of width DV) for
// gfx950.  One workgroup = NW waves = NW*32 query rows; each wave keeps its 32 q~ rows in
// registers as the MFMA B operand and streams BN-key blocks of k~ and v through LDS.
//
// Per key block, per wave:  S^T = k~ q~^T  (A = k~ rows from LDS, C: rows = keys, cols = queries),
// online softmax with the key axis inside each lane (row max needs one lane^32 exchange),
// O^T += v^T P^T  (A = v read with the transpose load, B = P^T straight from the C registers).
// The scores are the reference's SDPA scores on [content | mu cos | mu sin] operands
// (src/model/fpope_attention.py:166-177, src/model/fpope.py:409-417).
#include "pe_common.h"
#include "pe_internal.h"

namespace pe {

// MB: the explicit-mask instantiation (any operand type), which adds mask_l2 to every score.
template <int DT, int DQK, int DV, int BN, int NW, bool MB>
__global__ __launch_bounds__(NW * 64, 1) void fwd_kernel(CoreArgs a, int o_vec) {
  using E = typename Elem<DT>::T;
  using M = MT<DT>;
  constexpr int KC = M::KC, EPL = M::EPL, ESZ = M::ESZ;
  constexpr int BM = NW * 32, NT = NW * 64;
  constexpr int NCK = DQK * ESZ / 16, NCV = DV * ESZ / 16;
  constexpr int NQF = DQK / KC, NKT = BN / 32, NPF = BN / KC, NOT = DV / 32, SPT = 32 / KC;
  constexpr int SK_BYTES = BN * NCK * 16, SV_BYTES = BN * NCV * 16;
  constexpr int SO_STRIDE = DV * ESZ + 16;
  constexpr int SO_BYTES = BM * SO_STRIDE;
  constexpr int SMEM = (SK_BYTES + SV_BYTES) > SO_BYTES ? (SK_BYTES + SV_BYTES) : SO_BYTES;
  __shared__ __attribute__((aligned(16))) char smem[SMEM];
  char* sK = smem;
  char* sV = smem + SK_BYTES;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int nqb = (a.Sq + BM - 1) / BM;
  int qb, bh;
  map_block(blockIdx.x, nqb, a.B * a.Hq, a.causal != 0, qb, bh);
  const int b = bh / a.Hq, h = bh % a.Hq, hk = h / (a.Hq / a.Hkv);
  const int q0 = qb * BM, qw = q0 + w * 32, myq = qw + l32;
  const int off = a.causal_off;

  u32x4 qf[NQF];
  {
    const E* qrow = (const E*)a.q + ((int64_t)(b * a.Hq + h) * a.Sq + (myq < a.Sq ? myq : 0)) * DQK;
#pragma unroll
    for (int kk = 0; kk < NQF; ++kk) {
      u32x4 z = {0u, 0u, 0u, 0u};
      qf[kk] = myq < a.Sq ? *(const u32x4*)(qrow + kk * KC + g * EPL) : z;
    }
  }

  int kend = a.Sk;
  if (a.causal) kend = min(a.Sk, q0 + BM + off);
  const int nkb = kend > 0 ? (kend + BN - 1) / BN : 0;
  const char* kbase = (const char*)((const E*)a.k + (int64_t)(b * a.Hkv + hk) * a.Sk * DQK);
  const char* vbase = (const char*)((const E*)a.v + b * a.v_sb + hk * a.v_sh);
  const int64_t krs = (int64_t)DQK * ESZ, vrs = a.v_ss * ESZ;

  const RowFrags<NCK> rk(perm_row<0>(l32), g);  // k~ row fragments (rows nt*32 + perm_row(l32))
  const ColFrags<NCV> cv(lane);                  // v transpose fragments
  f32x16 o[NOT];
#pragma unroll
  for (int t = 0; t < NOT; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[t][j] = 0.f;
  float m = -1e30f, l = 0.f;
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
    if (a.causal && k0 > qw + 31 + off) continue;  // whole block above this wave's diagonal

    f32x16 s[NKT];
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt) {
#pragma unroll
      for (int j = 0; j < 16; ++j) s[nt][j] = 0.f;
      const int row = nt * 32 + perm_row<DT>(l32);
#pragma unroll
      for (int kk = 0; kk < NQF; ++kk)
        s[nt] = M::mma(lds_row_frag<NCK>(sK, row, 2 * kk + g), qf[kk], s[nt]);
    }
    const bool edge = (a.causal && k0 + BN - 1 > qw + off) || (k0 + BN > a.Sk);
    float mx = m;
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float x = s[nt][j] * sl2;
        if constexpr (MB) x += mask_l2(a, b, h, myq, k0 + nt * 32 + c_logical<DT>(j, g));
        if (edge) {
          const int key = k0 + nt * 32 + c_logical<DT>(j, g);
          if (key >= a.Sk || (a.causal && key > myq + off)) x = -INFINITY;
        }
        s[nt][j] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, xor32(mx));
    const float alpha = exp2f(m - mx);
    m = mx;
    float rs = 0.f;
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float p = exp2f(s[nt][j] - m);
        s[nt][j] = p;
        rs += p;
      }
    l = l * alpha + rs;
#pragma unroll
    for (int t = 0; t < NOT; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[t][j] *= alpha;
    u32x4 pf[NPF];
#pragma unroll
    for (int ks = 0; ks < NPF; ++ks) pf[ks] = M::pack(s[ks / SPT], (ks % SPT) * EPL);
#pragma unroll
    for (int t = 0; t < NOT; ++t)
#pragma unroll
      for (int ks = 0; ks < NPF; ++ks)
        o[t] = M::mma(lds_col_frag<DT, NCV>(sV, ks * KC, t * 32, lane), pf[ks], o[t]);
  }

  const float lt = l + xor32(l);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  __syncthreads();
#pragma unroll
  for (int t = 0; t < NOT; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int dv = t * 32 + c_row(j, g);
      char* dst = smem + (w * 32 + l32) * SO_STRIDE + dv * ESZ;
      if constexpr (DT == 0) *(uint16_t*)dst = f2bf(o[t][j] * inv);
      else if constexpr (DT == 2) *(uint16_t*)dst = f2h(o[t][j] * inv);
      else *(float*)dst = o[t][j] * inv;
    }
  if (g == 0 && myq < a.Sq)
    a.lse[(int64_t)(b * a.Hq + h) * a.Sq + myq] = lt > 0.f ? (m + log2f(lt)) * LN2 : -INFINITY;
  __syncthreads();
  char* obase = (char*)a.o + (b * a.o_sb + h * a.o_sh) * ESZ;
  if (o_vec) {
    constexpr int CPR = DV * ESZ / 16;
    for (int q = tid; q < BM * CPR; q += NT) {
      const int row = q / CPR, c = q % CPR;
      if (q0 + row < a.Sq)
        *(u32x4*)(obase + (int64_t)(q0 + row) * a.o_ss * ESZ + c * 16) = *(const u32x4*)(smem + row * SO_STRIDE + c * 16);
    }
  } else {
    const int dvr = a.dv_real;
    for (int q = tid; q < BM * dvr; q += NT) {
      const int row = q / dvr, c = q % dvr;
      if (q0 + row < a.Sq)
        ((E*)(obase + (int64_t)(q0 + row) * a.o_ss * ESZ))[c] = *(const E*)(smem + row * SO_STRIDE + c * ESZ);
    }
  }
}

// bf16 forward tuned for gfx950: NW waves of 32 queries each (BM = 32*NW) share BN-key tiles of
// k~ and v that are double-buffered in LDS by direct global->LDS loads, so no prefetch registers
// are held and each wave keeps only its q~ fragments and the O^T accumulator.  With NW = 8 two
// waves share each SIMD (<= 256 registers per wave), so one wave's softmax overlaps the other's
// MFMAs.  The running max is raised lazily: O and l are rescaled only when some query's block
// max exceeds the current one by more than TAU (in log2 units), which bounds p by 2^TAU.
// MB: the explicit-mask instantiation, which adds mask_l2 to the scaled scores before the softmax.
template <int HT, int DQK, int DV, int BN, int NW, int NDW, int NSTG, bool MB = false>
__global__ __launch_bounds__(NW * 64, NW == 4 ? 2 : 1) void fwd_bf16_kernel(CoreArgs a, int o_vec) {
  using M = MT<HT>;  // HT: the 16-bit operand type, bf16 (0) or fp16 (2)
  constexpr int BM = NW * 32;
  constexpr int NCK = DQK / 8, NCV = DV / 8;
  constexpr int NQF = DQK / 16, NKT = BN / 32, NPF = BN / 16, NOT = DV / 32;
  constexpr int SK_BYTES = BN * NCK * 16, SV_BYTES = BN * NCV * 16, STAGE = SK_BYTES + SV_BYTES;
  constexpr int SO_STRIDE = DV * 2 + 16;
  constexpr int SMEM = (NSTG * STAGE) > (BM * SO_STRIDE) ? (NSTG * STAGE) : (BM * SO_STRIDE);
  static_assert(NSTG == 2 || NSTG == 3, "ring depth");
  static_assert(NDW >= 1 && NDW <= NW, "DMA waves");
  // A float mask can make a row's softmax peaky, one key carrying nearly all its weight.  With the
  // lazy max that key's probability reaches the 16-bit rounding as some 2^x, x in (0, TAU], not as
  // 1, and its rounding error goes straight into the output (twice the fp16 output error of an exact
  // running max measured with a N(0, 4) mask); with a float mask the max is raised exactly.  A bool
  // mask only removes keys and keeps the lazy max.
  constexpr float TAU = 8.f;
  const float tau = MB && a.mask_dtype != 3 ? 0.f : TAU;
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int nqb = (a.Sq + BM - 1) / BM;
  int qb, bh;
  map_block(blockIdx.x, nqb, a.B * a.Hq, a.causal != 0, qb, bh);
  const int b = bh / a.Hq, h = bh % a.Hq, hk = h / (a.Hq / a.Hkv);
  const int q0 = qb * BM, qw = q0 + w * 32, myq = qw + l32;
  const int off = a.causal_off;

  u32x4 qf[NQF];
  {
    const uint16_t* qrow = (const uint16_t*)a.q + ((int64_t)(b * a.Hq + h) * a.Sq + (myq < a.Sq ? myq : a.Sq - 1)) * DQK;
#pragma unroll
    for (int kk = 0; kk < NQF; ++kk) qf[kk] = *(const u32x4*)(qrow + kk * 16 + g * 8);
    // a wait the compiler sees, before any tile load is in flight (it costs only the q~ loads).  The
    // tile waits are inline asm, opaque to the compiler's wait-count pass; without this the q~
    // loads stay pending in its accounting and it puts vmcnt(18) .. vmcnt(3) ahead of the score
    // products of every tile, right after the DMA waves have issued the next tile.  (Removing that
    // chain measured no faster: the DMA waves are held about as long at the issue of the burst.)
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
  }

  int kend = a.Sk;
  if (a.causal) kend = min(a.Sk, q0 + BM + off);
  const int nkb = kend > 0 ? (kend + BN - 1) / BN : 0;
  const char* kbase = (const char*)((const uint16_t*)a.k + (int64_t)(b * a.Hkv + hk) * a.Sk * DQK);
  const char* vbase = (const char*)((const uint16_t*)a.v + b * a.v_sb + hk * a.v_sh);
  const int64_t krs = (int64_t)DQK * 2, vrs = a.v_ss * 2;

  constexpr int KSZ = 0;  // k~ tile swizzle kind (row reads only)
  const RowFrags<NCK, KSZ> rk(perm_row<0>(l32), g);  // k~ row fragments (rows nt*32 + perm_row(l32))
  constexpr int VSZ = 1;  // v tile swizzle kind (it is only read with the transpose load)
  const ColFrags<NCV, VSZ> cv(lane);                  // v transpose fragments
  f32x16 o[NOT];
#pragma unroll
  for (int t = 0; t < NOT; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[t][j] = 0.f;
  float m = -1e30f, l = 0.f;
  const float sl2 = a.scale * LOG2E;

  // The last NDW waves issue every tile load (per-lane offsets computed once; full tiles need no
  // vector math), NSTG - 1 tiles ahead.  Waves that issue none go straight to their products after
  // the barrier, so the two waves of a SIMD start each tile out of step.
  const bool dmaw = __builtin_amdgcn_readfirstlane(w) >= NW - NDW;
  const int dw = dmaw ? w - (NW - NDW) : 0;
  const DmaPlan<BN, NCK, NDW, KSZ> plan_k(dw, lane, (uint32_t)krs);
  const DmaPlan<BN, NCV, NDW, VSZ> plan_v(dw, lane, (uint32_t)vrs);
  constexpr int PER = DmaPlan<BN, NCK, NDW>::TPW + DmaPlan<BN, NCV, NDW>::TPW;
  const uint32_t smem_l = lds_addr(smem);
  auto issue = [&](int kb) {
    if (!dmaw) return;
    const int k0 = kb * BN;
    char* nK = smem + (kb % NSTG) * STAGE;
    const char* ksrc = kbase + (int64_t)k0 * krs;
    const char* vsrc = vbase + (int64_t)k0 * vrs;
    if (a.Sk - k0 >= BN) {
      const uint32_t nl = smem_l + (uint32_t)((kb % NSTG) * STAGE);
      plan_k.full(ksrc, nl, dw, (uint32_t)krs);
      plan_v.full(vsrc, nl + SK_BYTES, dw, (uint32_t)vrs);
    } else {
      // the last, partial tile: an opaque copy of the lane index keeps this path's offsets from
      // being hoisted out of the loop (they would hold registers for the whole loop)
      int ln = lane;
      asm volatile("" : "+v"(ln));
      dma_tile<BN, NCK, NDW, KSZ>(nK, ksrc, krs, a.Sk - k0, dw, ln);
      dma_tile<BN, NCV, NDW, VSZ>(nK + SK_BYTES, vsrc, vrs, a.Sk - k0, dw, ln);
    }
  };
#pragma unroll
  for (int i = 0; i < NSTG - 1; ++i)
    if (i < nkb) issue(i);
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * BN;
    // the slot offset is opaque to the compiler, which would otherwise keep a set of per-lane
    // fragment addresses for each slot
    int slot = (kb % NSTG) * STAGE;
    asm volatile("" : "+s"(slot));
    char* sK = smem + slot;
    char* sV = sK + SK_BYTES;
    // tile kb has landed once at most the loads of the tiles issued after it are outstanding
    if (NSTG == 3 && kb + 1 < nkb) wait_vmcnt<PER>();
    else dma_wait();
    __syncthreads();
    if (kb + NSTG - 1 < nkb) issue(kb + NSTG - 1);  // its slot held tile kb - 1
    if (a.causal && k0 > qw + 31 + off) continue;  // whole tile above this wave's diagonal

    f32x16 s[NKT];
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) s[nt][j] = 0.f;
    // the score products at raised priority, the rest at the lowest: a wave whose S is ready goes
    // ahead of the other wave's softmax and PV (the forward 0.5-1 % faster at every shape measured)
    __builtin_amdgcn_s_setprio(2);
    {
      // S = k~ q~^T: NKT*NQF products, each with its own k~ row fragment, through a fenced ring
      // of depth FD (reads FD products ahead; left to itself the scheduler waits on every read
      // right before its product); consecutive products alternate accumulators
      constexpr int NF = NKT * NQF, FD = 3;
      u32x4 kq[FD];
#pragma unroll
      for (int i = 0; i < FD; ++i) kq[i] = rk.read(sK, (i % NKT) * 32, i / NKT);
#pragma unroll
      for (int i = 0; i < NF; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        const u32x4 cur = kq[i % FD];
        if (i + FD < NF) kq[i % FD] = rk.read(sK, ((i + FD) % NKT) * 32, (i + FD) / NKT);
        __builtin_amdgcn_sched_barrier(0);
        s[i % NKT] = M::mma(cur, qf[i / NKT], s[i % NKT]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
    // the running max is kept in log2 units; as sl2 > 0 it is the max of the raw scores times
    // sl2, and each probability is one fma and one exp2 of a raw score
    const bool edge = (a.causal && k0 + BN - 1 > qw + off) || (k0 + BN > a.Sk);
    if constexpr (MB) {  // the scores in log2 units with the mask added; the softmax takes them as they are
      if (a.mask_vec) {  // values j = 8 hf .. 8 hf + 7 of tile nt are 8 consecutive keys: one vector read
        const int qc = myq < a.Sq ? myq : a.Sq - 1;
        const int64_t rowb = b * a.m_sb + h * a.m_sh + (int64_t)qc * a.m_sq;
#pragma unroll
        for (int nt = 0; nt < NKT; ++nt)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int key0 = k0 + nt * 32 + hf * 16 + g * 8;  // c_logical(8 hf + e, g) - e
            float mv[8];
            if (key0 < a.Sk) {
              mask_row8(a, rowb + key0, mv);
            } else {  // keys past Sk (Sk % 8 == 0: none of the 8 is inside), masked by the edge test below
#pragma unroll
              for (int e = 0; e < 8; ++e) mv[e] = 0.f;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) s[nt][hf * 8 + e] = fmaf(s[nt][hf * 8 + e], sl2, mv[e]);
          }
      } else {
#pragma unroll
        for (int nt = 0; nt < NKT; ++nt)
#pragma unroll
          for (int j = 0; j < 16; ++j)
            s[nt][j] = fmaf(s[nt][j], sl2, mask_l2(a, b, h, myq, k0 + nt * 32 + c_logical<0>(j, g)));
      }
    }
    if (edge) {
#pragma unroll
      for (int nt = 0; nt < NKT; ++nt)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = k0 + nt * 32 + c_logical<0>(j, g);
          if (key >= a.Sk || (a.causal && key > myq + off)) s[nt][j] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[nt][j]);
    mx = fmaxf(mx, xor32(mx)) * (MB ? 1.f : sl2);
    if (__any(mx > m + tau)) {
      const float mn = fmaxf(m, mx);
      const float alpha = fast_exp2(m - mn);
      m = mn;
      l *= alpha;
#pragma unroll
      for (int t = 0; t < NOT; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[t][j] *= alpha;
    }
    float rs = 0.f;
#pragma unroll
    for (int nt = 0; nt < NKT; ++nt)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float p = fast_exp2(MB ? s[nt][j] - m : fmaf(s[nt][j], sl2, -m));
        s[nt][j] = p;
        rs += p;
      }
    l += rs;
    u32x4 pf[NPF];
#pragma unroll
    for (int ks = 0; ks < NPF; ++ks) pf[ks] = M::pack(s[ks / 2], (ks % 2) * 8);
    {
      // O^T += v^T P^T: NOT*NPF products with v transpose fragments, same fenced ring
      constexpr int NF = NOT * NPF, FD = 4;
      u32x4 vq[FD];
#pragma unroll
      for (int i = 0; i < FD; ++i) vq[i] = cv.read(sV, (i / NOT) * 16, (i % NOT) * 32);
#pragma unroll
      for (int i = 0; i < NF; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        const u32x4 cur = vq[i % FD];
        if (i + FD < NF) vq[i % FD] = cv.read(sV, ((i + FD) / NOT) * 16, ((i + FD) % NOT) * 32);
        __builtin_amdgcn_sched_barrier(0);
        o[i % NOT] = M::mma(cur, pf[i / NOT], o[i % NOT]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  const float lt = l + xor32(l);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  __syncthreads();
#pragma unroll
  for (int t = 0; t < NOT; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int dv = t * 32 + c_row(j, g);
      *(uint16_t*)(smem + (w * 32 + l32) * SO_STRIDE + dv * 2) = HT == 0 ? f2bf(o[t][j] * inv) : f2h(o[t][j] * inv);
    }
  if (g == 0 && myq < a.Sq)
    a.lse[(int64_t)(b * a.Hq + h) * a.Sq + myq] = lt > 0.f ? (m + __log2f(lt)) * LN2 : -INFINITY;
  __syncthreads();
  char* obase = (char*)a.o + (b * a.o_sb + h * a.o_sh) * 2;
  if (o_vec) {
    constexpr int CPR = DV * 2 / 16;
    for (int q = tid; q < BM * CPR; q += NW * 64) {
      const int row = q / CPR, c = q % CPR;
      if (q0 + row < a.Sq)
        *(u32x4*)(obase + (int64_t)(q0 + row) * a.o_ss * 2 + c * 16) = *(const u32x4*)(smem + row * SO_STRIDE + c * 16);
    }
  } else {
    const int dvr = a.dv_real;
    for (int q = tid; q < BM * dvr; q += NW * 64) {
      const int row = q / dvr, c = q % dvr;
      if (q0 + row < a.Sq)
        ((uint16_t*)(obase + (int64_t)(q0 + row) * a.o_ss * 2))[c] = *(const uint16_t*)(smem + row * SO_STRIDE + c * 2);
    }
  }
}

template <int HT, int DQK, int DV>
static int run_fwd_bf16(const CoreArgs& a, hipStream_t s) {
  constexpr int NW = 8;
  // four DMA waves, a double-buffered ring (a 3-tile ring measured 1.44 against 1.41 ms)
  constexpr int NDW = 4, NSTG = 2;
  const int BM = NW * 32;
  const int nqb = (a.Sq + BM - 1) / BM;
  const int grid = nqb * a.B * a.Hq;
  // a grid of 256-query blocks that leaves CUs idle (short sequences, few heads): 128-query blocks
  // of four waves, two workgroups per CU, double the workgroups and halve the longest causal block
  const bool small = (int64_t)grid < a.n_cu;
  const int grid4 = ((a.Sq + 127) / 128) * a.B * a.Hq;
  const int o_vec = (a.dv_real == DV) && ((uintptr_t)a.o % 16 == 0) && ((a.o_ss * 2) % 16 == 0) &&
                    ((a.o_sh * 2) % 16 == 0) && ((a.o_sb * 2) % 16 == 0);
  if (a.mask) {  // explicit mask: the 64-key tiles of eight waves only
    hipLaunchKernelGGL((fwd_bf16_kernel<HT, DQK, DV, 64, NW, NDW, NSTG, true>), dim3(grid), dim3(NW * 64), 0, s, a,
                       o_vec);
    return hipGetLastError() == hipSuccess ? 0 : -7;
  }
  // 96-key tiles spread each step's barrier and tile wait over 1.5 times the products (forward
  // 1.37 vs 1.40 ms at S = 16384, 3 % faster at S = 2048); on short sequences the wider diagonal
  // tiles waste more than that saves (S = 512: 0.023 vs 0.021 ms), so they keep 64-key tiles
  if (small)
    hipLaunchKernelGGL((fwd_bf16_kernel<HT, DQK, DV, 64, 4, 4, NSTG>), dim3(grid4), dim3(4 * 64), 0, s, a, o_vec);
  else if (a.Sk >= 2048)
    hipLaunchKernelGGL((fwd_bf16_kernel<HT, DQK, DV, 96, NW, NDW, NSTG>), dim3(grid), dim3(NW * 64), 0, s, a, o_vec);
  else
    hipLaunchKernelGGL((fwd_bf16_kernel<HT, DQK, DV, 64, NW, NDW, NSTG>), dim3(grid), dim3(NW * 64), 0, s, a, o_vec);
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

template <int DT, int DQK, int DV, bool MB>
static int run_fwd(const CoreArgs& a, hipStream_t s) {
  constexpr int NW = 4;
  constexpr int BN = DT != 1 ? 64 : 32;
  const int BM = NW * 32;
  const int nqb = (a.Sq + BM - 1) / BM;
  const int grid = nqb * a.B * a.Hq;
  const int o_vec = (a.dv_real == DV) && ((uintptr_t)a.o % 16 == 0) &&
                    ((a.o_ss * MT<DT>::ESZ) % 16 == 0) && ((a.o_sh * MT<DT>::ESZ) % 16 == 0) &&
                    ((a.o_sb * MT<DT>::ESZ) % 16 == 0);
  hipLaunchKernelGGL((fwd_kernel<DT, DQK, DV, BN, NW, MB>), dim3(grid), dim3(NW * 64), 0, s, a, o_vec);
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

bool core_supported(int dqk, int dv) {
  return (dqk == 64 && dv == 64) || (dqk == 128 && dv == 64) || (dqk == 128 && dv == 128) ||
         (dqk == 256 && dv == 128) || (dqk == 256 && dv == 64) || (dqk == 64 && dv == 128);
}

template <int DT>
static int fwd_dt(int dqk, int dv, const CoreArgs& a, hipStream_t s) {
  if constexpr (DT == 1) {
    if (a.mask) {  // explicit mask in fp32: the generic kernel (16-bit: run_fwd_bf16's mask instantiation)
      if (dqk == 64 && dv == 64) return run_fwd<DT, 64, 64, true>(a, s);
      if (dqk == 64 && dv == 128) return run_fwd<DT, 64, 128, true>(a, s);
      if (dqk == 128 && dv == 64) return run_fwd<DT, 128, 64, true>(a, s);
      if (dqk == 128 && dv == 128) return run_fwd<DT, 128, 128, true>(a, s);
      if (dqk == 256 && dv == 64) return run_fwd<DT, 256, 64, true>(a, s);
      if (dqk == 256 && dv == 128) return run_fwd<DT, 256, 128, true>(a, s);
      return -3;
    }
  }
  if constexpr (DT != 1) {
    if (dqk == 64 && dv == 64) return run_fwd_bf16<DT, 64, 64>(a, s);
    if (dqk == 64 && dv == 128) return run_fwd_bf16<DT, 64, 128>(a, s);
    if (dqk == 128 && dv == 64) return run_fwd_bf16<DT, 128, 64>(a, s);
    if (dqk == 128 && dv == 128) return run_fwd_bf16<DT, 128, 128>(a, s);
    if (dqk == 256 && dv == 64) return run_fwd_bf16<DT, 256, 64>(a, s);
    if (dqk == 256 && dv == 128) return run_fwd_bf16<DT, 256, 128>(a, s);
    return -3;
  } else {
    if (dqk == 64 && dv == 64) return run_fwd<DT, 64, 64, false>(a, s);
    if (dqk == 64 && dv == 128) return run_fwd<DT, 64, 128, false>(a, s);
    if (dqk == 128 && dv == 64) return run_fwd<DT, 128, 64, false>(a, s);
    if (dqk == 128 && dv == 128) return run_fwd<DT, 128, 128, false>(a, s);
    if (dqk == 256 && dv == 64) return run_fwd<DT, 256, 64, false>(a, s);
    if (dqk == 256 && dv == 128) return run_fwd<DT, 256, 128, false>(a, s);
    return -3;
  }
}

// dt: 0 bf16, 1 fp32, 2 fp16 operands
int launch_fwd(int dt, int dqk, int dv, const CoreArgs& a, hipStream_t s) {
  if (dt == 0) return fwd_dt<0>(dqk, dv, a, s);
  if (dt == 2) return fwd_dt<2>(dqk, dv, a, s);
  return fwd_dt<1>(dqk, dv, a, s);
}

}  // namespace pe
