// Attention of a few new query rows against a cache of transformed keys and values (the KV-cache
// path of FPoPEGroupedQueryAttentionWithCache.forward, src/model/fpope_attention.py:226-327, whose
// cache holds [k_c | PoPE(k_r)] and whose mask is bottom-right, :313-317).
//
// Decode is bound by reading the cache, not by the matrix cores, so the work is split over the
// keys: a (batch, kv head, 32-row query tile) is cut into `nunit` key ranges of 32-key blocks, one
// per wave.  The tile's q~ rows (the MFMA B operand) sit in LDS, shared by the workgroup's 4 waves.
// A wave reads its k~ rows straight from HBM as A operands (16 contiguous bytes per lane and
// k-step), stages each 32-key v block in one of its two LDS slots for the transpose read, loads the
// next block while it computes the current one, and keeps an online softmax.  Its
// unnormalised O^T, running max and row sum go to a partials buffer; a second kernel merges the
// ranges of every row in a fixed order (no atomics, bitwise reproducible).
//
// Query rows of one kv head's GQA group share the tile: row r of tile qt is query head
// hk * grp + r / Sq, query r % Sq (Sq new queries, grp = Hq / Hkv), so one decoded token of eight
// query heads per kv head fills eight MFMA columns instead of one.
#include "pe_common.h"
#include "pe_internal.h"

namespace pe {

// One wave per SIMD: the plan launches about one 4-wave workgroup per CU, and the whole register
// file then holds the q~ fragments' ring, the k~ fragments of the block in flight and the PV
// accumulators without spills (352 VGPRs at QK 256 / V 128 in bf16; 2.7 % faster than the
// 256-register build, which spilled around its loop).
template <int DT, int DQK, int DV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void decode_split_kernel(DecodeArgs a) {
  using E = typename Elem<DT>::T;
  using M = MT<DT>;
  constexpr int KC = M::KC, EPL = M::EPL, ESZ = M::ESZ;
  constexpr int NQF = DQK / KC, NCV = DV * ESZ / 16, NOT = DV / 32, NPF = 32 / KC;
  constexpr int SV = 32 * NCV * 16;  // one 32-key v block
  constexpr int NV = 32 * NCV / 64;  // DMA instructions per v block
  constexpr int NCQ = 2 * NQF;       // 16-byte chunks per q~ row (fragment kk of lane half g is chunk 2 kk + g)
  constexpr int QROW = NCQ * 16;
  // [4 waves][2 slots] v blocks, then the tile's 32 q~ rows (shared by the 4 waves)
  __shared__ __attribute__((aligned(1024))) char smem[8 * SV + 32 * QROW];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
  char* const vslot[2] = {smem + (2 * w) * SV, smem + (2 * w + 1) * SV};  // this wave's two v slots
  const int ubs = a.nunit / 4;
  int bid = blockIdx.x;
  const int ub = bid % ubs;
  bid /= ubs;
  const int qt = bid % a.nqt, bh = bid / a.nqt;
  const int b = bh / a.Hkv, hk = bh % a.Hkv, grp = a.Hq / a.Hkv;
  const int u = ub * 4 + w;
  const int nrows = grp * a.Sq;
  const int r = qt * 32 + l32;  // this lane's query row (C column)
  const int rr = r < nrows ? r : nrows - 1;
  const int h = hk * grp + rr / a.Sq, qi = rr % a.Sq;

  // this wave's 32-key blocks [kb0, kb1); keys past the tile's last visible key are skipped
  const int nkb = (a.L + 31) / 32;
  const int kb0 = (int)((int64_t)u * nkb / a.nunit), kb1 = (int)((int64_t)(u + 1) * nkb / a.nunit);
  int kmax = a.L - 1;  // the last key any row of this tile sees
  if (a.causal) {
    const int rlast = min(nrows, qt * 32 + 32) - 1;
    int last_q = 0;  // the largest query index among the tile's rows
    if (rlast / a.Sq > (qt * 32) / a.Sq) last_q = a.Sq - 1;
    else last_q = rlast % a.Sq;
    kmax = min(kmax, last_q + a.off);
  }
  const int kend = kmax < 0 ? kb0 : min(kb1, kmax / 32 + 1);

  const E* kbase = (const E*)a.k + (int64_t)(b * a.Hkv + hk) * a.cap * DQK;
  const char* vbase = (const char*)a.v + (int64_t)(b * a.Hkv + hk) * a.cap * DV * ESZ;
  f32x16 o[NOT];
#pragma unroll
  for (int t = 0; t < NOT; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[t][j] = 0.f;
  float m = -1e30f, l = 0.f;
  const float sl2 = a.scale * LOG2E;

  // The next block's loads are in flight while a block is computed.  The k~ rows go straight to
  // registers as A operands (lane (l32, g) takes key k0 + perm_row(l32), clamped into the cache), and
  // each fragment is refilled with the next block's row right after its score product.  The v rows go
  // by DMA into the wave's other LDS slot (rows at or past L re-read row L - 1).  Issue order per
  // block: the refill loads, then the next v block; the wait before the PV products leaves exactly
  // those outstanding.  The compiler does not see the DMA, so its waits for a refilled fragment in the
  // next block may also drain that block's own v loads (issued after the refills), which its PV
  // products need anyway, but never loads of a later block.
  auto krow_of = [&](int kb) {
    return kbase + (int64_t)min(kb * 32 + perm_row<DT>(l32), a.L - 1) * DQK;
  };
  auto issue_v = [&](int kb, char* slot) {
    dma_tile<32, NCV, 1>(slot, vbase + (int64_t)kb * 32 * DV * ESZ, (int64_t)DV * ESZ, a.L - kb * 32, 0, lane);
  };
  u32x4 kf[NQF];
  if (kb0 < kend) {
    const E* krow = krow_of(kb0);
#pragma unroll
    for (int kk = 0; kk < NQF; ++kk) kf[kk] = *(const u32x4*)(krow + kk * KC + g * EPL);
    issue_v(kb0, vslot[0]);
  }
  // The 4 waves of a workgroup share the tile's query rows, so wave 0 stages them in LDS once (while
  // the first block's loads are in flight) and every wave reads its B fragments from there per block
  // (64 registers fewer than holding them).  Chunk c of row x is stored at chunk c ^ (x % NCQ), so
  // the 32 rows of one fragment read spread over the banks.  The barrier waits only for the LDS
  // writes: __syncthreads() would also drain the block loads in flight.
  char* const qlds = smem + 8 * SV;
  const uint32_t qrd = (uint32_t)l32 * QROW;
  const uint32_t qsw = (uint32_t)(l32 & (NCQ - 1));
  bool staged = false;
  if constexpr (DT == 0) {
    if (a.qraw) {
      // the raw rows transformed here, element by element with the vectorised prologue's arithmetic
      // (softplus magnitude times cos / sin of fl(pos * freq), rounded to bf16), so the operand
      // rows are bitwise those the prologue would write; tile rows past the query rows are zero
      // (their columns are never stored).  Element (x, d) of the tile goes to column d (cos) and
      // Dr + d (sin) of row x, chunk-swizzled as above.
      const int tid = threadIdx.x, Dr = a.Dr;
      const int nreal = min(32, nrows - qt * 32);
      for (int i = tid; i < (32 - nreal) * NCQ; i += 256) {
        const int x = nreal + i / NCQ, c = i % NCQ;
        *(u32x4*)(qlds + x * QROW + ((c ^ (x & (NCQ - 1))) << 4)) = u32x4{0u, 0u, 0u, 0u};
      }
      for (int i = tid; i < nreal * Dr; i += 256) {
        const int x = i / Dr, d = i % Dr;
        const int rq = qt * 32 + x, hq = hk * grp + rq / a.Sq, iq = rq % a.Sq;
        const uint16_t raw = ((const uint16_t*)a.qraw)[b * a.qr_s[0] + hq * a.qr_s[1] + (int64_t)iq * a.qr_s[2] + d];
        const float mu = softplus_f(__builtin_bit_cast(float, (uint32_t)raw << 16));
        float sn, cs;
        pe_sincos(mul_nc(pe_pos(a.start_pos + iq, a.pos_round), a.freqs[d]), sn, cs);
        const uint32_t pr = pack_bf2(mul_nc(mu, cs), mul_nc(mu, sn));
        const int cc = d, cs_ = Dr + d;
        *(uint16_t*)(qlds + x * QROW + ((((uint32_t)cc >> 3) ^ (uint32_t)(x & (NCQ - 1))) << 4) + (cc & 7) * 2) = (uint16_t)pr;
        *(uint16_t*)(qlds + x * QROW + ((((uint32_t)cs_ >> 3) ^ (uint32_t)(x & (NCQ - 1))) << 4) + (cs_ & 7) * 2) =
            (uint16_t)(pr >> 16);
      }
      staged = true;
    }
  }
  if (!staged && w == 0) {
    const E* qrow = (const E*)a.q + ((int64_t)(b * a.Hq + h) * a.Sq + qi) * DQK;
    u32x4 qv[NQF];
#pragma unroll
    for (int kk = 0; kk < NQF; ++kk) qv[kk] = *(const u32x4*)(qrow + kk * KC + g * EPL);
#pragma unroll
    for (int kk = 0; kk < NQF; ++kk) *(u32x4*)(qlds + qrd + (((uint32_t)(2 * kk + g) ^ qsw) << 4)) = qv[kk];
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  auto qfrag = [&](int kk) { return *(const u32x4*)(qlds + qrd + (((uint32_t)(2 * kk + g) ^ qsw) << 4)); };
  constexpr int FD = 3;  // q~ fragments read ahead of their product
  auto block = [&](const int kb, auto next_tag) {
    constexpr bool NEXT = decltype(next_tag)::value;
    const int k0 = kb * 32, sl = (kb - kb0) & 1;
    const E* krn = krow_of(kb + 1);
    f32x16 s;
#pragma unroll
    for (int j = 0; j < 16; ++j) s[j] = 0.f;
    // q~ fragments read FD products ahead; the fences (mask 0x406: vector, scalar and transcendental
    // work may cross) keep the LDS reads, the refill loads and the products in program order, so the
    // compiler neither hoists every read nor issues the refills early, which would need registers
    u32x4 qr[FD];
#pragma unroll
    for (int i = 0; i < FD; ++i) qr[i] = qfrag(i);
#pragma unroll
    for (int kk = 0; kk < NQF; ++kk) {
      __builtin_amdgcn_sched_barrier(0x406);
      const u32x4 cur = qr[kk % FD];
      if (kk + FD < NQF) qr[kk % FD] = qfrag(kk + FD);
      __builtin_amdgcn_sched_barrier(0x406);
      s = M::mma(kf[kk], cur, s);
      if constexpr (NEXT) kf[kk] = *(const u32x4*)(krn + kk * KC + g * EPL);
    }
    __builtin_amdgcn_sched_barrier(0);
    float mx = m;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int key = k0 + c_logical<DT>(j, g);
      float x = s[j] * sl2;
      if (key >= a.L || (a.causal && key > qi + a.off)) x = -INFINITY;
      s[j] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, xor32(mx));
    const float alpha = exp2f(m - mx);
    m = mx;
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float p = exp2f(s[j] - m);
      s[j] = p;
      rs += p;
    }
    l = l * alpha + rs;
#pragma unroll
    for (int t = 0; t < NOT; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[t][j] *= alpha;
    u32x4 pf[NPF];
#pragma unroll
    for (int ks = 0; ks < NPF; ++ks) pf[ks] = M::pack(s, ks * EPL);
    // the slot of block kb + 1 held block kb - 1, whose PV products have read it
    if constexpr (NEXT) {
      issue_v(kb + 1, vslot[sl ^ 1]);
      wait_vmcnt<NQF + NV>();  // v block kb has landed; the refills and v block kb + 1 may not have
    } else {
      wait_vmcnt<0>();
    }
    const char* vt = vslot[sl];
#pragma unroll
    for (int t = 0; t < NOT; ++t)
#pragma unroll
      for (int ks = 0; ks < NPF; ++ks) o[t] = M::mma(lds_col_frag<DT, NCV>(vt, ks * KC, t * 32, lane), pf[ks], o[t]);
  };
  int kb = kb0;
  for (; kb + 1 < kend; ++kb) block(kb, std::true_type{});
  if (kb < kend) block(kb, std::false_type{});

  // partials of this wave's range: [bh][qt][u] blocks of 32 rows (rows past the tile's query rows
  // are neither written nor read)
  const int64_t pb = ((int64_t)bh * a.nqt + qt) * a.nunit + u;
  const float lt = l + xor32(l);
  if (r >= nrows) return;
  float* po = a.part_o + pb * 32 * DV;
#pragma unroll
  for (int t = 0; t < NOT; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) po[(int64_t)l32 * DV + t * 32 + c_row(j, g)] = o[t][j];
  if (g == 0) {
    a.part_m[pb * 32 + l32] = m;
    a.part_l[pb * 32 + l32] = lt;
  }
}

// One workgroup of MT threads per query row of a tile: the ranges' partials merged as
// O = sum_u O_u 2^(m_u - M) / sum_u l_u 2^(m_u - M), M = max_u m_u; lse = (M + log2 l) ln 2.
// Thread t takes ranges t, t + MT, ... for the max and the weights; for O, thread (c, j) =
// (t % DV, t / DV) sums the ranges u = j (mod MT / DV) of column c in increasing u (loads issued
// eight at a time), and the MT / DV group sums are added in group order.  Every sum runs in a fixed
// order, so the result is bitwise reproducible.
template <int DV>
__global__ __launch_bounds__(1024) void decode_merge_kernel(DecodeArgs a) {
  constexpr int MT = 1024, NWV = MT / 64, G = MT / DV;
  __shared__ float wts[512];
  __shared__ float red[G][DV];
  __shared__ float wred[2][NWV];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // (bh, qt, row) over the rpt = min(32, query rows) rows a tile can hold: a tile of a few decoded
  // rows launches only those
  const int grp = a.Hq / a.Hkv, nrows = grp * a.Sq, rpt = min(32, nrows);
  const int64_t rowid = blockIdx.x;
  const int row = (int)(rowid % rpt);
  const int64_t tile = rowid / rpt;
  const int qt = (int)(tile % a.nqt);
  const int bh = (int)(tile / a.nqt);
  const int r = qt * 32 + row;
  if (r >= nrows) return;  // uniform over the workgroup
  const int b = bh / a.Hkv, hk = bh % a.Hkv;
  const int h = hk * grp + r / a.Sq, qi = r % a.Sq;
  const int64_t p0 = ((int64_t)bh * a.nqt + qt) * a.nunit;

  float mloc = -1e30f;
  for (int u = tid; u < a.nunit; u += MT) mloc = fmaxf(mloc, a.part_m[(p0 + u) * 32 + row]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, o, 64));
  if (lane == 0) wred[0][w] = mloc;
  __syncthreads();
  float M = wred[0][0];
#pragma unroll
  for (int i = 1; i < NWV; ++i) M = fmaxf(M, wred[0][i]);
  float lloc = 0.f;
  for (int u = tid; u < a.nunit; u += MT) {
    const float wt = exp2f(a.part_m[(p0 + u) * 32 + row] - M);
    wts[u] = wt;
    lloc += a.part_l[(p0 + u) * 32 + row] * wt;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) lloc += __shfl_xor(lloc, o, 64);
  if (lane == 0) wred[1][w] = lloc;
  __syncthreads();
  float lsum = 0.f;
#pragma unroll
  for (int i = 0; i < NWV; ++i) lsum += wred[1][i];
  const int c = tid % DV, j = tid / DV;
  const float* po = a.part_o + (p0 * 32 + row) * DV + c;  // range u at po + u * 32 * DV
  float acc = 0.f;
  int u = j;
  for (; u + 7 * G < a.nunit; u += 8 * G) {
    float x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = po[(int64_t)(u + i * G) * 32 * DV];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += x[i] * wts[u + i * G];
  }
  for (; u < a.nunit; u += G) acc += po[(int64_t)u * 32 * DV] * wts[u];
  red[j][c] = acc;
  __syncthreads();
  if (tid < DV) {
    float osum = 0.f;
#pragma unroll
    for (int i = 0; i < G; ++i) osum += red[i][tid];
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    if (tid < a.dv_real)
      store_from_float(a.o, b * a.o_sb + h * a.o_sh + (int64_t)qi * a.o_ss + tid, a.o_dtype, osum * inv);
    if (tid == 0) a.lse[(int64_t)(b * a.Hq + h) * a.Sq + qi] = lsum > 0.f ? (M + log2f(lsum)) * LN2 : -INFINITY;
  }
}

template <int DT, int DQK, int DV>
static int run_decode(const DecodeArgs& a, hipStream_t s) {
  const int64_t blocks = (int64_t)a.B * a.Hkv * a.nqt * (a.nunit / 4);
  hipLaunchKernelGGL((decode_split_kernel<DT, DQK, DV>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  const int64_t rows = (int64_t)a.B * a.Hkv * a.nqt * std::min(32, (a.Hq / a.Hkv) * a.Sq);
  hipLaunchKernelGGL((decode_merge_kernel<DV>), dim3((unsigned)rows), dim3(1024), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

template <int DT>
static int decode_dt(int dqk, int dv, const DecodeArgs& a, hipStream_t s) {
  if (dqk == 64 && dv == 64) return run_decode<DT, 64, 64>(a, s);
  if (dqk == 64 && dv == 128) return run_decode<DT, 64, 128>(a, s);
  if (dqk == 128 && dv == 64) return run_decode<DT, 128, 64>(a, s);
  if (dqk == 128 && dv == 128) return run_decode<DT, 128, 128>(a, s);
  if (dqk == 256 && dv == 64) return run_decode<DT, 256, 64>(a, s);
  if (dqk == 256 && dv == 128) return run_decode<DT, 256, 128>(a, s);
  return -3;
}

int launch_decode(int dt, int dqk, int dv, const DecodeArgs& a, hipStream_t s) {
  if (a.nunit % 4 != 0 || a.nunit <= 0 || a.nunit > 512 || a.nqt <= 0) return -2;
  if (dt == 0) return decode_dt<0>(dqk, dv, a, s);  // bf16
  if (dt == 2) return decode_dt<2>(dqk, dv, a, s);  // fp16
  return decode_dt<1>(dqk, dv, a, s);
}

}  // namespace pe
