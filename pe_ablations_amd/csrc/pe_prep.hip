// Elementwise kernels around the attention core (all HBM-bound, one wave or one thread per element
// row):
//   prep_kernel   forward positional transform, row -> [content | transform | zero pad]
//                 PoPE/FoPE (src/model/pope.py:124-183, src/model/fpope.py:266-338):
//                   mu = softplus(x); phi = fl(pos*freq) (+ delta on keys, added after the product,
//                   no fused multiply-add); [mu cos phi, mu sin phi]
//                 RoPE/NTK/YaRN (src/model/rope.py:35-57,209-217): interleaved pairs rotated by
//                   fl(pos*inv_freq), times mscale; optional QKNorm x/(||x||+1e-6)
//                   (src/model/normalization.py:54-55)
//   prebwd_kernel dO -> compute-dtype operand, Di = rowsum(dO o O)
//   inv_pope_kernel  gradient of the PoPE transform with per-block partial sums of dphi (key
//                 phase bias) and pos*dphi (frequencies)
//   inv_row_kernel   gradient of the RoPE / no-PE transform incl. the QKNorm backward
//   reduce_kernel fixed-order sum of the partials (bitwise reproducible)
#include "pe_common.h"
#include "pe_internal.h"

namespace pe {

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

constexpr int MAX_PAIRS_PER_LANE = 4;  // RoPE rows up to 512 dims

__global__ __launch_bounds__(256) void prep_kernel(PrepArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nrows = (int64_t)a.B * a.H * a.S;
  if (row >= nrows) return;
  const int s = (int)(row % a.S);
  const int bh = (int)(row / a.S);
  const int h = bh % a.H, b = bh / a.H;
  const float pos = pe_pos(a.start_pos + s, a.pos_round);
  const int64_t dbase = ((int64_t)bh * (a.dst_rows ? a.dst_rows : a.S) + a.dst_row0 + s) * a.width;

  for (int c = lane; c < a.Dc; c += 64) {
    const float x = load_as_float(a.xc, b * a.xc_s[0] + h * a.xc_s[1] + (int64_t)s * a.xc_s[2] + c * a.xc_s[3], a.xc_dtype);
    store_from_float(a.dst, dbase + c, a.dst_dtype, x);
  }
  const int64_t xr0 = b * a.xr_s[0] + h * a.xr_s[1] + (int64_t)s * a.xr_s[2];
  int used = a.Dc;
  if (a.mode == 0) {  // PoPE / FoPE
    for (int c = lane; c < a.Dr; c += 64) {
      const float x = load_as_float(a.xr, xr0 + c * a.xr_s[3], a.xr_dtype);
      const float mu = softplus_f(x);
      float ph = mul_nc(pos, a.freqs[c]);
      if (a.is_key && a.delta) ph = add_nc(ph, a.delta[h * a.delta_hs + c]);
      float sn, cs;
      pe_sincos(ph, sn, cs);
      store_from_float(a.dst, dbase + a.Dc + c, a.dst_dtype, mul_nc(mu, cs));
      store_from_float(a.dst, dbase + a.Dc + a.Dr + c, a.dst_dtype, mul_nc(mu, sn));
    }
    used += 2 * a.Dr;
  } else {  // RoPE (mode 1) or plain (mode 2): values kept in registers for the optional L2 norm
    // lane owns the chunk of pairs i = 4 lane + k (RoPE) or elements 2i, 2i+1 (plain, odd widths
    // allowed), the vector kernel's chunk of the same lane index
    float y0[MAX_PAIRS_PER_LANE], y1[MAX_PAIRS_PER_LANE];
    float ss = 0.f;
    const int npairs = (a.Dr + 1) / 2;
#pragma unroll
    for (int k = 0; k < MAX_PAIRS_PER_LANE; ++k) {
      const int i = 4 * lane + k;
      y0[k] = 0.f; y1[k] = 0.f;
      if (i < npairs) {
        const bool has1 = 2 * i + 1 < a.Dr;
        const float x0 = load_as_float(a.xr, xr0 + (2 * i) * a.xr_s[3], a.xr_dtype);
        const float x1 = has1 ? load_as_float(a.xr, xr0 + (2 * i + 1) * a.xr_s[3], a.xr_dtype) : 0.f;
        float sn, cs;
        rope_pair(a.mode, x0, x1, pos, a.mode == 1 ? a.freqs[i] : 0.f, a.mscale, y0[k], y1[k], sn, cs);
        ss = add_nc(ss, sq2(y0[k], y1[k]));
      }
    }
    float den = 1.f;
    if (a.l2norm) den = sqrtf(wave_sum(ss)) + 1e-6f;
#pragma unroll
    for (int k = 0; k < MAX_PAIRS_PER_LANE; ++k) {
      const int i = 4 * lane + k;
      if (i < npairs) {
        store_from_float(a.dst, dbase + a.Dc + 2 * i, a.dst_dtype, a.l2norm ? y0[k] / den : y0[k]);
        if (2 * i + 1 < a.Dr)
          store_from_float(a.dst, dbase + a.Dc + 2 * i + 1, a.dst_dtype, a.l2norm ? y1[k] / den : y1[k]);
      }
    }
    used += a.Dr;
  }
  for (int c = used + lane; c < a.width; c += 64) store_from_float(a.dst, dbase + c, a.dst_dtype, 0.f);
}

// One wave per padded row (b, h, s < S_pad).  Rows s < S: dO repack, Di, L2 = lse*log2(e) (a row
// without visible keys, lse = -inf, gets +inf so that its probabilities are 0).  Padding rows:
// Di = 0, L2 = +inf.
__global__ __launch_bounds__(256) void prebwd_kernel(PreBwdArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t prow = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nprows = (int64_t)a.B * a.H * a.s_pad;
  if (prow >= nprows) return;
  const int s = (int)(prow % a.s_pad);
  const int bh = (int)(prow / a.s_pad);
  if (s >= a.S) {
    if (lane == 0) { a.Di[prow] = 0.f; a.L2[prow] = INFINITY; }
    return;
  }
  const int h = bh % a.H, b = bh / a.H;
  const int64_t row = (int64_t)bh * a.S + s;
  const int64_t d0 = b * a.do_s[0] + h * a.do_s[1] + (int64_t)s * a.do_s[2];
  const int64_t o0 = b * a.o_s[0] + h * a.o_s[1] + (int64_t)s * a.o_s[2];
  float acc = 0.f;
  for (int c = lane; c < a.width; c += 64) {
    float d = 0.f;
    if (c < a.Dv) {
      d = load_as_float(a.dout, d0 + c * a.do_s[3], a.dout_dtype);
      acc += d * load_as_float(a.out, o0 + c * a.o_s[3], a.out_dtype);
    }
    if (a.dO_op) store_from_float(a.dO_op, row * a.width + c, a.op_dtype, d);
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    a.Di[prow] = acc;
    const float lv = a.lse[row];
    a.L2[prow] = lv == -INFINITY ? INFINITY : lv * LOG2E;
  }
}

// One block = rows [chunk*R, chunk*R + R) of one (b, h); TPR threads per row, 256/TPR rows at once.
template <int TPR>
__global__ __launch_bounds__(256) void inv_pope_kernel(InvArgs a) {
  constexpr int RS = 256 / TPR;
  __shared__ float red_d[RS][TPR];
  __shared__ float red_f[RS][TPR];
  const int tid = threadIdx.x, c = tid % TPR, rs = tid / TPR;
  const int chunks = (a.S + a.rows_per_block - 1) / a.rows_per_block;
  const int blk = blockIdx.x;
  const int bh = blk / chunks, chunk = blk % chunks;
  const int h = bh % a.H, b = bh / a.H;
  const int s0 = chunk * a.rows_per_block;
  const int s1 = min(a.S, s0 + a.rows_per_block);
  float acc_d = 0.f, acc_f = 0.f;
  const float fr = c < a.Dr ? a.freqs[c] : 0.f;
  const float dl = (c < a.Dr && a.is_key && a.delta) ? a.delta[h * a.delta_hs + c] : 0.f;
  for (int s = s0 + rs; s < s1; s += RS) {
    const int64_t grow = ((int64_t)bh * a.S + s) * a.width;
    for (int cc = c; cc < a.Dc; cc += TPR)
      store_from_float(a.dxc, b * a.dxc_s[0] + h * a.dxc_s[1] + (int64_t)s * a.dxc_s[2] + cc * a.dxc_s[3], a.dxc_dtype, a.g[grow + cc]);
    if (c < a.Dr) {
      const float pos = pe_pos(a.start_pos + s, a.pos_round);
      const float x = load_as_float(a.xr, b * a.xr_s[0] + h * a.xr_s[1] + (int64_t)s * a.xr_s[2] + c * a.xr_s[3], a.xr_dtype);
      float mu, sg;
      softplus_sigmoid(x, mu, sg);
      float ph = mul_nc(pos, fr);
      if (a.is_key && a.delta) ph = add_nc(ph, dl);
      float sn, cs;
      pe_sincos(ph, sn, cs);
      const float gc = a.g[grow + a.Dc + c], gs = a.g[grow + a.Dc + a.Dr + c];
      const float dmu = gc * cs + gs * sn;
      const float dph = mu * (gs * cs - gc * sn);
      store_from_float(a.dxr, b * a.dxr_s[0] + h * a.dxr_s[1] + (int64_t)s * a.dxr_s[2] + c * a.dxr_s[3], a.dxr_dtype, dmu * sg);
      acc_d += dph;
      acc_f += pos * dph;
    }
  }
  red_d[rs][c] = acc_d;
  red_f[rs][c] = acc_f;
  __syncthreads();
  if (rs == 0 && c < a.Dr) {
    float sd = 0.f, sf = 0.f;
    for (int r = 0; r < RS; ++r) { sd += red_d[r][c]; sf += red_f[r][c]; }
    if (a.part_delta) a.part_delta[(int64_t)blk * a.Dr + c] = sd;
    if (a.part_freq) a.part_freq[(int64_t)blk * a.Dr + c] = sf;
  }
}

// RoPE / no-PE gradient, one wave per row: y = z/(||z||+eps) (optional), z = mscale * rot(x).
//   dz = dy/(n+eps) - z (z.dy) / (n (n+eps)^2);  dx = mscale * rot^T(dz)
__global__ __launch_bounds__(256) void inv_row_kernel(InvArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nrows = (int64_t)a.B * a.H * a.S;
  if (row >= nrows) return;
  const int s = (int)(row % a.S);
  const int bh = (int)(row / a.S);
  const int h = bh % a.H, b = bh / a.H;
  const float pos = pe_pos(a.start_pos + s, a.pos_round);
  const int64_t grow = row * a.width;
  for (int c = lane; c < a.Dc; c += 64)
    store_from_float(a.dxc, b * a.dxc_s[0] + h * a.dxc_s[1] + (int64_t)s * a.dxc_s[2] + c * a.dxc_s[3], a.dxc_dtype, a.g[grow + c]);
  const int64_t xr0 = b * a.xr_s[0] + h * a.xr_s[1] + (int64_t)s * a.xr_s[2];
  const int64_t dx0 = b * a.dxr_s[0] + h * a.dxr_s[1] + (int64_t)s * a.dxr_s[2];
  const int npairs = a.Dr / 2;
  float z0[MAX_PAIRS_PER_LANE], z1[MAX_PAIRS_PER_LANE], g0[MAX_PAIRS_PER_LANE], g1[MAX_PAIRS_PER_LANE];
  float cs_[MAX_PAIRS_PER_LANE], sn_[MAX_PAIRS_PER_LANE];
  float ss = 0.f, zd = 0.f;
#pragma unroll
  for (int k = 0; k < MAX_PAIRS_PER_LANE; ++k) {
    const int i = 4 * lane + k;  // the chunk of 4 pairs of this lane (the vector kernel's order)
    z0[k] = z1[k] = g0[k] = g1[k] = 0.f;
    cs_[k] = 1.f; sn_[k] = 0.f;
    if (i < npairs) {
      const float x0 = load_as_float(a.xr, xr0 + (2 * i) * a.xr_s[3], a.xr_dtype);
      const float x1 = load_as_float(a.xr, xr0 + (2 * i + 1) * a.xr_s[3], a.xr_dtype);
      rope_pair(a.mode, x0, x1, pos, a.mode == 1 ? a.freqs[i] : 0.f, a.mscale, z0[k], z1[k], sn_[k], cs_[k]);
      g0[k] = a.g[grow + a.Dc + 2 * i];
      g1[k] = a.g[grow + a.Dc + 2 * i + 1];
      ss = add_nc(ss, sq2(z0[k], z1[k]));
      zd = add_nc(zd, dot2(z0[k], z1[k], g0[k], g1[k]));
    }
  }
  float c1 = 1.f, c2 = 0.f;
  if (a.l2norm) l2_coefs(wave_sum(ss), wave_sum(zd), c1, c2);
#pragma unroll
  for (int k = 0; k < MAX_PAIRS_PER_LANE; ++k) {
    const int i = 4 * lane + k;
    if (i < npairs) {
      float dx0v, dx1v;
      rope_pair_grad(a.mode, a.l2norm != 0, g0[k], g1[k], z0[k], z1[k], c1, c2, cs_[k], sn_[k], a.mscale, dx0v, dx1v);
      store_from_float(a.dxr, dx0 + (2 * i) * a.dxr_s[3], a.dxr_dtype, dx0v);
      store_from_float(a.dxr, dx0 + (2 * i + 1) * a.dxr_s[3], a.dxr_dtype, dx1v);
    }
  }
}

// One block per 64 output columns (the frequency gradient first, then the phase-bias gradient).
// Wave w sums rows w, w + RW, w + 2 RW, ... in increasing order and wave 0 adds the RW wave sums in
// order, so the result depends only on the partial layout, never on timing.
constexpr int RW = 16;

__global__ __launch_bounds__(RW * 64) void reduce_kernel(ReduceArgs a) {
  __shared__ float red[RW][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nfc = (a.Dr + 63) / 64;
  const int nd = a.delta_per_head ? a.Hkv * a.Dr : a.Dr;
  float s = 0.f;
  float* dst = nullptr;
  if ((int)blockIdx.x < nfc) {
    if (!a.dfreqs) return;
    const int c = blockIdx.x * 64 + lane;
    if (c < a.Dr) {
      dst = a.dfreqs + c;
      const int n = a.nq + a.nk;
#pragma unroll 8
      for (int i = w; i < n; i += RW)
        s += i < a.nq ? a.part_q_freq[(int64_t)i * a.Dr + c] : a.part_k_freq[(int64_t)(i - a.nq) * a.Dr + c];
    }
  } else {
    if (!a.ddelta) return;
    const int t = (blockIdx.x - nfc) * 64 + lane;
    if (t < nd) {
      dst = a.ddelta + t;
      const int c = t % a.Dr, hsel = t / a.Dr;
      if (a.delta_per_head) {  // rows of head hsel: (b * Hkv + hsel) * kbph + chunk
        const int kb = a.k_blocks_per_head, n = a.B * kb;
#pragma unroll 8
        for (int j = w; j < n; j += RW) {
          const int i = ((j / kb) * a.Hkv + hsel) * kb + j % kb;
          s += a.part_k_delta[(int64_t)i * a.Dr + c];
        }
      } else {
#pragma unroll 8
        for (int i = w; i < a.nk; i += RW) s += a.part_k_delta[(int64_t)i * a.Dr + c];
      }
    }
  }
  red[w][lane] = s;
  __syncthreads();
  if (w == 0 && dst) {
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < RW; ++i) tot += red[i][lane];
    *dst = tot;
  }
}

// ---------------------------------------------------------------------------------------------
// Vector forms of prep_kernel (PoPE / FoPE) and prebwd_kernel for bf16 rows with unit inner stride
// and 16-byte aligned row starts, the layout training hands over.  One thread owns 8 consecutive
// columns of one row: 16-byte loads and stores, same per-element arithmetic (bitwise identical
// operands), rows spread over as many threads as there are 8-column chunks.
// ---------------------------------------------------------------------------------------------
// thread t of a row: transform chunk t (cos chunk t, sin chunk t), then content chunks t, t + TPR,
// ... and zero padding chunks the same way; TPR = Dr / 8
// tab_out (query side, phases evaluated here): the rows of (b, h) = (0, 0) also write their cos /
// sin to the [S][2][Dr] phase table, the values launch_phase_table would write
__device__ __forceinline__ void prep_pope_vec_body(const PrepArgs& a, int64_t gid, float* tab_out = nullptr) {
  const int tpr = a.Dr >> 3;
  const int64_t row = gid / tpr;
  const int t = (int)(gid - row * tpr);
  if (row >= (int64_t)a.B * a.H * a.S) return;
  const int s = (int)(row % a.S);
  const int bh = (int)(row / a.S);
  const int h = bh % a.H, b = bh / a.H;
  const float pos = pe_pos(a.start_pos + s, a.pos_round);
  uint16_t* drow = (uint16_t*)a.dst + ((int64_t)bh * (a.dst_rows ? a.dst_rows : a.S) + a.dst_row0 + s) * a.width;
  const u32x4 xv = *(const u32x4*)((const uint16_t*)a.xr + b * a.xr_s[0] + h * a.xr_s[1] + (int64_t)s * a.xr_s[2] + t * 8);
  const f32x4 f0 = *(const f32x4*)(a.freqs + t * 8), f1 = *(const f32x4*)(a.freqs + t * 8 + 4);
  f32x4 d0 = {0.f, 0.f, 0.f, 0.f}, d1 = d0;
  const bool add = a.is_key && a.delta;
  if (add) {
    d0 = *(const f32x4*)(a.delta + h * a.delta_hs + t * 8);
    d1 = *(const f32x4*)(a.delta + h * a.delta_hs + t * 8 + 4);
  }
  float x[8];
  unpack8(xv, x);
  float cv[8], sv[8];
  if (a.tab && !a.is_key) {  // query phases from the table (shared by every batch and head)
    const float* tr = a.tab + (int64_t)s * 2 * a.Dr + t * 8;
    const f32x4 c0 = *(const f32x4*)tr, c1 = *(const f32x4*)(tr + 4);
    const f32x4 s0 = *(const f32x4*)(tr + a.Dr), s1 = *(const f32x4*)(tr + a.Dr + 4);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float mu = softplus_f(x[e]);
      cv[e] = mul_nc(mu, e < 4 ? c0[e] : c1[e - 4]);
      sv[e] = mul_nc(mu, e < 4 ? s0[e] : s1[e - 4]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float mu = softplus_f(x[e]);
      float ph = mul_nc(pos, e < 4 ? f0[e] : f1[e - 4]);
      if (add) ph = add_nc(ph, e < 4 ? d0[e] : d1[e - 4]);
      float sn, cs;
      pe_sincos(ph, sn, cs);
      cv[e] = mul_nc(mu, cs);
      sv[e] = mul_nc(mu, sn);
      if (tab_out && bh == 0) {
        tab_out[(int64_t)s * 2 * a.Dr + t * 8 + e] = cs;
        tab_out[(int64_t)s * 2 * a.Dr + a.Dr + t * 8 + e] = sn;
      }
    }
  }
  *(u32x4*)(drow + a.Dc + t * 8) =
      u32x4{pack_bf2(cv[0], cv[1]), pack_bf2(cv[2], cv[3]), pack_bf2(cv[4], cv[5]), pack_bf2(cv[6], cv[7])};
  *(u32x4*)(drow + a.Dc + a.Dr + t * 8) =
      u32x4{pack_bf2(sv[0], sv[1]), pack_bf2(sv[2], sv[3]), pack_bf2(sv[4], sv[5]), pack_bf2(sv[6], sv[7])};
  if (a.Dc > 0) {
    const uint16_t* xc = (const uint16_t*)a.xc + b * a.xc_s[0] + h * a.xc_s[1] + (int64_t)s * a.xc_s[2];
    for (int j = t; j < a.Dc / 8; j += tpr) *(u32x4*)(drow + j * 8) = *(const u32x4*)(xc + j * 8);
  }
  for (int j = (a.Dc + 2 * a.Dr) / 8 + t; j < a.width / 8; j += tpr) *(u32x4*)(drow + j * 8) = u32x4{0u, 0u, 0u, 0u};
  if (a.cdst) {  // the row's companion copy (KV-cache append: the value row)
    const uint16_t* crow = (const uint16_t*)a.cv + b * a.cv_s[0] + h * a.cv_s[1] + (int64_t)s * a.cv_s[2];
    uint16_t* cd = (uint16_t*)a.cdst + ((int64_t)bh * (a.dst_rows ? a.dst_rows : a.S) + a.dst_row0 + s) * a.cwidth;
    for (int j = t; j < a.cwidth / 8; j += tpr)
      *(u32x4*)(cd + j * 8) = j * 8 < a.cv_cols ? *(const u32x4*)(crow + j * 8) : u32x4{0u, 0u, 0u, 0u};
  }
}

__global__ __launch_bounds__(256) void prep_pope_vec_kernel(PrepArgs a) {
  prep_pope_vec_body(a, (int64_t)blockIdx.x * 256 + threadIdx.x);
}

// The same key-side work for a few rows (a decoded token's cache append): one thread per
// transformed element instead of eight, so a launch of a few hundred rows does not serialise
// eight softplus / sin / cos evaluations per thread; the per-element arithmetic is the vectorised
// body's, so the rows are bitwise the same.  Threads past the elements copy or clear one 16-byte
// chunk each: the content part, the operand row's zero padding and the companion value row.
constexpr int64_t PREP_SMALL_ELEMS = 8192;  // rows x Dr at most, for this path
__global__ __launch_bounds__(256) void prep_pope_small_kernel(PrepArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nrows = (int64_t)a.B * a.H * a.S, nel = nrows * a.Dr;
  const int ncc = a.Dc / 8, npad = (a.width - a.Dc - 2 * a.Dr) / 8, nval = a.cdst ? a.cwidth / 8 : 0;
  const int nch = ncc + npad + nval;
  const int64_t row = gid < nel ? gid / a.Dr : (gid - nel) / (nch > 0 ? nch : 1);
  if (row >= nrows) return;
  const int s = (int)(row % a.S), bh = (int)(row / a.S);
  const int h = bh % a.H, b = bh / a.H;
  const int64_t orow = (int64_t)bh * (a.dst_rows ? a.dst_rows : a.S) + a.dst_row0 + s;
  uint16_t* drow = (uint16_t*)a.dst + orow * a.width;
  if (gid < nel) {
    const int d = (int)(gid - row * a.Dr);
    const uint16_t raw = ((const uint16_t*)a.xr)[b * a.xr_s[0] + h * a.xr_s[1] + (int64_t)s * a.xr_s[2] + d];
    const float mu = softplus_f(__builtin_bit_cast(float, (uint32_t)raw << 16));
    float ph = mul_nc(pe_pos(a.start_pos + s, a.pos_round), a.freqs[d]);
    if (a.delta) ph = add_nc(ph, a.delta[h * a.delta_hs + d]);
    float sn, cs;
    pe_sincos(ph, sn, cs);
    const uint32_t pr = pack_bf2(mul_nc(mu, cs), mul_nc(mu, sn));
    drow[a.Dc + d] = (uint16_t)pr;
    drow[a.Dc + a.Dr + d] = (uint16_t)(pr >> 16);
    return;
  }
  const int j = (int)(gid - nel - row * nch);
  if (j < ncc) {
    const uint16_t* xc = (const uint16_t*)a.xc + b * a.xc_s[0] + h * a.xc_s[1] + (int64_t)s * a.xc_s[2];
    *(u32x4*)(drow + j * 8) = *(const u32x4*)(xc + j * 8);
  } else if (j < ncc + npad) {
    *(u32x4*)(drow + a.Dc + 2 * a.Dr + (j - ncc) * 8) = u32x4{0u, 0u, 0u, 0u};
  } else {
    const int c = j - ncc - npad;
    const uint16_t* crow = (const uint16_t*)a.cv + b * a.cv_s[0] + h * a.cv_s[1] + (int64_t)s * a.cv_s[2];
    uint16_t* cd = (uint16_t*)a.cdst + orow * a.cwidth;
    *(u32x4*)(cd + c * 8) = c * 8 < a.cv_cols ? *(const u32x4*)(crow + c * 8) : u32x4{0u, 0u, 0u, 0u};
  }
}

// one group of TPR = Dv / 8 lanes per padded row (TPR a power of two, groups never straddle a
// wave); Di is the group's fixed-order butterfly sum
__global__ __launch_bounds__(256) void prebwd_vec_kernel(PreBwdArgs a, int lg_tpr) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t prow = gid >> lg_tpr;
  const int t = (int)(gid & ((1 << lg_tpr) - 1));
  if (prow >= (int64_t)a.B * a.H * a.s_pad) return;
  const int s = (int)(prow % a.s_pad);
  const int bh = (int)(prow / a.s_pad);
  if (s >= a.S) {
    if (t == 0) { a.Di[prow] = 0.f; a.L2[prow] = INFINITY; }
    return;
  }
  const int h = bh % a.H, b = bh / a.H;
  const int64_t row = (int64_t)bh * a.S + s;
  const u32x4 dv = *(const u32x4*)((const uint16_t*)a.dout + b * a.do_s[0] + h * a.do_s[1] + (int64_t)s * a.do_s[2] + t * 8);
  const u32x4 ov = *(const u32x4*)((const uint16_t*)a.out + b * a.o_s[0] + h * a.o_s[1] + (int64_t)s * a.o_s[2] + t * 8);
  if (a.dO_op) *(u32x4*)((uint16_t*)a.dO_op + row * a.width + t * 8) = dv;
  float d[8], o[8];
  unpack8(dv, d);
  unpack8(ov, o);
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc += d[e] * o[e];
  for (int m = (1 << lg_tpr) >> 1; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (t == 0) {
    a.Di[prow] = acc;
    const float lv = a.lse[row];
    a.L2[prow] = lv == -INFINITY ? INFINITY : lv * LOG2E;
  }
}

// RoPE / no-PE prologue and its gradient, vector form: thread t of a row owns elements 8t .. 8t + 7
// of the positional part (the chunk of pairs 4t .. 4t + 3, as lane t of prep_kernel / inv_row_kernel
// does), TPR = Dr / 8 threads per row, a power of two up to 64, so that a row's threads sit in one
// wave and exit together.  16-byte loads and stores in any element type; QKNorm's row sums are the
// chunks' sums added by an xor butterfly over the row's threads.  Same per-element arithmetic and
// summation order as the scalar kernels: bitwise equal rows.
__global__ __launch_bounds__(256) void prep_rope_vec_kernel(PrepArgs a, int lg_tpr) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int tpr = 1 << lg_tpr;
  const int64_t row = gid >> lg_tpr;
  const int t = (int)(gid & (tpr - 1));
  if (row >= (int64_t)a.B * a.H * a.S) return;
  const int s = (int)(row % a.S);
  const int bh = (int)(row / a.S);
  const int h = bh % a.H, b = bh / a.H;
  const float pos = pe_pos(a.start_pos + s, a.pos_round);
  const int64_t drow = ((int64_t)bh * (a.dst_rows ? a.dst_rows : a.S) + a.dst_row0 + s) * a.width;
  float x[8], y[8];
  load8(a.xr, b * a.xr_s[0] + h * a.xr_s[1] + (int64_t)s * a.xr_s[2] + t * 8, a.xr_dtype, x);
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float sn, cs;
    rope_pair(a.mode, x[2 * k], x[2 * k + 1], pos, a.mode == 1 ? a.freqs[4 * t + k] : 0.f, a.mscale, y[2 * k],
              y[2 * k + 1], sn, cs);
    ss = add_nc(ss, sq2(y[2 * k], y[2 * k + 1]));
  }
  if (a.l2norm) {
    for (int m = tpr >> 1; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
    const float den = sqrtf(ss) + 1e-6f;
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = y[e] / den;
  }
  store8(a.dst, drow + a.Dc + t * 8, a.dst_dtype, y);
  if (a.Dc > 0) {
    const int64_t xc0 = b * a.xc_s[0] + h * a.xc_s[1] + (int64_t)s * a.xc_s[2];
    for (int j = t; j < a.Dc / 8; j += tpr) {
      float c[8];
      load8(a.xc, xc0 + j * 8, a.xc_dtype, c);
      store8(a.dst, drow + j * 8, a.dst_dtype, c);
    }
  }
  const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j = (a.Dc + a.Dr) / 8 + t; j < a.width / 8; j += tpr) store8(a.dst, drow + j * 8, a.dst_dtype, zero);
}

__global__ __launch_bounds__(256) void inv_rope_vec_kernel(InvArgs a, int lg_tpr) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int tpr = 1 << lg_tpr;
  const int64_t row = gid >> lg_tpr;
  const int t = (int)(gid & (tpr - 1));
  if (row >= (int64_t)a.B * a.H * a.S) return;
  const int s = (int)(row % a.S);
  const int bh = (int)(row / a.S);
  const int h = bh % a.H, b = bh / a.H;
  const float pos = pe_pos(a.start_pos + s, a.pos_round);
  const float* grow = a.g + row * a.width;
  if (a.Dc > 0) {
    const int64_t dc0 = b * a.dxc_s[0] + h * a.dxc_s[1] + (int64_t)s * a.dxc_s[2];
    for (int j = t; j < a.Dc / 8; j += tpr) {
      float c[8];
      load8(grow, j * 8, 1, c);
      store8(a.dxc, dc0 + j * 8, a.dxc_dtype, c);
    }
  }
  float x[8], gv[8], dx[8], fr4[4];
  load8(a.xr, b * a.xr_s[0] + h * a.xr_s[1] + (int64_t)s * a.xr_s[2] + t * 8, a.xr_dtype, x);
  load8(grow, a.Dc + t * 8, 1, gv);
#pragma unroll
  for (int k = 0; k < 4; ++k) fr4[k] = a.mode == 1 ? a.freqs[4 * t + k] : 0.f;
  inv_rope_chunk(a.mode, a.l2norm != 0, fr4, pos, a.mscale, tpr, x, gv, dx);
  store8(a.dxr, b * a.dxr_s[0] + h * a.dxr_s[1] + (int64_t)s * a.dxr_s[2] + t * 8, a.dxr_dtype, dx);
}

bool aligned16(const void* p, int64_t s0, int64_t s1, int64_t s2) {
  return ((uintptr_t)p % 16) == 0 && s0 % 8 == 0 && s1 % 8 == 0 && s2 % 8 == 0;
}

// rows of a view that 16-byte accesses of 8 elements can read: unit inner stride, every row start
// 16-byte aligned for the element type (dtype 1 = fp32, else 16-bit)
static bool rows16(const void* p, int dtype, const int64_t (&st)[4]) {
  const int64_t e = dtype == 1 ? 4 : 2;
  return p && st[3] == 1 && ((uintptr_t)p % 16) == 0 && (st[0] * e) % 16 == 0 && (st[1] * e) % 16 == 0 &&
         (st[2] * e) % 16 == 0;
}

// log2 of the vector RoPE / no-PE kernels' threads per row (Dr / 8, a power of two up to 64), or -1
static int rope_vec_lg(int mode, int Dr, int Dc) {
  if ((mode != 1 && mode != 2) || Dr <= 0 || Dr % 8 != 0 || Dc % 8 != 0 || Dr > 512) return -1;
  const int tpr = Dr / 8;
  if (tpr & (tpr - 1)) return -1;
  int lg = 0;
  while ((1 << lg) < tpr) ++lg;
  return lg;
}

static int prep_rope_vec_lg(const PrepArgs& a) {
  const int lg = rope_vec_lg(a.mode, a.Dr, a.Dc);
  if (lg < 0 || a.cdst || a.width % 8 != 0 || ((uintptr_t)a.dst % 16) != 0 || !rows16(a.xr, a.xr_dtype, a.xr_s) ||
      (a.Dc > 0 && !rows16(a.xc, a.xc_dtype, a.xc_s)))
    return -1;
  return lg;
}

static int inv_rope_vec_lg(const InvArgs& a) {
  const int lg = rope_vec_lg(a.mode, a.Dr, a.Dc);
  if (lg < 0 || a.width % 4 != 0 || ((uintptr_t)a.g % 16) != 0 || !rows16(a.xr, a.xr_dtype, a.xr_s) ||
      !rows16(a.dxr, a.dxr_dtype, a.dxr_s) || (a.Dc > 0 && !rows16(a.dxc, a.dxc_dtype, a.dxc_s)))
    return -1;
  return lg;
}

static bool prep_vec_ok(const PrepArgs& a) {
  return a.mode == 0 && a.dst_dtype == 0 && a.xr_dtype == 0 && a.Dr > 0 && a.Dr % 8 == 0 &&
         a.Dc % 8 == 0 && a.width % 8 == 0 && a.xr_s[3] == 1 &&
         aligned16(a.xr, a.xr_s[0], a.xr_s[1], a.xr_s[2]) && ((uintptr_t)a.dst % 16) == 0 &&
         ((uintptr_t)a.freqs % 16) == 0 &&
         (!a.is_key || !a.delta || (((uintptr_t)a.delta % 16) == 0 && a.delta_hs % 4 == 0)) &&
         (a.Dc == 0 || (a.xc_dtype == 0 && a.xc_s[3] == 1 && aligned16(a.xc, a.xc_s[0], a.xc_s[1], a.xc_s[2])));
}

bool prep_vec_copy_ok(const PrepArgs& a) {
  return prep_vec_ok(a) && a.cv && a.cdst && a.cv_s[3] == 1 && aligned16(a.cv, a.cv_s[0], a.cv_s[1], a.cv_s[2]) &&
         ((uintptr_t)a.cdst % 16) == 0 && a.cv_cols % 8 == 0 && a.cwidth % 8 == 0 && a.cv_cols <= a.cwidth;
}

bool prep_vec_query_ok(const PrepArgs& a) {
  return prep_vec_ok(a) && !a.is_key && a.Dc == 0 && a.width == 2 * a.Dr;
}

int launch_prep(const PrepArgs& a, hipStream_t s) {
  const int64_t nrows = (int64_t)a.B * a.H * a.S;
  const bool vec = prep_vec_ok(a);
  if (a.cdst && !(vec && prep_vec_copy_ok(a))) return -2;  // the caller checks prep_vec_copy_ok first
  if (vec && a.is_key && nrows * a.Dr <= PREP_SMALL_ELEMS) {
    const int64_t nch = a.Dc / 8 + (a.width - a.Dc - 2 * a.Dr) / 8 + (a.cdst ? a.cwidth / 8 : 0);
    const int64_t nthr = nrows * (a.Dr + nch);
    hipLaunchKernelGGL(prep_pope_small_kernel, dim3((unsigned)((nthr + 255) / 256)), dim3(256), 0, s, a);
  } else if (vec) {
    const int64_t nthr = nrows * (a.Dr / 8);
    hipLaunchKernelGGL(prep_pope_vec_kernel, dim3((unsigned)((nthr + 255) / 256)), dim3(256), 0, s, a);
  } else if (const int lg = prep_rope_vec_lg(a); lg >= 0) {
    const int64_t nthr = nrows << lg;
    hipLaunchKernelGGL(prep_rope_vec_kernel, dim3((unsigned)((nthr + 255) / 256)), dim3(256), 0, s, a, lg);
  } else {
    hipLaunchKernelGGL(prep_kernel, dim3((unsigned)((nrows + 3) / 4)), dim3(256), 0, s, a);
  }
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

__device__ __forceinline__ void phase_table_body(const float* freqs, int start, int S, int Dr, int pos_round,
                                                 float* tab, int64_t gid) {
  if (gid >= (int64_t)S * Dr) return;
  const int s = (int)(gid / Dr), c = (int)(gid % Dr);
  float sn, cs;
  pe_sincos(mul_nc(pe_pos(start + s, pos_round), freqs[c]), sn, cs);
  tab[(int64_t)s * 2 * Dr + c] = cs;
  tab[(int64_t)s * 2 * Dr + Dr + c] = sn;
}

__global__ __launch_bounds__(256) void phase_table_kernel(const float* freqs, int start, int S, int Dr, int pos_round,
                                                          float* tab) {
  phase_table_body(freqs, start, S, Dr, pos_round, tab, (int64_t)blockIdx.x * 256 + threadIdx.x);
}

// the key prologue (vectorised path) and the query phase table in one launch: blocks below nblk
// transform key rows, the rest write the table; the two share no data
__global__ __launch_bounds__(256) void prep_vec_and_table_kernel(PrepArgs a, unsigned nblk, const float* freqs,
                                                                 int start, int S, int Dr, int pos_round, float* tab) {
  if (blockIdx.x < nblk) prep_pope_vec_body(a, (int64_t)blockIdx.x * 256 + threadIdx.x);
  else phase_table_body(freqs, start, S, Dr, pos_round, tab, (int64_t)(blockIdx.x - nblk) * 256 + threadIdx.x);
}

// Both sides of a small prologue in one launch: blocks below nkblk transform key rows, the rest
// query rows, which evaluate their own phases (no table to wait for) and, in the rows of (0, 0),
// write the phase table.  The per-element arithmetic is the two-launch path's, so every value is
// bitwise the same.
__global__ __launch_bounds__(256) void prep_qk_vec_kernel(PrepArgs ak, PrepArgs aq, unsigned nkblk, float* tab) {
  if (blockIdx.x < nkblk) prep_pope_vec_body(ak, (int64_t)blockIdx.x * 256 + threadIdx.x);
  else prep_pope_vec_body(aq, (int64_t)(blockIdx.x - nkblk) * 256 + threadIdx.x, tab);
}

// Query rows without a content part or padding, QHG heads per thread: thread (b, head group, s,
// chunk t) evaluates the sin / cos of its 8 phases fl(pos * freq) once, then transforms chunk t of
// the rows (b, h, s) of the group's heads, whose x chunks it loads up front.  A query phase does
// not depend on the head, so the table (cos row then sin row per position) that the dQ epilogue
// reads is written by the threads of (b, group) = (0, 0), and no table read sits on this path.
// Per element the arithmetic is prep_pope_vec_body's, so the rows and the table are bitwise those
// of the table launch plus the table-reading query launch.
constexpr int QHG = 8;
__device__ __forceinline__ void prep_pope_qheads_body(const PrepArgs& a, int64_t gid, float* tab) {
  const int tpr = a.Dr >> 3, ngrp = (a.H + QHG - 1) / QHG;
  const int64_t unit = gid / tpr;
  const int t = (int)(gid - unit * tpr);
  if (unit >= (int64_t)a.B * ngrp * a.S) return;
  const int s = (int)(unit % a.S);
  const int64_t bg = unit / a.S;
  const int hg = (int)(bg % ngrp), b = (int)(bg / ngrp), h0 = hg * QHG;
  const uint16_t* xb = (const uint16_t*)a.xr + b * a.xr_s[0] + (int64_t)s * a.xr_s[2] + t * 8;
  u32x4 xv[QHG];
#pragma unroll
  for (int j = 0; j < QHG; ++j)
    if (h0 + j < a.H) xv[j] = *(const u32x4*)(xb + (int64_t)(h0 + j) * a.xr_s[1]);
  const float pos = pe_pos(a.start_pos + s, a.pos_round);
  const f32x4 f0 = *(const f32x4*)(a.freqs + t * 8), f1 = *(const f32x4*)(a.freqs + t * 8 + 4);
  float cs[8], sn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) pe_sincos(mul_nc(pos, e < 4 ? f0[e] : f1[e - 4]), sn[e], cs[e]);
  if (tab && (b | hg) == 0) {
    float* tr = tab + (int64_t)s * 2 * a.Dr + t * 8;
    *(f32x4*)tr = f32x4{cs[0], cs[1], cs[2], cs[3]};
    *(f32x4*)(tr + 4) = f32x4{cs[4], cs[5], cs[6], cs[7]};
    *(f32x4*)(tr + a.Dr) = f32x4{sn[0], sn[1], sn[2], sn[3]};
    *(f32x4*)(tr + a.Dr + 4) = f32x4{sn[4], sn[5], sn[6], sn[7]};
  }
#pragma unroll
  for (int j = 0; j < QHG; ++j) {
    const int h = h0 + j;
    if (h >= a.H) break;
    float x[8], cv[8], sv[8];
    unpack8(xv[j], x);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float mu = softplus_f(x[e]);
      cv[e] = mul_nc(mu, cs[e]);
      sv[e] = mul_nc(mu, sn[e]);
    }
    uint16_t* drow = (uint16_t*)a.dst + ((int64_t)(b * a.H + h) * (a.dst_rows ? a.dst_rows : a.S) + a.dst_row0 + s) * a.width;
    *(u32x4*)(drow + t * 8) =
        u32x4{pack_bf2(cv[0], cv[1]), pack_bf2(cv[2], cv[3]), pack_bf2(cv[4], cv[5]), pack_bf2(cv[6], cv[7])};
    *(u32x4*)(drow + a.Dr + t * 8) =
        u32x4{pack_bf2(sv[0], sv[1]), pack_bf2(sv[2], sv[3]), pack_bf2(sv[4], sv[5]), pack_bf2(sv[6], sv[7])};
  }
}

// The whole PoPE prologue in one launch: nkblk blocks of key rows (vector-bound: a sin / cos and a
// softplus per element) interleaved evenly with nqblk blocks of query rows (memory-bound: a
// softplus per element, phases shared over QHG heads), so that both kinds share every CU.  Block i
// is the query block cq(i) = floor(i * nqblk / n) when cq(i + 1) > cq(i), else the key block
// i - cq(i); over the n = nkblk + nqblk blocks this takes each index of either kind once.
__global__ __launch_bounds__(256) void prep_k_qheads_kernel(PrepArgs ak, PrepArgs aq, unsigned nkblk, unsigned nqblk,
                                                            float* tab) {
  const uint64_t i = blockIdx.x, n = (uint64_t)nkblk + nqblk;
  const uint64_t cq = i * nqblk / n, cq1 = (i + 1) * nqblk / n;
  if (cq1 > cq) prep_pope_qheads_body(aq, (int64_t)cq * 256 + threadIdx.x, tab);
  else prep_pope_vec_body(ak, (int64_t)(i - cq) * 256 + threadIdx.x);
}

// prologues of at most this many 256-thread blocks (keys and queries together) take one launch:
// they are bound by launch latency, not by the queries' extra sin / cos
constexpr int64_t PREP_QK_MAX_BLOCKS = 1024;

int launch_prep_k_qheads(const PrepArgs& ak, const PrepArgs& aq, float* tab, hipStream_t s) {
  if (!prep_vec_ok(ak) || !prep_vec_query_ok(aq) || ak.cdst || aq.cdst || aq.tab || !ak.is_key || aq.Dr != ak.Dr ||
      !tab || (uintptr_t)tab % 16 != 0)
    return 1;
  const int64_t nk = (int64_t)ak.B * ak.H * ak.S * (ak.Dr / 8);
  const int64_t nq = (int64_t)aq.B * ((aq.H + QHG - 1) / QHG) * aq.S * (aq.Dr / 8);
  const int64_t nkblk = (nk + 255) / 256, nqblk = (nq + 255) / 256;
  if (nk == 0 || nq == 0) return 1;
  if (nkblk + nqblk > 0x7fffffff) return -2;
  hipLaunchKernelGGL(prep_k_qheads_kernel, dim3((unsigned)(nkblk + nqblk)), dim3(256), 0, s, ak, aq, (unsigned)nkblk,
                     (unsigned)nqblk, tab);
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

int launch_prep_qk(const PrepArgs& ak, const PrepArgs& aq, float* tab, hipStream_t s) {
  if (!prep_vec_ok(ak) || !prep_vec_ok(aq) || ak.cdst || aq.cdst || aq.tab || !ak.is_key || aq.is_key ||
      aq.Dr != ak.Dr)
    return 1;
  const int64_t nk = (int64_t)ak.B * ak.H * ak.S * (ak.Dr / 8), nq = (int64_t)aq.B * aq.H * aq.S * (aq.Dr / 8);
  const int64_t nkblk = (nk + 255) / 256, nqblk = (nq + 255) / 256;
  if (nkblk + nqblk > PREP_QK_MAX_BLOCKS || nk * 8 <= PREP_SMALL_ELEMS || nk == 0 || nq == 0) return 1;
  hipLaunchKernelGGL(prep_qk_vec_kernel, dim3((unsigned)(nkblk + nqblk)), dim3(256), 0, s, ak, aq, (unsigned)nkblk,
                     tab);
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

int launch_prep_and_table(const PrepArgs& a, const float* freqs, int start, int S, int Dr, int pos_round, float* tab,
                          hipStream_t s) {
  const int64_t nrows = (int64_t)a.B * a.H * a.S;
  const int64_t nt = (int64_t)S * Dr;
  if (!prep_vec_ok(a) || a.cdst || nt == 0) {
    int rc = launch_phase_table(freqs, start, S, Dr, pos_round, tab, s);
    return rc ? rc : launch_prep(a, s);
  }
  const int64_t nblk = (nrows * (a.Dr / 8) + 255) / 256, ntab = (nt + 255) / 256;
  if (nblk + ntab > 0x7fffffff) return -2;
  hipLaunchKernelGGL(prep_vec_and_table_kernel, dim3((unsigned)(nblk + ntab)), dim3(256), 0, s, a, (unsigned)nblk,
                     freqs, start, S, Dr, pos_round, tab);
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

int launch_phase_table(const float* freqs, int start, int S, int Dr, int pos_round, float* tab, hipStream_t s) {
  const int64_t n = (int64_t)S * Dr;
  if (n == 0) return 0;
  hipLaunchKernelGGL(phase_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, freqs, start, S, Dr, pos_round,
                     tab);
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

int launch_prebwd(const PreBwdArgs& a, hipStream_t s) {
  const int tpr = a.Dv / 8;
  const bool vec = a.dout_dtype == 0 && a.out_dtype == 0 && a.Dv % 8 == 0 && tpr <= 64 && (tpr & (tpr - 1)) == 0 &&
                   a.do_s[3] == 1 && a.o_s[3] == 1 && aligned16(a.dout, a.do_s[0], a.do_s[1], a.do_s[2]) &&
                   aligned16(a.out, a.o_s[0], a.o_s[1], a.o_s[2]) &&
                   (!a.dO_op || (a.op_dtype == 0 && a.width == a.Dv && ((uintptr_t)a.dO_op % 16) == 0));
  const int64_t nrows = (int64_t)a.B * a.H * a.s_pad;
  if (vec) {
    int lg = 0;
    while ((1 << lg) < tpr) ++lg;
    hipLaunchKernelGGL(prebwd_vec_kernel, dim3((unsigned)((nrows * tpr + 255) / 256)), dim3(256), 0, s, a, lg);
  } else {
    hipLaunchKernelGGL(prebwd_kernel, dim3((unsigned)((nrows + 3) / 4)), dim3(256), 0, s, a);
  }
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

int inv_blocks(int B, int H, int S, int rows_per_block) {
  return B * H * ((S + rows_per_block - 1) / rows_per_block);
}

int launch_inv(const InvArgs& a, int* nblocks_out, hipStream_t s) {
  if (a.mode == 0) {
    const int nb = inv_blocks(a.B, a.H, a.S, a.rows_per_block);
    if (nblocks_out) *nblocks_out = nb;
    if (a.Dr <= 32) hipLaunchKernelGGL(inv_pope_kernel<32>, dim3(nb), dim3(256), 0, s, a);
    else if (a.Dr <= 64) hipLaunchKernelGGL(inv_pope_kernel<64>, dim3(nb), dim3(256), 0, s, a);
    else if (a.Dr <= 128) hipLaunchKernelGGL(inv_pope_kernel<128>, dim3(nb), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(inv_pope_kernel<256>, dim3(nb), dim3(256), 0, s, a);
  } else {
    if (nblocks_out) *nblocks_out = 0;
    const int64_t nrows = (int64_t)a.B * a.H * a.S;
    if (const int lg = inv_rope_vec_lg(a); lg >= 0)
      hipLaunchKernelGGL(inv_rope_vec_kernel, dim3((unsigned)(((nrows << lg) + 255) / 256)), dim3(256), 0, s, a, lg);
    else
      hipLaunchKernelGGL(inv_row_kernel, dim3((unsigned)((nrows + 3) / 4)), dim3(256), 0, s, a);
  }
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

int launch_reduce(const ReduceArgs& a, hipStream_t s) {
  const int nd = a.delta_per_head ? a.Hkv * a.Dr : a.Dr;
  const int nblk = (a.Dr + 63) / 64 + (nd + 63) / 64;
  hipLaunchKernelGGL(reduce_kernel, dim3(nblk), dim3(RW * 64), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

}  // namespace pe
