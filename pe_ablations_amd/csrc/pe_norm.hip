// RMSNorm kernels (HBM-bound, one wave per row / token, WPB rows per workgroup).
//
//   rmsnorm_kernel         y = (x * rsqrt(mean(x^2) + eps)).type_as(x) * w over the last dim
//                          (src/model/normalization.py:7-27): statistics and products in fp32, the
//                          normalised value rounded to x's dtype, the product with the weight
//                          rounded to bf16 only when x and w are both bf16 (torch's type promotion)
//   prep_pope_norm_kernel  the same RMSNorm over all H*Dr features of a token's position
//                          projection (qr_norm / kr_norm, src/model/fpope_attention.py:88-90,
//                          132-137) followed by the PoPE transform of each head's Dr slice
//                          (src/model/pope.py:124-183), written straight into the attention
//                          kernels' operand rows [content | mu cos | mu sin | 0]
//
// Each lane owns CPL 8-element chunks of its wave's row in registers (chunk c = lane + 64 k), so
// the row is read from HBM once and all of a lane's loads are in flight together.  The sum of
// squares is reduced by the wave's xor butterfly, which leaves the same value in every lane and
// depends on nothing but the row, so no LDS and no barrier are involved and the waves of a
// workgroup (rows of their own) never wait for each other.
#include "pe_common.h"
#include "pe_internal.h"

namespace pe {

constexpr int WPB = 4;      // waves, i.e. rows, per workgroup
constexpr int MAXCPL = 16;  // chunks per lane: rows up to 64 * MAXCPL * 8 = 8192 elements

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// y's dtype code under torch's type promotion of (normalised value in x's dtype) * weight: the
// 16-bit type when x and w share it, else fp32 (bf16 * fp16 promotes to fp32 as well)
__host__ __device__ inline int norm_y_dtype(int x_dtype, int w_dtype) {
  return (x_dtype == w_dtype && x_dtype != 1) ? x_dtype : 1;
}

// normalise one chunk in place: n = fl(x * r) rounded to x's dtype, y = fl(n * w) rounded to y's
__device__ __forceinline__ void norm_chunk(float (&x)[8], float r, int x_dtype, const void* w, int w_dtype,
                                           int64_t wi) {
  float wv[8];
  load8(w, wi, w_dtype, wv);
  const int ydt = norm_y_dtype(x_dtype, w_dtype);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float n = round_to(x[e] * r, x_dtype);
    x[e] = round_to(n * wv[e], ydt);
  }
}

template <int CPL>
__global__ __launch_bounds__(WPB * 64) void rmsnorm_kernel(NormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * WPB + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // whole waves: the kernel has no barrier
  const int nch = a.n >> 3;
  float x[CPL][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = lane + k * 64;
    if (c < nch) {
      load8(a.x, row * a.x_rs + c * 8, a.x_dtype, x[k]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[k][e] * x[k][e];
    }
  }
  // torch: mean = sum * (1/n), then rsqrt(mean + eps)
  const float r = rsqrtf(wave_sum(ss) * (1.0f / (float)a.n) + a.eps);
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = lane + k * 64;
    if (c < nch) {
      norm_chunk(x[k], r, a.x_dtype, a.w, a.w_dtype, c * 8);
      store8(a.y, row * a.y_rs + c * 8, a.y_dtype, x[k]);
    }
  }
}

template <int DDT, int CPL>
__global__ __launch_bounds__(WPB * 64) void prep_pope_norm_kernel(PrepArgs a) {
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * WPB + (threadIdx.x >> 6);
  if (tok >= a.B * a.S) return;  // whole waves: the kernel has no barrier
  const int tpr = a.Dr >> 3;
  const int nch = a.H * tpr;
  const int b = tok / a.S, s = tok - b * a.S;
  const float pos = pe_pos(a.start_pos + s, a.pos_round);
  float x[CPL][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = lane + k * 64;
    if (c < nch) {
      const int h = c / tpr, t = c - h * tpr;
      load8(a.xr, b * a.xr_s[0] + h * a.xr_s[1] + (int64_t)s * a.xr_s[2] + t * 8, a.xr_dtype, x[k]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[k][e] * x[k][e];
    }
  }
  const float r = rsqrtf(wave_sum(ss) * (1.0f / (float)(a.H * a.Dr)) + a.norm_eps);
  const bool add = a.is_key && a.delta;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = lane + k * 64;
    if (c < nch) {
      const int h = c / tpr, t = c - h * tpr;
      norm_chunk(x[k], r, a.xr_dtype, a.norm_w, a.norm_w_dtype, c * 8);
      const f32x4 f0 = *(const f32x4*)(a.freqs + t * 8), f1 = *(const f32x4*)(a.freqs + t * 8 + 4);
      f32x4 d0 = {0.f, 0.f, 0.f, 0.f}, d1 = d0;
      if (add) {
        d0 = *(const f32x4*)(a.delta + h * a.delta_hs + t * 8);
        d1 = *(const f32x4*)(a.delta + h * a.delta_hs + t * 8 + 4);
      }
      float cv[8], sv[8];
      if (a.tab && !a.is_key) {  // query phases from the table (the same values pe_sincos gives)
        const float* tr = a.tab + (int64_t)s * 2 * a.Dr + t * 8;
        const f32x4 c0 = *(const f32x4*)tr, c1 = *(const f32x4*)(tr + 4);
        const f32x4 s0 = *(const f32x4*)(tr + a.Dr), s1 = *(const f32x4*)(tr + a.Dr + 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float mu = softplus_f(x[k][e]);
          cv[e] = mul_nc(mu, e < 4 ? c0[e] : c1[e - 4]);
          sv[e] = mul_nc(mu, e < 4 ? s0[e] : s1[e - 4]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float mu = softplus_f(x[k][e]);
          float ph = mul_nc(pos, e < 4 ? f0[e] : f1[e - 4]);
          if (add) ph = add_nc(ph, e < 4 ? d0[e] : d1[e - 4]);
          float sn, cs;
          pe_sincos(ph, sn, cs);
          cv[e] = mul_nc(mu, cs);
          sv[e] = mul_nc(mu, sn);
        }
      }
      const int64_t drow = ((int64_t)(b * a.H + h) * a.S + s) * a.width;
      store8(a.dst, drow + a.Dc + t * 8, DDT, cv);
      store8(a.dst, drow + a.Dc + a.Dr + t * 8, DDT, sv);
    }
  }
  if (a.Dc > 0) {  // content part: converted copy
    const int cpr = a.Dc >> 3;
    for (int c = lane; c < a.H * cpr; c += 64) {
      const int h = c / cpr, j = c - h * cpr;
      float v[8];
      load8(a.xc, b * a.xc_s[0] + h * a.xc_s[1] + (int64_t)s * a.xc_s[2] + j * 8, a.xc_dtype, v);
      store8(a.dst, ((int64_t)(b * a.H + h) * a.S + s) * a.width + j * 8, DDT, v);
    }
  }
  const int used = a.Dc + 2 * a.Dr;
  const int ppr = (a.width - used) >> 3;
  for (int c = lane; c < a.H * ppr; c += 64) {
    const int h = c / ppr, j = c - h * ppr;
    const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    store8(a.dst, ((int64_t)(b * a.H + h) * a.S + s) * a.width + used + j * 8, DDT, z);
  }
}

// chunks per lane for a row of nch 8-element chunks: the smallest instantiated count that covers it
static int chunks_per_lane(int nch) {
  int c = 1;
  while (c < MAXCPL && 64 * c < nch) c *= 2;
  return c;
}

// calls f with the chunk count as a compile-time constant (a power of two up to MAXCPL)
template <typename F>
static void with_cpl(int cpl, F&& f) {
  switch (cpl) {
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 8: f(std::integral_constant<int, 8>{}); break;
    default: f(std::integral_constant<int, 16>{}); break;
  }
}

// 16-byte aligned base and 8-element chunks that stay 16-byte aligned along every stride
static bool rows_aligned(const void* p, int dtype, int64_t s0, int64_t s1, int64_t s2) {
  const int64_t q = dtype == 1 ? 4 : 8;
  return ((uintptr_t)p % 16) == 0 && s0 % q == 0 && s1 % q == 0 && s2 % q == 0;
}

int launch_rmsnorm(const NormArgs& a, hipStream_t s) {
  if (a.rows <= 0 || a.rows > 0x7fffffff || a.n <= 0) return -2;
  if (a.n % 8 != 0 || a.n > 64 * MAXCPL * 8) return -3;
  if (a.x_dtype < 0 || a.x_dtype > 2 || a.w_dtype < 0 || a.w_dtype > 2) return -4;
  if (a.y_dtype != norm_y_dtype(a.x_dtype, a.w_dtype)) return -4;
  if (!rows_aligned(a.x, a.x_dtype, a.x_rs, 0, 0) || !rows_aligned(a.y, a.y_dtype, a.y_rs, 0, 0) ||
      ((uintptr_t)a.w % 16) != 0)
    return -5;
  const dim3 grid((unsigned)((a.rows + WPB - 1) / WPB));
  with_cpl(chunks_per_lane(a.n >> 3), [&](auto c) {
    hipLaunchKernelGGL((rmsnorm_kernel<decltype(c)::value>), grid, dim3(WPB * 64), 0, s, a);
  });
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

// RMSNorm backward (the autograd of rmsnorm_kernel's expression, src/model/normalization.py:22-27,
// in fp32): with r = rsqrt(mean(x^2) + eps) (the forward's sum, in the forward's order) and
// nc = (x r) rounded to x's dtype,
//   gc = (dy w) rounded to x's dtype   (the product in y's dtype, the gradient of the cast value)
//   (y's dtype: the 16-bit type when x and w share it, else fp32)
//   c  = sum_j gc_j x_j                 (the gradient reaching r through x * r)
//   dx = gc r + x (2/n) (-r^3 c / 2)    (rsqrt's and mean's gradients), rounded to x's dtype
//   dw = sum over rows of (dy nc)       (each product rounded to y's dtype when y is bf16; the sum
//                                         in fp32, rounded to the weight's dtype)
// One wave per row, rpw consecutive rows per wave.  Each lane accumulates dw for its own chunks
// over its rows; the WPB waves of a workgroup add theirs through LDS in wave order, one 512-feature
// slab at a time, into the workgroup's partial row, which rmsnorm_dw_reduce_kernel sums in a
// fixed order.  Fixed order throughout: the result is bitwise reproducible.
template <int CPL>
__global__ __launch_bounds__(WPB * 64) void rmsnorm_bwd_kernel(NormBwdArgs a) {
  __shared__ __attribute__((aligned(16))) float slab[WPB][64 * 8];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nch = a.n >> 3;
  const int ydt = norm_y_dtype(a.x_dtype, a.w_dtype);
  float dwa[CPL][8];
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) dwa[k][e] = 0.f;
  const int64_t row0 = ((int64_t)blockIdx.x * WPB + w) * a.rpw;
  for (int i = 0; i < a.rpw; ++i) {
    const int64_t row = row0 + i;
    if (row >= a.rows) break;
    float x[CPL][8];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int c = lane + k * 64;
      if (c < nch) {
        load8(a.x, row * a.x_rs + c * 8, a.x_dtype, x[k]);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += x[k][e] * x[k][e];
      }
    }
    const float r = rsqrtf(wave_sum(ss) * (1.0f / (float)a.n) + a.eps);
    float gc[CPL][8];
    float cs = 0.f;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int c = lane + k * 64;
      if (c < nch) {
        float dy[8], wv[8];
        load8(a.dy, row * a.dy_rs + c * 8, ydt, dy);
        load8(a.w, c * 8, a.w_dtype, wv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float g = round_to(round_to(dy[e] * wv[e], ydt), a.x_dtype);
          gc[k][e] = g;
          cs += g * x[k][e];
          const float nc = round_to(x[k][e] * r, a.x_dtype);
          dwa[k][e] += round_to(dy[e] * nc, ydt);
        }
      }
    }
    const float cr = wave_sum(cs) * (-0.5f * r * r * r) * (2.0f / (float)a.n);
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int c = lane + k * 64;
      if (c < nch) {
        float dx[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) dx[e] = gc[k][e] * r + x[k][e] * cr;
        store8(a.dx, row * a.dx_rs + c * 8, a.x_dtype, dx);
      }
    }
  }
  // the workgroup's partial dw row: waves add in order, 512 features (one chunk per lane) a slab
  float* prow = a.part + (int64_t)blockIdx.x * a.n;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    if (64 * k >= nch) break;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 8; ++e) slab[w][lane * 8 + e] = dwa[k][e];
    __syncthreads();
    for (int f = threadIdx.x; f < 64 * 8; f += WPB * 64) {
      const int c = k * 64 + f / 8;
      if (c < nch) {
        float acc = slab[0][f];
#pragma unroll
        for (int ww = 1; ww < WPB; ++ww) acc += slab[ww][f];
        prow[k * 512 + f] = acc;
      }
    }
  }
}

// dw[f] = the groups' partial rows summed in a fixed order, rounded to dw's dtype: a workgroup of
// 1024 threads takes 32 features, its 32 waves' half-rows (slice j = thread / 32) sum the groups
// j, j + 32, j + 64, ... in increasing order with eight loads in flight, and one wave adds the 32
// slice sums in slice order.  (One thread per feature walking every group in turn waited on each
// load: 118 us per call for 512 groups.)
__global__ __launch_bounds__(1024) void rmsnorm_dw_reduce_kernel(const float* __restrict__ part, int groups, int n,
                                                                 void* dw, int dw_dtype) {
  __shared__ float red[32][33];
  const int lc = threadIdx.x & 31, j = threadIdx.x >> 5;
  const int f = blockIdx.x * 32 + lc;
  float acc = 0.f;
  if (f < n) {
    int g = j;
    for (; g + 7 * 32 < groups; g += 8 * 32) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = part[(int64_t)(g + u * 32) * n + f];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += v[u];
    }
    for (; g < groups; g += 32) acc += part[(int64_t)g * n + f];
  }
  red[j][lc] = acc;
  __syncthreads();
  if (j == 0 && f < n) {
    float t = red[0][lc];
    for (int i = 1; i < 32; ++i) t += red[i][lc];
    store_from_float(dw, f, dw_dtype, t);
  }
}

// rows per wave: about two workgroups per compute unit, at most 32 rows per wave
static int bwd_rows_per_wave(int64_t rows, int n_cu) {
  const int64_t waves = (int64_t)WPB * 2 * (n_cu > 0 ? n_cu : 256);
  int64_t r = (rows + waves - 1) / waves;
  return (int)(r < 1 ? 1 : (r > 32 ? 32 : r));
}

int64_t rmsnorm_bwd_part_floats(int64_t rows, int n, int n_cu) {
  const int64_t per = (int64_t)WPB * bwd_rows_per_wave(rows, n_cu);
  return ((rows + per - 1) / per) * (int64_t)n;
}

int launch_rmsnorm_bwd(NormBwdArgs a, int n_cu, hipStream_t s) {
  if (a.rows <= 0 || a.rows > 0x7fffffff || a.n <= 0) return -2;
  if (a.n % 8 != 0 || a.n > 64 * MAXCPL * 8) return -3;
  if (a.x_dtype < 0 || a.x_dtype > 2 || a.w_dtype < 0 || a.w_dtype > 2) return -4;
  if (a.dw_dtype != a.w_dtype) return -4;
  const int ydt = norm_y_dtype(a.x_dtype, a.w_dtype);
  if (!rows_aligned(a.x, a.x_dtype, a.x_rs, 0, 0) || !rows_aligned(a.dy, ydt, a.dy_rs, 0, 0) ||
      !rows_aligned(a.dx, a.x_dtype, a.dx_rs, 0, 0) || ((uintptr_t)a.w % 16) != 0 || ((uintptr_t)a.part % 16) != 0)
    return -5;
  a.rpw = bwd_rows_per_wave(a.rows, n_cu);
  const int64_t per = (int64_t)WPB * a.rpw;
  const int groups = (int)((a.rows + per - 1) / per);
  with_cpl(chunks_per_lane(a.n >> 3), [&](auto c) {
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<decltype(c)::value>), dim3(groups), dim3(WPB * 64), 0, s, a);
  });
  if (hipGetLastError() != hipSuccess) return -7;
  hipLaunchKernelGGL(rmsnorm_dw_reduce_kernel, dim3((a.n + 31) / 32), dim3(1024), 0, s, (const float*)a.part, groups,
                     a.n, a.dw, a.dw_dtype);
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

// SwiGLU of the feed-forward block, silu(gate) * x over bf16 (src/model/ffn.py:17-27), as torch
// evaluates F.silu(gate) * x: the silu in fp32 as g / (1 + exp(-g)) rounded to bf16, then the
// product in fp32 rounded to bf16, so the result is bitwise torch's; one pass over the two inputs
// instead of two kernels and an intermediate tensor.  Eight elements per thread.
__global__ __launch_bounds__(256) void swiglu_kernel(const u32x4* __restrict__ x, const u32x4* __restrict__ gate,
                                                     u32x4* __restrict__ out, int64_t n8) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  float xf[8], gf[8];
  unpack8(x[i], xf);
  unpack8(gate[i], gf);
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = round_bf16(gf[e] / (1.f + expf(-gf[e]))) * xf[e];
  out[i] = u32x4{pack_bf2(r[0], r[1]), pack_bf2(r[2], r[3]), pack_bf2(r[4], r[5]), pack_bf2(r[6], r[7])};
}

int launch_swiglu(const void* x, const void* gate, void* out, int64_t n, hipStream_t s) {
  if (n < 0 || n % 8 != 0) return -2;
  if (((uintptr_t)x | (uintptr_t)gate | (uintptr_t)out) % 16) return -5;
  const int64_t n8 = n / 8;
  if (n8 == 0) return 0;
  if ((n8 + 255) / 256 > 0x7fffffff) return -2;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s, (const u32x4*)x,
                     (const u32x4*)gate, (u32x4*)out, n8);
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

int launch_prep_norm(const PrepArgs& a, hipStream_t s) {
  if (a.mode != 0 || !a.norm_w || a.norm_w_dtype < 0 || a.norm_w_dtype > 2 || a.xr_dtype < 0 || a.xr_dtype > 2 ||
      a.dst_dtype < 0 || a.dst_dtype > 2)
    return -4;
  if (a.dst_rows != 0 || a.dst_row0 != 0) return -2;  // writes contiguous (B, H, S, width) rows only
  if (a.Dr <= 0 || a.Dr % 8 != 0 || a.Dc % 8 != 0 || a.width % 8 != 0 || a.H * (a.Dr / 8) > 64 * MAXCPL) return -3;
  if ((int64_t)a.B * a.S > 0x7fffffff) return -2;
  const bool ok = a.xr_s[3] == 1 && rows_aligned(a.xr, a.xr_dtype, a.xr_s[0], a.xr_s[1], a.xr_s[2]) &&
                  ((uintptr_t)a.dst % 16) == 0 && ((uintptr_t)a.freqs % 16) == 0 && ((uintptr_t)a.norm_w % 16) == 0 &&
                  (!a.is_key || !a.delta || (((uintptr_t)a.delta % 16) == 0 && a.delta_hs % 4 == 0)) &&
                  (a.Dc == 0 || (a.xc_s[3] == 1 && rows_aligned(a.xc, a.xc_dtype, a.xc_s[0], a.xc_s[1], a.xc_s[2])));
  if (!ok) return -5;
  const dim3 grid((unsigned)(((int64_t)a.B * a.S + WPB - 1) / WPB));
  with_cpl(chunks_per_lane(a.H * (a.Dr / 8)), [&](auto c) {
    constexpr int C = decltype(c)::value;
    if (a.dst_dtype == 0) hipLaunchKernelGGL((prep_pope_norm_kernel<0, C>), grid, dim3(WPB * 64), 0, s, a);
    else if (a.dst_dtype == 2) hipLaunchKernelGGL((prep_pope_norm_kernel<2, C>), grid, dim3(WPB * 64), 0, s, a);
    else hipLaunchKernelGGL((prep_pope_norm_kernel<1, C>), grid, dim3(WPB * 64), 0, s, a);
  });
  return hipGetLastError() == hipSuccess ? 0 : -7;
}

}  // namespace pe
