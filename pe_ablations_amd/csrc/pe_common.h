// Device-side building blocks shared by the gfx950 PE-attention kernels.
//
// Matrix core layout (v_mfma_f32_32x32x16_bf16 / _f16 / v_mfma_f32_32x32x2_f32, wave64), lane l, l32 = l%32,
// g = l/32:
//   A operand : row l32, contraction elements g*EPL .. g*EPL+EPL-1 of the current KC-wide step
//   B operand : col l32, same contraction elements
//   C / D     : 16 floats; value j sits at row (j/4)*8 + g*4 + j%4, col l32
// Each lane feeds one 16-byte fragment per operand per step: 8 bf16 (KC = 16, one MFMA) or
// 4 fp32 (KC = 8, four 32x32x2 MFMAs whose contraction pairs are {e, 4+e}).
//
// A C tile is turned into the contraction operand of the next product (P -> PV, dS -> dS K) in
// registers.  For that, value j of lane group g must be contraction element s*EPL + e of step s.
// fp32 satisfies this directly; for bf16 the A-operand rows of the producing product are loaded
// with bits 2 and 3 of the row index swapped (perm_row), after which value j of lane group g is
// logical row c_logical(j, g) = (j/8)*16 + g*8 + j%8.
//
// LDS tiles are row-major with 16-byte chunks XOR-swizzled per row.  Operands whose contraction
// runs along tile rows (V in PV, dO / Q~ / K~ in the gradient products) are read with the gfx950
// transpose load ds_read_b64_tr_b16: inside each 16-lane group, output lane j, element m is
// element j%4 of the 8 bytes read by source lane j/4 + 4m.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pe {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

// ------------------------------------------------------------------ element conversions
__device__ __forceinline__ uint16_t f2bf(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);  // round-to-nearest-even (v_cvt_pk_bf16_f32)
}
// two floats -> one dword of bf16 (lo in bits 0-15), round-to-nearest-even; written as a vector
// conversion so that it is one v_cvt_pk_bf16_f32 with both sources (the scalar form compiles to a
// conversion per element plus shifts and ORs)
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}
__device__ __forceinline__ float bf2f(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}

__device__ __forceinline__ float round_bf16(float x) { return bf2f(f2bf(x)); }

// fp16 the same way (v_cvt_pk_f16_f32 / v_cvt_f32_f16, round-to-nearest-even)
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, h2_t));
}
__device__ __forceinline__ void unpack_h2(uint32_t v, float& lo, float& hi) {
  const f32x2_t f = __builtin_convertvector(__builtin_bit_cast(h2_t, v), f32x2_t);
  lo = f[0];
  hi = f[1];
}
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
__device__ __forceinline__ float round_f16(float x) { return (float)(_Float16)x; }

// Element types by the C ABI's dtype codes: 0 bf16, 1 fp32, 2 fp16.  The matrix-core kernels take
// the 16-bit ones (HT 0 or 2) as a template parameter; these pack two floats into the operand dword
// and round one float to the type.
template <int HT> __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  static_assert(HT == 0 || HT == 2, "16-bit type");
  if constexpr (HT == 0) return pack_bf2(lo, hi);
  else return pack_h2(lo, hi);
}
// round to the element type of dtype code `dt` (identity for fp32)
__device__ __forceinline__ float round_to(float x, int dt) {
  return dt == 0 ? round_bf16(x) : (dt == 2 ? round_f16(x) : x);
}

// A position as the phase product sees it (PE_POS_*): exact (0), or first rounded to the nearest
// bf16 (1) or fp16 (2), ties to even, which is what torch.arange(..., dtype=x.dtype) holds for a
// bf16 / fp16 x (fp16 overflows to inf past 65519)
__device__ __forceinline__ float pe_pos(int p, int rounding) {
  const float x = (float)p;
  if (rounding == 1) return round_bf16(x);
  if (rounding == 2) return (float)(_Float16)x;
  return x;
}

__device__ __forceinline__ void unpack8(const u32x4& v, float (&x)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __builtin_bit_cast(float, v[i] << 16);
    x[2 * i + 1] = __builtin_bit_cast(float, v[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void unpack8_h(const u32x4& v, float (&x)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) unpack_h2(v[i], x[2 * i], x[2 * i + 1]);
}

// 8 consecutive elements starting at element i (16-byte aligned) as floats / from floats;
// dtype 0 = bf16 (one 16-byte access), 1 = fp32 (two), 2 = fp16 (one)
__device__ __forceinline__ void load8(const void* p, int64_t i, int dtype, float (&x)[8]) {
  if (dtype == 0) {
    unpack8(*(const u32x4*)((const uint16_t*)p + i), x);
  } else if (dtype == 2) {
    unpack8_h(*(const u32x4*)((const uint16_t*)p + i), x);
  } else {
    const f32x4 a = *(const f32x4*)((const float*)p + i), b = *(const f32x4*)((const float*)p + i + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) { x[e] = a[e]; x[e + 4] = b[e]; }
  }
}
__device__ __forceinline__ void store8(void* p, int64_t i, int dtype, const float (&x)[8]) {
  if (dtype == 0) {
    *(u32x4*)((uint16_t*)p + i) =
        u32x4{pack_bf2(x[0], x[1]), pack_bf2(x[2], x[3]), pack_bf2(x[4], x[5]), pack_bf2(x[6], x[7])};
  } else if (dtype == 2) {
    *(u32x4*)((uint16_t*)p + i) =
        u32x4{pack_h2(x[0], x[1]), pack_h2(x[2], x[3]), pack_h2(x[4], x[5]), pack_h2(x[6], x[7])};
  } else {
    *(f32x4*)((float*)p + i) = f32x4{x[0], x[1], x[2], x[3]};
    *(f32x4*)((float*)p + i + 4) = f32x4{x[4], x[5], x[6], x[7]};
  }
}

// The same accesses inside the 16-bit kernels' epilogues, whose views hold either fp32 (dtype 1) or
// the kernel's own 16-bit type HT (the host passes nothing else): two cases, chosen at compile time,
// so the other 16-bit type adds no code to the kernels.
template <int HT> __device__ __forceinline__ void load8t(const void* p, int64_t i, int dtype, float (&x)[8]) {
  if (dtype != 1) {
    if constexpr (HT == 0) unpack8(*(const u32x4*)((const uint16_t*)p + i), x);
    else unpack8_h(*(const u32x4*)((const uint16_t*)p + i), x);
  } else {
    const f32x4 a = *(const f32x4*)((const float*)p + i), b = *(const f32x4*)((const float*)p + i + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) { x[e] = a[e]; x[e + 4] = b[e]; }
  }
}
template <int HT> __device__ __forceinline__ void store8t(void* p, int64_t i, int dtype, const float (&x)[8]) {
  if (dtype != 1) {
    *(u32x4*)((uint16_t*)p + i) = u32x4{pack2<HT>(x[0], x[1]), pack2<HT>(x[2], x[3]), pack2<HT>(x[4], x[5]),
                                        pack2<HT>(x[6], x[7])};
  } else {
    *(f32x4*)((float*)p + i) = f32x4{x[0], x[1], x[2], x[3]};
    *(f32x4*)((float*)p + i + 4) = f32x4{x[4], x[5], x[6], x[7]};
  }
}
template <int HT> __device__ __forceinline__ float load_as_float_t(const void* p, int64_t i, int dtype) {
  if (dtype == 1) return ((const float*)p)[i];
  if constexpr (HT == 0) return bf2f(((const uint16_t*)p)[i]);
  else return h2f(((const uint16_t*)p)[i]);
}
template <int HT> __device__ __forceinline__ void store_from_float_t(void* p, int64_t i, int dtype, float x) {
  if (dtype == 1) ((float*)p)[i] = x;
  else if constexpr (HT == 0) ((uint16_t*)p)[i] = f2bf(x);
  else ((uint16_t*)p)[i] = f2h(x);
}

// storage element per compute dtype: DT 0 = bf16 (raw uint16), DT 1 = fp32, DT 2 = fp16 (raw uint16)
template <int DT> struct Elem;
template <> struct Elem<0> { using T = uint16_t; };
template <> struct Elem<1> { using T = float; };
template <> struct Elem<2> { using T = uint16_t; };

__device__ __forceinline__ float load_as_float(const void* p, int64_t i, int dtype) {
  if (dtype == 0) return bf2f(((const uint16_t*)p)[i]);
  if (dtype == 2) return h2f(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}
__device__ __forceinline__ void store_from_float(void* p, int64_t i, int dtype, float x) {
  if (dtype == 0) ((uint16_t*)p)[i] = f2bf(x);
  else if (dtype == 2) ((uint16_t*)p)[i] = f2h(x);
  else ((float*)p)[i] = x;
}

// ------------------------------------------------------------------ matrix-core traits
// The explicit mask of (b, h, q, k) in log2 units (pe_internal.h, CoreArgs::mask): 0 or -inf for a
// bool mask, the float's value times log2(e) otherwise (values below -FLT_MAX / log2(e) overflow to
// -inf, i.e. masked).  q and k are clamped into the view, so padding rows and keys past the end read
// an element of the view and are masked by the caller.
template <class A> __device__ __forceinline__ float mask_elem_l2(const A& a, int64_t i) {  // element i
  if (a.mask_dtype == 3) return ((const uint8_t*)a.mask)[i] ? 0.f : -INFINITY;
  return load_as_float(a.mask, i, a.mask_dtype) * LOG2E;
}
template <class A> __device__ __forceinline__ float mask_l2(const A& a, int b, int h, int q, int k) {
  q = q < a.Sq ? q : a.Sq - 1;
  k = k < a.Sk ? k : a.Sk - 1;
  return mask_elem_l2(a, b * a.m_sb + h * a.m_sh + (int64_t)q * a.m_sq + (int64_t)k * a.m_sk);
}

// The mask of 8 consecutive keys at element offset `i` of a mask_vec view (pe_internal.h), in log2
// units as mask_l2: one 8- or 16-byte load for bool and 16-bit masks, two for fp32.
template <class A> __device__ __forceinline__ void mask_row8(const A& a, int64_t i, float (&mv)[8]) {
  if (a.mask_dtype == 3) {
    const u32x2 w = *(const u32x2*)((const uint8_t*)a.mask + i);
#pragma unroll
    for (int e = 0; e < 8; ++e) mv[e] = ((w[e >> 2] >> ((e & 3) * 8)) & 0xffu) ? 0.f : -INFINITY;
  } else if (a.mask_dtype == 1) {
    const f32x4 x0 = *(const f32x4*)((const float*)a.mask + i), x1 = *(const f32x4*)((const float*)a.mask + i + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      mv[e] = x0[e] * LOG2E;
      mv[4 + e] = x1[e] * LOG2E;
    }
  } else {
    const u32x4 w = *(const u32x4*)((const uint16_t*)a.mask + i);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t hv = (uint16_t)(w[e >> 1] >> ((e & 1) * 16));
      mv[e] = (a.mask_dtype == 0 ? bf2f(hv) : h2f(hv)) * LOG2E;
    }
  }
}

template <int DT> struct MT;
template <> struct MT<0> {
  static constexpr int KC = 16, EPL = 8, ESZ = 2;
  __device__ __forceinline__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // pack 8 consecutive C values (base j0) of a tile into one operand fragment
  __device__ __forceinline__ static u32x4 pack(const f32x16& c, int j0) {
    u32x4 r;
    r[0] = pack_bf2(c[j0 + 0], c[j0 + 1]);
    r[1] = pack_bf2(c[j0 + 2], c[j0 + 3]);
    r[2] = pack_bf2(c[j0 + 4], c[j0 + 5]);
    r[3] = pack_bf2(c[j0 + 6], c[j0 + 7]);
    return r;
  }
};
template <> struct MT<2> {  // fp16 operands, the same fragment layout as bf16
  static constexpr int KC = 16, EPL = 8, ESZ = 2;
  typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
  __device__ __forceinline__ static u32x4 pack(const f32x16& c, int j0) {
    u32x4 r;
    r[0] = pack_h2(c[j0 + 0], c[j0 + 1]);
    r[1] = pack_h2(c[j0 + 2], c[j0 + 3]);
    r[2] = pack_h2(c[j0 + 4], c[j0 + 5]);
    r[3] = pack_h2(c[j0 + 6], c[j0 + 7]);
    return r;
  }
};
template <> struct MT<1> {
  static constexpr int KC = 8, EPL = 4, ESZ = 4;
  __device__ __forceinline__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    // element-wise extraction into scalars first: bit-casting an ext-vector element lvalue
    // directly has been observed to read element 0 for every e
    const uint32_t a0 = a.x, a1 = a.y, a2 = a.z, a3 = a.w;
    const uint32_t b0 = b.x, b1 = b.y, b2 = b.z, b3 = b.w;
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a0), __uint_as_float(b0), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a1), __uint_as_float(b1), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a2), __uint_as_float(b2), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a3), __uint_as_float(b3), c, 0, 0, 0);
    return c;
  }
  __device__ __forceinline__ static u32x4 pack(const f32x16& c, int j0) {
    u32x4 r;
    r.x = __float_as_uint(c[j0 + 0]);
    r.y = __float_as_uint(c[j0 + 1]);
    r.z = __float_as_uint(c[j0 + 2]);
    r.w = __float_as_uint(c[j0 + 3]);
    return r;
  }
};

// physical C row of value j in lane group g
__device__ __forceinline__ int c_row(int j, int g) { return ((j >> 2) << 3) + (g << 2) + (j & 3); }

template <int DT> __device__ __forceinline__ int perm_row(int r) {
  if constexpr (DT != 1) return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
  else return r;
}
// logical row (contraction index) of C value j in lane group g after perm_row loading
template <int DT> __device__ __forceinline__ int c_logical(int j, int g) {
  if constexpr (DT != 1) return ((j >> 3) << 4) + (g << 3) + (j & 7);
  else return ((j >> 2) << 3) + (g << 2) + (j & 3);
}

// ------------------------------------------------------------------ swizzled LDS tiles
// NCH = 16-byte chunks per row (a power of two, >= 8).  Chunk c of row r is stored in slot
// c ^ swz(r).  gfx950's LDS has 64 4-byte banks (16 slots of 16 bytes).  Row fragments
// (ds_read_b128) put 16 consecutive rows on one logical chunk, so swz must be a bijection of r mod
// 16 (with the row parity when a row is only 8 slots); transpose reads (ds_read_b64_tr_b16) touch
// chunks 4a .. 4a+3 of 4 consecutive rows.  With the default permutation (SZ = 0) the 32-lane halves
// of every transpose read share banks two ways (SQ_LDS_BANK_CONFLICT charges 2 of its 4 LDS cycles).
// SZ = 1 selects r2 | r3<<1 | r0<<2 | r1<<3 for rows of 16 or more slots, under which both access
// kinds are conflict-free.  An isolated read probe showed no gain from it (4.8 clk per transpose read
// per CU either way, row fragments 6% slower), but in the kernels it measured faster on every tile
// that takes transpose reads: the dQ GEMM's dS and k~ tiles (dQ 3.6% faster), the forward's v tile
// and the dK/dV kernel's q~ and dO tiles (together 0.5-1% of a step).  Tiles read only by rows keep
// SZ = 0.
template <int NCH, int SZ = 0> __device__ __forceinline__ int swz(int r) {
  static_assert(NCH >= 8, "rows must span at least 8 slots");
  if constexpr (NCH >= 16 && SZ == 1)
    return ((r >> 2) & 1) | (((r >> 3) & 1) << 1) | ((r & 1) << 2) | (((r >> 1) & 1) << 3);
  else if constexpr (NCH >= 16)
    return ((r >> 2) & 1) | ((r & 1) << 1) | (((r >> 1) & 1) << 2) | (((r >> 3) & 1) << 3);
  else
    return ((r >> 2) & 1) | (((r >> 1) & 1) << 1) | (((r >> 3) & 1) << 2);
}
template <int NCH, int SZ = 0> __device__ __forceinline__ uint32_t tile_off(int row, int chunk) {
  return (uint32_t)(row * (NCH * 16) + ((chunk ^ swz<NCH, SZ>(row)) << 4));
}

// One lane's 16-byte row fragment: chunk `chunk` of row `row`.
template <int NCH> __device__ __forceinline__ u32x4 lds_row_frag(const char* tile, int row, int chunk) {
  return *(const u32x4*)(tile + tile_off<NCH>(row, chunk));
}

// Operand fragment whose contraction runs down the tile rows: rows k0 + g*EPL .. +EPL-1,
// column n0 + l32 (element units).
template <int DT, int NCH> __device__ __forceinline__ u32x4 lds_col_frag(const char* tile, int k0, int n0, int lane) {
  if constexpr (DT != 1) {
    const int i = lane & 15, G4 = (lane >> 4) & 3;
    const int col = n0 + ((G4 & 1) << 4) + ((i & 3) << 2);
    const int row = k0 + ((lane >> 5) << 3) + (i >> 2);
    const uint32_t o0 = tile_off<NCH>(row, col >> 3) + ((col & 7) << 1);
    const uint32_t o1 = tile_off<NCH>(row + 4, col >> 3) + ((col & 7) << 1);
    s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + o0));
    s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + o1));
    u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
    u32x4 r;
    r[0] = ua[0]; r[1] = ua[1]; r[2] = ub[0]; r[3] = ub[1];
    return r;
  } else {
    const int col = n0 + (lane & 31);
    const int row = k0 + ((lane >> 5) << 2);
    u32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      r[e] = *(const uint32_t*)(tile + tile_off<NCH>(row + e, col >> 2) + ((col & 3) << 2));
    return r;
  }
}

// Fragment addressing with per-lane bases.  The XOR swizzle only touches chunk bits 0-3 (0-2 for
// 8-slot rows) and depends only on row bits 0-3, so a fragment at row offset k0 (a multiple of 16
// rows) and column offset n0 (a multiple of 32 columns) is a per-lane base chosen by (n0 / 32) % 4
// plus the immediate k0 * row_bytes + (n0 / 128) * 256.  Hoisted, eight base registers stand in for
// the per-fragment address registers the compiler otherwise keeps for every fragment read.
template <int NCH, int SZ = 0> struct ColFrags {  // transpose reads, as lds_col_frag<0, NCH>
  uint32_t b[4][2];                               // [(n0 / 32) % 4][rows +0 / +4]
  __device__ __forceinline__ explicit ColFrags(int lane) {
    const int i = lane & 15, G4 = (lane >> 4) & 3;
    const int colq = ((G4 & 1) << 4) + ((i & 3) << 2);
    const int row = ((lane >> 5) << 3) + (i >> 2);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int col = (j * 32 + colq) % (NCH * 8);
        b[j][hh] = tile_off<NCH, SZ>(row + 4 * hh, col >> 3) + ((col & 7) << 1);
      }
  }
  // k0 % 16 == 0, n0 % 32 == 0, both compile-time after unrolling
  __device__ __forceinline__ u32x4 read(const char* tile, int k0, int n0) const {
    const uint32_t add = (uint32_t)(k0 * NCH * 16 + (n0 / 128) * 256);
    const int j = (n0 / 32) & 3;
    const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + b[j][0] + add));
    const s16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + b[j][1] + add));
    const u32x2 ux = __builtin_bit_cast(u32x2, x), uy = __builtin_bit_cast(u32x2, y);
    return u32x4{ux[0], ux[1], uy[0], uy[1]};
  }
};
// One 32-column group of transpose-read fragments at a runtime column offset n0 (any multiple of
// 8): the per-lane base of rows 0 / 4 of the group; fragment rows k0 (a multiple of 16) are an
// immediate.  Two registers per column group.
template <int NCH, int SZ = 0> struct ColBase {
  uint32_t b0, b1;
  ColBase() = default;
  __device__ __forceinline__ ColBase(int lane, int n0) {
    const int i = lane & 15, G4 = (lane >> 4) & 3;
    const int col = n0 + ((G4 & 1) << 4) + ((i & 3) << 2);
    const int row = ((lane >> 5) << 3) + (i >> 2);
    b0 = tile_off<NCH, SZ>(row, col >> 3) + ((col & 7) << 1);
    b1 = tile_off<NCH, SZ>(row + 4, col >> 3) + ((col & 7) << 1);
  }
  __device__ __forceinline__ u32x4 read(const char* tile, int k0) const {
    const uint32_t add = (uint32_t)(k0 * NCH * 16);
    const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + b0 + add));
    const s16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + b1 + add));
    const u32x2 ux = __builtin_bit_cast(u32x2, x), uy = __builtin_bit_cast(u32x2, y);
    return u32x4{ux[0], ux[1], uy[0], uy[1]};
  }
};
// The same two address forms with the lane's row term left out: the caller adds it once per tile
// (row_ptr), and the XOR parts, which are equal for 16- and 32-chunk rows, are shared between
// tiles of both widths.  ColX: row term ((lane >> 5) * 8 + (lane & 15) / 4) * NCH * 16; RowX: rl *
// NCH * 16.
template <int NCH, int SZ = 0> struct ColX {
  uint32_t b[4][2];
  __device__ __forceinline__ explicit ColX(int lane) {
    const int i = lane & 15, G4 = (lane >> 4) & 3;
    const int colq = ((G4 & 1) << 4) + ((i & 3) << 2);
    const int row = ((lane >> 5) << 3) + (i >> 2);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        b[j][hh] = (uint32_t)((((((j * 32 + colq) % (NCH * 8)) >> 3) ^ swz<NCH, SZ>(row + 4 * hh)) << 4) | ((colq & 7) << 1));
  }
  __device__ __forceinline__ static uint32_t row_term(int lane) {
    return (uint32_t)((((lane >> 5) << 3) + ((lane & 15) >> 2)) * NCH * 16);
  }
  __device__ __forceinline__ u32x4 read(const char* row_ptr, int k0, int n0) const {
    const uint32_t add = (uint32_t)(k0 * NCH * 16 + (n0 / 128) * 256);
    const int j = (n0 / 32) & 3;
    const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(row_ptr + b[j][0] + add));
    const s16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(row_ptr + b[j][1] + add + 4 * NCH * 16));
    const u32x2 ux = __builtin_bit_cast(u32x2, x), uy = __builtin_bit_cast(u32x2, y);
    return u32x4{ux[0], ux[1], uy[0], uy[1]};
  }
};
template <int NCH, int SZ = 0> struct RowX {
  uint32_t b[8];
  __device__ __forceinline__ RowX(int rl, int g) {
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = (uint32_t)((((2 * j + g) % NCH) ^ swz<NCH, SZ>(rl)) << 4);
  }
  __device__ __forceinline__ u32x4 read(const char* row_ptr, int row0, int kk) const {
    return *(const u32x4*)(row_ptr + b[kk & 7] + (uint32_t)(row0 * NCH * 16 + (kk >> 3) * 256));
  }
};
template <int NCH, int SZ = 0> struct RowFrags {  // row fragments, as lds_row_frag<NCH>(tile, row0 + rl, 2 * kk + g)
  uint32_t b[8];                                  // [kk % 8]
  // rl < 32: the lane's row within a 32-row tile (perm_row(l32) for the products that need it)
  __device__ __forceinline__ RowFrags(int rl, int g) {
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = tile_off<NCH, SZ>(rl, (2 * j + g) % NCH);
  }
  // row0 % 32 == 0, compile-time kk
  __device__ __forceinline__ u32x4 read(const char* tile, int row0, int kk) const {
    return *(const u32x4*)(tile + b[kk & 7] + (uint32_t)(row0 * NCH * 16 + (kk >> 3) * 256));
  }
};

// Cooperative copy of ROWS x (NCH*16 bytes) from global (row stride in bytes) into a swizzled
// tile; rows >= nvalid are zero-filled.  All NT threads of the block participate.
template <int ROWS, int NCH, int NT>
__device__ __forceinline__ void copy_tile(char* tile, const char* src, int64_t row_stride_bytes,
                                          int nvalid, int tid) {
  constexpr int TOTAL = ROWS * NCH;
#pragma unroll
  for (int it = 0; it < (TOTAL + NT - 1) / NT; ++it) {
    const int q = it * NT + tid;
    if ((TOTAL % NT) == 0 || q < TOTAL) {
      const int row = q / NCH, c = q % NCH;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (row < nvalid) v = *(const u32x4*)(src + row * row_stride_bytes + c * 16);
      *(u32x4*)(tile + tile_off<NCH>(row, c)) = v;
    }
  }
}

// Two-phase variant: issue the global loads into registers first, store to LDS later.
template <int ROWS, int NCH, int NT> struct TileStage {
  static constexpr int N = (ROWS * NCH + NT - 1) / NT;
  u32x4 r[N];
  __device__ __forceinline__ void load(const char* src, int64_t row_stride_bytes, int nvalid, int tid) {
#pragma unroll
    for (int it = 0; it < N; ++it) {
      const int q = it * NT + tid;
      const int row = q / NCH, c = q % NCH;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (((ROWS * NCH) % NT == 0 || q < ROWS * NCH) && row < nvalid)
        v = *(const u32x4*)(src + row * row_stride_bytes + c * 16);
      r[it] = v;
    }
  }
  __device__ __forceinline__ void store(char* tile, int tid) const {
#pragma unroll
    for (int it = 0; it < N; ++it) {
      const int q = it * NT + tid;
      if ((ROWS * NCH) % NT == 0 || q < ROWS * NCH) {
        const int row = q / NCH, c = q % NCH;
        *(u32x4*)(tile + tile_off<NCH>(row, c)) = r[it];
      }
    }
  }
};

// Direct global -> LDS copy (global_load_lds_dwordx4) of a ROWS x NCH-chunk tile into the
// swizzled layout above.  One wave instruction fills 64 consecutive 16-byte LDS slots; each lane
// fetches the logical chunk that the swizzle places in its slot.  Rows at or beyond `nvalid`
// (>= 1) re-read row nvalid-1, so every address stays inside the source; the kernels mask those
// rows.  Completion is tracked by vmcnt: call dma_wait() before the barrier that publishes the
// tile.  All NW waves participate; ROWS*NCH must be a multiple of 64*NW.
// Addressing: instruction i of wave w fills the 64/NCH rows r0 | x (x = lane / NCH < 64/NCH, r0 a
// multiple of 64/NCH).  swz is a bit permutation of the row bits, so swz(r0 | x) = swz(r0) ^
// swz(x) and the lane's source offset is r0*stride + x*stride + ((lane % NCH) ^ swz(x) ^ swz(r0))*16:
// two per-lane constants and one XOR + add per instruction with wave-uniform r0 terms.  A tile
// with rows past the end takes the general path that clamps each row.
// One wave-wide 16-byte-per-lane global -> LDS copy (global_load_lds_dwordx4): lane l's 16 bytes
// land at LDS address `lds` + 16*l.  It is issued as inline asm so that the compiler does not
// track it: for the builtin, the compiler cannot tell the transpose reads (ds_read_b64_tr_b16) from
// reads of the tile being loaded and makes the first such read after every DMA issue wait for all
// DMA in flight (vmcnt(0)), which serialises the load of the next tile with the current one.
// Every caller instead waits for its DMA with an explicit vmcnt and a barrier before the
// destination is read.  The s_nop covers the one wait state an M0 write needs before an LDS DMA.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
// LDS byte address of a __shared__ object: the low 32 bits of its generic (flat) address
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)p; }
// a wave-uniform 64-bit address in an SGPR pair (readfirstlane returns int: each half is taken
// back as uint32_t so that the low half is zero-extended, not sign-extended into the high one)
__device__ __forceinline__ uint64_t uniform64(const void* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  return ((uint64_t)hi << 32) | (uint64_t)lo;
}
// dma16 with a wave-uniform base in SGPRs and a 32-bit per-lane byte offset (no per-lane 64-bit
// address arithmetic).  When the compiler holds the base in VGPRs, uniform64 becomes
// v_readfirstlane, a VALU write of SGPRs; a VMEM instruction that reads such SGPRs needs 5 wait
// states after the write, and the compiler does not pad across inline asm (with fewer, the load
// read a stale base half and faulted).  The asm therefore copies the base with one SALU move,
// which has no such hazard towards the load, and which also provides the wait state an M0 write
// needs before an LDS DMA.
__device__ __forceinline__ void dma16s(uint32_t voff, const void* base, uint32_t lds) {
  uint64_t sb;
  asm volatile("s_mov_b64 %0, %2\n\tglobal_load_lds_dwordx4 %1, %0"
               : "=&s"(sb)
               : "v"(voff), "s"(uniform64(base)), "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}

template <int ROWS, int NCH, int NW, int SZ = 0>
__device__ __forceinline__ void dma_tile(char* tile, const char* src, int64_t row_stride_bytes,
                                         int nvalid, int w, int lane) {
  constexpr int TOTAL = ROWS * NCH;
  constexpr int RPI = 64 / NCH;  // rows per wave instruction
  static_assert(TOTAL % (64 * NW) == 0, "tile must split into whole wave instructions");
  static_assert(NCH <= 64, "a row must fit one wave instruction");
  const uint32_t rs = (uint32_t)row_stride_bytes;
  if (nvalid >= ROWS) {
    const int x = lane / NCH;
    const uint32_t U = (uint32_t)(((lane % NCH) ^ swz<NCH, SZ>(x)) << 4);
    const uint32_t X = (uint32_t)x * rs;
#pragma unroll
    for (int i = 0; i < TOTAL / (64 * NW); ++i) {
      const int base = (i * NW + w) * 64;
      const int r0 = base / NCH;
      const uint32_t S = (uint32_t)(swz<NCH, SZ>(r0) << 4);
      dma16(src + (uint32_t)r0 * rs + (X + (U ^ S)), lds_addr(tile) + base * 16);
    }
    (void)RPI;
  } else {
#pragma unroll
    for (int i = 0; i < TOTAL / (64 * NW); ++i) {
      const int base = (i * NW + w) * 64;
      const int slot = base + lane;
      const int row = slot / NCH, pc = slot % NCH;
      const int lc = pc ^ swz<NCH, SZ>(row);
      const int r = row < nvalid ? row : nvalid - 1;
      dma16(src + (r * rs + (uint32_t)(lc * 16)), lds_addr(tile) + base * 16);
    }
  }
}

// dma_tile with the per-lane source offsets of a whole tile computed once: each of a wave's TPW
// instructions per tile takes a wave-uniform row base (tile source + its first row times the row
// stride, in SGPRs) and a 32-bit per-lane offset, so a full tile costs no vector instructions
// beyond the loads.  The per-lane part (row within the instruction, swizzled chunk) depends on the
// instruction's first row only through the swizzle, i.e. through that row mod 16, so a wave keeps
// one offset per residue class: P = 16 / gcd(16, NW * rows per instruction) of them, at most TPW.
// Tiles with rows past the end of the source take dma_tile's clamping path instead.
template <int ROWS, int NCH, int NW, int SZ = 0> struct DmaPlan {
  static constexpr int TPW = ROWS * NCH / (64 * NW);
  static constexpr int RPI = 64 / NCH;
  static constexpr int STEP = (NW * RPI) % 16;  // first-row advance per instruction, mod 16
  static constexpr int P0 = STEP == 0 ? 1 : (STEP % 8 == 0 ? 2 : (STEP % 4 == 0 ? 4 : (STEP % 2 == 0 ? 8 : 16)));
  static constexpr int P = P0 < TPW ? P0 : TPW;
  static_assert(ROWS * NCH % (64 * NW) == 0 && NCH <= 64, "whole wave instructions");
  uint32_t off[P];
  __device__ __forceinline__ DmaPlan(int w, int lane, uint32_t rs) {
    const int x = lane / NCH;
    const uint32_t U = (uint32_t)(((lane % NCH) ^ swz<NCH, SZ>(x)) << 4);
#pragma unroll
    for (int c = 0; c < P; ++c) {
      const int r0 = (c * NW + w) * RPI;
      off[c] = (uint32_t)x * rs + (U ^ (uint32_t)(swz<NCH, SZ>(r0) << 4));
    }
  }
  // all ROWS rows of the tile starting at `src` (wave-uniform) are inside the source
  __device__ __forceinline__ void full(const char* src, uint32_t lds_tile, int w, uint32_t rs) const {
    const int wu = __builtin_amdgcn_readfirstlane(w);
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const uint32_t r0 = (uint32_t)((i * NW + wu) * RPI);
      dma16s(off[i % P], src + (uint64_t)r0 * rs, lds_tile + (uint32_t)((i * NW + wu) * 64 * 16));
    }
  }
};

// Plain (unswizzled) DMA of `nchunks` <= 64 consecutive 16-byte chunks by one wave.
__device__ __forceinline__ void dma_row(char* dst, const char* src, int nchunks, int lane) {
  if (lane < nchunks) dma16(src + lane * 16, lds_addr(dst));
}

__device__ __forceinline__ void dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// wait until at most N vector memory operations of this wave are outstanding (they retire in issue
// order, so everything issued before the last N has completed)
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32, 64); }
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ------------------------------------------------------------------ scalar math (reference semantics)
// torch softplus (beta 1, threshold 20) and its derivative, the logistic sigmoid, from one
// exponential: e = exp(-|x|), softplus = max(x, 0) + log1p(e), sigmoid = (x >= 0 ? 1 : e) / (1 + e).
// log1p(e) = log(u) * e / (u - 1) with u = fl(1 + e) (Goldberg's accurate log1p, "What every computer
// scientist should know about floating-point arithmetic", Thm. 4) keeps small softplus values to a
// few ulp.  Hardware exp2 / log2 / rcp: softplus within ~3 ulp, sigmoid within 1.2e-7 of torch.
__device__ __forceinline__ void softplus_sigmoid(float x, float& sp, float& sg) {
  const float e = __builtin_amdgcn_exp2f(-__builtin_fabsf(x) * LOG2E);
  const float u = 1.f + e;
  const float ru = __builtin_amdgcn_rcpf(u);
  const float l1p = u == 1.f ? e : __builtin_amdgcn_logf(u) * LN2 * (e * __builtin_amdgcn_rcpf(u - 1.f));
  sp = x > 20.f ? x : __builtin_fmaxf(x, 0.f) + l1p;
  sg = (x >= 0.f ? 1.f : e) * ru;
}
__device__ __forceinline__ float softplus_f(float x) {
  float sp, sg;
  softplus_sigmoid(x, sp, sg);
  return sp;
}

// Products and sums rounded one by one, as the reference's torch ops round them (t * w, then
// + delta).  hipcc contracts a multiply that feeds an add into one fma by default, __fmul_rn /
// __fadd_rn included once both sit in one basic block; instructions built under this pragma carry
// no contraction flag, so they stay separate after inlining.
__device__ __forceinline__ float mul_nc(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_nc(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float sub_nc(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}

// sin and cos of an fp32 phase.  Cody-Waite reduction by pi/2 with a three-part constant
// (P1 + P2 + P3 = pi/2 to ~2^-73): for |x| < 2^17 the first fma is exact (x and k*P1 are multiples
// of 2^-23 whose difference is below 2), so r carries ~1 ulp; then the Taylor series of sin (to r^11)
// and cos (to r^12) on |r| <= pi/4, whose truncation error is below 1e-11.  Max abs error 9.2e-8
// over |x| < 2^17, measured against float64; larger phases take the library routine.
__device__ __forceinline__ void pe_sincos(float x, float& sn, float& cs) {
  if (__builtin_fabsf(x) >= 131072.f) {
    sincosf(x, &sn, &cs);
    return;
  }
  constexpr float P1 = 0x1.921fb6p+0f, P2 = -0x1.777a5cp-25f, P3 = -0x1p-49f;
  const float k = __builtin_rintf(x * 0.636619772f);
  float r = __builtin_fmaf(-k, P1, x);
  r = __builtin_fmaf(-k, P2, r);
  r = __builtin_fmaf(-k, P3, r);
  const float r2 = r * r;
  float ps = -2.50521084e-8f;                  // -1/11!
  ps = __builtin_fmaf(ps, r2, 2.75573192e-6f);  // 1/9!
  ps = __builtin_fmaf(ps, r2, -1.98412698e-4f); // -1/7!
  ps = __builtin_fmaf(ps, r2, 8.33333333e-3f);  // 1/5!
  ps = __builtin_fmaf(ps, r2, -1.66666667e-1f); // -1/3!
  const float s = __builtin_fmaf(r2 * r, ps, r);
  float pc = 2.08767570e-9f;                    // 1/12!
  pc = __builtin_fmaf(pc, r2, -2.75573192e-7f); // -1/10!
  pc = __builtin_fmaf(pc, r2, 2.48015873e-5f);  // 1/8!
  pc = __builtin_fmaf(pc, r2, -1.38888889e-3f); // -1/6!
  pc = __builtin_fmaf(pc, r2, 4.16666667e-2f);  // 1/4!
  const float c = __builtin_fmaf(r2 * r2, pc, __builtin_fmaf(-0.5f, r2, 1.f));
  const int q = (int)k & 3;
  const float s1 = (q & 1) ? c : s, c1 = (q & 1) ? s : c;
  sn = (q & 2) ? -s1 : s1;
  cs = ((q + 1) & 2) ? -c1 : c1;
}

// Gradient of one PoPE element y = [mu cos phi, mu sin phi] (mu = softplus(x), phi = fl(pos*freq)
// (+ delta, added after the product)): from the pair (gc, gs) writes dx = (gc cos + gs sin)
// sigmoid(x) and returns dphi = mu (gs cos - gc sin).
// The same with sin / cos of the phase given.  The products and sums are written out (one fma
// each, the other product unfused) so that every caller rounds them alike: left to the compiler,
// the contraction of gc*cs + gs*sn depends on the surrounding code, and the element-wise and
// vectorised epilogues would differ in the last bit.
__device__ __forceinline__ float inv_pope_elem_cs(float x, float sn, float cs, float gc, float gs, float& dx) {
  float mu, sg;
  softplus_sigmoid(x, mu, sg);
  dx = mul_nc(__builtin_fmaf(gc, cs, mul_nc(gs, sn)), sg);
  return mul_nc(mu, __builtin_fmaf(gs, cs, -mul_nc(gc, sn)));
}
__device__ __forceinline__ float inv_pope_elem(float x, float pos, float freq, float dl, bool key,
                                               float gc, float gs, float& dx) {
  float ph = mul_nc(pos, freq);
  if (key) ph = add_nc(ph, dl);
  float sn, cs;
  pe_sincos(ph, sn, cs);
  return inv_pope_elem_cs(x, sn, cs, gc, gs, dx);
}

// RoPE (mode 1) or no-PE (mode 2) forward of one pair (x0, x1) of a row, src/model/rope.py:35-57:
// y = mscale * (x0 cos - x1 sin, x0 sin + x1 cos) at angle fl(pos * inv_freq), or y = x; each product
// and sum rounded on its own, as torch's ops round them.  cs / sn are kept for the gradient.
__device__ __forceinline__ void rope_pair(int mode, float x0, float x1, float pos, float fr, float ms, float& y0,
                                          float& y1, float& sn, float& cs) {
  if (mode == 1) {
    pe_sincos(mul_nc(pos, fr), sn, cs);
    y0 = sub_nc(mul_nc(x0, cs), mul_nc(x1, sn)) * ms;
    y1 = add_nc(mul_nc(x0, sn), mul_nc(x1, cs)) * ms;
  } else {
    sn = 0.f; cs = 1.f;
    y0 = x0; y1 = x1;
  }
}
__device__ __forceinline__ float sq2(float a, float b) { return add_nc(mul_nc(a, a), mul_nc(b, b)); }
__device__ __forceinline__ float dot2(float a0, float a1, float b0, float b1) {
  return add_nc(mul_nc(a0, b0), mul_nc(a1, b1));
}
// Gradient of one pair through QKNorm (y = z / (||z|| + 1e-6), src/model/normalization.py:54-55) and
// the rotation: d = dy c1 - z c2 (d = dy without the norm), dx = mscale * rot^T(d) (dx = d for no-PE)
__device__ __forceinline__ void rope_pair_grad(int mode, bool l2, float g0, float g1, float z0, float z1, float c1,
                                               float c2, float cs, float sn, float ms, float& dx0, float& dx1) {
  float d0 = g0, d1 = g1;
  if (l2) {
    d0 = sub_nc(mul_nc(g0, c1), mul_nc(z0, c2));
    d1 = sub_nc(mul_nc(g1, c1), mul_nc(z1, c2));
  }
  if (mode == 1) {
    dx0 = mul_nc(add_nc(mul_nc(d0, cs), mul_nc(d1, sn)), ms);
    dx1 = mul_nc(sub_nc(mul_nc(d1, cs), mul_nc(d0, sn)), ms);
  } else {
    dx0 = d0; dx1 = d1;
  }
}
// QKNorm's row sums (||z||^2, and z . dy in the gradient): each lane or thread sums the pairs of its
// chunk of 4 consecutive pairs in order, and the chunks' sums are added by an xor butterfly over the
// chunks (lanes past the row's chunks hold 0, which leaves every sum unchanged).  The scalar and the
// vector kernels below both follow this order, so they produce bitwise equal rows.
__device__ __forceinline__ void l2_coefs(float ss, float zd, float& c1, float& c2) {
  const float n = sqrtf(ss);
  const float ne = add_nc(n, 1e-6f);
  c1 = 1.f / ne;
  c2 = n > 0.f ? zd / mul_nc(mul_nc(n, ne), ne) : 0.f;
}

// The gradient of one 8-element chunk (pairs 4t .. 4t + 3) of a RoPE / no-PE row through QKNorm: x
// the raw inputs, g the gradient of the transformed chunk, fr4 the chunk's 4 inverse frequencies
// (RoPE), tpr threads per row, adjacent and aligned in the wave (QKNorm's row sums by an xor
// butterfly over them).  Every thread of a row group must call it together.
__device__ __forceinline__ void inv_rope_chunk(int mode, bool l2, const float (&fr4)[4], float pos, float ms, int tpr,
                                               const float (&x)[8], const float (&g)[8], float (&dx)[8]) {
  float z[8], sn[4], cs[4];
  float ss = 0.f, zd = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    rope_pair(mode, x[2 * k], x[2 * k + 1], pos, fr4[k], ms, z[2 * k], z[2 * k + 1], sn[k], cs[k]);
    ss = add_nc(ss, sq2(z[2 * k], z[2 * k + 1]));
    zd = add_nc(zd, dot2(z[2 * k], z[2 * k + 1], g[2 * k], g[2 * k + 1]));
  }
  float c1 = 1.f, c2 = 0.f;
  if (l2) {
    for (int m = tpr >> 1; m >= 1; m >>= 1) {
      ss += __shfl_xor(ss, m, 64);
      zd += __shfl_xor(zd, m, 64);
    }
    l2_coefs(ss, zd, c1, c2);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k)
    rope_pair_grad(mode, l2, g[2 * k], g[2 * k + 1], z[2 * k], z[2 * k + 1], c1, c2, cs[k], sn[k], ms, dx[2 * k],
                   dx[2 * k + 1]);
}

// Launch-order remap.  Blocks are issued heaviest first (LPT for the causal triangle) and, when the
// number of (batch, head) pairs divides by the 8 XCDs, every block of one head lands on the same
// XCD (hardware dispatch is round-robin over XCDs) so its K/V stays in that XCD's L2.
__device__ __forceinline__ void map_block(int bid, int nblk, int nbh, bool heavy_last_index,
                                          int& blk, int& bh) {
  int j, hsel;
  if ((nbh & 7) == 0) {
    const int x = bid & 7, hp = nbh >> 3;
    j = (bid >> 3) / hp;
    hsel = x * hp + (bid >> 3) % hp;
  } else {
    j = bid / nbh;
    hsel = bid % nbh;
  }
  blk = heavy_last_index ? (nblk - 1 - j) : j;
  bh = hsel;
}

}  // namespace pe
