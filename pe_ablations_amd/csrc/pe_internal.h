// Internal launch interface between the C-ABI host code (pe_api.cpp) and the kernel translation
// units.  Operand buffers are the library's own layout: (B, H, S, W) contiguous, W a tile width.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pe {

// Inverse PoPE transform fused into a gradient kernel's epilogue: the raw positional input x and
// the view its gradient is written through, plus per-block partial sums of dphi and pos*dphi
// (block = (b, h, tile) in that order; either pointer may be NULL).
struct EpiPoPE {
  const void* x; int x_dtype; int64_t x_s[4];
  void* dx; int dx_dtype; int64_t dx_s[4];
  void* dxc; int dxc_dtype; int64_t dxc_s[4];  // content-part gradient (split form, Dc > 0)
  int start_pos;
  int pos_round;  // PE_POS_* rounding of positions
  float* part_delta;
  float* part_freq;
};

// Packed bf16 dS of one (batch, head): 4 KiB blocks of 32 keys x 64 queries, key-row major.  Key
// row r (32 keys) of key block kb = r / 4 (128 keys) holds the 64-query blocks ds_first(kb) ..
// nqt - 1 that the causal dK/dV kernels store for it, contiguously, so block (r, j) sits at
// ds_row_base(r) + j - ds_first(r / 4).  Causal: ds_first(kb) = max(0, 2 kb - e) with
// e = ceil(causal_off / 64) (the kernels start at query max(0, 128 kb - causal_off)); without the
// mask every row holds all nqt blocks.  ds_row_base(r) = r nqt - 4 F(r / 4) - (r % 4) ds_first(r / 4)
// with F(K) = sum_{kb < K} ds_first(kb) = n (K - 1 + m - e), m = ceil(e / 2), n = max(0, K - m).
// Half the square at Sq = Sk.
__host__ __device__ inline int ds_first(int kb, int e, int causal) {
  const int f = 2 * kb - e;
  return causal && f > 0 ? f : 0;
}
__host__ __device__ inline int64_t ds_row_base(int r, int e, int nqt, int causal) {
  if (!causal) return (int64_t)r * nqt;
  const int64_t K = r / 4, m = (e + 1) / 2, n = K > m ? K - m : 0;
  return (int64_t)r * nqt - 4 * n * (K - 1 + m - e) - (int64_t)(r % 4) * ds_first(r / 4, e, causal);
}

// Attention core over transformed operands.
struct CoreArgs {
  const void* q;    // (B, Hq, Sq, DQK) contiguous, compute dtype
  const void* k;    // (B, Hkv, Sk, DQK)
  const void* v;    // (B, Hkv, Sk, DV) rows of v_row elements (>= DV), compute dtype
  int64_t v_sb, v_sh, v_ss;  // element strides of v
  int B, Hq, Hkv, Sq, Sk;
  int dv_real;      // value columns actually produced (<= DV)
  int causal;       // 0 none, else masked when s > t + causal_off
  int causal_off;
  float scale;      // softmax scale
  // forward outputs
  void* o; int64_t o_sb, o_sh, o_ss; int o_dtype;
  float* lse;       // (B, Hq, Sq)
  // backward inputs / outputs
  const void* dO;   // (B, Hq, Sq, DV) compute dtype; the generic kernels need it contiguous (padded)
  int64_t do_sb, do_sh, do_ss;  // element strides of dO (read by the bf16 dK/dV kernel)
  const float* Di;  // (B, Hq, sq_pad)  rowsum(dO * O), 0 on padding rows
  const float* L2;  // (B, Hq, sq_pad)  lse * log2(e), +inf on padding rows and rows without keys
  int sq_pad;       // Sq rounded up to a multiple of 64
  const float* lse_in;
  uint16_t* dS;     // bf16 dS per (b, h) in MFMA fragment order: 4 KiB blocks of 32 keys x 64
                    // queries, block (k/32, q/64) at (ds_row_base(k/32) + q/64 - ds_first(k/128)) *
                    // 4096 bytes within the (b, h) region of ds_head blocks; inside a block, key kl
                    // and query chunk r = (q%64)/8 at chunk ((r>>1)*64 + (r&1)*32 + kl)
  int ds_nqt;       // 64-query blocks per head (ceil(Sq / 256) * 4)
  int ds_rows;      // key rows per head (Sk rounded up to 128)
  int ds_e;         // ceil(causal_off / 64) (causal only)
  int64_t ds_head;  // blocks per (b, h) region: ds_row_base(ds_rows / 32)
  const float* qtab;  // query phase table of launch_phase_table ([Sq][2][Dr]) or null
  float* dq_t;      // (B, Hq, Sq, DQK) fp32, already multiplied by scale
  float* dk_t;      // (B, Hkv, Sk, DQK) fp32, already multiplied by scale (summed over the GQA group)
  void* dv; int64_t dv_sb, dv_sh, dv_ss; int dv_dtype;
  // fused inverse transform (bf16 PoPE with DQK = Dc + 2*Dr, Dc = 0 or Dc = DQK/2): when set the
  // gradient kernels write dq / dk (and the content parts dq_c / dk_c) through eq / ek instead of
  // dq_t / dk_t
  int fuse_inv; int Dr; int Dc;
  const float* freqs; const float* delta; int64_t delta_hs;
  EpiPoPE eq, ek;
  // fused RoPE / no-PE gradient (16-bit compute, transformed width 64, no content part, vector views):
  // the dQ GEMM and the dK/dV kernel apply the QKNorm and rotation backward of their staged dq~ / dk~
  // rows and write dq / dk through eq / ek (x, dx, start_pos, pos_round); freqs holds the inverse
  // frequencies.  rope_mode 1 = RoPE, 2 = no PE; rope_l2 = QKNorm; rope_ms = mscale
  int rope_fuse, rope_mode, rope_l2; float rope_ms;
  int n_cu;  // compute units of the device: launchers pick smaller blocks when a grid would not fill them
  // backward head group: the gradient kernels cover the (batch, kv head) units bh0 .. bh0 + nbh - 1
  // (flattened b * Hkv + hk) and their query heads; dS holds that group only, indexed from its first
  // query head (b * Hq + h - bh0 * Hq / Hkv), so one capped buffer serves every group in turn
  int bh0, nbh;
  // query-head split of the bf16 / fp16 dK/dV pair kernel: qsplit (a divisor of Hq / Hkv) workgroups
  // per key block share out the group's query heads; workgroup j writes fp32 partials to dk_t slice
  // j ((B, Hkv, Sk, DQK) each, already multiplied by scale) and dv_part slice j ((B, Hkv, Sk, DV)
  // each), summed in slice order by dkdv_combine in the dQ launch.  1: off (dv and dk written directly)
  int qsplit;
  float* dv_part;
  // explicit attention mask (SDPA's attn_mask, src/model/attention.py:91-96), read by the mask (MB)
  // instantiations of the tuned forward and dK/dV pair kernel and of the generic kernels: element
  // (b, h, q, k) at mask + b m_sb + h m_sh + q m_sq + k m_sk (element strides, 0 where the mask
  // broadcasts); mask_dtype 3 = bool bytes (nonzero: the key takes part), else a PE_DTYPE_* float
  // added to the scaled score.  null: no mask.
  const void* mask;
  int64_t m_sb, m_sh, m_sq, m_sk;
  int mask_dtype;
  // set by the host when the view takes 8-element vector reads: unit key stride, every other stride
  // a multiple of 8 elements, Sk % 8 == 0 and a 16-byte aligned base (mask_row8)
  int mask_vec;
};

int launch_fwd(int dt, int dqk, int dv, const CoreArgs& a, hipStream_t s);
int launch_bwd_dkdv(int dt, int dqk, int dv, const CoreArgs& a, hipStream_t s);
int launch_bwd_dq(int dt, int dqk, int dv, const CoreArgs& a, hipStream_t s);
bool core_supported(int dqk, int dv);
// 16-bit widths served by the dK/dV pair kernel (with the dQ GEMM over its stored dS); the explicit-
// mask backward runs them there too, and the generic kernels elsewhere
inline bool pair_shape(int dqk, int dv) { return (dqk == 128 || dqk == 256) && (dv == 64 || dv == 128); }

// Elementwise transform: one wave per (b, h, s) row.
struct PrepArgs {
  const void* xc; int xc_dtype; int64_t xc_s[4];
  const void* xr; int xr_dtype; int64_t xr_s[4];
  void* dst; int dst_dtype; int width;           // (B, H, S, width) contiguous
  int B, H, S, Dc, Dr, mode, start_pos, l2norm, is_key;
  int pos_round;  // PE_POS_* rounding of positions (PoPE)
  const float* freqs; const float* delta; int64_t delta_hs;
  float mscale;
  // RMSNorm of xr over all H*Dr features of a token before the transform (launch_prep_norm only)
  const void* norm_w; int norm_w_dtype; float norm_eps;
  // query side only: cos / sin of fl((start_pos + s) * freq) as [S][2][Dr] fp32 (launch_phase_table),
  // read instead of evaluated by the vectorised PoPE prologue; null evaluates them
  const float* tab;
  // destination rows: (b, h, s) goes to row (b * H + h) * dst_rows + dst_row0 + s of dst; dst_rows
  // 0 means S (a contiguous (B, H, S, width) buffer).  A KV cache of capacity C takes new rows at
  // position p with dst_rows = C, dst_row0 = p.
  int dst_rows, dst_row0;
  // optional rows copied alongside (launch_prep's vectorised PoPE path only, see prep_vec_copy_ok):
  // row (b, h, s) of cv (bf16, unit inner stride, cv_cols values) goes to row
  // (b * H + h) * dst_rows + dst_row0 + s of cdst (width cwidth, zero padded); the KV-cache append
  // writes the new value rows in the launch that transforms the new key rows
  const void* cv; int64_t cv_s[4]; int cv_cols; void* cdst; int cwidth;
};
int launch_prep(const PrepArgs& a, hipStream_t s);
// whether launch_prep takes the vectorised PoPE path for `a` and can copy the rows described by
// its cv / cdst fields in the same launch
bool prep_vec_copy_ok(const PrepArgs& a);
// whether `a` (query side) takes the vectorised PoPE path with no content part and no padding, the
// case whose per-element arithmetic the decode split kernel repeats for its own query rows
bool prep_vec_query_ok(const PrepArgs& a);
// cos / sin of the query phases fl(pe_pos(start + s) * freqs[c]) for s < S, c < Dr into tab
// [S][2][Dr] (cos row then sin row), with the same routine and rounding as the prologue kernels
int launch_phase_table(const float* freqs, int start, int S, int Dr, int pos_round, float* tab, hipStream_t s);
// launch_prep(a) (the key side) and launch_phase_table(...) together: one launch on the vectorised
// path, else the two launches in turn
int launch_prep_and_table(const PrepArgs& a, const float* freqs, int start, int S, int Dr, int pos_round, float* tab,
                          hipStream_t s);
// both sides of a small vectorised PoPE prologue (ak: keys, aq: queries with aq.tab null) in one
// launch, the queries evaluating their own phases and the rows of (0, 0) writing tab; returns 1
// without launching when the shape or layout does not qualify (the caller then takes the two-launch
// path)
int launch_prep_qk(const PrepArgs& ak, const PrepArgs& aq, float* tab, hipStream_t s);
// both sides of a larger vectorised PoPE prologue in one launch (ak: keys; aq: queries without a
// content part or padding, aq.tab null): query threads evaluate each phase once for several heads
// and the rows of b = 0 write tab; returns 1 without launching when the layout does not qualify
int launch_prep_k_qheads(const PrepArgs& ak, const PrepArgs& aq, float* tab, hipStream_t s);
// PoPE prologue with the RMSNorm fused in: one workgroup per token (all heads)
int launch_prep_norm(const PrepArgs& a, hipStream_t s);

// Attention of Sq new query rows (transformed, (B, Hq, Sq, DQK) contiguous) against the first L
// rows of a cache of transformed keys (B, Hkv, cap, DQK) and values (B, Hkv, cap, DV), split over
// `nunit` key ranges per (b, kv head, 32-row query tile) and merged in range order.
struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  int B, Hq, Hkv, Sq, L, cap;
  int causal, off;  // with causal, key s is visible to query i iff s <= i + off
  float scale;
  int nqt;          // 32-row tiles of the (Hq / Hkv) * Sq query rows of one kv head
  int nunit;        // key ranges per tile, a multiple of 4 (one per wave)
  float* part_o;    // [B*Hkv][nqt][nunit][32][DV] unnormalised O relative to part_m
  float* part_m;    // [B*Hkv][nqt][nunit][32] running max of the scaled scores, log2 units
  float* part_l;    // [B*Hkv][nqt][nunit][32] sum of 2^(score - part_m)
  void* o; int64_t o_sb, o_sh, o_ss; int o_dtype; int dv_real;
  float* lse;       // (B, Hq, Sq)
  // raw bf16 query rows (B, Hq, Sq, Dr) that the split kernel transforms itself (PoPE, no content
  // part, 2 Dr = the operand width, at most 8 rows per tile), with phases
  // fl(pe_pos(start_pos + i) * freqs[d]); null: q holds the rows the prologue transformed
  const void* qraw; int64_t qr_s[4]; const float* freqs; int Dr, start_pos, pos_round;
};
int launch_decode(int dt, int dqk, int dv, const DecodeArgs& a, hipStream_t s);
// most query rows per tile that the decode split kernel transforms itself
constexpr int DECODE_FUSED_ROWS = 8;

// Stand-alone RMSNorm over the last dim of a (rows, n) view.
struct NormArgs {
  const void* x; int x_dtype; int64_t x_rs;
  const void* w; int w_dtype;
  void* y; int y_dtype; int64_t y_rs;
  int64_t rows; int n; float eps;
};
int launch_rmsnorm(const NormArgs& a, hipStream_t s);
// RMSNorm backward: dx (x's dtype) and the weight gradient dw (the weight's dtype) from
// dy (y's dtype, bf16 exactly when x and w are both bf16); per-workgroup partial sums of dw go to
// `part` ([groups][n] fp32) and are summed in workgroup order by a second launch
struct NormBwdArgs {
  const void* x; int x_dtype; int64_t x_rs;
  const void* w; int w_dtype;
  const void* dy; int64_t dy_rs;
  void* dx; int64_t dx_rs;
  void* dw; int dw_dtype;
  float* part;
  int64_t rows; int n; float eps;
  int rpw;  // rows per wave (a workgroup of WPB waves covers WPB * rpw consecutive rows)
};
// fp32 floats of partial-sum workspace launch_rmsnorm_bwd needs for rows x n
int64_t rmsnorm_bwd_part_floats(int64_t rows, int n, int n_cu);
int launch_rmsnorm_bwd(NormBwdArgs a, int n_cu, hipStream_t s);
// silu(gate) * x over n bf16 elements (n % 8 == 0, 16-byte aligned pointers)
int launch_swiglu(const void* x, const void* gate, void* out, int64_t n, hipStream_t s);

// dO repack (to compute dtype, width DV, contiguous), Di = rowsum(dO * O) and the log2-scaled
// lse, both into (B, H, S_pad) arrays whose padding rows hold Di = 0, L2 = +inf.
struct PreBwdArgs {
  const void* dout; int dout_dtype; int64_t do_s[4];
  const void* out; int out_dtype; int64_t o_s[4];
  void* dO_op; int op_dtype; int width;
  const float* lse; float* Di; float* L2; int s_pad;
  int B, H, S, Dv;
};
int launch_prebwd(const PreBwdArgs& a, hipStream_t s);

// Inverse transform: dx~ (fp32, (B,H,S,width)) -> dxc, dxr, plus per-block partial sums of the
// phase gradient for the key phase bias and for the frequencies.
struct InvArgs {
  const float* g; int width;
  const void* xr; int xr_dtype; int64_t xr_s[4];
  void* dxc; int dxc_dtype; int64_t dxc_s[4];
  void* dxr; int dxr_dtype; int64_t dxr_s[4];
  int B, H, S, Dc, Dr, mode, start_pos, l2norm, is_key;
  int pos_round;  // PE_POS_* rounding of positions (PoPE)
  const float* freqs; const float* delta; int64_t delta_hs;
  float mscale;
  float* part_delta;   // (nblocks, Dr) or NULL
  float* part_freq;    // (nblocks, Dr) or NULL
  int rows_per_block;
};
int launch_inv(const InvArgs& a, int* nblocks_out, hipStream_t s);
int inv_blocks(int B, int H, int S, int rows_per_block);

// Deterministic reduction of the partials.
struct ReduceArgs {
  const float* part_q_freq; int nq;       // q-side blocks (freq partials)
  const float* part_k_freq; const float* part_k_delta; int nk;
  int k_blocks_per_head;                  // consecutive blocks belong to one (b, h): order (b, h, chunk)
  int Hkv, B, Dr;
  int delta_per_head;
  float* dfreqs; float* ddelta;
};
int launch_reduce(const ReduceArgs& a, hipStream_t s);

}  // namespace pe
