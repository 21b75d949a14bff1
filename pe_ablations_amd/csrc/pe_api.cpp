// C-ABI entry points of libpe_attn.so (declared in include/pe_attn.h).  Host code only (plus the
// static scratch array of pe_attn_fwd_noalloc): validates the parameter block, carves the
// caller's workspace and enqueues the kernels on the caller's stream.  No allocation, no
// synchronisation; the only global mutable state is a per-device "is this a gfx950" flag with the
// device's CU count, and the per-device address of the static scratch, each computed once under a
// mutex.
#include <hip/hip_runtime.h>
#include <string.h>
#include <algorithm>
#include <atomic>
#include <mutex>

#include "pe_attn.h"
#include "pe_internal.h"

namespace {

constexpr size_t ALIGN = 256;
inline size_t align_up(size_t x) { return (x + ALIGN - 1) / ALIGN * ALIGN; }
// Rows per inverse-transform block: 256, halved (down to 16) until the grid has 2048 blocks.  A
// thread walks rows_per_block / (256 / threads per row) rows one after another, each a dependent
// global round trip, so short sequences need short blocks to spread over the chip.
int inv_rows(int B, int H, int S) {
  int r = 256;
  while (r > 16 && (int64_t)B * H * ((S + r - 1) / r) < 2048) r /= 2;
  return r;
}

int qk_width(const pe_attn_params* p) {
  return p->Dc + (p->mode == PE_MODE_POPE ? 2 * p->Dr : p->Dr);
}
int pad_qk(int w) { return w <= 64 ? 64 : w <= 128 ? 128 : w <= 256 ? 256 : -1; }
int pad_v(int d) { return d <= 64 ? 64 : d <= 128 ? 128 : -1; }
size_t esz(const pe_attn_params* p) { return p->dtype == PE_DTYPE_FP32 ? 4 : 2; }
// a 16-bit compute dtype (bf16 or fp16): the matrix-core kernels of the 16-bit path
bool half_dt(int dtype) { return dtype == PE_DTYPE_BF16 || dtype == PE_DTYPE_FP16; }
bool valid_dt(int dtype) { return dtype == PE_DTYPE_BF16 || dtype == PE_DTYPE_FP32 || dtype == PE_DTYPE_FP16; }

struct Layout {
  int dqk, dv;
  size_t q_off, k_off, v_off, tab_off, fwd_total;
  size_t do_off, di_off, l2_off, dq_off, dk_off, pq_off, pk_off, pkd_off, dvp_off, ds_off, bwd_total;
  int ksplit;    // query-head split of the dK/dV pair kernel (pe::CoreArgs::qsplit)
  int sq_pad;
  int ds_nqt, ds_rows, ds_e;
  int64_t ds_head;
  int ds_group;  // (batch, kv head) units per backward head group (pe_attn_bwd loops over groups)
  int nq_blocks, nk_blocks;
};

// the query phases are shared by every batch and head, so PoPE evaluates them once per call
bool use_qtab(const pe_attn_params* p) { return p->mode == PE_MODE_POPE && p->Dr > 0 && p->Dr % 8 == 0; }

// bf16 fused PoPE form whose transformed width is exactly 2*Dr of 128 or 256: the gradient kernels
// apply the inverse transform in their epilogues and write dq / dk directly, so the backward needs
// no fp32 dq~ / dk~ buffers (pe_attn_bwd's input checks require the q / k views whenever Dr > 0)
bool fused_bwd(const pe_attn_params* p) {
  return half_dt(p->dtype) && p->mode == PE_MODE_POPE && p->Dc == 0 && (p->Dr == 64 || p->Dr == 128) &&
         pad_qk(qk_width(p)) == 2 * p->Dr;
}

// Compute units of an MI355X.  The query-head split of dK/dV below depends on the shape only (not
// on the device queried), so a workspace size taken before any device call stays valid.
constexpr int kSplitCus = 256;

// dK/dV pair kernel (16-bit, transformed width 128 / 256, value width 64 / 128) on a grid of fewer
// key blocks than compute units: each key block's GQA group of query heads is shared out over up
// to Hq / Hkv workgroups (a power of two dividing it) until the grid reaches the compute units
int key_split(const pe_attn_params* p, int dqk, int dv) {
  if (!half_dt(p->dtype) || !((dqk == 128 || dqk == 256) && (dv == 64 || dv == 128))) return 1;
  const int grp = p->Hq / p->Hkv;
  const int64_t blocks = (int64_t)p->B * p->Hkv * ((p->Sk + 127) / 128);
  int ks = 1;
  while (grp % (2 * ks) == 0 && blocks * ks < kSplitCus) ks *= 2;
  return ks;
}

// a view the vectorised epilogues can read or write 8 elements at a time: unit dim stride and
// every row 16-byte aligned
bool vec16(const pe_tensor_t* t) {
  if (!t || !t->data) return false;
  const int64_t e = t->dtype == PE_DTYPE_FP32 ? 4 : 2;
  return t->stride[3] == 1 && (uintptr_t)t->data % 16 == 0 && (t->stride[0] * e) % 16 == 0 &&
         (t->stride[1] * e) % 16 == 0 && (t->stride[2] * e) % 16 == 0;
}

// the reference module's split form [content 64 | PoPE 2 x 32] (QK width 128, value width 64 or
// 128) in bf16: the gradient kernels' epilogues also apply its inverse transform and copy the
// content gradient, when every view they touch takes 16-byte vector access
bool fused_split_bwd(const pe_attn_params* p, const pe_tensor_t* qr, const pe_tensor_t* kr,
                     const pe_tensor_t* dqc, const pe_tensor_t* dqr, const pe_tensor_t* dkc,
                     const pe_tensor_t* dkr) {
  return half_dt(p->dtype) && p->mode == PE_MODE_POPE && p->Dc == 64 && p->Dr == 32 &&
         (p->Dv == 64 || p->Dv == 128) && vec16(qr) && vec16(kr) && vec16(dqc) && vec16(dqr) && vec16(dkc) &&
         vec16(dkr);
}

// The explicit-mask backward (pe_attn_bwd_masked) at the pair kernel's 16-bit widths runs the same
// kernels as the unmasked one, without the query-head split; elsewhere it runs the generic kernels,
// which write fp32 dq~ / dk~ for the stand-alone inverse transform and store no dS.
bool generic_masked(const pe_attn_params* p, bool masked) {
  return masked && !(half_dt(p->dtype) && pe::pair_shape(pad_qk(qk_width(p)), pad_v(p->Dv)));
}

Layout layout(const pe_attn_params* p, bool masked = false) {
  Layout L{};
  L.dqk = pad_qk(qk_width(p));
  L.dv = pad_v(p->Dv);
  const bool gm = generic_masked(p, masked);
  const size_t e = esz(p);
  const size_t nq = (size_t)p->B * p->Hq * p->Sq, nk = (size_t)p->B * p->Hkv * p->Sk;
  L.q_off = 0;
  L.k_off = L.q_off + align_up(nq * L.dqk * e);
  L.v_off = L.k_off + align_up(nk * L.dqk * e);
  L.tab_off = L.v_off + align_up(nk * L.dv * e);
  // query phase table (cos / sin of fl(pos * freq), fp32 [Sq][2][Dr]) for the PoPE prologue and the
  // dQ epilogue
  L.fwd_total = L.tab_off + (use_qtab(p) ? align_up((size_t)p->Sq * 2 * p->Dr * 4) : 0);
  // per-block partial sums of the phase gradient: blocks of the inverse-transform kernel
  // (inv_rows rows, at most 256), or of the gradient kernels when the transform is fused into their
  // epilogues (dQ GEMM: 256 queries, dK/dV: 128 keys); the buffers are sized for the larger count
  L.nq_blocks = p->mode == PE_MODE_POPE ? pe::inv_blocks(p->B, p->Hq, p->Sq, inv_rows(p->B, p->Hq, p->Sq)) : 0;
  L.nk_blocks = p->mode == PE_MODE_POPE
                    ? pe::inv_blocks(p->B, p->Hkv, p->Sk, std::min(128, inv_rows(p->B, p->Hkv, p->Sk))) : 0;
  L.do_off = 0;
  L.sq_pad = (p->Sq + 127) / 128 * 128;
  const size_t nq_pad = (size_t)p->B * p->Hq * L.sq_pad;
  L.di_off = L.do_off + align_up(nq * L.dv * e);
  L.l2_off = L.di_off + align_up(nq_pad * 4);
  L.dq_off = L.l2_off + align_up(nq_pad * 4);
  const bool fb = !gm && fused_bwd(p);
  L.ksplit = masked ? 1 : key_split(p, L.dqk, L.dv);
  L.dk_off = L.dq_off + (fb ? 0 : align_up(nq * L.dqk * 4));
  // dk~ (unfused) or the split's partial dk~ slices
  L.pq_off = L.dk_off + (fb && L.ksplit == 1 ? 0 : align_up(nk * L.dqk * 4 * L.ksplit));
  L.pk_off = L.pq_off + align_up((size_t)L.nq_blocks * p->Dr * 4);
  L.pkd_off = L.pk_off + align_up((size_t)L.nk_blocks * p->Dr * 4);
  L.dvp_off = L.pkd_off + align_up((size_t)L.nk_blocks * p->Dr * 4);
  L.ds_off = L.dvp_off + (L.ksplit > 1 ? align_up(nk * L.dv * 4 * L.ksplit) : 0);
  // bf16 path: dS in fragment order, 4 KiB blocks packed per (b, h) to the blocks the causal
  // dK/dV kernel stores (pe::ds_row_base), written by it for the dQ GEMM.  The dQ GEMM's masked
  // edge steps also load up to four blocks before a key row's first stored one; those lie in the
  // earlier rows of the same or the previous (b, h), never before the buffer or past its end.
  L.ds_nqt = (p->Sq + 255) / 256 * 4;
  L.ds_rows = (p->Sk + 127) / 128 * 128;
  const int causal = p->causal != PE_CAUSAL_NONE;
  const int off = p->causal == PE_CAUSAL_BOTTOM_RIGHT ? p->Sk - p->Sq : 0;
  L.ds_e = causal ? (off + 63) / 64 : 0;
  L.ds_head = pe::ds_row_base(L.ds_rows / 32, L.ds_e, L.ds_nqt, causal);
  // dS of one (batch, kv head) unit: its query heads' regions; as many units per group as the cap
  // holds (at least one)
  const int units = p->B * p->Hkv;
  const bool store_ds = half_dt(p->dtype) && !gm;
  const size_t unit_bytes = (size_t)(p->Hq / p->Hkv) * L.ds_head * 4096;
  L.ds_group = units;
  if (store_ds && unit_bytes > 0 && (size_t)units * unit_bytes > PE_BWD_DS_CAP_BYTES)
    L.ds_group = std::max<int>(1, (int)(PE_BWD_DS_CAP_BYTES / unit_bytes));
  const size_t ds_bytes = store_ds ? (size_t)L.ds_group * unit_bytes : 0;
  L.bwd_total = L.ds_off + align_up(ds_bytes);
  return L;
}

// Profiling hook: process-wide array of 2*PE_STAGE_COUNT caller-owned hipEvent_t (may be NULL).
// Process-wide rather than per thread because torch's autograd engine runs backward passes on
// its own device thread.
std::atomic<void* const*> g_stage_events{nullptr};

inline void stage_mark(int stage, int end, hipStream_t s) {
  void* const* evs = g_stage_events.load(std::memory_order_acquire);
  if (!evs) return;
  void* ev = evs[2 * stage + end];
  if (ev) (void)hipEventRecord((hipEvent_t)ev, s);
}

int check_tensor(const pe_tensor_t* t, bool required) {
  if (!t) return required ? PE_ERR_NULL : PE_OK;
  if (!t->data) return required ? PE_ERR_NULL : PE_OK;
  if (!valid_dt(t->dtype)) return PE_ERR_MODE;
  if (t->stride[3] != 1) return PE_ERR_STRIDE;
  return PE_OK;
}

// an explicit mask view (B, Hq, Sq, Sk): bool bytes or a float type, element strides >= 0 (0 where
// it broadcasts), the base aligned to its element
int check_mask(const pe_tensor_t* m) {
  if (!m || !m->data) return PE_ERR_NULL;
  if (m->dtype != PE_DTYPE_BOOL && !valid_dt(m->dtype)) return PE_ERR_MODE;
  for (int i = 0; i < 4; ++i)
    if (m->stride[i] < 0) return PE_ERR_STRIDE;
  const uintptr_t e = m->dtype == PE_DTYPE_BOOL ? 1 : m->dtype == PE_DTYPE_FP32 ? 4 : 2;
  if ((uintptr_t)m->data % e) return PE_ERR_STRIDE;
  return PE_OK;
}

void set_mask(pe::CoreArgs& c, const pe_tensor_t* m) {
  if (!m) return;
  c.mask = m->data;
  c.m_sb = m->stride[0]; c.m_sh = m->stride[1]; c.m_sq = m->stride[2]; c.m_sk = m->stride[3];
  c.mask_dtype = m->dtype;
  c.mask_vec = m->stride[3] == 1 && m->stride[2] % 8 == 0 && m->stride[1] % 8 == 0 && m->stride[0] % 8 == 0 &&
               c.Sk % 8 == 0 && (uintptr_t)m->data % 16 == 0;
}

int dev_flags[64];  // 0 unknown, 1 gfx950, 2 other
int dev_cus[64];    // compute units of the device (set with its flag)
std::mutex dev_mu;

int device_ok() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return PE_ERR_NO_DEVICE;
  if (dev >= 64) return PE_OK;
  std::lock_guard<std::mutex> lk(dev_mu);
  if (dev_flags[dev] == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return PE_ERR_NO_DEVICE;
    dev_cus[dev] = prop.multiProcessorCount;
    dev_flags[dev] = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
  }
  return dev_flags[dev] == 1 ? PE_OK : PE_ERR_NO_DEVICE;
}

// CU count of the current device (MI355X: 256), for launch shapes that must fill the chip; every
// entry point calls device_ok first, which records it
int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lk(dev_mu);
  return dev_cus[dev] > 0 ? dev_cus[dev] : 256;
}

bool v_direct(const pe_attn_params* p, const pe_tensor_t* v, int dvp) {
  const int64_t e = (int64_t)esz(p);
  return v->dtype == p->dtype && p->Dv == dvp && ((uintptr_t)v->data % 16) == 0 &&
         (v->stride[0] * e) % 16 == 0 && (v->stride[1] * e) % 16 == 0 && (v->stride[2] * e) % 16 == 0;
}

void fill_prep(pe::PrepArgs& a, const pe_attn_params* p, int is_key, const pe_tensor_t* xc,
               const pe_tensor_t* xr, const float* freqs, const float* delta, void* dst, int width) {
  memset(&a, 0, sizeof(a));
  if (xc && xc->data) {
    a.xc = xc->data; a.xc_dtype = xc->dtype;
    for (int i = 0; i < 4; ++i) a.xc_s[i] = xc->stride[i];
  }
  a.xr = xr->data; a.xr_dtype = xr->dtype;
  for (int i = 0; i < 4; ++i) a.xr_s[i] = xr->stride[i];
  a.dst = dst; a.dst_dtype = p->dtype; a.width = width;
  a.B = p->B; a.H = is_key ? p->Hkv : p->Hq; a.S = is_key ? p->Sk : p->Sq;
  a.Dc = p->Dc; a.Dr = p->Dr; a.mode = p->mode;
  a.start_pos = is_key ? p->start_pos_k : p->start_pos_q;
  a.pos_round = p->position_rounding;
  a.l2norm = p->qk_l2norm; a.is_key = is_key;
  a.freqs = freqs; a.delta = delta; a.delta_hs = p->delta_head_stride;
  a.mscale = p->rope_mscale;
}

pe::CoreArgs core_args(const pe_attn_params* p, const Layout& L, const char* ws,
                       const pe_tensor_t* v) {
  pe::CoreArgs c;
  memset(&c, 0, sizeof(c));
  c.q = ws + L.q_off;
  c.k = ws + L.k_off;
  if (v_direct(p, v, L.dv)) {
    c.v = v->data; c.v_sb = v->stride[0]; c.v_sh = v->stride[1]; c.v_ss = v->stride[2];
  } else {
    c.v = ws + L.v_off; c.v_ss = L.dv; c.v_sh = (int64_t)p->Sk * L.dv; c.v_sb = (int64_t)p->Hkv * p->Sk * L.dv;
  }
  c.B = p->B; c.Hq = p->Hq; c.Hkv = p->Hkv; c.Sq = p->Sq; c.Sk = p->Sk;
  c.n_cu = device_cus();
  c.dv_real = p->Dv;
  c.causal = p->causal != PE_CAUSAL_NONE;
  c.causal_off = p->causal == PE_CAUSAL_BOTTOM_RIGHT ? p->Sk - p->Sq : 0;
  c.scale = p->scale;
  c.bh0 = 0;
  c.nbh = p->B * p->Hkv;
  c.qsplit = 1;
  return c;
}

}  // namespace

extern "C" {

int pe_attn_version(void) { return PE_ATTN_ABI_VERSION; }

int pe_attn_set_stage_events(void* const* events) {
  g_stage_events.store(events, std::memory_order_release);
  return PE_OK;
}

const char* pe_attn_strerror(int code) {
  switch (code) {
    case PE_OK: return "success";
    case PE_ERR_NULL: return "pe_attn: a required pointer is NULL";
    case PE_ERR_SHAPE: return "pe_attn: invalid shape (sizes must be positive, Hq divisible by Hkv, Sq <= Sk for bottom-right causal)";
    case PE_ERR_HEAD_DIM: return "pe_attn: unsupported head width (transformed q/k width must be <= 256, value width <= 128, PoPE dims <= 256)";
    case PE_ERR_MODE: return "pe_attn: invalid mode, dtype or causal flag (RoPE needs an even width)";
    case PE_ERR_STRIDE: return "pe_attn: last-dimension stride must be 1";
    case PE_ERR_WORKSPACE: return "pe_attn: workspace missing or too small";
    case PE_ERR_LAUNCH: return "pe_attn: kernel launch failed";
    case PE_ERR_NO_DEVICE: return "pe_attn: current device is not an MI355X (gfx950)";
    case PE_ERR_SCRATCH_LIMIT: return "pe_attn: the call needs more than the library's static scratch (pe_attn_noalloc_scratch_bytes); use the workspace entry point";
    default: return "pe_attn: unknown error";
  }
}

int pe_attn_check(const pe_attn_params* p) {
  if (!p) return PE_ERR_NULL;
  if (p->B <= 0 || p->Hq <= 0 || p->Hkv <= 0 || p->Sq <= 0 || p->Sk <= 0 || p->Dv <= 0 || p->Dr < 0 || p->Dc < 0)
    return PE_ERR_SHAPE;
  if (p->Hq % p->Hkv != 0) return PE_ERR_SHAPE;
  if (p->mode < 0 || p->mode > 2 || !valid_dt(p->dtype) || p->causal < 0 || p->causal > 2)
    return PE_ERR_MODE;
  if (p->mode != PE_MODE_POPE && (p->Dr % 2) != 0) return PE_ERR_MODE;
  if (p->position_rounding < PE_POS_EXACT || p->position_rounding > PE_POS_FP16 ||
      (p->position_rounding != PE_POS_EXACT && p->mode != PE_MODE_POPE))
    return PE_ERR_MODE;
  if (p->causal == PE_CAUSAL_BOTTOM_RIGHT && p->Sq > p->Sk) return PE_ERR_SHAPE;
  if (p->causal == PE_CAUSAL_TOP_LEFT && p->Sq != p->Sk) return PE_ERR_SHAPE;
  if (qk_width(p) <= 0 || pad_qk(qk_width(p)) < 0 || pad_v(p->Dv) < 0) return PE_ERR_HEAD_DIM;
  if (p->Dr > 256 || (p->mode != PE_MODE_POPE && p->Dr > 2 * 64 * 4)) return PE_ERR_HEAD_DIM;
  if (!pe::core_supported(pad_qk(qk_width(p)), pad_v(p->Dv))) return PE_ERR_HEAD_DIM;
  return PE_OK;
}

int pe_attn_operand_width(const pe_attn_params* p) {
  if (pe_attn_check(p) != PE_OK) return -1;
  return pad_qk(qk_width(p));
}

size_t pe_attn_fwd_workspace_bytes(const pe_attn_params* p) {
  if (pe_attn_check(p) != PE_OK) return 0;
  return layout(p).fwd_total;
}

size_t pe_attn_bwd_workspace_bytes(const pe_attn_params* p) {
  if (pe_attn_check(p) != PE_OK) return 0;
  return layout(p).bwd_total;
}

size_t pe_attn_bwd_masked_workspace_bytes(const pe_attn_params* p) {
  if (pe_attn_check(p) != PE_OK) return 0;
  return layout(p, true).bwd_total;
}

int pe_attn_transform(const pe_attn_params* p, int is_key, const pe_tensor_t* xc, const pe_tensor_t* xr,
                      const float* freqs, const float* delta, void* dst, void* stream) {
  int rc = pe_attn_check(p);
  if (rc) return rc;
  if ((rc = check_tensor(xr, p->Dr > 0))) return rc;
  if ((rc = check_tensor(xc, p->Dc > 0))) return rc;
  if (!dst || (p->mode != PE_MODE_NONE && p->Dr > 0 && !freqs)) return PE_ERR_NULL;
  if ((rc = device_ok())) return rc;
  pe::PrepArgs a;
  fill_prep(a, p, is_key, xc, xr, freqs, delta, dst, pad_qk(qk_width(p)));
  return pe::launch_prep(a, (hipStream_t)stream);
}

size_t pe_attn_transform_bwd_workspace_bytes(const pe_attn_params* p, int is_key) {
  if (pe_attn_check(p) != PE_OK) return 0;
  if (p->mode != PE_MODE_POPE) return ALIGN;
  const int H = is_key ? p->Hkv : p->Hq, S = is_key ? p->Sk : p->Sq;
  const int nb = pe::inv_blocks(p->B, H, S, inv_rows(p->B, H, S));
  return 2 * align_up((size_t)nb * (p->Dr > 0 ? p->Dr : 1) * 4);
}

int pe_attn_transform_bwd(const pe_attn_params* p, int is_key, const float* g, const pe_tensor_t* xr,
                          const float* freqs, const float* delta, const pe_tensor_t* dxc,
                          const pe_tensor_t* dxr, float* dfreqs, float* ddelta, void* workspace,
                          size_t ws_bytes, void* stream) {
  int rc = pe_attn_check(p);
  if (rc) return rc;
  if ((rc = check_tensor(xr, p->Dr > 0)) || (rc = check_tensor(dxr, p->Dr > 0)) ||
      (rc = check_tensor(dxc, p->Dc > 0)))
    return rc;
  if (!g || (p->mode != PE_MODE_NONE && p->Dr > 0 && !freqs)) return PE_ERR_NULL;
  const size_t need = pe_attn_transform_bwd_workspace_bytes(p, is_key);
  if (!workspace || ws_bytes < need) return PE_ERR_WORKSPACE;
  if ((rc = device_ok())) return rc;
  hipStream_t s = (hipStream_t)stream;
  const int H = is_key ? p->Hkv : p->Hq, S = is_key ? p->Sk : p->Sq;
  const int rows = inv_rows(p->B, H, S);
  const int nb = pe::inv_blocks(p->B, H, S, rows);
  float* part_f = (float*)workspace;
  float* part_d = (float*)((char*)workspace + need / 2);
  pe::InvArgs ia;
  memset(&ia, 0, sizeof(ia));
  ia.g = g;
  ia.width = pad_qk(qk_width(p));
  if (xr && xr->data) { ia.xr = xr->data; ia.xr_dtype = xr->dtype; for (int i = 0; i < 4; ++i) ia.xr_s[i] = xr->stride[i]; }
  if (dxc && dxc->data) { ia.dxc = (void*)dxc->data; ia.dxc_dtype = dxc->dtype; for (int i = 0; i < 4; ++i) ia.dxc_s[i] = dxc->stride[i]; }
  if (dxr && dxr->data) { ia.dxr = (void*)dxr->data; ia.dxr_dtype = dxr->dtype; for (int i = 0; i < 4; ++i) ia.dxr_s[i] = dxr->stride[i]; }
  ia.B = p->B; ia.H = H; ia.S = S;
  ia.Dc = p->Dc; ia.Dr = p->Dr; ia.mode = p->mode;
  ia.start_pos = is_key ? p->start_pos_k : p->start_pos_q;
  ia.pos_round = p->position_rounding;
  ia.l2norm = p->qk_l2norm; ia.is_key = is_key;
  ia.freqs = freqs; ia.delta = is_key ? delta : nullptr; ia.delta_hs = p->delta_head_stride;
  ia.mscale = p->rope_mscale;
  ia.part_delta = (is_key && p->mode == PE_MODE_POPE) ? part_d : nullptr;
  ia.part_freq = p->mode == PE_MODE_POPE ? part_f : nullptr;
  ia.rows_per_block = rows;
  if (ia.Dr == 0 && ia.Dc > 0) ia.mode = PE_MODE_NONE;
  if ((rc = pe::launch_inv(ia, nullptr, s))) return rc;
  if (p->mode == PE_MODE_POPE && p->Dr > 0 && (dfreqs || (is_key && ddelta))) {
    pe::ReduceArgs ra;
    memset(&ra, 0, sizeof(ra));
    if (is_key) {
      ra.part_k_freq = part_f; ra.part_k_delta = part_d; ra.nk = nb;
    } else {
      ra.part_q_freq = part_f; ra.nq = nb;
    }
    ra.k_blocks_per_head = (S + rows - 1) / rows;
    ra.Hkv = H; ra.B = p->B; ra.Dr = p->Dr;
    ra.delta_per_head = p->delta_head_stride != 0;
    ra.dfreqs = dfreqs; ra.ddelta = is_key ? ddelta : nullptr;
    if ((rc = pe::launch_reduce(ra, s))) return rc;
  }
  return PE_OK;
}

static int fwd_impl(const pe_attn_params* p, const pe_norm_params* nrm, const pe_tensor_t* qc,
                    const pe_tensor_t* qr, const pe_tensor_t* kc, const pe_tensor_t* kr, const pe_tensor_t* v,
                    const float* freqs, const float* delta, const pe_tensor_t* out, float* lse,
                    void* fwd_workspace, size_t fwd_ws_bytes, void* stream, const pe_tensor_t* mask = nullptr) {
  int rc = pe_attn_check(p);
  if (rc) return rc;
  if (mask && (rc = check_mask(mask))) return rc;
  if (nrm) {
    if (p->mode != PE_MODE_POPE || p->Dr <= 0) return PE_ERR_MODE;
    if (!nrm->q_weight || !nrm->k_weight) return PE_ERR_NULL;
    if (!valid_dt(nrm->weight_dtype)) return PE_ERR_MODE;
  }
  if ((rc = check_tensor(qr, p->Dr > 0)) || (rc = check_tensor(kr, p->Dr > 0)) ||
      (rc = check_tensor(qc, p->Dc > 0)) || (rc = check_tensor(kc, p->Dc > 0)) ||
      (rc = check_tensor(v, true)) || (rc = check_tensor(out, true)))
    return rc;
  if (!lse || (p->mode != PE_MODE_NONE && p->Dr > 0 && !freqs)) return PE_ERR_NULL;
  if (out->dtype != p->dtype) return PE_ERR_MODE;
  const Layout L = layout(p);
  if (!fwd_workspace || fwd_ws_bytes < L.fwd_total) return PE_ERR_WORKSPACE;
  if ((rc = device_ok())) return rc;
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)fwd_workspace;

  pe::PrepArgs a;
  stage_mark(PE_STAGE_FWD_PREP, 0, s);
  float* qtab = use_qtab(p) ? (float*)(ws + L.tab_off) : nullptr;
  if (nrm) {
    if (qtab && (rc = pe::launch_phase_table(freqs, p->start_pos_q, p->Sq, p->Dr, p->position_rounding, qtab, s)))
      return rc;
    fill_prep(a, p, 0, qc, qr, freqs, nullptr, ws + L.q_off, L.dqk);
    a.tab = qtab;
    a.norm_w = nrm->q_weight; a.norm_w_dtype = nrm->weight_dtype; a.norm_eps = nrm->eps;
    if ((rc = pe::launch_prep_norm(a, s))) return rc;
    fill_prep(a, p, 1, kc, kr, freqs, delta, ws + L.k_off, L.dqk);
    a.norm_w = nrm->k_weight; a.norm_w_dtype = nrm->weight_dtype; a.norm_eps = nrm->eps;
    if ((rc = pe::launch_prep_norm(a, s))) return rc;
  } else {
    // small shapes: both sides in one launch; larger ones without a content part: both sides in
    // one launch with each query phase evaluated once for several heads; else keys first, with the
    // query phase table in the same launch, and the queries, which read the table, after it
    fill_prep(a, p, 1, kc, kr, freqs, delta, ws + L.k_off, L.dqk);
    pe::PrepArgs aq;
    fill_prep(aq, p, 0, qc, qr, freqs, nullptr, ws + L.q_off, L.dqk);
    rc = qtab ? pe::launch_prep_qk(a, aq, qtab, s) : 1;
    if (rc == 1 && qtab) rc = pe::launch_prep_k_qheads(a, aq, qtab, s);
    if (rc == 1) {
      if (qtab) rc = pe::launch_prep_and_table(a, freqs, p->start_pos_q, p->Sq, p->Dr, p->position_rounding, qtab, s);
      else rc = pe::launch_prep(a, s);
      if (rc) return rc;
      aq.tab = qtab;
      rc = pe::launch_prep(aq, s);
    }
    if (rc) return rc;
  }
  if (!v_direct(p, v, L.dv)) {
    pe_attn_params pv = *p;
    pv.mode = PE_MODE_NONE; pv.Dc = 0; pv.Dr = p->Dv; pv.qk_l2norm = 0;
    fill_prep(a, &pv, 1, nullptr, v, nullptr, nullptr, ws + L.v_off, L.dv);
    if ((rc = pe::launch_prep(a, s))) return rc;
  }
  stage_mark(PE_STAGE_FWD_PREP, 1, s);
  pe::CoreArgs c = core_args(p, L, ws, v);
  c.o = (void*)out->data; c.o_sb = out->stride[0]; c.o_sh = out->stride[1]; c.o_ss = out->stride[2];
  c.o_dtype = out->dtype;
  c.lse = lse;
  set_mask(c, mask);
  stage_mark(PE_STAGE_FWD_CORE, 0, s);
  rc = pe::launch_fwd(p->dtype, L.dqk, L.dv, c, s);
  stage_mark(PE_STAGE_FWD_CORE, 1, s);
  return rc;
}

int pe_attn_fwd(const pe_attn_params* p, const pe_tensor_t* qc, const pe_tensor_t* qr,
                const pe_tensor_t* kc, const pe_tensor_t* kr, const pe_tensor_t* v,
                const float* freqs, const float* delta, const pe_tensor_t* out, float* lse,
                void* fwd_workspace, size_t fwd_ws_bytes, void* stream) {
  return fwd_impl(p, nullptr, qc, qr, kc, kr, v, freqs, delta, out, lse, fwd_workspace, fwd_ws_bytes, stream);
}

int pe_attn_fwd_masked(const pe_attn_params* p, const pe_tensor_t* qc, const pe_tensor_t* qr,
                       const pe_tensor_t* kc, const pe_tensor_t* kr, const pe_tensor_t* v,
                       const float* freqs, const float* delta, const pe_tensor_t* mask, const pe_tensor_t* out,
                       float* lse, void* fwd_workspace, size_t fwd_ws_bytes, void* stream) {
  if (!mask) return PE_ERR_NULL;
  return fwd_impl(p, nullptr, qc, qr, kc, kr, v, freqs, delta, out, lse, fwd_workspace, fwd_ws_bytes, stream, mask);
}

}  // extern "C"

namespace {

// Library-owned scratch for pe_attn_fwd_noalloc: the forward workspace (transformed operands, value
// repack, query phase table) of calls that may not allocate.  Each GPU the library runs on holds
// its own copy from code-object load until the process ends.  In host code `scratch` names a
// host-side stand-in, never the device memory: its address on the current device comes from
// hipGetSymbolAddress, once per device, and only that pointer is handed to kernels.
__device__ __align__(256) char scratch[PE_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64];  // per device ordinal; nullptr until resolved

// device address of `scratch` on the current device (resolved on the first call per device)
int scratch_on_current_device(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return PE_ERR_NO_DEVICE;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return PE_ERR_LAUNCH;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return PE_OK;
}

}  // namespace

extern "C" {

size_t pe_attn_noalloc_scratch_bytes(void) { return PE_NOALLOC_SCRATCH_BYTES; }

int pe_attn_fwd_noalloc(const pe_attn_params* p, const pe_tensor_t* qc, const pe_tensor_t* qr,
                        const pe_tensor_t* kc, const pe_tensor_t* kr, const pe_tensor_t* v,
                        const float* freqs, const float* delta, const pe_tensor_t* out, float* lse,
                        void* stream) {
  int rc = pe_attn_check(p);
  if (rc) return rc;
  if (layout(p).fwd_total > PE_NOALLOC_SCRATCH_BYTES) return PE_ERR_SCRATCH_LIMIT;
  if ((rc = device_ok())) return rc;
  void* ws = nullptr;
  if ((rc = scratch_on_current_device(&ws))) return rc;
  // every byte the kernels read from the workspace is written earlier in the same call (operand
  // rows including their zero padding, the phase table, the value repack), so nothing is cleared
  return fwd_impl(p, nullptr, qc, qr, kc, kr, v, freqs, delta, out, lse, ws, PE_NOALLOC_SCRATCH_BYTES, stream);
}

int pe_attn_value_width(const pe_attn_params* p) {
  if (pe_attn_check(p) != PE_OK) return -1;
  return pad_v(p->Dv);
}

}  // extern "C"

namespace {

// Work split and workspace of pe_attn_decode: transformed queries, then the per-range partials.
struct DecodePlan {
  int nqt, nunit;
  size_t q_bytes, po_off, pm_off, pl_off, total;
};

DecodePlan decode_plan(const pe_attn_params* p) {
  DecodePlan d{};
  const int grp = p->Hq / p->Hkv;
  d.nqt = (int)(((int64_t)grp * p->Sq + 31) / 32);
  const int64_t tiles = (int64_t)p->B * p->Hkv * d.nqt;
  const int nkb = (p->Sk + 31) / 32;
  // about 1024 waves over the GPU (one 4-wave workgroup per CU of the MI355X: in one A/B at 16384
  // cached rows 1024 measured 44.8 us per decode step against 53.2 for 512, 45.6 for 768, 46.1 for
  // 2048 and 49.8 for 4096), at least two 32-key blocks per range, a multiple of 4 ranges.  A fixed
  // count, not the device's: the workspace query and the call must size the partials alike.
  int64_t nu = (1024 + tiles - 1) / tiles;
  nu = std::min<int64_t>(nu, (nkb + 1) / 2);
  nu = std::max<int64_t>(4, std::min<int64_t>(512, (nu + 3) / 4 * 4));
  d.nunit = (int)nu;
  const size_t rows = (size_t)tiles * d.nunit * 32;
  d.q_bytes = align_up((size_t)p->B * p->Hq * p->Sq * pad_qk(qk_width(p)) * esz(p));
  d.po_off = d.q_bytes;
  d.pm_off = d.po_off + align_up(rows * pad_v(p->Dv) * 4);
  d.pl_off = d.pm_off + align_up(rows * 4);
  d.total = d.pl_off + align_up(rows * 4);
  return d;
}

// the parameter block of the new key rows written by pe_attn_cache_append: Sk rows per kv head
int append_params(const pe_attn_params* p, pe_attn_params* q) {
  *q = *p;
  q->Hq = p->Hkv;
  q->Sq = p->Sk;
  q->causal = PE_CAUSAL_NONE;
  return pe_attn_check(q);
}

}  // namespace

extern "C" {

int pe_attn_cache_append(const pe_attn_params* p, const pe_tensor_t* kc, const pe_tensor_t* kr,
                         const pe_tensor_t* v, const float* freqs, const float* delta, void* k_cache,
                         void* v_cache, int32_t capacity, void* stream) {
  if (!p) return PE_ERR_NULL;
  pe_attn_params pa;
  int rc = append_params(p, &pa);
  if (rc) return rc;
  if (p->start_pos_k < 0 || capacity <= 0 || (int64_t)p->start_pos_k + p->Sk > capacity) return PE_ERR_SHAPE;
  if ((rc = check_tensor(kr, p->Dr > 0)) || (rc = check_tensor(kc, p->Dc > 0)) || (rc = check_tensor(v, true)))
    return rc;
  if (!k_cache || !v_cache || (p->mode != PE_MODE_NONE && p->Dr > 0 && !freqs)) return PE_ERR_NULL;
  if ((uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16) return PE_ERR_STRIDE;
  if ((rc = device_ok())) return rc;
  hipStream_t s = (hipStream_t)stream;
  pe::PrepArgs a;
  fill_prep(a, &pa, 1, kc, kr, freqs, delta, k_cache, pad_qk(qk_width(&pa)));
  a.dst_rows = capacity;
  a.dst_row0 = p->start_pos_k;
  // the value rows go out in the key rows' launch when both take the vectorised path (bf16 PoPE
  // rows, 16-byte aligned, unit inner stride), otherwise in a launch of their own
  a.cv = v->data; a.cv_cols = p->Dv; a.cdst = v_cache; a.cwidth = pad_v(p->Dv);
  for (int i = 0; i < 4; ++i) a.cv_s[i] = v->stride[i];
  if (v->dtype == PE_DTYPE_BF16 && p->dtype == PE_DTYPE_BF16 && pe::prep_vec_copy_ok(a)) return pe::launch_prep(a, s);
  a.cv = nullptr; a.cdst = nullptr;
  if ((rc = pe::launch_prep(a, s))) return rc;
  pe_attn_params pv = pa;
  pv.mode = PE_MODE_NONE; pv.Dc = 0; pv.Dr = p->Dv; pv.qk_l2norm = 0;
  fill_prep(a, &pv, 1, nullptr, v, nullptr, nullptr, v_cache, pad_v(p->Dv));
  a.dst_rows = capacity;
  a.dst_row0 = p->start_pos_k;
  return pe::launch_prep(a, s);
}

size_t pe_attn_decode_workspace_bytes(const pe_attn_params* p) {
  if (pe_attn_check(p) != PE_OK) return 0;
  return decode_plan(p).total;
}

int pe_attn_decode(const pe_attn_params* p, const pe_tensor_t* qc, const pe_tensor_t* qr,
                   const void* k_cache, const void* v_cache, int32_t capacity, const float* freqs,
                   const pe_tensor_t* out, float* lse, void* workspace, size_t ws_bytes, void* stream) {
  int rc = pe_attn_check(p);
  if (rc) return rc;
  if (capacity < p->Sk) return PE_ERR_SHAPE;
  if ((rc = check_tensor(qr, p->Dr > 0)) || (rc = check_tensor(qc, p->Dc > 0)) || (rc = check_tensor(out, true)))
    return rc;
  if (!k_cache || !v_cache || !lse || (p->mode != PE_MODE_NONE && p->Dr > 0 && !freqs)) return PE_ERR_NULL;
  if ((uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16) return PE_ERR_STRIDE;
  if (out->dtype != p->dtype) return PE_ERR_MODE;
  const DecodePlan d = decode_plan(p);
  if (!workspace || ws_bytes < d.total) return PE_ERR_WORKSPACE;
  if ((rc = device_ok())) return rc;
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const int dqk = pad_qk(qk_width(p)), dv = pad_v(p->Dv);
  pe::PrepArgs a;
  fill_prep(a, p, 0, qc, qr, freqs, nullptr, ws, dqk);
  // a tile of few query rows (one decoded token of a small GQA group) is transformed inside the
  // split kernel, with the prologue's arithmetic, instead of in a launch of its own
  const bool fuse_q = p->dtype == PE_DTYPE_BF16 && (int64_t)(p->Hq / p->Hkv) * p->Sq <= pe::DECODE_FUSED_ROWS &&
                      pe::prep_vec_query_ok(a);
  if (!fuse_q && (rc = pe::launch_prep(a, s))) return rc;
  pe::DecodeArgs da;
  memset(&da, 0, sizeof(da));
  if (fuse_q) {
    da.qraw = qr->data;
    for (int i = 0; i < 4; ++i) da.qr_s[i] = qr->stride[i];
    da.freqs = freqs; da.Dr = p->Dr; da.start_pos = p->start_pos_q; da.pos_round = p->position_rounding;
  }
  da.q = ws; da.k = k_cache; da.v = v_cache;
  da.B = p->B; da.Hq = p->Hq; da.Hkv = p->Hkv; da.Sq = p->Sq; da.L = p->Sk; da.cap = capacity;
  da.causal = p->causal != PE_CAUSAL_NONE;
  da.off = p->causal == PE_CAUSAL_BOTTOM_RIGHT ? p->Sk - p->Sq : 0;
  da.scale = p->scale;
  da.nqt = d.nqt; da.nunit = d.nunit;
  da.part_o = (float*)(ws + d.po_off);
  da.part_m = (float*)(ws + d.pm_off);
  da.part_l = (float*)(ws + d.pl_off);
  da.o = (void*)out->data; da.o_sb = out->stride[0]; da.o_sh = out->stride[1]; da.o_ss = out->stride[2];
  da.o_dtype = out->dtype; da.dv_real = p->Dv;
  da.lse = lse;
  return pe::launch_decode(p->dtype, dqk, dv, da, s);
}

int pe_attn_fwd_normed(const pe_attn_params* p, const pe_norm_params* n, const pe_tensor_t* qc,
                       const pe_tensor_t* qr, const pe_tensor_t* kc, const pe_tensor_t* kr,
                       const pe_tensor_t* v, const float* freqs, const float* delta,
                       const pe_tensor_t* out, float* lse, void* fwd_workspace, size_t fwd_ws_bytes,
                       void* stream) {
  if (!n) return PE_ERR_NULL;
  return fwd_impl(p, n, qc, qr, kc, kr, v, freqs, delta, out, lse, fwd_workspace, fwd_ws_bytes, stream);
}

int pe_rmsnorm_fwd(const void* x, int32_t x_dtype, int64_t x_row_stride, int64_t rows, int32_t n,
                   const void* weight, int32_t weight_dtype, float eps, void* y, int32_t y_dtype,
                   int64_t y_row_stride, void* stream) {
  if (!x || !weight || !y) return PE_ERR_NULL;
  int rc = device_ok();
  if (rc) return rc;
  pe::NormArgs a;
  a.x = x; a.x_dtype = x_dtype; a.x_rs = x_row_stride;
  a.w = weight; a.w_dtype = weight_dtype;
  a.y = y; a.y_dtype = y_dtype; a.y_rs = y_row_stride;
  a.rows = rows; a.n = n; a.eps = eps;
  return pe::launch_rmsnorm(a, (hipStream_t)stream);
}

// the backward's row partition assumes MI355X's 256 compute units in both the workspace size and
// the launch, so the size a caller allocated always matches the launch
constexpr int kNormBwdCus = 256;

size_t pe_rmsnorm_bwd_workspace_bytes(int64_t rows, int32_t n) {
  if (rows <= 0 || n <= 0) return 0;
  return align_up((size_t)pe::rmsnorm_bwd_part_floats(rows, n, kNormBwdCus) * 4);
}

int pe_rmsnorm_bwd(const void* x, int32_t x_dtype, int64_t x_row_stride, int64_t rows, int32_t n,
                   const void* weight, int32_t weight_dtype, float eps, const void* dy, int64_t dy_row_stride,
                   void* dx, int64_t dx_row_stride, void* dw, void* workspace, size_t ws_bytes, void* stream) {
  if (!x || !weight || !dy || !dx || !dw || !workspace) return PE_ERR_NULL;
  if (rows <= 0 || n <= 0) return PE_ERR_SHAPE;
  if (ws_bytes < pe_rmsnorm_bwd_workspace_bytes(rows, n)) return PE_ERR_WORKSPACE;
  int rc = device_ok();
  if (rc) return rc;
  pe::NormBwdArgs a;
  memset(&a, 0, sizeof(a));
  a.x = x; a.x_dtype = x_dtype; a.x_rs = x_row_stride;
  a.w = weight; a.w_dtype = weight_dtype;
  a.dy = dy; a.dy_rs = dy_row_stride;
  a.dx = dx; a.dx_rs = dx_row_stride;
  a.dw = dw; a.dw_dtype = weight_dtype;
  a.part = (float*)workspace;
  a.rows = rows; a.n = n; a.eps = eps;
  return pe::launch_rmsnorm_bwd(a, kNormBwdCus, (hipStream_t)stream);
}

int pe_swiglu_fwd(const void* x, const void* gate, void* out, int64_t n, void* stream) {
  if (!x || !gate || !out) return PE_ERR_NULL;
  if (n < 0 || n % 8 != 0) return PE_ERR_SHAPE;
  if (((uintptr_t)x | (uintptr_t)gate | (uintptr_t)out) % 16) return PE_ERR_STRIDE;
  const int rc = device_ok();
  if (rc) return rc;
  return pe::launch_swiglu(x, gate, out, n, (hipStream_t)stream);
}

}  // extern "C"

static int bwd_impl(const pe_attn_params* p, const pe_tensor_t* qc, const pe_tensor_t* qr,
                    const pe_tensor_t* kc, const pe_tensor_t* kr, const pe_tensor_t* v,
                    const float* freqs, const float* delta, const pe_tensor_t* mask, const pe_tensor_t* out,
                    const float* lse, const pe_tensor_t* dout, const pe_tensor_t* dqc, const pe_tensor_t* dqr,
                    const pe_tensor_t* dkc, const pe_tensor_t* dkr, const pe_tensor_t* dv,
                    float* dfreqs, float* ddelta, const void* fwd_workspace, size_t fwd_ws_bytes,
                    void* bwd_workspace, size_t bwd_ws_bytes, void* stream) {
  int rc = pe_attn_check(p);
  if (rc) return rc;
  const bool masked = mask != nullptr;
  if (masked && (rc = check_mask(mask))) return rc;
  if ((rc = check_tensor(qr, p->Dr > 0)) || (rc = check_tensor(kr, p->Dr > 0)) ||
      (rc = check_tensor(qc, p->Dc > 0)) || (rc = check_tensor(kc, p->Dc > 0)) ||
      (rc = check_tensor(v, true)) || (rc = check_tensor(out, true)) || (rc = check_tensor(dout, true)) ||
      (rc = check_tensor(dqr, p->Dr > 0)) || (rc = check_tensor(dkr, p->Dr > 0)) ||
      (rc = check_tensor(dqc, p->Dc > 0)) || (rc = check_tensor(dkc, p->Dc > 0)) ||
      (rc = check_tensor(dv, true)))
    return rc;
  if (!lse || (p->mode != PE_MODE_NONE && p->Dr > 0 && !freqs)) return PE_ERR_NULL;
  // 16-bit compute: the gradient kernels' epilogues read the operands and write the gradients in
  // fp32 or in the compute's own 16-bit type, not in the other one
  if (half_dt(p->dtype)) {
    for (const pe_tensor_t* t : {qc, qr, kc, kr, v, dqc, dqr, dkc, dkr, dv})
      if (t && t->data && t->dtype != p->dtype && t->dtype != PE_DTYPE_FP32) return PE_ERR_MODE;
  }
  const Layout L = layout(p, masked);
  if (!fwd_workspace || fwd_ws_bytes < L.fwd_total || !bwd_workspace || bwd_ws_bytes < L.bwd_total)
    return PE_ERR_WORKSPACE;
  if ((rc = device_ok())) return rc;
  hipStream_t s = (hipStream_t)stream;
  const char* fws = (const char*)fwd_workspace;
  char* bws = (char*)bwd_workspace;
  const int dt = p->dtype;  // the kernels' dtype codes are the ABI's

  pe::PreBwdArgs pb;
  memset(&pb, 0, sizeof(pb));
  pb.dout = dout->data; pb.dout_dtype = dout->dtype;
  pb.out = out->data; pb.out_dtype = out->dtype;
  for (int i = 0; i < 4; ++i) { pb.do_s[i] = dout->stride[i]; pb.o_s[i] = out->stride[i]; }
  // the bf16 dK/dV kernel reads dO in place when its rows are 16-byte aligned and exactly Dv wide
  const bool gm = generic_masked(p, masked);
  const bool do_direct = half_dt(dt) && !gm && v_direct(p, dout, L.dv);
  pb.dO_op = do_direct ? nullptr : bws + L.do_off; pb.op_dtype = p->dtype; pb.width = L.dv;
  pb.Di = (float*)(bws + L.di_off);
  pb.L2 = (float*)(bws + L.l2_off);
  pb.lse = lse;
  pb.s_pad = L.sq_pad;
  pb.B = p->B; pb.H = p->Hq; pb.S = p->Sq; pb.Dv = p->Dv;
  stage_mark(PE_STAGE_BWD_PRE, 0, s);
  if ((rc = pe::launch_prebwd(pb, s))) return rc;
  stage_mark(PE_STAGE_BWD_PRE, 1, s);

  pe::CoreArgs c = core_args(p, L, fws, v);
  if (do_direct) {
    c.dO = dout->data; c.do_sb = dout->stride[0]; c.do_sh = dout->stride[1]; c.do_ss = dout->stride[2];
  } else {
    c.dO = bws + L.do_off; c.do_ss = L.dv; c.do_sh = (int64_t)p->Sq * L.dv; c.do_sb = (int64_t)p->Hq * p->Sq * L.dv;
  }
  c.Di = (const float*)(bws + L.di_off);
  c.L2 = (const float*)(bws + L.l2_off);
  c.sq_pad = L.sq_pad;
  c.dS = (uint16_t*)(bws + L.ds_off);
  c.ds_nqt = L.ds_nqt;
  c.ds_rows = L.ds_rows;
  c.ds_e = L.ds_e;
  c.ds_head = L.ds_head;
  c.lse_in = lse;
  c.dq_t = (float*)(bws + L.dq_off);
  c.qtab = use_qtab(p) ? (const float*)(fws + L.tab_off) : nullptr;
  c.dk_t = (float*)(bws + L.dk_off);
  c.qsplit = L.ksplit;
  c.dv_part = L.ksplit > 1 ? (float*)(bws + L.dvp_off) : nullptr;
  c.dv = (void*)dv->data; c.dv_sb = dv->stride[0]; c.dv_sh = dv->stride[1]; c.dv_ss = dv->stride[2];
  c.dv_dtype = dv->dtype;
  set_mask(c, mask);
  stage_mark(PE_STAGE_BWD_DKDV, 0, s);
  // fused form in bf16 with both halves of a column in one wave: the gradient kernels apply the
  // inverse PoPE transform in their epilogues
  const bool split = !gm && fused_split_bwd(p, qr, kr, dqc, dqr, dkc, dkr);
  const bool fuse = (!gm && fused_bwd(p)) || split;
  // RoPE / no-PE (QKNorm included) at transformed width 64, the reference's head width, with vector
  // views: the dQ GEMM and the dK/dV kernel apply the gradient in their epilogues instead of the
  // stand-alone kernels below (the workspace still reserves dq~ / dk~: alignment is a call-time fact)
  const bool rfuse = !gm && half_dt(dt) && (p->mode == PE_MODE_ROPE || p->mode == PE_MODE_NONE) && p->Dc == 0 &&
                     p->Dr == 64 && L.dqk == 64 && vec16(qr) && vec16(kr) && vec16(dqr) && vec16(dkr);
  const int nqg = (p->Sq + 255) / 256, nkg = (p->Sk + 127) / 128;
  auto view = [p](pe::EpiPoPE& e, const pe_tensor_t* x, const pe_tensor_t* dx, int start) {
    e.x = x->data; e.x_dtype = x->dtype;
    e.dx = (void*)dx->data; e.dx_dtype = dx->dtype;
    for (int i = 0; i < 4; ++i) { e.x_s[i] = x->stride[i]; e.dx_s[i] = dx->stride[i]; }
    e.start_pos = start;
    e.pos_round = p->position_rounding;
  };
  if (rfuse) {
    c.rope_fuse = 1;
    c.rope_mode = p->mode;
    c.rope_l2 = p->qk_l2norm;
    c.rope_ms = p->rope_mscale;
    c.freqs = freqs;
    view(c.eq, qr, dqr, p->start_pos_q);
    view(c.ek, kr, dkr, p->start_pos_k);
  }
  if (fuse) {
    c.fuse_inv = 1;
    c.Dr = p->Dr;
    c.Dc = p->Dc;
    c.freqs = freqs;
    c.delta = delta;
    c.delta_hs = p->delta_head_stride;
    view(c.eq, qr, dqr, p->start_pos_q);
    view(c.ek, kr, dkr, p->start_pos_k);
    if (split) {
      auto cview = [](pe::EpiPoPE& e, const pe_tensor_t* dxc) {
        e.dxc = (void*)dxc->data; e.dxc_dtype = dxc->dtype;
        for (int i = 0; i < 4; ++i) e.dxc_s[i] = dxc->stride[i];
      };
      cview(c.eq, dqc);
      cview(c.ek, dkc);
    }
    c.eq.part_freq = dfreqs ? (float*)(bws + L.pq_off) : nullptr;
    c.ek.part_freq = dfreqs ? (float*)(bws + L.pk_off) : nullptr;
    c.ek.part_delta = ddelta ? (float*)(bws + L.pkd_off) : nullptr;
  }
  // the gradient kernels over head groups whose dS fits the workspace (one group up to the cap);
  // with several groups the dK/dV stage mark spans every group's kernels and the dQ mark is empty
  const int units = p->B * p->Hkv;
  const int group = L.ds_group;
  for (int g0 = 0; g0 < units; g0 += group) {
    c.bh0 = g0;
    c.nbh = std::min(group, units - g0);
    if ((rc = pe::launch_bwd_dkdv(dt, L.dqk, L.dv, c, s))) return rc;
    if (group == units) {
      stage_mark(PE_STAGE_BWD_DKDV, 1, s);
      stage_mark(PE_STAGE_BWD_DQ, 0, s);
    }
    if ((rc = pe::launch_bwd_dq(dt, L.dqk, L.dv, c, s))) return rc;
  }
  if (group != units) {
    stage_mark(PE_STAGE_BWD_DKDV, 1, s);
    stage_mark(PE_STAGE_BWD_DQ, 0, s);
  }
  stage_mark(PE_STAGE_BWD_DQ, 1, s);
  stage_mark(PE_STAGE_BWD_INV, 0, s);

  for (int side = 0; side < 2 && !fuse && !rfuse; ++side) {
    const bool key = side == 1;
    const pe_tensor_t* xr = key ? kr : qr;
    const pe_tensor_t* dxc = key ? dkc : dqc;
    const pe_tensor_t* dxr = key ? dkr : dqr;
    pe::InvArgs ia;
    memset(&ia, 0, sizeof(ia));
    ia.g = (const float*)(bws + (key ? L.dk_off : L.dq_off));
    ia.width = L.dqk;
    if (xr && xr->data) { ia.xr = xr->data; ia.xr_dtype = xr->dtype; for (int i = 0; i < 4; ++i) ia.xr_s[i] = xr->stride[i]; }
    if (dxc && dxc->data) { ia.dxc = (void*)dxc->data; ia.dxc_dtype = dxc->dtype; for (int i = 0; i < 4; ++i) ia.dxc_s[i] = dxc->stride[i]; }
    if (dxr && dxr->data) { ia.dxr = (void*)dxr->data; ia.dxr_dtype = dxr->dtype; for (int i = 0; i < 4; ++i) ia.dxr_s[i] = dxr->stride[i]; }
    ia.B = p->B; ia.H = key ? p->Hkv : p->Hq; ia.S = key ? p->Sk : p->Sq;
    ia.Dc = p->Dc; ia.Dr = p->Dr; ia.mode = p->mode;
    ia.start_pos = key ? p->start_pos_k : p->start_pos_q;
    ia.pos_round = p->position_rounding;
    ia.l2norm = p->qk_l2norm; ia.is_key = key;
    ia.freqs = freqs; ia.delta = key ? delta : nullptr; ia.delta_hs = p->delta_head_stride;
    ia.mscale = p->rope_mscale;
    ia.part_delta = key ? (float*)(bws + L.pkd_off) : nullptr;
    ia.part_freq = (float*)(bws + (key ? L.pk_off : L.pq_off));
    ia.rows_per_block = inv_rows(ia.B, ia.H, ia.S);
    if (ia.Dr == 0 && ia.Dc > 0) ia.mode = PE_MODE_NONE;
    int nb = 0;
    if ((rc = pe::launch_inv(ia, &nb, s))) return rc;
  }
  if (p->mode == PE_MODE_POPE && p->Dr > 0 && (dfreqs || ddelta)) {
    pe::ReduceArgs ra;
    memset(&ra, 0, sizeof(ra));
    ra.part_q_freq = (const float*)(bws + L.pq_off); ra.nq = L.nq_blocks;
    ra.part_k_freq = (const float*)(bws + L.pk_off); ra.part_k_delta = (const float*)(bws + L.pkd_off);
    ra.nk = L.nk_blocks;
    if (fuse) {
      ra.nq = p->B * p->Hq * nqg;
      ra.nk = p->B * p->Hkv * nkg;
      ra.k_blocks_per_head = nkg;
    } else {
      const int kr_rows = inv_rows(p->B, p->Hkv, p->Sk);
      ra.nq = pe::inv_blocks(p->B, p->Hq, p->Sq, inv_rows(p->B, p->Hq, p->Sq));
      ra.nk = pe::inv_blocks(p->B, p->Hkv, p->Sk, kr_rows);
      ra.k_blocks_per_head = (p->Sk + kr_rows - 1) / kr_rows;
    }
    ra.Hkv = p->Hkv; ra.B = p->B; ra.Dr = p->Dr;
    ra.delta_per_head = p->delta_head_stride != 0;
    ra.dfreqs = dfreqs; ra.ddelta = ddelta;
    if ((rc = pe::launch_reduce(ra, s))) return rc;
  }
  stage_mark(PE_STAGE_BWD_INV, 1, s);
  return PE_OK;
}

extern "C" {

int pe_attn_bwd(const pe_attn_params* p, const pe_tensor_t* qc, const pe_tensor_t* qr,
                const pe_tensor_t* kc, const pe_tensor_t* kr, const pe_tensor_t* v,
                const float* freqs, const float* delta, const pe_tensor_t* out, const float* lse,
                const pe_tensor_t* dout, const pe_tensor_t* dqc, const pe_tensor_t* dqr,
                const pe_tensor_t* dkc, const pe_tensor_t* dkr, const pe_tensor_t* dv,
                float* dfreqs, float* ddelta, const void* fwd_workspace, size_t fwd_ws_bytes,
                void* bwd_workspace, size_t bwd_ws_bytes, void* stream) {
  return bwd_impl(p, qc, qr, kc, kr, v, freqs, delta, nullptr, out, lse, dout, dqc, dqr, dkc, dkr, dv, dfreqs,
                  ddelta, fwd_workspace, fwd_ws_bytes, bwd_workspace, bwd_ws_bytes, stream);
}

int pe_attn_bwd_masked(const pe_attn_params* p, const pe_tensor_t* qc, const pe_tensor_t* qr,
                       const pe_tensor_t* kc, const pe_tensor_t* kr, const pe_tensor_t* v,
                       const float* freqs, const float* delta, const pe_tensor_t* mask, const pe_tensor_t* out,
                       const float* lse, const pe_tensor_t* dout, const pe_tensor_t* dqc, const pe_tensor_t* dqr,
                       const pe_tensor_t* dkc, const pe_tensor_t* dkr, const pe_tensor_t* dv,
                       float* dfreqs, float* ddelta, const void* fwd_workspace, size_t fwd_ws_bytes,
                       void* bwd_workspace, size_t bwd_ws_bytes, void* stream) {
  if (!mask) return PE_ERR_NULL;
  return bwd_impl(p, qc, qr, kc, kr, v, freqs, delta, mask, out, lse, dout, dqc, dqr, dkc, dkr, dv, dfreqs,
                  ddelta, fwd_workspace, fwd_ws_bytes, bwd_workspace, bwd_ws_bytes, stream);
}

}  // extern "C"
