/*
 * pe_attn.h -- C ABI of the MI355X (gfx950) positional-encoding attention library (libpe_attn.so).
 *
 * Fused causal attention, forward and backward, for PoPE / FoPE / RoPE(NTK, YaRN) / no-PE.  The
 * positional transform (softplus magnitude + polar phase, or the interleaved rotation) is applied
 * by the library; callers hand over the raw projections.  Plain C types only: device pointers,
 * sizes, strides, a hipStream_t passed as void*.  The library never allocates, frees or
 * synchronises: the caller owns every output and the workspace, and every call is asynchronous
 * on the given stream.  All functions return 0 or a negative PE_ERR_* code.
 *
 * Which reference interface each entry point replaces (shyampathak22/pe_ablations):
 *   pe_attn_fwd  -- PoPEEmbedding.forward_query/forward_key (src/model/pope.py:124-183) or
 *                   FoPEPoPEEmbedding.forward_query/forward_key (src/model/fpope.py:266-338), the
 *                   content|position concat, GQA repeat_interleave and the causal
 *                   F.scaled_dot_product_attention call of FPoPEGroupedQueryAttention.forward
 *                   (src/model/fpope_attention.py:145-177); for RoPE the apply_rotary_emb +
 *                   QKNorm + SDPA span of GroupedQueryAttention.forward (src/model/attention.py:69-96,
 *                   src/model/rope.py:35-57,209-217); and the removed fused kernel entry
 *                   triton_fpope_attention(q,k,v,freqs,bias,start_pos,return_lse=True)
 *                   (scripts/diagnose_kernel.py:180-188) / fpope_attention_forward
 *                   (tests/test_fpope.py:222-226).
 *   pe_attn_bwd  -- the autograd backward of that span (torch SDPA backward + the eager transform's
 *                   backward), i.e. the removed _fpope_attention_bwd_kernel_{dk,dq,dv} launches and
 *                   their host-side partial reduction (scripts/debug_backward.py:118-197,226-227).
 */
#ifndef PE_ATTN_H
#define PE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PE_ATTN_ABI_VERSION 2

/* positional-encoding mode */
enum {
  PE_MODE_POPE = 0, /* PoPE / FoPE: x -> [mu cos(pos*freq (+delta)), mu sin(...)], mu = softplus  */
  PE_MODE_ROPE = 1, /* RoPE / NTK / YaRN: interleaved pairs rotated by pos*inv_freq, times mscale */
  PE_MODE_NONE = 2  /* no positional transform (reference pe_mode "nope", or fpope=None modules) */
};

/* element types of tensors crossing the boundary.  A compute dtype (pe_attn_params.dtype) of bf16
 * or fp16 runs the matrix products on 16-bit operands with fp32 accumulation (fp16: the reference
 * trainer's mixed_precision fp16, src/training/trainer.py:343-347); fp32 runs them in fp32. */
enum { PE_DTYPE_BF16 = 0, PE_DTYPE_FP32 = 1, PE_DTYPE_FP16 = 2 };
/* element type of an explicit attention mask only: one byte per element, nonzero = the key takes
 * part (torch.bool, SDPA's boolean attn_mask) */
enum { PE_DTYPE_BOOL = 3 };

/* how the PoPE / FoPE phase product sees a position p (pe_attn_params.position_rounding) */
enum {
  PE_POS_EXACT = 0, /* fl(p * freq) with p exact in fp32 (PoPEEmbedding, src/model/pope.py:110-119)  */
  PE_POS_BF16 = 1,  /* p rounded to bf16 first: FoPE's arange(..., dtype=x.dtype) for bf16 x
                       (src/model/fpope.py:285,322) */
  PE_POS_FP16 = 2   /* p rounded to fp16 first (the same under fp16 autocast; inf beyond 65519) */
};

/* causal masking: key s visible to query t iff s <= t + off */
enum {
  PE_CAUSAL_NONE = 0,
  PE_CAUSAL_TOP_LEFT = 1,    /* off = 0: SDPA is_causal (src/model/fpope_attention.py:171-177) */
  PE_CAUSAL_BOTTOM_RIGHT = 2 /* off = Sk - Sq: KV-cache mask (src/model/fpope_attention.py:313-317) */
};

/* error codes */
enum {
  PE_OK = 0,
  PE_ERR_NULL = -1,          /* required pointer is NULL */
  PE_ERR_SHAPE = -2,         /* non-positive size, Hq % Hkv != 0, Sq != Sk for top-left causal, ... */
  PE_ERR_HEAD_DIM = -3,      /* transformed q/k width or value width outside what the kernels tile */
  PE_ERR_MODE = -4,          /* unknown mode / dtype / causal value, odd RoPE width */
  PE_ERR_STRIDE = -5,        /* last-dim stride != 1 or misaligned base pointer */
  PE_ERR_WORKSPACE = -6,     /* workspace NULL or smaller than pe_attn_*_workspace_bytes */
  PE_ERR_LAUNCH = -7,        /* a kernel launch failed (hipGetLastError) */
  PE_ERR_NO_DEVICE = -8,     /* no gfx950 device is current */
  PE_ERR_SCRATCH_LIMIT = -9  /* pe_attn_fwd_noalloc: workspace need exceeds the static scratch */
};

/* A (B, H, S, D) tensor view: device pointer, element type, element strides in (B, H, S, D)
 * order.  stride[3] must be 1. */
typedef struct {
  const void* data;
  int32_t dtype;
  int32_t reserved;
  int64_t stride[4];
} pe_tensor_t;

typedef struct {
  int32_t B, Hq, Hkv, Sq, Sk;
  int32_t Dc;     /* content (pass-through) dims ahead of the positional part; 0 in the fused form   */
  int32_t Dr;     /* positional dims before the transform (PoPE adds 2*Dr to the QK width, RoPE Dr) */
  int32_t Dv;     /* value / output head width                                                       */
  int32_t mode;   /* PE_MODE_*                                                                       */
  int32_t dtype;  /* compute dtype of the transformed operands, the output and dV: PE_DTYPE_*       */
  int32_t causal; /* PE_CAUSAL_*                                                                     */
  int32_t start_pos_q, start_pos_k; /* absolute position of row 0 (phases only)                      */
  int32_t qk_l2norm;                /* QKNorm x / (||x|| + 1e-6) after the transform (RoPE / NONE)   */
  float scale;                      /* softmax scale applied to q~ . k~                              */
  float rope_mscale;                /* YaRN mscale multiplying rotated q and k (1 otherwise)         */
  int64_t delta_head_stride;        /* PoPE key phase bias: 0 = (Dr,) shared, else per kv head     */
  int32_t position_rounding;        /* PE_POS_* (PoPE mode only; 0 = exact positions)              */
  int32_t reserved;                 /* 0                                                           */
} pe_attn_params;

/* Host-only validation of a parameter block (no device work). */
int pe_attn_check(const pe_attn_params* p);

/* Bytes of caller-provided device workspace each pass needs (0 on invalid params).  The forward
 * workspace holds the transformed operands; pass the SAME, unmodified forward workspace to
 * pe_attn_bwd.
 *
 * The bf16 backward stores the score gradient dS of the causal triangle (2 bytes per visible
 * (query, key) pair, about Sq * Sk bytes per query head) for its dQ pass.  Its share of the backward
 * workspace is capped at PE_BWD_DS_CAP_BYTES: the backward runs its two gradient kernels over
 * groups of (batch, kv head) units, each with its query heads, whose dS fits the cap, reusing one
 * buffer (one group, the whole problem, up to the cap; at H = 16, D = 128 that is S = 16384).  A
 * single kv head whose query heads' dS alone exceeds the cap (Sq = Sk beyond about 68k with one query
 * head per kv head) still gets its whole dS; the reported size then exceeds the cap by that much. */
#define PE_BWD_DS_CAP_BYTES ((size_t)4608 << 20) /* 4.5 GiB */
size_t pe_attn_fwd_workspace_bytes(const pe_attn_params* p);
size_t pe_attn_bwd_workspace_bytes(const pe_attn_params* p);

/* Forward.  qc/kc: content parts (data may be NULL when Dc == 0); qr/kr: positional parts
 * (B,Hq|Hkv,S,Dr); v (B,Hkv,Sk,Dv).  freqs: PoPE/FoPE per-dim frequency (Dr,) or RoPE inverse
 * frequency (Dr/2,), fp32; delta: PoPE key phase bias as used (already clamped by the caller),
 * NULL for none.  out (B,Hq,Sq,Dv) in p->dtype, written through its strides; lse (B,Hq,Sq) fp32
 * natural-log logsumexp of the scaled scores (-inf for a row with no visible key). */
int pe_attn_fwd(const pe_attn_params* p,
                const pe_tensor_t* qc, const pe_tensor_t* qr,
                const pe_tensor_t* kc, const pe_tensor_t* kr,
                const pe_tensor_t* v,
                const float* freqs, const float* delta,
                const pe_tensor_t* out, float* lse,
                void* fwd_workspace, size_t fwd_ws_bytes, void* stream);

/* Backward.  Inputs as for pe_attn_fwd plus out/lse from it and dout (B,Hq,Sq,Dv).  Gradients are
 * written through the tensor views dqc/dqr/dkc/dkr (same shapes and dtypes as the inputs;
 * dqc/dkc data may be NULL when Dc == 0) and dv (dtype p->dtype).  dfreqs (Dr,) and ddelta
 * (Dr,) or (Hkv, Dr) are fp32 and overwritten; either may be NULL to skip it.  With a 16-bit
 * p->dtype, qc/qr/kc/kr/v and the gradients are each fp32 or p->dtype (the other 16-bit type:
 * PE_ERR_MODE). */
int pe_attn_bwd(const pe_attn_params* p,
                const pe_tensor_t* qc, const pe_tensor_t* qr,
                const pe_tensor_t* kc, const pe_tensor_t* kr,
                const pe_tensor_t* v,
                const float* freqs, const float* delta,
                const pe_tensor_t* out, const float* lse, const pe_tensor_t* dout,
                const pe_tensor_t* dqc, const pe_tensor_t* dqr,
                const pe_tensor_t* dkc, const pe_tensor_t* dkr,
                const pe_tensor_t* dv,
                float* dfreqs, float* ddelta,
                const void* fwd_workspace, size_t fwd_ws_bytes,
                void* bwd_workspace, size_t bwd_ws_bytes, void* stream);

/* Explicit attention masks: F.scaled_dot_product_attention(q, k, v, attn_mask=mask) of
 * GroupedQueryAttention.forward (src/model/attention.py:91-96), which the reference module calls with
 * is_causal=False when a mask is given (pass PE_CAUSAL_NONE to match; a causal value applies both).
 * mask is a (B, Hq, Sq, Sk) view, indexed by the query head: PE_DTYPE_BOOL (nonzero = attend) or a
 * float type whose value is added to the scaled score; element strides may be 0 where it broadcasts
 * (torch's expand) and must not be negative.  A row whose every key is masked gives out = 0, lse =
 * -inf and zero gradients, as torch's SDPA does.  Float values below -FLT_MAX / log2(e) count as
 * -inf.  With a 16-bit compute type the forward runs the tuned kernel's mask instantiation, and at
 * transformed widths 128 / 256 with value widths 64 / 128 so does the backward (the dK/dV pair
 * kernel and the dQ GEMM over its stored dS, capped as in pe_attn_bwd); fp32 and the other widths
 * run the generic kernels, which store no dS.  The backward's workspace is
 * pe_attn_bwd_masked_workspace_bytes, the forward's pe_attn_fwd_workspace_bytes.  Arguments
 * otherwise as pe_attn_fwd / pe_attn_bwd; the mask has no gradient. */
size_t pe_attn_bwd_masked_workspace_bytes(const pe_attn_params* p);
int pe_attn_fwd_masked(const pe_attn_params* p,
                       const pe_tensor_t* qc, const pe_tensor_t* qr,
                       const pe_tensor_t* kc, const pe_tensor_t* kr,
                       const pe_tensor_t* v,
                       const float* freqs, const float* delta,
                       const pe_tensor_t* mask,
                       const pe_tensor_t* out, float* lse,
                       void* fwd_workspace, size_t fwd_ws_bytes, void* stream);
int pe_attn_bwd_masked(const pe_attn_params* p,
                       const pe_tensor_t* qc, const pe_tensor_t* qr,
                       const pe_tensor_t* kc, const pe_tensor_t* kr,
                       const pe_tensor_t* v,
                       const float* freqs, const float* delta,
                       const pe_tensor_t* mask,
                       const pe_tensor_t* out, const float* lse, const pe_tensor_t* dout,
                       const pe_tensor_t* dqc, const pe_tensor_t* dqr,
                       const pe_tensor_t* dkc, const pe_tensor_t* dkr,
                       const pe_tensor_t* dv,
                       float* dfreqs, float* ddelta,
                       const void* fwd_workspace, size_t fwd_ws_bytes,
                       void* bwd_workspace, size_t bwd_ws_bytes, void* stream);

/* RMSNorm weights of the position projections (qr_norm / kr_norm of FPoPEGroupedQueryAttention,
 * src/model/fpope_attention.py:88-90,132-137; RMSNorm, src/model/normalization.py:7-27). */
typedef struct {
  const void* q_weight;  /* (Hq * Dr,) */
  const void* k_weight;  /* (Hkv * Dr,) */
  int32_t weight_dtype;  /* PE_DTYPE_* of both */
  float eps;             /* RMSNorm eps (the module default is 1e-6) */
} pe_norm_params;

/* Forward that allocates nothing: pe_attn_fwd with the workspace taken from a static device array
 * of PE_NOALLOC_SCRATCH_BYTES held by the library on each GPU from the load of its code object
 * (under the HIP runtime's default deferred loading: the first call of this entry on that GPU) to
 * process exit).  No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Calls whose
 * forward workspace (pe_attn_fwd_workspace_bytes) exceeds the scratch return PE_ERR_SCRATCH_LIMIT.
 * All calls on one GPU share its scratch: calls that overlap in time on one GPU (different streams
 * or threads) race and must be serialised by the caller.  Outputs are as for pe_attn_fwd; the
 * scratch cannot serve pe_attn_bwd (use pe_attn_fwd with a caller workspace for training). */
#define PE_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)
size_t pe_attn_noalloc_scratch_bytes(void);
int pe_attn_fwd_noalloc(const pe_attn_params* p,
                        const pe_tensor_t* qc, const pe_tensor_t* qr,
                        const pe_tensor_t* kc, const pe_tensor_t* kr,
                        const pe_tensor_t* v,
                        const float* freqs, const float* delta,
                        const pe_tensor_t* out, float* lse, void* stream);

/* Forward with the RMSNorm of the raw position projections fused into the PoPE prologue: qr / kr
 * are wq_r(x) / wk_r(x) as (B,H,S,Dr) views of (B,S,H*Dr) rows, and each token's H*Dr features are
 * normalised together, y = (x * rsqrt(mean(x^2) + eps)).type_as(x) * weight, before the transform
 * (one kernel per side instead of the module's eager norm plus the prologue).  Replaces the
 * qr_norm / kr_norm calls of src/model/fpope_attention.py:132-137 together with everything
 * pe_attn_fwd replaces.  PoPE / FoPE mode only; H*Dr <= 8192, Dr % 8 == 0, 16-byte aligned rows.
 * Forward only: the workspace holds operands of the normalised projections, so training calls
 * apply the norm themselves and use pe_attn_fwd / pe_attn_bwd. */
int pe_attn_fwd_normed(const pe_attn_params* p, const pe_norm_params* n,
                       const pe_tensor_t* qc, const pe_tensor_t* qr,
                       const pe_tensor_t* kc, const pe_tensor_t* kr,
                       const pe_tensor_t* v,
                       const float* freqs, const float* delta,
                       const pe_tensor_t* out, float* lse,
                       void* fwd_workspace, size_t fwd_ws_bytes, void* stream);

/* KV-cache decode: the cache path of FPoPEGroupedQueryAttentionWithCache.forward
 * (src/model/fpope_attention.py:226-327).  The reference caches the transformed keys
 * [k_c | PoPE(k_r)] and the values (:283-299) and attends to the first cache_len rows with SDPA under
 * a bottom-right causal mask (:301-324).  Here the caches are caller-owned device buffers:
 *   k_cache (B, Hkv, capacity, pe_attn_operand_width(p)) in p->dtype: the library's operand rows
 *           [content | transform | zero pad], whose first Dc + 2*Dr (PoPE) columns are the
 *           reference's cached key layout;
 *   v_cache (B, Hkv, capacity, pe_attn_value_width(p)) in p->dtype, zero-padded.
 *
 * pe_attn_cache_append: transforms p->Sk new key rows (kc / kr / v views (B, Hkv, Sk, *), phases at
 * positions start_pos_k + s, key phase bias delta) and writes them, with their values, to cache rows
 * start_pos_k .. start_pos_k + Sk - 1 (the reference's k_cache[:, :, start_pos:start_pos+S] = k_new,
 * :294-296).  start_pos_k + Sk must not exceed capacity.
 *
 * pe_attn_decode: p->Sq new query rows (qc / qr views (B, Hq, Sq, *), phases at start_pos_q + t)
 * attend to the first p->Sk cached rows (Sk = the reference's cache_len, new rows included);
 * p->causal BOTTOM_RIGHT gives the reference's mask, key s visible to query t iff
 * s <= t + Sk - Sq.  out (B, Hq, Sq, Dv) and lse (B, Hq, Sq) as for pe_attn_fwd.  The work is split
 * over key ranges whose partial results are merged in a fixed order (bitwise reproducible); the
 * workspace holds the transformed queries and the partials.  Forward only. */
int pe_attn_value_width(const pe_attn_params* p);
int pe_attn_cache_append(const pe_attn_params* p,
                         const pe_tensor_t* kc, const pe_tensor_t* kr, const pe_tensor_t* v,
                         const float* freqs, const float* delta,
                         void* k_cache, void* v_cache, int32_t capacity, void* stream);
size_t pe_attn_decode_workspace_bytes(const pe_attn_params* p);
int pe_attn_decode(const pe_attn_params* p,
                   const pe_tensor_t* qc, const pe_tensor_t* qr,
                   const void* k_cache, const void* v_cache, int32_t capacity,
                   const float* freqs, const pe_tensor_t* out, float* lse,
                   void* workspace, size_t ws_bytes, void* stream);

/* RMSNorm forward over the last dim of a (rows, n) view with unit element stride
 * (src/model/normalization.py:7-27, the module on hidden states and on the position
 * projections): y = (x * rsqrt(mean(x^2) + eps)).type_as(x) * weight, in fp32; y_dtype must be
 * bf16 when x and weight are both bf16 and fp32 otherwise (torch's type promotion).  n % 8 == 0,
 * n <= 8192, 16-byte aligned base pointers, row strides multiples of 16 bytes. */
int pe_rmsnorm_fwd(const void* x, int32_t x_dtype, int64_t x_row_stride, int64_t rows, int32_t n,
                   const void* weight, int32_t weight_dtype, float eps,
                   void* y, int32_t y_dtype, int64_t y_row_stride, void* stream);

/* RMSNorm backward for pe_rmsnorm_fwd's expression, as autograd differentiates it in fp32
 * (src/model/normalization.py:22-27): from dy (y's dtype: bf16 exactly when x and weight are both
 * bf16) writes dx (x's dtype) and the weight gradient dw (weight's dtype, summed over the rows in a
 * fixed order, bitwise reproducible).  Same shape and alignment rules as pe_rmsnorm_fwd; the
 * workspace (pe_rmsnorm_bwd_workspace_bytes) holds per-workgroup partial sums of dw.  The training
 * path of the fused position-projection norm (pe_attn_fwd_normed) runs it after pe_attn_bwd, which
 * no reference interface exposes as one call: it replaces the autograd of RMSNorm.forward. */
size_t pe_rmsnorm_bwd_workspace_bytes(int64_t rows, int32_t n);
int pe_rmsnorm_bwd(const void* x, int32_t x_dtype, int64_t x_row_stride, int64_t rows, int32_t n,
                   const void* weight, int32_t weight_dtype, float eps,
                   const void* dy, int64_t dy_row_stride, void* dx, int64_t dx_row_stride, void* dw,
                   void* workspace, size_t ws_bytes, void* stream);

/* SwiGLU forward of the feed-forward block (src/model/ffn.py:17-27, SwiGLU.forward(x, gate) =
 * F.silu(gate) * x): out = bf16(bf16(gate / (1 + exp(-gate))) * x) element by element over n
 * contiguous bf16 values, bitwise what torch computes for the two bf16 ops.  n % 8 == 0, 16-byte
 * aligned pointers (out may alias x or gate).  Forward only: the module calls it when no gradient
 * is needed. */
int pe_swiglu_fwd(const void* x, const void* gate, void* out, int64_t n, void* stream);

/* Elementwise positional prologue on its own (the HBM-bound half of the forward): writes the
 * transformed rows [content | transform | zero pad] of x into dst (B,H,S,width) contiguous in
 * p->dtype, width = pe_attn_operand_width(p).  is_key selects the key phase bias.  Replaces
 * forward_query / forward_key (src/model/pope.py:124-183) as a standalone op. */
int pe_attn_transform(const pe_attn_params* p, int is_key,
                      const pe_tensor_t* xc, const pe_tensor_t* xr,
                      const float* freqs, const float* delta,
                      void* dst, void* stream);
int pe_attn_operand_width(const pe_attn_params* p);

/* Backward of pe_attn_transform (the autograd of forward_query / forward_key,
 * src/model/pope.py:124-183, src/model/fpope.py:266-338).  g: gradient of the transformed rows,
 * fp32 (B,H,S,width) contiguous (width = pe_attn_operand_width).  Writes dxc (data may be NULL
 * when Dc == 0) and dxr through their views; for PoPE also dfreqs (Dr,) and, for keys, ddelta
 * ((Dr,) shared or (H,Dr) per head), fp32, overwritten, either may be NULL.  The workspace holds
 * the per-block partial sums behind the deterministic reduction. */
size_t pe_attn_transform_bwd_workspace_bytes(const pe_attn_params* p, int is_key);
int pe_attn_transform_bwd(const pe_attn_params* p, int is_key, const float* g,
                          const pe_tensor_t* xr, const float* freqs, const float* delta,
                          const pe_tensor_t* dxc, const pe_tensor_t* dxr,
                          float* dfreqs, float* ddelta,
                          void* workspace, size_t ws_bytes, void* stream);

const char* pe_attn_strerror(int code);
int pe_attn_version(void);

/* Kernel stages of pe_attn_fwd / pe_attn_bwd that can be bracketed by caller-owned HIP events. */
enum {
  PE_STAGE_FWD_PREP = 0, /* q/k (and v repack) positional transform kernels     */
  PE_STAGE_FWD_CORE = 1, /* attention forward kernel                             */
  PE_STAGE_BWD_PRE = 2,  /* dO repack + Di = rowsum(dO o O)                      */
  PE_STAGE_BWD_DKDV = 3, /* dK~/dV kernel (owns key blocks)                      */
  PE_STAGE_BWD_DQ = 4,   /* dQ~ kernel (owns query blocks)                       */
  PE_STAGE_BWD_INV = 5,  /* inverse transform + phase-bias / frequency reduction */
  PE_STAGE_COUNT = 6
};

/* Profiling hook (no counterpart in the reference, whose harnesses time whole calls with
 * torch.cuda.synchronize + perf_counter, scripts/benchmark_fpope_vs_rope.py:67-78).  Sets, for the
 * whole process (autograd runs backward passes on its own thread), an array of 2*PE_STAGE_COUNT
 * hipEvent_t handles: events[2*i] is recorded on the call's stream right before stage i's first
 * kernel and events[2*i+1] right after its last.  NULL entries are skipped; pass NULL to switch
 * the hook off.  The array must stay valid until the hook is switched off or replaced.  Meant for
 * a single-threaded benchmark: concurrent calls would record into the same events. */
int pe_attn_set_stage_events(void* const* events);

#ifdef __cplusplus
}
#endif

#endif /* PE_ATTN_H */
