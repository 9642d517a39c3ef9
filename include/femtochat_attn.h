/*
 * femtochat_attn.h — C ABI of the MI355X (gfx950) flash-attention library
 * libfemtochat_attn.so.
 *
 * The library is the device backend for femtochat's attention plug-in API
 * (`Kernels.attention / attention! / Δattention! / attention_state`,
 * reference src/kernels.jl:417-433).  A host binding (the Python module
 * femtochat_amd.kernels, or a Julia `ccall` extension) owns every buffer and
 * passes raw device pointers; the library validates the descriptor on the
 * host, then launches its HIP kernels asynchronously on the caller's stream.
 *
 * Tensor layout is the reference's column-major layout, written here as C
 * row-major index expressions (0-based):
 *   Q, O, dO, dQ  (D,H,T,B)   : X[((b*T + t)*H   + h)*D + d]
 *   K, V, dK, dV  (D,Hkv,T,B) : X[((b*T + t)*Hkv + h)*D + d]
 *   l, m          (1,T,H,B)   : x[(b*H + h)*T + t]            (float32)
 *   positions     (T,B) Int32 : p[b*T + t]
 *
 * Semantics (reference src/kernels.jl:30-42, 131-219, 287-379):
 *   key k is visible to query q iff  q-left <= k <= q+right, and k <= q when
 *   (left,right) == (-1,0) (the causal sentinel).  With positions, a key must
 *   also satisfy k >= q - positions[q] (it lies in the query's document).
 *   m = max over visible keys of S/sqrt(D) (natural-log units);
 *   l = sum over visible keys of exp(S/sqrt(D) - m);  O = sum P V.
 *   A query with no visible key gets O = 0, l = 0, m = -FLT_MAX.
 *   GQA: query head h (0-based) reads KV head h / (H/Hkv).
 *   The backward ADDS into dQ/dK/dV unless FC_FLAG_OVERWRITE is set
 *   (reference src/kernels.jl:358,371,374; ext/FemtoChatCUDAExt.jl:1756-1760).
 *
 * Errors: every entry point returns an fc_status; nothing is thrown across
 * the ABI.  fc_last_error() gives the calling thread's last message.
 * Threading: reentrant; launches are asynchronous on the given stream; no
 * entry point synchronises the device or allocates device memory.
 */
#ifndef FEMTOCHAT_ATTN_H
#define FEMTOCHAT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FC_ATTN_ABI_VERSION 1

typedef enum {
  FC_OK = 0,
  FC_ERR_INVALID_ARGUMENT = 1, /* bad shape, window, dtype, null pointer */
  FC_ERR_UNSUPPORTED = 2,      /* valid but not implemented (e.g. head_dim) */
  FC_ERR_WORKSPACE = 3,        /* workspace missing or too small */
  FC_ERR_HIP = 4               /* a HIP runtime call failed */
} fc_status;

typedef enum { FC_F32 = 0, FC_BF16 = 1 } fc_dtype;

typedef enum {
  /* fp32 in, fp32 MFMA, fp32 out (analogue of SIMTInstruction,
     reference ext/FemtoChatCUDAExt.jl:243-1002) */
  FC_MODE_EXACT = 0,
  /* bf16 Q/K/V/dO, bf16 MFMA with fp32 accumulation and statistics; P and dS
     rounded to bf16 before their second product (analogue of
     TensorCoreInstruction, reference ext/FemtoChatCUDAExt.jl:1004-2068) */
  FC_MODE_FAST = 1
} fc_mode;

/* fc_attn_desc.flags */
#define FC_FLAG_OVERWRITE 1u /* backward writes dQ/dK/dV instead of adding */

typedef struct {
  int32_t D, H, Hkv, T, B;      /* head_dim, query heads, KV heads, tokens, batch */
  int32_t win_left, win_right;  /* window (left,right); (-1,0) = causal */
  int32_t mode;                 /* fc_mode */
  int32_t in_dtype;             /* Q, K, V  (EXACT: F32; FAST: BF16) */
  int32_t out_dtype;            /* O        (EXACT: F32; FAST: BF16 or F32) */
  int32_t dout_dtype;           /* dO       (EXACT: F32; FAST: BF16 or F32) */
  int32_t grad_dtype;           /* dQ,dK,dV (EXACT: F32; FAST: BF16 or F32) */
  uint32_t flags;               /* FC_FLAG_* */
} fc_attn_desc;

typedef enum { FC_PASS_FORWARD = 0, FC_PASS_BACKWARD = 1 } fc_pass;

/* Workspace bytes the given pass needs (0 is possible).  positions_given
   selects the document-mask variant.  Mirrors the scratch the reference
   allocates per call (ext/FemtoChatCUDAExt.jl:1797-1801), here caller-owned. */
fc_status fc_attn_workspace_bytes(const fc_attn_desc* desc, int32_t pass,
                                  int32_t positions_given, size_t* bytes);

/* Forward: writes O, l, m.  Replaces
   `attention!(𝒜, O, ℓ, m, Q, K, V, window)` (reference src/kernels.jl:419,
   CPU body :131-219; CUDA ext/FemtoChatCUDAExt.jl:1242-1260).
   positions may be NULL (reference semantics, no document mask).
   The workspace is optional (NULL and 0 are accepted) for head_dim 16, 32,
   64 and 128: in fast mode with positions, a workspace of
   fc_attn_workspace_bytes(FC_PASS_FORWARD) bytes, 256-byte aligned, lets the
   kernel take the query tiles in order of decreasing work (long documents
   first); the results are the same.  Every other head_dim (48, 80, 96, 112)
   runs on copies zero-padded to the next of those widths held in the
   workspace, which is then required (FC_ERR_WORKSPACE without it). */
fc_status fc_attn_fwd(const fc_attn_desc* desc, const void* Q, const void* K,
                      const void* V, const int32_t* positions, void* O,
                      float* l, float* m, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Backward: adds (or, with FC_FLAG_OVERWRITE, writes) dQ, dK, dV.  Replaces
   `Δattention!(𝒜, dQ, dK, dV, dO, Q, K, V, O, ℓ, m, window)` (reference
   src/kernels.jl:420, CPU body :287-379; CUDA ext/FemtoChatCUDAExt.jl:1771-1790). */
fc_status fc_attn_bwd(const fc_attn_desc* desc, const void* dO, const void* Q,
                      const void* K, const void* V, const void* O,
                      const float* l, const float* m, const int32_t* positions,
                      void* dQ, void* dK, void* dV, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Backward without a workspace argument and without any allocation: the same
   kernels and results as fc_attn_bwd, with the workspace taken from a scratch
   array of FC_ATTN_NOALLOC_SCRATCH_BYTES that the library holds on each GPU
   it runs on until the process ends.  No counterpart in the reference: it is
   for callers that cannot allocate device memory (code under HIP graph
   capture, serving loops, harnesses that forbid hipMalloc).  A problem whose
   fc_attn_workspace_bytes(FC_PASS_BACKWARD) exceeds the limit gets
   FC_ERR_WORKSPACE.  Every call on one GPU shares that GPU's array: calls
   that overlap on one GPU (different streams, or threads without ordering)
   race; calls on one stream are ordered and safe.  The current device must
   be the stream's device. */
#define FC_ATTN_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
fc_status fc_attn_bwd_noalloc(const fc_attn_desc* desc, const void* dO,
                              const void* Q, const void* K, const void* V,
                              const void* O, const float* l, const float* m,
                              const int32_t* positions, void* dQ, void* dK,
                              void* dV, void* stream);

/* ---- Attention prologue ---------------------------------------------------
 * Rotary embedding followed by the RMS norm over the head dimension scaled by
 * 1.2, applied to Q or K as CausalSelfAttention does before calling
 * attention (reference src/gpt.jl:101-106: apply_rotary_embedding :53-77,
 * norm :15-20; tables from rotary_embeddings, src/parameters.jl:409-427),
 * writing the result in the attention kernels' layout.
 *   X, Y, dY, dX  (D,NH,T,B) : X[((b*T + t)*NH + h)*D + d]   (NH = n_head for
 *                                                             Q, n_kv_head for K)
 *   sin, cos      (D/2,L)    : s[p*(D/2) + j]  float32, column p = position p
 *   positions     (T,B)      : p[b*T + t], or NULL for position t (the
 *                              reference's rotary_factors, src/gpt.jl:43-49)
 * With d = D/2, c = cos[pos], s = sin[pos]:
 *   u[j] = x[j] c[j] + x[j+d] s[j],  u[j+d] = -x[j] s[j] + x[j+d] c[j],
 *   Y = u / sqrt(sum(u^2)/D + eps) * 1.2,  eps = eps(eltype) (2^-7 bf16, 2^-23 f32),
 * rounded after every operation in bf16 as Julia's BFloat16 arithmetic is.
 * A position outside [0, L) yields NaN for that vector (an index error in
 * the reference).  X and the tables must be 16-byte aligned. */
typedef struct {
  int32_t D, NH, T, B;  /* head_dim, heads of this tensor, tokens, batch */
  int32_t table_len;    /* L: columns of the sin/cos tables */
  int32_t dtype;        /* FC_F32 or FC_BF16: element type of X, Y, dY, dX */
  uint32_t flags;       /* FC_FLAG_OVERWRITE: the backward writes dX instead of adding */
} fc_rope_norm_desc;

/* Forward of the prologue: Y from X.  Replaces the four lines
   `Q = apply_rotary_embedding(Q, rope_cos, rope_sin); ...; Q = eltype(Q).(norm(Q) .* 1.2f0)`
   (reference src/gpt.jl:103-106) for one tensor. */
fc_status fc_rope_norm_fwd(const fc_rope_norm_desc* desc, const void* X,
                           const float* sin_table, const float* cos_table,
                           const int32_t* positions, void* Y, void* stream);

/* Backward of the prologue: adds (or, with FC_FLAG_OVERWRITE, writes) dX =
   (dY/dX)^T dY, recomputing the rotation and the norm from X; the gradient
   of the exact function in fp32 at the rounded rotation.  Replaces the
   reverse pass the reference gets from Enzyme through those lines
   (ext/FemtoChatEnzymeExt.jl differentiates the model around the attention
   rule). */
fc_status fc_rope_norm_bwd(const fc_rope_norm_desc* desc, const void* dY,
                           const void* X, const float* sin_table,
                           const float* cos_table, const int32_t* positions,
                           void* dX, void* stream);

/* ---- Conversions the host binding needs ----------------------------------
 * dst[i] = src[i] for 0 <= i < n, converted: float32 -> bfloat16 rounds to
 * nearest even (NaN stays NaN, +-Inf stays +-Inf), bfloat16 -> float32 is
 * exact, equal dtypes copy.  Replaces the conversion attention_inputs makes
 * for the tensor-core path (reference ext/FemtoChatCUDAExt.jl:229-230, there
 * to Float16) and the Float32.(x) of a bf16 result, so a binding converts
 * without GPU code of its own.  Pointers must be aligned to their element
 * size; the source and destination must not overlap, except that equal
 * pointers with equal dtypes (an in-place copy) are allowed: any other
 * overlap, including src == dst with different dtypes, returns
 * FC_ERR_INVALID_ARGUMENT. */
fc_status fc_convert(const void* src, int32_t src_dtype, void* dst,
                     int32_t dst_dtype, int64_t n, void* stream);

/* bytes bytes of dst set to zero by a kernel (not a memset, so a captured
   graph replays it correctly).  Replaces zero(x) / fill!(x, 0) of a device
   buffer (the reference's zeroed gradients, ext/FemtoChatEnzymeExt.jl). */
fc_status fc_fill_zero(void* dst, size_t bytes, void* stream);

/* Last error message of the calling thread ("" if none). */
const char* fc_last_error(void);

/* Device introspection, the analogue of `capabilities()`
   (reference ext/FemtoChatCUDAExt.jl:177-208). */
typedef struct {
  char name[64];
  char arch[32];            /* e.g. "gfx950" */
  int32_t compute_units;
  int32_t wavefront_size;
  int32_t lds_bytes_per_block;
  int32_t max_threads_per_block;
  int32_t clock_khz;
  int64_t global_mem_bytes;
} fc_caps;
fc_status fc_capabilities(int32_t device, fc_caps* caps);

/* Supported head dims are reported as a bitmask: bit (D/16 - 1) set when
   head_dim D is supported (every multiple of 16 up to 128, as the
   reference's tensor-core path accepts, ext/FemtoChatCUDAExt.jl:214-223;
   the kernels are compiled for 16, 32, 64 and 128 and the other widths run
   zero-padded to the next of them). */
uint32_t fc_attn_supported_head_dims(void);

int32_t fc_abi_version(void);

/* Kernel timing for measurement harnesses.  While enabled, every kernel the
   library launches is bracketed by HIP events on its stream (no host sync).
   fc_profile_collect synchronises on those events and returns, per kernel
   name, the launch count and total milliseconds; it then clears the records.
   No counterpart in the reference (its driver times whole steps,
   scripts/train.jl:136-175). */
typedef struct {
  char kernel[48];
  int32_t launches;
  double total_ms;
} fc_kernel_time;
fc_status fc_profile_enable(int32_t enable);
fc_status fc_profile_collect(fc_kernel_time* out, int32_t capacity,
                             int32_t* count);

#ifdef __cplusplus
}
#endif

#endif /* FEMTOCHAT_ATTN_H */
