/* femtochat_loss.h — C ABI of the loss-side kernels in libfemtochat_attn.so
 * (gfx950): cross-entropy over vocabulary columns and its gradient, the
 * embedding gather and its scatter-add gradient.
 *
 * Conventions are those of femtochat_attn.h: every entry point returns an
 * fc_status (message in fc_last_error()), all pointers are device pointers
 * in the reference's column-major layout, launches are asynchronous on the
 * caller's HIP stream, and the library allocates nothing.
 *
 *   logits, dlogits (V, T, B) float32 : x[token*V + v], token = b*T + t
 *   targets, tokens (T, B)             : i[token], int32 or int64, values in
 *                                         [index_base, index_base + V)
 *   weights, dweights (D, vocab) float32: w[id*D + d]
 *   y, dy (D, T, B)                    : y[token*D + d], float32 or bfloat16
 */
#ifndef FEMTOCHAT_LOSS_H
#define FEMTOCHAT_LOSS_H

#include <stddef.h>
#include <stdint.h>

#include "femtochat_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { FC_REDUCE_NONE = 0, FC_REDUCE_SUM = 1, FC_REDUCE_MEAN = 2 } fc_reduction;
typedef enum { FC_INDEX_I32 = 0, FC_INDEX_I64 = 1 } fc_index_type;

typedef struct {
  int32_t V;            /* vocabulary size: length of a logits column */
  int32_t index_base;   /* 1: targets are Julia indices 1..V; 0: 0..V-1 */
  int64_t N;            /* tokens (T*B) */
  int64_t ignore_index; /* target value that means "no target" (the reference's ignore_index, default -1) */
  int32_t index_type;   /* fc_index_type of targets */
  int32_t reduction;    /* fc_reduction */
  uint32_t flags;       /* FC_FLAG_OVERWRITE: the gradient writes dlogits instead of adding */
} fc_xent_desc;

/* Per-token losses max + log(sum(exp(x - max))) - x[target], 0 where the
   target is ignore_index, NaN where it is outside the vocabulary.  Optional
   outputs: lse (N floats, the per-token log-sum-exp, which the gradient can
   reuse), reduced (1 float: the sum, or the mean over valid targets for
   FC_REDUCE_MEAN) and count (1 float: the number of valid targets).
   Replaces `cross_entropy(logits, targets, ignore_index, reduction)`
   (reference src/gpt.jl:175-195; CUDA ext/FemtoChatCUDAExt.jl:44-50). */
fc_status fc_cross_entropy_fwd(const fc_xent_desc* desc, const float* logits, const void* targets,
                               float* losses, float* lse, float* reduced, float* count, void* stream);

/* Number of valid targets (target != ignore_index) into count[0]: the
   `sum(t -> t != ignore, targets)` of the reference's mean gradient
   (ext/FemtoChatCUDAExt.jl:57). */
fc_status fc_cross_entropy_count(const fc_xent_desc* desc, const void* targets, float* count, void* stream);

/* dlogits += scale * (softmax(x) - onehot(target)) for every valid target,
   scale = dy[0] / count[0] (mean), dy[0] (sum) or dy[token] (none); tokens
   with an ignored target are left untouched.  lse may be null (recomputed
   from the logits) or the forward's.  Replaces
   `cross_entropy_gradient!(δ, logits, targets, dy, ignore_index, reduction)`
   (reference src/kernels.jl:16-28; CUDA ext/FemtoChatCUDAExt.jl:56-61). */
fc_status fc_cross_entropy_bwd(const fc_xent_desc* desc, float* dlogits, const float* logits, const void* targets,
                               const float* dy, const float* count, const float* lse, void* stream);

/* Forward and gradient in one pass over the logits, for the loss as the last
   node of the step: the losses (and optionally lse and the reduced value, as
   fc_cross_entropy_fwd) and dlogits += (or, with FC_FLAG_OVERWRITE, =)
   scale * (softmax(x) - onehot(target)) with scale from dy and count as
   fc_cross_entropy_bwd (count from fc_cross_entropy_count for the mean).
   One workgroup holds a token's column in registers: V a multiple of 4 and
   at most 32768, logits and dlogits 16-byte aligned (FC_ERR_UNSUPPORTED
   otherwise).  No reference counterpart as one call: it is the reference's
   cross_entropy then cross_entropy_gradient! (src/gpt.jl:175-195,
   src/kernels.jl:16-28) with the logits read once instead of twice or three times. */
fc_status fc_cross_entropy_fused(const fc_xent_desc* desc, const float* logits, const void* targets, float* losses,
                                 float* lse, float* reduced, float* dlogits, const float* dy, const float* count,
                                 void* stream);

typedef struct {
  int32_t D;          /* embedding width: length of a weight column */
  int32_t vocab;      /* number of weight columns */
  int64_t N;          /* tokens */
  int32_t index_base; /* 1: Julia token indices, 0: zero-based */
  int32_t index_type; /* fc_index_type of tokens */
  int32_t y_dtype;    /* FC_F32 or FC_BF16: element type of y (forward) and dy (backward) */
  uint32_t flags;     /* reserved, 0 */
} fc_embed_desc;

/* y[:, t] = weights[:, tokens[t]] (converted to y_dtype); a token id outside
   the table gives a NaN column.  Replaces `(𝔼::Embedding)(tokens)`
   (reference src/gpt.jl:34, followed by the `F.(x)` conversion of :137;
   CUDA ext/FemtoChatCUDAExt.jl:63-76). */
fc_status fc_embedding_fwd(const fc_embed_desc* desc, const float* weights, const void* tokens, void* y,
                           void* stream);

/* dweights[:, tokens[t]] += dy[:, t] with fp32 atomic adds (repeated tokens
   accumulate; zero values and ids outside the table are skipped).  Replaces
   `embedding_gradient!(δ, dy, tokens)` (reference src/kernels.jl:8-14; CUDA
   ext/FemtoChatCUDAExt.jl:78-94). */
fc_status fc_embedding_bwd(const fc_embed_desc* desc, float* dweights, const void* dy, const void* tokens,
                           void* stream);

/* Bytes of the caller-owned workspace of fc_embedding_bwd_sorted for these
   N and vocab (the sort's keys and token indices and its temporary storage). */
fc_status fc_embedding_bwd_workspace_bytes(const fc_embed_desc* desc, size_t* bytes);

/* The gradient of fc_embedding_bwd, deterministic: the tokens are sorted by
   id (a stable device radix sort), and each id's dy columns are summed in
   token order, skipping zero values, from -0; the sum is then added to
   dweights[:, id] once.  The same inputs give the same bits on every call,
   with no atomics.  workspace: at least fc_embedding_bwd_workspace_bytes,
   256-byte aligned.  The sort (rocPRIM's device radix sort) clears its
   counters with hipMemsetAsync, so this call is not for HIP graph capture
   (fc_embedding_bwd is).  No reference counterpart as one call: the reference's
   embedding_gradient! (src/kernels.jl:8-14; CUDA ext/FemtoChatCUDAExt.jl:78-94)
   adds with atomics in no fixed order. */
fc_status fc_embedding_bwd_sorted(const fc_embed_desc* desc, float* dweights, const void* dy, const void* tokens,
                                  void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FEMTOCHAT_LOSS_H */
