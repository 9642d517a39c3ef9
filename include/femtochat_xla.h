/* femtochat_xla.h — callbacks for an XLA typed-FFI custom call on ROCm.
 *
 * The reference reaches its CUDA kernels from compiled (Reactant/XLA) code
 * through a small FFI handler that passes XLA's stream and buffers, inputs
 * first and then outputs, to a callback `bool callback(void* stream, void**
 * buffers)` given as the attribute `callback_ptr`
 * (deps/reactant/xla_ffi.cpp:7-28; buffer order ext/reactant/cuda_call.jl:18-25).
 * There the callback re-enters Julia.  Here it is a native function that
 * runs the MI355X kernels directly on XLA's stream: bind a call site once
 * (its shapes and types are static in the compiled program), and register
 * the same handler for platform "ROCM" with the returned pointer.
 *
 * A bound callback returns false on failure, with the message in
 * fc_xla_last_error().  Bindings live until the process ends (as the
 * reference's registry does); at most 256 can be made.
 */
#ifndef FEMTOCHAT_XLA_H
#define FEMTOCHAT_XLA_H

#include <stdbool.h>
#include <stdint.h>
#include <stddef.h>

#include "femtochat_attn.h"
#include "femtochat_loss.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The callback type of the reference's handler (xla_ffi.cpp:21). */
typedef bool (*fc_xla_callback)(void* stream, void** buffers);

/* Attention forward, the Reactant `Forward` (ext/FemtoChatReactantExt.jl:172-175):
   buffers = (Q, K, V, [positions,] O, l, m).  Null on an invalid descriptor. */
fc_xla_callback fc_xla_bind_attention_fwd(const fc_attn_desc* desc, int32_t has_positions);

/* Attention backward, the Reactant `Backward` with accumulate=false
   (ext/FemtoChatReactantExt.jl:176-185; the gradients are overwritten):
   buffers = (dO, Q, K, V, O, l, m, [positions,] dQ, dK, dV[, workspace]).
   *workspace_bytes receives the size of the trailing workspace buffer the
   call site must declare as an extra output (0: no workspace buffer).  The
   buffer needs no more alignment than XLA gives (64 bytes): the size includes
   255 bytes of slack and the callback works from the buffer's first 256-byte
   boundary, which fc_attn_bwd requires. */
fc_xla_callback fc_xla_bind_attention_bwd(const fc_attn_desc* desc, int32_t has_positions,
                                          size_t* workspace_bytes);

/* Embedding forward, `EmbeddingForward` (ext/FemtoChatReactantExt.jl:238-242):
   buffers = (weights, tokens, y). */
fc_xla_callback fc_xla_bind_embedding_fwd(const fc_embed_desc* desc);

/* Embedding backward, `EmbeddingBackward` (ext/FemtoChatReactantExt.jl:243-246):
   buffers = (dy, weights, tokens, y, dweights); dweights is zeroed, then the
   gradient is scattered into it. */
fc_xla_callback fc_xla_bind_embedding_bwd(const fc_embed_desc* desc);

/* Message of the last failed callback or binding ("" if none). */
const char* fc_xla_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* FEMTOCHAT_XLA_H */
