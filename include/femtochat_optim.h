/* femtochat_optim.h — C ABI of the optimizer kernels in libfemtochat_attn.so
 * (gfx950): the AdamW step, the CUDA backend's final Adam and Muon writes,
 * the parameter gather/scatter between flat storage and stacked matrices,
 * and Polar Express (Muon's orthogonalisation) over a stack of matrices.
 *
 * Conventions are those of femtochat_attn.h (fc_status returns, device
 * pointers, asynchronous on the caller's stream, no allocation on the hot
 * path).  Matrices are the reference's column-major arrays; every
 * elementwise update follows the reference's operation order in fp32 without
 * fused multiply-adds, as Julia evaluates it.
 */
#ifndef FEMTOCHAT_OPTIM_H
#define FEMTOCHAT_OPTIM_H

#include <stddef.h>
#include <stdint.h>

#include "femtochat_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
  int64_t n;         /* elements of theta, grad, m, v */
  int32_t t;         /* step count after this step's increment (1 for the first step) */
  float alpha;       /* learning rate */
  float beta1, beta2;
  float eps;
  float lambda;      /* decoupled weight decay */
  float grad_scale;  /* N_t: the gradient is divided by it (1 for none) */
} fc_adamw_desc;

/* One AdamW step on float32 arrays: the moments (adam_moments!, reference
   src/optim.jl:32-38), the decay theta *= 1 - alpha lambda and the
   bias-corrected update (:82-94), in one pass.  The bias corrections
   1 - beta^t are formed on the host as Julia's Float32 power does. */
fc_status fc_adamw_step(const fc_adamw_desc* desc, float* theta, const float* grad, float* m, float* v,
                        void* stream);

/* The CUDA backend's final Adam write (ext/FemtoChatCUDAExt.jl:99-106):
   Theta[offset+i] = Theta[offset+i] (1 - eta lambda) - alpha m[i] / (sqrt(v[i] / beta) + eps)
   for i < n, with alpha (bias-corrected rate), beta (second-moment
   correction) and eta (uncorrected rate) as 1-element device arrays. */
fc_status fc_adam_update(int64_t n, int64_t offset, float lambda, float eps, float* Theta, const float* m,
                         const float* v, const float* alpha, const float* beta, const float* eta, void* stream);

/* Muon's final write (ext/FemtoChatCUDAExt.jl:108-119, src/optim.jl:238-247)
   for count matrices of width elements stacked in X:
   Theta[offsets[k]+i] -= eta x + eta lambda Theta[..] [x Theta[..] >= 0],
   x = X[k*width + i]; eta and lambda are 1-element device arrays, offsets
   int64 device array (zero-based element offsets into Theta). */
fc_status fc_muon_update(int64_t width, int32_t count, float* Theta, const float* X, const float* eta,
                         const float* lambda, const int64_t* offsets, void* stream);

/* stack[k*width + i] = vector[offsets[k] + i] (gather!) and the reverse
   (scatter!) (src/optim.jl:262-276; ext/FemtoChatCUDAExt.jl:127-149). */
fc_status fc_param_gather(int64_t width, int32_t count, float* stack, const float* vector, const int64_t* offsets,
                          void* stream);
fc_status fc_param_scatter(int64_t width, int32_t count, float* vector, const float* stack, const int64_t* offsets,
                           void* stream);

typedef struct {
  int32_t m, n;   /* rows and columns of each matrix */
  int32_t count;  /* matrices in the stack (k) */
  int32_t steps;  /* iterations (the reference's default is 5; beyond 5 the last coefficients repeat) */
  int32_t dtype;  /* compute type of the iteration buffers X, A, B, Y: FC_F32, or FC_BF16 (the
                     reference's compute_type=BFloat16, as scripts/train.jl passes it; products
                     accumulate in fp32 and round to bf16 as they are stored) */
} fc_polar_desc;

/* Bytes of the caller-owned workspace of fc_polar_express (X, Y, A, B and
   the per-matrix scale, as the reference's polar_workspace, plus 512 bytes
   per matrix of partial sums for the norm). */
fc_status fc_polar_workspace_bytes(const fc_polar_desc* desc, size_t* bytes);

/* Polar Express in place on G (m, n, count) float32 (reference
   src/optim.jl:115-149): X = G (or G^T when m > n) / (1.01 ||G||_F + 1e-6),
   then per step A = X X^T, B = b A + c A A, X = a X + B X, and G = X (or
   X^T), with b A and a X folded into the products' beta terms (the
   reference's CUBLAS gemmStridedBatchedEx, ext/FemtoChatCUDAExt.jl:121-125).
   In bf16 with min(m, n) and max(m, n) multiples of 128 the products are the
   library's own MFMA kernels (the last one writes G); otherwise they are
   strided-batched rocBLAS GEMMs, whose handle (one per device, created on
   the first such call) owns rocBLAS's own device workspace.  Everything else
   is in the caller's workspace.  Calls from several threads are serialised
   while they enqueue their products. */
fc_status fc_polar_express(const fc_polar_desc* desc, float* G, void* workspace, size_t workspace_bytes,
                           void* stream);

/* Polar Express of several stacks at once (the reference's Muon groups,
   src/optim.jl:278-309, one per matrix shape), each as fc_polar_express with
   its own workspace.  The stacks run concurrently on four helper streams
   forked from and joined back to the caller's stream with events, so the
   small batched products of different stacks share the GPU; the helper
   streams, their rocBLAS handles and the events are created on the first call
   per device and kept until the process ends. */
fc_status fc_polar_express_grouped(int32_t count, const fc_polar_desc* descs, float* const* G,
                                   void* const* workspaces, const size_t* workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FEMTOCHAT_OPTIM_H */
