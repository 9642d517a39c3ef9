// Loss-side kernels (gfx950): cross-entropy over a vocabulary column and its
// gradient, the embedding gather and its scatter-add gradient.
//
// Semantics (reference):
//   cross_entropy            src/gpt.jl:175-195, ext/FemtoChatCUDAExt.jl:21-54
//     loss[t] = max + log(sum(exp(x - max))) - x[target[t]], 0 if ignored;
//   cross_entropy_gradient!  src/kernels.jl:16-28, CUDAExt:56-61
//     delta[:, t] += scale[t] (softmax(x) - onehot(target[t])), skipped if ignored;
//   embedding                src/gpt.jl:34, CUDAExt:63-76   y[:, t] = W[:, tokens[t]];
//   embedding_gradient!      src/kernels.jl:8-14, CUDAExt:78-94
//     dW[:, tokens[t]] += dy[:, t], zero values skipped (no atomics for padding).
// Layout: column-major as the reference (a token's vocabulary column, or an
// embedding column, is contiguous).
//
// All four are HBM-bound.  Cross-entropy: one 256-thread workgroup per token;
// a single pass keeps a running (max, sum of exp) per thread, eight 16-byte
// loads in flight per round, combined across the workgroup at the end.  The
// gradient reuses the forward's log-sum-exp when the caller passes it (one
// read of the logits instead of two).
#include "attn_launch.hpp"
#include "attn_device.hpp"

#include <cmath>

namespace fc {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kFwdBatch = 8;  // 16-byte loads in flight per thread in a forward round (4, 8, 16 within 1%)
constexpr int kBwdBatch = 8;  // chunks per backward round (4, 8 measured within 3%)

template <typename I>
__device__ inline int64_t read_index(const void* p, int64_t i) {
  return (int64_t) static_cast<const I*>(p)[i];
}

__device__ inline int64_t index_at(const void* p, int64_t i, int type) {
  return type == 1 ? read_index<int64_t>(p, i) : read_index<int32_t>(p, i);
}

// (m, s) with s = sum exp(x - m) over what a thread or group has seen; s = 0
// means nothing seen (m is then -inf and must not enter an exponent).
struct Lse {
  float m, s;
};

__device__ inline Lse combine(Lse a, Lse b) {
  const float m = fmaxf(a.m, b.m);
  const float sa = a.s == 0.0f ? 0.0f : a.s * exp2f((a.m - m) * kLog2e);
  const float sb = b.s == 0.0f ? 0.0f : b.s * exp2f((b.m - m) * kLog2e);
  return Lse{m, sa + sb};
}

// Workgroup-wide combine of every thread's (m, s); all threads get the result.
__device__ inline Lse block_combine(Lse v) {
  __shared__ float sm[4], ss[4];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = combine(v, Lse{__shfl_xor(v.m, o), __shfl_xor(v.s, o)});
  const int wave = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) {
    sm[wave] = v.m;
    ss[wave] = v.s;
  }
  __syncthreads();
  Lse r{sm[0], ss[0]};
#pragma unroll
  for (int w = 1; w < 4; ++w) r = combine(r, Lse{sm[w], ss[w]});
  __syncthreads();  // the shared slots are free again when this returns
  return r;
}

// One thread's pass over its part of a column: values j = tid*4 + 1024 k
// (vectorised) or j = tid + 256 k (scalar).  Each round loads up to eight
// 16-byte chunks, then folds their maximum into m with one rescale of s.
// kStream: the column is read only once (the forward), so the loads are
// nontemporal (25% faster at 8192 x 32768); the gradient, which reads the
// column again, keeps it in the caches.
template <bool kVec, bool kStream = false>
__device__ inline Lse column_pass(const float* col, int V) {
  Lse acc{-INFINITY, 0.0f};
  if (kVec) {
    const int chunks = V / 4;
    for (int base = threadIdx.x; base < chunks; base += 256 * kFwdBatch) {
      f32x4 v[kFwdBatch];
      float bm = -INFINITY;
#pragma unroll
      for (int k = 0; k < kFwdBatch; ++k) {
        const int c = base + 256 * k;
        const f32x4* p = reinterpret_cast<const f32x4*>(col + 4 * c);
        v[k] = c < chunks ? (kStream ? __builtin_nontemporal_load(p) : *p) : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      }
#pragma unroll
      for (int k = 0; k < kFwdBatch; ++k) bm = fmaxf(bm, fmaxf(fmaxf(v[k][0], v[k][1]), fmaxf(v[k][2], v[k][3])));
      const float m = fmaxf(acc.m, bm);
      float s = acc.s == 0.0f ? 0.0f : acc.s * exp2f((acc.m - m) * kLog2e);
#pragma unroll
      for (int k = 0; k < kFwdBatch; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) s += exp2f((v[k][i] - m) * kLog2e);  // exp2(-inf) = 0 for padding
      acc = Lse{m, s};
    }
  } else {
    for (int j = threadIdx.x; j < V; j += 256) acc = combine(acc, Lse{col[j], 1.0f});
  }
  return acc;
}

template <bool kVec>
__global__ __launch_bounds__(256) void xent_fwd_kernel(XentArgs a) {
  const int64_t token = blockIdx.x;
  const float* col = a.logits + token * (int64_t)a.V;
  const Lse r = block_combine(column_pass<kVec, true>(col, a.V));
  if (threadIdx.x == 0) {
    const float lse = r.m + logf(r.s);
    const int64_t raw = index_at(a.targets, token, a.index_type);
    const int64_t t = raw - a.index_base;
    float loss = 0.0f;
    if (raw != a.ignore_index) loss = (t >= 0 && t < a.V) ? lse - col[t] : __builtin_nanf("");
    a.losses[token] = loss;
    if (a.lse != nullptr) a.lse[token] = lse;
  }
}

// reduced[0] = sum of losses (or their mean over valid targets), reduced[1] =
// number of valid targets; one workgroup, float64 accumulation.
__global__ __launch_bounds__(1024) void xent_reduce_kernel(XentArgs a) {
  __shared__ double part[16];
  __shared__ double cnt[16];
  double s = 0.0, c = 0.0;
  for (int64_t i = threadIdx.x; i < a.N; i += 1024) {
    if (a.losses != nullptr) s += (double)a.losses[i];
    c += index_at(a.targets, i, a.index_type) != a.ignore_index ? 1.0 : 0.0;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    s += __shfl_xor(s, o);
    c += __shfl_xor(c, o);
  }
  if ((threadIdx.x & 63) == 0) {
    part[threadIdx.x / 64] = s;
    cnt[threadIdx.x / 64] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double S = 0.0, C = 0.0;
    for (int w = 0; w < 16; ++w) {
      S += part[w];
      C += cnt[w];
    }
    if (a.reduced != nullptr) a.reduced[0] = (float)(a.reduction == 2 ? S / C : S);
    if (a.count != nullptr) *a.count = (float)C;
  }
}

template <bool kVec>
__global__ __launch_bounds__(256) void xent_bwd_kernel(XentArgs a) {
  const int64_t token = blockIdx.x;
  const int64_t raw = index_at(a.targets, token, a.index_type);
  if (raw == a.ignore_index) return;  // the reference adds zero (uniform per workgroup)
  const float* col = a.logits + token * (int64_t)a.V;
  float* out = a.dlogits + token * (int64_t)a.V;
  float lse;
  if (a.lse_in != nullptr) {
    lse = a.lse_in[token];
  } else {
    const Lse r = block_combine(column_pass<kVec>(col, a.V));
    lse = r.m + logf(r.s);
  }
  // scale = dy / count(valid) ("mean"), dy ("sum"), dy[token] ("none"); the
  // division is the reference's fp32 `dy ./ sum(valid)`.
  float w = a.dy[a.reduction == 0 ? token : 0];
  if (a.reduction == 2) w = w / *a.count;
  const int64_t t = raw - a.index_base;  // outside [0, V): no one-hot term, as the reference's comparison
  if (kVec) {
    // rounds of kBwdBatch 16-byte chunks: every load of a round (logits and,
    // when accumulating, the gradient) is issued before its arithmetic
    const int chunks = a.V / 4;
    for (int base = threadIdx.x; base < chunks; base += 256 * kBwdBatch) {
      f32x4 x[kBwdBatch], o[kBwdBatch];
#pragma unroll
      for (int k = 0; k < kBwdBatch; ++k) {
        const int c = base + 256 * k;
        if (c < chunks) {
          x[k] = *reinterpret_cast<const f32x4*>(col + 4 * c);
          o[k] = a.overwrite ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : *reinterpret_cast<const f32x4*>(out + 4 * c);
        }
      }
#pragma unroll
      for (int k = 0; k < kBwdBatch; ++k) {
        const int c = base + 256 * k;
        if (c >= chunks) continue;
        f32x4 g;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = exp2f((x[k][i] - lse) * kLog2e);
          g[i] = w * (p - (4 * c + i == t ? 1.0f : 0.0f));
        }
        // nontemporal store (1.6% faster here; not in the fused kernel, where it was slower)
        __builtin_nontemporal_store(a.overwrite ? g : o[k] + g, reinterpret_cast<f32x4*>(out + 4 * c));
      }
    }
  } else {
    for (int j = threadIdx.x; j < a.V; j += 256) {
      const float p = exp2f((col[j] - lse) * kLog2e);
      const float g = w * (p - (j == t ? 1.0f : 0.0f));
      out[j] = a.overwrite ? g : out[j] + g;
    }
  }
}

// ---- fused forward and gradient ------------------------------------------------
// One 1024-thread workgroup per token holds the whole column in registers
// (up to kFusedChunks 16-byte chunks per thread: V <= 4096 kFusedChunks),
// so the logits are read once: maximum, sum of exponentials, the loss, and
// the gradient scale (p - onehot) written (or added) in the same pass.
constexpr int kFusedChunks = 8;
constexpr int kFusedThreads = 1024;

__device__ inline float block_reduce_1024(float v, bool is_max, float* slots) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float u = __shfl_xor(v, o);
    v = is_max ? fmaxf(v, u) : v + u;
  }
  if ((threadIdx.x & 63) == 0) slots[threadIdx.x / 64] = v;
  __syncthreads();
  float r = slots[0];
#pragma unroll
  for (int w = 1; w < 16; ++w) r = is_max ? fmaxf(r, slots[w]) : r + slots[w];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kFusedThreads) void xent_fused_kernel(XentArgs a) {
  __shared__ float slots[16];
  const int64_t token = blockIdx.x;
  const float* col = a.logits + token * (int64_t)a.V;
  float* out = a.dlogits + token * (int64_t)a.V;
  const int chunks = a.V / 4;
  f32x4 x[kFusedChunks];
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kFusedChunks; ++k) {
    const int c = threadIdx.x + kFusedThreads * k;
    x[k] = c < chunks ? *reinterpret_cast<const f32x4*>(col + 4 * c) : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    mx = fmaxf(mx, fmaxf(fmaxf(x[k][0], x[k][1]), fmaxf(x[k][2], x[k][3])));
  }
  const float M = block_reduce_1024(mx, true, slots);
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < kFusedChunks; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i) sum += exp2f((x[k][i] - M) * kLog2e);
  const float lse = M + logf(block_reduce_1024(sum, false, slots));
  const int64_t raw = index_at(a.targets, token, a.index_type);
  const int64_t t = raw - a.index_base;
  const bool valid = raw != a.ignore_index;
  if (threadIdx.x == 0) {
    a.losses[token] = valid ? ((t >= 0 && t < a.V) ? lse - col[t] : __builtin_nanf("")) : 0.0f;
    if (a.lse != nullptr) a.lse[token] = lse;
  }
  if (!valid) return;  // uniform: the gradient column is left untouched, as the separate gradient does
  float w = a.dy[a.reduction == 0 ? token : 0];
  if (a.reduction == 2) w = w / *a.count;
#pragma unroll
  for (int k = 0; k < kFusedChunks; ++k) {
    const int c = threadIdx.x + kFusedThreads * k;
    if (c >= chunks) continue;
    f32x4 g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = exp2f((x[k][i] - lse) * kLog2e);
      g[i] = w * (p - (4 * c + i == t ? 1.0f : 0.0f));
    }
    f32x4* o = reinterpret_cast<f32x4*>(out + 4 * c);
    *o = a.overwrite ? g : *o + g;
  }
}

// ---- embedding ----------------------------------------------------------------
// One wave per token, 16-byte chunks of its column (D % 4 == 0) or scalars.
template <bool kVec, typename Y>
__global__ __launch_bounds__(256) void embed_fwd_kernel(EmbedArgs a) {
  const int64_t token = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  if (token >= a.N) return;
  const int lane = threadIdx.x & 63;
  const int64_t id = index_at(a.tokens, token, a.index_type) - a.index_base;
  const bool ok = id >= 0 && id < a.vocab;  // an out-of-range id poisons its column (an index error in the reference)
  const float* w = a.weights + (ok ? id : 0) * (int64_t)a.D;
  Y* y = static_cast<Y*>(a.y) + token * (int64_t)a.D;
  const float poison = ok ? 1.0f : __builtin_nanf("");
  if (kVec) {
    for (int c = lane; c < a.D / 4; c += 64) {
      f32x4 v = *reinterpret_cast<const f32x4*>(w + 4 * c);
      if (!ok) v = f32x4{poison, poison, poison, poison};
      if constexpr (sizeof(Y) == 4) {
        *reinterpret_cast<f32x4*>(y + 4 * c) = v;
      } else {
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<bf16x4*>(y + 4 * c) = __builtin_convertvector(v, bf16x4);
      }
    }
  } else {
    for (int j = lane; j < a.D; j += 64) y[j] = static_cast<Y>(ok ? w[j] : poison);
  }
}

template <bool kVec, typename Y>
__global__ __launch_bounds__(256) void embed_bwd_kernel(EmbedArgs a) {
  const int64_t token = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  if (token >= a.N) return;
  const int lane = threadIdx.x & 63;
  const int64_t id = index_at(a.tokens, token, a.index_type) - a.index_base;
  if (id < 0 || id >= a.vocab) return;  // nothing to add for an id outside the table
  float* dw = a.dweights + id * (int64_t)a.D;
  const Y* dy = static_cast<const Y*>(a.dy) + token * (int64_t)a.D;
  auto add = [&](int j, float v) {
    if (v != 0.0f) unsafeAtomicAdd(dw + j, v);  // hardware fp32 atomic add in L2
  };
  if (kVec) {
    for (int c = lane; c < a.D / 4; c += 64) {
      f32x4 v;
      if constexpr (sizeof(Y) == 4) {
        v = *reinterpret_cast<const f32x4*>(dy + 4 * c);
      } else {
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        v = __builtin_convertvector(*reinterpret_cast<const bf16x4*>(dy + 4 * c), f32x4);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) add(4 * c + i, v[i]);
    }
  } else {
    for (int j = lane; j < a.D; j += 64) add(j, static_cast<float>(dy[j]));
  }
}

}  // namespace

hipError_t launch_xent_fwd(const XentArgs& a, hipStream_t s) {
  const bool vec = a.V % 4 == 0 && (reinterpret_cast<uintptr_t>(a.logits) & 15) == 0;
  const ProfileMark mk = profile_begin(s);
  if (vec) hipLaunchKernelGGL(xent_fwd_kernel<true>, dim3((unsigned)a.N), dim3(256), 0, s, a);
  else hipLaunchKernelGGL(xent_fwd_kernel<false>, dim3((unsigned)a.N), dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  profile_end(mk, "xent_fwd", s);
  if (e != hipSuccess || (a.reduced == nullptr && a.count == nullptr)) return e;
  hipLaunchKernelGGL(xent_reduce_kernel, dim3(1), dim3(1024), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_xent_count(const XentArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(xent_reduce_kernel, dim3(1), dim3(1024), 0, s, a);
  return hipGetLastError();
}

bool xent_fused_supported(const XentArgs& a) {
  return a.V % 4 == 0 && a.V <= 4 * kFusedThreads * kFusedChunks &&
         ((reinterpret_cast<uintptr_t>(a.logits) | reinterpret_cast<uintptr_t>(a.dlogits)) & 15) == 0;
}

hipError_t launch_xent_fused(const XentArgs& a, hipStream_t s) {
  const ProfileMark mk = profile_begin(s);
  hipLaunchKernelGGL(xent_fused_kernel, dim3((unsigned)a.N), dim3(kFusedThreads), 0, s, a);
  hipError_t e = hipGetLastError();
  profile_end(mk, "xent_fused", s);
  if (e != hipSuccess || (a.reduced == nullptr)) return e;
  // count is the caller's input here (it scaled the gradient): the reduction
  // writes only the loss sum or mean.
  XentArgs r = a;
  r.count = nullptr;
  hipLaunchKernelGGL(xent_reduce_kernel, dim3(1), dim3(1024), 0, s, r);
  return hipGetLastError();
}

hipError_t launch_xent_bwd(const XentArgs& a, hipStream_t s) {
  const bool vec = a.V % 4 == 0 && ((reinterpret_cast<uintptr_t>(a.logits) | reinterpret_cast<uintptr_t>(a.dlogits)) & 15) == 0;
  const ProfileMark mk = profile_begin(s);
  if (vec) hipLaunchKernelGGL(xent_bwd_kernel<true>, dim3((unsigned)a.N), dim3(256), 0, s, a);
  else hipLaunchKernelGGL(xent_bwd_kernel<false>, dim3((unsigned)a.N), dim3(256), 0, s, a);
  const hipError_t e = hipGetLastError();
  profile_end(mk, "xent_bwd", s);
  return e;
}

hipError_t launch_embed(const EmbedArgs& a, bool backward, bool bf16_y, hipStream_t s) {
  const bool vec = a.D % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(backward ? (const void*)a.dweights : (const void*)a.weights) |
                     reinterpret_cast<uintptr_t>(backward ? a.dy : (const void*)a.y)) &
                    15) == 0;
  const dim3 grid((unsigned)((a.N + 3) / 4)), block(256);
  const ProfileMark mk = profile_begin(s);
  if (backward) {
    if (bf16_y) {
      if (vec) hipLaunchKernelGGL((embed_bwd_kernel<true, bf16>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((embed_bwd_kernel<false, bf16>), grid, block, 0, s, a);
    } else {
      if (vec) hipLaunchKernelGGL((embed_bwd_kernel<true, float>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((embed_bwd_kernel<false, float>), grid, block, 0, s, a);
    }
  } else {
    if (bf16_y) {
      if (vec) hipLaunchKernelGGL((embed_fwd_kernel<true, bf16>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((embed_fwd_kernel<false, bf16>), grid, block, 0, s, a);
    } else {
      if (vec) hipLaunchKernelGGL((embed_fwd_kernel<true, float>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((embed_fwd_kernel<false, float>), grid, block, 0, s, a);
    }
  }
  const hipError_t e = hipGetLastError();
  profile_end(mk, backward ? "embed_bwd" : "embed_fwd", s);
  return e;
}

}  // namespace fc
