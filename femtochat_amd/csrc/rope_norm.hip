// Attention prologue: rotary embedding, then RMS norm over the head
// dimension scaled by 1.2, for Q or K in the kernel layout (gfx950).
//
// Semantics (reference src/gpt.jl:101-106 with apply_rotary_embedding
// :53-77 and norm :15-20; tables from src/parameters.jl:409-427):
//   u[j]     =  x[j] c[j] + x[j+d] s[j]          (d = D/2, j < d)
//   u[j+d]   = -x[j] s[j] + x[j+d] c[j]
//   y        =  u / sqrt(sum(u^2)/D + eps) * 1.2,   eps = eps(eltype(x))
// with c, s the columns of the cos/sin tables at the token's position (its
// index t, or positions[t, b] when given).  In bf16 each operation rounds to
// bf16 as Julia's BFloat16 arithmetic does: the tables are rounded to bf16,
// every product and sum of the rotation is rounded, the norm divides in fp32
// (sum of squares in fp32) and rounds, and the product by 1.2 rounds again.
// fp32 follows the same steps without contraction into fused multiply-adds
// (Julia does not contract either).
//
// The backward recomputes u and the norm from x and returns
//   g  = 1.2 dy,   y' = u / r,   du = (g - y' (g . y') / D) / r,
//   dx[j] = du[j] c[j] - du[j+d] s[j],  dx[j+d] = du[j] s[j] + du[j+d] c[j]
// in fp32 (the gradient of the exact function at the rounded rotation).
//
// Work split: one head vector per D/16 consecutive threads, each holding
// eight rotation pairs (elements j..j+7 and j+d..j+d+7, one 16-byte bf16
// load per half), so the rotation needs no cross-lane exchange and the sum
// of squares is a butterfly over D/16 lanes; each thread takes four vectors
// and issues all their loads before any arithmetic.  Memory-bound: a vector
// is read and written once; the tables stay in L2.
#include "attn_launch.hpp"
#include "attn_device.hpp"

#pragma clang fp contract(off)

namespace fc {

namespace {

__device__ inline float bf(float x) { return static_cast<float>(static_cast<bf16>(x)); }

// Eight consecutive elements (16 bytes of bf16, 32 of fp32).
template <typename E>
struct Eight;

template <>
struct Eight<float> {
  __device__ static inline void load(const float* p, float* v) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
  __device__ static inline void store(float* p, const float* v, bool accumulate) {
    f32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = v[i];
      b[i] = v[4 + i];
    }
    if (accumulate) {
      a += *reinterpret_cast<const f32x4*>(p);
      b += *reinterpret_cast<const f32x4*>(p + 4);
    }
    *reinterpret_cast<f32x4*>(p) = a;
    *reinterpret_cast<f32x4*>(p + 4) = b;
  }
};

template <>
struct Eight<bf16> {
  __device__ static inline void load(const bf16* p, float* v) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(a[i]);
  }
  __device__ static inline void store(bf16* p, const float* v, bool accumulate) {
    bf16x8 a;
    if (accumulate) {
      const bf16x8 o = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = static_cast<bf16>(v[i] + static_cast<float>(o[i]));
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = static_cast<bf16>(v[i]);
    }
    *reinterpret_cast<bf16x8*>(p) = a;
  }
};

// Sum over the G = D/16 lanes of one vector (consecutive lanes).
template <int G>
__device__ inline float group_sum(float v) {
#pragma unroll
  for (int o = 1; o < G; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

// A thread's share of one vector: eight rotation pairs (elements j0..j0+7 and
// j0+d..j0+d+7), their table entries and the rotated values u (rounded as
// the element type rounds).
template <int D, typename E>
struct Share {
  static constexpr int d = D / 2;
  float x1[8], x2[8], c[8], s[8];

  __device__ inline void load(const E* xv, const float* sin_t, const float* cos_t, int pos, int table_len,
                              int j0) {
    Eight<E>::load(xv + j0, x1);
    Eight<E>::load(xv + d + j0, x2);
    const bool ok = pos >= 0 && pos < table_len;
    const float* sp = sin_t + (int64_t)(ok ? pos : 0) * d + j0;
    const float* cp = cos_t + (int64_t)(ok ? pos : 0) * d + j0;
    Eight<float>::load(sp, s);
    Eight<float>::load(cp, c);
    constexpr bool kB = sizeof(E) == 2;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // A position outside the tables poisons the vector (NaN), as an out of
      // range table index is an error in the reference.
      c[i] = ok ? (kB ? bf(c[i]) : c[i]) : __builtin_nanf("");
      s[i] = ok ? (kB ? bf(s[i]) : s[i]) : __builtin_nanf("");
    }
  }
  // Rotates in place: x1, x2 become u[j], u[j+d].
  __device__ inline void rotate() {
    constexpr bool kB = sizeof(E) == 2;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float u1, u2;
      if (kB) {
        u1 = bf(bf(x1[i] * c[i]) + bf(x2[i] * s[i]));
        u2 = bf(bf(x1[i] * -s[i]) + bf(x2[i] * c[i]));
      } else {
        u1 = x1[i] * c[i] + x2[i] * s[i];
        u2 = x1[i] * -s[i] + x2[i] * c[i];
      }
      x1[i] = u1;
      x2[i] = u2;
    }
  }
  // sqrt(sum(u^2)/D + eps) over the vector (after rotate()).
  __device__ inline float rms() const {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += x1[i] * x1[i] + x2[i] * x2[i];
    ss = group_sum<D / 16>(ss);
    constexpr float eps = sizeof(E) == 2 ? 0.0078125f : 1.1920928955078125e-7f;  // eps(BFloat16), eps(Float32)
    return sqrtf(ss / static_cast<float>(D) + eps);
  }
};

// Thread geometry: G = D/16 lanes per vector, each thread NV vectors spaced
// by the number of groups in the grid (consecutive groups take consecutive
// vectors, so a wave's loads are contiguous); every load of a thread is
// issued before its arithmetic.
constexpr int kNV = 4;

template <int D, typename E>
__global__ __launch_bounds__(256) void rope_norm_fwd_kernel(RopeNormArgs a) {
  constexpr int G = D / 16, d = D / 2;
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int j0 = 8 * (int)(tid % G);
  const int64_t group = tid / G, ngroups = (int64_t)gridDim.x * (256 / G);
  Share<D, E> sh[kNV];
#pragma unroll
  for (int k = 0; k < kNV; ++k) {
    const int64_t vec = min(group + k * ngroups, a.vectors - 1);  // clamped: loads stay in range
    const int64_t tok = vec / a.NH;  // b*T + t
    const int pos = a.pos ? a.pos[tok] : (int)(tok % a.T);
    sh[k].load(static_cast<const E*>(a.X) + vec * D, a.sin_t, a.cos_t, pos, a.table_len, j0);
  }
#pragma unroll
  for (int k = 0; k < kNV; ++k) {
    const int64_t vec = group + k * ngroups;
    sh[k].rotate();
    const float r = sh[k].rms();
    if (vec >= a.vectors) continue;  // whole groups (G divides 64), after the group's shuffles
    constexpr bool kB = sizeof(E) == 2;
    float y1[8], y2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (kB) {
        y1[i] = bf(bf(sh[k].x1[i] / r) * 1.2f);
        y2[i] = bf(bf(sh[k].x2[i] / r) * 1.2f);
      } else {
        y1[i] = sh[k].x1[i] / r * 1.2f;
        y2[i] = sh[k].x2[i] / r * 1.2f;
      }
    }
    E* yv = static_cast<E*>(a.Y) + vec * D;
    Eight<E>::store(yv + j0, y1, false);
    Eight<E>::store(yv + d + j0, y2, false);
  }
}

template <int D, typename E>
__global__ __launch_bounds__(256) void rope_norm_bwd_kernel(RopeNormArgs a) {
  constexpr int G = D / 16, d = D / 2;
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int j0 = 8 * (int)(tid % G);
  const int64_t group = tid / G, ngroups = (int64_t)gridDim.x * (256 / G);
  Share<D, E> sh[kNV];
  float g1[kNV][8], g2[kNV][8];
#pragma unroll
  for (int k = 0; k < kNV; ++k) {
    const int64_t vec = min(group + k * ngroups, a.vectors - 1);
    const int64_t tok = vec / a.NH;
    const int pos = a.pos ? a.pos[tok] : (int)(tok % a.T);
    sh[k].load(static_cast<const E*>(a.X) + vec * D, a.sin_t, a.cos_t, pos, a.table_len, j0);
    Eight<E>::load(static_cast<const E*>(a.dY) + vec * D + j0, g1[k]);
    Eight<E>::load(static_cast<const E*>(a.dY) + vec * D + d + j0, g2[k]);
  }
#pragma unroll
  for (int k = 0; k < kNV; ++k) {
    const int64_t vec = group + k * ngroups;
    sh[k].rotate();
    const float r = sh[k].rms();
    float gy = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      g1[k][i] *= 1.2f;
      g2[k][i] *= 1.2f;
      gy += g1[k][i] * (sh[k].x1[i] / r) + g2[k][i] * (sh[k].x2[i] / r);
    }
    gy = group_sum<G>(gy) / static_cast<float>(D);
    if (vec >= a.vectors) continue;
    float dx1[8], dx2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float du1 = (g1[k][i] - (sh[k].x1[i] / r) * gy) / r;
      const float du2 = (g2[k][i] - (sh[k].x2[i] / r) * gy) / r;
      dx1[i] = du1 * sh[k].c[i] - du2 * sh[k].s[i];
      dx2[i] = du1 * sh[k].s[i] + du2 * sh[k].c[i];
    }
    E* dxv = static_cast<E*>(a.dX) + vec * D;
    Eight<E>::store(dxv + j0, dx1, a.accumulate != 0);
    Eight<E>::store(dxv + d + j0, dx2, a.accumulate != 0);
  }
}

template <int D, typename E>
hipError_t launch_t(const RopeNormArgs& a, bool backward, hipStream_t s) {
  constexpr int G = D / 16;
  const int64_t groups = (a.vectors + kNV - 1) / kNV;
  const dim3 grid((unsigned)((groups * G + 255) / 256)), block(256);
  const ProfileMark mk = profile_begin(s);
  if (backward) hipLaunchKernelGGL((rope_norm_bwd_kernel<D, E>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((rope_norm_fwd_kernel<D, E>), grid, block, 0, s, a);
  const hipError_t e = hipGetLastError();
  profile_end(mk, backward ? (sizeof(E) == 2 ? "rope_norm_bwd_bf16" : "rope_norm_bwd_f32")
                           : (sizeof(E) == 2 ? "rope_norm_fwd_bf16" : "rope_norm_fwd_f32"),
              s);
  return e;
}

template <typename E>
hipError_t launch_e(int D, const RopeNormArgs& a, bool backward, hipStream_t s) {
  switch (D) {
    case 16: return launch_t<16, E>(a, backward, s);
    case 32: return launch_t<32, E>(a, backward, s);
    case 64: return launch_t<64, E>(a, backward, s);
    case 128: return launch_t<128, E>(a, backward, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_rope_norm(int D, bool bf16_storage, const RopeNormArgs& a, bool backward, hipStream_t s) {
  return bf16_storage ? launch_e<bf16>(D, a, backward, s) : launch_e<float>(D, a, backward, s);
}

}  // namespace fc
