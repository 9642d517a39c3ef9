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
#include <type_traits>

#include "attn_launch.hpp"
#include "attn_device.hpp"

#pragma clang fp contract(off)

namespace fc {

namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Rounds a and b to bf16 (nearest, ties to even) with one packed conversion
// and widens them back to fp32.
// (The conversion is written as the instruction itself: the vector-type
// route through __builtin_convertvector makes the compiler keep the rotation
// arrays in scratch memory.)
__device__ inline void bf2(float& a, float& b) {
  uint32_t w;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(w) : "v"(a), "v"(b));
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}

__device__ inline uint32_t divide(uint32_t n, FastDiv f) { return (__umulhi(n, f.m) + n) >> f.l; }

// The table row of vector vec (= (b*T + t)*NH + h): positions[b, t], or t.
// (Whether positions are given is a template parameter: a branch on it
// would make every vector's loads wait for the previous vector's.)
template <bool kPos>
__device__ inline int position_of(const RopeNormArgs& a, uint32_t vec) {
  const uint32_t tok = divide(vec, a.by_NH);  // b*T + t
  if (kPos) return a.pos[tok];
  return (int)(tok - divide(tok, a.by_T) * (uint32_t)a.T);
}

// Eight consecutive elements (16 bytes of bf16, 32 of fp32).
template <typename E>
struct Eight;

template <>
struct Eight<float> {
  struct Raw {
    f32x4 a, b;
  };
  __device__ static inline Raw load_raw(const float* p) {
    return Raw{*reinterpret_cast<const f32x4*>(p), *reinterpret_cast<const f32x4*>(p + 4)};
  }
  __device__ static inline void unpack(const Raw& r, float* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = r.a[i];
      v[4 + i] = r.b[i];
    }
  }
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
  using Raw = bf16x8;
  __device__ static inline Raw load_raw(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
  __device__ static inline void unpack(const Raw& r, float* v) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(r[i]);
  }
  __device__ static inline void load(const bf16* p, float* v) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(a[i]);
  }
  __device__ static inline void store(bf16* p, const float* v, bool accumulate) {
    f32x8 w;
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = v[i];
    if (accumulate) {
      const bf16x8 o = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] += static_cast<float>(o[i]);
    }
    *reinterpret_cast<bf16x8*>(p) = __builtin_convertvector(w, bf16x8);
  }
};

// Sum over the G = D/16 lanes of one vector (consecutive lanes, G <= 8),
// with DPP adds: swap neighbours, swap pairs (quad_perm), then add the other
// quad of the eight (row_half_mirror).  Addition commutes, so every lane of
// the group ends with the same bits.  All lanes must be active.
template <int G>
__device__ inline float group_sum(float v) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8, "group of 1, 2, 4 or 8 lanes");
  auto step = [](float x, auto ctrl) __attribute__((always_inline)) {
    const int y = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(ctrl)::value, 0xF, 0xF, false);
    return x + __builtin_bit_cast(float, y);
  };
  if (G >= 2) v = step(v, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  if (G >= 4) v = step(v, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  if (G >= 8) v = step(v, std::integral_constant<int, 0x141>{});  // row_half_mirror
  return v;
}

// u / r correctly rounded, from y = RN(1/r): q = RN(u y), e = u - r q (exact
// in one fused multiply-add), RN(q + e y) (Markstein's correction; exact for
// r in [2^-12, 2^64) and |u| >= 2^-100, where the remainder cannot
// underflow; u is then not zero, so the sign needs no care).
__device__ inline float quotient(float u, float r, float y) {
  const float q = u * y;
  const float e = __builtin_fmaf(-r, q, u);
  return __builtin_fmaf(e, y, q);
}

// A thread's share of one vector: eight rotation pairs (elements j0..j0+7 and
// j0+d..j0+d+7), their table entries and the rotated values u (rounded as
// the element type rounds).
template <int D, typename E>
struct Share {
  static constexpr int d = D / 2;
  static constexpr bool kB = sizeof(E) == 2;
  // As loaded (kept packed while the loads are in flight) ...
  typename Eight<E>::Raw x1r, x2r;
  Eight<float>::Raw cr, sr;
  bool ok;
  // ... and as fp32 values once rotate() has run.
  float x1[8], x2[8], c[8], s[8];

  __device__ inline void load(const E* xv, const float* sin_t, const float* cos_t, int pos, int table_len,
                              int j0) {
    x1r = Eight<E>::load_raw(xv + j0);
    x2r = Eight<E>::load_raw(xv + d + j0);
    ok = pos >= 0 && pos < table_len;
    const int64_t row = (int64_t)(ok ? pos : 0) * d + j0;
    sr = Eight<float>::load_raw(sin_t + row);
    cr = Eight<float>::load_raw(cos_t + row);
  }
  // Rotates: x1, x2 become u[j], u[j+d].  bf16 rounds the tables and every
  // product and sum.
  __device__ inline void rotate() {
    Eight<E>::unpack(x1r, x1);
    Eight<E>::unpack(x2r, x2);
    Eight<float>::unpack(sr, s);
    Eight<float>::unpack(cr, c);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (kB) {
        bf2(c[i], s[i]);
        float p1 = x1[i] * c[i], p2 = x2[i] * s[i];
        float p3 = x1[i] * -s[i], p4 = x2[i] * c[i];
        bf2(p1, p2);
        bf2(p3, p4);
        float u1 = p1 + p2, u2 = p3 + p4;
        bf2(u1, u2);
        x1[i] = u1;
        x2[i] = u2;
      } else {
        const float u1 = x1[i] * c[i] + x2[i] * s[i];
        const float u2 = x1[i] * -s[i] + x2[i] * c[i];
        x1[i] = u1;
        x2[i] = u2;
      }
    }
  }
  // sqrt(sum(u^2)/D + eps) over the vector (after rotate()); NaN for a
  // position outside the tables, which poisons the vector as an out of
  // range table index is an error in the reference.
  __device__ inline float rms() const {
    // (fused: the order and rounding of this sum are not the reference's
    // anyway, which sums in its own order)
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(x2[i], x2[i], __builtin_fmaf(x1[i], x1[i], ss));
    ss = group_sum<D / 16>(ss);
    constexpr float eps = kB ? 0.0078125f : 1.1920928955078125e-7f;  // eps(BFloat16), eps(Float32)
    const float r = sqrtf(ss / static_cast<float>(D) + eps);
    return ok ? r : __builtin_nanf("");
  }
  // Whether quotient() is exact for every u of this share.
  __device__ inline bool fast_quotient(float r) const {
    float m = fminf(fabsf(x1[0]), fabsf(x2[0]));
#pragma unroll
    for (int i = 1; i < 8; ++i) m = fminf(m, fminf(fabsf(x1[i]), fabsf(x2[i])));
    return (r < 0x1p64f) & (m >= 0x1p-100f);  // false for r = NaN; a NaN u gives NaN either way
  }
};

// Thread geometry: G = D/16 lanes per vector, each thread NV vectors spaced
// by the number of groups in the grid (consecutive groups take consecutive
// vectors, so a wave's loads are contiguous); every load of a thread is
// issued before its arithmetic.  The forward takes four vectors per thread,
// the backward (which holds dY too) two: the fastest of 2, 4 and 8 for each.
// (The forward is bound by its VALU instructions, about 25 per element for
// bf16 at four cycles each; a grid-stride loop that prefetches the next
// sweep's loads during the current sweep's arithmetic measured slower.)
constexpr int kFwdNV = 4, kBwdNV = 2;

template <int D, typename E, bool kPos>
__global__ __launch_bounds__(256) void rope_norm_fwd_kernel(RopeNormArgs a) {
  constexpr int G = D / 16, d = D / 2, kNV = kFwdNV;
  constexpr bool kB = sizeof(E) == 2;
  const uint32_t tid = blockIdx.x * 256 + threadIdx.x;
  const int j0 = 8 * (int)(tid % G);
  const uint32_t group = tid / G, ngroups = gridDim.x * (256 / G);
  Share<D, E> sh[kNV];
#pragma unroll
  for (int k = 0; k < kNV; ++k) {
    const uint32_t vec = min(group + k * ngroups, (uint32_t)a.vectors - 1);  // clamped: loads stay in range
    sh[k].load(static_cast<const E*>(a.X) + (int64_t)vec * D, a.sin_t, a.cos_t, position_of<kPos>(a, vec),
               a.table_len, j0);
  }
#pragma unroll
  for (int k = 0; k < kNV; ++k) {
    const uint32_t vec = group + k * ngroups;
    sh[k].rotate();
    const float r = sh[k].rms();
    if (vec >= (uint32_t)a.vectors) continue;  // whole groups (G divides 64), after the group's shuffles
    E* yv = static_cast<E*>(a.Y) + (int64_t)vec * D;
    // y = bf(bf(u / r) * 1.2) (fp32: u / r * 1.2); each branch computes and
    // stores on its own so no array lives across the branch.
    auto emit = [&](auto div) __attribute__((always_inline)) {
      float t1[8], t2[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        t1[i] = div(sh[k].x1[i]);
        t2[i] = div(sh[k].x2[i]);
        if (kB) bf2(t1[i], t2[i]);
        t1[i] *= 1.2f;
        t2[i] *= 1.2f;
      }
      Eight<E>::store(yv + j0, t1, false);
      Eight<E>::store(yv + d + j0, t2, false);
    };
    if (sh[k].fast_quotient(r)) {
      const float y = 1.0f / r;
      emit([&](float u) __attribute__((always_inline)) { return quotient(u, r, y); });
    } else {
      emit([&](float u) __attribute__((always_inline)) { return u / r; });
    }
  }
}

template <int D, typename E, bool kPos>
__global__ __launch_bounds__(256) void rope_norm_bwd_kernel(RopeNormArgs a) {
  constexpr int G = D / 16, d = D / 2, kNV = kBwdNV;
  const uint32_t tid = blockIdx.x * 256 + threadIdx.x;
  const int j0 = 8 * (int)(tid % G);
  const uint32_t group = tid / G, ngroups = gridDim.x * (256 / G);
  Share<D, E> sh[kNV];
  float g1[kNV][8], g2[kNV][8];
#pragma unroll
  for (int k = 0; k < kNV; ++k) {
    const uint32_t vec = min(group + k * ngroups, (uint32_t)a.vectors - 1);
    sh[k].load(static_cast<const E*>(a.X) + (int64_t)vec * D, a.sin_t, a.cos_t, position_of<kPos>(a, vec), a.table_len, j0);
    Eight<E>::load(static_cast<const E*>(a.dY) + (int64_t)vec * D + j0, g1[k]);
    Eight<E>::load(static_cast<const E*>(a.dY) + (int64_t)vec * D + d + j0, g2[k]);
  }
#pragma unroll
  for (int k = 0; k < kNV; ++k) {
    const uint32_t vec = group + k * ngroups;
    sh[k].rotate();
    // fp32 gradient: products with y = 1/r (a few units in the last place)
    const float y = 1.0f / sh[k].rms();
    float gy = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      g1[k][i] *= 1.2f;
      g2[k][i] *= 1.2f;
      sh[k].x1[i] *= y;  // u / r
      sh[k].x2[i] *= y;
      gy += g1[k][i] * sh[k].x1[i] + g2[k][i] * sh[k].x2[i];
    }
    gy = group_sum<G>(gy) / static_cast<float>(D);
    if (vec >= (uint32_t)a.vectors) continue;
    float dx1[8], dx2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float du1 = (g1[k][i] - sh[k].x1[i] * gy) * y;
      const float du2 = (g2[k][i] - sh[k].x2[i] * gy) * y;
      dx1[i] = du1 * sh[k].c[i] - du2 * sh[k].s[i];
      dx2[i] = du1 * sh[k].s[i] + du2 * sh[k].c[i];
    }
    E* dxv = static_cast<E*>(a.dX) + (int64_t)vec * D;
    Eight<E>::store(dxv + j0, dx1, a.accumulate != 0);
    Eight<E>::store(dxv + d + j0, dx2, a.accumulate != 0);
  }
}

template <int D, typename E>
hipError_t launch_t(const RopeNormArgs& a, bool backward, hipStream_t s) {
  constexpr int G = D / 16;
  const int nv = backward ? kBwdNV : kFwdNV;
  const int64_t groups = ((int64_t)a.vectors + nv - 1) / nv;
  const dim3 grid((unsigned)((groups * G + 255) / 256)), block(256);
  const ProfileMark mk = profile_begin(s);
  if (backward) {
    if (a.pos) hipLaunchKernelGGL((rope_norm_bwd_kernel<D, E, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((rope_norm_bwd_kernel<D, E, false>), grid, block, 0, s, a);
  } else {
    if (a.pos) hipLaunchKernelGGL((rope_norm_fwd_kernel<D, E, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((rope_norm_fwd_kernel<D, E, false>), grid, block, 0, s, a);
  }
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
