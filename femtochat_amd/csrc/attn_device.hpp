// Device-side building blocks shared by the attention kernels (gfx950 only).
//
// Matrix products use the 32x32 MFMA family:
//   fast mode : v_mfma_f32_32x32x16_bf16  (one instruction per 16-wide k chunk)
//   exact mode: v_mfma_f32_32x32x2_f32    (eight instructions per 16-wide k chunk)
// A k chunk of 16 is carried per lane as an 8-element fragment.  Lane l
// (g = l/32) holds row/column l%32 of the operand and 8 of the 16 k values.
// The k values a lane group holds only need to agree between the A and the B
// operand of one product, so two k orders are used:
//   natural  : k = 8g + e                       (contiguous, 16-byte reads)
//   acc order: k = 8(e/4) + 4g + e%4            (the row order of a 32x32
//                                                accumulator, so P and dS feed
//                                                the next product directly)
// Accumulator layout (32x32, 16 floats per lane): element r of lane l is
// row 8(r/4) + 4g + r%4, column l%32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_index.hpp"

namespace fc {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kFltMax = 3.402823466e38f;
constexpr float kFltEps = 1.1920928955078125e-7f;  // eps(Float32)

template <typename E> struct Mma;

template <> struct Mma<bf16> {
  using frag = bf16x8;
  static constexpr bool kBF16 = true;
  __device__ static inline f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // 8 contiguous elements (16-byte aligned).
  __device__ static inline frag load8(const bf16* p) { return *reinterpret_cast<const frag*>(p); }
  // Elements [8h, 8h+8) of an accumulator, rounded to bf16 (round to nearest even).
  template <int H>
  __device__ static inline frag from_acc(const f32x16& c) {
    frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = static_cast<bf16>(c[8 * H + e]);
    return f;
  }
  __device__ static inline frag zero() {
    frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = static_cast<bf16>(0.0f);
    return f;
  }
};

template <> struct Mma<float> {
  using frag = f32x8;
  static constexpr bool kBF16 = false;
  __device__ static inline f32x16 mma(frag a, frag b, f32x16 c) {
#pragma unroll
    for (int e = 0; e < 8; ++e) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], b[e], c, 0, 0, 0);
    return c;
  }
  __device__ static inline frag load8(const float* p) {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(p);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(p + 4);
    frag f;
#pragma unroll
    for (int e = 0; e < 4; ++e) { f[e] = lo[e]; f[e + 4] = hi[e]; }
    return f;
  }
  template <int H>
  __device__ static inline frag from_acc(const f32x16& c) {
    frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = c[8 * H + e];
    return f;
  }
  __device__ static inline frag zero() {
    frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = 0.0f;
    return f;
  }
};

__device__ inline f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// Row (within a 32-row block) of accumulator element r for lane group g.
__device__ constexpr int acc_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// Fragment in accumulator k order from a bf16 tile stored transposed
// (row = output column, k contiguous): p points at Xt[col][k0].
__device__ inline bf16x8 load_tr_bf16(const bf16* p, int g) {
  const uint2 lo = *reinterpret_cast<const uint2*>(p + 4 * g);
  const uint2 hi = *reinterpret_cast<const uint2*>(p + 8 + 4 * g);
  uint4 u = make_uint4(lo.x, lo.y, hi.x, hi.y);
  return __builtin_bit_cast(bf16x8, u);
}

// Fragment in accumulator k order from an fp32 tile in natural layout
// (row = k, column contiguous): p points at X[k0][col], ld = row stride.
__device__ inline f32x8 load_kt_f32(const float* p, int ld, int g) {
  f32x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = p[(8 * (e >> 2) + 4 * g + (e & 3)) * ld];
  return f;
}

// Wavefront reductions over the 32 lanes of one half (both halves hold the
// same queries, so reducing within 32 lanes is enough).
__device__ inline int wave_min32(int v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
  return v;
}
__device__ inline int wave_max32(int v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}
__device__ inline int wave_min64(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
  return v;
}
__device__ inline int wave_max64(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}

// Visible key range of query q (0-based): lb <= k <= ub.  left/right are the
// normalised window (causal -> left = T); pos is the row's positions or null.
__device__ inline int key_lb(int q, int T, int left, const int32_t* pos) {
  if (q >= T) return T;
  int lb = q - left;
  if (pos != nullptr) lb = max(lb, q - pos[q]);
  return max(lb, 0);
}
__device__ inline int key_ub(int q, int T, int right) {
  if (q >= T) return -1;
  return min(q + right, T - 1);
}

// Loads a tile of R token rows x D columns of a token-major matrix (row
// pitch in elements) into registers, 4 rows x 16 bytes per task, then writes
// it to LDS in natural layout and/or (bf16 only) transposed layout.
// Rows at or beyond T read as zero.
template <typename E, int D, int R>
struct TileStage {
  static constexpr int kEPC = 16 / sizeof(E);  // elements per 16-byte chunk
  static constexpr int kCPR = D / kEPC;        // chunks per row
  static constexpr int kTasks = (R / 4) * kCPR;
  static constexpr int kPer = (kTasks + kThreads - 1) / kThreads;
  uint4 v[kPer][4];

  __device__ inline void load(const E* base, int64_t pitch, int row0, int T, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int task = tid + i * kThreads;
      if (kTasks % kThreads == 0 || task < kTasks) {
        const int ch = task % kCPR, rq = task / kCPR;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = row0 + 4 * rq + j;
          v[i][j] = row < T ? *reinterpret_cast<const uint4*>(base + (int64_t)row * pitch + ch * kEPC)
                            : make_uint4(0u, 0u, 0u, 0u);
        }
      }
    }
  }

  __device__ inline void store_nat(E* lds, int ld, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int task = tid + i * kThreads;
      if (kTasks % kThreads == 0 || task < kTasks) {
        const int ch = task % kCPR, rq = task / kCPR;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<uint4*>(lds + (4 * rq + j) * ld + ch * kEPC) = v[i][j];
      }
    }
  }

  // Transposed store (bf16): Xt[col][row], row stride ldt elements.
  __device__ inline void store_tr(bf16* lds, int ldt, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int task = tid + i * kThreads;
      if (kTasks % kThreads == 0 || task < kTasks) {
        const int ch = task % kCPR, rq = task / kCPR;
        const uint32_t* r0 = reinterpret_cast<const uint32_t*>(&v[i][0]);
        const uint32_t* r1 = reinterpret_cast<const uint32_t*>(&v[i][1]);
        const uint32_t* r2 = reinterpret_cast<const uint32_t*>(&v[i][2]);
        const uint32_t* r3 = reinterpret_cast<const uint32_t*>(&v[i][3]);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          // column 8ch + 2w (low halves) and 8ch + 2w + 1 (high halves)
          uint2 lo, hi;
          lo.x = (r0[w] & 0xffffu) | (r1[w] << 16);
          lo.y = (r2[w] & 0xffffu) | (r3[w] << 16);
          hi.x = (r0[w] >> 16) | (r1[w] & 0xffff0000u);
          hi.y = (r2[w] >> 16) | (r3[w] & 0xffff0000u);
          *reinterpret_cast<uint2*>(lds + (8 * ch + 2 * w) * ldt + 4 * rq) = lo;
          *reinterpret_cast<uint2*>(lds + (8 * ch + 2 * w + 1) * ldt + 4 * rq) = hi;
        }
      }
    }
  }
};

__device__ inline float to_f32(float x) { return x; }
__device__ inline float to_f32(bf16 x) { return static_cast<float>(x); }

template <typename T> __device__ inline T from_f32(float x);
template <> __device__ inline float from_f32<float>(float x) { return x; }
template <> __device__ inline bf16 from_f32<bf16>(float x) { return static_cast<bf16>(x); }

// Stores 4 consecutive values (optionally adding the existing ones first,
// in fp32, before the single final rounding).
template <typename T>
__device__ inline void store4(T* p, f32x4 v, bool accumulate) {
  if (accumulate) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] += to_f32(p[i]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = from_f32<T>(v[i]);
}

}  // namespace fc
