// Optimizer kernels (gfx950) and their C ABI (include/femtochat_optim.h).
//
// Elementwise updates follow the reference's operation order in fp32 without
// contraction (Julia does not fuse multiply-adds), so they agree bit for bit
// with a float32 restatement: the AdamW step (src/optim.jl:32-38,82-94), the
// CUDA final writes (ext/FemtoChatCUDAExt.jl:99-119) and the parameter
// gather/scatter (src/optim.jl:262-276).  All are HBM-bound: 16-byte
// accesses where the sizes allow, a scalar tail otherwise.
//
// Polar Express (src/optim.jl:115-149) normalises each matrix by its
// Frobenius norm (a two-stage float64 reduction), copies it into the iteration
// buffer (transposed through LDS when m > n, so the Gram matrix is the
// smaller one) and runs three batched products per step with the elementwise
// terms folded into their beta: in bf16, for sizes that are multiples of 128,
// the MFMA kernel below (whose last product writes the result), otherwise
// strided-batched rocBLAS GEMMs followed by a copy back.
#include "../../include/femtochat_optim.h"
#include "attn_launch.hpp"
#include "attn_device.hpp"
#include "attn_fast.hpp"

#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <type_traits>
#include <utility>

#pragma clang fp contract(off)

namespace fc {
namespace {

fc_status failf(fc_status code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
fc_status failf(fc_status code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return set_error(code, buf);
}

fc_status launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return failf(FC_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
  clear_error();
  return FC_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

unsigned grid_for(int64_t items, int per_block = 256, int64_t cap = 65536) {
  const int64_t b = (items + per_block - 1) / per_block;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(b, cap));
}

// Julia's Float32 ^ Int (t >= 1): x*x*x in Float32 for t = 3, otherwise
// square-and-multiply in Float64 rounded to Float32.
float julia_pow(float x, int t) {
  if (t == 3) return (x * x) * x;
  double y = 1.0, b = (double)x;
  bool first = true;
  for (int p = t; p > 0; p >>= 1) {
    if (p & 1) {
      y = first ? b : y * b;
      first = false;
    }
    if (p > 1) b = b * b;
  }
  return (float)y;
}

// ---- AdamW ----------------------------------------------------------------------
struct AdamScalars {
  float b1, omb1, b2, omb2, decay, c1, c2, alpha, eps, nscale;
};

__device__ inline void adamw_one(float& th, float g, float& m, float& v, const AdamScalars& s) {
  const float gn = g / s.nscale;
  m = s.b1 * m + s.omb1 * gn;
  v = s.b2 * v + s.omb2 * (gn * gn);
  th = th * s.decay;
  th = th - (s.alpha * (m / s.c1)) / (sqrtf(v / s.c2) + s.eps);
}

__global__ __launch_bounds__(256) void adamw_kernel(int64_t n, float* th, const float* g, float* m, float* v,
                                                    AdamScalars s, bool vec) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nv = vec ? n / 4 : 0;
  // Streaming (nontemporal) accesses: every byte is touched once, and
  // keeping it out of the caches' reuse measured 7% faster at 2^26 elements.
  for (int64_t c = i0; c < nv; c += stride) {
    f32x4 T = __builtin_nontemporal_load(reinterpret_cast<f32x4*>(th) + c);
    const f32x4 G = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(g) + c);
    f32x4 M = __builtin_nontemporal_load(reinterpret_cast<f32x4*>(m) + c);
    f32x4 Vv = __builtin_nontemporal_load(reinterpret_cast<f32x4*>(v) + c);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float t = T[k], mm = M[k], vv = Vv[k];
      adamw_one(t, G[k], mm, vv, s);
      T[k] = t;
      M[k] = mm;
      Vv[k] = vv;
    }
    __builtin_nontemporal_store(T, reinterpret_cast<f32x4*>(th) + c);
    __builtin_nontemporal_store(M, reinterpret_cast<f32x4*>(m) + c);
    __builtin_nontemporal_store(Vv, reinterpret_cast<f32x4*>(v) + c);
  }
  for (int64_t i = 4 * nv + i0; i < n; i += stride) adamw_one(th[i], g[i], m[i], v[i], s);
}

__global__ __launch_bounds__(256) void adam_update_kernel(int64_t n, float* Th, const float* m, const float* v,
                                                          const float* alpha, const float* beta, const float* eta,
                                                          float lambda, float eps) {
  const float a = *alpha, b = *beta, decay = 1.0f - *eta * lambda;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
    Th[i] = Th[i] * decay - (a * m[i]) / (sqrtf(v[i] / b) + eps);
}

// ---- Muon -------------------------------------------------------------------------
__device__ inline float muon_one(float th, float x, float eta, float lambda) {
  // eta x + ((eta lambda) th) * (x th >= 0), where Float32 * false is a zero
  // with the product's sign (Julia's Bool multiplication)
  float decay = (eta * lambda) * th;
  if (!(x * th >= 0.0f)) decay = copysignf(0.0f, decay);
  return th - (eta * x + decay);
}

__global__ __launch_bounds__(256) void muon_kernel(int64_t width, float* Th, const float* X, const float* eta,
                                                   const float* lambda, const int64_t* offsets) {
  const int k = blockIdx.y;
  const float h = *eta, l = *lambda;
  float* t = Th + offsets[k];
  const float* x = X + (int64_t)k * width;
  const int64_t stride = (int64_t)gridDim.x * 256, i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  // 16-byte accesses when this matrix's slices are aligned (uniform per workgroup)
  const int64_t nv = ((reinterpret_cast<uintptr_t>(t) | reinterpret_cast<uintptr_t>(x)) & 15) == 0 ? width / 4 : 0;
  for (int64_t c = i0; c < nv; c += stride) {
    f32x4 T = reinterpret_cast<f32x4*>(t)[c];
    const f32x4 Xv = reinterpret_cast<const f32x4*>(x)[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) T[e] = muon_one(T[e], Xv[e], h, l);
    reinterpret_cast<f32x4*>(t)[c] = T;
  }
  for (int64_t i = 4 * nv + i0; i < width; i += stride) t[i] = muon_one(t[i], x[i], h, l);
}

template <bool kGather>
__global__ __launch_bounds__(256) void param_copy_kernel(int64_t width, float* stack, float* vector,
                                                         const int64_t* offsets) {
  const int k = blockIdx.y;
  float* s = stack + (int64_t)k * width;
  float* v = vector + offsets[k];
  const int64_t stride = (int64_t)gridDim.x * 256, i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nv = ((reinterpret_cast<uintptr_t>(s) | reinterpret_cast<uintptr_t>(v)) & 15) == 0 ? width / 4 : 0;
  for (int64_t c = i0; c < nv; c += stride) {
    if (kGather) reinterpret_cast<f32x4*>(s)[c] = reinterpret_cast<const f32x4*>(v)[c];
    else reinterpret_cast<f32x4*>(v)[c] = reinterpret_cast<const f32x4*>(s)[c];
  }
  for (int64_t i = 4 * nv + i0; i < width; i += stride) {
    if (kGather) s[i] = v[i];
    else v[i] = s[i];
  }
}

// ---- Polar Express -------------------------------------------------------------------
// scale[k] = 1.01 sqrt(sum G_k^2) + 1e-6, summed in float64 in two stages:
// kNormParts workgroups per matrix write partial sums, which the copy into
// the iteration buffer adds in a fixed order (one wave's butterfly, the same
// in every workgroup): deterministic.
constexpr int kNormParts = 64;

__global__ __launch_bounds__(256) void norm_partial_kernel(int64_t size, const float* G, double* partial) {
  __shared__ double part[4];
  const int k = blockIdx.y;
  const float* g = G + (int64_t)k * size;
  const int64_t stride = (int64_t)kNormParts * 256, i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  // 16-byte loads when the matrix is 16-byte aligned (uniform per workgroup),
  // four loads in flight per thread; a fixed order either way
  const int64_t nv = (reinterpret_cast<uintptr_t>(g) & 15) == 0 ? size / 4 : 0;
  double s = 0.0;
  int64_t c = i0;
  for (; c + 3 * stride < nv; c += 4 * stride) {
    f32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = reinterpret_cast<const f32x4*>(g)[c + u * stride];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) s += (double)v[u][e] * (double)v[u][e];
  }
  for (; c < nv; c += stride) {
    const f32x4 v = reinterpret_cast<const f32x4*>(g)[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) s += (double)v[e] * (double)v[e];
  }
  for (int64_t i = 4 * nv + i0; i < size; i += stride) s += (double)g[i] * (double)g[i];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x / 64] = s;
  __syncthreads();
  if (threadIdx.x == 0) partial[k * kNormParts + blockIdx.x] = ((part[0] + part[1]) + part[2]) + part[3];
}


// dst (rows R, cols C, column-major) = src^T / scale (src: C rows, R cols) or
// src / scale, per matrix (blockIdx.z), through a 32x32 LDS tile; the value
// is computed in fp32 and rounded once to the destination type.
template <typename S>
__device__ inline float ld(const S* p) { return static_cast<float>(*p); }
template <typename T>
__device__ inline void st(T* p, float v) { *p = static_cast<T>(v); }

template <bool kTranspose, typename S, typename T>
__global__ __launch_bounds__(256) void copy_scaled_kernel(int R, int C, const S* src, T* dst, const double* partial,
                                                          float* scale_out) {
  // with partial sums: divide by this matrix's scale (also stored once)
  __shared__ float s_scale;
  float sc = 1.0f;
  if (partial != nullptr) {
    if (threadIdx.x < 64) {
      double v = partial[blockIdx.z * kNormParts + threadIdx.x];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
      if (threadIdx.x == 0) {
        s_scale = 1.01f * sqrtf((float)v) + 1e-6f;
        if (blockIdx.x == 0 && blockIdx.y == 0) scale_out[blockIdx.z] = s_scale;
      }
    }
    __syncthreads();
    sc = s_scale;
  }
  __shared__ float tile[32][33];
  const int64_t mat = (int64_t)R * C;
  const S* s = src + blockIdx.z * mat;
  T* d = dst + blockIdx.z * mat;
  const int r0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x / 32;  // 32 x 8
  if (kTranspose) {
    // d(r, c) = s(c, r): load s's columns r0.. (contiguous in c), store d's columns c0.. (contiguous in r)
    for (int j = ty; j < 32; j += 8) {
      const int r = r0 + j, c = c0 + tx;
      if (r < R && c < C) tile[j][tx] = ld(s + (int64_t)r * C + c);
    }
    __syncthreads();
    for (int j = ty; j < 32; j += 8) {
      const int c = c0 + j, r = r0 + tx;
      if (r < R && c < C) st(d + (int64_t)c * R + r, partial ? tile[tx][j] / sc : tile[tx][j]);
    }
  } else {
    for (int j = ty; j < 32; j += 8) {
      const int c = c0 + j, r = r0 + tx;
      if (r < R && c < C) {
        const float v = ld(s + (int64_t)c * R + r);
        st(d + (int64_t)c * R + r, partial ? v / sc : v);
      }
    }
  }
}

// ---- bf16 batched GEMM of the Polar Express iteration ------------------------------
// D(i, j) = alpha sum_k P(i, k) Q(k, j) + beta C(i, j), per matrix of a strided
// batch, bf16 operands, fp32 accumulation, one rounding to bf16 at the store.
//   kTr:  P(i, k) at P[k ldp + i], Q(k, j) at Q[k ldq + j]  (contiguous in i, j)
//   else: P(i, k) at P[i ldp + k], Q(k, j) at Q[j ldq + k]  (contiguous in k)
//   C, D  column-major M x N (leading dimension M)
// A workgroup of four waves computes a 128 x 128 tile of D, each wave 64 x 64
// as 2 x 2 blocks of v_mfma_f32_32x32x16_bf16 (128 x 64 and 64 x 32, 2 x 1
// blocks, for grids that would leave CUs idle).  The k loop runs in steps of
// 64 through kStages LDS stages filled by direct global->LDS loads (two, at
// two workgroups per CU; three, at one, when the grid leaves CUs free): the
// next kStages - 1 steps' loads are in flight while a step's products run,
// with one barrier per step.  The fragment reads of each 16-wide chunk are
// issued ahead of the previous chunk's products.  Tiles:
//   * kTr: k-major tiles (64 rows of k, 128 values of i or j, 256 B per row,
//     the 16-byte units of row r XOR-swizzled by 4(r mod 4) + (r/4 mod 4)),
//     read with ds_read_b64_tr_b16, four k of one column per 8-byte read;
//   * otherwise i- and j-major tiles (128 rows, 64 k, 128 B per row, units
//     swizzled by (r/2) mod 8), one 16-byte read per fragment (the transposed
//     reads take about twice as long for the same bytes).
// Both reads are free of bank conflicts and give lane l (g = l/32) the column
// l mod 32 and k = 8g + e, e < 8, so P and Q fragments pair in the MFMA.
// The epilogue leaves through LDS: each wave writes its fp32 quadrant by
// column (padded), then eight lanes cover one 128-byte column segment of D,
// adding beta C (loaded in that layout before the k loop) and rounding once.
// M, N multiples of 128, K a multiple of 64, every operand under 2^31 bytes
// (checked by the caller): all tiles are whole and every offset is 32-bit.
struct PolarGemm {
  const bf16* P;
  const bf16* Q;
  const bf16* C;
  bf16* D;
  int64_t sp, sq, sd;  // batch strides (elements); C has D's
  int ldp, ldq;
  int M, N, K;
  float alpha, beta;
  // gmode 1: instead of D, G[j M + i] = D(i, j) widened to fp32; gmode 2:
  // G[i N + j] = D(i, j) (the transpose), both per matrix of M N floats
  float* G = nullptr;
  int gmode = 0;
};

constexpr int kGemmTile = 128, kGemmK = 64;
// epilogue quadrant: 64 columns of 64 fp32, padded to 272 bytes (conflict-free
// 16-byte writes by column and reads by row group)
constexpr int kQuadPitch = 272, kQuadBytes = 64 * kQuadPitch;

// Unit swizzles of LDS tile rows: 16 units (256 B) per row; 8 units read
// along rows (i- or j-major, 16-byte reads); 8 units read across rows
// (k-major narrow tiles, transposed reads), kUPR = -8.
template <int kUPR>
__device__ constexpr int gemm_swz(int r) {
  return kUPR == 16 ? (4 * (r & 3) + ((r >> 2) & 3)) : kUPR == 8 ? ((r >> 1) & 7) : 4 * ((r >> 1) & 1);
}

// Per-lane global byte offsets of one wave's share of a tile's DMA: kRows
// rows of |kUPR| 16-byte units, 1 KB blocks, block b filled by wave b mod 4;
// lane l of block b writes physical unit 64 b + l.
template <int kUPR, int kRowsT = 1024 / (kUPR < 0 ? -kUPR : kUPR)>
struct GemmDma {
  static constexpr int kUnits = kUPR < 0 ? -kUPR : kUPR;
  static constexpr int kRows = kRowsT;  // 16 KB tiles by default
  static constexpr int kPer = kRows * kUnits / 64 / kWaves;
  int goff[kPer];
  __device__ inline void init(int wave, int lane, int pitch_bytes) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int unit = 64 * (wave + kWaves * j) + lane;
      const int row = unit / kUnits, pu = unit % kUnits;
      goff[j] = row * pitch_bytes + 16 * (pu ^ gemm_swz<kUPR>(row));
    }
  }
  __device__ inline void issue(u32x4s words, int tile_off, uint32_t lds, int wave) const {
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      dma_load16(words, goff[j] + tile_off, __builtin_amdgcn_readfirstlane(lds + 1024 * (wave + kWaves * j)));
  }
};

// Waits until at most N of this wave's global loads (LDS-DMA included) are
// outstanding (gfx9 s_waitcnt: vmcnt in bits 3:0 and 15:14; expcnt and
// lgkmcnt left at their maxima, i.e. not waited for).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// kNarrow (when 128 x 128 tiles would not fill the CUs): 128 x 64 tiles,
// each wave 64 x 32 (2 x 1 blocks); the Q tile is 64 rows by 64 values (128 B
// per row; k-major, its units are swizzled by 4 ((r/2) mod 2), which keeps
// its transposed reads free of bank conflicts).
template <bool kTr, int kStages, bool kNarrow = false>
__global__ __launch_bounds__(256, kStages == 2 ? 2 : 1) void polar_gemm_kernel(PolarGemm a) {
  constexpr int kTN = kNarrow ? 64 : kGemmTile;  // tile width (j)
  constexpr int kNY = kTN / 64;                   // 32-column blocks per wave
  constexpr int kQBytes = kNarrow ? 8192 : 16384;
  constexpr int kStageBytes = 16384 + kQBytes;
  // kStages stages of [P, Q] tiles; after the k loop, each wave's 64 x 32 kNY
  // fp32 quadrant (columns of kQuadPitch bytes)
  constexpr int kLds = kStageBytes * kStages > 4 * kQuadBytes ? kStageBytes * kStages : 4 * kQuadBytes;
  __shared__ __attribute__((aligned(1024))) char lds[kLds];
  auto tile = [&](int stage, int which) __attribute__((always_inline)) { return lds + kStageBytes * stage + 16384 * which; };
  const int tm = a.M / kGemmTile, tiles = tm * (a.N / kTN);
  // XCD-aware order: workgroup w runs on XCD w mod 8, so the eight XCDs take
  // contiguous runs of tiles (whole matrices, sharing operands in their L2)
  int w = blockIdx.x;
  if ((gridDim.x & 7) == 0) w = (w & 7) * (gridDim.x >> 3) + (w >> 3);
  const int b = w / tiles, t = w - b * tiles;
  const int i0 = (t % tm) * kGemmTile, j0 = (t / tm) * kTN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wi = wave & 1, wj = wave >> 1, l32 = lane & 31, g = lane >> 5;

  const u32x4s pw = buffer_words(a.P + b * a.sp, (uint32_t)((int64_t)(kTr ? a.K : a.M) * a.ldp * 2));
  const u32x4s qw = buffer_words(a.Q + b * a.sq, (uint32_t)((int64_t)(kTr ? a.K : a.N) * a.ldq * 2));
  using Dma = GemmDma<kTr ? 16 : 8>;
  Dma pdma;
  pdma.init(wave, lane, 2 * a.ldp);
  using QDma = typename std::conditional<kNarrow, GemmDma<kTr ? -8 : 8, 64>, Dma>::type;
  QDma qdma;
  qdma.init(wave, lane, 2 * a.ldq);
  // tile origin of k step s: rows 64s, columns i0 (P) or j0 (Q) when kTr,
  // else rows i0 or j0, columns 64s
  auto issue = [&](int s, int stage) __attribute__((always_inline)) {
    pdma.issue(pw, kTr ? 2 * (kGemmK * s * a.ldp + i0) : 2 * (i0 * a.ldp + kGemmK * s), lds_addr(tile(stage, 0)), wave);
    qdma.issue(qw, kTr ? 2 * (kGemmK * s * a.ldq + j0) : 2 * (j0 * a.ldq + kGemmK * s), lds_addr(tile(stage, 1)), wave);
  };

  // fragment offsets: k-major tiles (rows 8g + 4e + a, a = (lane mod 16)/4,
  // column 16 ((lane/16) mod 2) + 4 (lane mod 4), +64 B per 32-column block)
  int tr[2], trn[2];  // 256-byte rows (P, wide Q); 128-byte rows (narrow Q, wave's block 4 wj units in)
  {
    const int s = lane & 15, ar = s >> 2, cc = s & 3, u = 2 * ((lane >> 4) & 1) + (cc >> 1);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int r = 8 * g + 4 * e + ar;
      tr[e] = 256 * r + 16 * (u ^ gemm_swz<16>(r)) + 8 * (cc & 1);
      trn[e] = 128 * r + 16 * ((4 * wj + u) ^ (4 * ((r >> 1) & 1))) + 8 * (cc & 1);
    }
  }
  // i- or j-major tiles: row 64 wi + 32 x + l32 (P) or 64 wj + 32 y + l32 (Q),
  // unit 2c + g (chunk c is ^ 32c)
  const int nat = l32 * 128 + 16 * (g ^ gemm_swz<8>(l32));
  const int natp = nat + 64 * 128 * wi, natq = nat + 32 * kNY * 128 * wj;

  f32x16 acc[2][kNY];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < kNY; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[x][y][r] = 0.0f;

  // The output leaves through LDS: lane l of a wave owns, in pass t < 8, column
  // 8t + l/8 of its quadrant, rows 8 (l mod 8) .. +7 (16 bytes of bf16), so
  // eight lanes write one whole 128-byte column segment.  C is loaded in the
  // same layout before the k loop (its loads complete under the first wait).
  const int64_t dbytes = (int64_t)a.M * a.N * 2;
  const auto rd = make_rsrc(a.D + b * a.sd, (uint32_t)dbytes);
  const bool has_c = a.beta != 0.0f;  // without C the loads read zero records: no memory access
  const auto rc = make_rsrc(has_c ? a.C + b * a.sd : a.D, has_c ? (uint32_t)dbytes : 0u);
  const auto rg = make_rsrc(a.gmode != 0 ? static_cast<const void*>(a.G + b * (int64_t)a.M * a.N) : a.D, a.gmode != 0 ? (uint32_t)(2 * dbytes) : 0u);
  const int orow = 64 * wi + 8 * (lane & 7), ocol = 32 * kNY * wj + (lane >> 3);
  auto out_off = [&](int t) __attribute__((always_inline)) { return 2 * ((j0 + ocol + 8 * t) * a.M + i0 + orow); };
  constexpr int kPasses = 4 * kNY;
  u32x4 cw[kPasses];
#pragma unroll
  for (int t = 0; t < kPasses; ++t) cw[t] = __builtin_amdgcn_raw_buffer_load_b128(rc, out_off(t), 0, 0);

  // k steps s .. s + kStages - 2 are in flight while step s is multiplied
  // (each wave issues kDmaPer loads per step); a step's stage is refilled
  // after the barrier that follows every wave's last read of it
  constexpr int kDmaPer = Dma::kPer + QDma::kPer;
  const int steps = a.K / kGemmK;
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s)
    if (s < steps) issue(s, s);
  for (int s = 0; s < steps; ++s) {
    const int stage = s % kStages;
    if (s + kStages - 2 < steps) wait_vmcnt<kDmaPer * (kStages - 2)>();
    else wait_vmcnt<0>();
    __syncthreads();
    if (s + kStages - 1 < steps) issue(s + kStages - 1, (s + kStages - 1) % kStages);
    const char* pt = tile(stage, 0);
    const char* qt = tile(stage, 1);
    // fragments of chunk c + 1 are read while chunk c's products run
    bf16x8 pf[2][2], qf[2][kNY];
    auto read = [&](int c, bf16x8* p, bf16x8* q) __attribute__((always_inline)) {
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        if (kTr) {
          const int blk = 128 * wi + 64 * x;
          p[x] = lds_tr_frag(pt, (tr[0] + 4096 * c) ^ blk, (tr[1] + 4096 * c) ^ blk);
        } else {
          p[x] = as_bf16x8(lds_load16(pt, (natp + 4096 * x) ^ (32 * c)));
        }
      }
#pragma unroll
      for (int y = 0; y < kNY; ++y) {
        if (kTr && kNarrow) {
          q[y] = lds_tr_frag(qt, trn[0] + 2048 * c, trn[1] + 2048 * c);
        } else if (kTr) {
          const int blk = 128 * wj + 64 * y;
          q[y] = lds_tr_frag(qt, (tr[0] + 4096 * c) ^ blk, (tr[1] + 4096 * c) ^ blk);
        } else {
          q[y] = as_bf16x8(lds_load16(qt, (natq + 4096 * y) ^ (32 * c)));
        }
      }
    };
    read(0, pf[0], qf[0]);
#pragma unroll
    for (int c = 0; c < kGemmK / 16; ++c) {
      if (c + 1 < kGemmK / 16) read(c + 1, pf[(c + 1) & 1], qf[(c + 1) & 1]);
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < kNY; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf[c & 1][x], qf[c & 1][y], acc[x][y], 0, 0, 0);
    }
    // keep that order through scheduling: LDS reads of chunk c + 1 ahead of
    // the products of chunk c (masks: 0x100 LDS read, 0x008 MFMA)
    constexpr int kReads = kTr ? 4 + 2 * kNY : 2 + kNY;
    __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);
#pragma unroll
    for (int c = 0; c < kGemmK / 16 - 1; ++c) {
      __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * kNY, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * kNY, 0);
  }
  __syncthreads();  // every wave's last reads of the stages precede the quadrant writes

  // accumulators -> the wave's quadrant in LDS: lane l holds column l32 of
  // each block and rows 8q + 4g + 0..3 (q < 4), one 16-byte write each
  char* quad = lds + wave * kQuadBytes;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < kNY; ++y)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = a.alpha * acc[x][y][4 * q + e];
        *reinterpret_cast<f32x4*>(quad + (32 * y + l32) * kQuadPitch + 4 * (32 * x + 8 * q + 4 * g)) = v;
      }
  __syncthreads();
  auto pack = [](float x, float y) __attribute__((always_inline)) {
    return (uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16>(x)) |
           ((uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16>(y)) << 16);
  };
#pragma unroll
  for (int t = 0; t < kPasses; ++t) {
    const char* src = quad + (8 * t + (lane >> 3)) * kQuadPitch + 32 * (lane & 7);
    const f32x4 lo4 = *reinterpret_cast<const f32x4*>(src), hi4 = *reinterpret_cast<const f32x4*>(src + 16);
    float v[8] = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
    if (has_c) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] += a.beta * __uint_as_float(cw[t][e] << 16);
        v[2 * e + 1] += a.beta * __uint_as_float(cw[t][e] & 0xffff0000u);
      }
    }
    if (a.gmode == 0) {
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{pack(v[0], v[1]), pack(v[2], v[3]), pack(v[4], v[5]), pack(v[6], v[7])},
                                             rd, out_off(t), 0, 0);
      continue;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = static_cast<float>(static_cast<bf16>(v[e]));  // the bf16 iterate, widened
    if (a.gmode == 1) {
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])},
                                             rg, 2 * out_off(t), 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])},
                                             rg, 2 * out_off(t) + 16, 0, 0);
    } else {  // back into the quadrant, for the transposed pass
      *reinterpret_cast<f32x4*>(const_cast<char*>(src)) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4*>(const_cast<char*>(src) + 16) = f32x4{v[4], v[5], v[6], v[7]};
    }
  }
  if (a.gmode == 2) {
    // lane l, pass t: quadrant row (64/kLpr) t + l/kLpr, columns 8 (l mod kLpr)
    // .. +7, i.e. 32 contiguous bytes of a row of G^T (kLpr lanes: one row
    // segment of the quadrant's width)
    __syncthreads();
    constexpr int kLpr = 4 * kNY;
    const int c0 = 8 * (lane % kLpr);
#pragma unroll
    for (int t = 0; t < kPasses; ++t) {
      const int r = (64 / kLpr) * t + lane / kLpr;
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = *reinterpret_cast<const float*>(quad + (c0 + e) * kQuadPitch + 4 * r);
      const int goff = 4 * ((i0 + 64 * wi + r) * a.N + j0 + 32 * kNY * wj + c0);
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])},
                                             rg, goff, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])},
                                             rg, goff + 16, 0, 0);
    }
  }
}

// True when the Polar Express products of these sizes fit polar_gemm_kernel.
bool polar_gemm_fits(int lo, int hi) {
  return lo % kGemmTile == 0 && hi % kGemmTile == 0 && (int64_t)lo * hi * 4 < ((int64_t)1 << 31);
}

// Compute units of the current device (cached per device).
int cu_count() {
  static int cus[16] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  int& c = cus[dev & 15];
  if (c == 0 && hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) c = 256;
  return c;
}

// Two stages (two workgroups per CU) when the grid fills the GPU twice over,
// otherwise three (one workgroup per CU, two k steps in flight); products
// whose 128 x 128 grid would leave CUs idle take 128 x 64 tiles.
void polar_gemm(bool tr, const PolarGemm& a, int batch, hipStream_t s, int cus) {
  const int64_t grid = (int64_t)(a.M / kGemmTile) * (a.N / kGemmTile) * batch;
  const bool deep = grid < 2 * (int64_t)cus;
  const dim3 g((unsigned)grid), b(256);
  if (grid < (int64_t)cus) {
    if (tr) hipLaunchKernelGGL((polar_gemm_kernel<true, 3, true>), dim3((unsigned)(2 * grid)), b, 0, s, a);
    else hipLaunchKernelGGL((polar_gemm_kernel<false, 3, true>), dim3((unsigned)(2 * grid)), b, 0, s, a);
  } else if (tr && deep) hipLaunchKernelGGL((polar_gemm_kernel<true, 3>), g, b, 0, s, a);
  else if (tr) hipLaunchKernelGGL((polar_gemm_kernel<true, 2>), g, b, 0, s, a);
  else if (deep) hipLaunchKernelGGL((polar_gemm_kernel<false, 3>), g, b, 0, s, a);
  else hipLaunchKernelGGL((polar_gemm_kernel<false, 2>), g, b, 0, s, a);
}

// The untransposed copy in (m <= n: X has G's layout): X = G / scale per
// matrix (blockIdx.y), 16-byte loads, the scale from the partial sums as in
// copy_scaled_kernel.  Needs size % 4 == 0 and 16-byte aligned G and X.
template <typename T>
__global__ __launch_bounds__(256) void scale_copy_kernel(int64_t size, const float* G, T* X, const double* partial,
                                                         float* scale_out) {
  __shared__ float s_scale;
  if (threadIdx.x < 64) {
    double v = partial[blockIdx.y * kNormParts + threadIdx.x];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    if (threadIdx.x == 0) {
      s_scale = 1.01f * sqrtf((float)v) + 1e-6f;
      if (blockIdx.x == 0) scale_out[blockIdx.y] = s_scale;
    }
  }
  __syncthreads();
  const float sc = s_scale;
  const f32x4* g = reinterpret_cast<const f32x4*>(G + blockIdx.y * size);
  T* x = X + blockIdx.y * size;
  const int64_t n4 = size / 4, stride = (int64_t)gridDim.x * 256;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < n4; c += stride) {
    const f32x4 v = __builtin_nontemporal_load(g + c);
    if constexpr (sizeof(T) == 2) {
      typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
      bf16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = static_cast<bf16>(v[e] / sc);
      *reinterpret_cast<bf16x4*>(x + 4 * c) = o;
    } else {
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = v[e] / sc;
      *reinterpret_cast<f32x4*>(x + 4 * c) = o;
    }
  }
}

struct PolarLayout {
  size_t X, Y, A, B, scale, partial, total;
};

PolarLayout polar_layout(const fc_polar_desc& d) {
  const size_t lo = std::min(d.m, d.n), hi = std::max(d.m, d.n), k = d.count;
  const size_t e = d.dtype == FC_BF16 ? 2 : 4;  // element size of the iteration buffers
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  PolarLayout L{};
  L.X = 0;
  L.Y = L.X + up(lo * hi * k * e);
  L.A = L.Y + up(lo * hi * k * e);
  L.B = L.A + up(lo * lo * k * e);
  L.scale = L.B + up(lo * lo * k * e);
  L.partial = L.scale + up(k * 4);
  L.total = L.partial + up(k * kNormParts * 8);
  return L;
}

// (a, b, c) of each step (src/optim.jl:97-103), as the reference's Float32 literals.
constexpr float kPolar[5][3] = {
    {8.156554524902461f, -22.48329292557795f, 15.878769915207462f},
    {4.042929935166739f, -2.808917465908714f, 0.5000178451051316f},
    {3.8916678022926607f, -2.772484153217685f, 0.5060648178503393f},
    {3.285753657755655f, -2.3681294933425376f, 0.46449024233003106f},
    {2.3465413258596377f, -1.7097828382687081f, 0.42323551169305323f},
};

// One rocBLAS handle per device, created on first use (it allocates its own
// workspace then) and used under a lock.
std::mutex g_blas_mutex;
rocblas_handle g_blas[16] = {};

rocblas_handle blas_handle(int dev) {
  rocblas_handle& h = g_blas[dev & 15];
  if (h == nullptr && rocblas_create_handle(&h) != rocblas_status_success) h = nullptr;
  return h;
}

// D = alpha op(A) op(B) + beta C over a strided batch; operands and results
// of type t (fp32 or bf16), fp32 accumulation and scalars.
// Helper streams for fc_polar_express_grouped: per device, kHelpers streams
// (default priority), each with its own rocBLAS handle (so concurrent GEMMs
// never share rocBLAS's workspace), and the fork/join events; created on
// first use and kept until the process ends.
constexpr int kHelpers = 4;
struct Fork {
  hipStream_t stream[kHelpers];
  rocblas_handle blas[kHelpers];
  hipEvent_t start, done[kHelpers];
};
Fork* g_fork[16] = {};

Fork* fork_for(int dev) {
  Fork*& f = g_fork[dev & 15];
  if (f != nullptr) return f;
  Fork* n = new Fork{};
  bool ok = hipEventCreateWithFlags(&n->start, hipEventDisableTiming) == hipSuccess;
  for (int j = 0; j < kHelpers && ok; ++j) {
    ok = hipStreamCreateWithFlags(&n->stream[j], hipStreamNonBlocking) == hipSuccess &&
         hipEventCreateWithFlags(&n->done[j], hipEventDisableTiming) == hipSuccess &&
         rocblas_create_handle(&n->blas[j]) == rocblas_status_success;
  }
  if (!ok) return nullptr;  // (the partial objects are left to the process end)
  f = n;
  return f;
}

rocblas_status gemm(rocblas_handle h, rocblas_datatype t, rocblas_operation ta, rocblas_operation tb, int m, int n,
                    int k, float alpha, const void* A, int lda, int64_t sa, const void* B, int ldb, int64_t sb,
                    float beta, const void* C, int ldc, int64_t sc, void* D, int batch) {
  return rocblas_gemm_strided_batched_ex(h, ta, tb, m, n, k, &alpha, A, t, lda, sa, B, t, ldb, sb, &beta, C, t, ldc,
                                         sc, D, t, ldc, sc, batch, rocblas_datatype_f32_r,
                                         rocblas_gemm_algo_standard, 0, 0);
}

}  // namespace
}  // namespace fc

using namespace fc;

extern "C" {

fc_status fc_adamw_step(const fc_adamw_desc* d, float* theta, const float* grad, float* m, float* v, void* stream) {
  if (d == nullptr) return failf(FC_ERR_INVALID_ARGUMENT, "fc_adamw_step: descriptor is null");
  if (d->n <= 0 || d->t < 1)
    return failf(FC_ERR_INVALID_ARGUMENT, "fc_adamw_step: n must be positive and t >= 1 (n=%lld t=%d)",
                 (long long)d->n, d->t);
  if (!theta || !grad || !m || !v) return failf(FC_ERR_INVALID_ARGUMENT, "fc_adamw_step: a pointer is null");
  if (((reinterpret_cast<uintptr_t>(theta) | reinterpret_cast<uintptr_t>(grad) | reinterpret_cast<uintptr_t>(m) |
        reinterpret_cast<uintptr_t>(v)) & 3) != 0)
    return failf(FC_ERR_INVALID_ARGUMENT, "fc_adamw_step: arrays must be 4-byte aligned");
  AdamScalars s;
  s.b1 = d->beta1;
  s.omb1 = 1.0f - d->beta1;
  s.b2 = d->beta2;
  s.omb2 = 1.0f - d->beta2;
  s.decay = 1.0f - d->alpha * d->lambda;
  s.c1 = 1.0f - julia_pow(d->beta1, d->t);
  s.c2 = 1.0f - julia_pow(d->beta2, d->t);
  s.alpha = d->alpha;
  s.eps = d->eps;
  s.nscale = d->grad_scale;
  const bool vec = aligned16(theta) && aligned16(grad) && aligned16(m) && aligned16(v);
  hipLaunchKernelGGL(adamw_kernel, dim3(grid_for(vec ? d->n / 4 : d->n)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), d->n, theta, grad, m, v, s, vec);
  return launched("AdamW");
}

fc_status fc_adam_update(int64_t n, int64_t offset, float lambda, float eps, float* Theta, const float* m,
                         const float* v, const float* alpha, const float* beta, const float* eta, void* stream) {
  if (n <= 0 || offset < 0) return failf(FC_ERR_INVALID_ARGUMENT, "fc_adam_update: n must be positive, offset >= 0");
  if (!Theta || !m || !v || !alpha || !beta || !eta)
    return failf(FC_ERR_INVALID_ARGUMENT, "fc_adam_update: a pointer is null");
  hipLaunchKernelGGL(adam_update_kernel, dim3(grid_for(n)), dim3(256), 0, static_cast<hipStream_t>(stream), n,
                     Theta + offset, m, v, alpha, beta, eta, lambda, eps);
  return launched("Adam update");
}

fc_status fc_muon_update(int64_t width, int32_t count, float* Theta, const float* X, const float* eta,
                         const float* lambda, const int64_t* offsets, void* stream) {
  if (width <= 0 || count <= 0 || count > 65535)
    return failf(FC_ERR_INVALID_ARGUMENT, "fc_muon_update: width must be positive and count in [1, 65535]");
  if (!Theta || !X || !eta || !lambda || !offsets) return failf(FC_ERR_INVALID_ARGUMENT, "fc_muon_update: a pointer is null");
  hipLaunchKernelGGL(muon_kernel, dim3(grid_for((width + 3) / 4, 256, 4096), count), dim3(256), 0,
                     static_cast<hipStream_t>(stream), width, Theta, X, eta, lambda, offsets);
  return launched("Muon update");
}

static fc_status param_copy(bool gather, int64_t width, int32_t count, float* stack, float* vector,
                            const int64_t* offsets, void* stream) {
  if (width <= 0 || count <= 0 || count > 65535)
    return failf(FC_ERR_INVALID_ARGUMENT, "parameter copy: width must be positive and count in [1, 65535]");
  if (!stack || !vector || !offsets) return failf(FC_ERR_INVALID_ARGUMENT, "parameter copy: a pointer is null");
  const dim3 grid(grid_for((width + 3) / 4, 256, 4096), count);
  if (gather) hipLaunchKernelGGL(param_copy_kernel<true>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), width, stack, vector, offsets);
  else hipLaunchKernelGGL(param_copy_kernel<false>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), width, stack, vector, offsets);
  return launched(gather ? "gather" : "scatter");
}

fc_status fc_param_gather(int64_t width, int32_t count, float* stack, const float* vector, const int64_t* offsets,
                          void* stream) {
  return param_copy(true, width, count, stack, const_cast<float*>(vector), offsets, stream);
}

fc_status fc_param_scatter(int64_t width, int32_t count, float* vector, const float* stack, const int64_t* offsets,
                           void* stream) {
  return param_copy(false, width, count, const_cast<float*>(stack), vector, offsets, stream);
}

static fc_status polar_check(const fc_polar_desc* d) {
  if (d == nullptr) return failf(FC_ERR_INVALID_ARGUMENT, "polar express: descriptor is null");
  if (d->m <= 0 || d->n <= 0 || d->count <= 0 || d->steps < 0)
    return failf(FC_ERR_INVALID_ARGUMENT, "polar express: sizes must be positive (m=%d n=%d count=%d steps=%d)", d->m,
                 d->n, d->count, d->steps);
  if (d->count > 65535) return failf(FC_ERR_UNSUPPORTED, "polar express: at most 65535 matrices");
  if (d->dtype != FC_F32 && d->dtype != FC_BF16)
    return failf(FC_ERR_INVALID_ARGUMENT, "polar express: dtype must be FC_F32 or FC_BF16");
  return FC_OK;
}

fc_status fc_polar_workspace_bytes(const fc_polar_desc* d, size_t* bytes) {
  const fc_status st = polar_check(d);
  if (st != FC_OK) return st;
  if (bytes == nullptr) return failf(FC_ERR_INVALID_ARGUMENT, "polar express: bytes is null");
  *bytes = polar_layout(*d).total;
  clear_error();
  return FC_OK;
}

// Host-side checks of one stack's call (nothing is launched).
static fc_status polar_args(const fc_polar_desc* d, const float* G, const void* workspace, size_t workspace_bytes) {
  const fc_status st = polar_check(d);
  if (st != FC_OK) return st;
  if (G == nullptr) return failf(FC_ERR_INVALID_ARGUMENT, "polar express: G is null");
  const PolarLayout L = polar_layout(*d);
  if (workspace == nullptr || workspace_bytes < L.total)
    return failf(FC_ERR_WORKSPACE, "polar express needs %zu workspace bytes, got %zu", L.total, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return failf(FC_ERR_WORKSPACE, "polar express: workspace must be 256-byte aligned");
  return FC_OK;
}

// Polar Express of one stack on stream s with the rocBLAS handle h (held by
// the caller under g_blas_mutex).
static fc_status polar_run(const fc_polar_desc* d, float* G, void* workspace, size_t workspace_bytes, hipStream_t s,
                           rocblas_handle h) {
  fc_status st = polar_args(d, G, workspace, workspace_bytes);
  if (st != FC_OK) return st;
  const PolarLayout L = polar_layout(*d);
  char* ws = static_cast<char*>(workspace);
  char* X = ws + L.X;
  char* Y = ws + L.Y;
  char* A = ws + L.A;
  char* B = ws + L.B;
  float* scale = reinterpret_cast<float*>(ws + L.scale);
  double* partial = reinterpret_cast<double*>(ws + L.partial);
  const int m = d->m, n = d->n, k = d->count;
  const bool transposed = m > n, half = d->dtype == FC_BF16;
  const int lo = std::min(m, n), hi = std::max(m, n);
  const int64_t sx = (int64_t)lo * hi, sa = (int64_t)lo * lo;

  hipLaunchKernelGGL(norm_partial_kernel, dim3(kNormParts, k), dim3(256), 0, s, (int64_t)m * n, G, partial);
  if ((st = launched("polar norm")) != FC_OK) return st;
  // X (lo x hi) = G / scale, or G^T / scale, rounded to the compute type
  const dim3 tiles((lo + 31) / 32, (hi + 31) / 32, k), back((hi + 31) / 32, (lo + 31) / 32, k);
  const int64_t msize = (int64_t)m * n;
  const bool flat = !transposed && msize % 4 == 0 && aligned16(G) && aligned16(X);
  const dim3 flat_grid((unsigned)std::min<int64_t>((msize / 4 + 255) / 256, std::max<int64_t>(1, 2048 / k)), k);
  if (flat && half) {
    hipLaunchKernelGGL(scale_copy_kernel<bf16>, flat_grid, dim3(256), 0, s, msize, G, reinterpret_cast<bf16*>(X), partial, scale);
  } else if (flat) {
    hipLaunchKernelGGL(scale_copy_kernel<float>, flat_grid, dim3(256), 0, s, msize, G, reinterpret_cast<float*>(X), partial, scale);
  } else if (half) {
    if (transposed) hipLaunchKernelGGL((copy_scaled_kernel<true, float, bf16>), tiles, dim3(256), 0, s, lo, hi, G, reinterpret_cast<bf16*>(X), partial, scale);
    else hipLaunchKernelGGL((copy_scaled_kernel<false, float, bf16>), tiles, dim3(256), 0, s, lo, hi, G, reinterpret_cast<bf16*>(X), partial, scale);
  } else {
    if (transposed) hipLaunchKernelGGL((copy_scaled_kernel<true, float, float>), tiles, dim3(256), 0, s, lo, hi, G, reinterpret_cast<float*>(X), partial, scale);
    else hipLaunchKernelGGL((copy_scaled_kernel<false, float, float>), tiles, dim3(256), 0, s, lo, hi, G, reinterpret_cast<float*>(X), partial, scale);
  }
  if ((st = launched("polar copy in")) != FC_OK) return st;

  if (half && polar_gemm_fits(lo, hi)) {
    const bf16* none = nullptr;
    const int cus = cu_count();
    for (int i = 0; i < d->steps; ++i) {
      const float* c = kPolar[std::min(i, 4)];
      bf16* x = reinterpret_cast<bf16*>(X);
      bf16* y = reinterpret_cast<bf16*>(Y);
      bf16* a = reinterpret_cast<bf16*>(A);
      bf16* b = reinterpret_cast<bf16*>(B);
      // A = X X^T: P(i, p) = X(i, p), Q(p, j) = X(j, p), both contiguous in i, j
      polar_gemm(true, PolarGemm{x, x, none, a, sx, sx, sa, lo, lo, lo, lo, hi, 1.0f, 0.0f}, k, s, cus);
      // B = c A A + b A: Q(q, j) = A(q, j), contiguous in q; A is symmetric
      // (X X^T), so P(i, q) is read as A(q, i), also contiguous in q
      polar_gemm(false, PolarGemm{a, a, a, b, sa, sa, sa, lo, lo, lo, lo, lo, c[2], c[1]}, k, s, cus);
      // Y = B X + a X: Q(q, p) = X(q, p), contiguous in q; P(i, q) read as
      // B(q, i) (B = c A A + b A is symmetric)
      // (the last step writes G itself: the bf16 iterate widened to fp32, as
      // G = X or X^T)
      const bool last = i + 1 == d->steps;
      polar_gemm(false, PolarGemm{b, x, x, y, sa, sx, sx, lo, lo, lo, hi, lo, 1.0f, c[0], G, last ? (transposed ? 2 : 1) : 0},
                 k, s, cus);
      std::swap(X, Y);
    }
    if ((st = launched("polar express GEMM")) != FC_OK) return st;
    if (d->steps > 0) return FC_OK;
  } else {
    if (rocblas_set_stream(h, s) != rocblas_status_success) return failf(FC_ERR_HIP, "rocblas_set_stream failed");
    const auto N = rocblas_operation_none, T = rocblas_operation_transpose;
    const rocblas_datatype t = half ? rocblas_datatype_bf16_r : rocblas_datatype_f32_r;
    for (int i = 0; i < d->steps; ++i) {
      const float* c = kPolar[std::min(i, 4)];
      rocblas_status r;
      // A = X X^T
      r = gemm(h, t, N, T, lo, lo, hi, 1.0f, X, lo, sx, X, lo, sx, 0.0f, A, lo, sa, A, k);
      // B = c A A + b A
      if (r == rocblas_status_success) r = gemm(h, t, N, N, lo, lo, lo, c[2], A, lo, sa, A, lo, sa, c[1], A, lo, sa, B, k);
      // Y = B X + a X, then X <-> Y
      if (r == rocblas_status_success) r = gemm(h, t, N, N, lo, hi, lo, 1.0f, B, lo, sa, X, lo, sx, c[0], X, lo, sx, Y, k);
      if (r != rocblas_status_success) return failf(FC_ERR_HIP, "polar express: rocBLAS GEMM failed (%d)", (int)r);
      std::swap(X, Y);
    }
  }
  // G = X, or X^T (widened to fp32)
  if (half) {
    if (transposed) hipLaunchKernelGGL((copy_scaled_kernel<true, bf16, float>), back, dim3(256), 0, s, hi, lo, reinterpret_cast<const bf16*>(X), G, nullptr, nullptr);
    else hipLaunchKernelGGL((copy_scaled_kernel<false, bf16, float>), tiles, dim3(256), 0, s, lo, hi, reinterpret_cast<const bf16*>(X), G, nullptr, nullptr);
  } else {
    if (transposed) hipLaunchKernelGGL((copy_scaled_kernel<true, float, float>), back, dim3(256), 0, s, hi, lo, reinterpret_cast<const float*>(X), G, nullptr, nullptr);
    else hipLaunchKernelGGL((copy_scaled_kernel<false, float, float>), tiles, dim3(256), 0, s, lo, hi, reinterpret_cast<const float*>(X), G, nullptr, nullptr);
  }
  return launched("polar copy out");
}

fc_status fc_polar_express(const fc_polar_desc* d, float* G, void* workspace, size_t workspace_bytes, void* stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return failf(FC_ERR_HIP, "polar express: hipGetDevice failed");
  std::lock_guard<std::mutex> lock(g_blas_mutex);
  rocblas_handle h = blas_handle(dev);
  if (h == nullptr) return failf(FC_ERR_HIP, "polar express: rocblas_create_handle failed");
  return polar_run(d, G, workspace, workspace_bytes, static_cast<hipStream_t>(stream), h);
}

fc_status fc_polar_express_grouped(int32_t count, const fc_polar_desc* descs, float* const* G, void* const* workspaces,
                                   const size_t* workspace_bytes, void* stream) {
  if (count <= 0 || descs == nullptr || G == nullptr || workspaces == nullptr || workspace_bytes == nullptr)
    return failf(FC_ERR_INVALID_ARGUMENT, "polar express grouped: count must be positive and the arrays non-null");
  // Every stack is checked before anything is launched, so a rejected call
  // leaves no work behind on the helper streams.
  for (int i = 0; i < count; ++i) {
    const fc_status st = polar_args(&descs[i], G[i], workspaces[i], workspace_bytes[i]);
    if (st != FC_OK) return st;
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return failf(FC_ERR_HIP, "polar express grouped: hipGetDevice failed");
  std::lock_guard<std::mutex> lock(g_blas_mutex);
  Fork* f = fork_for(dev);
  if (f == nullptr) return failf(FC_ERR_HIP, "polar express grouped: helper streams could not be created");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // fork: every helper stream waits for the caller's stream
  if (hipEventRecord(f->start, s) != hipSuccess) return failf(FC_ERR_HIP, "hipEventRecord failed");
  const int used = std::min<int>(count, kHelpers);
  for (int j = 0; j < used; ++j)
    if (hipStreamWaitEvent(f->stream[j], f->start, 0) != hipSuccess) return failf(FC_ERR_HIP, "hipStreamWaitEvent failed");
  fc_status first = FC_OK;
  for (int i = 0; i < count && first == FC_OK; ++i) {
    const int j = i % kHelpers;
    first = polar_run(&descs[i], G[i], workspaces[i], workspace_bytes[i], f->stream[j], f->blas[j]);
  }
  // join, also after a failed launch: the caller's stream waits for every
  // helper stream, so nothing enqueued there outlives the caller's view
  for (int j = 0; j < used; ++j) {
    if ((hipEventRecord(f->done[j], f->stream[j]) != hipSuccess || hipStreamWaitEvent(s, f->done[j], 0) != hipSuccess) &&
        first == FC_OK)
      first = failf(FC_ERR_HIP, "polar express grouped: join failed");
  }
  if (first == FC_OK) clear_error();
  return first;
}

}  // extern "C"
