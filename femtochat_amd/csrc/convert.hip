// Element-wise dtype conversion and zero fill for the host binding, so that a
// binding needs no GPU code of its own: the reference converts the inputs of
// its tensor-core path at attention_inputs (ext/FemtoChatCUDAExt.jl:229-230)
// and allocates zeroed gradients (zero(...) in its Enzyme rule); a Julia
// binding of this library calls these entry points instead of broadcasting
// on the device.  HBM-bound: 16-byte accesses where the pointers allow.
#include "../../include/femtochat_attn.h"
#include "attn_launch.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>

namespace fc {
namespace {

typedef __bf16 bf16_t;

constexpr int kConvThreads = 256;
constexpr int64_t kMaxBlocks = 8192;

// float32 -> bfloat16, round to nearest even (the hardware conversion).
__global__ __launch_bounds__(kConvThreads) void f32_to_bf16_vec(const float4* __restrict__ src,
                                                                 uint4* __restrict__ dst, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; i < n8; i += (int64_t)gridDim.x * kConvThreads) {
    const float4 a = src[2 * i];
    const float4 b = src[2 * i + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w[k] = (uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16_t>(v[2 * k])) |
             ((uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16_t>(v[2 * k + 1])) << 16);
    dst[i] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// bfloat16 -> float32 (exact).
__global__ __launch_bounds__(kConvThreads) void bf16_to_f32_vec(const uint4* __restrict__ src,
                                                                 float4* __restrict__ dst, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; i < n8; i += (int64_t)gridDim.x * kConvThreads) {
    const uint4 u = src[i];
    dst[2 * i] = make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                             __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
    dst[2 * i + 1] = make_float4(__uint_as_float(u.z << 16), __uint_as_float(u.z & 0xffff0000u),
                                 __uint_as_float(u.w << 16), __uint_as_float(u.w & 0xffff0000u));
  }
}

// Any pair of dtypes, one element per thread (unaligned pointers, tails).
__global__ __launch_bounds__(kConvThreads) void convert_scalar(const void* src, int src_bf16, void* dst,
                                                               int dst_bf16, int64_t begin, int64_t n) {
  for (int64_t i = begin + (int64_t)blockIdx.x * kConvThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kConvThreads) {
    const float v = src_bf16 ? __uint_as_float((uint32_t)static_cast<const unsigned short*>(src)[i] << 16)
                             : static_cast<const float*>(src)[i];
    if (dst_bf16) static_cast<bf16_t*>(dst)[i] = static_cast<bf16_t>(v);
    else static_cast<float*>(dst)[i] = v;
  }
}

__global__ __launch_bounds__(kConvThreads) void zero_vec(uint4* dst, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; i < n16; i += (int64_t)gridDim.x * kConvThreads)
    dst[i] = make_uint4(0u, 0u, 0u, 0u);
}

__global__ __launch_bounds__(kConvThreads) void zero_bytes(unsigned char* dst, int64_t begin, int64_t n) {
  for (int64_t i = begin + (int64_t)blockIdx.x * kConvThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kConvThreads)
    dst[i] = 0;
}

unsigned blocks_for(int64_t items) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>((items + kConvThreads - 1) / kConvThreads, kMaxBlocks));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Rows of src_cols values copied into rows of dst_cols values (eight per
// thread; both counts are multiples of 16): columns past src_cols become
// zero, columns past dst_cols are dropped; with accumulate the destination's
// values are added in fp32 before the one rounding.  Pads a head dim to a
// compiled width and drops the padding again (attn_api.hip).
template <typename S, typename T>
__global__ __launch_bounds__(kConvThreads) void repack_rows(const S* __restrict__ src, T* __restrict__ dst,
                                                            int64_t rows, int src_cols, int dst_cols, int accumulate) {
  const int groups = dst_cols / 8;
  const int64_t n = rows * groups;
  for (int64_t i = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kConvThreads) {
    const int64_t row = i / groups;
    const int c0 = 8 * (int)(i - row * groups);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = c0 < src_cols ? static_cast<float>(src[row * src_cols + c0 + e]) : 0.0f;
    T* d = dst + row * dst_cols + c0;
    if (accumulate) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] += static_cast<float>(d[e]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] = static_cast<T>(v[e]);
  }
}

}  // namespace

hipError_t launch_repack(const RepackArgs& a, hipStream_t s) {
  const int64_t items = a.rows * (a.dst_cols / 8);
  const dim3 grid(blocks_for(items)), block(kConvThreads);
  if (a.src_bf16 && a.dst_bf16)
    hipLaunchKernelGGL((repack_rows<bf16_t, bf16_t>), grid, block, 0, s, static_cast<const bf16_t*>(a.src),
                       static_cast<bf16_t*>(a.dst), a.rows, a.src_cols, a.dst_cols, a.accumulate);
  else if (a.src_bf16)
    hipLaunchKernelGGL((repack_rows<bf16_t, float>), grid, block, 0, s, static_cast<const bf16_t*>(a.src),
                       static_cast<float*>(a.dst), a.rows, a.src_cols, a.dst_cols, a.accumulate);
  else if (a.dst_bf16)
    hipLaunchKernelGGL((repack_rows<float, bf16_t>), grid, block, 0, s, static_cast<const float*>(a.src),
                       static_cast<bf16_t*>(a.dst), a.rows, a.src_cols, a.dst_cols, a.accumulate);
  else
    hipLaunchKernelGGL((repack_rows<float, float>), grid, block, 0, s, static_cast<const float*>(a.src),
                       static_cast<float*>(a.dst), a.rows, a.src_cols, a.dst_cols, a.accumulate);
  return hipGetLastError();
}

}  // namespace fc

extern "C" {

fc_status fc_convert(const void* src, int32_t src_dtype, void* dst, int32_t dst_dtype, int64_t n, void* stream) {
  if (!fc::valid_dtype(src_dtype) || !fc::valid_dtype(dst_dtype))
    return fc::set_error(FC_ERR_INVALID_ARGUMENT, "fc_convert: dtypes must be FC_F32 or FC_BF16");
  if (n < 0) return fc::set_error(FC_ERR_INVALID_ARGUMENT, "fc_convert: n is negative");
  if (n == 0) {
    fc::clear_error();
    return FC_OK;
  }
  if (src == nullptr || dst == nullptr) return fc::set_error(FC_ERR_INVALID_ARGUMENT, "fc_convert: a pointer is null");
  const size_t esrc = src_dtype == FC_BF16 ? 2 : 4, edst = dst_dtype == FC_BF16 ? 2 : 4;
  if ((reinterpret_cast<uintptr_t>(src) & (esrc - 1)) != 0 || (reinterpret_cast<uintptr_t>(dst) & (edst - 1)) != 0)
    return fc::set_error(FC_ERR_INVALID_ARGUMENT, "fc_convert: pointers must be aligned to their element size");
  // The kernels read and write through restrict pointers: a thread may write
  // bytes that another is still to read unless each element maps onto itself.
  const uintptr_t s0 = reinterpret_cast<uintptr_t>(src), d0 = reinterpret_cast<uintptr_t>(dst);
  const bool overlap = s0 < d0 + (uintptr_t)n * edst && d0 < s0 + (uintptr_t)n * esrc;
  if (overlap && !(s0 == d0 && src_dtype == dst_dtype))
    return fc::set_error(FC_ERR_INVALID_ARGUMENT,
                         "fc_convert: source and destination overlap (allowed only when equal with equal dtypes)");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const fc::ProfileMark mk = fc::profile_begin(s);
  int64_t done = 0;
  if (src_dtype != dst_dtype && fc::aligned16(src) && fc::aligned16(dst)) {
    const int64_t n8 = n / 8;
    if (n8 > 0) {
      if (src_dtype == FC_F32)
        hipLaunchKernelGGL(fc::f32_to_bf16_vec, dim3(fc::blocks_for(n8)), dim3(fc::kConvThreads), 0, s,
                           static_cast<const float4*>(src), static_cast<uint4*>(dst), n8);
      else
        hipLaunchKernelGGL(fc::bf16_to_f32_vec, dim3(fc::blocks_for(n8)), dim3(fc::kConvThreads), 0, s,
                           static_cast<const uint4*>(src), static_cast<float4*>(dst), n8);
    }
    done = 8 * n8;
  }
  if (done < n)
    hipLaunchKernelGGL(fc::convert_scalar, dim3(fc::blocks_for(n - done)), dim3(fc::kConvThreads), 0, s, src,
                       src_dtype == FC_BF16 ? 1 : 0, dst, dst_dtype == FC_BF16 ? 1 : 0, done, n);
  const hipError_t e = hipGetLastError();
  fc::profile_end(mk, "convert", s);
  if (e != hipSuccess) return fc::set_error(FC_ERR_HIP, "fc_convert: launch failed");
  fc::clear_error();
  return FC_OK;
}

fc_status fc_fill_zero(void* dst, size_t bytes, void* stream) {
  if (bytes == 0) {
    fc::clear_error();
    return FC_OK;
  }
  if (dst == nullptr) return fc::set_error(FC_ERR_INVALID_ARGUMENT, "fc_fill_zero: dst is null");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const fc::ProfileMark mk = fc::profile_begin(s);
  unsigned char* p = static_cast<unsigned char*>(dst);
  // Unaligned head, 16-byte body, tail.
  const int64_t head = std::min<int64_t>((int64_t)bytes, (int64_t)((16 - (reinterpret_cast<uintptr_t>(p) & 15)) & 15));
  const int64_t n16 = ((int64_t)bytes - head) / 16;
  if (head > 0) hipLaunchKernelGGL(fc::zero_bytes, dim3(1), dim3(fc::kConvThreads), 0, s, p, (int64_t)0, head);
  if (n16 > 0)
    hipLaunchKernelGGL(fc::zero_vec, dim3(fc::blocks_for(n16)), dim3(fc::kConvThreads), 0, s,
                       reinterpret_cast<uint4*>(p + head), n16);
  const int64_t tail0 = head + 16 * n16;
  if (tail0 < (int64_t)bytes)
    hipLaunchKernelGGL(fc::zero_bytes, dim3(1), dim3(fc::kConvThreads), 0, s, p, tail0, (int64_t)bytes);
  const hipError_t e = hipGetLastError();
  fc::profile_end(mk, "fill_zero", s);
  if (e != hipSuccess) return fc::set_error(FC_ERR_HIP, "fc_fill_zero: launch failed");
  fc::clear_error();
  return FC_OK;
}

}  // extern "C"
