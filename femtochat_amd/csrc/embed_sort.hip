// Deterministic embedding gradient (gfx950): the tokens are sorted by table
// column (rocPRIM's stable device radix sort over (id, token) pairs), then
// one wave per run of equal ids sums that run's dy rows in token order and
// adds the sum to the column once: no atomics, and the same bits on every
// call.  The reference adds with one atomic per element
// (ext/FemtoChatCUDAExt.jl:78-94, src/kernels.jl:8-14), skipping zero
// values; the sum here skips them too and starts from -0, so a column that
// receives nothing but zeros keeps its bits.
#include "attn_launch.hpp"
#include "attn_device.hpp"

#include <hip/hip_runtime.h>
#include <rocprim/device/device_radix_sort.hpp>

#include <cstdint>

namespace fc {
namespace {

__device__ inline int64_t token_at(const void* p, int64_t i, int type) {
  return type == 1 ? static_cast<const int64_t*>(p)[i] : (int64_t) static_cast<const int32_t*>(p)[i];
}

// key[t] = table column of token t (vocab, which sorts last, for an id
// outside the table), val[t] = t.
__global__ __launch_bounds__(256) void embed_keys_kernel(EmbedArgs a, uint32_t* key, uint32_t* val) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < a.N; t += stride) {
    const int64_t id = token_at(a.tokens, t, a.index_type) - a.index_base;
    key[t] = (id >= 0 && id < a.vocab) ? (uint32_t)id : (uint32_t)a.vocab;
    val[t] = (uint32_t)t;
  }
}

template <typename Y>
__device__ inline float as_float(Y v) { return static_cast<float>(v); }

// One wave per sorted position i; the wave at the head of a run of equal
// ids sums the run (lane d: elements d, d + 64, ... of each dy row, in the
// run's token order) and adds the sums to the column.
template <typename Y>
__global__ __launch_bounds__(256) void embed_runs_kernel(EmbedArgs a, const uint32_t* key, const uint32_t* tok) {
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= a.N) return;
  const int lane = threadIdx.x & 63;
  const uint32_t id = key[i];
  if (id >= (uint32_t)a.vocab || (i > 0 && key[i - 1] == id)) return;  // not a run head, or outside the table
  float* dw = a.dweights + (int64_t)id * a.D;
  const Y* dy = static_cast<const Y*>(a.dy);
  for (int d0 = 0; d0 < a.D; d0 += 64 * 8) {
    float s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = -0.0f;
    for (int64_t j = i; j < a.N && key[j] == id; ++j) {
      const Y* row = dy + (int64_t)tok[j] * a.D;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = d0 + lane + 64 * e;
        if (d < a.D) {
          const float v = as_float(row[d]);
          s[e] = v != 0.0f ? s[e] + v : s[e];
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = d0 + lane + 64 * e;
      if (d < a.D) dw[d] = dw[d] + s[e];
    }
  }
}

int key_bits(int vocab) {
  int bits = 1;
  while (bits < 32 && ((uint64_t)1 << bits) <= (uint64_t)vocab) ++bits;  // vocab itself is the sentinel
  return bits;
}

}  // namespace

EmbedSortLayout embed_sort_layout(int64_t N, int vocab) {
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  EmbedSortLayout L{};
  size_t temp = 0;
  uint32_t* none = nullptr;
  if (rocprim::radix_sort_pairs(nullptr, temp, none, none, none, none, (unsigned)N, 0, key_bits(vocab)) != hipSuccess)
    temp = 0;
  L.key_in = 0;
  L.key_out = L.key_in + up(N * 4);
  L.val_in = L.key_out + up(N * 4);
  L.val_out = L.val_in + up(N * 4);
  L.temp = L.val_out + up(N * 4);
  L.temp_bytes = temp;
  L.total = L.temp + up(temp);
  return L;
}

hipError_t launch_embed_sorted(const EmbedArgs& a, bool bf16_dy, void* workspace, hipStream_t s) {
  const EmbedSortLayout L = embed_sort_layout(a.N, a.vocab);
  char* ws = static_cast<char*>(workspace);
  uint32_t* key_in = reinterpret_cast<uint32_t*>(ws + L.key_in);
  uint32_t* key_out = reinterpret_cast<uint32_t*>(ws + L.key_out);
  uint32_t* val_in = reinterpret_cast<uint32_t*>(ws + L.val_in);
  uint32_t* val_out = reinterpret_cast<uint32_t*>(ws + L.val_out);
  const unsigned kgrid = (unsigned)std::min<int64_t>((a.N + 255) / 256, 4096);
  hipLaunchKernelGGL(embed_keys_kernel, dim3(kgrid), dim3(256), 0, s, a, key_in, val_in);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  size_t temp = L.temp_bytes;
  e = rocprim::radix_sort_pairs(ws + L.temp, temp, key_in, key_out, val_in, val_out, (unsigned)a.N, 0,
                                key_bits(a.vocab), s);
  if (e != hipSuccess) return e;
  const unsigned rgrid = (unsigned)((a.N + 3) / 4);
  if (bf16_dy) hipLaunchKernelGGL(embed_runs_kernel<bf16>, dim3(rgrid), dim3(256), 0, s, a, key_out, val_out);
  else hipLaunchKernelGGL(embed_runs_kernel<float>, dim3(rgrid), dim3(256), 0, s, a, key_out, val_out);
  return hipGetLastError();
}

}  // namespace fc
