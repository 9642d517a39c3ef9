// Internal interface between the C ABI (attn_api.hip) and the kernels
// (attn_fwd.hip, attn_bwd.hip).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/femtochat_attn.h"
#include "attn_problem.hpp"
#include <stddef.h>
#include <stdint.h>

namespace fc {

struct FwdArgs {
  const void* Q;
  const void* K;
  const void* V;
  const int32_t* pos;
  const int32_t* order;  // fast mode with positions: query tiles in work order, or null
  int local_order;       // fast mode, narrow window: row-local order (windowed())
  void* O;
  float* l;
  float* m;
  int H, Hkv, T, B, group, left, right;
  int out_bf16;
  float scale_log2;
};

struct PreArgs {
  const void* dO;
  const void* O;
  const float* l;
  const float* m;
  float* delta;
  float* lse2;
  void* dO16;  // bf16 copy of an fp32 dO (fast mode only), else null
  int* queue;  // the dK/dV kernel's work counters (kXcds), reset here; null when not used
  int H, T, B;
  int dO_bf16, O_bf16;
};

struct BoundsArgs {
  const int32_t* pos;
  int32_t* chunk_lb;  // [B][ceil(T/32)][2] = (min, max) of key_lb
  int T, B, left;
};

// Work order of the fast kernels with positions: attn_problem.hpp.
struct OrderArgs {
  const int32_t* chunk_lb;  // the bounds kernel's output
  int32_t* qorder;          // query tiles by decreasing key tiles, or null
  int32_t* korder;          // key tiles by decreasing query steps, or null
  int T, B, left, right;
};

struct BwdArgs {
  const void* dO;  // in the input element type (bf16 copy when needed)
  const void* Q;
  const void* K;
  const void* V;
  const float* delta;
  const float* lse2;
  // stats != 0 (fast mode, bf16 O and dO): the dQ kernel computes Delta and
  // lse2 itself from O, dO, l, m and writes them to delta_out/lse2_out for
  // the dK/dV kernel, which then runs after it (no preprocess launch).
  int stats;
  const void* O;
  const float* l;
  const float* m;
  float* delta_out;
  float* lse2_out;
  const int32_t* pos;
  const int32_t* chunk_lb;
  const int32_t* qorder;  // fast mode with positions: dQ tiles in work order, or null
  const int32_t* korder;  // and the dK/dV kernel's key tiles, or null
  int local_order;        // fast mode, narrow window: the dK/dV kernel's key tiles in row-local order (windowed())
  void* dQ;
  void* dK;
  void* dV;
  // Work counters of the fast dK/dV kernel (workspace, one per XCD): zeroed
  // by the kernel that runs just before it (the preprocess, or the dQ
  // kernel with stats).
  int* queue;
  int H, Hkv, T, B, group, left, right;
  int grad_bf16, accumulate;
  float scale;       // 1/sqrt(D)
  float scale_log2;  // log2(e)/sqrt(D)
};

// Attention prologue (rope_norm.hip): rotary embedding then RMS norm x 1.2
// of one tensor (Q or K) with NH heads; vectors = B*T*NH head vectors.
// n / d for 0 <= n < 2^31 by a multiply and a shift: with 2^(l-1) < d <= 2^l
// and m = floor(2^32 (2^l - d) / d) + 1, n / d = (umulhi(n, m) + n) >> l
// (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994).
struct FastDiv {
  uint32_t m;
  int l;
};
inline FastDiv fast_div(uint32_t d) {
  int l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  return FastDiv{uint32_t((((uint64_t(1) << l) - d) << 32) / d + 1), l};
}

struct RopeNormArgs {
  const void* X;
  void* Y;          // forward output
  const void* dY;   // backward input
  void* dX;         // backward output
  const float* sin_t;  // (table_len, D/2): column p = position p
  const float* cos_t;
  const int32_t* pos;  // (B, T) or null: position = token index
  int vectors;       // B*T*NH < 2^30
  int NH, T, table_len;
  FastDiv by_NH, by_T;
  int accumulate;   // backward adds into dX
};
hipError_t launch_rope_norm(int D, bool bf16_storage, const RopeNormArgs& a, bool backward, hipStream_t s);

// The thread-local error message returned by fc_last_error (attn_api.hip).
fc_status set_error(fc_status code, const char* message);
void clear_error();

// Cross-entropy over vocabulary columns (loss.hip).
struct XentArgs {
  const float* logits;   // (V, N) column-major: token t's column at t*V
  const void* targets;   // N indices (int32 or int64)
  float* losses;         // N (forward)
  float* lse;            // N or null (forward: log-sum-exp per token)
  float* reduced;        // null or [1]: sum or mean of the losses
  float* count;          // null or [1]: number of valid targets (forward, count); read by the mean gradient
  float* dlogits;        // (V, N) (backward)
  const float* dy;       // 1 value (sum, mean) or N (none) (backward)
  const float* lse_in;   // N or null (backward: recompute)
  int64_t N;
  int V;
  int64_t ignore_index;
  int index_base, index_type;  // index_type 0: int32, 1: int64
  int reduction;               // 0 none, 1 sum, 2 mean
  int overwrite;               // backward writes instead of adding
};
hipError_t launch_xent_fwd(const XentArgs& a, hipStream_t s);
hipError_t launch_xent_count(const XentArgs& a, hipStream_t s);
hipError_t launch_xent_bwd(const XentArgs& a, hipStream_t s);
bool xent_fused_supported(const XentArgs& a);
hipError_t launch_xent_fused(const XentArgs& a, hipStream_t s);

// Embedding gather and scatter-add (loss.hip).
struct EmbedArgs {
  const float* weights;  // (D, vocab) column-major
  float* dweights;
  const void* tokens;    // N indices
  void* y;               // (D, N), float32 or bf16
  const void* dy;        // (D, N), float32 or bf16
  int64_t N;
  int D, vocab;
  int index_base, index_type;
};
hipError_t launch_embed(const EmbedArgs& a, bool backward, bool bf16_y, hipStream_t s);

// Workspace of the sorted (deterministic) embedding gradient: keys and token
// indices before and after the sort, and the sort's own temporary storage
// (byte offsets, 256-aligned).
struct EmbedSortLayout {
  size_t key_in, key_out, val_in, val_out, temp, temp_bytes, total;
};
EmbedSortLayout embed_sort_layout(int64_t N, int vocab);
hipError_t launch_embed_sorted(const EmbedArgs& a, bool bf16_dy, void* workspace, hipStream_t s);

// Row repacking between head dims (convert.hip): rows of src_cols values
// into rows of dst_cols values, zero-filled or truncated, optionally added
// to the destination's values (fp32, one rounding).
struct RepackArgs {
  const void* src;
  void* dst;
  int64_t rows;
  int src_cols, dst_cols;
  int src_bf16, dst_bf16;
  int accumulate;
};
hipError_t launch_repack(const RepackArgs& a, hipStream_t s);

// Compute units of the current device (cached per device).
hipError_t device_cus(int* cus);

// Kernel launchers (return the hipError_t of the launch).
hipError_t launch_fwd(const Problem& p, const FwdArgs& a, hipStream_t s);
hipError_t launch_bwd_pre(const Problem& p, const PreArgs& a, hipStream_t s);
hipError_t launch_bounds(const Problem& p, const BoundsArgs& a, hipStream_t s);
hipError_t launch_order(const Problem& p, const OrderArgs& a, hipStream_t s);
hipError_t launch_bwd_dkdv(const Problem& p, const BwdArgs& a, hipStream_t s);
hipError_t launch_bwd_dq(const Problem& p, const BwdArgs& a, hipStream_t s);
// Fast-mode (bf16) kernels, attn_fwd_fast.hip / attn_bwd_fast.hip.
hipError_t launch_fwd_fast(const Problem& p, const FwdArgs& a, hipStream_t s);
hipError_t launch_bwd_dkdv_fast(const Problem& p, const BwdArgs& a, hipStream_t s);
hipError_t launch_bwd_dq_fast(const Problem& p, const BwdArgs& a, hipStream_t s);
// The dK/dV kernel at head dims 16, 32 and 64 (attn_bwd_dkdv_vgpr.hip).
hipError_t launch_bwd_dkdv_fast_vgpr(const Problem& p, const BwdArgs& a, hipStream_t s);

// Profiling hooks (attn_api.hip): bracket one launch with events when enabled.
struct ProfileMark {
  void* begin = nullptr;
};
ProfileMark profile_begin(hipStream_t s);
void profile_end(const ProfileMark& mark, const char* kernel, hipStream_t s);

}  // namespace fc
