// Host-side problem description of the attention entry points: descriptor
// validation, the normalised window and the backward workspace layout.
// Plain C++ (no HIP), so a host-only harness can build and check it alone.
#pragma once

#include "../../include/femtochat_attn.h"

#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>

namespace fc {

// Normalised problem: window already mapped to (left,right) with the causal
// sentinel (-1,0) replaced by (T,0) and both extents clamped to [-T-1, T].
struct Problem {
  int D;   // the caller's head dim (the scale is 1/sqrt(D))
  int Dk;  // the head dim the kernels run with: D, or the compiled width D is zero-padded to
  int H, Hkv, T, B, group;
  int left, right;
  bool bf16;        // fast mode (bf16 inputs) vs exact mode (fp32)
  bool out_bf16;    // O storage
  bool dout_bf16;   // dO storage
  bool grad_bf16;   // dQ/dK/dV storage
  bool accumulate;  // backward adds into dQ/dK/dV
  bool positions;
};

// XCDs of an MI355X: the hardware sends workgroup id to XCD id % kXcds.
constexpr int kXcds = 8;

// Work order of the fast kernels with positions (attn_order_kernel in
// attn_bwd.hip): the tiles of all batch rows sorted by decreasing work, ties
// by index, so that the tiles of long documents start first.  The work is counted for the
// tilings below (fast forward and dQ: 128 queries per workgroup against
// 64-key tiles; fast dK/dV: 128 keys per item against 128-query steps); the
// kernels assert that they use them.  An order entry is b * n + tile with
// n = ceil(T / 128).
constexpr int kOrderRows = 128;         // queries (keys) per forward and dQ (dK/dV) item
constexpr int kOrderTile = 64;          // keys per step of a forward or dQ item
constexpr int kOrderKStep = 128;        // queries per step of a dK/dV item
constexpr int kOrderMaxItems = 4096;    // largest B * ceil(T / 128) the order kernel tabulates
inline bool order_fits(int T, int B) { return (int64_t)B * ((T + kOrderRows - 1) / kOrderRows) <= kOrderMaxItems; }

// Fast mode with positions takes the tiles in the work order when the order
// kernel's tables fit.
inline bool ordered(const Problem& p) { return p.bf16 && p.positions && order_fits(p.T, p.B); }

// A sliding window at most half the sequence (no positions): the tiles of a
// row do about the same work and consecutive tiles share most of their keys,
// so the fast forward and dK/dV kernels take each row's tiles one after
// another on one XCD (row-local order) instead of the longest-first order
// over all rows, which halves their HBM reads.
inline bool windowed(const Problem& p) {
  return p.bf16 && !p.positions && (int64_t)p.left + std::max(p.right, 0) + 1 <= p.T / 2;
}

// Head dims the kernels are compiled for; every other multiple of 16 up to
// 128 runs on copies zero-padded to the next of them (a zero column adds
// nothing to Q.K, dO.V or dO.O, and the padded output columns are dropped).
inline bool head_dim_compiled(int D) { return D == 16 || D == 32 || D == 64 || D == 128; }
inline bool head_dim_supported(int D) { return D >= 16 && D <= 128 && D % 16 == 0; }
inline int kernel_head_dim(int D) { return D <= 16 ? 16 : D <= 32 ? 32 : D <= 64 ? 64 : 128; }
inline bool padded(const Problem& p) { return p.Dk != p.D; }

inline bool valid_dtype(int32_t d) { return d == FC_F32 || d == FC_BF16; }

// Largest byte extent of one (batch, head) slice that the fast-mode kernels
// address with 32-bit buffer offsets: the last row's start plus one row.
inline int64_t fast_slice_bytes(int T, int heads, int D) { return (int64_t)(T - 1) * heads * D * 2 + 2 * D; }

// Validates the descriptor and fills the normalised problem; on failure
// writes a message into msg (msg_len bytes) and returns the status.
inline fc_status make_problem(const fc_attn_desc* d, Problem* p, char* msg, size_t msg_len) {
  auto bad = [&](fc_status code, const char* text) {
    snprintf(msg, msg_len, "%s", text);
    return code;
  };
  if (d == nullptr) return bad(FC_ERR_INVALID_ARGUMENT, "descriptor is null");
  if (d->D <= 0 || d->H <= 0 || d->Hkv <= 0 || d->T <= 0 || d->B <= 0) {
    snprintf(msg, msg_len, "sizes must be positive (D=%d H=%d Hkv=%d T=%d B=%d)", d->D, d->H, d->Hkv, d->T, d->B);
    return FC_ERR_INVALID_ARGUMENT;
  }
  if (d->H % d->Hkv != 0) {
    snprintf(msg, msg_len, "n_head %d is not a multiple of n_kv_head %d", d->H, d->Hkv);
    return FC_ERR_INVALID_ARGUMENT;
  }
  if (d->D % 16 != 0 || d->D > 128) {
    snprintf(msg, msg_len, "head_dim %d must be a multiple of 16 and at most 128", d->D);
    return FC_ERR_INVALID_ARGUMENT;
  }
  const int64_t rows = (int64_t)d->B * d->T * d->H;
  if (rows * kernel_head_dim(d->D) >= (int64_t)1 << 40 || rows > INT32_MAX / 2)
    return bad(FC_ERR_UNSUPPORTED, "problem too large");
  if (!valid_dtype(d->in_dtype) || !valid_dtype(d->out_dtype) || !valid_dtype(d->dout_dtype) ||
      !valid_dtype(d->grad_dtype))
    return bad(FC_ERR_INVALID_ARGUMENT, "dtype codes must be FC_F32 or FC_BF16");
  if (d->mode == FC_MODE_EXACT) {
    if (d->in_dtype != FC_F32 || d->out_dtype != FC_F32 || d->dout_dtype != FC_F32 || d->grad_dtype != FC_F32)
      return bad(FC_ERR_INVALID_ARGUMENT, "exact mode takes and returns float32 only");
  } else if (d->mode == FC_MODE_FAST) {
    if (d->in_dtype != FC_BF16)
      return bad(FC_ERR_INVALID_ARGUMENT, "fast mode takes bfloat16 Q/K/V (convert first, as attention_inputs does)");
    // The fast kernels read a (batch, head) slice through one buffer
    // descriptor with 32-bit offsets.
    const int Dk = kernel_head_dim(d->D);
    if (fast_slice_bytes(d->T, d->H, Dk) >= ((int64_t)1 << 31) || fast_slice_bytes(d->T, d->Hkv, Dk) >= ((int64_t)1 << 31)) {
      snprintf(msg, msg_len, "fast mode: a (batch, head) slice of T*H*D = %lld bf16 values spans 2^31 bytes or more",
               (long long)d->T * d->H * d->D);
      return FC_ERR_UNSUPPORTED;
    }
  } else {
    snprintf(msg, msg_len, "unknown mode %d", d->mode);
    return FC_ERR_INVALID_ARGUMENT;
  }
  if ((d->flags & ~FC_FLAG_OVERWRITE) != 0) {
    snprintf(msg, msg_len, "unknown flag bits 0x%x", d->flags);
    return FC_ERR_INVALID_ARGUMENT;
  }

  p->D = d->D;
  p->Dk = kernel_head_dim(d->D);
  p->H = d->H;
  p->Hkv = d->Hkv;
  p->T = d->T;
  p->B = d->B;
  p->group = d->H / d->Hkv;
  int64_t left = d->win_left, right = d->win_right;
  if (left == -1 && right == 0) left = d->T;  // causal sentinel (src/kernels.jl:35-36)
  // Clamping to [-T-1, T] keeps q - left and q + right in range without
  // changing which keys of [0, T) are visible.
  const int64_t lo = -(int64_t)d->T - 1, hi = d->T;
  p->left = (int)std::min(std::max(left, lo), hi);
  p->right = (int)std::min(std::max(right, lo), hi);
  p->bf16 = d->mode == FC_MODE_FAST;
  p->out_bf16 = d->out_dtype == FC_BF16;
  p->dout_bf16 = d->dout_dtype == FC_BF16;
  p->grad_bf16 = d->grad_dtype == FC_BF16;
  p->accumulate = (d->flags & FC_FLAG_OVERWRITE) == 0;
  p->positions = false;
  return FC_OK;
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
inline size_t chunk_bounds_bytes(const Problem& p) { return (size_t)p.B * ((p.T + 31) / 32) * 2 * sizeof(int32_t); }
inline size_t order_bytes(const Problem& p) { return (size_t)p.B * ((p.T + kOrderRows - 1) / kOrderRows) * sizeof(int32_t); }

// Workspace layout of the forward pass (byte offsets, 256-aligned): the
// padded copies of a non-compiled head dim (required then), and when the
// work order applies the per-32-query key bounds and the query tiles' order
// (optional: the forward of a compiled head dim runs without a workspace,
// in the default order).
struct FwdWorkspace {
  size_t chunk_lb, qorder, total;
};

// The problem the kernels run: a padded problem's head dim replaced by the
// compiled width (the scale still follows p.D).  A padded backward runs with
// float32 gradients that it overwrites; they are added to (or written into)
// the caller's gradients afterwards, rounded once.
inline Problem kernel_problem(const Problem& p, bool backward) {
  Problem k = p;
  if (padded(p) && backward) {
    k.grad_bf16 = false;
    k.accumulate = false;
  }
  return k;
}

// Padded copies of a non-compiled head dim (byte offsets, 256-aligned):
// Q, K, V (input format), O (its format), and in the backward dO (its
// format) and float32 dQ, dK, dV, all with rows of Dk values.  The kernels'
// own workspace of the padded problem follows at `inner`.
struct PadWorkspace {
  size_t Q, K, V, O, dO, dQ, dK, dV, inner;
};

inline PadWorkspace pad_workspace(const Problem& p, bool backward) {
  PadWorkspace w{};
  if (!padded(p)) return w;
  const size_t nq = (size_t)p.B * p.T * p.H * p.Dk, nk = (size_t)p.B * p.T * p.Hkv * p.Dk;
  const size_t ein = p.bf16 ? 2 : 4, eout = p.out_bf16 ? 2 : 4, edo = p.dout_bf16 ? 2 : 4;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = align256(off + bytes);
    return at;
  };
  w.Q = take(nq * ein);
  w.K = take(nk * ein);
  w.V = take(nk * ein);
  w.O = take(nq * eout);
  if (backward) {
    w.dO = take(nq * edo);
    w.dQ = take(nq * 4);
    w.dK = take(nk * 4);
    w.dV = take(nk * 4);
  }
  w.inner = off;
  return w;
}

inline FwdWorkspace fwd_workspace(const Problem& p) {
  FwdWorkspace w{};
  size_t off = pad_workspace(p, false).inner;  // padded copies first, if any
  if (ordered(p)) {
    w.chunk_lb = off;
    off = align256(off + chunk_bounds_bytes(p));
    w.qorder = off;
    off = align256(off + order_bytes(p));
  }
  w.total = off;
  return w;
}

// Workspace layout of the backward pass (byte offsets, 256-aligned): the
// padded copies of a non-compiled head dim, then Delta and the base-2
// log-sum-exp per query, per-32-query key bounds with
// positions, a bf16 copy of an fp32 dO in fast mode, in fast mode the
// dK/dV kernel's work counters, and the dQ and dK/dV orders when the work
// order applies.
struct BwdWorkspace {
  size_t delta, lse2, chunk_lb, dO16, queue, qorder, korder, total;
};

inline BwdWorkspace bwd_workspace(const Problem& p) {
  BwdWorkspace w{};
  const size_t nq = (size_t)p.B * p.H * p.T;
  size_t off = pad_workspace(p, true).inner;  // padded copies first, if any
  w.delta = off;
  off = align256(off + nq * sizeof(float));
  w.lse2 = off;
  off = align256(off + nq * sizeof(float));
  w.chunk_lb = off;
  if (p.positions) off = align256(off + chunk_bounds_bytes(p));
  w.dO16 = off;
  if (p.bf16 && !p.dout_bf16) off = align256(off + nq * p.Dk * sizeof(uint16_t));
  w.queue = off;  // the fast dK/dV kernel's work counters, one per XCD
  if (p.bf16) off = align256(off + kXcds * sizeof(int32_t));
  w.qorder = off;
  if (ordered(p)) off = align256(off + order_bytes(p));
  w.korder = off;
  if (ordered(p)) off = align256(off + order_bytes(p));
  w.total = off;
  return w;
}

}  // namespace fc
