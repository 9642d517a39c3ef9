// Flash-attention backward, fast mode: the dK/dV kernel (persistent,
// KV-stationary) and its launcher template.  Included by the translation
// units that instantiate it: attn_bwd_fast.hip (D = 128) and
// attn_bwd_dkdv_vgpr.hip (D <= 64, built so that every MFMA result lands in
// ordinary vector registers; at D = 128 the accumulators need the
// accumulation registers).
#pragma once

#include "attn_fast.hpp"
#include "attn_launch.hpp"

#include <type_traits>

namespace fc {

template <int D>
struct DkdvFastCfg {
  static constexpr int kBK = 128;  // keys per workgroup
  static constexpr int kBQ = 128;  // queries per step
  static constexpr int kKC = D / 16;
  static constexpr int kDB = D < 32 ? 1 : D / 32;
  static constexpr int kTileBytes = kBQ * 2 * D;
  static constexpr int kStageBytes = 2 * kTileBytes;  // Q, dO
};

// One step of the dK/dV kernel: the wave's 32 keys against one staged tile
// of BQ queries, processed as NQB blocks of 32 queries.
//
// The body is a pipeline over the blocks.  Phase i holds the S, dP products
// of block i, the softmax of block i-1 and the dV, dK products of block i-2,
// so every softmax runs under MFMAs of other blocks: at one wave per SIMD a
// VALU instruction only overlaps an MFMA when it sits between MFMAs in the
// wave's own instruction stream, and sched_group_barrier interleaves them
// (plus the LDS reads) within each phase.  LDS fragments are requested a
// phase, or a few products, before their use.
template <int D>
struct DkdvStep {
  using C = DkdvFastCfg<D>;
  using M = Mma<bf16>;
  static constexpr int BQ = C::kBQ, KC = C::kKC, DB = C::kDB, NQB = BQ / 32;
  static constexpr int NPH = NQB + 2;            // phases of the body
  static constexpr int NTR = 2 * DB;             // transposed fragments per operand and block
  static constexpr int NPRE = NTR < 2 ? NTR : 2;  // of them requested one phase early
  static constexpr int kSchedVALU = 0x2, kSchedMFMA = 0x8, kSchedDSRead = 0x100;

  // dma(k), k = 0..NPH-1, issues a share of the next tile's loads; the body
  // calls it at its phase boundaries so the loads queue behind the products
  // instead of all at once.
  template <typename Dma>
  __device__ __attribute__((always_inline)) static inline void run(const Dma& dma, const char* Qs, const char* Os, const float* lse,
                                    const float* delta, const int* lbs, const int* lbc, const bf16x8* kf,
                                    const bf16x8* vf, f32x16* dk, f32x16* dv, const FragOffsets<D>& fo, int q0,
                                    int key, int kw0, int kw1, int g, int T, int right, float c2) {
    // Smallest and largest key lower bound over the tile's queries, from the
    // per-chunk bounds published with the tile (no cross-lane reduction).
    int lbmin = lbc[0], lbmax = lbc[NQB];
#pragma unroll
    for (int c = 1; c < NQB; ++c) {
      lbmin = min(lbmin, lbc[c]);
      lbmax = max(lbmax, lbc[NQB + c]);
    }
    // LDS broadcasts, the same on every lane: scalar branches below.
    lbmin = __builtin_amdgcn_readfirstlane(lbmin);
    lbmax = __builtin_amdgcn_readfirstlane(lbmax);
    const int ubmin = q0 + BQ - 1 >= T ? -1 : key_ub(q0, T, right);  // ub is monotone in q
    const int ubmax = key_ub(min(q0 + BQ - 1, T - 1), T, right);
    if (lbmin > kw1 || ubmax < kw0) {
#pragma unroll
      for (int k = 0; k < NPH; ++k) dma(k);
      return;
    }
    // Straight-line bodies: steps inside every row's window skip the mask,
    // steps cut by only one side of it test only that side.
    const bool lower = lbmax > kw0, upper = kw1 > ubmin;
    if (!lower && !upper)
      body<0>(dma, Qs, Os, lse, delta, lbs, kf, vf, dk, dv, fo, q0, key, g, T, right, c2);
    else if (!lower)
      body<kUpper>(dma, Qs, Os, lse, delta, lbs, kf, vf, dk, dv, fo, q0, key, g, T, right, c2);
    else if (!upper)
      body<kLower>(dma, Qs, Os, lse, delta, lbs, kf, vf, dk, dv, fo, q0, key, g, T, right, c2);
    else
      body<kBoth>(dma, Qs, Os, lse, delta, lbs, kf, vf, dk, dv, fo, q0, key, g, T, right, c2);
  }

  __device__ static inline void stats(const float* lse, const float* delta, int qb, int g, f32x4* L, f32x4* Dl) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i0 = 32 * qb + 8 * j + 4 * g;
      L[j] = *reinterpret_cast<const f32x4*>(&lse[i0]);
      Dl[j] = *reinterpret_cast<const f32x4*>(&delta[i0]);
    }
  }
  // Key lower bounds of the block's rows, and a factor 0 on rows with a
  // single visible key (whose dS is zero), else 1.
  __device__ static inline void bounds(const int* lbs, int qb, int g, i32x4* LB, f32x4* Z) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i0 = 32 * qb + 8 * j + 4 * g;
      LB[j] = *reinterpret_cast<const i32x4*>(&lbs[i0]);
      Z[j] = *reinterpret_cast<const f32x4*>(&lbs[BQ + i0]);
    }
  }

  // P = exp2(S c2 - lse2), dS = P (dP - Delta), both rounded to bf16 as the
  // operands of dV += P^T dO and dK += dS^T Q.
  // The mask (kSides != 0) is branch-free: P is zero unless key >= lb(q)
  // (kLower) and key - q <= right (kUpper), dS = P (dP - Delta) z(q) with
  // z = 0 on rows with a single visible key.  Rows at or beyond T have
  // lse2 = +inf, so P and dS vanish there without a test; a key at or past T
  // only occurs in steps that test the upper side.
  template <int kSides>
  __device__ __attribute__((always_inline)) static inline void softmax(f32x16& s, f32x16& dp, const f32x4* L, const f32x4* Dl, const i32x4* LB,
                                        const f32x4* Z, int qb, int q0, int key, int g, int T, int right, float c2,
                                        bf16x8* pf, bf16x8* sf) {
    // key - q <= right  <=>  x >= -(8j + t) for row 4g + 8j + t; a key at or
    // past T (the last key tile's padding) fails it for every row, so that
    // P and dS stay zero there even for a row whose lse2 is -inf.
    const int x = key < T ? q0 + 32 * qb + 4 * g - key + right : -(1 << 30);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int r = 4 * j + t;
        float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c2, -L[j][t]));
        if (kSides & kUpper) p = x >= -(8 * j + t) ? p : 0.0f;
        if (kSides & kLower) p = key >= LB[j][t] ? p : 0.0f;
        float ds = p * (dp[r] - Dl[j][t]);
        if (kSides) ds *= Z[j][t];
        s[r] = p;
        dp[r] = ds;
      }
    }
    pf[0] = M::from_acc<0>(s);
    pf[1] = M::from_acc<1>(s);
    sf[0] = M::from_acc<0>(dp);
    sf[1] = M::from_acc<1>(dp);
  }

  __device__ static inline bf16x8 trq(const char* tile, int qb, int i, const FragOffsets<D>& fo) {
    const int h = i / DB, db = i - h * DB;
    return lds_tr_frag(tile + (32 * qb + 16 * h) * 2 * D, fo.tr(0, db), fo.tr(1, db));
  }

  template <int kSides, typename Dma>
  __device__ __attribute__((always_inline)) static inline void body(const Dma& dma, const char* Qs, const char* Os, const float* lse,
                                     const float* delta, const int* lbs, const bf16x8* kf, const bf16x8* vf,
                                     f32x16* dk, f32x16* dv, const FragOffsets<D>& fo, int q0, int key, int g,
                                     int T, int right, float c2) {
    constexpr int M1 = 2 * KC;   // MFMAs of S, dP per block
    constexpr int M2 = 2 * NTR;  // MFMAs of dV, dK per block
    f32x16 s[NQB], dp[NQB];
    f32x4 L[NQB][4], Dl[NQB][4];
    i32x4 LB[NQB][4];
    f32x4 Z[NQB][4];
    bf16x8 pf[NQB][2], sf[NQB][2];
    bf16x8 ofr[NQB][NTR], qfr[NQB][NTR];  // index h * DB + db
#pragma unroll
    for (int ph = 0; ph < NPH; ++ph) {
      const int b1 = ph, bs = ph - 1, b2 = ph - 2;  // blocks of the three stages
      dma(ph);
      __builtin_amdgcn_sched_barrier(0);
      if (b1 < NQB) {
        const char* qt = Qs + 32 * b1 * 2 * D;
        const char* ot = Os + 32 * b1 * 2 * D;
        bf16x8 qa[KC], oa[KC];
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          qa[c] = as_bf16x8(lds_load16(qt, fo.nat(c)));
          oa[c] = as_bf16x8(lds_load16(ot, fo.nat(c)));
        }
        stats(lse, delta, b1, g, L[b1], Dl[b1]);
        if (kSides) bounds(lbs, b1, g, LB[b1], Z[b1]);
        s[b1] = zero16();
        dp[b1] = zero16();
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          s[b1] = M::mma(qa[c], kf[c], s[b1]);
          dp[b1] = M::mma(oa[c], vf[c], dp[b1]);
        }
      }
      if (b2 >= 0) {
#pragma unroll
        for (int i = NPRE; i < NTR; ++i) {
          ofr[b2][i] = trq(Os, b2, i, fo);
          qfr[b2][i] = trq(Qs, b2, i, fo);
        }
#pragma unroll
        for (int i = 0; i < NTR; ++i) {
          const int h = i / DB, db = i - h * DB;
          dv[db] = M::mma(pf[b2][h], ofr[b2][i], dv[db]);
          dk[db] = M::mma(sf[b2][h], qfr[b2][i], dk[db]);
        }
      }
      if (bs >= 0 && bs < NQB) {
        softmax<kSides>(s[bs], dp[bs], L[bs], Dl[bs], LB[bs], Z[bs], bs, q0, key, g, T, right, c2, pf[bs],
                           sf[bs]);
        // First transposed fragments of the block, for the next phase.
#pragma unroll
        for (int i = 0; i < NPRE; ++i) {
          ofr[bs][i] = trq(Os, bs, i, fo);
          qfr[bs][i] = trq(Qs, bs, i, fo);
        }
      }
      // Interleave: one MFMA, a few LDS reads, a few VALU instructions.
      const int nmf = (b1 < NQB ? M1 : 0) + (b2 >= 0 ? M2 : 0);
      const bool valu = bs >= 0 && bs < NQB;
      if (ph == 0) __builtin_amdgcn_sched_group_barrier(kSchedDSRead, 6, 0);
      else __builtin_amdgcn_sched_group_barrier(kSchedDSRead, 2, 0);
#pragma unroll
      for (int i = 0; i < 2 * (M1 > M2 ? M1 : M2); ++i) {
        if (i < nmf) {
          __builtin_amdgcn_sched_group_barrier(kSchedMFMA, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDSRead, 2, 0);
          if (valu && nmf > 16) __builtin_amdgcn_sched_group_barrier(kSchedVALU, 4, 0);
          if (valu && nmf <= 16) __builtin_amdgcn_sched_group_barrier(kSchedVALU, 8, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
};

template <int D>
__global__ __launch_bounds__(kThreads, 1) void attn_bwd_dkdv_fast_kernel(BwdArgs a) {
  using C = DkdvFastCfg<D>;
  constexpr int BQ = C::kBQ, KC = C::kKC, DB = C::kDB;
  // Two stage buffers as distinct objects, so the compiler can tell the LDS
  // loads of one from the DMA writes into the other.
  __shared__ __attribute__((aligned(1024))) char bufA[C::kStageBytes];
  __shared__ __attribute__((aligned(1024))) char bufB[C::kStageBytes];
  __shared__ __attribute__((aligned(16))) float s_lse[2][BQ];
  __shared__ __attribute__((aligned(16))) float s_delta[2][BQ];
  __shared__ __attribute__((aligned(16))) int s_lb[2][2 * BQ];  // per slot: lb, then z as float (see softmax)
  __shared__ __attribute__((aligned(16))) int s_lbc[2][2][BQ / 32];  // per slot: chunk min, max of s_lb
  constexpr int kVisTiles = 256;  // query tiles whose visibility is tabulated in LDS
  __shared__ unsigned char s_vis[kVisTiles];

  __shared__ int s_next;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 5, l32 = lane & 31;
  const int T = a.T;
  const int qpitch = a.H * D * 2, kpitch = a.Hkv * D * 2;
  const int64_t qrec = (int64_t)(T - 1) * qpitch + 2 * D;
  const int64_t krec = (int64_t)(T - 1) * kpitch + 2 * D;
  const int nchunks = (T + 31) / 32;

  // Work items are (key tile, batch, KV head), key tiles that the most query
  // tiles can see first (item = rank * rows + row).  The grid is one
  // workgroup per CU; each takes item blockIdx.x first and then the next
  // unclaimed item of its XCD's share (items i with i % 8 equal to the
  // XCD, blockIdx.x % 8, to which the hardware sends the workgroup), from one
  // counter per XCD that the preceding kernel zeroed.  So the heaviest items
  // go first, every workgroup stays busy to the end, and with a multiple of
  // 8 rows each (batch, KV head) row stays on one XCD, whose L2 then serves
  // its Q and dO tiles to all its key tiles.
  const int rows = a.Hkv * a.B;
  const int n_kt = (T + C::kBK - 1) / C::kBK;
  const int n_items = n_kt * rows;
  const int xcd = (int)blockIdx.x % kXcds;
  static_assert(C::kBK == kOrderRows && C::kBQ == kOrderKStep, "the work order counts this tiling");
  // (batch, KV head, key tile) of an item: in the work order (korder[k] =
  // b * n_kt + kt names the k-th key tile, whose Hkv KV heads are
  // consecutive items), in the row-local order (the key tiles of one (batch,
  // KV head) one after another on one XCD, as for the query tiles), else
  // key tiles outer and rows inner.
  auto decode = [&](int item, int& ib, int& ikvh, int& ikt) {
    if (a.korder != nullptr) {
      const int k = item / a.Hkv;
      ikvh = item - k * a.Hkv;
      const int e = a.korder[k];
      ib = e / n_kt;
      ikt = e - ib * n_kt;
    } else if (a.local_order) {
      const int e = xcd_chunk_entry(item, n_items);
      ikt = e % n_kt;
      const int bk = e / n_kt;
      ib = bk / a.Hkv;
      ikvh = bk - ib * a.Hkv;
    } else {
      const int row = item % rows;
      ikt = item / rows;
      ib = row / a.Hkv;
      ikvh = row - ib * a.Hkv;
    }
  };
  const int xcd_first = ((int)gridDim.x - xcd + kXcds - 1) / kXcds;  // items taken first by this XCD's workgroups

  // K and V of the wave's 32 keys of an item as B operands (lane = key).
  // The next item's are loaded while this item's dK and dV are stored.
  bf16x8 kf[KC], vf[KC];
  auto load_kv = [&](int item) {
    int ib, ikvh, ikt;
    decode(item, ib, ikvh, ikt);
    const int64_t base = (((int64_t)ib * T * a.Hkv + ikvh) * D) * 2;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(static_cast<const char*>(a.K) + base, (uint32_t)krec);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(static_cast<const char*>(a.V) + base, (uint32_t)krec);
    const int koff = (ikt * C::kBK + 32 * wave + l32) * kpitch + 16 * g;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      kf[c] = as_bf16x8(buf_load16(rk, koff + 32 * c, 0));
      vf[c] = as_bf16x8(buf_load16(rv, koff + 32 * c, 0));
    }
  };

  // State of the current item, set by setup(); the step lambdas read it.
  int b = 0, kvh = 0, k0 = 0, k1 = 0, kw0 = 0, kw1 = 0, key = 0;
  const int32_t* pos = nullptr;
  const int32_t* clb = nullptr;
  int qt_begin = 0, n_qt_tiles = 0, t_first = 0, G = 0;
  bool vis_table = false;
  f32x16 dk[DB], dv[DB];  // the item's dK (unscaled) and dV

  // With positions, a query tile is skipped when no query of it can see a key
  // of [k0, k1] (its smallest key lower bound exceeds k1).  The answers are
  // tabulated in LDS per item so the step loop reads no global memory.
  // The chunk index is clamped rather than tested, so the loads issue
  // together (one memory round trip, not one per chunk): a clamped index
  // repeats the tile's last chunk, which leaves the minimum unchanged.
  auto tile_visible_global = [&](int qt) -> bool {
    const int c0 = (qt * BQ) / 32;
    int lo = clb[2 * c0];
#pragma unroll
    for (int c = 1; c < BQ / 32; ++c) lo = min(lo, clb[2 * min(c0 + c, nchunks - 1)]);
    return lo <= k1;
  };
  auto tile_visible = [&](int qt) -> bool {
    if (clb == nullptr) return true;
    return vis_table ? s_vis[qt - qt_begin] != 0 : tile_visible_global(qt);
  };
  // A step is (head of the group, query tile): heads outer, tiles inner,
  // invisible tiles skipped.  step.h == group marks the end.
  struct Step {
    int h, t;
  };
  auto first_tile = [&](int t) -> int {
    while (t < n_qt_tiles && !tile_visible(qt_begin + t)) ++t;
    return t;
  };
  auto advance = [&](Step s) -> Step {
    const int t = first_tile(s.t + 1);
    return t < n_qt_tiles ? Step{s.h, t} : Step{s.h + 1, t_first};
  };
  // Decodes an item and tabulates its tile visibility (ends with a barrier).
  auto setup = [&](int it) {
    int kt;
    decode(it, b, kvh, kt);
    k0 = kt * C::kBK;
    k1 = min(k0 + C::kBK, T) - 1;
    kw0 = k0 + 32 * wave;
    kw1 = kw0 + 31;
    key = kw0 + l32;
    pos = a.pos ? a.pos + (int64_t)b * T : nullptr;
    clb = a.chunk_lb ? a.chunk_lb + (int64_t)b * nchunks * 2 : nullptr;
    // Query tiles that can see [k0, k1]: q in [k0 - right, k1 + left].
    const int qlo = max(0, k0 - a.right);
    const int qhi = min(T - 1, k1 + a.left);
    qt_begin = qlo / BQ;
    n_qt_tiles = qhi >= qlo ? qhi / BQ - qt_begin + 1 : 0;
    vis_table = clb != nullptr && n_qt_tiles <= kVisTiles;
    if (vis_table) {
      for (int t = tid; t < n_qt_tiles; t += kThreads) s_vis[t] = tile_visible_global(qt_begin + t) ? 1 : 0;
    }
    __syncthreads();
    t_first = first_tile(0);
    G = t_first < n_qt_tiles ? a.group : 0;  // no visible tile: no step
  };
  FragOffsets<D> fo;
  fo.init(lane);
  DmaPlan<D, BQ> plan;
  plan.init(wave, lane, qpitch);
  float st_lse = 0.0f, st_delta = 0.0f;
  int st_q = 0, st_pos = 0, st_cmin = 0, st_cmax = 0;
  const float c2 = a.scale_log2;

  // issue() starts loading step st: the row statistics, positions and chunk
  // bounds into registers, each load unconditional (clamped index, or a
  // stand-in array when there are no positions) so that no wait for it is
  // needed before publish(), which consumes them after the step's compute.
  // The next tile's Q and dO loads: descriptors set by issue(), loads issued
  // a quarter at a time by the step body (dma_part), without a branch so the
  // body stays one straight line.  With no next step the descriptors have no
  // records and the loads write zeros into the idle buffer.
  u32x4s nx_q = {0u, 0u, 0u, 0u}, nx_o = {0u, 0u, 0u, 0u};
  uint32_t nx_at = 0;
  // Phases 0..3 of a step issue the loads, so they have the rest of the step
  // to land; later phases issue none.
  constexpr int NPH = DkdvStep<D>::NPH, NDMA = NPH < 4 ? NPH : 4;
  constexpr int kPer = (DmaPlan<D, BQ>::kPerWave + NDMA - 1) / NDMA;
  auto dma_part = [&](int k) {
#pragma unroll
    for (int j = k * kPer; j < (k + 1) * kPer; ++j) {
      plan.issue_one(nx_q, nx_at, wave, j);
      plan.issue_one(nx_o, nx_at + C::kTileBytes, wave, j);
    }
  };
  auto no_issue = [&](char* buf) {
    nx_at = lds_addr(buf);
    nx_q = buffer_words(a.Q, 0);
    nx_o = buffer_words(a.dO, 0);
  };
  auto issue = [&](Step st, char* buf) {
    const int h = kvh * a.group + st.h;
    const int q0 = (qt_begin + st.t) * BQ;
    const int64_t hoff = (((int64_t)b * T * a.H + h) * D) * 2;
    nx_at = lds_addr(buf);
    nx_q = tile_words(static_cast<const char*>(a.Q) + hoff, qrec, (int64_t)q0 * qpitch);
    nx_o = tile_words(static_cast<const char*>(a.dO) + hoff, qrec, (int64_t)q0 * qpitch);
    const int64_t srow = ((int64_t)b * a.H + h) * T;
    const int32_t* stand_in = reinterpret_cast<const int32_t*>(a.delta + srow);  // T readable words
    if (tid < BQ) {
      const int qq = q0 + tid;
      const int qc = min(qq, T - 1);
      st_q = qq;
      st_lse = a.lse2[srow + qc];
      st_delta = a.delta[srow + qc];
      st_pos = (pos != nullptr ? pos : stand_in)[qc];
    }
    if (tid < BQ / 32) {
      // The bounds kernel's per-chunk (min, max) key lower bound.
      const int c = min(q0 / 32 + tid, nchunks - 1);
      const int32_t* cb = clb != nullptr ? clb + 2 * c : stand_in;
      st_cmin = cb[0];
      st_cmax = cb[clb != nullptr ? 1 : 0];
    }
  };
  auto publish = [&](int slot) {
    if (tid < BQ) {
      const bool in = st_q < T;
      s_lse[slot][tid] = in ? st_lse : INFINITY;
      s_delta[slot][tid] = in ? st_delta : 0.0f;
      int lb = T;
      if (in) lb = max(0, max(st_q - a.left, pos != nullptr ? st_q - st_pos : 0));
      s_lb[slot][tid] = lb;
      s_lb[slot][BQ + tid] = __builtin_bit_cast(int, key_ub(st_q, T, a.right) > lb ? 1.0f : 0.0f);
    }
    if (tid < BQ / 32) {
      // Key lower bounds of chunk tid of the tile (queries at or beyond T
      // count as T): monotone in the query without positions, tabulated per
      // chunk with them.
      const int qc0 = (st_q - tid) + 32 * tid;  // st_q is q0 + tid here
      int lo = key_lb(qc0, T, a.left, nullptr), hi = key_lb(qc0 + 31, T, a.left, nullptr);
      if (clb != nullptr) {
        lo = qc0 < T ? st_cmin : T;
        hi = qc0 < T ? st_cmax : T;
      }
      s_lbc[slot][0][tid] = lo;
      s_lbc[slot][1][tid] = hi;
    }
  };
  // Inlined by force: with four step bodies per buffer the compiler would
  // otherwise make this a call (all live registers saved around it).
  auto compute = [&](Step st, const char* buf, int slot) __attribute__((always_inline)) {
    const int q0 = (qt_begin + st.t) * BQ;
    DkdvStep<D>::run(dma_part, buf, buf + C::kTileBytes, s_lse[slot], s_delta[slot], s_lb[slot], s_lbc[slot][0], kf, vf, dk, dv,
                     fo, q0, key, kw0, kw1, g, T, a.right, c2);
  };

  // The first step of the item set up last: its tile into bufA and its row
  // statistics into registers (published before the item's first step).
  auto start = [&]() {
    if (G > 0) {
      issue(Step{0, t_first}, bufA);
#pragma unroll
      for (int k = 0; k < NPH; ++k) dma_part(k);
    }
  };

  int item = blockIdx.x;
  if (item < n_items) {
    load_kv(item);
    setup(item);
    start();
    if (G > 0) publish(0);
  }
  while (item < n_items) {
  // Claim the next item now; its index is read once this item's steps are done.
  int claimed = 0;
  if (tid == 0) claimed = xcd + kXcds * (xcd_first + atomicAdd(a.queue + xcd, 1));

#pragma unroll
  for (int i = 0; i < DB; ++i) {
    dk[i] = zero16();
    dv[i] = zero16();
  }
  Step st{0, t_first};
  dma_wait_barrier();
  while (st.h < G) {
    const Step st1 = advance(st);
    if (st1.h < G) issue(st1, bufB);
    else no_issue(bufB);
    compute(st, bufA, 0);
    if (st1.h < G) publish(1);
    dma_wait_barrier();
    if (st1.h >= G) break;
    const Step st2 = advance(st1);
    if (st2.h < G) issue(st2, bufA);
    else no_issue(bufA);
    compute(st1, bufB, 1);
    if (st2.h < G) publish(0);
    dma_wait_barrier();
    st = st2;
  }

  if (tid == 0) s_next = claimed;
  __syncthreads();
  const int next = s_next;
  // This item's stores need its row and keys; the next item's K, V, first
  // tile and row statistics load meanwhile.
  const int eb = b, ekvh = kvh, ekw0 = kw0;
  if (next < n_items) {
    load_kv(next);
    setup(next);
    start();
  }

  // Accumulator row = key, column = head-dim index.  The stores go through a
  // buffer descriptor over this (batch, KV head)'s rows with the whole offset
  // in the lane's voffset: keys at or past T fall outside the descriptor and
  // the hardware drops them, so no store needs a branch or 64-bit address
  // arithmetic.  (A slice of 2^31 bytes or more takes the plain loop below.)
  const int64_t row_elems = (int64_t)a.Hkv * D;  // elements between consecutive keys
  const int64_t slice0 = (int64_t)eb * T * row_elems + (int64_t)ekvh * D;
  const int esz = a.grad_bf16 ? 2 : 4;
  const int64_t slice_bytes = ((int64_t)(T - 1) * row_elems + D) * esz;
  if (slice_bytes < ((int64_t)1 << 31)) {
    const auto rk = make_rsrc(static_cast<const char*>(a.dK) + slice0 * esz, (uint32_t)slice_bytes);
    const auto rv = make_rsrc(static_cast<const char*>(a.dV) + slice0 * esz, (uint32_t)slice_bytes);
    // The accumulators leave through each wave's part of the idle stage
    // buffer (free until the next item's first barrier; the next item's
    // first tile loads into the other one), so that stores cover whole rows.
    auto pack = [](float x, float y) __attribute__((always_inline)) {
      return (uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16>(x)) |
             ((uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16>(y)) << 16);
    };
    if (a.grad_bf16 && !a.accumulate) {
      // Overwritten bf16 gradients: each wave writes its 32 keys' dK and dV
      // (2 bytes per value, straight from the accumulators) into a row-major
      // tile of its own, 16-byte units XOR-swizzled by the row, then stores
      // 16 bytes per lane, a store instruction covering 64 / U whole rows.
      constexpr int RB = 2 * D, U = RB / 16, RPI = 64 / U;
      static_assert(kWaves * 2 * 32 * RB <= C::kStageBytes, "dK and dV tiles of every wave fit a stage buffer");
      // An opaque zero in the tile address keeps its offsets from being
      // hoisted out of the item loop (where they would only take registers).
      int z;
      asm volatile("v_mov_b32 %0, 0" : "=v"(z));
      char* tile = bufB + wave * (2 * 32 * RB);  // dK rows, then dV rows
      auto at = [&](int row, int d) { return row * RB + 16 * ((d / 8) ^ (row & (U - 1))) + 2 * (d % 8); };
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int d = 32 * db + l32 + z;
        if (d < D) {
#pragma unroll
          for (int r = 0; r < 16; r += 2) {
            const int row = acc_row(r, g) + z;  // rows r and r + 1 are keys row and row + 1
            const uint32_t pk = pack(dk[db][r] * a.scale, dk[db][r + 1] * a.scale);
            const uint32_t pv = pack(dv[db][r], dv[db][r + 1]);
            *reinterpret_cast<unsigned short*>(tile + at(row, d)) = (unsigned short)pk;
            *reinterpret_cast<unsigned short*>(tile + at(row + 1, d)) = (unsigned short)(pk >> 16);
            *reinterpret_cast<unsigned short*>(tile + 32 * RB + at(row, d)) = (unsigned short)pv;
            *reinterpret_cast<unsigned short*>(tile + 32 * RB + at(row + 1, d)) = (unsigned short)(pv >> 16);
          }
        }
      }
      wave_lds_sync();
#pragma unroll
      for (int i = 0; i < 32 / RPI; ++i) {
        const int row = i * RPI + (lane + z) / U, u = (lane + z) % U;
        const int off = row * RB + 16 * (u ^ (row & (U - 1)));
        const uint4 k4 = *reinterpret_cast<const uint4*>(tile + off);
        const uint4 v4 = *reinterpret_cast<const uint4*>(tile + 32 * RB + off);
        const int voff = (int)(((int64_t)(ekw0 + row) * row_elems + 8 * u) * 2);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{k4.x, k4.y, k4.z, k4.w}, rk, voff, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{v4.x, v4.y, v4.z, v4.w}, rv, voff, 0, 0);
      }
    } else {
      // fp32 or accumulated gradients: dK, then dV, staged as fp32 rows in
      // each wave's part of the idle stage buffer and read back 16 bytes
      // (four values) per lane, added to the caller's values when
      // accumulating, rounded once and stored as whole rows.
      constexpr int RB = 4 * D, U = RB / 16, RPI = 64 / U;  // fp32 rows
      static_assert(kWaves * 32 * RB <= C::kStageBytes, "a tensor's tiles of every wave fit a stage buffer");
      int z;  // an opaque zero, as above
      asm volatile("v_mov_b32 %0, 0" : "=v"(z));
      char* tile = bufB + wave * (32 * RB);
      auto unit = [&](int row, int u) { return row * RB + 16 * (u ^ (row & (U - 1))); };
      auto pass = [&](const f32x16* acc, float sc, const __amdgpu_buffer_rsrc_t& rs) __attribute__((always_inline)) {
        constexpr int NI = 32 / RPI;
        auto voff_of = [&](int i) {
          const int row = i * RPI + (lane + z) / U, u = (lane + z) % U;
          return (int)(((int64_t)(ekw0 + row) * row_elems + 4 * u) * esz);
        };
        // The caller's values, all requested before any is used (out-of-range
        // loads read zero).
        u32x2 old2[NI];  // bf16 gradients
        u32x4 old4[NI];  // fp32 gradients
        if (a.accumulate) {
          if (a.grad_bf16) {
#pragma unroll
            for (int i = 0; i < NI; ++i) old2[i] = __builtin_amdgcn_raw_buffer_load_b64(rs, voff_of(i), 0, 0);
          } else {
#pragma unroll
            for (int i = 0; i < NI; ++i) old4[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff_of(i), 0, 0);
          }
        }
        // The previous pass's reads of the tile come before these writes, and
        // the writes before this pass's reads (other lanes' rows).
        wave_lds_sync();
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int d = 32 * db + l32 + z;
          if (d < D) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int row = acc_row(r, g) + z;
              *reinterpret_cast<float*>(tile + unit(row, d / 4) + 4 * (d % 4)) = acc[db][r] * sc;
            }
          }
        }
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int row = i * RPI + (lane + z) / U, u = (lane + z) % U;
          const uint4 w = *reinterpret_cast<const uint4*>(tile + unit(row, u));
          float v[4] = {__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w)};
          const int voff = voff_of(i);
          if (a.grad_bf16) {
            if (a.accumulate) {
              v[0] += __uint_as_float(old2[i][0] << 16);
              v[1] += __uint_as_float(old2[i][0] & 0xffff0000u);
              v[2] += __uint_as_float(old2[i][1] << 16);
              v[3] += __uint_as_float(old2[i][1] & 0xffff0000u);
            }
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{pack(v[0], v[1]), pack(v[2], v[3])}, rs, voff, 0, 0);
          } else {
            if (a.accumulate) {
#pragma unroll
              for (int k = 0; k < 4; ++k) v[k] += __uint_as_float(old4[i][k]);
            }
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])}, rs, voff,
                0, 0);
          }
        }
      };
      pass(dk, a.scale, rk);
      pass(dv, 1.0f, rv);
    }
  } else {
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    const int d = 32 * db + l32;
    if (d < D) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = ekw0 + acc_row(r, g);
        if (kk < T) {
          const int64_t off = ((int64_t)eb * T + kk) * a.Hkv * D + (int64_t)ekvh * D + d;
          float vk = dk[db][r] * a.scale, vv = dv[db][r];
          if (a.grad_bf16) {
            bf16* pk = static_cast<bf16*>(a.dK) + off;
            bf16* pv = static_cast<bf16*>(a.dV) + off;
            if (a.accumulate) {
              vk += to_f32(*pk);
              vv += to_f32(*pv);
            }
            *pk = static_cast<bf16>(vk);
            *pv = static_cast<bf16>(vv);
          } else {
            float* pk = static_cast<float*>(a.dK) + off;
            float* pv = static_cast<float*>(a.dV) + off;
            if (a.accumulate) {
              vk += *pk;
              vv += *pv;
            }
            *pk = vk;
            *pv = vv;
          }
        }
      }
    }
  }
  }
  if (next < n_items && G > 0) publish(0);
  item = next;
  }
}

template <int D>
static hipError_t launch_dkdv_fast_t(const Problem& p, const BwdArgs& a, hipStream_t s) {
  const int n_kt = (p.T + DkdvFastCfg<D>::kBK - 1) / DkdvFastCfg<D>::kBK;
  const int n_items = n_kt * p.Hkv * p.B;
  int cus = 0;
  const hipError_t ec = device_cus(&cus);
  if (ec != hipSuccess) return ec;
  // Every XCD needs a workgroup unless every item has its own.
  const int slots = cus >= kXcds && cus < n_items ? cus : n_items;
  const dim3 grid(slots), block(kThreads);
  const ProfileMark mk = profile_begin(s);
  hipLaunchKernelGGL((attn_bwd_dkdv_fast_kernel<D>), grid, block, 0, s, a);
  const hipError_t e = hipGetLastError();
  profile_end(mk, "attn_bwd_dkdv_bf16", s);
  return e;
}

}  // namespace fc
