// Flash-attention backward, fast mode (bf16 inputs, fp32 accumulation), gfx950.
//
// Semantics as the exact-mode kernels (attn_bwd.hip, which also holds the
// preprocess) and the reference backward (src/kernels.jl:287-379; P and dS
// rounded to bf16 before their second product and dS = 0 for a query with a
// single visible key, ext/FemtoChatCUDAExt.jl:1915-1946).
//
//  * attn_bwd_dkdv_fast: persistent, one workgroup per CU; an item is 128
//    keys of one (batch, KV head), taken heaviest first from a counter per
//    XCD (or in the work order with positions, or row by row for a narrow
//    window).  Each wave keeps its 32 keys' K and V in registers (B operands
//    of S = Q K^T and dP = dO V^T), loops over the GQA group's heads and the
//    query tiles (128 queries) that can see the keys, and accumulates dK and
//    dV in registers.  Q and dO tiles are staged once into swizzled LDS and
//    read both as natural fragments (for S, dP) and through
//    ds_read_b64_tr_b16 (for dV += P^T dO and dK += dS^T Q).
//  * attn_bwd_dq_fast: a workgroup owns 128 queries of one (batch, head);
//    S^T and dP^T are recomputed with the query as the lane index so dS^T is
//    directly the B operand of dQ^T += K^T dS^T; K and V tiles are staged once
//    and K is also read transposed; dQ leaves through LDS in whole rows.
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

// ---------------------------------------------------------------------------
template <int D>
struct DqFastCfg {
  static constexpr int kBM = 128;  // queries per workgroup
  static constexpr int kBN = 64;   // keys per tile
  static constexpr int kKC = D / 16;
  static constexpr int kDB = D < 32 ? 1 : D / 32;
  static constexpr int kTileBytes = kBN * 2 * D;
  static constexpr int kStageBytes = 2 * kTileBytes;  // K, V
};

template <int D>
__global__ __launch_bounds__(kThreads, 2) void attn_bwd_dq_fast_kernel(BwdArgs a) {
  using C = DqFastCfg<D>;
  using M = Mma<bf16>;
  constexpr int BN = C::kBN, KC = C::kKC, DB = C::kDB, NKB = BN / 32;
  __shared__ __attribute__((aligned(1024))) char bufA[C::kStageBytes];
  __shared__ __attribute__((aligned(1024))) char bufB[C::kStageBytes];
  __shared__ int s_bounds[2][kWaves];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 5, l32 = lane & 31;
  const int T = a.T;
  const int n_qt = (T + C::kBM - 1) / C::kBM;
  static_assert(C::kBM == kOrderRows && C::kBN == kOrderTile, "the work order counts this tiling");
  int b, h, qt;
  // The row-local order is not used here: in same-box A/B runs on C4's
  // window layers it halved this kernel's HBM reads but cost it 1.5-2% of its
  // time (with and without full tiles first).
  if (a.qorder != nullptr) {
    ordered_query_item(blockIdx.x, a.qorder, n_qt, a.H, a.Hkv, a.group, b, h, qt);
  } else {
    const GridItem it0 = heavy_first(blockIdx.x, a.H * a.B);
    qt = n_qt - 1 - it0.rank;  // longest query tiles first
    query_row(it0.row, a.B, a.Hkv, a.group, b, h);
  }
  const int kvh = h / a.group;
  // Running first (it computes the statistics), this kernel resets the
  // dK/dV kernel's work counters.
  if (a.stats && blockIdx.x == 0 && tid < kXcds) a.queue[tid] = 0;

  const int qpitch = a.H * D * 2, kpitch = a.Hkv * D * 2;
  const int64_t qrec = (int64_t)(T - 1) * qpitch + 2 * D;
  const int64_t krec = (int64_t)(T - 1) * kpitch + 2 * D;
  const int64_t hoff = (((int64_t)b * T * a.H + h) * D) * 2;
  const char* Kb = static_cast<const char*>(a.K) + (((int64_t)b * T * a.Hkv + kvh) * D) * 2;
  const char* Vb = static_cast<const char*>(a.V) + (((int64_t)b * T * a.Hkv + kvh) * D) * 2;
  const int32_t* pos = a.pos ? a.pos + (int64_t)b * T : nullptr;

  const int q = qt * C::kBM + wave * 32 + l32;
  const int lb = key_lb(q, T, a.left, pos), ub = key_ub(q, T, a.right);
  const bool multiple = ub > lb;
  const int wlb_min = wave_min32(lb), wlb_max = wave_max32(lb);
  const int wub_min = wave_min32(ub), wub_max = wave_max32(ub);
  if (lane == 0) {
    s_bounds[0][wave] = wlb_min;
    s_bounds[1][wave] = wub_max;
  }
  const int64_t si = ((int64_t)b * a.H + h) * T + q;
  // The row's statistics (l and m, or lse2 and Delta) load first and
  // unconditionally (a query past T reads row T-1 and discards it), so they
  // share one memory round trip with the fragment loads below.
  const int64_t sc = si - q + min(q, T - 1);
  const float st_a = (a.stats ? a.m : a.lse2)[sc];
  const float st_b = (a.stats ? a.l : a.delta)[sc];

  bf16x8 qf[KC], of[KC], ov[KC];
  const int qoff = q * qpitch + 16 * g;
  {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(static_cast<const char*>(a.Q) + hoff, (uint32_t)qrec);
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<const char*>(a.dO) + hoff, (uint32_t)qrec);
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      qf[c] = as_bf16x8(buf_load16(rq, qoff + 32 * c, 0));
      of[c] = as_bf16x8(buf_load16(ro, qoff + 32 * c, 0));
    }
    if (a.stats) {
      const __amdgpu_buffer_rsrc_t rO = make_rsrc(static_cast<const char*>(a.O) + hoff, (uint32_t)qrec);
#pragma unroll
      for (int c = 0; c < KC; ++c) ov[c] = as_bf16x8(buf_load16(rO, qoff + 32 * c, 0));
    }
  }
  FragOffsets<D> fo;
  fo.init(lane);
  DmaPlan<D, BN> plan;
  plan.init(wave, lane, kpitch);

  __syncthreads();
  int kmin = s_bounds[0][0], kmax = s_bounds[1][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    kmin = min(kmin, s_bounds[0][w]);
    kmax = max(kmax, s_bounds[1][w]);
  }
  const int kt0 = (kmin / BN) * BN;
  const int ntiles = kmax >= kmin ? (kmax - kt0) / BN + 1 : 0;

  // The next tile's K and V loads: descriptors set by issue(), loads issued a
  // share at a time at the phase boundaries of the tile body (dma_part),
  // branch-free: with no next tile the descriptors have no records and the
  // loads write zeros into the idle buffer.
  u32x4s nx_k = {0u, 0u, 0u, 0u}, nx_v = {0u, 0u, 0u, 0u};
  uint32_t nx_at = 0;
  // Phases 0 and 1 of a tile issue the loads, so they have the rest of the
  // tile to land.
  constexpr int NPH = 4, NDMA = 2;
  constexpr int kPer = (DmaPlan<D, BN>::kPerWave + NDMA - 1) / NDMA;
  auto dma_part = [&](int k) {
#pragma unroll
    for (int j = k * kPer; j < (k + 1) * kPer; ++j) {
      plan.issue_one(nx_k, nx_at, wave, j);
      plan.issue_one(nx_v, nx_at + C::kTileBytes, wave, j);
    }
  };
  auto issue = [&](int it, char* buf) {
    nx_at = lds_addr(buf);
    if (it < ntiles) {
      const int64_t row0 = (int64_t)(kt0 + it * BN) * kpitch;
      nx_k = tile_words(Kb, krec, row0);
      nx_v = tile_words(Vb, krec, row0);
    } else {
      nx_k = buffer_words(Kb, 0);
      nx_v = buffer_words(Vb, 0);
    }
  };
  // The first tile's loads go out before anything waits for the loads above.
  if (ntiles > 0) {
    issue(0, bufA);
#pragma unroll
    for (int k = 0; k < NPH; ++k) dma_part(k);
  }

  float neg_lse, dlt;
  if (a.stats) {
    // The backward preprocess for this workgroup's queries (the sum over D
    // is split between the two half-waves, which hold alternate 8-element
    // runs of the head dimension), written out for the dK/dV kernel.
    float part = 0.0f;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
#pragma unroll
      for (int e = 0; e < 8; ++e) part += static_cast<float>(of[c][e]) * static_cast<float>(ov[c][e]);
    }
    dlt = part + __shfl_xor(part, 32);
    neg_lse = q < T ? -(st_a * kLog2e + __builtin_amdgcn_logf(fmaxf(st_b, kFltEps))) : -INFINITY;
    dlt = q < T ? dlt : 0.0f;
  } else {
    neg_lse = q < T ? -st_a : -INFINITY;
    dlt = q < T ? st_b : 0.0f;
  }
  f32x16 dq[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) dq[i] = zero16();
  const float c2 = a.scale_log2;

  // Tile body: a pipeline over the tile's two 32-key blocks, phase i holding
  // S^T, dP^T of block i, the softmax of block i-1 and dQ^T += K^T dS^T of
  // block i-2, with MFMAs, LDS reads and VALU interleaved.
  constexpr int kSchedVALU = 0x2, kSchedMFMA = 0x8, kSchedDSRead = 0x100;
  constexpr int M1 = 2 * KC, M2 = 2 * DB;
  auto body = [&](auto mask_tag, int kt, const char* Ks) {
    constexpr bool need_mask = decltype(mask_tag)::value;
    const char* Vs = Ks + C::kTileBytes;
    f32x16 s[NKB], dp[NKB];
    bf16x8 sf[NKB][2];
#pragma unroll
    for (int ph = 0; ph < NKB + 2; ++ph) {
      const int b1 = ph, bs = ph - 1, b2 = ph - 2;
      dma_part(ph);
      __builtin_amdgcn_sched_barrier(0);
      if (b1 < NKB) {
        s[b1] = zero16();
        dp[b1] = zero16();
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          const bf16x8 ka = as_bf16x8(lds_load16(Ks + 32 * b1 * 2 * D, fo.nat(c)));
          s[b1] = M::mma(ka, qf[c], s[b1]);
        }
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          const bf16x8 va = as_bf16x8(lds_load16(Vs + 32 * b1 * 2 * D, fo.nat(c)));
          dp[b1] = M::mma(va, of[c], dp[b1]);
        }
      }
      if (b2 >= 0) {
        // dQ^T += K^T dS^T for the block's 2 chunks of 16 keys.
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const char* kchunk = Ks + 16 * (2 * b2 + hh) * 2 * D;
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const bf16x8 kfr = lds_tr_frag(kchunk, fo.tr(0, db), fo.tr(1, db));
            dq[db] = M::mma(kfr, sf[b2][hh], dq[db]);
          }
        }
      }
      if (bs >= 0 && bs < NKB) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[bs][r], c2, neg_lse));
          float ds = p * (dp[bs][r] - dlt);
          if (need_mask) {
            const int kk = kt + 32 * bs + acc_row(r, g);
            ds = ((kk >= lb) & (kk <= ub) & multiple) ? ds : 0.0f;
          }
          dp[bs][r] = ds;
        }
        sf[bs][0] = M::from_acc<0>(dp[bs]);
        sf[bs][1] = M::from_acc<1>(dp[bs]);
      }
      const int nmf = (b1 < NKB ? M1 : 0) + (b2 >= 0 ? M2 : 0);
      const bool valu = bs >= 0 && bs < NKB;
      __builtin_amdgcn_sched_group_barrier(kSchedDSRead, 4, 0);
#pragma unroll
      for (int i = 0; i < M1 + M2; ++i) {
        if (i < nmf) {
          __builtin_amdgcn_sched_group_barrier(kSchedMFMA, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDSRead, 2, 0);
          if (valu) __builtin_amdgcn_sched_group_barrier(kSchedVALU, 5, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto compute = [&](int it, const char* Ks) {
    const int kt = kt0 + it * BN;
    if (wlb_min > kt + BN - 1 || wub_max < kt) {
#pragma unroll
      for (int k = 0; k < NPH; ++k) dma_part(k);
      return;
    }
    if (wlb_max <= kt && kt + BN - 1 <= wub_min) body(std::false_type{}, kt, Ks);
    else body(std::true_type{}, kt, Ks);
  };

  dma_wait_barrier();
  for (int it = 0; it < ntiles; it += 2) {
    issue(it + 1, bufB);
    compute(it, bufA);
    dma_wait_barrier();
    if (it + 1 >= ntiles) break;
    issue(it + 2, bufA);
    compute(it + 1, bufB);
    dma_wait_barrier();
  }

  // Delta and lse2 for the dK/dV kernel, stored after the tile loop so that
  // its first barrier does not wait for them.
  if (a.stats && q < T && g == 0) {
    a.delta_out[si] = dlt;
    a.lse2_out[si] = -neg_lse;
  }

  // dQ goes out through LDS (the stage buffers are idle after the tile loop's
  // last barrier): each wave writes its 32 rows x D of scaled fp32 dQ into a
  // row-major tile of its own, 16-byte units XOR-swizzled by the row, then
  // takes whole rows, 16 bytes of output per lane (plus the caller's values
  // when accumulating, added in fp32 before the one rounding).
  {
    constexpr int RB = 4 * D;  // bytes per staged fp32 row
    constexpr int U = RB / 16;
    static_assert(2 * 32 * RB <= C::kStageBytes, "two waves' tiles per stage buffer");
    char* tile = (wave < 2 ? bufA : bufB) + (wave & 1) * (32 * RB);
    auto unit_at = [&](int row, int u) { return row * RB + 16 * (u ^ (row & (U - 1))); };
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = 32 * db + 8 * j + 4 * g;  // four consecutive d of row l32
        if (d0 < D) {
          float v[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = dq[db][4 * j + t] * a.scale;
          *reinterpret_cast<uint4*>(tile + unit_at(l32, d0 / 4)) =
              make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
        }
      }
    }
    const int q0w = q - l32;  // the wave's first query
    auto emit = [&](auto elem) __attribute__((always_inline)) {
      using E = decltype(elem);
      constexpr int EPL = 16 / (int)sizeof(E);  // output elements per lane
      constexpr int LPR = D / EPL;              // lanes per row
      constexpr int RPI = 64 / LPR;             // rows per instruction
      constexpr int NI = 32 / RPI;
      E* base = static_cast<E*>(a.dQ) + ((int64_t)b * T * a.H + h) * D;
      // When accumulating, the caller's values are all requested before the
      // first is used (rows past T read the slice's last row, unused).
      uint4 old[NI];
      if (a.accumulate) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int row = i * RPI + lane / LPR, e0 = EPL * (lane % LPR);
          const int qr = epilogue_row(q0w, row, T);
          old[i] = *reinterpret_cast<const uint4*>(base + (int64_t)qr * a.H * D + e0);
        }
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int row = i * RPI + lane / LPR, e0 = EPL * (lane % LPR);
        float v[EPL];
#pragma unroll
        for (int k = 0; k < EPL / 4; ++k) {
          const uint4 w = *reinterpret_cast<const uint4*>(tile + unit_at(row, e0 / 4 + k));
          v[4 * k] = __uint_as_float(w.x), v[4 * k + 1] = __uint_as_float(w.y);
          v[4 * k + 2] = __uint_as_float(w.z), v[4 * k + 3] = __uint_as_float(w.w);
        }
        if (q0w + row < T) {
          E* p = base + (int64_t)(q0w + row) * a.H * D + e0;
          if (a.accumulate) {
            const E* o = reinterpret_cast<const E*>(&old[i]);
#pragma unroll
            for (int k = 0; k < EPL; ++k) v[k] += to_f32(o[k]);
          }
          uint4 out;
          E* po = reinterpret_cast<E*>(&out);
#pragma unroll
          for (int k = 0; k < EPL; ++k) po[k] = from_f32<E>(v[k]);
          *reinterpret_cast<uint4*>(p) = out;
        }
      }
    };
    if (a.grad_bf16) emit(bf16{});
    else emit(0.0f);
  }
}

// ---------------------------------------------------------------------------
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

template <int D>
static hipError_t launch_dq_fast_t(const Problem& p, const BwdArgs& a, hipStream_t s) {
  const int n_qt = (p.T + DqFastCfg<D>::kBM - 1) / DqFastCfg<D>::kBM;
  const dim3 grid(n_qt * p.H * p.B), block(kThreads);
  const ProfileMark mk = profile_begin(s);
  hipLaunchKernelGGL((attn_bwd_dq_fast_kernel<D>), grid, block, 0, s, a);
  const hipError_t e = hipGetLastError();
  profile_end(mk, "attn_bwd_dq_bf16", s);
  return e;
}

hipError_t launch_bwd_dkdv_fast(const Problem& p, const BwdArgs& a, hipStream_t s) {
  switch (p.Dk) {
    case 16: return launch_dkdv_fast_t<16>(p, a, s);
    case 32: return launch_dkdv_fast_t<32>(p, a, s);
    case 64: return launch_dkdv_fast_t<64>(p, a, s);
    case 128: return launch_dkdv_fast_t<128>(p, a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_bwd_dq_fast(const Problem& p, const BwdArgs& a, hipStream_t s) {
  switch (p.Dk) {
    case 16: return launch_dq_fast_t<16>(p, a, s);
    case 32: return launch_dq_fast_t<32>(p, a, s);
    case 64: return launch_dq_fast_t<64>(p, a, s);
    case 128: return launch_dq_fast_t<128>(p, a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fc
