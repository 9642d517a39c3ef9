// Flash-attention backward for gfx950.
//
// Semantics follow the reference backward (src/kernels.jl:287-379:
// P = exp(S/sqrt(D) - m) / max(l, eps), Delta = rowsum(dO.O),
// dS = P (dP - Delta), dQ += K dS / sqrt(D), dK += Q dS^T / sqrt(D),
// dV += dO P^T) and, for the fast mode, ext/FemtoChatCUDAExt.jl:1829-2068
// (P and dS rounded to the input format before their second product, a query
// with a single visible key gets dS = 0, fp32 accumulation, optional add into
// the caller's gradients before the one final rounding).
//
// Three kernels, all deterministic (no atomics):
//  * attn_bwd_pre  : Delta and the base-2 log-sum-exp per query, and a bf16
//                    copy of dO when the caller hands fp32 dO in fast mode;
//  * attn_bwd_dkdv : one workgroup per (key tile of 128, KV head, batch); the
//                    4 waves own 32 keys each with K and V resident in
//                    registers, and loop over every query head of the GQA
//                    group and every query tile that can see the keys, so the
//                    group's contributions to dK/dV are summed in registers;
//  * attn_bwd_dq   : one workgroup per (query tile of 128, head, batch); it
//                    recomputes S^T and dP^T with the query as the lane index
//                    so dS^T is directly the B operand of dQ^T += K^T dS^T.
#include "attn_device.hpp"
#include "attn_launch.hpp"

#include <type_traits>

namespace fc {

// ---------------------------------------------------------------------------
// Preprocess: Delta = sum_d dO*O (fp32), lse2 = m*log2(e) + log2(max(l, eps)).
template <int D, typename TO, typename TD>
__global__ __launch_bounds__(kThreads) void attn_bwd_pre_kernel(PreArgs a) {
  constexpr int LPQ = D / 8;            // lanes per query, 8 elements each
  constexpr int QPB = kThreads / LPQ;   // queries per block
  const int tid = threadIdx.x;
  const int sub = tid % LPQ;
  const int64_t idx = (int64_t)blockIdx.x * QPB + tid / LPQ;  // (b, t, h) order
  const int64_t n = (int64_t)a.B * a.T * a.H;
  if (a.queue != nullptr && blockIdx.x == 0 && tid < kXcds) a.queue[tid] = 0;
  float acc = 0.0f;
  if (idx < n) {
    const TD* dO = static_cast<const TD*>(a.dO) + idx * D + 8 * sub;
    const TO* O = static_cast<const TO*>(a.O) + idx * D + 8 * sub;
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = to_f32(dO[e]);
      acc += x[e] * to_f32(O[e]);
    }
    if (a.dO16 != nullptr) {
      bf16* out = static_cast<bf16*>(a.dO16) + idx * D + 8 * sub;
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = static_cast<bf16>(x[e]);
    }
  }
#pragma unroll
  for (int o = LPQ / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if (idx < n && sub == 0) {
    const int h = (int)(idx % a.H);
    const int64_t bt = idx / a.H;
    const int t = (int)(bt % a.T), b = (int)(bt / a.T);
    const int64_t si = ((int64_t)b * a.H + h) * a.T + t;
    a.delta[si] = acc;
    a.lse2[si] = a.m[si] * kLog2e + __builtin_amdgcn_logf(fmaxf(a.l[si], kFltEps));
  }
}

// Per 32-query chunk (min, max) of the document-aware key lower bound (a
// query at or beyond T counts as T).  One lane per query, so a half-wave
// reads one chunk's 32 positions in one coalesced access and reduces them.
__global__ __launch_bounds__(kThreads) void attn_bounds_kernel(BoundsArgs a) {
  const int nc = (a.T + 31) / 32;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t chunk = i >> 5;
  const bool live = chunk < (int64_t)nc * a.B;  // uniform over each half-wave
  const int b = live ? (int)(chunk / nc) : 0;
  const int q = live ? 32 * (int)(chunk - (int64_t)b * nc) + (int)(i & 31) : a.T;
  const int lb = key_lb(q, a.T, a.left, a.pos + (int64_t)b * a.T);
  const int lo = wave_min32(lb), hi = wave_max32(lb);
  if (live && (i & 31) == 0) {
    a.chunk_lb[2 * chunk] = lo;
    a.chunk_lb[2 * chunk + 1] = hi;
  }
}

// Work order of the fast kernels' tiles with positions, in one workgroup.
// The smallest key lower bound of every 128-query tile (from the chunk
// bounds) goes to LDS; then the work of each item of 128 rows, in steps:
//  * query tile [q0, q1] (forward and dQ): the 64-key tiles from the one
//    holding its smallest lower bound up to the one holding key_ub(q1);
//  * key tile [k0, k1] (dK/dV): the 128-query tiles between k0 - right and
//    k1 + left whose smallest lower bound is at most k1, which are the
//    tiles the dK/dV kernel visits;
// and finally each item's rank: the items of more work, plus the items of
// equal work and lower index.  order[rank] = item.  The inner loops read
// LDS in runs of 8 with no exit inside a run, so the reads of a run are in
// flight together.
constexpr int kOrderThreads = 1024;
constexpr int kOrderRun = 8;

__global__ __launch_bounds__(kOrderThreads) void attn_order_kernel(OrderArgs a) {
  static_assert(kOrderKStep == kOrderRows, "a dK/dV step is one tabulated query tile");
  __shared__ int s_lb[kOrderMaxItems + kOrderRun];
  __shared__ __attribute__((aligned(16))) int s_work[kOrderMaxItems + kOrderRun];
  const int tid = threadIdx.x, T = a.T;
  const int nc = (T + 31) / 32, n128 = (T + kOrderRows - 1) / kOrderRows;
  const int items = a.B * n128;
  constexpr int kChunks = kOrderRows / 32;
  for (int i = tid; i < items; i += kOrderThreads) {
    const int b = i / n128, t = i - b * n128;
    const int32_t* cb = a.chunk_lb + (int64_t)b * nc * 2;
    int lo = T;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) lo = min(lo, cb[2 * min(kChunks * t + c, nc - 1)]);  // loads without a branch
    s_lb[i] = lo;
  }
  // Padding after the last item: never counted (ranks) or masked (key steps).
  if (tid < kOrderRun) s_work[items + tid] = INT_MIN;

  // sub lanes (a power of two up to a wave) count one item's rank together,
  // each over every sub-th run of kOrderRun items, and add their counts
  // with shuffles.
  int sub = 1;
  while (sub < kWave && sub * 2 * items <= kOrderThreads) sub *= 2;
  const int per = kOrderThreads / sub, part = tid & (sub - 1);
  auto rank_into = [&](int32_t* order) {
    for (int i0 = 0; i0 < items; i0 += per) {  // the same trip count on every lane
      const int i = i0 + tid / sub;
      const bool live = i < items;
      const int w = s_work[live ? i : 0];
      int r = 0;
      for (int j0 = kOrderRun * part; j0 < items; j0 += kOrderRun * sub) {
        int v[kOrderRun];
#pragma unroll
        for (int e = 0; e < kOrderRun; ++e) v[e] = s_work[j0 + e];
#pragma unroll
        for (int e = 0; e < kOrderRun; ++e) r += (v[e] > w || (v[e] == w && j0 + e < i)) ? 1 : 0;
      }
      for (int o = 1; o < sub; o <<= 1) r += __shfl_xor(r, o);
      if (live && part == 0) order[r] = i;
    }
  };
  __syncthreads();
  if (a.qorder != nullptr) {
    for (int i = tid; i < items; i += kOrderThreads) {
      const int t = i % n128;
      const int kmin = s_lb[i];
      const int kmax = key_ub(min(t * kOrderRows + kOrderRows - 1, T - 1), T, a.right);
      s_work[i] = kmax >= kmin ? (kmax - (kmin / kOrderTile) * kOrderTile) / kOrderTile + 1 : 0;
    }
    __syncthreads();
    rank_into(a.qorder);
    __syncthreads();
  }
  if (a.korder != nullptr) {
    for (int i = tid; i < items; i += kOrderThreads) {
      const int b = i / n128, t = i - b * n128;
      const int k0 = t * kOrderRows, k1 = min(k0 + kOrderRows, T) - 1;
      const int qlo = max(0, k0 - a.right), qhi = min(T - 1, k1 + a.left);
      int n = 0;
      if (qhi >= qlo) {
        const int* row = s_lb + b * n128;
        const int ulast = qhi / kOrderKStep;
        for (int u0 = qlo / kOrderKStep; u0 <= ulast; u0 += kOrderRun) {
          int v[kOrderRun];
#pragma unroll
          for (int e = 0; e < kOrderRun; ++e) v[e] = row[u0 + e];  // within the padded table
#pragma unroll
          for (int e = 0; e < kOrderRun; ++e) n += (u0 + e <= ulast && v[e] <= k1) ? 1 : 0;
        }
      }
      s_work[i] = n;
    }
    __syncthreads();
    rank_into(a.korder);
  }
}

// ---------------------------------------------------------------------------
template <typename E, int D>
struct DkdvCfg {
  static constexpr bool kBF = std::is_same<E, bf16>::value;
  static constexpr int kBK = 128;               // keys per workgroup (4 x 32)
  static constexpr int kBQ = kBF ? 64 : 32;     // queries per tile
  static constexpr int kKC = D / 16;
  static constexpr int kDP = D < 32 ? 32 : D;
  static constexpr int kDB = kDP / 32;
  static constexpr int kLD = kBF ? D + 8 : D + 4;  // natural tile row stride
  static constexpr int kLDT = kBQ + 4;             // transposed tile row stride
  static constexpr int kNat = kBQ * kLD;
  static constexpr int kTr = kBF ? kDP * kLDT : 0;
  // Q, dO natural (+ transposed in bf16): one stage
  static constexpr int kStage = 2 * kNat + 2 * kTr;
};

template <typename E, int D>
__global__ __launch_bounds__(kThreads, 1) void attn_bwd_dkdv_kernel(BwdArgs a) {
  using M = Mma<E>;
  using C = DkdvCfg<E, D>;
  constexpr int BQ = C::kBQ, KC = C::kKC, DB = C::kDB, NQB = BQ / 32;
  __shared__ __attribute__((aligned(16))) E smem[2 * C::kStage];
  __shared__ __attribute__((aligned(16))) float s_lse[2][BQ];
  __shared__ __attribute__((aligned(16))) float s_delta[2][BQ];
  __shared__ __attribute__((aligned(16))) int s_lb[2][BQ];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 5, l32 = lane & 31;
  const int T = a.T;
  const int n_kt = (T + C::kBK - 1) / C::kBK;
  // Key tiles that the most query tiles can see come first, over the whole grid.
  const GridItem it0 = heavy_first(blockIdx.x, a.Hkv * a.B);
  const int bkv = it0.row;
  const int kt = it0.rank;
  const int b = bkv / a.Hkv, kvh = bkv - b * a.Hkv;
  const int k0 = kt * C::kBK;
  const int k1 = min(k0 + C::kBK, T) - 1;
  const int kw0 = k0 + 32 * wave, kw1 = kw0 + 31;
  const int key = kw0 + l32;

  const int64_t qpitch = (int64_t)a.H * D, kpitch = (int64_t)a.Hkv * D;
  const E* Kb = static_cast<const E*>(a.K) + ((int64_t)b * T * a.Hkv + kvh) * D;
  const E* Vb = static_cast<const E*>(a.V) + ((int64_t)b * T * a.Hkv + kvh) * D;
  const int32_t* pos = a.pos ? a.pos + (int64_t)b * T : nullptr;
  const int nchunks = (T + 31) / 32;
  const int32_t* clb = a.chunk_lb ? a.chunk_lb + (int64_t)b * nchunks * 2 : nullptr;

  // K and V of this wave's 32 keys, as B operands (lane = key).
  typename M::frag kf[KC], vf[KC];
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    kf[c] = key < T ? M::load8(Kb + (int64_t)key * kpitch + 16 * c + 8 * g) : M::zero();
    vf[c] = key < T ? M::load8(Vb + (int64_t)key * kpitch + 16 * c + 8 * g) : M::zero();
  }
  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) {
    dk[i] = zero16();
    dv[i] = zero16();
  }

  // Query tiles that can see [k0, k1]: q in [k0 - right, k1 + left].
  const int qlo = max(0, k0 - a.right);
  const int qhi = min(T - 1, k1 + a.left);
  const int qt_begin = qlo / BQ;
  const int qt_end = qhi >= qlo ? qhi / BQ : qt_begin - 1;  // inclusive
  const int n_qt_tiles = qt_end - qt_begin + 1;             // per head
  const int total_steps = n_qt_tiles > 0 ? n_qt_tiles * a.group : 0;

  // A step is (head in group, query tile); tiles no document can see are
  // skipped when positions are given.
  auto tile_visible = [&](int qt) -> bool {
    if (clb == nullptr) return true;
    const int c0 = (qt * BQ) / 32;
    int lo = clb[2 * c0];
#pragma unroll
    for (int c = 1; c < BQ / 32; ++c)
      if (c0 + c < nchunks) lo = min(lo, clb[2 * (c0 + c)]);
    return lo <= k1;
  };
  auto next_step = [&](int st) -> int {
    while (st < total_steps && !tile_visible(qt_begin + st % n_qt_tiles)) ++st;
    return st;
  };

  TileStage<E, D, BQ> qst, ost;
  auto stage_load = [&](int st) {
    const int h = kvh * a.group + st / n_qt_tiles;
    const int q0 = (qt_begin + st % n_qt_tiles) * BQ;
    const E* Qb = static_cast<const E*>(a.Q) + ((int64_t)b * T * a.H + h) * D;
    const E* Ob = static_cast<const E*>(a.dO) + ((int64_t)b * T * a.H + h) * D;
    qst.load(Qb, qpitch, q0, T, tid);
    ost.load(Ob, qpitch, q0, T, tid);
  };
  auto stage_store = [&](int st, int buf) {
    const int h = kvh * a.group + st / n_qt_tiles;
    const int q0 = (qt_begin + st % n_qt_tiles) * BQ;
    E* base = smem + buf * C::kStage;
    qst.store_nat(base, C::kLD, tid);
    ost.store_nat(base + C::kNat, C::kLD, tid);
    if constexpr (C::kBF) {
      qst.store_tr(base + 2 * C::kNat, C::kLDT, tid);
      ost.store_tr(base + 2 * C::kNat + C::kTr, C::kLDT, tid);
    }
    if (tid < BQ) {
      const int q = q0 + tid;
      const int64_t si = ((int64_t)b * a.H + h) * T + q;
      s_lse[buf][tid] = q < T ? a.lse2[si] : INFINITY;
      s_delta[buf][tid] = q < T ? a.delta[si] : 0.0f;
      s_lb[buf][tid] = key_lb(q, T, a.left, pos);
    }
  };

  int st = next_step(0);
  if (st < total_steps) {
    stage_load(st);
    stage_store(st, 0);
  }
  int buf = 0;
  while (st < total_steps) {
    const int st_next = next_step(st + 1);
    const bool more = st_next < total_steps;
    if (more) stage_load(st_next);
    __syncthreads();

    const int q0 = (qt_begin + st % n_qt_tiles) * BQ;
    const E* Qs = smem + buf * C::kStage;
    const E* Os = Qs + C::kNat;
    const int* lbs = s_lb[buf];
    // Tile bounds on the key range of its queries (queries >= T have lb = T).
    int lbmin = lbs[0], lbmax = lbs[0];
    {
      const int v = lane < BQ ? lbs[lane] : lbs[0];
      lbmin = wave_min64(v);
      lbmax = wave_max64(v);
    }
    const int ubmin = q0 + BQ - 1 >= T ? -1 : key_ub(q0, T, a.right);  // ub is monotone in q
    const int ubmax = key_ub(min(q0 + BQ - 1, T - 1), T, a.right);
    const bool active = !(lbmin > kw1 || ubmax < kw0);
    if (active) {
      f32x16 s[NQB], dp[NQB];
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        s[qb] = zero16();
        dp[qb] = zero16();
      }
#pragma unroll
      for (int c = 0; c < KC; ++c) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          const auto qfrag = M::load8(Qs + (32 * qb + l32) * C::kLD + 16 * c + 8 * g);
          s[qb] = M::mma(qfrag, kf[c], s[qb]);
          const auto ofrag = M::load8(Os + (32 * qb + l32) * C::kLD + 16 * c + 8 * g);
          dp[qb] = M::mma(ofrag, vf[c], dp[qb]);
        }
      }
      const bool need_mask = !(lbmax <= kw0 && kw1 <= ubmin);
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i0 = 32 * qb + 8 * j + 4 * g;
          const f32x4 L = *reinterpret_cast<const f32x4*>(&s_lse[buf][i0]);
          const f32x4 Dl = *reinterpret_cast<const f32x4*>(&s_delta[buf][i0]);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int r = 4 * j + t;
            float p = __builtin_amdgcn_exp2f(s[qb][r] * a.scale_log2 - L[t]);
            float ds = p * (dp[qb][r] - Dl[t]);
            if (need_mask) {
              const int qq = q0 + i0 + t;
              const int lbq = lbs[i0 + t];
              const int ubq = key_ub(qq, T, a.right);
              const bool vis = key >= lbq && key <= ubq;
              p = vis ? p : 0.0f;
              ds = (vis && ubq > lbq) ? ds : 0.0f;
            }
            s[qb][r] = p;
            dp[qb][r] = ds;
          }
        }
      }
      // dV += P^T dO, dK += dS^T Q  (k = query, accumulator order)
      const E* Qt = Qs + 2 * C::kNat;
      const E* Ot = Qt + C::kTr;
#pragma unroll
      for (int kc = 0; kc < BQ / 16; ++kc) {
        const auto pf = (kc & 1) ? M::template from_acc<1>(s[kc >> 1]) : M::template from_acc<0>(s[kc >> 1]);
        const auto sf = (kc & 1) ? M::template from_acc<1>(dp[kc >> 1]) : M::template from_acc<0>(dp[kc >> 1]);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          typename M::frag of, qfr;
          if constexpr (C::kBF) {
            of = load_tr_bf16(Ot + (32 * db + l32) * C::kLDT + 16 * kc, g);
            qfr = load_tr_bf16(Qt + (32 * db + l32) * C::kLDT + 16 * kc, g);
          } else {
            const int col = D < 32 ? min(32 * db + l32, D - 1) : 32 * db + l32;
            of = load_kt_f32(Os + 16 * kc * C::kLD + col, C::kLD, g);
            qfr = load_kt_f32(Qs + 16 * kc * C::kLD + col, C::kLD, g);
          }
          dv[db] = M::mma(pf, of, dv[db]);
          dk[db] = M::mma(sf, qfr, dk[db]);
        }
      }
    }

    if (more) stage_store(st_next, buf ^ 1);
    buf ^= 1;
    st = st_next;
  }

  // Store: accumulator row = key, column = head-dim index.
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    const int d = 32 * db + l32;
    if (d < D) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = kw0 + acc_row(r, g);
        if (kk < T) {
          const int64_t off = ((int64_t)b * T + kk) * kpitch + (int64_t)kvh * D + d;
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

// ---------------------------------------------------------------------------
template <typename E, int D>
struct DqCfg {
  static constexpr bool kBF = std::is_same<E, bf16>::value;
  static constexpr int kBM = 128;             // queries per workgroup
  static constexpr int kBN = kBF ? 64 : 32;   // keys per tile
  static constexpr int kKC = D / 16;
  static constexpr int kDP = D < 32 ? 32 : D;
  static constexpr int kDB = kDP / 32;
  static constexpr int kLD = kBF ? D + 8 : D + 4;
  static constexpr int kLDT = kBN + 4;
  static constexpr int kNat = kBN * kLD;
  static constexpr int kTr = kBF ? kDP * kLDT : 0;
  static constexpr int kStage = 2 * kNat + kTr;  // K, V natural + K^T
};

template <typename E, int D>
__global__ __launch_bounds__(kThreads, 1) void attn_bwd_dq_kernel(BwdArgs a) {
  using M = Mma<E>;
  using C = DqCfg<E, D>;
  constexpr int BN = C::kBN, KC = C::kKC, DB = C::kDB, NKB = BN / 32;
  __shared__ __attribute__((aligned(16))) E smem[2 * C::kStage];
  __shared__ int s_bounds[2][kWaves];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 5, l32 = lane & 31;
  const int T = a.T;
  const int n_qt = (T + C::kBM - 1) / C::kBM;
  const GridItem it0 = heavy_first(blockIdx.x, a.H * a.B);
  const int qt = n_qt - 1 - it0.rank;  // longest query tiles first, over the whole grid
  int b, h;
  query_row(it0.row, a.B, a.Hkv, a.group, b, h);
  const int kvh = h / a.group;

  const int64_t qpitch = (int64_t)a.H * D, kpitch = (int64_t)a.Hkv * D;
  const E* Qb = static_cast<const E*>(a.Q) + ((int64_t)b * T * a.H + h) * D;
  const E* Ob = static_cast<const E*>(a.dO) + ((int64_t)b * T * a.H + h) * D;
  const E* Kb = static_cast<const E*>(a.K) + ((int64_t)b * T * a.Hkv + kvh) * D;
  const E* Vb = static_cast<const E*>(a.V) + ((int64_t)b * T * a.Hkv + kvh) * D;
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
  const float lse = q < T ? a.lse2[si] : INFINITY;
  const float dlt = q < T ? a.delta[si] : 0.0f;

  typename M::frag qf[KC], of[KC];
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    qf[c] = q < T ? M::load8(Qb + (int64_t)q * qpitch + 16 * c + 8 * g) : M::zero();
    of[c] = q < T ? M::load8(Ob + (int64_t)q * qpitch + 16 * c + 8 * g) : M::zero();
  }
  f32x16 dq[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) dq[i] = zero16();

  __syncthreads();
  int kmin = s_bounds[0][0], kmax = s_bounds[1][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    kmin = min(kmin, s_bounds[0][w]);
    kmax = max(kmax, s_bounds[1][w]);
  }
  const int kt0 = (kmin / BN) * BN;
  const int ntiles = kmax >= kmin ? (kmax - kt0) / BN + 1 : 0;

  TileStage<E, D, BN> kst, vst;
  auto store_stage = [&](int buf) {
    E* base = smem + buf * C::kStage;
    kst.store_nat(base, C::kLD, tid);
    vst.store_nat(base + C::kNat, C::kLD, tid);
    if constexpr (C::kBF) kst.store_tr(base + 2 * C::kNat, C::kLDT, tid);
  };
  if (ntiles > 0) {
    kst.load(Kb, kpitch, kt0, T, tid);
    vst.load(Vb, kpitch, kt0, T, tid);
    store_stage(0);
  }
  for (int it = 0; it < ntiles; ++it) {
    const int kt = kt0 + it * BN;
    const E* Ks = smem + (it & 1) * C::kStage;
    const E* Vs = Ks + C::kNat;
    const E* Kt = Vs + C::kNat;
    const bool more = it + 1 < ntiles;
    if (more) {
      kst.load(Kb, kpitch, kt + BN, T, tid);
      vst.load(Vb, kpitch, kt + BN, T, tid);
    }
    __syncthreads();

    const bool active = !(wlb_min > kt + BN - 1 || wub_max < kt);
    if (active) {
      f32x16 s[NKB], dp[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        s[kb] = zero16();
        dp[kb] = zero16();
      }
#pragma unroll
      for (int c = 0; c < KC; ++c) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const auto kfrag = M::load8(Ks + (32 * kb + l32) * C::kLD + 16 * c + 8 * g);
          s[kb] = M::mma(kfrag, qf[c], s[kb]);
          const auto vfrag = M::load8(Vs + (32 * kb + l32) * C::kLD + 16 * c + 8 * g);
          dp[kb] = M::mma(vfrag, of[c], dp[kb]);
        }
      }
      const bool need_mask = !(wlb_max <= kt && kt + BN - 1 <= wub_min);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(s[kb][r] * a.scale_log2 - lse);
          float ds = p * (dp[kb][r] - dlt);
          if (need_mask) {
            const int kk = kt + 32 * kb + acc_row(r, g);
            const bool vis = kk >= lb && kk <= ub;
            ds = (vis && multiple) ? ds : 0.0f;
          }
          dp[kb][r] = ds;
        }
      }
#pragma unroll
      for (int kc = 0; kc < BN / 16; ++kc) {
        const auto sf = (kc & 1) ? M::template from_acc<1>(dp[kc >> 1]) : M::template from_acc<0>(dp[kc >> 1]);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          typename M::frag kfr;
          if constexpr (C::kBF) kfr = load_tr_bf16(Kt + (32 * db + l32) * C::kLDT + 16 * kc, g);
          else kfr = load_kt_f32(Ks + 16 * kc * C::kLD + (D < 32 ? min(32 * db + l32, D - 1) : 32 * db + l32), C::kLD, g);
          dq[db] = M::mma(kfr, sf, dq[db]);
        }
      }
    }
    if (more) store_stage((it + 1) & 1);
  }

  if (q < T) {
    const int64_t orow = ((int64_t)b * T + q) * a.H + h;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = 32 * db + 8 * j + 4 * g;
        if (d0 < D) {
          f32x4 v;
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = dq[db][4 * j + t] * a.scale;
          if (a.grad_bf16) store4(static_cast<bf16*>(a.dQ) + orow * D + d0, v, a.accumulate);
          else store4(static_cast<float*>(a.dQ) + orow * D + d0, v, a.accumulate);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------

template <int D, typename TO, typename TD>
static hipError_t launch_pre_t(const Problem& p, const PreArgs& a, hipStream_t s) {
  constexpr int QPB = kThreads / (D / 8);
  const int64_t n = (int64_t)p.B * p.T * p.H;
  const dim3 grid((unsigned)((n + QPB - 1) / QPB)), block(kThreads);
  const ProfileMark mk = profile_begin(s);
  hipLaunchKernelGGL((attn_bwd_pre_kernel<D, TO, TD>), grid, block, 0, s, a);
  const hipError_t e = hipGetLastError();
  profile_end(mk, "attn_bwd_pre", s);
  return e;
}

template <int D>
static hipError_t launch_pre_d(const Problem& p, const PreArgs& a, hipStream_t s) {
  if (a.O_bf16) {
    return a.dO_bf16 ? launch_pre_t<D, bf16, bf16>(p, a, s) : launch_pre_t<D, bf16, float>(p, a, s);
  }
  return a.dO_bf16 ? launch_pre_t<D, float, bf16>(p, a, s) : launch_pre_t<D, float, float>(p, a, s);
}

hipError_t launch_bwd_pre(const Problem& p, const PreArgs& a, hipStream_t s) {
  switch (p.Dk) {
    case 16: return launch_pre_d<16>(p, a, s);
    case 32: return launch_pre_d<32>(p, a, s);
    case 64: return launch_pre_d<64>(p, a, s);
    case 128: return launch_pre_d<128>(p, a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_bounds(const Problem& p, const BoundsArgs& a, hipStream_t s) {
  const int64_t n = (int64_t)((p.T + 31) / 32) * p.B * 32;  // one lane per query slot
  const dim3 grid((unsigned)((n + kThreads - 1) / kThreads)), block(kThreads);
  const ProfileMark mk = profile_begin(s);
  hipLaunchKernelGGL(attn_bounds_kernel, grid, block, 0, s, a);
  const hipError_t e = hipGetLastError();
  profile_end(mk, "attn_bounds", s);
  return e;
}

hipError_t launch_order(const Problem& p, const OrderArgs& a, hipStream_t s) {
  if (!order_fits(p.T, p.B)) return hipErrorInvalidValue;
  const ProfileMark mk = profile_begin(s);
  hipLaunchKernelGGL(attn_order_kernel, dim3(1), dim3(kOrderThreads), 0, s, a);
  const hipError_t e = hipGetLastError();
  profile_end(mk, "attn_order", s);
  return e;
}

template <typename E, int D>
static hipError_t launch_dkdv_t(const Problem& p, const BwdArgs& a, hipStream_t s) {
  const int n_kt = (p.T + DkdvCfg<E, D>::kBK - 1) / DkdvCfg<E, D>::kBK;
  const dim3 grid(n_kt * p.Hkv * p.B), block(kThreads);
  const ProfileMark mk = profile_begin(s);
  hipLaunchKernelGGL((attn_bwd_dkdv_kernel<E, D>), grid, block, 0, s, a);
  const hipError_t e = hipGetLastError();
  profile_end(mk, p.bf16 ? "attn_bwd_dkdv_bf16" : "attn_bwd_dkdv_f32", s);
  return e;
}

template <typename E, int D>
static hipError_t launch_dq_t(const Problem& p, const BwdArgs& a, hipStream_t s) {
  const int n_qt = (p.T + DqCfg<E, D>::kBM - 1) / DqCfg<E, D>::kBM;
  const dim3 grid(n_qt * p.H * p.B), block(kThreads);
  const ProfileMark mk = profile_begin(s);
  hipLaunchKernelGGL((attn_bwd_dq_kernel<E, D>), grid, block, 0, s, a);
  const hipError_t e = hipGetLastError();
  profile_end(mk, p.bf16 ? "attn_bwd_dq_bf16" : "attn_bwd_dq_f32", s);
  return e;
}

#define FC_DISPATCH_D(FN, E)                       \
  switch (p.Dk) {                                   \
    case 16: return FN<E, 16>(p, a, s);            \
    case 32: return FN<E, 32>(p, a, s);            \
    case 64: return FN<E, 64>(p, a, s);            \
    case 128: return FN<E, 128>(p, a, s);          \
    default: return hipErrorInvalidValue;          \
  }

hipError_t launch_bwd_dkdv(const Problem& p, const BwdArgs& a, hipStream_t s) {
  if (p.bf16) return launch_bwd_dkdv_fast(p, a, s);
  FC_DISPATCH_D(launch_dkdv_t, float)
}

hipError_t launch_bwd_dq(const Problem& p, const BwdArgs& a, hipStream_t s) {
  if (p.bf16) return launch_bwd_dq_fast(p, a, s);
  FC_DISPATCH_D(launch_dq_t, float)
}

}  // namespace fc
