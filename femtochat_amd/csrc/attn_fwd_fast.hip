// Flash-attention forward, fast mode (bf16 Q/K/V, fp32 accumulation), gfx950.
//
// Semantics as the exact-mode kernel (attn_fwd.hip) and the reference forward
// (src/kernels.jl:131-219; fast-mode rounding of P before P.V and l summed
// from unrounded probabilities as in ext/FemtoChatCUDAExt.jl:1380-1411).
//
// Work split: a workgroup of 4 waves (one per SIMD, two workgroups per CU)
// owns 128 queries of one (batch, head); each wave owns 32 queries (kWQ; the
// code allows kNQB 32-query blocks per wave) and computes S^T = K Q^T with
// the query as the lane index, so P^T is directly the B operand of
// O^T += V^T P^T.  K and V tiles of 64 keys are staged by LDS-DMA into
// swizzled LDS (two stages); K is read as natural fragments and V through
// ds_read_b64_tr_b16, so no transposed copy is written.
//
// A tile is processed as kNKB 32-key blocks in a pipeline of kNKB + 2 phases:
// phase i holds the S products of block i, the softmax of block i-1 and the
// P.V products of block i-2, with one MFMA, a few LDS reads and a few VALU
// instructions interleaved (sched_group_barrier): at one wave per SIMD a VALU
// instruction only overlaps an MFMA when it sits between MFMAs in the wave's
// own instruction stream.
//
// Softmax in base 2 with log2(e)/sqrt(D) folded into one FMA per score, row
// maxima combined over the two half-waves with v_permlane32_swap.  The
// exponent reference m_ref of a row is the maximum of the first block in
// which the row sees a key (O and l are still zero then; its largest P is
// exactly 1, as with a running maximum) and is never moved, so O is never
// rescaled: probabilities may grow up to 2^64 against m_ref, which fp32 and
// bf16 hold with the same relative precision as values near 1.  A
// block maximum beyond that flags the wave, which then recomputes its rows
// after the tile loop with a plain two-pass method (exact maximum first)
// reading K and V from global memory.  P is rounded to bf16 against m_ref and
// the row sum is taken over unrounded P, as in the reference.  O leaves
// through LDS in whole rows.
#include "attn_fast.hpp"
#include "attn_launch.hpp"

namespace fc {

template <int D>
struct FwdFastCfg {
  static constexpr int kWQ = 32;              // queries per wave
  static constexpr int kBM = kWaves * kWQ;    // queries per workgroup
  static constexpr int kBN = 64;              // keys per tile
  static constexpr int kNQB = kWQ / 32;       // query blocks per wave
  static constexpr int kNKB = kBN / 32;       // key blocks per tile
  static constexpr int kKC = D / 16;
  static constexpr int kDB = D < 32 ? 1 : D / 32;
  static constexpr int kTileBytes = kBN * 2 * D;
  static constexpr int kStageBytes = 2 * kTileBytes;  // K, V
};

constexpr float kGrowthLimit = 64.0f;  // log2 units above m_ref that flag the wave

// Value of the other half-wave's lane (lane l <-> l ^ 32).
__device__ inline float other_half(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                  false, false);
  // r[0]: lanes 32..63 hold lanes 0..31 of v; r[1]: lanes 0..31 hold lanes 32..63.
  return __builtin_bit_cast(float, (__lane_id() >= 32) ? r[0] : r[1]);
}

// Masks the scores of a 32-key block (S^T, lane = query) outside [lb, ub]:
// key = k0 + acc_row(r, g), testing only the bounds in kSides.
template <int kSides = kBoth>
__device__ inline void mask_block(f32x16& s, int k0, int g, int lb, int ub) {
  const int x = k0 + 4 * g - lb, y = ub - (k0 + 4 * g);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int c = 8 * (r >> 2) + (r & 3);
    bool in = true;
    if (kSides & kLower) in = in & (x >= -c);
    if (kSides & kUpper) in = in & (y >= c);
    s[r] = in ? s[r] : -INFINITY;
  }
}

// Maxima propagate NaN, as Julia's max does: llvm.maximum compiles to one
// v_maximum3_f32 per two new values and, unlike fmaxf, needs no canonicalising
// v_max_f32 in front of MFMA results.
__device__ inline float nan_max(float x, float y) { return __builtin_elementwise_maximum(x, y); }

__device__ inline float max16(const f32x16& s) {
  float m = nan_max(s[0], s[1]);
#pragma unroll
  for (int r = 2; r < 16; r += 2) m = nan_max(nan_max(m, s[r]), s[r + 1]);
  return m;
}

template <int D>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_fast_kernel(FwdArgs a) {
  using C = FwdFastCfg<D>;
  using M = Mma<bf16>;
  constexpr int BN = C::kBN, KC = C::kKC, DB = C::kDB, NQB = C::kNQB, NKB = C::kNKB;
  constexpr int NPH = NKB + 2;  // phases per tile
  constexpr int kSchedVALU = 0x2, kSchedMFMA = 0x8, kSchedDSRead = 0x100;
  // Two stage buffers as distinct objects, so the compiler can tell the LDS
  // loads of one from the DMA writes into the other.
  __shared__ __attribute__((aligned(1024))) char bufA[C::kStageBytes];
  __shared__ __attribute__((aligned(1024))) char bufB[C::kStageBytes];
  __shared__ int s_bounds[2][kWaves];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 5, l32 = lane & 31;
  const int T = a.T;
  const int n_qt = (T + C::kBM - 1) / C::kBM;
  static_assert(C::kBM == kOrderRows && C::kBN == kOrderTile, "the work order counts this tiling");
  int b, h, qt;
  if (a.order != nullptr) {
    ordered_query_item(blockIdx.x, a.order, n_qt, a.H, a.Hkv, a.group, b, h, qt);
  } else if (a.local_order) {
    // Query tiles from ceil(left / BM) on see a whole window.
    local_query_item(blockIdx.x, (int)gridDim.x, n_qt, local_full_from(n_qt, a.left, C::kBM), a.B, a.Hkv,
                     a.group, b, h, qt);
  } else {
    const GridItem it0 = heavy_first(blockIdx.x, a.H * a.B);
    qt = n_qt - 1 - it0.rank;  // longest query tiles first
    query_row(it0.row, a.B, a.Hkv, a.group, b, h);
  }
  const int kvh = h / a.group;

  const int qpitch = a.H * D * 2, kpitch = a.Hkv * D * 2;  // bytes between tokens
  const char* Qb = static_cast<const char*>(a.Q) + (((int64_t)b * T * a.H + h) * D) * 2;
  const char* Kb = static_cast<const char*>(a.K) + (((int64_t)b * T * a.Hkv + kvh) * D) * 2;
  const char* Vb = static_cast<const char*>(a.V) + (((int64_t)b * T * a.Hkv + kvh) * D) * 2;
  const int64_t qrec = (int64_t)(T - 1) * qpitch + 2 * D;  // valid bytes of a slice
  const int64_t krec = (int64_t)(T - 1) * kpitch + 2 * D;
  const int32_t* pos = a.pos ? a.pos + (int64_t)b * T : nullptr;

  // Queries of the wave's blocks and their visible key ranges.
  int qv[NQB], lb[NQB], ub[NQB];
  int wlb_min = T, wlb_max = 0, wub_min = T, wub_max = -1;
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    qv[qb] = qt * C::kBM + wave * C::kWQ + 32 * qb + l32;
    lb[qb] = key_lb(qv[qb], T, a.left, pos);
    ub[qb] = key_ub(qv[qb], T, a.right);
    wlb_min = min(wlb_min, wave_min32(lb[qb]));
    wlb_max = max(wlb_max, wave_max32(lb[qb]));
    wub_min = min(wub_min, wave_min32(ub[qb]));
    wub_max = max(wub_max, wave_max32(ub[qb]));
  }
  // The reductions are the same on every lane; saying so moves the per-tile
  // decisions below to scalar branches (as vector values the compiler made
  // them exec-masked and copied the accumulators at every join).
  wlb_min = __builtin_amdgcn_readfirstlane(wlb_min);
  wlb_max = __builtin_amdgcn_readfirstlane(wlb_max);
  wub_min = __builtin_amdgcn_readfirstlane(wub_min);
  wub_max = __builtin_amdgcn_readfirstlane(wub_max);
  if (lane == 0) {
    s_bounds[0][wave] = wlb_min;
    s_bounds[1][wave] = wub_max;
  }

  // Q fragments (B operand: lane = query, 8 contiguous head-dim values).
  bf16x8 qf[NQB][KC];
  {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(Qb, (uint32_t)qrec);
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      const int qoff = min(qv[qb], T - 1) * qpitch + 16 * g;
#pragma unroll
      for (int c = 0; c < KC; ++c) qf[qb][c] = as_bf16x8(buf_load16(rq, qoff + 32 * c, 0));
    }
  }

  FragOffsets<D> fo;
  fo.init(lane);
  DmaPlan<D, BN> plan;
  plan.init(wave, lane, kpitch);

  f32x16 o[NQB][DB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
    for (int db = 0; db < DB; ++db) o[qb][db] = zero16();
  }
  float m_ref[NQB], m_true[NQB], l_half[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    m_ref[qb] = -INFINITY;   // exponent reference of the row (same on both half-waves)
    m_true[qb] = -INFINITY;  // row maximum of c2 * S (same on both half-waves)
    l_half[qb] = 0.0f;       // sum of P over this half-wave's keys, against m_ref
  }
  const float c2 = a.scale_log2;

  __syncthreads();
  int kmin = s_bounds[0][0], kmax = s_bounds[1][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    kmin = min(kmin, s_bounds[0][w]);
    kmax = max(kmax, s_bounds[1][w]);
  }
  kmin = __builtin_amdgcn_readfirstlane(kmin);
  kmax = __builtin_amdgcn_readfirstlane(kmax);
  const int kt0 = (kmin / BN) * BN;
  const int ntiles = kmax >= kmin ? (kmax - kt0) / BN + 1 : 0;

  // The next tile's K and V loads, issued a share at a time in the first
  // four phases of the current tile (branch-free: with no next tile the
  // descriptors have no records and the loads write zeros into the idle
  // buffer).
  u32x4s nx_k = {0u, 0u, 0u, 0u}, nx_v = {0u, 0u, 0u, 0u};
  uint32_t nx_at = 0;
  constexpr int NDMA = 4;
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

  bool flag = false;  // a block maximum outgrew m_ref by more than kGrowthLimit

  // Softmax pieces for one 32-key block of one query block: the row maximum
  // (combined over the half-waves) and P with its unrounded sum.
  auto block_max = [&](f32x16& sv, int qb) -> float {
    const float mx = max16(sv) * c2;
    const float mq = nan_max(mx, other_half(mx));
    m_true[qb] = nan_max(m_true[qb], mq);
    return mq;
  };
  auto exp_block = [&](f32x16& sv, int qb, bf16x8* pfo) {
    const float neg_m = m_ref[qb] == -INFINITY ? 0.0f : -m_ref[qb];
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[r], c2, neg_m));
      sv[r] = p;
      psum += p;
    }
    l_half[qb] += psum;
    pfo[0] = M::from_acc<0>(sv);
    pfo[1] = M::from_acc<1>(sv);
  };

  auto body = [&](auto mask_tag, int kt, const char* Ks) {
    constexpr int kSides = decltype(mask_tag)::value;  // bounds that cut the tile (0: none)
    constexpr bool need_mask = kSides != 0;
    const char* Vs = Ks + C::kTileBytes;
    f32x16 s[NKB][NQB];
    bf16x8 pf[NKB][NQB][2];
#pragma unroll
    for (int ph = 0; ph < NPH; ++ph) {
      const int bS = ph, bX = ph - 1, bP = ph - 2;  // blocks of the three stages
      if (ph < NDMA) dma_part(ph);
      __builtin_amdgcn_sched_barrier(0);
      if (bS < NKB) {
        // S^T = K Q^T for key block bS and both query blocks.
        bf16x8 kfr[KC];
#pragma unroll
        for (int c = 0; c < KC; ++c) kfr[c] = as_bf16x8(lds_load16(Ks + 32 * bS * 2 * D, fo.nat(c)));
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) s[bS][qb] = zero16();
#pragma unroll
        for (int c = 0; c < KC; ++c) {
#pragma unroll
          for (int qb = 0; qb < NQB; ++qb) s[bS][qb] = M::mma(kfr[c], qf[qb][c], s[bS][qb]);
        }
      }
      if (bP >= 0) {
        // O^T += V^T P^T, 16 keys per product, each V fragment for both query blocks.
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const char* vchunk = Vs + 16 * (2 * bP + hh) * 2 * D;
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const bf16x8 vfr = lds_tr_frag(vchunk, fo.tr(0, db), fo.tr(1, db));
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) o[qb][db] = M::mma(vfr, pf[bP][qb][hh], o[qb][db]);
          }
        }
      }
      if (bX >= 0 && bX < NKB) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          if (need_mask) mask_block<kSides>(s[bX][qb], kt + 32 * bX, g, lb[qb], ub[qb]);
          const float mq = block_max(s[bX][qb], qb);
          // A row's first visible key sets the reference (nothing to rescale).
          m_ref[qb] = m_ref[qb] == -INFINITY ? mq : m_ref[qb];
          flag |= mq > m_ref[qb] + kGrowthLimit;
          exp_block(s[bX][qb], qb, pf[bX][qb]);
        }
      }
      const int nmf = (bS < NKB ? NQB * KC : 0) + (bP >= 0 ? NQB * 2 * DB : 0);
      const bool valu = bX >= 0 && bX < NKB;
      __builtin_amdgcn_sched_group_barrier(kSchedDSRead, 6, 0);
#pragma unroll
      for (int i = 0; i < 2 * NQB * (KC > 2 * DB ? KC : 2 * DB); ++i) {
        if (i < nmf) {
          __builtin_amdgcn_sched_group_barrier(kSchedMFMA, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDSRead, 2, 0);
          if (valu) __builtin_amdgcn_sched_group_barrier(kSchedVALU, 6, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto compute = [&](int it, const char* Ks) {
    const int kt = kt0 + it * BN;
    if (wlb_min > kt + BN - 1 || wub_max < kt) {
#pragma unroll
      for (int k = 0; k < NDMA; ++k) dma_part(k);
      return;
    }
    const bool lower = wlb_max > kt, upper = kt + BN - 1 > wub_min;
    if (!lower && !upper) body(std::integral_constant<int, 0>{}, kt, Ks);
    else if (!lower) body(std::integral_constant<int, kUpper>{}, kt, Ks);
    else if (!upper) body(std::integral_constant<int, kLower>{}, kt, Ks);
    else body(std::integral_constant<int, kBoth>{}, kt, Ks);
  };

  if (ntiles > 0) {
    issue(0, bufA);
#pragma unroll
    for (int k = 0; k < NDMA; ++k) dma_part(k);
  }
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

  if (__builtin_amdgcn_ballot_w64(flag) != 0) {
    // Scores grew too far above the reference: recompute this wave's rows
    // with the exact maximum first (K and V straight from global memory).
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(Kb, (uint32_t)krec);
    const bf16* Vg = reinterpret_cast<const bf16*>(Vb);
    const int kpe = kpitch / 2;  // elements between tokens
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      const int klo = (wave_min32(lb[qb]) / 32) * 32, khi = wave_max32(ub[qb]);
      auto scores = [&](int k0) -> f32x16 {
        f32x16 sv = zero16();
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          const bf16x8 kfr = as_bf16x8(buf_load16(rk, (k0 + l32) * kpitch + 16 * g + 32 * c, 0));
          sv = M::mma(kfr, qf[qb][c], sv);
        }
        mask_block(sv, k0, g, lb[qb], ub[qb]);
        return sv;
      };
      float mx = -INFINITY;
      for (int k0 = klo; k0 <= khi; k0 += 32) mx = nan_max(mx, max16(scores(k0)) * c2);
      const float mq = nan_max(mx, other_half(mx));
      m_true[qb] = mq;
      m_ref[qb] = mq;
      l_half[qb] = 0.0f;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[qb][db] = zero16();
      for (int k0 = klo; k0 <= khi; k0 += 32) {
        f32x16 sv = scores(k0);
        bf16x8 pfr[2];
        exp_block(sv, qb, pfr);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            // V^T fragment: row d, keys in accumulator k order.
            const int d = min(32 * db + l32, D - 1);
            bf16x8 vfr;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int key = k0 + 16 * hh + 8 * (e >> 2) + 4 * g + (e & 3);
              vfr[e] = key < T ? Vg[(int64_t)key * kpe + d] : static_cast<bf16>(0.0f);
            }
            o[qb][db] = M::mma(vfr, pfr[hh], o[qb][db]);
          }
        }
      }
    }
  }

  // O goes out through LDS (the stage buffers are idle after the tile loop's
  // last barrier): each wave writes its 32 rows x D into a row-major tile of
  // its own, 16-byte units XOR-swizzled by the row, then stores whole rows
  // at 16 bytes per lane (a store instruction covers 64 / U full rows)
  // instead of 16 bytes of each of 32 rows.
  static_assert(NQB == 1, "one 32-query block per wave");
  auto store_o = [&](auto elem) __attribute__((always_inline)) {
    using E = decltype(elem);
    constexpr int RB = D * (int)sizeof(E);  // bytes per output row
    constexpr int U = RB / 16;              // 16-byte units per row
    static_assert(2 * 32 * RB <= C::kStageBytes, "two waves' tiles per stage buffer");
    char* tile = (wave < 2 ? bufA : bufB) + (wave & 1) * (32 * RB);
    const float lt = l_half[0] + other_half(l_half[0]);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = 32 * db + 8 * j + 4 * g;  // four consecutive d of row l32
        if (d0 < D) {
          const int byte = d0 * (int)sizeof(E);
          const int at = l32 * RB + 16 * ((byte / 16) ^ (l32 & (U - 1))) + byte % 16;
          float v[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = o[0][db][4 * j + t] * inv;
          if constexpr (sizeof(E) == 2) {
            auto pack = [](float x, float y) __attribute__((always_inline)) {
              return (uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16>(x)) |
                     ((uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16>(y)) << 16);
            };
            *reinterpret_cast<uint2*>(tile + at) = make_uint2(pack(v[0], v[1]), pack(v[2], v[3]));
          } else {
            *reinterpret_cast<uint4*>(tile + at) =
                make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
          }
        }
      }
    }
    wave_lds_sync();  // the tile's rows come from other lanes
    constexpr int RPI = 64 / U;  // rows per store instruction
    const int q0w = qv[0] - l32;  // the wave's first query
    char* obase = static_cast<char*>(a.O) + (((int64_t)b * T * a.H + h) * D) * (int64_t)sizeof(E);
    const int64_t opitch = (int64_t)a.H * RB;  // bytes between consecutive queries
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int row = i * RPI + lane / U, u = lane % U;
      const uint4 val = *reinterpret_cast<const uint4*>(tile + row * RB + 16 * (u ^ (row & (U - 1))));
      if (q0w + row < T) *reinterpret_cast<uint4*>(obase + (q0w + row) * opitch + 16 * u) = val;
    }
  };
  if (a.out_bf16) store_o(bf16{});
  else store_o(0.0f);

#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const int q = qv[qb];
    const float mt = m_true[qb];
    const float lt = l_half[qb] + other_half(l_half[qb]);
    if (q < T) {
      if (g == 0) {
        const int64_t si = ((int64_t)b * a.H + h) * T + q;
        const bool any = mt != -INFINITY;
        a.l[si] = any ? lt * __builtin_amdgcn_exp2f(m_ref[qb] - mt) : 0.0f;
        a.m[si] = any ? mt * kLn2 : -kFltMax;
      }
    }
  }
}

template <int D>
static hipError_t launch_fwd_fast_t(const Problem& p, const FwdArgs& a, hipStream_t s) {
  const int n_qt = (p.T + FwdFastCfg<D>::kBM - 1) / FwdFastCfg<D>::kBM;
  const dim3 grid(n_qt * p.H * p.B), block(kThreads);
  const ProfileMark mk = profile_begin(s);
  hipLaunchKernelGGL((attn_fwd_fast_kernel<D>), grid, block, 0, s, a);
  const hipError_t e = hipGetLastError();
  profile_end(mk, "attn_fwd_bf16", s);
  return e;
}

hipError_t launch_fwd_fast(const Problem& p, const FwdArgs& a, hipStream_t s) {
  switch (p.Dk) {
    case 16: return launch_fwd_fast_t<16>(p, a, s);
    case 32: return launch_fwd_fast_t<32>(p, a, s);
    case 64: return launch_fwd_fast_t<64>(p, a, s);
    case 128: return launch_fwd_fast_t<128>(p, a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fc
