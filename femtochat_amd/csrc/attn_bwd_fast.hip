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
//
// The dK/dV kernel itself is in attn_bwd_dkdv_fast.hpp; this unit
// instantiates it for D = 128, attn_bwd_dkdv_vgpr.hip for D <= 64.
#include "attn_bwd_dkdv_fast.hpp"

#include <type_traits>

namespace fc {

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
    wave_lds_sync();  // the tile's rows come from other lanes
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
    case 16:
    case 32:
    case 64: return launch_bwd_dkdv_fast_vgpr(p, a, s);
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
