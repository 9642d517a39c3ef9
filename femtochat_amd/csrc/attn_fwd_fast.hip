// Flash-attention forward, fast mode (bf16 Q/K/V, fp32 accumulation), gfx950.
//
// Semantics as the exact-mode kernel (attn_fwd.hip) and the reference forward
// (src/kernels.jl:131-219; fast-mode rounding of P before P.V and l summed
// from unrounded probabilities as in ext/FemtoChatCUDAExt.jl:1380-1411).
//
// Work split: a workgroup of 4 waves owns 128 queries of one (batch, head);
// each wave owns 32 queries and computes S^T = K Q^T with its query as the
// lane index, so the online softmax needs a single lane l <-> l^32 exchange per
// key tile and P^T is directly the B operand of O^T += V^T P^T.  K and V tiles
// (64 keys) are staged once per workgroup into swizzled LDS (double-buffered,
// register prefetch through buffer loads), K read as natural fragments and V
// through ds_read_b64_tr_b16, so no transposed copy is written.
//
// Softmax in base 2 with log2(e)/sqrt(D) folded into one FMA per score.  The
// exponent reference m_ref only moves when the running maximum exceeds it by
// more than 8 (probabilities stay <= 2^8), which skips the O rescale on most
// tiles; O and l share m_ref, so O/l is unchanged, and l is reported against
// the true maximum at the end.
#include "attn_fast.hpp"
#include "attn_launch.hpp"

namespace fc {

template <int D>
struct FwdFastCfg {
  static constexpr int kBM = 128;  // queries per workgroup
  static constexpr int kBN = 64;   // keys per tile
  static constexpr int kKC = D / 16;
  static constexpr int kDB = D < 32 ? 1 : D / 32;
  static constexpr int kTileBytes = kBN * 2 * D;
  static constexpr int kStageBytes = 2 * kTileBytes;  // K, V
};

constexpr float kRescaleThreshold = 8.0f;  // log2 units

template <int D>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_fast_kernel(FwdArgs a) {
  using C = FwdFastCfg<D>;
  using M = Mma<bf16>;
  constexpr int BN = C::kBN, KC = C::kKC, DB = C::kDB, NKB = BN / 32;
  __shared__ __attribute__((aligned(16))) char smem[2 * C::kStageBytes];
  __shared__ int s_bounds[2][kWaves];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 5, l32 = lane & 31;
  const int T = a.T;
  const int n_qt = (T + C::kBM - 1) / C::kBM;
  const int id = xcd_remap(blockIdx.x, n_qt * a.H * a.B);
  const int bh = id / n_qt;
  const int qt = n_qt - 1 - (id - bh * n_qt);  // longest query tiles first
  const int b = bh / a.H, h = bh - b * a.H;
  const int kvh = h / a.group;

  const int qpitch = a.H * D * 2, kpitch = a.Hkv * D * 2;  // bytes between tokens
  const char* Qb = static_cast<const char*>(a.Q) + (((int64_t)b * T * a.H + h) * D) * 2;
  const char* Kb = static_cast<const char*>(a.K) + (((int64_t)b * T * a.Hkv + kvh) * D) * 2;
  const char* Vb = static_cast<const char*>(a.V) + (((int64_t)b * T * a.Hkv + kvh) * D) * 2;
  const int64_t qrec = (int64_t)(T - 1) * qpitch + 2 * D;  // valid bytes of a slice
  const int64_t krec = (int64_t)(T - 1) * kpitch + 2 * D;
  const int32_t* pos = a.pos ? a.pos + (int64_t)b * T : nullptr;

  const int q = qt * C::kBM + wave * 32 + l32;
  const int lb = key_lb(q, T, a.left, pos), ub = key_ub(q, T, a.right);
  const int wlb_min = wave_min32(lb), wlb_max = wave_max32(lb);
  const int wub_min = wave_min32(ub), wub_max = wave_max32(ub);
  if (lane == 0) {
    s_bounds[0][wave] = wlb_min;
    s_bounds[1][wave] = wub_max;
  }

  // Q fragments (B operand: lane = query, 8 contiguous head-dim values).
  bf16x8 qf[KC];
  {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(Qb, (uint32_t)qrec);
    const int qoff = q * qpitch + 16 * g;
#pragma unroll
    for (int c = 0; c < KC; ++c) qf[c] = as_bf16x8(buf_load16(rq, qoff + 32 * c, 0));
  }

  FragOffsets<D> fo;
  fo.init(lane);
  StagePlan<D, BN, kThreads> plan;
  plan.init(tid, kpitch);
  StageRegs<D, BN, kThreads> kst, vst;

  f32x16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) o[i] = zero16();
  float m_true = -INFINITY, m_ref = -INFINITY, l_run = 0.0f;
  const float c2 = a.scale_log2;

  __syncthreads();
  int kmin = s_bounds[0][0], kmax = s_bounds[1][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    kmin = min(kmin, s_bounds[0][w]);
    kmax = max(kmax, s_bounds[1][w]);
  }
  const int kt0 = (kmin / BN) * BN;
  const int ntiles = kmax >= kmin ? (kmax - kt0) / BN + 1 : 0;

  if (ntiles > 0) {
    kst.load(plan, tile_rsrc(Kb, krec, (int64_t)kt0 * kpitch));
    vst.load(plan, tile_rsrc(Vb, krec, (int64_t)kt0 * kpitch));
    kst.store(plan, smem);
    vst.store(plan, smem + C::kTileBytes);
  }

  for (int it = 0; it < ntiles; ++it) {
    const int kt = kt0 + it * BN;
    const char* Ks = smem + (it & 1) * C::kStageBytes;
    const char* Vs = Ks + C::kTileBytes;
    const bool more = it + 1 < ntiles;
    if (more) {
      kst.load(plan, tile_rsrc(Kb, krec, (int64_t)(kt + BN) * kpitch));
      vst.load(plan, tile_rsrc(Vb, krec, (int64_t)(kt + BN) * kpitch));
    }
    __syncthreads();

    if (!(wlb_min > kt + BN - 1 || wub_max < kt)) {
      // S^T = K Q^T for the wave's 32 queries and the tile's 64 keys.
      f32x16 s[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) s[kb] = zero16();
#pragma unroll
      for (int c = 0; c < KC; ++c) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const bf16x8 kfrag = as_bf16x8(lds_load16(Ks + 32 * kb * 2 * D, fo.nat(c)));
          s[kb] = M::mma(kfrag, qf[c], s[kb]);
        }
      }

      // Mask (only on tiles crossing a window or document edge), row maximum.
      const bool need_mask = !(wlb_max <= kt && kt + BN - 1 <= wub_min);
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kt + 32 * kb + acc_row(r, g);
            if (key < lb || key > ub) s[kb][r] = -INFINITY;
          }
        }
      }
      float mx = s[0][0];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      m_true = fmaxf(m_true, mx * c2);
      // Move the exponent reference only when probabilities would exceed 2^8.
      const bool move = m_true > m_ref + kRescaleThreshold;
      if (__builtin_amdgcn_ballot_w64(move) != 0) {
        // Lanes that keep their reference (possibly still -inf) scale by 1;
        // a reference moving up from -inf scales the empty state by 0.
        const float alpha = move ? __builtin_amdgcn_exp2f(m_ref - m_true) : 1.0f;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db] *= alpha;
        m_ref = move ? m_true : m_ref;
      }
      const float neg_m = m_ref == -INFINITY ? 0.0f : -m_ref;
      float psum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][r], c2, neg_m));
          s[kb][r] = p;
          psum += p;
        }
      }
      l_run += psum;

      // O^T += V^T P^T, 16 keys per product.
#pragma unroll
      for (int kc = 0; kc < BN / 16; ++kc) {
        const bf16x8 pf = (kc & 1) ? M::from_acc<1>(s[kc >> 1]) : M::from_acc<0>(s[kc >> 1]);
        const char* vchunk = Vs + 16 * kc * 2 * D;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16x8 vfrag = lds_tr_frag(vchunk, fo.tr(0, db), fo.tr(1, db));
          o[db] = M::mma(vfrag, pf, o[db]);
        }
      }
    }

    if (more) {
      char* nxt = smem + ((it + 1) & 1) * C::kStageBytes;
      kst.store(plan, nxt);
      vst.store(plan, nxt + C::kTileBytes);
    }
  }

  const float lt = l_run + __shfl_xor(l_run, 32);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
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
          for (int t = 0; t < 4; ++t) v[t] = o[db][4 * j + t] * inv;
          if (a.out_bf16) store4(static_cast<bf16*>(a.O) + orow * D + d0, v, false);
          else store4(static_cast<float*>(a.O) + orow * D + d0, v, false);
        }
      }
    }
    if (g == 0) {
      const int64_t si = ((int64_t)b * a.H + h) * T + q;
      const bool any = m_true != -INFINITY;
      a.l[si] = any ? lt * __builtin_amdgcn_exp2f(m_ref - m_true) : 0.0f;
      a.m[si] = any ? m_true * kLn2 : -kFltMax;
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
  switch (p.D) {
    case 16: return launch_fwd_fast_t<16>(p, a, s);
    case 32: return launch_fwd_fast_t<32>(p, a, s);
    case 64: return launch_fwd_fast_t<64>(p, a, s);
    case 128: return launch_fwd_fast_t<128>(p, a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fc
