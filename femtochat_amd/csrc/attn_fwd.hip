// Flash-attention forward for gfx950.
//
// Behaviour follows the reference forward (src/kernels.jl:131-219 for the
// semantics of O, l and m; ext/FemtoChatCUDAExt.jl:1295-1463 for the fast
// mode: fp32 statistics, P rounded to the input format before P.V, l summed
// from the unrounded probabilities).  The design is this file's own:
//
//  * one workgroup = 4 waves x 32 queries of one (batch, head); the grid is
//    spread over the 8 XCDs so that the query tiles of one head share an L2;
//  * each wave computes S^T = K Q^T (keys x queries) with 32x32 MFMA, so a
//    lane owns one query column: the online softmax needs one cross-lane
//    exchange (lane l <-> l^32) per key tile and the probabilities are already
//    the B operand of O^T += V^T P^T;
//  * K is staged in LDS in natural layout, V transposed (bf16) so that the
//    V^T operand is two 8-byte LDS reads per fragment; both double-buffered
//    with register prefetch, one barrier per key tile;
//  * key tiles outside [min lb, max ub] of the workgroup are never visited,
//    fully visible tiles skip the mask, and waves with no visible key in a
//    tile skip its products.
#include "attn_device.hpp"
#include "attn_launch.hpp"

#include <type_traits>

namespace fc {

template <typename E, int D>
struct FwdCfg {
  static constexpr bool kBF = std::is_same<E, bf16>::value;
  static constexpr int kBM = 128;                // queries per workgroup
  static constexpr int kBN = kBF ? 64 : 32;      // keys per tile
  static constexpr int kKC = D / 16;             // 16-wide head-dim chunks
  static constexpr int kDP = D < 32 ? 32 : D;    // head dim padded to 32
  static constexpr int kDB = kDP / 32;           // 32-wide head-dim blocks
  static constexpr int kLDK = kBF ? D + 8 : D + 4;   // K row stride
  static constexpr int kLDVT = kBN + 4;              // V^T row stride (bf16)
  static constexpr int kLDV = D + 4;                 // V row stride (fp32)
  static constexpr int kKElems = kBN * kLDK;
  static constexpr int kVElems = kBF ? kDP * kLDVT : kBN * kLDV;
  static constexpr int kStage = kKElems + kVElems;
};

template <typename E, int D>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(FwdArgs a) {
  using M = Mma<E>;
  using C = FwdCfg<E, D>;
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
  const E* Kb = static_cast<const E*>(a.K) + ((int64_t)b * T * a.Hkv + kvh) * D;
  const E* Vb = static_cast<const E*>(a.V) + ((int64_t)b * T * a.Hkv + kvh) * D;
  const int32_t* pos = a.pos ? a.pos + (int64_t)b * T : nullptr;

  const int q = qt * C::kBM + wave * 32 + l32;
  const int lb = key_lb(q, T, a.left, pos), ub = key_ub(q, T, a.right);
  const int wlb_min = wave_min32(lb), wlb_max = wave_max32(lb);
  const int wub_min = wave_min32(ub), wub_max = wave_max32(ub);
  if (lane == 0) {
    s_bounds[0][wave] = wlb_min;
    s_bounds[1][wave] = wub_max;
  }

  typename M::frag qf[KC];
#pragma unroll
  for (int c = 0; c < KC; ++c)
    qf[c] = q < T ? M::load8(Qb + (int64_t)q * qpitch + 16 * c + 8 * g) : M::zero();

  f32x16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) o[i] = zero16();
  float m_run = -INFINITY, l_run = 0.0f;

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
  if (ntiles > 0) {
    kst.load(Kb, kpitch, kt0, T, tid);
    vst.load(Vb, kpitch, kt0, T, tid);
    kst.store_nat(smem, C::kLDK, tid);
    if constexpr (C::kBF) vst.store_tr(smem + C::kKElems, C::kLDVT, tid);
    else vst.store_nat(smem + C::kKElems, C::kLDV, tid);
  }

  for (int it = 0; it < ntiles; ++it) {
    const int kt = kt0 + it * BN;
    const E* Ks = smem + (it & 1) * C::kStage;
    const E* Vs = Ks + C::kKElems;
    const bool more = it + 1 < ntiles;
    if (more) {
      kst.load(Kb, kpitch, kt + BN, T, tid);
      vst.load(Vb, kpitch, kt + BN, T, tid);
    }
    __syncthreads();

    const bool active = !(wlb_min > kt + BN - 1 || wub_max < kt);
    if (active) {
      f32x16 s[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) s[kb] = zero16();
#pragma unroll
      for (int c = 0; c < KC; ++c) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const auto kfrag = M::load8(Ks + (32 * kb + l32) * C::kLDK + 16 * c + 8 * g);
          s[kb] = M::mma(kfrag, qf[c], s[kb]);
        }
      }

      const bool need_mask = !(wlb_max <= kt && kt + BN - 1 <= wub_min);
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = s[kb][r] * a.scale_log2;
          if (need_mask) {
            const int key = kt + 32 * kb + acc_row(r, g);
            if (key < lb || key > ub) x = -INFINITY;
          }
          s[kb][r] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float safe = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - safe);
      float psum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(s[kb][r] - safe);
          s[kb][r] = p;
          psum += p;
        }
      }
      l_run = l_run * alpha + psum;
      m_run = m_new;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] *= alpha;

#pragma unroll
      for (int kc = 0; kc < BN / 16; ++kc) {
        const auto pf = (kc & 1) ? M::template from_acc<1>(s[kc >> 1]) : M::template from_acc<0>(s[kc >> 1]);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          typename M::frag vfrag;
          if constexpr (C::kBF) {
            vfrag = load_tr_bf16(Vs + (32 * db + l32) * C::kLDVT + 16 * kc, g);
          } else {
            const int col = D < 32 ? min(32 * db + l32, D - 1) : 32 * db + l32;  // rows >= D unused
            vfrag = load_kt_f32(Vs + 16 * kc * C::kLDV + col, C::kLDV, g);
          }
          o[db] = M::mma(vfrag, pf, o[db]);
        }
      }
    }

    if (more) {
      E* Kn = smem + ((it + 1) & 1) * C::kStage;
      kst.store_nat(Kn, C::kLDK, tid);
      if constexpr (C::kBF) vst.store_tr(Kn + C::kKElems, C::kLDVT, tid);
      else vst.store_nat(Kn + C::kKElems, C::kLDV, tid);
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
      a.l[si] = lt;
      a.m[si] = m_run == -INFINITY ? -kFltMax : m_run * kLn2;
    }
  }
}

template <typename E, int D>
static hipError_t launch_fwd_t(const Problem& p, const FwdArgs& a, hipStream_t s) {
  const int n_qt = (p.T + FwdCfg<E, D>::kBM - 1) / FwdCfg<E, D>::kBM;
  const dim3 grid(n_qt * p.H * p.B), block(kThreads);
  const ProfileMark mk = profile_begin(s);
  hipLaunchKernelGGL((attn_fwd_kernel<E, D>), grid, block, 0, s, a);
  const hipError_t e = hipGetLastError();
  profile_end(mk, p.bf16 ? "attn_fwd_bf16" : "attn_fwd_f32", s);
  return e;
}

template <typename E>
static hipError_t launch_fwd_e(const Problem& p, const FwdArgs& a, hipStream_t s) {
  switch (p.Dk) {
    case 16: return launch_fwd_t<E, 16>(p, a, s);
    case 32: return launch_fwd_t<E, 32>(p, a, s);
    case 64: return launch_fwd_t<E, 64>(p, a, s);
    case 128: return launch_fwd_t<E, 128>(p, a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fwd(const Problem& p, const FwdArgs& a, hipStream_t s) {
  return p.bf16 ? launch_fwd_fast(p, a, s) : launch_fwd_e<float>(p, a, s);
}


}  // namespace fc
