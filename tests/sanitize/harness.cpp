// Host-only harness run under AddressSanitizer and UndefinedBehaviorSanitizer
// by tests/test_sanitize.py: the attention descriptor validation and the
// backward workspace layout (femtochat_amd/csrc/attn_problem.hpp, the code
// every entry point runs on the host before a launch), and the float32 FA-1
// restatement oracle/fa1.c on ragged shapes, checked against a direct float64
// softmax attention.
#include "../../femtochat_amd/csrc/attn_index.hpp"
#include "../../femtochat_amd/csrc/attn_problem.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

extern "C" {
void fa1_forward(const float* Q, const float* K, const float* V, const int* positions, float* O, float* l, float* m,
                 int D, int H, int Hkv, int T, int B, int left, int right, int causal, int nthreads);
void fa1_backward(const float* dO, const float* Q, const float* K, const float* V, const float* O, const float* l,
                  const float* m, const int* positions, float* dQ, float* dK, float* dV, int D, int H, int Hkv,
                  int T, int B, int left, int right, int causal, int nthreads);
}

static int failures = 0;
#define CHECK(cond)                                                    \
  do {                                                                 \
    if (!(cond)) {                                                     \
      std::fprintf(stderr, "FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond); \
      ++failures;                                                      \
    }                                                                  \
  } while (0)

static fc_attn_desc desc(int D, int H, int Hkv, int T, int B, int mode = FC_MODE_FAST) {
  fc_attn_desc d;
  std::memset(&d, 0, sizeof(d));
  d.D = D, d.H = H, d.Hkv = Hkv, d.T = T, d.B = B, d.win_left = -1, d.win_right = 0, d.mode = mode;
  const int t = mode == FC_MODE_FAST ? FC_BF16 : FC_F32;
  d.in_dtype = d.out_dtype = d.dout_dtype = d.grad_dtype = t;
  return d;
}

static void validation() {
  char msg[256];
  fc::Problem p;
  // valid descriptors, windows normalised
  fc_attn_desc d = desc(128, 10, 5, 2048, 16);
  CHECK(fc::make_problem(&d, &p, msg, sizeof msg) == FC_OK);
  CHECK(p.left == 2048 && p.right == 0 && p.group == 2 && p.bf16 && p.accumulate);
  d.win_left = 1 << 30, d.win_right = -(1 << 30);
  CHECK(fc::make_problem(&d, &p, msg, sizeof msg) == FC_OK && p.left == 2048 && p.right == -2049);
  // invalid ones, each with a message that fits the buffer
  const struct {
    int D, H, Hkv, T, B, mode, flags;
    fc_status want;
  } bad[] = {{128, 5, 2, 64, 1, FC_MODE_FAST, 0, FC_ERR_INVALID_ARGUMENT},
             {24, 4, 2, 64, 1, FC_MODE_FAST, 0, FC_ERR_INVALID_ARGUMENT},
             {144, 4, 2, 64, 1, FC_MODE_FAST, 0, FC_ERR_INVALID_ARGUMENT},
             {128, 4, 2, 0, 1, FC_MODE_FAST, 0, FC_ERR_INVALID_ARGUMENT},
             {128, 4, 2, 64, -3, FC_MODE_FAST, 0, FC_ERR_INVALID_ARGUMENT},
             {128, 4, 2, 64, 1, 9, 0, FC_ERR_INVALID_ARGUMENT},
             {128, 4, 2, 64, 1, FC_MODE_FAST, 8, FC_ERR_INVALID_ARGUMENT},
             {128, 10, 5, 1 << 21, 1, FC_MODE_FAST, 0, FC_ERR_UNSUPPORTED},  // slice past 2^31 bytes
             {128, 1 << 20, 1, 1 << 20, 1 << 10, FC_MODE_FAST, 0, FC_ERR_UNSUPPORTED}};
  for (const auto& b : bad) {
    fc_attn_desc e = desc(b.D, b.H, b.Hkv, b.T, b.B);
    e.mode = b.mode;
    e.flags = (uint32_t)b.flags;
    char small[24];  // truncation must stay inside the buffer
    CHECK(fc::make_problem(&e, &p, small, sizeof small) == b.want);
    CHECK(std::strlen(small) < sizeof small);
  }
  CHECK(fc::make_problem(nullptr, &p, msg, sizeof msg) == FC_ERR_INVALID_ARGUMENT);
  // Every multiple of 16 up to 128 is accepted; the kernels run the next
  // compiled width, and the padded copies lead both workspaces without
  // overlapping each other or the kernels' own regions.
  for (int D = 16; D <= 128; D += 16) {
    for (int mode : {FC_MODE_FAST, FC_MODE_EXACT}) {
      fc_attn_desc e = desc(D, 4, 2, 333, 3, mode);
      CHECK(fc::make_problem(&e, &p, msg, sizeof msg) == FC_OK);
      CHECK(p.D == D && p.Dk >= D && p.Dk - D < 64 && fc::head_dim_compiled(p.Dk));
      CHECK(fc::padded(p) == !fc::head_dim_compiled(D));
      const size_t el = mode == FC_MODE_FAST ? 2 : 4, nq = 3ull * 333 * 4 * p.Dk, nk = 3ull * 333 * 2 * p.Dk;
      const fc::PadWorkspace pf = fc::pad_workspace(p, false), pb = fc::pad_workspace(p, true);
      if (!fc::padded(p)) {
        CHECK(pf.inner == 0 && pb.inner == 0 && fc::fwd_workspace(p).total == 0);
        continue;
      }
      CHECK(pf.Q == 0 && pf.K >= nq * el && pf.V >= pf.K + nk * el && pf.O >= pf.V + nk * el &&
            pf.inner >= pf.O + nq * el);
      CHECK(pb.dO >= pb.O + nq * el && pb.dQ >= pb.dO + nq * el && pb.dK >= pb.dQ + nq * 4 &&
            pb.dV >= pb.dK + nk * 4 && pb.inner >= pb.dV + nk * 4);
      CHECK(pb.inner % 256 == 0 && pb.dQ % 256 == 0);
      CHECK(fc::fwd_workspace(p).total == pf.inner);
      const fc::BwdWorkspace bw = fc::bwd_workspace(p);
      CHECK(bw.delta == pb.inner && bw.total > pb.inner);
      const fc::Problem k = fc::kernel_problem(p, true);
      CHECK(!k.grad_bf16 && !k.accumulate && k.D == D && k.Dk == p.Dk && fc::bwd_workspace(k).total == bw.total);
    }
  }
  fc_attn_desc x = desc(64, 4, 2, 100, 3, FC_MODE_EXACT);
  x.in_dtype = FC_BF16;
  CHECK(fc::make_problem(&x, &p, msg, sizeof msg) == FC_ERR_INVALID_ARGUMENT);
  // workspace layout: 256-aligned, growing with positions and an fp32 dO copy
  fc_attn_desc w = desc(128, 4, 2, 1000, 3);
  CHECK(fc::make_problem(&w, &p, msg, sizeof msg) == FC_OK);
  const fc::BwdWorkspace a = fc::bwd_workspace(p);
  p.positions = true;
  const fc::BwdWorkspace b = fc::bwd_workspace(p);
  p.dout_bf16 = false;
  const fc::BwdWorkspace c = fc::bwd_workspace(p);
  CHECK(a.total % 256 == 0 && b.total > a.total && c.total >= b.total + 2ull * 3 * 4 * 1000 * 128);
  CHECK(a.delta % 256 == 0 && a.lse2 % 256 == 0 && b.chunk_lb % 256 == 0 && c.dO16 % 256 == 0);
  // The regions of the ordered backward (fast mode, positions) follow each
  // other without overlap and end at total; the forward's workspace holds
  // only the chunk bounds and the query order, and only in that case.
  const size_t nchunk = 3 * 32 * 2 * 4, norder = 3 * 8 * 4;  // ceil(1000/32) chunks, ceil(1000/128) tiles
  CHECK(fc::ordered(p));
  CHECK(c.lse2 >= c.delta + 4ull * 3 * 4 * 1000 && c.chunk_lb >= c.lse2 + 4ull * 3 * 4 * 1000);
  CHECK(c.dO16 >= c.chunk_lb + nchunk && c.queue >= c.dO16 + 2ull * 3 * 4 * 1000 * 128);
  CHECK(c.qorder >= c.queue + fc::kXcds * 4 && c.korder >= c.qorder + norder && c.total >= c.korder + norder);
  CHECK(c.qorder % 256 == 0 && c.korder % 256 == 0 && c.total % 256 == 0);
  const fc::FwdWorkspace f = fc::fwd_workspace(p);
  CHECK(f.chunk_lb == 0 && f.qorder >= nchunk && f.qorder % 256 == 0 && f.total >= f.qorder + norder);
  p.positions = false;
  CHECK(fc::fwd_workspace(p).total == 0 && !fc::ordered(p));
  p.positions = true;
  p.T = 128 * 4096, p.B = 1;
  CHECK(fc::ordered(p) && fc::order_fits(p.T, p.B));
  p.T += 1;
  CHECK(!fc::ordered(p) && fc::fwd_workspace(p).total == 0);
}

// float64 softmax attention, one (batch, head), for the comparison.
static void naive(const std::vector<float>& Q, const std::vector<float>& K, const std::vector<float>& V, int D,
                  int H, int Hkv, int T, int b, int h, int left, int right, int causal, const int* pos,
                  std::vector<double>& O) {
  const int kv = h / (H / Hkv);
  std::vector<double> s(T);
  for (int q = 0; q < T; ++q) {
    double mx = -INFINITY;
    for (int k = 0; k < T; ++k) {
      bool vis = causal ? k <= q : (q - left <= k && k <= q + right);
      if (pos) vis = vis && k >= q - pos[b * T + q];
      double acc = 0;
      for (int d = 0; d < D; ++d)
        acc += (double)Q[((size_t)(b * T + q) * H + h) * D + d] * K[((size_t)(b * T + k) * Hkv + kv) * D + d];
      s[k] = vis ? acc / std::sqrt((double)D) : -INFINITY;
      mx = std::fmax(mx, s[k]);
    }
    double sum = 0;
    for (int k = 0; k < T; ++k) sum += s[k] == -INFINITY ? 0 : std::exp(s[k] - mx);
    for (int d = 0; d < D; ++d) {
      double o = 0;
      for (int k = 0; k < T; ++k)
        if (s[k] != -INFINITY) o += std::exp(s[k] - mx) / sum * V[((size_t)(b * T + k) * Hkv + kv) * D + d];
      O[(size_t)q * D + d] = o;
    }
  }
}

static void restatement(int D, int H, int Hkv, int T, int B, int left, int right, int causal, bool with_pos) {
  const size_t nq = (size_t)B * T * H * D, nk = (size_t)B * T * Hkv * D;
  std::vector<float> Q(nq), K(nk), V(nk), dO(nq), O(nq), l((size_t)B * H * T), m((size_t)B * H * T);
  std::vector<float> dQ(nq, 0.f), dK(nk, 0.f), dV(nk, 0.f);
  std::vector<int> pos((size_t)B * T);
  unsigned s = 12345u + (unsigned)T;
  auto rnd = [&]() {
    s = s * 1664525u + 1013904223u;
    return ((s >> 8) & 0xffff) / 32768.0f - 1.0f;
  };
  for (auto* v : {&Q, &K, &V, &dO})
    for (auto& x : *v) x = rnd();
  for (int b = 0; b < B; ++b)
    for (int t = 0, p = 3 * b; t < T; ++t, ++p) {
      if (p > 17 + 5 * b) p = 0;  // documents of a few lengths
      pos[(size_t)b * T + t] = p;
    }
  const int* P = with_pos ? pos.data() : nullptr;
  fa1_forward(Q.data(), K.data(), V.data(), P, O.data(), l.data(), m.data(), D, H, Hkv, T, B, left, right, causal, 1);
  fa1_backward(dO.data(), Q.data(), K.data(), V.data(), O.data(), l.data(), m.data(), P, dQ.data(), dK.data(),
               dV.data(), D, H, Hkv, T, B, left, right, causal, 1);
  double err = 0, scale = 0;
  std::vector<double> ref((size_t)T * D);
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      naive(Q, K, V, D, H, Hkv, T, b, h, left, right, causal, P, ref);
      for (int q = 0; q < T; ++q)
        for (int d = 0; d < D; ++d) {
          err = std::fmax(err, std::fabs(O[((size_t)(b * T + q) * H + h) * D + d] - ref[(size_t)q * D + d]));
          scale = std::fmax(scale, std::fabs(ref[(size_t)q * D + d]));
        }
    }
  for (auto* v : {&dQ, &dK, &dV})
    for (float x : *v) CHECK(std::isfinite(x));
  std::printf("fa1 D=%d H=%d Hkv=%d T=%d B=%d window=(%d,%d) causal=%d pos=%d: max|O-O64|/max|O64| = %.2e\n", D, H,
              Hkv, T, B, left, right, causal, (int)with_pos, err / scale);
  CHECK(err <= 1e-5 * scale);
}

// The row-local grid order of the fast forward (local_query_item with
// local_full_from, as attn_fwd_fast.hip calls them) must name every
// (batch, head, tile) item exactly once, with every index in range, for any
// window the descriptor accepts (left clamped to [-T-1, T]; a window that
// starts right of the query has left < 0).
static void grid_orders() {
  const int BM = 128;
  struct Shape { int B, Hkv, group, T; };
  const Shape shapes[] = {{16, 5, 2, 2048}, {2, 4, 2, 1000}, {3, 3, 1, 777}, {8, 1, 4, 300}, {1, 2, 3, 129}};
  for (const Shape& sh : shapes) {
    const int n_qt = (sh.T + BM - 1) / BM, H = sh.Hkv * sh.group, n_items = n_qt * H * sh.B;
    const int lefts[] = {-sh.T - 1, -300, -255, -256, -128, -127, -1, 0, 1, 127, 128, 129, 512, sh.T / 2, sh.T};
    for (int left : lefts) {
      const int full_from = fc::local_full_from(n_qt, left, BM);
      CHECK(full_from >= 0 && full_from <= n_qt);
      std::vector<int> seen((size_t)n_items, 0);
      bool in_range = true;
      for (int id = 0; id < n_items; ++id) {
        int b = -1, h = -1, tile = -1;
        fc::local_query_item(id, n_items, n_qt, full_from, sh.B, sh.Hkv, sh.group, b, h, tile);
        if (b < 0 || b >= sh.B || h < 0 || h >= H || tile < 0 || tile >= n_qt) {
          in_range = false;
          continue;
        }
        ++seen[((size_t)b * H + h) * n_qt + tile];
      }
      CHECK(in_range);
      bool once = true;
      for (int c : seen) once = once && c == 1;
      if (!in_range || !once)
        std::fprintf(stderr, "local order B=%d Hkv=%d group=%d T=%d left=%d is not a bijection\n", sh.B, sh.Hkv,
                     sh.group, sh.T, left);
      CHECK(once);
    }
  }
  // The accumulate epilogue's row for every lane of every wave: inside the
  // slice for ragged T, and the lane's own row whenever that row exists.
  for (int T : {1, 31, 32, 33, 129, 150, 777, 2000, 2048}) {
    const int n_waves = (T + 127) / 128 * 4;
    for (int w = 0; w < n_waves; ++w)
      for (int row = 0; row < 32; ++row) {
        const int q0 = 32 * w, r = fc::epilogue_row(q0, row, T);
        CHECK(r >= 0 && r < T);
        if (q0 + row < T) CHECK(r == q0 + row);
      }
  }
}

int main() {
  validation();
  grid_orders();
  restatement(16, 2, 1, 37, 2, -1, 0, 1, false);
  restatement(32, 4, 2, 600, 1, 100, 0, 0, false);  // two key blocks, a ragged one
  restatement(16, 2, 2, 530, 1, 50, 20, 0, true);
  restatement(16, 3, 1, 513, 1, -1, 0, 1, true);
  if (failures) {
    std::fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  std::printf("ok\n");
  return 0;
}
