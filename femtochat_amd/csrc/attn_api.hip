// C ABI of libfemtochat_attn.so: host-side validation, workspace sizing and
// dispatch to the gfx950 kernels.  Declarations and semantics are in
// include/femtochat_attn.h.
//
// Error handling mirrors the reference's rule that no exception crosses the
// foreign boundary (ext/reactant/cuda_call.jl:45-48): every failure becomes an
// fc_status plus a thread-local message.
#include "../../include/femtochat_attn.h"
#include "../../include/femtochat_loss.h"
#include "attn_launch.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace {

thread_local std::string g_last_error;

fc_status fail(fc_status code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
fc_status fail(fc_status code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

fc_status ok() {
  g_last_error.clear();
  return FC_OK;
}

}  // namespace

namespace fc {
hipError_t device_cus(int* cus) {
  static std::atomic<int> cache[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev >= 0 && dev < 64 && cache[dev].load(std::memory_order_relaxed) > 0) {
    *cus = cache[dev].load(std::memory_order_relaxed);
    return hipSuccess;
  }
  int n = 0;
  e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  if (n <= 0) return hipErrorInvalidDevice;
  if (dev >= 0 && dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  *cus = n;
  return hipSuccess;
}

// Shared with the other translation units of the library (fc_last_error).
fc_status set_error(fc_status code, const char* message) {
  g_last_error = message;
  return code;
}
void clear_error() { g_last_error.clear(); }
}  // namespace fc

namespace {

using fc::valid_dtype;

// Validates the descriptor and fills the normalised problem (attn_problem.hpp).
fc_status make_problem(const fc_attn_desc* d, fc::Problem* p) {
  char msg[256];
  const fc_status st = fc::make_problem(d, p, msg, sizeof(msg));
  if (st != FC_OK) return fail(st, "%s", msg);
  return FC_OK;
}

// ---- profiling --------------------------------------------------------------
struct Record {
  hipEvent_t begin, end;
  std::string kernel;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<Record> g_records;

}  // namespace

namespace fc {

ProfileMark profile_begin(hipStream_t s) {
  ProfileMark mk;
  {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (!g_prof_on) return mk;
  }
  hipEvent_t ev;
  if (hipEventCreate(&ev) != hipSuccess) return mk;
  (void)hipEventRecord(ev, s);
  mk.begin = ev;
  return mk;
}

void profile_end(const ProfileMark& mark, const char* kernel, hipStream_t s) {
  if (mark.begin == nullptr) return;
  hipEvent_t ev;
  if (hipEventCreate(&ev) != hipSuccess) {
    (void)hipEventDestroy(static_cast<hipEvent_t>(mark.begin));
    return;
  }
  (void)hipEventRecord(ev, s);
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_records.push_back(Record{static_cast<hipEvent_t>(mark.begin), ev, kernel});
}

}  // namespace fc

extern "C" {

int32_t fc_abi_version(void) { return FC_ATTN_ABI_VERSION; }

const char* fc_last_error(void) { return g_last_error.c_str(); }

uint32_t fc_attn_supported_head_dims(void) {
  uint32_t mask = 0;
  for (int D = 16; D <= 128; D += 16)
    if (fc::head_dim_supported(D)) mask |= 1u << (D / 16 - 1);
  return mask;
}

fc_status fc_attn_workspace_bytes(const fc_attn_desc* desc, int32_t pass, int32_t positions_given, size_t* bytes) {
  fc::Problem p;
  const fc_status st = make_problem(desc, &p);
  if (st != FC_OK) return st;
  if (bytes == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "bytes is null");
  p.positions = positions_given != 0;
  if (pass == FC_PASS_FORWARD) {
    *bytes = fc::fwd_workspace(p).total;
  } else if (pass == FC_PASS_BACKWARD) {
    *bytes = fc::bwd_workspace(p).total;
  } else {
    return fail(FC_ERR_INVALID_ARGUMENT, "unknown pass %d", pass);
  }
  return ok();
}

fc_status fc_attn_fwd(const fc_attn_desc* desc, const void* Q, const void* K, const void* V,
                      const int32_t* positions, void* O, float* l, float* m, void* workspace,
                      size_t workspace_bytes, void* stream) {
  fc::Problem p;
  fc_status st = make_problem(desc, &p);
  if (st != FC_OK) return st;
  if (Q == nullptr || K == nullptr || V == nullptr || O == nullptr || l == nullptr || m == nullptr)
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_attn_fwd: a required pointer is null");
  p.positions = positions != nullptr;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // The workspace is optional unless the head dim runs padded: with one,
  // fast mode with positions takes the query tiles in the work order.
  const fc::FwdWorkspace ws = fc::fwd_workspace(p);
  char* w = nullptr;
  if (ws.total > 0 && (workspace != nullptr || fc::padded(p))) {
    if (workspace == nullptr || workspace_bytes < ws.total)
      return fail(FC_ERR_WORKSPACE, "forward workspace needs %zu bytes, got %zu%s", ws.total, workspace_bytes,
                  fc::padded(p) ? " (head_dim runs on padded copies)" : "");
    if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
      return fail(FC_ERR_WORKSPACE, "workspace must be 256-byte aligned");
    w = static_cast<char*>(workspace);
  }
  hipError_t e = hipSuccess;
  // A non-compiled head dim: Q, K, V copied into rows of Dk values, zero
  // beyond D, and O written there first.
  const fc::PadWorkspace pw = fc::pad_workspace(p, false);
  void* Ok = O;
  if (fc::padded(p)) {
    const int64_t rq = (int64_t)p.B * p.T * p.H, rk = (int64_t)p.B * p.T * p.Hkv;
    const int in16 = p.bf16 ? 1 : 0;
    const fc::RepackArgs packs[3] = {{Q, w + pw.Q, rq, p.D, p.Dk, in16, in16, 0},
                                     {K, w + pw.K, rk, p.D, p.Dk, in16, in16, 0},
                                     {V, w + pw.V, rk, p.D, p.Dk, in16, in16, 0}};
    for (const fc::RepackArgs& r : packs) {
      e = fc::launch_repack(r, s);
      if (e != hipSuccess) return fail(FC_ERR_HIP, "padding launch failed: %s", hipGetErrorString(e));
    }
    Q = w + pw.Q;
    K = w + pw.K;
    V = w + pw.V;
    Ok = w + pw.O;
  }
  int32_t* order = nullptr;
  if (fc::ordered(p) && w != nullptr) {
    int32_t* chunk_lb = reinterpret_cast<int32_t*>(w + ws.chunk_lb);
    order = reinterpret_cast<int32_t*>(w + ws.qorder);
    e = fc::launch_bounds(p, fc::BoundsArgs{positions, chunk_lb, p.T, p.B, p.left}, s);
    if (e != hipSuccess) return fail(FC_ERR_HIP, "bounds launch failed: %s", hipGetErrorString(e));
    e = fc::launch_order(p, fc::OrderArgs{chunk_lb, order, nullptr, p.T, p.B, p.left, p.right}, s);
    if (e != hipSuccess) return fail(FC_ERR_HIP, "order launch failed: %s", hipGetErrorString(e));
  }
  fc::FwdArgs a{};
  a.Q = Q;
  a.K = K;
  a.V = V;
  a.pos = positions;
  a.order = order;
  a.local_order = fc::windowed(p) ? 1 : 0;
  a.O = Ok;
  a.l = l;
  a.m = m;
  a.H = p.H;
  a.Hkv = p.Hkv;
  a.T = p.T;
  a.B = p.B;
  a.group = p.group;
  a.left = p.left;
  a.right = p.right;
  a.out_bf16 = p.out_bf16 ? 1 : 0;
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)p.D));
  e = fc::launch_fwd(p, a, s);
  if (e != hipSuccess) return fail(FC_ERR_HIP, "forward launch failed: %s", hipGetErrorString(e));
  if (fc::padded(p)) {
    const int o16 = p.out_bf16 ? 1 : 0;
    e = fc::launch_repack(fc::RepackArgs{Ok, O, (int64_t)p.B * p.T * p.H, p.Dk, p.D, o16, o16, 0}, s);
    if (e != hipSuccess) return fail(FC_ERR_HIP, "unpadding launch failed: %s", hipGetErrorString(e));
  }
  return ok();
}

}  // extern "C"

namespace {

// Validation the two backward entry points share: the problem, the pointers.
fc_status bwd_problem(const char* who, const fc_attn_desc* desc, const void* dO, const void* Q, const void* K,
                      const void* V, const void* O, const float* l, const float* m, const int32_t* positions,
                      const void* dQ, const void* dK, const void* dV, fc::Problem* p) {
  const fc_status st = make_problem(desc, p);
  if (st != FC_OK) return st;
  if (dO == nullptr || Q == nullptr || K == nullptr || V == nullptr || O == nullptr || l == nullptr ||
      m == nullptr || dQ == nullptr || dK == nullptr || dV == nullptr)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: a required pointer is null", who);
  p->positions = positions != nullptr;
  return FC_OK;
}

// Launches the backward of a validated problem with its workspace at w
// (bwd_workspace(p).total bytes, 256-byte aligned).  Every workspace byte the
// kernels read is written earlier in the same sequence, so the workspace
// needs no clearing.
fc_status bwd_launch(const fc::Problem& p, const void* dO, const void* Q, const void* K, const void* V,
                     const void* O, const float* l, const float* m, const int32_t* positions, void* dQ, void* dK,
                     void* dV, char* w, hipStream_t s) {
  const fc::BwdWorkspace ws = fc::bwd_workspace(p);

  // Fast mode with bf16 O and dO: the dQ kernel computes the preprocess
  // itself and runs first; otherwise a preprocess launch (which also makes
  // the bf16 copy of an fp32 dO) precedes both kernels.
  const bool fused_stats = p.bf16 && p.out_bf16 && p.dout_bf16;
  fc::PreArgs pa{};
  pa.dO = dO;
  pa.O = O;
  pa.l = l;
  pa.m = m;
  pa.delta = reinterpret_cast<float*>(w + ws.delta);
  pa.lse2 = reinterpret_cast<float*>(w + ws.lse2);
  pa.dO16 = (p.bf16 && !p.dout_bf16) ? w + ws.dO16 : nullptr;
  int* queue = p.bf16 ? reinterpret_cast<int*>(w + ws.queue) : nullptr;
  pa.queue = fused_stats ? nullptr : queue;
  pa.H = p.H;
  pa.T = p.T;
  pa.B = p.B;
  pa.dO_bf16 = p.dout_bf16 ? 1 : 0;
  pa.O_bf16 = p.out_bf16 ? 1 : 0;
  hipError_t e = hipSuccess;
  if (!fused_stats) {
    e = fc::launch_bwd_pre(p, pa, s);
    if (e != hipSuccess) return fail(FC_ERR_HIP, "backward preprocess launch failed: %s", hipGetErrorString(e));
  }

  int32_t* chunk_lb = nullptr;
  if (p.positions) {
    chunk_lb = reinterpret_cast<int32_t*>(w + ws.chunk_lb);
    fc::BoundsArgs ba{positions, chunk_lb, p.T, p.B, p.left};
    e = fc::launch_bounds(p, ba, s);
    if (e != hipSuccess) return fail(FC_ERR_HIP, "bounds launch failed: %s", hipGetErrorString(e));
  }
  int32_t* qorder = nullptr;
  int32_t* korder = nullptr;
  if (fc::ordered(p)) {
    qorder = reinterpret_cast<int32_t*>(w + ws.qorder);
    korder = reinterpret_cast<int32_t*>(w + ws.korder);
    e = fc::launch_order(p, fc::OrderArgs{chunk_lb, qorder, korder, p.T, p.B, p.left, p.right}, s);
    if (e != hipSuccess) return fail(FC_ERR_HIP, "order launch failed: %s", hipGetErrorString(e));
  }

  fc::BwdArgs a{};
  a.dO = pa.dO16 != nullptr ? pa.dO16 : dO;
  a.Q = Q;
  a.K = K;
  a.V = V;
  a.delta = pa.delta;
  a.lse2 = pa.lse2;
  a.pos = positions;
  a.chunk_lb = chunk_lb;
  a.qorder = qorder;
  a.korder = korder;
  a.local_order = fc::windowed(p) ? 1 : 0;
  a.queue = queue;
  a.dQ = dQ;
  a.dK = dK;
  a.dV = dV;
  a.H = p.H;
  a.Hkv = p.Hkv;
  a.T = p.T;
  a.B = p.B;
  a.group = p.group;
  a.left = p.left;
  a.right = p.right;
  a.grad_bf16 = p.grad_bf16 ? 1 : 0;
  a.accumulate = p.accumulate ? 1 : 0;
  a.scale = (float)(1.0 / std::sqrt((double)p.D));
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)p.D));
  if (fused_stats) {
    a.stats = 1;
    a.O = O;
    a.l = l;
    a.m = m;
    a.delta_out = pa.delta;
    a.lse2_out = pa.lse2;
    e = fc::launch_bwd_dq(p, a, s);
    if (e != hipSuccess) return fail(FC_ERR_HIP, "dQ launch failed: %s", hipGetErrorString(e));
    e = fc::launch_bwd_dkdv(p, a, s);
    if (e != hipSuccess) return fail(FC_ERR_HIP, "dK/dV launch failed: %s", hipGetErrorString(e));
    return ok();
  }
  e = fc::launch_bwd_dkdv(p, a, s);
  if (e != hipSuccess) return fail(FC_ERR_HIP, "dK/dV launch failed: %s", hipGetErrorString(e));
  e = fc::launch_bwd_dq(p, a, s);
  if (e != hipSuccess) return fail(FC_ERR_HIP, "dQ launch failed: %s", hipGetErrorString(e));
  return ok();
}

// The backward of a validated problem: bwd_launch directly for a compiled
// head dim; otherwise the inputs are copied into rows of Dk values (zero
// beyond D), the kernels overwrite float32 gradients of that width, and
// their first D columns are added to (or written into) the caller's
// gradients, rounded once.
fc_status bwd_run(const fc::Problem& p, const void* dO, const void* Q, const void* K, const void* V,
                  const void* O, const float* l, const float* m, const int32_t* positions, void* dQ, void* dK,
                  void* dV, char* w, hipStream_t s) {
  if (!fc::padded(p)) return bwd_launch(p, dO, Q, K, V, O, l, m, positions, dQ, dK, dV, w, s);
  const fc::PadWorkspace pw = fc::pad_workspace(p, true);
  const int64_t rq = (int64_t)p.B * p.T * p.H, rk = (int64_t)p.B * p.T * p.Hkv;
  const int in16 = p.bf16 ? 1 : 0, o16 = p.out_bf16 ? 1 : 0, do16 = p.dout_bf16 ? 1 : 0;
  const fc::RepackArgs packs[5] = {{Q, w + pw.Q, rq, p.D, p.Dk, in16, in16, 0},
                                   {K, w + pw.K, rk, p.D, p.Dk, in16, in16, 0},
                                   {V, w + pw.V, rk, p.D, p.Dk, in16, in16, 0},
                                   {O, w + pw.O, rq, p.D, p.Dk, o16, o16, 0},
                                   {dO, w + pw.dO, rq, p.D, p.Dk, do16, do16, 0}};
  for (const fc::RepackArgs& r : packs) {
    const hipError_t e = fc::launch_repack(r, s);
    if (e != hipSuccess) return fail(FC_ERR_HIP, "padding launch failed: %s", hipGetErrorString(e));
  }
  const fc::Problem k = fc::kernel_problem(p, true);
  const fc_status st = bwd_launch(k, w + pw.dO, w + pw.Q, w + pw.K, w + pw.V, w + pw.O, l, m, positions, w + pw.dQ,
                                  w + pw.dK, w + pw.dV, w, s);
  if (st != FC_OK) return st;
  const int g16 = p.grad_bf16 ? 1 : 0, acc = p.accumulate ? 1 : 0;
  const fc::RepackArgs unpacks[3] = {{w + pw.dQ, dQ, rq, p.Dk, p.D, 0, g16, acc},
                                     {w + pw.dK, dK, rk, p.Dk, p.D, 0, g16, acc},
                                     {w + pw.dV, dV, rk, p.Dk, p.D, 0, g16, acc}};
  for (const fc::RepackArgs& r : unpacks) {
    const hipError_t e = fc::launch_repack(r, s);
    if (e != hipSuccess) return fail(FC_ERR_HIP, "unpadding launch failed: %s", hipGetErrorString(e));
  }
  return ok();
}

}  // namespace

extern "C" {

fc_status fc_attn_bwd(const fc_attn_desc* desc, const void* dO, const void* Q, const void* K, const void* V,
                      const void* O, const float* l, const float* m, const int32_t* positions, void* dQ,
                      void* dK, void* dV, void* workspace, size_t workspace_bytes, void* stream) {
  fc::Problem p;
  const fc_status st = bwd_problem("fc_attn_bwd", desc, dO, Q, K, V, O, l, m, positions, dQ, dK, dV, &p);
  if (st != FC_OK) return st;
  const fc::BwdWorkspace ws = fc::bwd_workspace(p);
  if (workspace == nullptr || workspace_bytes < ws.total)
    return fail(FC_ERR_WORKSPACE, "backward workspace needs %zu bytes, got %zu%s", ws.total, workspace_bytes,
                workspace == nullptr ? " (null)" : "");
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return fail(FC_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return bwd_run(p, dO, Q, K, V, O, l, m, positions, dQ, dK, dV, static_cast<char*>(workspace),
                 static_cast<hipStream_t>(stream));
}

}  // extern "C"

// Backward scratch of fc_attn_bwd_noalloc.  Each GPU the library runs on
// holds its own copy from the code object's load until the process ends.  In
// host code `scratch` names a host-side stand-in, never the device memory:
// the device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) unsigned char scratch[FC_ATTN_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[kMaxScratchDevices] = {};  // device ordinal -> that device's scratch

// The current device's scratch address, looked up on the first call on that
// device (with the device current, as hipGetSymbolAddress requires).
fc_status current_scratch(char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FC_ERR_HIP, "fc_attn_bwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(FC_ERR_UNSUPPORTED, "fc_attn_bwd_noalloc: device ordinal %d is %d or more", dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(FC_ERR_HIP, "fc_attn_bwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    if ((reinterpret_cast<uintptr_t>(ptr) & 255) != 0)
      return fail(FC_ERR_HIP, "fc_attn_bwd_noalloc: scratch on device %d is not 256-byte aligned", dev);
    g_scratch_ptr[dev] = static_cast<char*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return FC_OK;
}

}  // namespace

extern "C" {

fc_status fc_attn_bwd_noalloc(const fc_attn_desc* desc, const void* dO, const void* Q, const void* K, const void* V,
                              const void* O, const float* l, const float* m, const int32_t* positions, void* dQ,
                              void* dK, void* dV, void* stream) {
  fc::Problem p;
  fc_status st = bwd_problem("fc_attn_bwd_noalloc", desc, dO, Q, K, V, O, l, m, positions, dQ, dK, dV, &p);
  if (st != FC_OK) return st;
  const size_t need = fc::bwd_workspace(p).total;
  if (need > (size_t)FC_ATTN_NOALLOC_SCRATCH_BYTES)
    return fail(FC_ERR_WORKSPACE,
                "fc_attn_bwd_noalloc: the problem needs %zu bytes of scratch, more than the %zu the library holds "
                "per GPU (call fc_attn_bwd with a workspace instead)",
                need, (size_t)FC_ATTN_NOALLOC_SCRATCH_BYTES);
  char* w = nullptr;
  st = current_scratch(&w);
  if (st != FC_OK) return st;
  return bwd_run(p, dO, Q, K, V, O, l, m, positions, dQ, dK, dV, w, static_cast<hipStream_t>(stream));
}

// ---- attention prologue (rope_norm.hip) -----------------------------------
static fc_status rope_norm_args(const fc_rope_norm_desc* d, const void* X, const float* sin_table,
                                const float* cos_table, const char* who, fc::RopeNormArgs* a) {
  if (d == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "%s: descriptor is null", who);
  if (d->D <= 0 || d->NH <= 0 || d->T <= 0 || d->B <= 0 || d->table_len <= 0)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: sizes must be positive (D=%d NH=%d T=%d B=%d table_len=%d)", who, d->D,
                d->NH, d->T, d->B, d->table_len);
  if (d->D % 16 != 0 || d->D > 128)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: head_dim %d must be a multiple of 16 and at most 128", who, d->D);
  if (d->D != 16 && d->D != 32 && d->D != 64 && d->D != 128)
    return fail(FC_ERR_UNSUPPORTED, "%s: head_dim %d is not compiled in (supported: 16, 32, 64, 128)", who, d->D);
  if (!valid_dtype(d->dtype)) return fail(FC_ERR_INVALID_ARGUMENT, "%s: dtype must be FC_F32 or FC_BF16", who);
  if ((d->flags & ~FC_FLAG_OVERWRITE) != 0)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: unknown flag bits 0x%x", who, d->flags);
  const int64_t vectors = (int64_t)d->B * d->T * d->NH;
  if (vectors >= ((int64_t)1 << 30) || (int64_t)d->table_len * d->D >= INT32_MAX)
    return fail(FC_ERR_UNSUPPORTED, "%s: problem too large", who);
  if (X == nullptr || sin_table == nullptr || cos_table == nullptr)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: a required pointer is null", who);
  if ((reinterpret_cast<uintptr_t>(sin_table) | reinterpret_cast<uintptr_t>(cos_table) |
       reinterpret_cast<uintptr_t>(X)) % 16 != 0)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: X and the tables must be 16-byte aligned", who);
  *a = fc::RopeNormArgs{};
  a->X = X;
  a->sin_t = sin_table;
  a->cos_t = cos_table;
  a->vectors = (int)vectors;
  a->NH = d->NH;
  a->T = d->T;
  a->by_NH = fc::fast_div((uint32_t)d->NH);
  a->by_T = fc::fast_div((uint32_t)d->T);
  a->table_len = d->table_len;
  return FC_OK;
}

fc_status fc_rope_norm_fwd(const fc_rope_norm_desc* desc, const void* X, const float* sin_table,
                           const float* cos_table, const int32_t* positions, void* Y, void* stream) {
  fc::RopeNormArgs a;
  const fc_status st = rope_norm_args(desc, X, sin_table, cos_table, "fc_rope_norm_fwd", &a);
  if (st != FC_OK) return st;
  if (Y == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "fc_rope_norm_fwd: Y is null");
  if (reinterpret_cast<uintptr_t>(Y) % 16 != 0)
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_rope_norm_fwd: Y must be 16-byte aligned");
  a.Y = Y;
  a.pos = positions;
  const hipError_t e = fc::launch_rope_norm(desc->D, desc->dtype == FC_BF16, a, false, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(FC_ERR_HIP, "prologue launch failed: %s", hipGetErrorString(e));
  return ok();
}

fc_status fc_rope_norm_bwd(const fc_rope_norm_desc* desc, const void* dY, const void* X, const float* sin_table,
                           const float* cos_table, const int32_t* positions, void* dX, void* stream) {
  fc::RopeNormArgs a;
  const fc_status st = rope_norm_args(desc, X, sin_table, cos_table, "fc_rope_norm_bwd", &a);
  if (st != FC_OK) return st;
  if (dY == nullptr || dX == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "fc_rope_norm_bwd: dY or dX is null");
  if ((reinterpret_cast<uintptr_t>(dY) | reinterpret_cast<uintptr_t>(dX)) % 16 != 0)
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_rope_norm_bwd: dY and dX must be 16-byte aligned");
  a.dY = dY;
  a.dX = dX;
  a.pos = positions;
  a.accumulate = (desc->flags & FC_FLAG_OVERWRITE) == 0 ? 1 : 0;
  const hipError_t e = fc::launch_rope_norm(desc->D, desc->dtype == FC_BF16, a, true, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(FC_ERR_HIP, "prologue backward launch failed: %s", hipGetErrorString(e));
  return ok();
}

// ---- loss side (loss.hip) ------------------------------------------------------
static bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3) == 0; }

static fc_status xent_args(const fc_xent_desc* d, const void* targets, const char* who, fc::XentArgs* a) {
  if (d == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "%s: descriptor is null", who);
  if (d->V <= 0 || d->N <= 0) return fail(FC_ERR_INVALID_ARGUMENT, "%s: V and N must be positive (V=%d N=%lld)", who, d->V, (long long)d->N);
  if (d->N > INT32_MAX) return fail(FC_ERR_UNSUPPORTED, "%s: at most 2^31-1 tokens per call", who);
  if (d->index_base != 0 && d->index_base != 1) return fail(FC_ERR_INVALID_ARGUMENT, "%s: index_base must be 0 or 1", who);
  if (d->index_type != FC_INDEX_I32 && d->index_type != FC_INDEX_I64)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: index_type must be FC_INDEX_I32 or FC_INDEX_I64", who);
  if (d->reduction < FC_REDUCE_NONE || d->reduction > FC_REDUCE_MEAN)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: unknown reduction %d", who, d->reduction);
  if ((d->flags & ~FC_FLAG_OVERWRITE) != 0) return fail(FC_ERR_INVALID_ARGUMENT, "%s: unknown flag bits 0x%x", who, d->flags);
  if (targets == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "%s: targets is null", who);
  if ((reinterpret_cast<uintptr_t>(targets) & (d->index_type == FC_INDEX_I64 ? 7 : 3)) != 0)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: targets are not aligned to their element size", who);
  *a = fc::XentArgs{};
  a->targets = targets;
  a->N = d->N;
  a->V = d->V;
  a->ignore_index = d->ignore_index;
  a->index_base = d->index_base;
  a->index_type = d->index_type;
  a->reduction = d->reduction;
  a->overwrite = (d->flags & FC_FLAG_OVERWRITE) != 0;
  return FC_OK;
}

fc_status fc_cross_entropy_fwd(const fc_xent_desc* desc, const float* logits, const void* targets, float* losses,
                               float* lse, float* reduced, float* count, void* stream) {
  fc::XentArgs a;
  const fc_status st = xent_args(desc, targets, "fc_cross_entropy_fwd", &a);
  if (st != FC_OK) return st;
  if (logits == nullptr || losses == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "fc_cross_entropy_fwd: logits and losses are required");
  if (!aligned4(logits) || !aligned4(losses) || !aligned4(lse) || !aligned4(reduced) || !aligned4(count))
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_cross_entropy_fwd: float buffers must be 4-byte aligned");
  a.logits = logits;
  a.losses = losses;
  a.lse = lse;
  a.reduced = reduced;
  a.count = count;
  const hipError_t e = fc::launch_xent_fwd(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(FC_ERR_HIP, "cross-entropy launch failed: %s", hipGetErrorString(e));
  return ok();
}

fc_status fc_cross_entropy_count(const fc_xent_desc* desc, const void* targets, float* count, void* stream) {
  fc::XentArgs a;
  const fc_status st = xent_args(desc, targets, "fc_cross_entropy_count", &a);
  if (st != FC_OK) return st;
  if (count == nullptr || !aligned4(count)) return fail(FC_ERR_INVALID_ARGUMENT, "fc_cross_entropy_count: count is null or misaligned");
  a.count = count;
  const hipError_t e = fc::launch_xent_count(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(FC_ERR_HIP, "count launch failed: %s", hipGetErrorString(e));
  return ok();
}

fc_status fc_cross_entropy_bwd(const fc_xent_desc* desc, float* dlogits, const float* logits, const void* targets,
                               const float* dy, const float* count, const float* lse, void* stream) {
  fc::XentArgs a;
  const fc_status st = xent_args(desc, targets, "fc_cross_entropy_bwd", &a);
  if (st != FC_OK) return st;
  if (dlogits == nullptr || logits == nullptr || dy == nullptr)
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_cross_entropy_bwd: dlogits, logits and dy are required");
  if (desc->reduction == FC_REDUCE_MEAN && count == nullptr)
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_cross_entropy_bwd: the mean gradient needs the valid-target count");
  if (!aligned4(dlogits) || !aligned4(logits) || !aligned4(dy) || !aligned4(count) || !aligned4(lse))
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_cross_entropy_bwd: float buffers must be 4-byte aligned");
  a.dlogits = dlogits;
  a.logits = logits;
  a.dy = dy;
  a.count = const_cast<float*>(count);
  a.lse_in = lse;
  const hipError_t e = fc::launch_xent_bwd(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(FC_ERR_HIP, "cross-entropy gradient launch failed: %s", hipGetErrorString(e));
  return ok();
}

fc_status fc_cross_entropy_fused(const fc_xent_desc* desc, const float* logits, const void* targets, float* losses,
                                 float* lse, float* reduced, float* dlogits, const float* dy, const float* count,
                                 void* stream) {
  fc::XentArgs a;
  const fc_status st = xent_args(desc, targets, "fc_cross_entropy_fused", &a);
  if (st != FC_OK) return st;
  if (logits == nullptr || losses == nullptr || dlogits == nullptr || dy == nullptr)
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_cross_entropy_fused: logits, losses, dlogits and dy are required");
  if (desc->reduction == FC_REDUCE_MEAN && count == nullptr)
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_cross_entropy_fused: the mean gradient needs the valid-target count");
  if (!aligned4(losses) || !aligned4(lse) || !aligned4(reduced) || !aligned4(dy) || !aligned4(count))
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_cross_entropy_fused: float buffers must be 4-byte aligned");
  a.logits = logits;
  a.losses = losses;
  a.lse = lse;
  a.reduced = reduced;
  a.dlogits = dlogits;
  a.dy = dy;
  a.count = const_cast<float*>(count);
  if (!fc::xent_fused_supported(a))
    return fail(FC_ERR_UNSUPPORTED,
                "fc_cross_entropy_fused: needs V a multiple of 4, V <= 32768 and 16-byte aligned logits and dlogits "
                "(use fc_cross_entropy_fwd and fc_cross_entropy_bwd)");
  const hipError_t e = fc::launch_xent_fused(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(FC_ERR_HIP, "fused cross-entropy launch failed: %s", hipGetErrorString(e));
  return ok();
}

static fc_status embed_args(const fc_embed_desc* d, const void* tokens, const char* who, fc::EmbedArgs* a) {
  if (d == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "%s: descriptor is null", who);
  if (d->D <= 0 || d->vocab <= 0 || d->N <= 0)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: D, vocab and N must be positive (D=%d vocab=%d N=%lld)", who, d->D, d->vocab,
                (long long)d->N);
  if ((d->N + 3) / 4 > INT32_MAX) return fail(FC_ERR_UNSUPPORTED, "%s: too many tokens per call", who);
  if (d->index_base != 0 && d->index_base != 1) return fail(FC_ERR_INVALID_ARGUMENT, "%s: index_base must be 0 or 1", who);
  if (d->index_type != FC_INDEX_I32 && d->index_type != FC_INDEX_I64)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: index_type must be FC_INDEX_I32 or FC_INDEX_I64", who);
  if (!valid_dtype(d->y_dtype)) return fail(FC_ERR_INVALID_ARGUMENT, "%s: y_dtype must be FC_F32 or FC_BF16", who);
  if (d->flags != 0) return fail(FC_ERR_INVALID_ARGUMENT, "%s: unknown flag bits 0x%x", who, d->flags);
  if (tokens == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "%s: tokens is null", who);
  if ((reinterpret_cast<uintptr_t>(tokens) & (d->index_type == FC_INDEX_I64 ? 7 : 3)) != 0)
    return fail(FC_ERR_INVALID_ARGUMENT, "%s: tokens are not aligned to their element size", who);
  *a = fc::EmbedArgs{};
  a->tokens = tokens;
  a->N = d->N;
  a->D = d->D;
  a->vocab = d->vocab;
  a->index_base = d->index_base;
  a->index_type = d->index_type;
  return FC_OK;
}

fc_status fc_embedding_fwd(const fc_embed_desc* desc, const float* weights, const void* tokens, void* y, void* stream) {
  fc::EmbedArgs a;
  const fc_status st = embed_args(desc, tokens, "fc_embedding_fwd", &a);
  if (st != FC_OK) return st;
  if (weights == nullptr || y == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "fc_embedding_fwd: weights and y are required");
  if (!aligned4(weights) || (reinterpret_cast<uintptr_t>(y) & (desc->y_dtype == FC_BF16 ? 1 : 3)) != 0)
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_embedding_fwd: buffers are not aligned to their element size");
  a.weights = weights;
  a.y = y;
  const hipError_t e = fc::launch_embed(a, false, desc->y_dtype == FC_BF16, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(FC_ERR_HIP, "embedding launch failed: %s", hipGetErrorString(e));
  return ok();
}

fc_status fc_embedding_bwd(const fc_embed_desc* desc, float* dweights, const void* dy, const void* tokens, void* stream) {
  fc::EmbedArgs a;
  const fc_status st = embed_args(desc, tokens, "fc_embedding_bwd", &a);
  if (st != FC_OK) return st;
  if (dweights == nullptr || dy == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "fc_embedding_bwd: dweights and dy are required");
  if (!aligned4(dweights) || (reinterpret_cast<uintptr_t>(dy) & (desc->y_dtype == FC_BF16 ? 1 : 3)) != 0)
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_embedding_bwd: buffers are not aligned to their element size");
  a.dweights = dweights;
  a.dy = dy;
  const hipError_t e = fc::launch_embed(a, true, desc->y_dtype == FC_BF16, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(FC_ERR_HIP, "embedding gradient launch failed: %s", hipGetErrorString(e));
  return ok();
}

fc_status fc_embedding_bwd_workspace_bytes(const fc_embed_desc* desc, size_t* bytes) {
  fc::EmbedArgs a;
  static const int64_t no_tokens = 0;  // the query reads no tokens (aligned for either index type)
  const fc_status st = embed_args(desc, &no_tokens, "fc_embedding_bwd_workspace_bytes", &a);
  if (st != FC_OK) return st;
  if (bytes == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "fc_embedding_bwd_workspace_bytes: bytes is null");
  if (desc->N >= ((int64_t)1 << 31)) return fail(FC_ERR_UNSUPPORTED, "fc_embedding_bwd_workspace_bytes: at most 2^31 - 1 tokens");
  *bytes = fc::embed_sort_layout(desc->N, desc->vocab).total;
  return ok();
}

fc_status fc_embedding_bwd_sorted(const fc_embed_desc* desc, float* dweights, const void* dy, const void* tokens,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  fc::EmbedArgs a;
  const fc_status st = embed_args(desc, tokens, "fc_embedding_bwd_sorted", &a);
  if (st != FC_OK) return st;
  if (dweights == nullptr || dy == nullptr)
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_embedding_bwd_sorted: dweights and dy are required");
  if (!aligned4(dweights) || (reinterpret_cast<uintptr_t>(dy) & (desc->y_dtype == FC_BF16 ? 1 : 3)) != 0)
    return fail(FC_ERR_INVALID_ARGUMENT, "fc_embedding_bwd_sorted: buffers are not aligned to their element size");
  if (desc->N >= ((int64_t)1 << 31)) return fail(FC_ERR_UNSUPPORTED, "fc_embedding_bwd_sorted: at most 2^31 - 1 tokens");
  const size_t need = fc::embed_sort_layout(desc->N, desc->vocab).total;
  if (workspace == nullptr || workspace_bytes < need)
    return fail(FC_ERR_WORKSPACE, "fc_embedding_bwd_sorted needs %zu workspace bytes, got %zu", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return fail(FC_ERR_WORKSPACE, "fc_embedding_bwd_sorted: workspace must be 256-byte aligned");
  a.dweights = dweights;
  a.dy = dy;
  const hipError_t e = fc::launch_embed_sorted(a, desc->y_dtype == FC_BF16, workspace, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(FC_ERR_HIP, "sorted embedding gradient launch failed: %s", hipGetErrorString(e));
  return ok();
}

fc_status fc_capabilities(int32_t device, fc_caps* caps) {
  if (caps == nullptr) return fail(FC_ERR_INVALID_ARGUMENT, "caps is null");
  hipDeviceProp_t prop;
  const hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return fail(FC_ERR_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  std::memset(caps, 0, sizeof(*caps));
  std::snprintf(caps->name, sizeof(caps->name), "%s", prop.name);
  std::snprintf(caps->arch, sizeof(caps->arch), "%s", prop.gcnArchName);
  caps->compute_units = prop.multiProcessorCount;
  caps->wavefront_size = prop.warpSize;
  caps->lds_bytes_per_block = (int32_t)prop.sharedMemPerBlock;
  caps->max_threads_per_block = prop.maxThreadsPerBlock;
  caps->clock_khz = prop.clockRate;
  caps->global_mem_bytes = (int64_t)prop.totalGlobalMem;
  return ok();
}

fc_status fc_profile_enable(int32_t enable) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_on = enable != 0;
  return ok();
}

fc_status fc_profile_collect(fc_kernel_time* out, int32_t capacity, int32_t* count) {
  std::vector<Record> recs;
  {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    recs.swap(g_records);
  }
  std::map<std::string, std::pair<int32_t, double>> agg;
  hipError_t err = hipSuccess;
  for (const Record& r : recs) {
    float ms = 0.0f;
    hipError_t e = hipEventSynchronize(r.end);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.begin, r.end);
    if (e != hipSuccess && err == hipSuccess) err = e;
    auto& slot = agg[r.kernel];
    slot.first += 1;
    slot.second += ms;
    (void)hipEventDestroy(r.begin);
    (void)hipEventDestroy(r.end);
  }
  if (err != hipSuccess) return fail(FC_ERR_HIP, "profile events: %s", hipGetErrorString(err));
  int32_t n = 0;
  for (const auto& kv : agg) {
    if (out != nullptr && n < capacity) {
      std::memset(&out[n], 0, sizeof(out[n]));
      std::snprintf(out[n].kernel, sizeof(out[n].kernel), "%s", kv.first.c_str());
      out[n].launches = kv.second.first;
      out[n].total_ms = kv.second.second;
    }
    ++n;
  }
  if (count != nullptr) *count = n;
  return ok();
}

}  // extern "C"
