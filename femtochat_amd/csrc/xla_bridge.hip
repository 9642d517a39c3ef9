// Native callbacks for an XLA typed-FFI custom call (include/femtochat_xla.h).
//
// The reference's handler (deps/reactant/xla_ffi.cpp:7-28) hands XLA's stream
// and the call's buffers, inputs then outputs, to `bool callback(void*,
// void**)`.  Each bound call site here gets its own function pointer: a pool
// of kSlots trampolines, trampoline i running the descriptor stored in slot i
// through the library's C entry points on XLA's stream.
#include "../../include/femtochat_xla.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cstdio>
#include <mutex>
#include <string>
#include <utility>

namespace {

constexpr int kSlots = 256;

enum Kind { kAttnFwd = 1, kAttnBwd, kEmbedFwd, kEmbedBwd };

struct Slot {
  int kind;
  bool positions;
  fc_attn_desc attn;
  fc_embed_desc embed;
  size_t ws_bytes;
};

Slot g_slots[kSlots];
std::atomic<int> g_used{0};
std::mutex g_error_mutex;
std::string g_error;
thread_local std::string g_error_copy;

void set_error(const char* what) {
  std::lock_guard<std::mutex> lock(g_error_mutex);
  g_error = what;
}

bool report(fc_status st, const char* where) {
  if (st == FC_OK) return true;
  char buf[640];
  std::snprintf(buf, sizeof(buf), "%s: %s", where, fc_last_error());
  set_error(buf);
  return false;
}

// dweights := 0 with a kernel (no memset node if XLA captures the call).
__global__ void zero_kernel(float* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = i; j < n; j += stride) p[j] = 0.0f;
}

bool run(const Slot& s, void* stream, void** b) {
  if (b == nullptr) {
    set_error("callback: buffers is null");
    return false;
  }
  switch (s.kind) {
    case kAttnFwd: {
      const int o = s.positions ? 4 : 3;  // first output
      return report(fc_attn_fwd(&s.attn, b[0], b[1], b[2], s.positions ? static_cast<const int32_t*>(b[3]) : nullptr,
                                b[o], static_cast<float*>(b[o + 1]), static_cast<float*>(b[o + 2]), nullptr, 0, stream),
                    "attention forward");
    }
    case kAttnBwd: {
      const int o = s.positions ? 8 : 7;
      // XLA aligns the buffers it allocates to 64 bytes; the workspace output
      // is declared 255 bytes longer than the library needs and used from its
      // first 256-byte boundary.
      void* ws = nullptr;
      if (s.ws_bytes > 0 && b[o + 3] != nullptr)
        ws = reinterpret_cast<void*>((reinterpret_cast<uintptr_t>(b[o + 3]) + 255) & ~uintptr_t(255));
      return report(fc_attn_bwd(&s.attn, b[0], b[1], b[2], b[3], b[4], static_cast<const float*>(b[5]),
                                static_cast<const float*>(b[6]),
                                s.positions ? static_cast<const int32_t*>(b[7]) : nullptr, b[o], b[o + 1], b[o + 2],
                                ws, s.ws_bytes, stream),
                    "attention backward");
    }
    case kEmbedFwd:
      return report(fc_embedding_fwd(&s.embed, static_cast<const float*>(b[0]), b[1], b[2], stream),
                    "embedding forward");
    case kEmbedBwd: {
      float* dw = static_cast<float*>(b[4]);
      const int64_t n = (int64_t)s.embed.D * s.embed.vocab;
      if (dw == nullptr) {
        set_error("embedding backward: dweights is null");
        return false;
      }
      const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
      hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), dw, n);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) {
        set_error(hipGetErrorString(e));
        return false;
      }
      return report(fc_embedding_bwd(&s.embed, dw, b[0], b[2], stream), "embedding backward");
    }
    default:
      set_error("callback: unbound slot");
      return false;
  }
}

template <int I>
bool trampoline(void* stream, void** buffers) {
  return run(g_slots[I], stream, buffers);
}

template <int... I>
constexpr std::array<fc_xla_callback, sizeof...(I)> make_table(std::integer_sequence<int, I...>) {
  return {{&trampoline<I>...}};
}

const std::array<fc_xla_callback, kSlots> g_table = make_table(std::make_integer_sequence<int, kSlots>{});

fc_xla_callback bind(const Slot& s) {
  const int i = g_used.fetch_add(1);
  if (i >= kSlots) {
    g_used.store(kSlots);
    set_error("all 256 callback slots are bound");
    return nullptr;
  }
  g_slots[i] = s;
  return g_table[i];
}

}  // namespace

extern "C" {

fc_xla_callback fc_xla_bind_attention_fwd(const fc_attn_desc* desc, int32_t has_positions) {
  size_t bytes = 0;
  // validates the descriptor on the host
  if (!report(fc_attn_workspace_bytes(desc, FC_PASS_FORWARD, has_positions != 0, &bytes), "bind attention forward"))
    return nullptr;
  // The forward call site has no workspace buffer (its outputs are O, l, m):
  // head dims that run zero-padded need one.
  if (desc->D != 16 && desc->D != 32 && desc->D != 64 && desc->D != 128) {
    char buf[256];
    std::snprintf(buf, sizeof(buf),
                  "bind attention forward: head_dim %d runs on padded copies in a workspace, which the XLA forward "
                  "call site does not provide (head_dim 16, 32, 64 and 128 need none)",
                  desc->D);
    set_error(buf);
    return nullptr;
  }
  Slot s{};
  s.kind = kAttnFwd;
  s.positions = has_positions != 0;
  s.attn = *desc;
  return bind(s);
}

fc_xla_callback fc_xla_bind_attention_bwd(const fc_attn_desc* desc, int32_t has_positions, size_t* workspace_bytes) {
  if (workspace_bytes == nullptr) {
    set_error("bind attention backward: workspace_bytes is null");
    return nullptr;
  }
  Slot s{};
  s.kind = kAttnBwd;
  s.positions = has_positions != 0;
  if (desc == nullptr) {
    set_error("bind attention backward: descriptor is null");
    return nullptr;
  }
  s.attn = *desc;
  s.attn.flags |= FC_FLAG_OVERWRITE;  // the compiled backward writes its gradients (accumulate=false)
  if (!report(fc_attn_workspace_bytes(&s.attn, FC_PASS_BACKWARD, s.positions, &s.ws_bytes), "bind attention backward"))
    return nullptr;
  // Room to round the buffer XLA hands over (64-byte aligned) up to 256 bytes.
  *workspace_bytes = s.ws_bytes > 0 ? s.ws_bytes + 255 : 0;
  return bind(s);
}

static bool embed_valid(const fc_embed_desc* desc, const char* who) {
  if (desc == nullptr || desc->D <= 0 || desc->vocab <= 0 || desc->N <= 0 || desc->flags != 0 ||
      (desc->index_base != 0 && desc->index_base != 1) ||
      (desc->index_type != FC_INDEX_I32 && desc->index_type != FC_INDEX_I64) ||
      (desc->y_dtype != FC_F32 && desc->y_dtype != FC_BF16)) {
    char buf[160];
    std::snprintf(buf, sizeof(buf), "%s: invalid embedding descriptor", who);
    set_error(buf);
    return false;
  }
  return true;
}

fc_xla_callback fc_xla_bind_embedding_fwd(const fc_embed_desc* desc) {
  if (!embed_valid(desc, "bind embedding forward")) return nullptr;
  Slot s{};
  s.kind = kEmbedFwd;
  s.embed = *desc;
  return bind(s);
}

fc_xla_callback fc_xla_bind_embedding_bwd(const fc_embed_desc* desc) {
  if (!embed_valid(desc, "bind embedding backward")) return nullptr;
  Slot s{};
  s.kind = kEmbedBwd;
  s.embed = *desc;
  return bind(s);
}

const char* fc_xla_last_error(void) {
  std::lock_guard<std::mutex> lock(g_error_mutex);
  g_error_copy = g_error;
  return g_error_copy.c_str();
}

}  // extern "C"
