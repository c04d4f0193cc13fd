// ABI identity, error strings and per-device launch limits.
// Reference counterpart: sparse_pooling/kernels/cuda/abi.cu:17-62 (version + struct layouts) and
// kernels/cuda/launch.cuh:15-82 (per-device attribute cache guarded by a mutex).
#include <mutex>

#include "gl_common.h"
#include "gl_internal.h"

namespace gl {

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
size_t g_lds[kMaxDevices];  // 0 = not queried yet
}  // namespace

size_t max_lds_bytes() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_lds[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) return 0;
    g_lds[dev] = (size_t)v;
  }
  return g_lds[dev];
}

int set_lds_limit(const void* kernel, size_t bytes) {
  if (bytes <= 65536) return 0;
  if (bytes > max_lds_bytes()) return GL_ERR_LDS;
  hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  return e == hipSuccess ? 0 : (int)e;
}

namespace {
std::mutex g_trace_mu;
void** g_trace_events = nullptr;
int32_t* g_trace_ids = nullptr;
int g_trace_cap = 0, g_trace_used = 0;
bool g_trace_open = false;  // an event pair is half recorded
}  // namespace

void trace_before(hipStream_t s, int kernel_id) {
  std::lock_guard<std::mutex> lk(g_trace_mu);
  g_trace_open = false;
  if (!g_trace_events || g_trace_used >= g_trace_cap) return;
  if (hipEventRecord((hipEvent_t)g_trace_events[2 * g_trace_used], s) != hipSuccess) return;
  g_trace_ids[g_trace_used] = kernel_id;
  g_trace_open = true;
}

void trace_after(hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_trace_mu);
  if (!g_trace_open) return;
  g_trace_open = false;
  if (hipEventRecord((hipEvent_t)g_trace_events[2 * g_trace_used + 1], s) == hipSuccess) ++g_trace_used;
}

}  // namespace gl

using namespace gl;

#define OFF(S, f) ((long long)offsetof(S, f))

extern "C" int gl_abi_version(void) { return GL_ABI_VERSION; }

extern "C" int gl_trace_begin(void** events, int32_t* kernel_ids, int n_pairs) {
  if (!events || !kernel_ids || n_pairs < 1) return GL_ERR_ARG;
  std::lock_guard<std::mutex> lk(g_trace_mu);
  g_trace_events = events;
  g_trace_ids = kernel_ids;
  g_trace_cap = n_pairs;
  g_trace_used = 0;
  g_trace_open = false;
  return 0;
}

extern "C" int gl_trace_end(void) {
  std::lock_guard<std::mutex> lk(g_trace_mu);
  const int n = g_trace_used;
  g_trace_events = nullptr;
  g_trace_ids = nullptr;
  g_trace_cap = g_trace_used = 0;
  g_trace_open = false;
  return n;
}

extern "C" int gl_struct_layout(int which, long long* out, int n) {
  long long v[40];
  int c = 0;
  switch (which) {
    case 0: {
      typedef GlFwdArgs S;
      long long t[] = {(long long)sizeof(S), OFF(S, X), OFF(S, sxb), OFF(S, x_dtype), OFF(S, B), OFF(S, D), OFF(S, G),
                       OFF(S, S), OFF(S, K), OFF(S, act), OFF(S, pool), OFF(S, topk), OFF(S, rec_shift), OFF(S, sps), OFF(S, gs), OFF(S, idx), OFF(S, W),
                       OFF(S, bias), OFF(S, counts), OFF(S, sched), OFF(S, win), OFF(S, win_width), OFF(S, pre), OFF(S, winner),
                       OFF(S, pool_param), OFF(S, lse), OFF(S, ws),
                       OFF(S, ws_bytes), OFF(S, part_budget), OFF(S, w_dtype), OFF(S, relu_mask)};
      for (long long x : t) v[c++] = x;
      break;
    }
    case 1: {
      typedef GlBwdArgs S;
      long long t[] = {(long long)sizeof(S), OFF(S, X), OFF(S, sxb), OFF(S, x_dtype), OFF(S, B), OFF(S, D), OFF(S, G),
                       OFF(S, S), OFF(S, K), OFF(S, act), OFF(S, pool), OFF(S, topk), OFF(S, rec_shift), OFF(S, sps), OFF(S, gs), OFF(S, idx), OFF(S, W),
                       OFF(S, bias), OFF(S, counts), OFF(S, sched), OFF(S, win), OFF(S, win_width), OFF(S, g_pre), OFF(S, winner),
                       OFF(S, pool_param), OFF(S, pre), OFF(S, lse), OFF(S, dW),
                       OFF(S, db), OFF(S, dX), OFF(S, edges),
                       OFF(S, edges_bytes), OFF(S, ws), OFF(S, ws_bytes), OFF(S, dz_budget), OFF(S, w_dtype),
                       OFF(S, relu_mask)};
      for (long long x : t) v[c++] = x;
      break;
    }
    case 2: {
      typedef GlEdgeArgs S;
      long long t[] = {(long long)sizeof(S), OFF(S, idx), OFF(S, counts), OFF(S, D), OFF(S, G), OFF(S, S), OFF(S, K),
                       OFF(S, rec_shift), OFF(S, sps), OFF(S, gs), OFF(S, edges), OFF(S, edges_bytes), OFF(S, ws),
                       OFF(S, ws_bytes)};
      for (long long x : t) v[c++] = x;
      break;
    }
    case 3: {
      typedef GlAdamArgs S;
      long long t[] = {(long long)sizeof(S), OFF(S, p), OFF(S, g), OFF(S, m), OFF(S, v), OFF(S, n),
                       OFF(S, moments_dtype), OFF(S, lr), OFF(S, beta1), OFF(S, beta2), OFF(S, eps),
                       OFF(S, weight_decay), OFF(S, bc1), OFF(S, bc2), OFF(S, p_dtype), OFF(S, stochastic),
                       OFF(S, master), OFF(S, seed)};
      for (long long x : t) v[c++] = x;
      break;
    }
    case 4: {
      typedef GlCoverArgs S;
      long long t[] = {(long long)sizeof(S), OFF(S, W), OFF(S, a), OFF(S, nvalid), OFF(S, cand), OFF(S, R), OFF(S, gpb),
                       OFF(S, k), OFF(S, repair), OFF(S, importance), OFF(S, env), OFF(S, rec_idx), OFF(S, W_out),
                       OFF(S, missing0), OFF(S, swaps), OFF(S, loss), OFF(S, status)};
      for (long long x : t) v[c++] = x;
      break;
    }
    default:
      return GL_ERR_ARG;
  }
  if (out)
    for (int i = 0; i < c && i < n; ++i) out[i] = v[i];
  return c;
}

extern "C" const char* gl_error_string(int code) {
  switch (code) {
    case GL_OK: return "ok";
    case GL_ERR_ARG: return "invalid argument, shape or null pointer";
    case GL_ERR_UNSUPPORTED:
      return "unsupported variant (fan-in 8 or 16; activation identity|relu; pool mean|sum|max|topk_mean|lme|power|softmax)";
    case GL_ERR_WORKSPACE: return "workspace or output buffer smaller than required";
    case GL_ERR_LDS: return "a kernel's LDS working set exceeds the device's LDS per workgroup";
    case GL_ERR_EDGES: return "edge structure does not match this layer shape";
    case GL_ERR_DEVICE: return "no current HIP device or device attribute query failed";
    case GL_ERR_SCRATCH:
      return "gl_fwd_static: the partial results of one 4-token tile of this layer exceed the 64 MiB static scratch "
             "(use gl_fwd with a caller workspace)";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}
