// C ABI entry points of libwkv_hip.so (declared in include/wkv_hip.h).
//
// Argument checks happen here, on the host, before any launch: a kernel is
// only launched on shapes its grid and indexing were written for.  Nothing in
// this file allocates, frees or synchronises.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <initializer_list>
#include <mutex>
#include <string>

#include "../../include/wkv_hip.h"
#include "wkv_common.h"
#include "wkv_impl.h"

namespace wkv_host {

static thread_local std::string g_last_error;
// Events armed by wkv_time_next_call for the next entry point on this
// thread, and those of the entry point running now.
static thread_local CallEvents g_pending_events;
static thread_local CallEvents g_active_events;

CallEvents& active_events() { return g_active_events; }

// Moves the armed events (if any) to the running entry point for its
// duration.
struct TimingScope {
  TimingScope() {
    g_active_events = g_pending_events;
    g_pending_events = CallEvents{};
  }
  ~TimingScope() { g_active_events = CallEvents{}; }
};

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(WKV_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(err));
  }
  return WKV_OK;
}

// Channels per lane of the RWKV-4 kernels: 2 (one 32-bit bf16 pair / one
// 64-bit fp32 pair per lane per step) when that still gives every CU a row
// (B * ceil(C/128) >= 256 workgroups), else 1 for twice as many rows.
// WKV_VEC=1|2 in the environment overrides the choice (tuning only).
int pick_vec(int64_t B, int64_t C) {
  if (C % 2 != 0) return 1;
  static const int env = [] {
    const char* s = getenv("WKV_VEC");
    return s ? atoi(s) : 0;
  }();
  if (env == 1 || env == 2) return env;
  const int64_t rows2 = B * ((C + 127) / 128);
  return rows2 >= 256 ? 2 : 1;
}

// Parses "vec,L,W" from an environment variable (tile tuning only).
bool env_cfg(const char* name, int& vec, int& L, int& W) {
  const char* s = getenv(name);
  if (!s) return false;
  return sscanf(s, "%d,%d,%d", &vec, &L, &W) == 3;
}

int lb_poll_limit() {
  const char* s = getenv("WKV_LB_MAX_POLLS");
  if (!s) return wkv::kLbMaxPolls;
  return std::min(std::max(atoi(s), -1), wkv::kLbMaxPolls);
}

static bool dtype_ok(int dtype) { return dtype >= 0 && dtype <= 2; }

// Element-wise entry points work on whole 16-byte vectors.
static bool elementwise_ok(int64_t n, int dtype) {
  return n >= 0 && n % (dtype == 0 ? 4 : 8) == 0 && n / 8 < (int64_t(1) << 40);
}

// Tensors are read and written with vector instructions of up to 16 bytes.
static bool aligned16(std::initializer_list<const void*> ptrs) {
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
  return true;
}

// Every index the kernels form is int32 per dimension and size_t overall.
static bool dims_ok(int64_t B, int64_t T, int64_t C) {
  const int64_t lim = int64_t(1) << 31;
  return B >= 0 && T >= 0 && C >= 0 && B < lim && T < lim && C < lim && B * T < lim * 64;
}

// Fixed scratch of wkv4_backward_noalloc (checkpoint records, then the
// per-batch parameter-gradient partials).  Every GPU the library runs on holds
// its own copy until the process ends.  On the host this name is only a
// stand-in for the symbol: kernels get the device address that
// hipGetSymbolAddress returns for the current device (scratch_address below).
static __device__ __align__(256) unsigned char scratch[WKV4_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
static int scratch_address(void** out, const char* what) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess)
    return fail(WKV_ERR_LAUNCH, std::string(what) + ": hipGetDevice: " + hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(WKV_ERR_INVALID_ARGUMENT, std::string(what) + ": device index out of range");
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (err != hipSuccess || p == nullptr)
        return fail(WKV_ERR_LAUNCH, std::string(what) + ": hipGetSymbolAddress(scratch): " +
                                        hipGetErrorString(err));
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return WKV_OK;
}

}  // namespace wkv_host

using namespace wkv_host;

extern "C" {

size_t wkv4_forward_workspace_bytes(int64_t B, int64_t T, int64_t C) {
  if (!dims_ok(B, T, C)) return 0;
  return wkv4_fwd_workspace_bytes_impl(B, T, C);
}

// Shared checks of the forward entry points; 0 = proceed, -1 = nothing to
// do, else the status.
static int check_forward(const char* what, const void* k, const void* v, const float* td,
                         const float* tf, const void* r, bool need_r, const void* y, bool need_y,
                         const float* ck, bool need_ck, const void* ws, int64_t B, int64_t T,
                         int64_t C, int dtype) {
  const std::string w(what);
  if (!dtype_ok(dtype)) return fail(WKV_ERR_INVALID_ARGUMENT, w + ": unknown dtype");
  if (!dims_ok(B, T, C)) return fail(WKV_ERR_INVALID_ARGUMENT, w + ": bad sizes");
  if (B == 0 || T == 0 || C == 0) return -1;
  if (!k || !v || !td || !tf || (need_r && !r) || (need_y && !y) || (need_ck && !ck))
    return fail(WKV_ERR_INVALID_ARGUMENT, w + ": null pointer");
  if (!aligned16({k, v, r, y, ck, ws}))
    return fail(WKV_ERR_INVALID_ARGUMENT, w + ": tensors and workspace must be 16-byte aligned");
  return 0;
}

int wkv4_forward(const void* k, const void* v, const float* time_decay, const float* time_first,
                 void* y, void* workspace, size_t workspace_bytes, int64_t B, int64_t T,
                 int64_t C, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  const int rc = check_forward("wkv4_forward", k, v, time_decay, time_first, nullptr, false, y,
                               true, nullptr, false, workspace, B, T, C, dtype);
  if (rc) return rc < 0 ? WKV_OK : rc;
  return wkv4_forward_impl(k, v, time_decay, 0, time_first, y, nullptr, workspace,
                           workspace ? workspace_bytes : 0, int(B), int(T), int(C), dtype,
                           static_cast<hipStream_t>(stream));
}

size_t wkv4_checkpoint_bytes(int64_t B, int64_t T, int64_t C) {
  if (!dims_ok(B, T, C)) return 0;
  return wkv4_checkpoint_floats(B, T, C) * sizeof(float);
}

int wkv4_forward_checkpointed(const void* k, const void* v, const float* time_decay,
                              const float* time_first, void* y, float* checkpoint,
                              void* workspace, size_t workspace_bytes, int64_t B, int64_t T,
                              int64_t C, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  const int rc = check_forward("wkv4_forward_checkpointed", k, v, time_decay, time_first, nullptr,
                               false, y, false, checkpoint, true, workspace, B, T, C, dtype);
  if (rc) return rc < 0 ? WKV_OK : rc;
  return wkv4_forward_impl(k, v, time_decay, 0, time_first, y, checkpoint, workspace,
                           workspace ? workspace_bytes : 0, int(B), int(T), int(C), dtype,
                           static_cast<hipStream_t>(stream));
}

size_t wkv4_backward_workspace_bytes(int64_t B, int64_t T, int64_t C, int dtype) {
  if (!dtype_ok(dtype) || !dims_ok(B, T, C)) return 0;
  return wkv4_bwd_workspace_bytes_impl(B, T, C, dtype);
}

int wkv4_backward(const void* grad_y, const float* w, const float* u, const void* k, const void* v,
                  void* grad_k, void* grad_v, float* grad_time_decay, float* grad_time_first,
                  void* workspace, size_t workspace_bytes, int64_t B, int64_t T, int64_t C,
                  int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype)) return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward: unknown dtype");
  if (!dims_ok(B, T, C)) return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward: bad sizes");
  if (C == 0) return WKV_OK;
  if (!grad_time_decay || !grad_time_first)
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0 || T == 0) return wkv4_zero_param_grads(grad_time_decay, grad_time_first, int(C), s);
  if (!grad_y || !w || !u || !k || !v || !grad_k || !grad_v || !workspace)
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward: null pointer");
  const size_t need = wkv4_bwd_min_workspace_bytes_impl(B, T, C);
  if (workspace_bytes < need)
    return fail(WKV_ERR_WORKSPACE_TOO_SMALL,
                "wkv4_backward: workspace too small (need " + std::to_string(need) + " bytes)");
  if (!aligned16({grad_y, k, v, grad_k, grad_v, workspace}))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "wkv4_backward: grad_y, k, v, grad_k, grad_v, workspace must be 16-byte aligned");
  return wkv4_backward_impl(grad_y, w, u, k, v, grad_k, grad_v, grad_time_decay, grad_time_first,
                            workspace, workspace_bytes, int(B), int(T), int(C), dtype, s);
}

int wkv4_backward_noalloc(const void* grad_y, const float* w, const float* u, const void* k,
                          const void* v, void* grad_k, void* grad_v, float* grad_time_decay,
                          float* grad_time_first, int64_t B, int64_t T, int64_t C, int dtype,
                          void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_noalloc: unknown dtype");
  if (!dims_ok(B, T, C))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_noalloc: bad sizes");
  if (C == 0) return WKV_OK;
  // Checked before any pointer is looked at.  Records and partials are
  // written in full before they are read, so the scratch needs no clearing
  // between calls.
  const size_t need = wkv4_bwd_min_workspace_bytes_impl(B, T, C);
  if (need > size_t(WKV4_NOALLOC_SCRATCH_BYTES))
    return fail(WKV_ERR_WORKSPACE_TOO_SMALL,
                "wkv4_backward_noalloc: these sizes need " + std::to_string(need) +
                    " bytes of scratch, above the fixed maximum of " +
                    std::to_string(size_t(WKV4_NOALLOC_SCRATCH_BYTES)) +
                    " (use wkv4_backward with a workspace)");
  if (!grad_time_decay || !grad_time_first)
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_noalloc: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0 || T == 0) return wkv4_zero_param_grads(grad_time_decay, grad_time_first, int(C), s);
  if (!grad_y || !w || !u || !k || !v || !grad_k || !grad_v)
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_noalloc: null pointer");
  if (!aligned16({grad_y, k, v, grad_k, grad_v}))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "wkv4_backward_noalloc: grad_y, k, v, grad_k, grad_v must be 16-byte aligned");
  void* ws = nullptr;
  if (int rc = scratch_address(&ws, "wkv4_backward_noalloc")) return rc;
  // The split kernels run when their workspace fits in the scratch too.
  return wkv4_backward_impl(grad_y, w, u, k, v, grad_k, grad_v, grad_time_decay, grad_time_first,
                            ws, size_t(WKV4_NOALLOC_SCRATCH_BYTES), int(B), int(T), int(C), dtype,
                            s);
}

size_t wkv4_backward_checkpointed_workspace_bytes(int64_t B, int64_t T, int64_t C) {
  if (!dims_ok(B, T, C)) return 0;
  return wkv4_bwd_ck_workspace_bytes_impl(B, T, C);
}

int wkv4_backward_checkpointed(const void* grad_y, const float* time_decay,
                               const float* time_first, const void* k, const void* v,
                               const float* checkpoint, void* grad_k, void* grad_v,
                               float* grad_time_decay, float* grad_time_first, void* workspace,
                               size_t workspace_bytes, int64_t B, int64_t T, int64_t C, int dtype,
                               void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_checkpointed: unknown dtype");
  if (!dims_ok(B, T, C))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_checkpointed: bad sizes");
  if (C == 0) return WKV_OK;
  if (!grad_time_decay || !grad_time_first)
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_checkpointed: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0 || T == 0) return wkv4_zero_param_grads(grad_time_decay, grad_time_first, int(C), s);
  if (!grad_y || !time_decay || !time_first || !k || !v || !checkpoint || !grad_k || !grad_v ||
      !workspace)
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_checkpointed: null pointer");
  if (workspace_bytes < wkv4_partials_floats(B, C) * sizeof(float))
    return fail(WKV_ERR_WORKSPACE_TOO_SMALL, "wkv4_backward_checkpointed: workspace too small");
  if (!aligned16({grad_y, k, v, checkpoint, grad_k, grad_v, workspace}))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "wkv4_backward_checkpointed: tensors must be 16-byte aligned");
  return wkv4_backward_ck_impl(grad_y, time_decay, 0, time_first, k, v, checkpoint, grad_k,
                               grad_v, grad_time_decay, grad_time_first, workspace,
                               workspace_bytes, int(B), int(T), int(C), dtype, s);
}

int wkv4_forward_gated_checkpointed(const void* k, const void* v, const float* time_decay,
                                    const float* time_first, const void* r, void* y,
                                    float* checkpoint, void* workspace, size_t workspace_bytes,
                                    int64_t B, int64_t T, int64_t C, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  const int rc = check_forward("wkv4_forward_gated_checkpointed", k, v, time_decay, time_first, r,
                               true, y, true, checkpoint, false, workspace, B, T, C, dtype);
  if (rc) return rc < 0 ? WKV_OK : rc;
  return wkv4_forward_gated_impl(k, v, time_decay, time_first, r, y, checkpoint, workspace,
                                 workspace ? workspace_bytes : 0, int(B), int(T), int(C), dtype,
                                 static_cast<hipStream_t>(stream));
}

int wkv4_backward_gated_checkpointed(const void* grad_y, const float* time_decay,
                                     const float* time_first, const void* k, const void* v,
                                     const void* r, const float* checkpoint, void* grad_k,
                                     void* grad_v, void* grad_r, float* grad_time_decay,
                                     float* grad_time_first, void* workspace,
                                     size_t workspace_bytes, int64_t B, int64_t T, int64_t C,
                                     int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_gated_checkpointed: unknown dtype");
  if (!dims_ok(B, T, C))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_gated_checkpointed: bad sizes");
  if (C == 0) return WKV_OK;
  if (!grad_time_decay || !grad_time_first)
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_gated_checkpointed: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0 || T == 0) return wkv4_zero_param_grads(grad_time_decay, grad_time_first, int(C), s);
  if (!grad_y || !time_decay || !time_first || !k || !v || !r || !checkpoint || !grad_k ||
      !grad_v || !grad_r || !workspace)
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_backward_gated_checkpointed: null pointer");
  if (workspace_bytes < wkv4_partials_floats(B, C) * sizeof(float))
    return fail(WKV_ERR_WORKSPACE_TOO_SMALL,
                "wkv4_backward_gated_checkpointed: workspace too small");
  if (!aligned16({grad_y, k, v, r, checkpoint, grad_k, grad_v, grad_r, workspace}))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "wkv4_backward_gated_checkpointed: tensors must be 16-byte aligned");
  return wkv4_backward_gated_ck_impl(grad_y, time_decay, time_first, k, v, r, checkpoint, grad_k,
                                     grad_v, grad_r, grad_time_decay, grad_time_first, workspace,
                                     workspace_bytes, int(B), int(T), int(C), dtype, s);
}

int wkv4_decode_step(const void* k, const void* v, const float* time_decay, const float* time_first,
                     const float* num, const float* den, const float* log_scale, void* y,
                     float* num_out, float* den_out, float* log_scale_out, int64_t B, int64_t C,
                     int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype)) return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_decode_step: unknown dtype");
  if (!dims_ok(B, 1, C)) return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_decode_step: bad sizes");
  if (B == 0 || C == 0) return WKV_OK;
  if (!k || !v || !time_decay || !time_first || !num || !den || !log_scale || !y || !num_out ||
      !den_out || !log_scale_out)
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_decode_step: null pointer");
  if (!aligned16({k, v, num, den, log_scale, y, num_out, den_out, log_scale_out}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv4_decode_step: tensors must be 16-byte aligned");
  return wkv4_decode_impl(k, v, time_decay, time_first, num, den, log_scale, y, num_out, den_out,
                          log_scale_out, int(B), int(C), dtype, static_cast<hipStream_t>(stream));
}

int wkv7_forward(const void* r, const void* w, const void* k, const void* v, const void* a,
                 const void* b, const float* s0, void* y, float* s_out, int64_t B, int64_t T,
                 int64_t H, int64_t N, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype)) return fail(WKV_ERR_INVALID_ARGUMENT, "wkv7_forward: unknown dtype");
  if (N != 64) return fail(WKV_ERR_INVALID_ARGUMENT, "wkv7_forward: head size must be 64");
  if (!dims_ok(B, T, H * N)) return fail(WKV_ERR_INVALID_ARGUMENT, "wkv7_forward: bad sizes");
  if (B == 0 || H == 0) return WKV_OK;
  if (T > 0 && (!r || !w || !k || !v || !a || !b || !y))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv7_forward: null pointer");
  if (T == 0 && !s_out) return WKV_OK;
  if (!aligned16({r, w, k, v, a, b, s0, y, s_out}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv7_forward: tensors must be 16-byte aligned");
  return wkv7_forward_impl(r, w, k, v, a, b, s0, y, s_out, nullptr, int(B), int(T), int(H), dtype,
                           static_cast<hipStream_t>(stream));
}

size_t wkv7_checkpoint_bytes(int64_t B, int64_t T, int64_t H, int64_t N) {
  if (N != 64 || !dims_ok(B, T, H * N)) return 0;
  return wkv7_checkpoint_floats(B, T, H) * sizeof(float);
}

int wkv7_forward_checkpointed(const void* r, const void* w, const void* k, const void* v,
                              const void* a, const void* b, const float* s0, void* y,
                              float* s_out, float* checkpoint, int64_t B, int64_t T, int64_t H,
                              int64_t N, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv7_forward_checkpointed: unknown dtype");
  if (N != 64)
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv7_forward_checkpointed: head size must be 64");
  if (!dims_ok(B, T, H * N))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv7_forward_checkpointed: bad sizes");
  if (B == 0 || H == 0) return WKV_OK;
  if (T > 0 && (!r || !w || !k || !v || !a || !b || !checkpoint))
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv7_forward_checkpointed: null pointer");
  if (T == 0 && !s_out) return WKV_OK;
  if (!aligned16({r, w, k, v, a, b, s0, y, s_out, checkpoint}))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "wkv7_forward_checkpointed: tensors must be 16-byte aligned");
  return wkv7_forward_impl(r, w, k, v, a, b, s0, y, s_out, T > 0 ? checkpoint : nullptr, int(B),
                           int(T), int(H), dtype, static_cast<hipStream_t>(stream));
}

static int wkv7_backward_checks(const char* what, const void* r, const void* w, const void* k,
                                const void* v, const void* a, const void* b, const void* grad_y,
                                const float* grad_s_out, void* grad_r, void* grad_w, void* grad_k,
                                void* grad_v, void* grad_a, void* grad_b, float* grad_s0,
                                int64_t B, int64_t T, int64_t H, int64_t N, int dtype) {
  if (!dtype_ok(dtype)) return fail(WKV_ERR_INVALID_ARGUMENT, std::string(what) + ": unknown dtype");
  if (N != 64)
    return fail(WKV_ERR_INVALID_ARGUMENT, std::string(what) + ": head size must be 64");
  if (!dims_ok(B, T, H * N)) return fail(WKV_ERR_INVALID_ARGUMENT, std::string(what) + ": bad sizes");
  if (T > 0 && (!r || !w || !k || !v || !a || !b || !grad_y || !grad_r || !grad_w || !grad_k ||
                !grad_v || !grad_a || !grad_b))
    return fail(WKV_ERR_INVALID_ARGUMENT, std::string(what) + ": null pointer");
  if (!aligned16({r, w, k, v, a, b, grad_y, grad_s_out, grad_r, grad_w, grad_k, grad_v, grad_a,
                  grad_b, grad_s0}))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                std::string(what) + ": tensors must be 16-byte aligned");
  return WKV_OK;
}

size_t wkv7_backward_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t N) {
  return wkv7_checkpoint_bytes(B, T, H, N);
}

int wkv7_backward(const void* r, const void* w, const void* k, const void* v, const void* a,
                  const void* b, const float* s0, const void* grad_y, const float* grad_s_out,
                  void* grad_r, void* grad_w, void* grad_k, void* grad_v, void* grad_a,
                  void* grad_b, float* grad_s0, void* workspace, size_t workspace_bytes,
                  int64_t B, int64_t T, int64_t H, int64_t N, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  int rc = wkv7_backward_checks("wkv7_backward", r, w, k, v, a, b, grad_y, grad_s_out, grad_r,
                                grad_w, grad_k, grad_v, grad_a, grad_b, grad_s0, B, T, H, N,
                                dtype);
  if (rc) return rc;
  if (B == 0 || H == 0) return WKV_OK;
  if (T == 0 && !grad_s0) return WKV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* ck = nullptr;
  if (T > 0) {
    const size_t need = wkv7_checkpoint_floats(B, T, H) * sizeof(float);
    if (!workspace || workspace_bytes < need)
      return fail(WKV_ERR_WORKSPACE_TOO_SMALL,
                  "wkv7_backward: workspace too small (need " + std::to_string(need) + " bytes)");
    if (!aligned16({s0, workspace}))
      return fail(WKV_ERR_INVALID_ARGUMENT, "wkv7_backward: tensors must be 16-byte aligned");
    ck = static_cast<float*>(workspace);
    // The forward stage does not end the call: it carries no stop event.
    hipEvent_t stop = active_events().stop;
    active_events().stop = nullptr;
    rc = wkv7_forward_impl(r, w, k, v, a, b, s0, nullptr, nullptr, ck, int(B), int(T), int(H),
                           dtype, s);
    active_events().stop = stop;
    if (rc) return rc;
  }
  return wkv7_backward_ck_impl(r, w, k, v, a, b, grad_y, ck, grad_s_out, grad_r, grad_w, grad_k,
                               grad_v, grad_a, grad_b, grad_s0, int(B), int(T), int(H), dtype, s);
}

int wkv7_backward_checkpointed(const void* r, const void* w, const void* k, const void* v,
                               const void* a, const void* b, const float* checkpoint,
                               const void* grad_y, const float* grad_s_out, void* grad_r,
                               void* grad_w, void* grad_k, void* grad_v, void* grad_a,
                               void* grad_b, float* grad_s0, int64_t B, int64_t T, int64_t H,
                               int64_t N, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  int rc = wkv7_backward_checks("wkv7_backward_checkpointed", r, w, k, v, a, b, grad_y,
                                grad_s_out, grad_r, grad_w, grad_k, grad_v, grad_a, grad_b,
                                grad_s0, B, T, H, N, dtype);
  if (rc) return rc;
  if (B == 0 || H == 0) return WKV_OK;
  if (T == 0 && !grad_s0) return WKV_OK;
  if (T > 0 && !checkpoint)
    return fail(WKV_ERR_INVALID_ARGUMENT, "wkv7_backward_checkpointed: null pointer");
  if (!aligned16({checkpoint}))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "wkv7_backward_checkpointed: tensors must be 16-byte aligned");
  return wkv7_backward_ck_impl(r, w, k, v, a, b, grad_y, checkpoint, grad_s_out, grad_r, grad_w,
                               grad_k, grad_v, grad_a, grad_b, grad_s0, int(B), int(T), int(H),
                               dtype, static_cast<hipStream_t>(stream));
}

size_t lif_checkpoint_bytes(int64_t B, int64_t T, int64_t C) {
  if (!dims_ok(B, T, C)) return 0;
  return lif_checkpoint_floats(B, T, C) * sizeof(float);
}

size_t lif_forward_workspace_bytes(int64_t B, int64_t T, int64_t C) {
  if (!dims_ok(B, T, C)) return 0;
  return lif_fwd_workspace_bytes_impl(B, T, C);
}

size_t lif_backward_workspace_bytes(int64_t B, int64_t T, int64_t C) {
  if (!dims_ok(B, T, C)) return 0;
  return lif_bwd_workspace_bytes_impl(B, T, C);
}

static bool lif_params_ok(float decay, float threshold, float reset, float slope) {
  return std::isfinite(decay) && std::isfinite(threshold) && std::isfinite(reset) &&
         std::isfinite(slope) && slope > 0.f;
}

int lif_forward(const void* x, void* spikes, float* membrane_checkpoint, void* workspace,
                size_t workspace_bytes, int64_t B, int64_t T, int64_t C, float decay,
                float threshold, float reset, float slope, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype)) return fail(WKV_ERR_INVALID_ARGUMENT, "lif_forward: unknown dtype");
  if (!dims_ok(B, T, C)) return fail(WKV_ERR_INVALID_ARGUMENT, "lif_forward: bad sizes");
  if (!lif_params_ok(decay, threshold, reset, slope))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "lif_forward: parameters must be finite and surrogate_slope positive");
  if (B == 0 || T == 0 || C == 0) return WKV_OK;
  if (!x || !spikes) return fail(WKV_ERR_INVALID_ARGUMENT, "lif_forward: null pointer");
  if (!aligned16({x, spikes, membrane_checkpoint, workspace}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "lif_forward: tensors must be 16-byte aligned");
  return lif_forward_impl(x, spikes, membrane_checkpoint, workspace, workspace_bytes, int(B),
                          int(T), int(C), decay, threshold, reset, slope, dtype,
                          static_cast<hipStream_t>(stream));
}

int lif_residual_forward(const void* x, const float* residual, float* out,
                         float* membrane_checkpoint, void* workspace, size_t workspace_bytes,
                         int64_t B, int64_t T, int64_t C, float decay, float threshold,
                         float reset, float slope, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype)) return fail(WKV_ERR_INVALID_ARGUMENT, "lif_residual_forward: unknown dtype");
  if (!dims_ok(B, T, C)) return fail(WKV_ERR_INVALID_ARGUMENT, "lif_residual_forward: bad sizes");
  if (!lif_params_ok(decay, threshold, reset, slope))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "lif_residual_forward: parameters must be finite and surrogate_slope positive");
  if (B == 0 || T == 0 || C == 0) return WKV_OK;
  if (!lif_residual_ok(T, C, dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "lif_residual_forward: C must be a multiple of 8 and T*C*4 below 2^31");
  if (!x || !residual || !out || !membrane_checkpoint)
    return fail(WKV_ERR_INVALID_ARGUMENT, "lif_residual_forward: null pointer");
  if (!aligned16({x, residual, out, membrane_checkpoint, workspace}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "lif_residual_forward: tensors must be 16-byte aligned");
  return lif_residual_forward_impl(x, residual, out, membrane_checkpoint, workspace,
                                   workspace_bytes, int(B), int(T), int(C), decay, threshold,
                                   reset, slope, dtype, static_cast<hipStream_t>(stream));
}

int lif_residual_backward(const void* x, const float* grad_out, const float* membrane_checkpoint,
                          void* grad_x, void* workspace, size_t workspace_bytes, int64_t B,
                          int64_t T, int64_t C, float decay, float threshold, float reset,
                          float slope, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "lif_residual_backward: unknown dtype");
  if (!dims_ok(B, T, C)) return fail(WKV_ERR_INVALID_ARGUMENT, "lif_residual_backward: bad sizes");
  if (!lif_params_ok(decay, threshold, reset, slope))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "lif_residual_backward: parameters must be finite and surrogate_slope positive");
  if (B == 0 || T == 0 || C == 0) return WKV_OK;
  if (!lif_residual_ok(T, C, dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "lif_residual_backward: C must be a multiple of 8 and T*C*4 below 2^31");
  if (!x || !grad_out || !membrane_checkpoint || !grad_x)
    return fail(WKV_ERR_INVALID_ARGUMENT, "lif_residual_backward: null pointer");
  if (!aligned16({x, grad_out, membrane_checkpoint, grad_x, workspace}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "lif_residual_backward: tensors must be 16-byte aligned");
  return lif_residual_backward_impl(x, grad_out, membrane_checkpoint, grad_x, workspace,
                                    workspace_bytes, int(B), int(T), int(C), decay, threshold,
                                    reset, slope, dtype, static_cast<hipStream_t>(stream));
}

int lif_backward(const void* x, const void* grad_spikes, const float* membrane_checkpoint,
                 void* grad_x, void* workspace, size_t workspace_bytes, int64_t B, int64_t T,
                 int64_t C, float decay, float threshold, float reset, float slope, int dtype,
                 void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype)) return fail(WKV_ERR_INVALID_ARGUMENT, "lif_backward: unknown dtype");
  if (!dims_ok(B, T, C)) return fail(WKV_ERR_INVALID_ARGUMENT, "lif_backward: bad sizes");
  if (!lif_params_ok(decay, threshold, reset, slope))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "lif_backward: parameters must be finite and surrogate_slope positive");
  if (B == 0 || T == 0 || C == 0) return WKV_OK;
  if (!x || !grad_spikes || !membrane_checkpoint || !grad_x)
    return fail(WKV_ERR_INVALID_ARGUMENT, "lif_backward: null pointer");
  if (!aligned16({x, grad_spikes, membrane_checkpoint, grad_x, workspace}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "lif_backward: tensors must be 16-byte aligned");
  return lif_backward_impl(x, grad_spikes, membrane_checkpoint, grad_x, workspace,
                           workspace_bytes, int(B), int(T), int(C), decay, threshold, reset,
                           slope, dtype, static_cast<hipStream_t>(stream));
}

size_t token_shift_mix_workspace_bytes(int64_t n, int64_t B, int64_t T, int64_t C) {
  if (n < 1 || n > 3 || !dims_ok(B, T, C)) return 0;
  return shift_mix_partial_floats(n, B, T, C) * sizeof(float);
}

int token_shift_mix_forward(const void* x, int x_dtype, const float* mix, int64_t n, void* out0,
                            void* out1, void* out2, int out_dtype, int64_t B, int64_t T,
                            int64_t C, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(x_dtype) || !dtype_ok(out_dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_forward: unknown dtype");
  if (n < 1 || n > 3)
    return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_forward: 1 to 3 mixing vectors");
  if (!dims_ok(B, T, C)) return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_forward: bad sizes");
  if (B == 0 || T == 0 || C == 0) return WKV_OK;
  void* const out[3] = {out0, out1, out2};
  if (!x || !mix) return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_forward: null pointer");
  for (int j = 0; j < n; ++j) {
    if (!out[j]) return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_forward: null pointer");
    if (!aligned16({out[j]}))
      return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_forward: tensors must be 16-byte aligned");
  }
  if (!aligned16({x, mix}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_forward: tensors must be 16-byte aligned");
  return shift_mix_forward_impl(x, x_dtype, mix, out, out_dtype, int(n), int(B), int(T), int(C),
                                static_cast<hipStream_t>(stream));
}

int token_shift_mix_backward(const void* x, int x_dtype, const float* mix, int64_t n,
                             const void* grad0, const void* grad1, const void* grad2, int g_dtype,
                             void* grad_x, float* grad_mix, void* workspace,
                             size_t workspace_bytes, int64_t B, int64_t T, int64_t C,
                             void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(x_dtype) || !dtype_ok(g_dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_backward: unknown dtype");
  if (n < 1 || n > 3)
    return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_backward: 1 to 3 mixing vectors");
  if (!dims_ok(B, T, C))
    return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_backward: bad sizes");
  if (C == 0) return WKV_OK;
  if (B == 0 || T == 0) {
    if (!grad_mix) return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_backward: null pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int j = 0; j < n; j += 2) {
      const int rc = wkv4_zero_param_grads(grad_mix + j * C, grad_mix + (j + 1 < n ? j + 1 : j) * C,
                                           int(C), s);
      if (rc) return rc;
    }
    return WKV_OK;
  }
  const void* const g[3] = {grad0, grad1, grad2};
  if (!x || !mix || !grad_x || !grad_mix || !workspace)
    return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_backward: null pointer");
  for (int j = 0; j < n; ++j) {
    if (!g[j]) return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_backward: null pointer");
    if (!aligned16({g[j]}))
      return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_backward: tensors must be 16-byte aligned");
  }
  if (workspace_bytes < shift_mix_partial_floats(n, B, T, C) * sizeof(float))
    return fail(WKV_ERR_WORKSPACE_TOO_SMALL, "token_shift_mix_backward: workspace too small");
  if (!aligned16({x, mix, grad_x, grad_mix, workspace}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "token_shift_mix_backward: tensors must be 16-byte aligned");
  return shift_mix_backward_impl(x, x_dtype, mix, g, g_dtype, grad_x,
                                 static_cast<float*>(workspace), grad_mix, int(n), int(B), int(T),
                                 int(C), static_cast<hipStream_t>(stream));
}

int relu_square_forward(const void* x, void* y, int64_t n, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype)) return fail(WKV_ERR_INVALID_ARGUMENT, "relu_square_forward: unknown dtype");
  if (!elementwise_ok(n, dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "relu_square_forward: n must be a multiple of 16 bytes of elements");
  if (n == 0) return WKV_OK;
  if (!x || !y) return fail(WKV_ERR_INVALID_ARGUMENT, "relu_square_forward: null pointer");
  if (!aligned16({x, y}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "relu_square_forward: tensors must be 16-byte aligned");
  return relu_square_forward_impl(x, y, n, dtype, static_cast<hipStream_t>(stream));
}

int split_k_sum(const float* partial, float* out, int64_t S, int64_t N, void* stream) {
  set_error("");
  TimingScope timing;
  if (S <= 0 || N < 0 || S > (int64_t(1) << 20) || N > (int64_t(1) << 40))
    return fail(WKV_ERR_INVALID_ARGUMENT, "split_k_sum: bad sizes");
  if (N == 0) return WKV_OK;
  if (!partial || !out) return fail(WKV_ERR_INVALID_ARGUMENT, "split_k_sum: null pointer");
  if (N % 4 != 0 || !aligned16({partial, out}))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "split_k_sum: N must be a multiple of 4 and the tensors 16-byte aligned");
  return split_k_sum_impl(partial, out, S, N, static_cast<hipStream_t>(stream));
}

int relu_square_backward(const void* x, const void* grad_y, void* grad_x, int64_t n, int dtype,
                         void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "relu_square_backward: unknown dtype");
  if (!elementwise_ok(n, dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "relu_square_backward: n must be a multiple of 16 bytes of elements");
  if (n == 0) return WKV_OK;
  if (!x || !grad_y || !grad_x)
    return fail(WKV_ERR_INVALID_ARGUMENT, "relu_square_backward: null pointer");
  if (!aligned16({x, grad_y, grad_x}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "relu_square_backward: tensors must be 16-byte aligned");
  return relu_square_backward_impl(x, grad_y, grad_x, n, dtype, static_cast<hipStream_t>(stream));
}

int sigmoid_gate_forward(const void* r, const void* x, void* y, int64_t n, int dtype,
                         void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "sigmoid_gate_forward: unknown dtype");
  if (!elementwise_ok(n, dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "sigmoid_gate_forward: n must be a multiple of 16 bytes of elements");
  if (n == 0) return WKV_OK;
  if (!r || !x || !y) return fail(WKV_ERR_INVALID_ARGUMENT, "sigmoid_gate_forward: null pointer");
  if (!aligned16({r, x, y}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "sigmoid_gate_forward: tensors must be 16-byte aligned");
  return sigmoid_gate_forward_impl(r, x, y, n, dtype, static_cast<hipStream_t>(stream));
}

int sigmoid_gate_backward(const void* r, const void* x, const void* grad_y, void* grad_r,
                          void* grad_x, int64_t n, int dtype, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "sigmoid_gate_backward: unknown dtype");
  if (!elementwise_ok(n, dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "sigmoid_gate_backward: n must be a multiple of 16 bytes of elements");
  if (n == 0) return WKV_OK;
  if (!r || !x || !grad_y || !grad_r || !grad_x)
    return fail(WKV_ERR_INVALID_ARGUMENT, "sigmoid_gate_backward: null pointer");
  if (!aligned16({r, x, grad_y, grad_r, grad_x}))
    return fail(WKV_ERR_INVALID_ARGUMENT, "sigmoid_gate_backward: tensors must be 16-byte aligned");
  return sigmoid_gate_backward_impl(r, x, grad_y, grad_r, grad_x, n, dtype,
                                    static_cast<hipStream_t>(stream));
}

static bool ln_mix_dims_ok(int64_t n, int64_t B, int64_t T, int64_t C) {
  return (n == 2 || n == 3) && (C == 256 || C == 512) && dims_ok(B, T, C) &&
         B * T < (int64_t(1) << 31);
}

int layer_norm_shift_mix_forward(const float* x, const float* weight, const float* bias,
                                 float eps, const float* mix, int64_t n, void* out0, void* out1,
                                 void* out2, int out_dtype, float* mean, float* rstd, int64_t B,
                                 int64_t T, int64_t C, void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(out_dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "layer_norm_shift_mix_forward: unknown dtype");
  if (!ln_mix_dims_ok(n, B, T, C))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "layer_norm_shift_mix_forward: n in {2, 3}, C in {256, 512}, valid sizes");
  if (!(eps > 0.f)) return fail(WKV_ERR_INVALID_ARGUMENT, "layer_norm_shift_mix_forward: eps > 0");
  if (B == 0 || T == 0) return WKV_OK;
  void* const out[3] = {out0, out1, out2};
  if (!x || !weight || !bias || !mix || !mean || !rstd)
    return fail(WKV_ERR_INVALID_ARGUMENT, "layer_norm_shift_mix_forward: null pointer");
  for (int j = 0; j < n; ++j)
    if (!out[j] || !aligned16({out[j]}))
      return fail(WKV_ERR_INVALID_ARGUMENT,
                  "layer_norm_shift_mix_forward: null or unaligned output");
  if (!aligned16({x, weight, bias, mix}))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "layer_norm_shift_mix_forward: tensors must be 16-byte aligned");
  return ln_mix_forward_impl(x, weight, bias, mix, int(n), out, out_dtype, mean, rstd, int(B),
                             int(T), int(C), eps, static_cast<hipStream_t>(stream));
}

size_t layer_norm_shift_mix_workspace_bytes(int64_t n, int64_t B, int64_t T, int64_t C) {
  if (!ln_mix_dims_ok(n, B, T, C)) return 0;
  return size_t(n + 2) * size_t(ln_mix_workgroups(B, T)) * size_t(C) * sizeof(float);
}

int layer_norm_shift_mix_backward(const float* x, const float* weight, const float* bias,
                                  const float* mix, int64_t n, const float* mean,
                                  const float* rstd, const void* grad0, const void* grad1,
                                  const void* grad2, int g_dtype, float* grad_x,
                                  const float* grad_x_add, float* grad_params, void* workspace,
                                  size_t workspace_bytes, int64_t B, int64_t T, int64_t C,
                                  void* stream) {
  set_error("");
  TimingScope timing;
  if (!dtype_ok(g_dtype))
    return fail(WKV_ERR_INVALID_ARGUMENT, "layer_norm_shift_mix_backward: unknown dtype");
  if (!ln_mix_dims_ok(n, B, T, C))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "layer_norm_shift_mix_backward: n in {2, 3}, C in {256, 512}, valid sizes");
  if (B == 0 || T == 0) return WKV_OK;  // the caller zero-fills grad_params
  const void* const g[3] = {grad0, grad1, grad2};
  if (!x || !weight || !bias || !mix || !mean || !rstd || !grad_x || !grad_params || !workspace)
    return fail(WKV_ERR_INVALID_ARGUMENT, "layer_norm_shift_mix_backward: null pointer");
  for (int j = 0; j < n; ++j)
    if (!g[j] || !aligned16({g[j]}))
      return fail(WKV_ERR_INVALID_ARGUMENT,
                  "layer_norm_shift_mix_backward: null or unaligned gradient");
  if (!aligned16({x, weight, bias, mix, grad_x, grad_x_add, workspace}))
    return fail(WKV_ERR_INVALID_ARGUMENT,
                "layer_norm_shift_mix_backward: tensors must be 16-byte aligned");
  if (workspace_bytes < layer_norm_shift_mix_workspace_bytes(n, B, T, C))
    return fail(WKV_ERR_WORKSPACE_TOO_SMALL, "layer_norm_shift_mix_backward: workspace too small");
  return ln_mix_backward_impl(x, weight, bias, mix, int(n), mean, rstd, g, g_dtype, grad_x,
                              grad_x_add, static_cast<float*>(workspace), grad_params, int(B), int(T),
                              int(C), static_cast<hipStream_t>(stream));
}

int block_step_row(int pre, const wkv_step_row_args* a, void* stream) {
  set_error("");
  TimingScope timing;
  if (!a) return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: null args");
  if (pre < WKV_STEP_PRE_EMBED || pre > WKV_STEP_PRE_NONE)
    return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: unknown pre-operation");
  if (a->batch < 0 || a->batch >= (int64_t(1) << 31) || a->channels < 1 || a->channels > 4096)
    return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: batch >= 0 and 1 <= channels <= 4096");
  if (a->n_mix != 0 && a->n_mix != 2 && a->n_mix != 3)
    return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: n_mix must be 0, 2 or 3");
  if (a->batch == 0) return WKV_OK;
  if (!a->residual) return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: null residual");
  if (a->ln_weight == nullptr && a->n_mix != 0)
    return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: token shift needs the layer norm");
  if (a->ln_weight != nullptr && (!a->ln_bias || !a->out[0]))
    return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: null layer-norm bias or output");
  for (int j = 1; j < a->n_mix; ++j)
    if (!a->out[j]) return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: null output");
  if (a->n_mix > 0 && (!a->previous_in || !a->previous_out))
    return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: null token-shift state");
  for (int j = 0; j < a->n_mix; ++j)
    if (!a->mix[j]) return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: null mixing vector");
  if (pre == WKV_STEP_PRE_EMBED || pre == WKV_STEP_PRE_NONE) {
    if (pre == WKV_STEP_PRE_EMBED && (!a->ids || !a->embedding || a->vocab < 1))
      return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: null ids or embedding");
    if ((a->ln0_weight == nullptr) != (a->ln0_bias == nullptr))
      return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: ln0 weight and bias go together");
  } else {
    if (!a->add || !a->membrane_in || !a->membrane_out)
      return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: null LIF input or membrane");
    if (pre == WKV_STEP_PRE_GATE_LIF && !a->gate)
      return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: null gate");
  }
  if (!(a->ln_eps > 0.f)) return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_row: ln_eps > 0");
  return block_step_row_impl(pre, *a, static_cast<hipStream_t>(stream));
}

int block_step_wkv(const float* key, const float* value, const float* receptance,
                   const float* time_decay, const float* time_first, const float* num_in,
                   const float* den_in, const float* log_scale_in, float* num_out,
                   float* den_out, float* log_scale_out, float* out, int64_t B, int64_t C,
                   void* stream) {
  set_error("");
  TimingScope timing;
  if (B < 0 || C < 0 || B >= (int64_t(1) << 31) || C >= (int64_t(1) << 31) ||
      B * C >= (int64_t(1) << 40))
    return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_wkv: bad sizes");
  if (B == 0 || C == 0) return WKV_OK;
  if (!key || !value || !receptance || !time_decay || !time_first || !num_in || !den_in ||
      !log_scale_in || !num_out || !den_out || !log_scale_out || !out)
    return fail(WKV_ERR_INVALID_ARGUMENT, "block_step_wkv: null pointer");
  return block_step_wkv_impl(key, value, receptance, time_decay, time_first, num_in, den_in,
                             log_scale_in, num_out, den_out, log_scale_out, out, B, C,
                             static_cast<hipStream_t>(stream));
}

int wkv_time_next_call(void* start_event, void* stop_event) {
  g_pending_events = CallEvents{};
  g_pending_events.start = static_cast<hipEvent_t>(start_event);
  g_pending_events.stop = static_cast<hipEvent_t>(stop_event);
  return WKV_OK;
}

int wkv_time_next_kernel(void* start_event, void* stop_event, int kernel) {
  if (kernel < 0) return fail(WKV_ERR_INVALID_ARGUMENT, "wkv_time_next_kernel: negative index");
  g_pending_events = CallEvents{};
  g_pending_events.start = static_cast<hipEvent_t>(start_event);
  g_pending_events.stop = static_cast<hipEvent_t>(stop_event);
  g_pending_events.kernel = kernel;
  return WKV_OK;
}

const char* wkv_last_error_string(void) { return g_last_error.c_str(); }

const char* wkv_version(void) { return "wkv_hip 0.1.0 gfx950"; }

}  // extern "C"
