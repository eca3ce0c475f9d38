// Host-side interfaces between the translation units of libwkv_hip.so: the
// launchers each kernel file defines and capi.hip (the C ABI) calls, plus the
// tile-selection helpers the RWKV-4 files share.  Argument checks happen in
// capi.hip; these functions assume valid shapes and pointers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/wkv_hip.h"

namespace wkv_host {

// Channels per lane, steps per wave chunk, waves per workgroup.
struct TileCfg { int vec, L, W; };

// RWKV-4 tile selection (capi.hip): channels per lane for B, C; a "vec,L,W"
// override read from the environment (measurement only).
int pick_vec(int64_t B, int64_t C);
bool env_cfg(const char* name, int& vec, int& L, int& W);

// The split-over-time RWKV-4 kernels run for fewer than kSplitRows rows of 64
// channels, at least kSplitMinSegs segments and kSplitMinElems elements.
// Measured fwd+bwd (MI355X, bf16, one-row backward on its 16-wave tile):
// 96 rows or fewer the split wins by far (B=12 T=4096 C=512: 109 against
// 193 us; B=4 T=8192: 98 against 376 us), at 192 rows the two are within
// 2 % (B=24 T=3072 C=512: 149-154 against 151 us; B=16 T=1024 C=768 and
// T=2048: one-row 3 % and 1 % faster) and at 256 rows the one-row kernels
// win (116 against 135 us).  The split's fill, fix-up and batch-sum
// launches cost ~8-10 us per call.  split_mode() is WKV_SPLIT from the
// environment (0 off, 1 on, -1 unset: by these sizes).
constexpr int64_t kSplitRows = 192;
constexpr int64_t kSplitMinSegs = 32;
constexpr int64_t kSplitMinElems = int64_t(1) << 23;
int split_mode();
// Polls of one look-back word before a split workgroup gives up and leaves
// its row to the fix-up kernel: kLbMaxPolls, or WKV_LB_MAX_POLLS from the
// environment (-1 .. kLbMaxPolls; -1 gives up at once, so that a test can
// send every row through the fix-up path).
int lb_poll_limit();
// Fills `bytes` (a multiple of 16) of look-back workspace with all ones.
int lb_fill(void* ws, size_t bytes, hipStream_t stream);

// RWKV-4 forward (wkv4_fwd.hip).  decay_is_w: `decay` holds w itself rather
// than time_decay.  ck (may be null): checkpoint records.  ws (may be null):
// workspace of the split kernel, wkv4_fwd_workspace_bytes_impl bytes (0 when
// the one-row kernel runs).
int wkv4_forward_impl(const void* k, const void* v, const float* decay, int decay_is_w,
                      const float* tf, void* y, float* ck, void* ws, size_t ws_bytes, int B,
                      int T, int C, int dtype, hipStream_t stream);
int wkv4_forward_gated_impl(const void* k, const void* v, const float* decay, const float* tf,
                            const void* r, void* y, float* ck, void* ws, size_t ws_bytes, int B,
                            int T, int C, int dtype, hipStream_t stream);
size_t wkv4_fwd_workspace_bytes_impl(int64_t B, int64_t T, int64_t C);

// RWKV-4 backward (wkv4_bwd.hip).  ws: the [2][B][C] partials at least
// (wkv4_partials_floats); the split kernel runs when it is eligible and ws
// holds wkv4_bwd_ck_workspace_bytes_impl bytes.
int wkv4_backward_ck_impl(const void* gy, const float* decay, int decay_is_w, const float* u,
                          const void* k, const void* v, const float* ck, void* gk, void* gv,
                          float* gtd, float* gtf, void* ws, size_t ws_bytes, int B, int T, int C,
                          int dtype, hipStream_t stream);
int wkv4_backward_gated_ck_impl(const void* g, const float* decay, const float* u, const void* k,
                                const void* v, const void* r, const float* ck, void* gk,
                                void* gv, void* gr, float* gtd, float* gtf, void* ws,
                                size_t ws_bytes, int B, int T, int C, int dtype,
                                hipStream_t stream);
// From the inputs alone (records computed into the workspace first).
int wkv4_backward_impl(const void* gy, const float* w, const float* u, const void* k,
                       const void* v, void* gk, void* gv, float* gtd, float* gtf, void* ws,
                       size_t ws_bytes, int B, int T, int C, int dtype, hipStream_t stream);
size_t wkv4_bwd_ck_workspace_bytes_impl(int64_t B, int64_t T, int64_t C);
size_t wkv4_bwd_workspace_bytes_impl(int64_t B, int64_t T, int64_t C, int dtype);
size_t wkv4_bwd_min_workspace_bytes_impl(int64_t B, int64_t T, int64_t C);
size_t wkv4_checkpoint_floats(int64_t B, int64_t T, int64_t C);
size_t wkv4_partials_floats(int64_t B, int64_t C);
int wkv4_zero_param_grads(float* gtd, float* gtf, int C, hipStream_t stream);

int wkv4_decode_impl(const void*, const void*, const float*, const float*, const float*,
                     const float*, const float*, void*, float*, float*, float*, int, int, int,
                     hipStream_t);
int wkv7_forward_impl(const void*, const void*, const void*, const void*, const void*,
                      const void*, const float*, void*, float*, float*, int, int, int, int,
                      hipStream_t);
int wkv7_backward_ck_impl(const void*, const void*, const void*, const void*, const void*,
                          const void*, const void*, const float*, const float*, void*, void*,
                          void*, void*, void*, void*, float*, int, int, int, int, hipStream_t);
size_t wkv7_checkpoint_floats(int64_t, int64_t, int64_t);
size_t lif_checkpoint_floats(int64_t, int64_t, int64_t);
size_t shift_mix_partial_floats(int64_t, int64_t, int64_t, int64_t);
int shift_mix_forward_impl(const void*, int, const float*, void* const*, int, int, int, int, int,
                           hipStream_t);
int shift_mix_backward_impl(const void*, int, const float*, const void* const*, int, void*, float*,
                            float*, int, int, int, int, hipStream_t);
// Sequence LIF (lif.hip).  ws (may be null): workspace of the split
// forward, lif_fwd_workspace_bytes_impl bytes (0: no split for these sizes).
int lif_forward_impl(const void* x, void* spk, float* ck, void* ws, size_t ws_bytes, int B, int T,
                     int C, float decay, float threshold, float reset, float slope, int dtype,
                     hipStream_t stream);
size_t lif_fwd_workspace_bytes_impl(int64_t B, int64_t T, int64_t C);
int lif_backward_impl(const void* x, const void* gs, const float* ck, void* gx, void* ws,
                      size_t ws_bytes, int B, int T, int C, float decay, float threshold,
                      float reset, float slope, int dtype, hipStream_t stream);
size_t lif_bwd_workspace_bytes_impl(int64_t B, int64_t T, int64_t C);
int lif_residual_forward_impl(const void* x, const float* res, float* out, float* ck, void* ws,
                              size_t ws_bytes, int B, int T, int C, float decay, float threshold,
                              float reset, float slope, int dtype, hipStream_t stream);
int lif_residual_backward_impl(const void* x, const float* g, const float* ck, void* gx,
                               void* ws, size_t ws_bytes, int B, int T, int C, float decay,
                               float threshold, float reset, float slope, int dtype,
                               hipStream_t stream);
bool lif_residual_ok(int64_t, int64_t, int);
int relu_square_forward_impl(const void*, void*, int64_t, int, hipStream_t);
int relu_square_backward_impl(const void*, const void*, void*, int64_t, int, hipStream_t);
int sigmoid_gate_forward_impl(const void*, const void*, void*, int64_t, int, hipStream_t);
int sigmoid_gate_backward_impl(const void*, const void*, const void*, void*, void*, int64_t, int,
                               hipStream_t);
int block_step_row_impl(int, const wkv_step_row_args&, hipStream_t);
int ln_mix_forward_impl(const float*, const float*, const float*, const float*, int, void* const*,
                        int, float*, float*, int, int, int, float, hipStream_t);
int ln_mix_backward_impl(const float*, const float*, const float*, const float*, int,
                         const float*, const float*, const void* const*, int, float*,
                         const float*, float*, float*, int, int, int, hipStream_t);
int64_t ln_mix_workgroups(int64_t, int64_t);
int split_k_sum_impl(const float*, float*, int64_t, int64_t, hipStream_t);
int block_step_wkv_impl(const float*, const float*, const float*, const float*, const float*,
                        const float*, const float*, const float*, float*, float*, float*, float*,
                        int64_t, int64_t, hipStream_t);

}  // namespace wkv_host
