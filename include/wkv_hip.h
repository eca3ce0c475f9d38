/*
 * C ABI of the MI355X (gfx950) WKV library, libwkv_hip.so.
 *
 * Plain pointers and sizes only; every entry point launches asynchronously on
 * the HIP stream it is given (pass torch.cuda.current_stream().cuda_stream)
 * and never allocates, frees or synchronises.  Tensors are contiguous,
 * row-major: [B, T, C] with channels fastest, and their base addresses are
 * 16-byte aligned (the kernels use vector loads and stores).  Return value: 0 on success,
 * otherwise a nonzero code whose text wkv_last_error_string() gives (the
 * message is thread-local).
 *
 * The reference runs this path as Triton kernels behind torch.library ops; the
 * comment on each entry point names the reference interface it replaces.
 */
#ifndef WKV_HIP_H
#define WKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of the [B,T,C] tensors (k, v, y, grad_y, grad_k, grad_v).
 * Parameters (time_decay, time_first, w, u) and gradient sums are float32. */
enum wkv_dtype {
  WKV_DTYPE_F32 = 0,
  WKV_DTYPE_BF16 = 1,
  WKV_DTYPE_F16 = 2
};

enum wkv_status {
  WKV_OK = 0,
  WKV_ERR_INVALID_ARGUMENT = 1,
  WKV_ERR_LAUNCH = 2,
  WKV_ERR_WORKSPACE_TOO_SMALL = 3
};

/* Bytes of device workspace the RWKV-4 forward entry points can use for
 * these sizes: nonzero when fewer rows of 64 channels (B * ceil(C / 64))
 * than the GPU has CUs would leave it idle, and the sequence is then split
 * over workgroups that exchange their carries through the workspace; 0 when
 * the one-row-per-workgroup kernel runs.  Any workspace passed is filled by
 * the call itself (no clearing needed). */
size_t wkv4_forward_workspace_bytes(int64_t B, int64_t T, int64_t C);

/* RWKV-4 / SpikeGPT WKV forward.
 *
 * Replaces the kernel launch inside myelin::wkv_forward
 * (src/spikegpt/wkv_triton.py:147-158) and myelin::wkv_forward_bf16io
 * (src/spikegpt/wkv_bf16.py:143-154): y[b,t,c] from k, v [B,T,C] in `dtype`
 * with fp32 recurrence state.  Unlike the Triton kernel (which takes the
 * transformed w = -exp(time_decay) computed by the host wrapper), this entry
 * point takes the raw fp32 time_decay [C] and time_first [C] and applies
 * w = -exp(time_decay) itself, saving the wrapper's extra launch.
 * `workspace` (NULL allowed: then the one-row kernel runs) holds
 * wkv4_forward_workspace_bytes() bytes. */
int wkv4_forward(const void* k, const void* v, const float* time_decay, const float* time_first,
                 void* y, void* workspace, size_t workspace_bytes, int64_t B, int64_t T,
                 int64_t C, int dtype, void* stream);

/* Bytes of the forward-state checkpoint records for these sizes: 3 fp32
 * per (batch, block of 64 steps, channel) -- the state (A, B) = 2^o (p, q)
 * at the block start, laid out [3][B][ceil(T/64)][C].  They replace the
 * reference's three [B,T,C] fp32 replay buffers
 * (src/spikegpt/wkv_triton.py:170-172, wkv_bf16.py:167-169). */
size_t wkv4_checkpoint_bytes(int64_t B, int64_t T, int64_t C);

/* wkv4_forward that also writes the checkpoint records (y may be NULL to
 * write the records only).  Used by the training path so that the backward
 * reads the sequence once; no counterpart in the reference, whose autograd
 * re-runs the forward inside the backward kernel (wkv_triton.py:85-115). */
int wkv4_forward_checkpointed(const void* k, const void* v, const float* time_decay,
                              const float* time_first, void* y, float* checkpoint,
                              void* workspace, size_t workspace_bytes, int64_t B, int64_t T,
                              int64_t C, int dtype, void* stream);

/* Bytes of device workspace wkv4_backward uses for these sizes: the
 * checkpoint records it computes itself, then the per-batch parameter-
 * gradient partials and, for few rows, the split kernels' carries.  The call
 * accepts less (down to the records and the [2][B][C] partials) and then runs
 * the one-row kernels. */
size_t wkv4_backward_workspace_bytes(int64_t B, int64_t T, int64_t C, int dtype);

/* RWKV-4 / SpikeGPT WKV backward.
 *
 * Replaces the kernel launch and the batch sums inside myelin::wkv_backward
 * (src/spikegpt/wkv_triton.py:164-194) and myelin::wkv_backward_bf16io
 * (src/spikegpt/wkv_bf16.py:160-191).  Inputs: grad_y, k, v [B,T,C] in
 * `dtype`; w = -exp(time_decay) and u = time_first, fp32 [C] (the op's own
 * argument convention).  Outputs: grad_k, grad_v [B,T,C] in `dtype`;
 * grad_time_decay [C] (already multiplied by w, the chain rule through
 * w = -exp(time_decay)) and grad_time_first [C], both fp32 and summed over
 * the batch.  `workspace` must hold wkv4_backward_workspace_bytes() bytes. */
int wkv4_backward(const void* grad_y, const float* w, const float* u, const void* k, const void* v,
                  void* grad_k, void* grad_v, float* grad_time_decay, float* grad_time_first,
                  void* workspace, size_t workspace_bytes, int64_t B, int64_t T, int64_t C,
                  int dtype, void* stream);

/* Fixed scratch behind wkv4_backward_noalloc, per GPU: 16 MiB. */
#define WKV4_NOALLOC_SCRATCH_BYTES (16u << 20)

/* wkv4_backward without a workspace argument and without any allocation.
 *
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, kernels and results as wkv4_backward,
 * with the workspace taken from a fixed device array of
 * WKV4_NOALLOC_SCRATCH_BYTES per GPU (the library looks its address up once
 * per device and never frees it).  Sizes whose minimum workspace (the
 * records and the [2][B][C] partials wkv4_backward accepts at the least)
 * exceeds that maximum are rejected with WKV_ERR_WORKSPACE_TOO_SMALL.  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU (on
 * different streams, or from different threads) race and must be serialised
 * by the caller.  The stream must belong to the current device.  The split
 * kernels run when their workspace fits in the array as well. */
int wkv4_backward_noalloc(const void* grad_y, const float* w, const float* u, const void* k,
                          const void* v, void* grad_k, void* grad_v, float* grad_time_decay,
                          float* grad_time_first, int64_t B, int64_t T, int64_t C, int dtype,
                          void* stream);

/* Bytes of device workspace wkv4_backward_checkpointed uses: the per-batch
 * parameter-gradient partials (2*B*C fp32, the minimum it accepts), or for
 * few rows the split kernel's per-segment partials and carries. */
size_t wkv4_backward_checkpointed_workspace_bytes(int64_t B, int64_t T, int64_t C);

/* wkv4_backward from the records of wkv4_forward_checkpointed on the same
 * k, v, time_decay, time_first.  Takes the raw time_decay (w = -exp(.) is
 * applied in the kernel) and time_first; outputs as wkv4_backward.  This is
 * the reference autograd backward (wkv_triton.py:204-216, wkv_bf16.py:201-213)
 * without the forward replay pass. */
int wkv4_backward_checkpointed(const void* grad_y, const float* time_decay,
                               const float* time_first, const void* k, const void* v,
                               const float* checkpoint, void* grad_k, void* grad_v,
                               float* grad_time_decay, float* grad_time_first, void* workspace,
                               size_t workspace_bytes, int64_t B, int64_t T, int64_t C, int dtype,
                               void* stream);

/* The time mix's receptance gate folded into the WKV kernels
 * (language.py:1028-1035: sigmoid(r) * wkv): y = sigmoid(r) * wkv(k, v)
 * with the roundings of the separate ops (wkv and sigmoid(r) each rounded to
 * the element type, then the product), so y equals wkv4_forward followed by
 * sigmoid_gate_forward bit for bit.  r [B,T,C] in dtype; y required;
 * checkpoint optional (NULL: none), as wkv4_forward_checkpointed. */
int wkv4_forward_gated_checkpointed(const void* k, const void* v, const float* time_decay,
                                    const float* time_first, const void* r, void* y,
                                    float* checkpoint, void* workspace, size_t workspace_bytes,
                                    int64_t B, int64_t T, int64_t C, int dtype, void* stream);

/* Backward of wkv4_forward_gated_checkpointed from its records: grad_y is
 * the gradient of the gated output; writes grad_k, grad_v, grad_r (dtype)
 * and the parameter gradients, equal to sigmoid_gate_backward followed by
 * wkv4_backward_checkpointed.  Workspace as wkv4_backward_checkpointed. */
int wkv4_backward_gated_checkpointed(const void* grad_y, const float* time_decay,
                                     const float* time_first, const void* k, const void* v,
                                     const void* r, const float* checkpoint, void* grad_k,
                                     void* grad_v, void* grad_r, float* grad_time_decay,
                                     float* grad_time_first, void* workspace,
                                     size_t workspace_bytes, int64_t B, int64_t T, int64_t C,
                                     int dtype, void* stream);

/* Single-token WKV decode step for generation.
 *
 * Replaces the eager WKV arithmetic of SpikeTimeMix.step
 * (src/spikegpt/language.py:989-1012), which has no op in the reference.
 * k, v [B,C] in `dtype`; time_decay, time_first fp32 [C]; state
 * (numerator, denominator, log_scale) fp32 [B,C], natural-log units as in the
 * reference.  Writes y [B,C] in `dtype` and the next state to
 * num_out/den_out/log_scale_out (which may alias the inputs). */
int wkv4_decode_step(const void* k, const void* v, const float* time_decay, const float* time_first,
                     const float* num, const float* den, const float* log_scale, void* y,
                     float* num_out, float* den_out, float* log_scale_out, int64_t B, int64_t C,
                     int dtype, void* stream);

/* RWKV-7 DPLR recurrence forward, per (batch, head) with head size N = 64:
 *   S_t = S_{t-1} (diag(w_t) + a_t b_t^T) + v_t k_t^T,   y_t = S_t r_t
 * r, w, k, v, a, b, y: [B,T,H,64] in `dtype`; S is [N_v=64, N_k=64] fp32.
 * s0 (optional, may be NULL = zeros) and s_out (optional, may be NULL):
 * [B,H,64,64] fp32.  All pointers 16-byte aligned.  The reference's RWKV-7
 * code was deleted (benchmarks/results/optimizer_wkv_experiments_5090.md:3,
 * where its arithmetic came from the external `fla` package); this op has no
 * surviving counterpart there. */
int wkv7_forward(const void* r, const void* w, const void* k, const void* v, const void* a,
                 const void* b, const float* s0, void* y, float* s_out, int64_t B, int64_t T,
                 int64_t H, int64_t N, int dtype, void* stream);

/* Bytes of the RWKV-7 checkpoint records: one per 8-step block,
 * [B*H][ceil(T/8)][72][64] fp32; rows 0-63 hold the 64x64 state at the
 * block's first step, row 64 + s holds S_{t-1} a_t of its step s. */
size_t wkv7_checkpoint_bytes(int64_t B, int64_t T, int64_t H, int64_t N);

/* wkv7_forward that also writes the state checkpoints (y and s_out may be
 * NULL).  Used by the training path so that the backward does not replay the
 * sequence from its start; no counterpart in the reference. */
int wkv7_forward_checkpointed(const void* r, const void* w, const void* k, const void* v,
                              const void* a, const void* b, const float* s0, void* y,
                              float* s_out, float* checkpoint, int64_t B, int64_t T, int64_t H,
                              int64_t N, int dtype, void* stream);

/* Bytes of device workspace wkv7_backward needs (the checkpoints it computes
 * itself). */
size_t wkv7_backward_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t N);

/* RWKV-7 DPLR backward.  Inputs as wkv7_forward plus grad_y [B,T,H,64] in
 * `dtype` and grad_s_out [B,H,64,64] fp32 (gradient of the final state; may be
 * NULL = zeros).  Outputs grad_r, grad_w, grad_k, grad_v, grad_a, grad_b
 * [B,T,H,64] in `dtype` and grad_s0 [B,H,64,64] fp32 (may be NULL).
 * `workspace` must hold wkv7_backward_workspace_bytes() bytes.  No
 * counterpart in the reference (see wkv7_forward). */
int wkv7_backward(const void* r, const void* w, const void* k, const void* v, const void* a,
                  const void* b, const float* s0, const void* grad_y, const float* grad_s_out,
                  void* grad_r, void* grad_w, void* grad_k, void* grad_v, void* grad_a,
                  void* grad_b, float* grad_s0, void* workspace, size_t workspace_bytes,
                  int64_t B, int64_t T, int64_t H, int64_t N, int dtype, void* stream);

/* wkv7_backward from the checkpoints of wkv7_forward_checkpointed on the same
 * inputs and initial state (no workspace). */
int wkv7_backward_checkpointed(const void* r, const void* w, const void* k, const void* v,
                               const void* a, const void* b, const float* checkpoint,
                               const void* grad_y, const float* grad_s_out, void* grad_r,
                               void* grad_w, void* grad_k, void* grad_v, void* grad_a,
                               void* grad_b, float* grad_s0, int64_t B, int64_t T, int64_t H,
                               int64_t N, int dtype, void* stream);

/* Bytes of the sequence-LIF membrane checkpoints for these sizes: fp32
 * [B][ceil(T/32)][C], the membrane at the start of every 32-step block. */
size_t lif_checkpoint_bytes(int64_t B, int64_t T, int64_t C);

/* Bytes of device workspace lif_forward and lif_residual_forward use to split
 * the sequence over time for these sizes (the membranes at the segment
 * boundaries, fp32); 0 when these sizes are not split.  With a smaller or
 * NULL workspace the forward runs as one pass over time, with the same
 * results bit for bit. */
size_t lif_forward_workspace_bytes(int64_t B, int64_t T, int64_t C);

/* Sequence LIF activation forward (SpikeGPT's spiking residual gate).
 *
 * Replaces the fused LIF launch inside SpikingSequenceLIF.forward
 * (src/spikegpt/language.py:848-907, which calls the external myelin
 * package's Triton kernels surrogate_lif_bf16io / the fp32 LIF function) and
 * its eager fallback loop (language.py:908-918, step :813-840).  x and spikes:
 * [B,T,C] in `dtype` (channels fastest, no [T,B,C] transpose); fp32 membrane
 * starting at 0: h = m*decay + x, spike = [slope*(h - threshold) >= 0],
 * m = h*(1 - spike) + reset*spike.  Spikes are exact 0/1.  membrane_checkpoint
 * (may be NULL) receives lif_checkpoint_bytes() bytes for lif_backward.
 * workspace (may be NULL): lif_forward_workspace_bytes() bytes let the
 * sequence be split over time (same results).  decay = 1 - 1/tau; slope > 0. */
int lif_forward(const void* x, void* spikes, float* membrane_checkpoint, void* workspace,
                size_t workspace_bytes, int64_t B, int64_t T, int64_t C, float decay,
                float threshold, float reset, float slope, int dtype, void* stream);

/* Bytes of device workspace lif_backward and lif_residual_backward use to
 * split the sequence over time (the gradient carries at the segment
 * boundaries, fp32); 0 when these sizes are not split.  With a smaller or
 * NULL workspace the backward runs as one pass, with the same results bit
 * for bit. */
size_t lif_backward_workspace_bytes(int64_t B, int64_t T, int64_t C);

/* Sequence LIF backward: grad_x [B,T,C] in `dtype` from x, grad_spikes and the
 * forward's membrane checkpoints, with the arctan surrogate derivative
 * ds/dh = slope * 0.5 / (1 + (pi/2 * slope*(h - threshold))^2) and the reset
 * path differentiated (autograd through language.py:833-839).  The
 * surrogate's exact form lives in the external myelin package, absent from
 * the reference tree; this is SpikingJelly's ATan surrogate with alpha =
 * slope.  workspace (may be NULL): lif_backward_workspace_bytes() bytes. */
int lif_backward(const void* x, const void* grad_spikes, const float* membrane_checkpoint,
                 void* grad_x, void* workspace, size_t workspace_bytes, int64_t B, int64_t T,
                 int64_t C, float decay, float threshold, float reset, float slope, int dtype,
                 void* stream);

/* Bytes of device workspace token_shift_mix_backward needs for n mixing
 * vectors (per-(batch, chunk of steps) partial sums, fp32; the chunk length,
 * 8 to 64 steps, follows from B, T and C). */
size_t token_shift_mix_workspace_bytes(int64_t n, int64_t B, int64_t T, int64_t C);

/* Fused token-shift mixing (the time-mix and channel-mix prologue).
 *
 * Replaces the eager _time_shift / _mix_with_previous of
 * src/spikegpt/language.py:344-353 as SpikeTimeMix.forward (:1016-1018, n =
 * 3: k, v, r) and SpikeChannelMix.forward (:1190-1191, n = 2: k, r) call it,
 * together with autocast's cast of the result: for j < n,
 *   out_j[b,t,c] = x[b,t,c] * mix[j][c] + x[b,t-1,c] * (1 - mix[j][c]),
 * x[b,-1,c] = 0, in fp32 (products, then the sum), rounded once to
 * out_dtype.  x [B,T,C] in x_dtype; mix [n][C] fp32; out0..out{n-1} [B,T,C]
 * (unused ones NULL).  dtype pairs: (f32 -> f32|bf16|f16), (bf16 -> bf16),
 * (f16 -> f16). */
int token_shift_mix_forward(const void* x, int x_dtype, const float* mix, int64_t n, void* out0,
                            void* out1, void* out2, int out_dtype, int64_t B, int64_t T,
                            int64_t C, void* stream);

/* Backward of token_shift_mix_forward: grad_x [B,T,C] in x_dtype,
 *   grad_x[b,t,c] = sum_j g_j[b,t,c] mix[j][c] + g_j[b,t+1,c] (1 - mix[j][c]),
 * and grad_mix [n][C] fp32, grad_mix[j][c] = sum_{b,t} g_j (x[t] - x[t-1])
 * (summed in a fixed order).  grad0..grad{n-1} [B,T,C] in g_dtype (the
 * output type of the forward, or x_dtype).  `workspace` must hold
 * token_shift_mix_workspace_bytes() bytes. */
int token_shift_mix_backward(const void* x, int x_dtype, const float* mix, int64_t n,
                             const void* grad0, const void* grad1, const void* grad2, int g_dtype,
                             void* grad_x, float* grad_mix, void* workspace,
                             size_t workspace_bytes, int64_t B, int64_t T, int64_t C,
                             void* stream);

/* Squared ReLU of the channel mix, y = max(x, 0)^2, computed in fp32 and
 * rounded once to `dtype`: the values of torch.relu(key).square()
 * (src/spikegpt/language.py:1192) under autocast, where the square runs in
 * fp32 and the next projection casts.  n elements, a multiple of 16 bytes of
 * them (8 bf16/fp16 or 4 fp32). */
int relu_square_forward(const void* x, void* y, int64_t n, int dtype, void* stream);

/* Backward of relu_square_forward: grad_x = grad_y * 2 max(x, 0). */
int relu_square_backward(const void* x, const void* grad_y, void* grad_x, int64_t n, int dtype,
                         void* stream);

/* Sum of S fp32 partials: out[n] = sum_{s<S} partial[s][n], added in the
 * order s = 0, 1, ..., S-1.  partial [S][N], out [N]; N a multiple of 4.
 * The split-K weight gradients of the model's projections (each a sum of
 * GEMMs over slices of the B*T rows) end with it; the weight gradient of
 * the reference's nn.Linear projections (language.py:952-955, 1155-1157) is
 * one GEMM over all rows. */
int split_k_sum(const float* partial, float* out, int64_t S, int64_t N, void* stream);

/* Receptance gate y = sigmoid(r) * x (language.py:1035 sigmoid(r) * wkv and
 * :1194 sigmoid(r) * value): sigmoid rounded to `dtype`, then the product
 * rounded, as the two eager 16-bit kernels do.  n as relu_square_forward. */
int sigmoid_gate_forward(const void* r, const void* x, void* y, int64_t n, int dtype,
                         void* stream);

/* Backward of sigmoid_gate_forward: grad_x = g s, grad_r = g x s (1 - s),
 * s = sigmoid(r) in fp32. */
int sigmoid_gate_backward(const void* r, const void* x, const void* grad_y, void* grad_r,
                          void* grad_x, int64_t n, int dtype, void* stream);

/* LIF forward fused with the block's residual add (src/spikegpt/language.py:
 * 1326-1330, residual + lif(...)): out = residual + spikes(x), fp32
 * [B,T,C]; x in `dtype`; residual fp32 (out may alias it: then the sequence
 * is not split over time); membrane checkpoint as lif_forward; workspace as
 * lif_forward (lif_forward_workspace_bytes).  C a multiple of 8,
 * T*C*4 < 2^31. */
int lif_residual_forward(const void* x, const float* residual, float* out,
                         float* membrane_checkpoint, void* workspace, size_t workspace_bytes,
                         int64_t B, int64_t T, int64_t C, float decay, float threshold,
                         float reset, float slope, int dtype, void* stream);

/* Backward of lif_residual_forward for x: grad_x (`dtype`) from grad_out
 * (fp32, the gradient of out; the residual's gradient is grad_out itself);
 * workspace as lif_backward. */
int lif_residual_backward(const void* x, const float* grad_out, const float* membrane_checkpoint,
                          void* grad_x, void* workspace, size_t workspace_bytes, int64_t B,
                          int64_t T, int64_t C, float decay, float threshold, float reset,
                          float slope, int dtype, void* stream);

/* ---- Layer norm fused into the token-shift mix -----------------------------
 *
 * Replaces a block half's layer norm followed by its token-shift mixes,
 * self.att(self.ln1(x)) / self.ffn(self.ln2(x)) with _mix_with_previous
 * (src/spikegpt/language.py:1341-1356, 344-353): per row, F.layer_norm with
 * weight and bias, then out_j = y mu_j + y[t-1] (1 - mu_j), rounded once to
 * out_dtype.  x fp32 [B,T,C] with C = 256 or 512; weight, bias fp32 [C]; mix
 * fp32 [n][C], n = 2 or 3; out0..out{n-1} [B,T,C]; mean, rstd fp32 [B*T]
 * (saved for the backward). */
int layer_norm_shift_mix_forward(const float* x, const float* weight, const float* bias,
                                 float eps, const float* mix, int64_t n, void* out0, void* out1,
                                 void* out2, int out_dtype, float* mean, float* rstd, int64_t B,
                                 int64_t T, int64_t C, void* stream);

/* Bytes of workspace layer_norm_shift_mix_backward needs (column partial
 * sums), 0 for unsupported sizes. */
size_t layer_norm_shift_mix_workspace_bytes(int64_t n, int64_t B, int64_t T, int64_t C);

/* Backward: grad0..grad{n-1} [B,T,C] in g_dtype; writes grad_x fp32 [B,T,C]
 * and grad_params fp32 [n + 2][C] = (grad_mix_0 .. grad_mix_{n-1},
 * grad_weight, grad_bias), each summed over all rows in a fixed order.
 * grad_x_add (optional, NULL for none): fp32 [B,T,C] added to grad_x, the
 * gradient x receives through its other use (a block's residual stream,
 * language.py:1326-1330), so no separate add is needed. */
int layer_norm_shift_mix_backward(const float* x, const float* weight, const float* bias,
                                  const float* mix, int64_t n, const float* mean,
                                  const float* rstd, const void* grad0, const void* grad1,
                                  const void* grad2, int g_dtype, float* grad_x,
                                  const float* grad_x_add, float* grad_params, void* workspace,
                                  size_t workspace_bytes, int64_t B, int64_t T, int64_t C,
                                  void* stream);

/* ---- One-token block step (generation) ------------------------------------
 *
 * Replace the eager element-wise work of SpikeGPTBlock.step
 * (src/spikegpt/language.py:1301-1335) between its projections; the caller
 * runs the projections (GEMMs).  All tensors fp32 [B][C] unless noted; state
 * is read from *_in and written to *_out, which may be the same buffer. */

/* Pre-operation of block_step_row. */
enum wkv_step_pre {
  /* residual = [ln0](spike(embedding[ids]))  (language.py:1386-1394, 1317) */
  WKV_STEP_PRE_EMBED = 0,
  /* residual += LIF(add)  (first LIF of the block, language.py:1326-1327) */
  WKV_STEP_PRE_LIF = 1,
  /* residual += LIF(sigmoid(gate) * add)  (channel-mix gate :1187, second
   * LIF :1329-1330) */
  WKV_STEP_PRE_GATE_LIF = 2,
  /* residual = [ln0](residual): a block's own input (language.py:1317) */
  WKV_STEP_PRE_NONE = 3
};

typedef struct wkv_step_row_args {
  const int64_t* ids;          /* EMBED: token ids [B] */
  const float* embedding;      /* EMBED: [vocab][C] */
  int64_t vocab;               /* EMBED: rows of embedding; an id outside
                                  [0, vocab) gives a NaN row (no read) */
  float embedding_slope;       /* EMBED: spike = [slope * e >= 0] */
  int embedding_spike;         /* EMBED: 0 = raw embedding (spike_embedding off) */
  const float* ln0_weight;     /* EMBED, NONE: layer 0's ln0 (NULL: none) */
  const float* ln0_bias;
  const float* add;            /* LIF / GATE_LIF input */
  const float* gate;           /* GATE_LIF: receptance logits */
  const float* membrane_in;    /* LIF membrane state */
  float* membrane_out;
  float lif_decay, lif_threshold, lif_reset, lif_slope;
  int spiking;                 /* 0: LIF is the identity (config.spiking off) */
  float* residual;             /* written (EMBED) or updated (LIF, GATE_LIF) */
  const float* ln_weight;      /* layer norm applied to the new residual
                                  (NULL with n_mix 0: residual update only) */
  const float* ln_bias;
  float ln_eps;                /* also used for ln0 */
  const float* mix[3];         /* n_mix token-shift mixing vectors, [C] each */
  int n_mix;                   /* 3 (time mix k, v, r), 2 (channel mix k, r),
                                  0 (out[0] = the layer norm itself) */
  const float* previous_in;    /* token-shift state: the previous token's
                                  layer-norm output */
  float* previous_out;
  float* out[3];               /* out[j] = ln * mix[j] + previous * (1 - mix[j]) */
  int64_t batch, channels;     /* C <= 4096 */
} wkv_step_row_args;

/* One workgroup per batch row: the pre-operation, the residual write, a
 * layer norm, and the token-shift mixes (SpikeTimeMix.step :996-998,
 * SpikeChannelMix.step :1181-1182), in one launch. */
int block_step_row(int pre, const wkv_step_row_args* args, void* stream);

/* WKV state update and receptance gate of SpikeTimeMix.step
 * (language.py:999-1012): out = sigmoid(receptance) * wkv, state (numerator,
 * denominator, log_scale) in the reference's natural-log units; time_decay and
 * time_first [C] raw parameters (decay = -exp(time_decay)). */
int block_step_wkv(const float* key, const float* value, const float* receptance,
                   const float* time_decay, const float* time_first, const float* num_in,
                   const float* den_in, const float* log_scale_in, float* num_out,
                   float* den_out, float* log_scale_out, float* out, int64_t B, int64_t C,
                   void* stream);

/* Measurement hook; no counterpart in the reference.  Arms two HIP events
 * (hipEvent_t, created with timing enabled; either may be NULL) for the next
 * entry point called on this thread: its first kernel dispatch records
 * start_event at the kernel's start and its last dispatch records stop_event
 * at the kernel's end.  The events ride on the dispatch packets
 * (hipExtLaunchKernel), so the stream gets no extra marker packets and the
 * elapsed time is the kernels' own, as a kernel trace reports it.  One call
 * consumes the pair; an entry point that launches nothing leaves the events
 * unrecorded. */
int wkv_time_next_call(void* start_event, void* stop_event);

/* As wkv_time_next_call, but both events are bound to one kernel dispatch
 * of the next entry point: the `kernel`-th (from 0) kernel it launches, so
 * that one kernel's own duration is measured (e.g. the reverse sweep of a
 * backward without the batch-sum kernel after it).  No reference
 * counterpart; measurement only. */
int wkv_time_next_kernel(void* start_event, void* stop_event, int kernel);

/* Text of the last error raised on the calling thread ("" if none). */
const char* wkv_last_error_string(void);

/* Library version string. */
const char* wkv_version(void);

#ifdef __cplusplus
}
#endif

#endif /* WKV_HIP_H */
