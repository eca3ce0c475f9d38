// One-token SpikeGPT block step for generation, fused, for gfx950.
//
// The reference advances a block by one token in eager PyTorch
// (SpikeGPTBlock.step, src/spikegpt/language.py:1301-1335, with
// SpikeTimeMix.step :989-1012, SpikeChannelMix.step :1174-1188 and
// SpikingSequenceLIF.step :813-840): ~60 element-wise launches per layer
// around its seven projections.  Here everything between two projections is
// one launch, so a layer is four kernels plus the GEMMs:
//
//   row(embed | input | gated LIF) -> LN1 -> token shift (k, v, r) [row kernel]
//   k, v, r projections
//   WKV state update + sigmoid(r) * wkv                             [wkv kernel]
//   output projection
//   row(LIF of the output)  -> LN2 -> token shift (k, r)           [row kernel]
//   key / receptance projections, relu^2, value projection
//
// and the next layer's row kernel (or the final one, which applies ln_out)
// takes the channel mix's sigmoid(r) * value through the second LIF.
//
// Row kernel: one 256-thread workgroup per batch row; thread t owns channels
// t, t + 256, ... (EPT of them, coalesced).  The layer norms reduce the row in
// two passes (mean, then the centred second moment) from registers: a wave
// sum through DPP/permute, then four wave partials through LDS in fixed
// order.  All arithmetic is fp32 as in the reference's fp32 step; the state
// (previous-token rows, WKV numerator/denominator/log-scale, LIF membranes)
// is read from *_in and written to *_out, which may alias (each element is
// read and written by the same thread).
#include "../../include/wkv_hip.h"
#include "wkv_common.h"

namespace wkv {

constexpr int kStepThreads = 256;

enum StepPre : int {
  kPreEmbed = WKV_STEP_PRE_EMBED,
  kPreLif = WKV_STEP_PRE_LIF,
  kPreGateLif = WKV_STEP_PRE_GATE_LIF,
  kPreNone = WKV_STEP_PRE_NONE
};

using StepRowArgs = ::wkv_step_row_args;

// Sum over the workgroup's 256 threads, identical in every thread.
__device__ __forceinline__ float step_block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();  // red[] may still be read from the previous sum
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// x <- layer_norm(x) * weight + bias over the row's C channels (F.layer_norm,
// biased variance); slots past C hold 0 and stay out of the sums.
template <int EPT>
__device__ __forceinline__ void step_layer_norm(float (&x)[EPT], const float* __restrict__ w,
                                                const float* __restrict__ bias, float eps, int C,
                                                float* red) {
  const int tid = threadIdx.x;
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) s += x[e];
  const float mean = step_block_sum(s, red) / float(C);
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int c = tid + e * kStepThreads;
    const float d = c < C ? x[e] - mean : 0.f;
    q = fmaf(d, d, q);
  }
  const float var = step_block_sum(q, red) / float(C);
  const float rstd = 1.f / sqrtf(var + eps);
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int c = tid + e * kStepThreads;
    if (c < C) x[e] = (x[e] - mean) * rstd * w[c] + bias[c];
  }
}

__device__ __forceinline__ float step_sigmoid(float r) { return 1.f / (1.f + expf(-r)); }

template <int PRE, int N, int EPT>
__global__ __launch_bounds__(kStepThreads) void block_step_row_kernel(StepRowArgs a) {
  __shared__ float red[4];
  const int C = int(a.channels);
  const int tid = threadIdx.x;
  const size_t row = size_t(blockIdx.x) * size_t(C);
  float x[EPT];
  if constexpr (PRE == kPreEmbed) {
    // Spiking embedding (language.py:1386-1394): [slope * e >= 0].
    // An id outside the table reads nothing and poisons the row with NaN.
    const int64_t id = a.ids[blockIdx.x];
    const bool valid = id >= 0 && id < a.vocab;
    const float* e = a.embedding + (valid ? size_t(id) * size_t(C) : 0);
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int c = tid + i * kStepThreads;
      float v = 0.f;
      if (c < C) {
        v = valid ? e[c] : __builtin_nanf("");
        if (a.embedding_spike && valid) v = a.embedding_slope * v >= 0.f ? 1.f : 0.f;
      }
      x[i] = v;
    }
    if (a.ln0_weight != nullptr) step_layer_norm<EPT>(x, a.ln0_weight, a.ln0_bias, a.ln_eps, C, red);
  } else if constexpr (PRE == kPreNone) {
    // A block's own input (SpikeGPTBlock.step, language.py:1317).
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int c = tid + i * kStepThreads;
      x[i] = c < C ? a.residual[row + c] : 0.f;
    }
    if (a.ln0_weight != nullptr) step_layer_norm<EPT>(x, a.ln0_weight, a.ln0_bias, a.ln_eps, C, red);
  } else {
    // residual + LIF(in), in = the output projection (first LIF) or
    // sigmoid(r) * value (second LIF); language.py:833-839, 1326-1330.
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int c = tid + i * kStepThreads;
      float v = 0.f;
      if (c < C) {
        float in = a.add[row + c];
        if constexpr (PRE == kPreGateLif) in = step_sigmoid(a.gate[row + c]) * in;
        if (a.spiking) {
          const float h = a.membrane_in[row + c] * a.lif_decay + in;
          const float s = a.lif_slope * (h - a.lif_threshold) >= 0.f ? 1.f : 0.f;
          a.membrane_out[row + c] = h * (1.f - s) + a.lif_reset * s;
          in = s;
        } else if (a.membrane_out != a.membrane_in) {
          a.membrane_out[row + c] = a.membrane_in[row + c];
        }
        v = a.residual[row + c] + in;
      }
      x[i] = v;
    }
  }
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int c = tid + i * kStepThreads;
    if (c < C) a.residual[row + c] = x[i];
  }
  if (a.ln_weight == nullptr) return;  // residual update only (n_mix == 0)
  step_layer_norm<EPT>(x, a.ln_weight, a.ln_bias, a.ln_eps, C, red);
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int c = tid + i * kStepThreads;
    if (c >= C) continue;
    if constexpr (N == 0) {
      a.out[0][row + c] = x[i];
    } else {
      // inputs * mu + previous * (1 - mu)  (language.py:996-998, 1181-1182)
      const float p = a.previous_in[row + c];
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const float mu = a.mix[j][c];
        a.out[j][row + c] = x[i] * mu + p * (1.f - mu);
      }
      a.previous_out[row + c] = x[i];
    }
  }
}

// WKV state update and receptance gate of SpikeTimeMix.step
// (language.py:999-1012): out = sigmoid(r) * wkv, state in natural-log units.
template <int VEC>
__global__ __launch_bounds__(256) void block_step_wkv_kernel(
    const float* __restrict__ key, const float* __restrict__ value,
    const float* __restrict__ receptance, const float* __restrict__ time_decay,
    const float* __restrict__ time_first, const float* num_in, const float* den_in,
    const float* ls_in, float* num_out, float* den_out, float* ls_out, float* __restrict__ out,
    int64_t n, int C) {
  const int64_t i0 = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * VEC;
  if (i0 >= n) return;
  const int c0 = int(i0 % C);
  Pack<F32, VEC> kp, vp, rp, np, dp, lp;
  kp.load(key + i0);
  vp.load(value + i0);
  rp.load(receptance + i0);
  np.load(num_in + i0);
  dp.load(den_in + i0);
  lp.load(ls_in + i0);
  float o[VEC], no[VEC], dn[VEC], ls[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    const float k = kp.x[c], v = vp.x[c];
    const float decay = -expf(time_decay[c0 + c]);
    const float first = time_first[c0 + c];
    const float l0 = lp.x[c];
    float nxt = fmaxf(l0, first + k);
    float s_old = expf(l0 - nxt);
    float s_new = expf(first + k - nxt);
    const float mixed = (s_old * np.x[c] + s_new * v) / (s_old * dp.x[c] + s_new);
    o[c] = step_sigmoid(rp.x[c]) * mixed;
    const float decayed = l0 + decay;
    nxt = fmaxf(decayed, k);
    s_old = expf(decayed - nxt);
    s_new = expf(k - nxt);
    no[c] = s_old * np.x[c] + s_new * v;
    dn[c] = s_old * dp.x[c] + s_new;
    ls[c] = nxt;
  }
  store_vec<F32, VEC>(out + i0, o);
  store_vec<F32, VEC>(num_out + i0, no);
  store_vec<F32, VEC>(den_out + i0, dn);
  store_vec<F32, VEC>(ls_out + i0, ls);
}

}  // namespace wkv

// ------------------------------------------------------------ launchers ----
namespace wkv_host {

int decode_vec(int64_t n, int64_t C);

template <int PRE, int N, int EPT>
static int row_launch(const wkv::StepRowArgs& a, hipStream_t s) {
  launch(wkv::block_step_row_kernel<PRE, N, EPT>, dim3(unsigned(a.batch)), dim3(wkv::kStepThreads),
         s, true, a);
  return check_launch("block_step_row_kernel");
}

template <int PRE, int N>
static int row_ept(const wkv::StepRowArgs& a, hipStream_t s) {
  const int64_t ept = (a.channels + wkv::kStepThreads - 1) / wkv::kStepThreads;
  if (ept <= 1) return row_launch<PRE, N, 1>(a, s);
  if (ept <= 2) return row_launch<PRE, N, 2>(a, s);
  if (ept <= 3) return row_launch<PRE, N, 3>(a, s);
  if (ept <= 4) return row_launch<PRE, N, 4>(a, s);
  if (ept <= 8) return row_launch<PRE, N, 8>(a, s);
  return row_launch<PRE, N, 16>(a, s);
}

template <int PRE>
static int row_n(const wkv::StepRowArgs& a, hipStream_t s) {
  switch (a.n_mix) {
    case 0: return row_ept<PRE, 0>(a, s);
    case 2: return row_ept<PRE, 2>(a, s);
    case 3: return row_ept<PRE, 3>(a, s);
    default: return fail(1, "block_step_row: n_mix must be 0, 2 or 3");
  }
}

int block_step_row_impl(int pre, const wkv::StepRowArgs& a, hipStream_t s) {
  switch (pre) {
    case wkv::kPreEmbed: return row_n<wkv::kPreEmbed>(a, s);
    case wkv::kPreLif: return row_n<wkv::kPreLif>(a, s);
    case wkv::kPreGateLif: return row_n<wkv::kPreGateLif>(a, s);
    case wkv::kPreNone: return row_n<wkv::kPreNone>(a, s);
    default: return fail(1, "block_step_row: unknown pre-op");
  }
}

int block_step_wkv_impl(const float* k, const float* v, const float* r, const float* td,
                        const float* tf, const float* num_in, const float* den_in,
                        const float* ls_in, float* num_out, float* den_out, float* ls_out,
                        float* out, int64_t B, int64_t C, hipStream_t s) {
  const int64_t n = B * C;
  bool vec4 = decode_vec(n, C) == 4;
  for (const void* p : {static_cast<const void*>(k), static_cast<const void*>(v),
                        static_cast<const void*>(r), static_cast<const void*>(num_in),
                        static_cast<const void*>(den_in), static_cast<const void*>(ls_in),
                        static_cast<const void*>(num_out), static_cast<const void*>(den_out),
                        static_cast<const void*>(ls_out), static_cast<const void*>(out)})
    vec4 = vec4 && reinterpret_cast<uintptr_t>(p) % 16 == 0;
  if (vec4) {
    launch(wkv::block_step_wkv_kernel<4>, dim3(unsigned((n / 4 + 255) / 256)), dim3(256), s, true,
           k, v, r, td, tf, num_in, den_in, ls_in, num_out, den_out, ls_out, out, n, int(C));
  } else {
    launch(wkv::block_step_wkv_kernel<1>, dim3(unsigned((n + 255) / 256)), dim3(256), s, true, k,
           v, r, td, tf, num_in, den_in, ls_in, num_out, den_out, ls_out, out, n, int(C));
  }
  return check_launch("block_step_wkv_kernel");
}

}  // namespace wkv_host
