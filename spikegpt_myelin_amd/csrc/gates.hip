// Element-wise activations around SpikeGPT's projections, fused, for gfx950:
//
//  * squared ReLU of the channel mix, y = max(x, 0)^2
//    (src/spikegpt/language.py:1192, torch.relu(key).square());
//  * receptance gate, y = sigmoid(r) * x, of the time mix (:1035,
//    sigmoid(r) * wkv) and the channel mix (:1194, sigmoid(r) * value).
//
// Values match the eager expressions under autocast: the squared ReLU is
// computed in fp32 from the 16-bit input and rounded once (autocast runs
// square in fp32 and casts at the next projection); the gate rounds
// sigmoid(r) to the element type first and then the product, as the two eager
// bf16 kernels do.  Backward:
//   squared ReLU: gx = g * 2 max(x, 0);
//   gate:         gx = g * s,  gr = g * x * s (1 - s),  s = sigmoid(r) (fp32,
//                 gate_sigmoid: the short form for the 16-bit types).
// One pass each, 16-byte loads and stores per lane (8 bf16 or 4 fp32); the
// eager forms take two to four passes plus fp32 temporaries.
#include "wkv_common.h"

namespace wkv {

template <typename E>
struct Vec16 {
  static constexpr int N = 16 / int(sizeof(typename E::raw));
};

template <typename E>
__device__ __forceinline__ void unpack16(const u32x4& v, float (&f)[Vec16<E>::N]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  if constexpr (__is_same(E, F32)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (__is_same(E, BF16)) {
        f[2 * i] = __uint_as_float(w[i] << 16);
        f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        f[2 * i] = f16_bits_to_float(w[i] & 0xffffu);
        f[2 * i + 1] = f16_bits_to_float(w[i] >> 16);
      }
    }
  }
}

template <typename E>
__device__ __forceinline__ u32x4 pack16(const float (&f)[Vec16<E>::N]) {
  OutPack<E, Vec16<E>::N> o;
  o.set(f);
  return u32x4{o.u[0], o.u[1], o.u[2], o.u[3]};
}

// Elements [i*N, i*N + N) per thread; n is a multiple of N (checked on the
// host), so no tail.
template <typename E>
__global__ __launch_bounds__(256) void relu_square_fwd_kernel(const u32x4* __restrict__ x,
                                                              u32x4* __restrict__ y, int64_t nv) {
  constexpr int N = Vec16<E>::N;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= nv) return;
  float f[N];
  unpack16<E>(__builtin_nontemporal_load(x + i), f);
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const float r = fmaxf(f[j], 0.f);
    f[j] = r * r;
  }
  __builtin_nontemporal_store(pack16<E>(f), y + i);
}

template <typename E>
__global__ __launch_bounds__(256) void relu_square_bwd_kernel(const u32x4* __restrict__ x,
                                                              const u32x4* __restrict__ g,
                                                              u32x4* __restrict__ gx, int64_t nv) {
  constexpr int N = Vec16<E>::N;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= nv) return;
  float fx[N], fg[N];
  unpack16<E>(__builtin_nontemporal_load(x + i), fx);
  unpack16<E>(__builtin_nontemporal_load(g + i), fg);
#pragma unroll
  for (int j = 0; j < N; ++j) fx[j] = fg[j] * (2.f * fmaxf(fx[j], 0.f));
  __builtin_nontemporal_store(pack16<E>(fx), gx + i);
}

template <typename E>
__global__ __launch_bounds__(256) void sigmoid_gate_fwd_kernel(const u32x4* __restrict__ r,
                                                               const u32x4* __restrict__ x,
                                                               u32x4* __restrict__ y, int64_t nv) {
  constexpr int N = Vec16<E>::N;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= nv) return;
  float fr[N], fx[N];
  unpack16<E>(__builtin_nontemporal_load(r + i), fr);
  unpack16<E>(__builtin_nontemporal_load(x + i), fx);
#pragma unroll
  for (int j = 0; j < N; ++j) fr[j] = round_to<E>(gate_sigmoid<E>(fr[j])) * fx[j];
  __builtin_nontemporal_store(pack16<E>(fr), y + i);
}

template <typename E>
__global__ __launch_bounds__(256) void sigmoid_gate_bwd_kernel(const u32x4* __restrict__ r,
                                                               const u32x4* __restrict__ x,
                                                               const u32x4* __restrict__ g,
                                                               u32x4* __restrict__ gr,
                                                               u32x4* __restrict__ gx, int64_t nv) {
  constexpr int N = Vec16<E>::N;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= nv) return;
  float fr[N], fx[N], fg[N];
  unpack16<E>(__builtin_nontemporal_load(r + i), fr);
  unpack16<E>(__builtin_nontemporal_load(x + i), fx);
  unpack16<E>(__builtin_nontemporal_load(g + i), fg);
#pragma unroll
  for (int j = 0; j < N; ++j) {
    float grad_r;
    fx[j] = gate_backward<E>(fg[j], gate_sigmoid<E>(fr[j]), fx[j], grad_r);
    fr[j] = grad_r;
  }
  __builtin_nontemporal_store(pack16<E>(fr), gr + i);
  __builtin_nontemporal_store(pack16<E>(fx), gx + i);
}

}  // namespace wkv

// ------------------------------------------------------------ launchers ----
namespace wkv_host {

using wkv::u32x4;

// Number of 16-byte vectors in n elements of `dtype` (n a multiple of the
// vector width, checked by the caller).
static int64_t vec_count(int64_t n, int dtype) { return n / (dtype == 0 ? 4 : 8); }

template <typename F, typename... Args>
static int launch_1d(F kernel, int64_t nv, hipStream_t stream, Args... args) {
  const int64_t blocks = (nv + 255) / 256;
  launch(kernel, dim3(unsigned(blocks)), dim3(256), stream, true, args..., nv);
  return check_launch("gate kernel");
}

int relu_square_forward_impl(const void* x, void* y, int64_t n, int dtype, hipStream_t s) {
  const int64_t nv = vec_count(n, dtype);
  auto X = static_cast<const u32x4*>(x);
  auto Y = static_cast<u32x4*>(y);
  switch (dtype) {
    case 0: return launch_1d(wkv::relu_square_fwd_kernel<wkv::F32>, nv, s, X, Y);
    case 1: return launch_1d(wkv::relu_square_fwd_kernel<wkv::BF16>, nv, s, X, Y);
    case 2: return launch_1d(wkv::relu_square_fwd_kernel<wkv::F16>, nv, s, X, Y);
    default: return fail(1, "relu_square: unknown dtype");
  }
}

int relu_square_backward_impl(const void* x, const void* g, void* gx, int64_t n, int dtype,
                              hipStream_t s) {
  const int64_t nv = vec_count(n, dtype);
  auto X = static_cast<const u32x4*>(x);
  auto G = static_cast<const u32x4*>(g);
  auto GX = static_cast<u32x4*>(gx);
  switch (dtype) {
    case 0: return launch_1d(wkv::relu_square_bwd_kernel<wkv::F32>, nv, s, X, G, GX);
    case 1: return launch_1d(wkv::relu_square_bwd_kernel<wkv::BF16>, nv, s, X, G, GX);
    case 2: return launch_1d(wkv::relu_square_bwd_kernel<wkv::F16>, nv, s, X, G, GX);
    default: return fail(1, "relu_square: unknown dtype");
  }
}

int sigmoid_gate_forward_impl(const void* r, const void* x, void* y, int64_t n, int dtype,
                              hipStream_t s) {
  const int64_t nv = vec_count(n, dtype);
  auto R = static_cast<const u32x4*>(r);
  auto X = static_cast<const u32x4*>(x);
  auto Y = static_cast<u32x4*>(y);
  switch (dtype) {
    case 0: return launch_1d(wkv::sigmoid_gate_fwd_kernel<wkv::F32>, nv, s, R, X, Y);
    case 1: return launch_1d(wkv::sigmoid_gate_fwd_kernel<wkv::BF16>, nv, s, R, X, Y);
    case 2: return launch_1d(wkv::sigmoid_gate_fwd_kernel<wkv::F16>, nv, s, R, X, Y);
    default: return fail(1, "sigmoid_gate: unknown dtype");
  }
}

int sigmoid_gate_backward_impl(const void* r, const void* x, const void* g, void* gr, void* gx,
                               int64_t n, int dtype, hipStream_t s) {
  const int64_t nv = vec_count(n, dtype);
  auto R = static_cast<const u32x4*>(r);
  auto X = static_cast<const u32x4*>(x);
  auto G = static_cast<const u32x4*>(g);
  auto GR = static_cast<u32x4*>(gr);
  auto GX = static_cast<u32x4*>(gx);
  switch (dtype) {
    case 0: return launch_1d(wkv::sigmoid_gate_bwd_kernel<wkv::F32>, nv, s, R, X, G, GR, GX);
    case 1: return launch_1d(wkv::sigmoid_gate_bwd_kernel<wkv::BF16>, nv, s, R, X, G, GR, GX);
    case 2: return launch_1d(wkv::sigmoid_gate_bwd_kernel<wkv::F16>, nv, s, R, X, G, GR, GX);
    default: return fail(1, "sigmoid_gate: unknown dtype");
  }
}

}  // namespace wkv_host
