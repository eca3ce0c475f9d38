// Single-token WKV decode state update for gfx950.
//
// One generated token advances every (b, c) lane of a layer's state
// (numerator, denominator, log_scale) by one step of the recurrence in
// src/spikegpt/language.py:989-1012, which the reference runs as ~20 eager
// element-wise launches per layer.  Here it is one launch: each thread owns
// VEC consecutive channels, reads k, v and the state once and writes y and the
// new state once (36 B per fp32 lane).  The state stays in the reference's
// natural-log units so that callers holding a reference-format state can pass
// it unchanged.
#include "wkv_common.h"

namespace wkv {

template <typename E, int VEC>
__global__ __launch_bounds__(256) void wkv4_decode_kernel(
    const typename E::raw* __restrict__ k, const typename E::raw* __restrict__ v,
    const float* __restrict__ time_decay, const float* __restrict__ time_first,
    const float* num, const float* den, const float* log_scale,
    typename E::raw* __restrict__ y, float* num_out, float* den_out, float* ls_out, int B,
    int C) {
  const int64_t i0 = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * VEC;
  if (i0 >= int64_t(B) * C) return;
  const int c0 = int(i0 % C);
  Pack<E, VEC> kp, vp;
  kp.load(k + i0);
  vp.load(v + i0);
  Pack<F32, VEC> np, dp, lp;
  np.load(num + i0);
  dp.load(den + i0);
  lp.load(log_scale + i0);
  float yo[VEC], no[VEC], dn[VEC], ls[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    const float kk = kp.get(c);
    const float vv = vp.get(c);
    const float decay = -expf(time_decay[c0 + c]);
    const float first = time_first[c0 + c];
    const float l0 = lp.x[c];
    float nxt = fmaxf(l0, first + kk);
    float a = expf(l0 - nxt);
    float b = expf(first + kk - nxt);
    yo[c] = (a * np.x[c] + b * vv) / (a * dp.x[c] + b);
    const float decayed = l0 + decay;
    nxt = fmaxf(decayed, kk);
    a = expf(decayed - nxt);
    b = expf(kk - nxt);
    no[c] = a * np.x[c] + b * vv;
    dn[c] = a * dp.x[c] + b;
    ls[c] = nxt;
  }
  store_vec<E, VEC>(y + i0, yo);
  store_vec<F32, VEC>(num_out + i0, no);
  store_vec<F32, VEC>(den_out + i0, dn);
  store_vec<F32, VEC>(ls_out + i0, ls);
}

}  // namespace wkv

namespace wkv_host {

// Channels per thread of the one-token kernels: the widest vector that still
// launches at least 2^17 threads.  A token step is a single latency-bound
// round trip, so at B*C of a few hundred thousand more threads beat wider
// vectors (B=256, C=768: 4.0 us per layer at 4 channels, 3.5 at 1).
int decode_vec(int64_t n, int64_t C) {
  constexpr int64_t kMinThreads = int64_t(1) << 17;
  if (C % 4 == 0 && n / 4 >= kMinThreads) return 4;
  if (C % 2 == 0 && n / 2 >= kMinThreads) return 2;
  return 1;
}

template <typename E>
static int launch_decode(const void* k, const void* v, const float* td, const float* tf,
                         const float* num, const float* den, const float* ls, void* y,
                         float* num_out, float* den_out, float* ls_out, int B, int C,
                         hipStream_t stream) {
  using raw = typename E::raw;
  const int64_t n = int64_t(B) * C;
  const int vec = decode_vec(n, C);
  if (C % 4 == 0 && vec == 4) {
    const int64_t threads = n / 4;
    launch(wkv::wkv4_decode_kernel<E, 4>, dim3(unsigned((threads + 255) / 256)),
                       dim3(256), stream, true, static_cast<const raw*>(k),
                       static_cast<const raw*>(v), td, tf, num, den, ls, static_cast<raw*>(y),
                       num_out, den_out, ls_out, B, C);
  } else if (C % 2 == 0 && vec == 2) {
    const int64_t threads = n / 2;
    launch(wkv::wkv4_decode_kernel<E, 2>, dim3(unsigned((threads + 255) / 256)),
                       dim3(256), stream, true, static_cast<const raw*>(k),
                       static_cast<const raw*>(v), td, tf, num, den, ls, static_cast<raw*>(y),
                       num_out, den_out, ls_out, B, C);
  } else {
    launch(wkv::wkv4_decode_kernel<E, 1>, dim3(unsigned((n + 255) / 256)),
                       dim3(256), stream, true, static_cast<const raw*>(k),
                       static_cast<const raw*>(v), td, tf, num, den, ls, static_cast<raw*>(y),
                       num_out, den_out, ls_out, B, C);
  }
  return check_launch("wkv4_decode_kernel");
}

int wkv4_decode_impl(const void* k, const void* v, const float* td, const float* tf,
                     const float* num, const float* den, const float* ls, void* y,
                     float* num_out, float* den_out, float* ls_out, int B, int C, int dtype,
                     hipStream_t stream) {
  switch (dtype) {
    case 0:
      return launch_decode<wkv::F32>(k, v, td, tf, num, den, ls, y, num_out, den_out, ls_out, B,
                                     C, stream);
    case 1:
      return launch_decode<wkv::BF16>(k, v, td, tf, num, den, ls, y, num_out, den_out, ls_out, B,
                                      C, stream);
    case 2:
      return launch_decode<wkv::F16>(k, v, td, tf, num, den, ls, y, num_out, den_out, ls_out, B,
                                     C, stream);
    default:
      return fail(1, "wkv4_decode_step: unknown dtype");
  }
}

}  // namespace wkv_host
