// RWKV-7 DPLR ("diagonal plus low rank") recurrence, forward, for gfx950.
//
// Per (batch, head) with head size N = 64 and state S[i][j] (i: value index,
// j: key index), for each step t:
//   S <- S (diag(w_t) + a_t b_t^T) + v_t k_t^T,   y_t = S r_t.
// Row i evolves as  S_i <- S_i * w + (S_i . a) b + v_i k ,  so the 64 rows
// are independent recurrences sharing the step's vectors.  One workgroup owns
// one (batch, head); NT threads share a row, each holding N/NT state columns
// in registers; the step's six input vectors are staged through LDS
// (double-buffered, loaded one step ahead) and the two row dot products
// (S_i . a and S_i . r) are reduced across the NT threads with cross-lane
// shuffles.  The arithmetic is fp32 on the vector ALUs: ~5 operations per
// state element per step, no matrix cores.
//
// The reference's RWKV-7 code was deleted
// (benchmarks/results/optimizer_wkv_experiments_5090.md:3); the output
// convention here (y_t = S_t r_t on the post-update state, no scale) is this
// library's own.
#include "wkv_common.h"

namespace wkv {

template <typename E, int NT>
__global__ __launch_bounds__(64 * NT) void wkv7_fwd_kernel(
    const typename E::raw* __restrict__ r, const typename E::raw* __restrict__ w,
    const typename E::raw* __restrict__ k, const typename E::raw* __restrict__ v,
    const typename E::raw* __restrict__ a, const typename E::raw* __restrict__ b,
    const float* __restrict__ s0, typename E::raw* __restrict__ y, float* __restrict__ s_out,
    int T, int H) {
  constexpr int N = 64;
  constexpr int CPT = N / NT;
  using raw = typename E::raw;
  __shared__ float vec[2][6][N];  // r, w, k, v, a, b

  const int bh = blockIdx.x;
  const int bi = bh / H;
  const int h = bh - bi * H;
  const int tid = threadIdx.x;
  const int row = tid / NT;
  const int part = tid - row * NT;
  const int j0 = part * CPT;
  const raw* src[6] = {r, w, k, v, a, b};

  float S[CPT];
  const size_t sbase = (size_t(bh) * N + row) * N + j0;
#pragma unroll
  for (int j = 0; j < CPT; ++j) S[j] = s0 ? s0[sbase + j] : 0.f;

  auto step_base = [&](int t) { return ((size_t(bi) * T + t) * H + h) * N; };
  const int which = tid / N;
  const int idx = tid - which * N;
  const bool loader = tid < 6 * N;
  if (loader && T > 0) vec[0][which][idx] = load_scalar<E>(src[which] + step_base(0) + idx);
  __syncthreads();

  for (int t = 0; t < T; ++t) {
    const int cur = t & 1;
    float nxt = 0.f;
    if (loader && t + 1 < T) nxt = load_scalar<E>(src[which] + step_base(t + 1) + idx);

    float rj[CPT], wj[CPT], kj[CPT], aj[CPT], bj[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      rj[j] = vec[cur][0][j0 + j];
      wj[j] = vec[cur][1][j0 + j];
      kj[j] = vec[cur][2][j0 + j];
      aj[j] = vec[cur][4][j0 + j];
      bj[j] = vec[cur][5][j0 + j];
    }
    const float vi = vec[cur][3][row];

    float sa = 0.f;
#pragma unroll
    for (int j = 0; j < CPT; ++j) sa = fmaf(S[j], aj[j], sa);
#pragma unroll
    for (int m = 1; m < NT; m <<= 1) sa += __shfl_xor(sa, m, NT);

    float yp = 0.f;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      S[j] = fmaf(S[j], wj[j], fmaf(sa, bj[j], vi * kj[j]));
      yp = fmaf(S[j], rj[j], yp);
    }
#pragma unroll
    for (int m = 1; m < NT; m <<= 1) yp += __shfl_xor(yp, m, NT);
    if (part == 0) store_scalar<E>(y + step_base(t) + row, yp);

    if (loader && t + 1 < T) vec[cur ^ 1][which][idx] = nxt;
    __syncthreads();
  }
  if (s_out) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) s_out[sbase + j] = S[j];
  }
}

}  // namespace wkv

namespace wkv_host {

template <typename E>
static int launch_wkv7(const void* r, const void* w, const void* k, const void* v, const void* a,
                       const void* b, const float* s0, void* y, float* s_out, int B, int T,
                       int H, hipStream_t stream) {
  using raw = typename E::raw;
  constexpr int NT = 16;
  hipLaunchKernelGGL((wkv::wkv7_fwd_kernel<E, NT>), dim3(unsigned(B) * H), dim3(64 * NT), 0,
                     stream, static_cast<const raw*>(r), static_cast<const raw*>(w),
                     static_cast<const raw*>(k), static_cast<const raw*>(v),
                     static_cast<const raw*>(a), static_cast<const raw*>(b), s0,
                     static_cast<raw*>(y), s_out, T, H);
  return check_launch("wkv7_fwd_kernel");
}

int wkv7_forward_impl(const void* r, const void* w, const void* k, const void* v, const void* a,
                      const void* b, const float* s0, void* y, float* s_out, int B, int T, int H,
                      int dtype, hipStream_t stream) {
  switch (dtype) {
    case 0: return launch_wkv7<wkv::F32>(r, w, k, v, a, b, s0, y, s_out, B, T, H, stream);
    case 1: return launch_wkv7<wkv::BF16>(r, w, k, v, a, b, s0, y, s_out, B, T, H, stream);
    case 2: return launch_wkv7<wkv::F16>(r, w, k, v, a, b, s0, y, s_out, B, T, H, stream);
    default: return fail(1, "wkv7_forward: unknown dtype");
  }
}

}  // namespace wkv_host
