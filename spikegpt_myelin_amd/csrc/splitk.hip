// Sum of S partial matrices (split-K weight gradients): out[n] =
// sum_{s<S} partial[s][n], fp32, added in the order s = 0, 1, ..., S-1 (the
// result does not depend on the launch).  Each thread owns 4 consecutive
// elements and reads them from every partial with 16-byte loads: a wave reads
// 1 KB contiguous per partial, and all S loads of a thread are independent.
#include "wkv_common.h"

namespace wkv {

__global__ __launch_bounds__(256) void split_k_sum_kernel(const float* __restrict__ partial,
                                                          float* __restrict__ out, int S,
                                                          int64_t N) {
  const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= N) return;
  if (i + 4 <= N) {
    float4 a = *reinterpret_cast<const float4*>(partial + i);
    for (int s = 1; s < S; ++s) {
      const float4 b = *reinterpret_cast<const float4*>(partial + size_t(s) * N + i);
      a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
    }
    *reinterpret_cast<float4*>(out + i) = a;
  } else {
    for (int64_t j = i; j < N; ++j) {
      float a = partial[j];
      for (int s = 1; s < S; ++s) a += partial[size_t(s) * N + j];
      out[j] = a;
    }
  }
}

}  // namespace wkv

namespace wkv_host {

int split_k_sum_impl(const float* partial, float* out, int64_t S, int64_t N, hipStream_t stream) {
  const int64_t threads = (N + 3) / 4;
  const unsigned grid = unsigned((threads + 255) / 256);
  launch(wkv::split_k_sum_kernel, dim3(grid), dim3(256), stream, true, partial, out, int(S), N);
  return check_launch("split_k_sum_kernel");
}

}  // namespace wkv_host
