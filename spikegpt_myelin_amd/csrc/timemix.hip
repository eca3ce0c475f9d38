// Token-shift mixing of SpikeGPT's time-mix and channel-mix blocks, fused,
// for gfx950.
//
// Math (src/spikegpt/language.py:344-353, used at :1016-1018 and
// :1190-1191): for mixing vectors mu_j [C], j < N (N = 3 for k, v, r of the
// time mix, 2 for k, r of the channel mix),
//   out_j[b,t,c] = x[b,t,c] * mu_j[c] + x[b,t-1,c] * (1 - mu_j[c])
// with x[b,-1,c] = 0, evaluated in fp32 with the reference's operation order
// (two products, then the sum) and rounded once to the output type -- the
// values the eager expression followed by autocast's bf16 cast produces.
// Backward:
//   gx[b,t,c]  = sum_j g_j[b,t,c] mu_j[c] + g_j[b,t+1,c] (1 - mu_j[c])
//   gmu_j[c]   = sum_{b,t} g_j[b,t,c] (x[b,t,c] - x[b,t-1,c]).
//
// The eager reference makes ~5 passes over [B,T,C] per mixing vector and
// another for the cast (fp32, ~42 B per element each); here one pass reads x
// once and writes the N outputs (4 + 2N bytes per element for fp32 in, bf16
// out), and the backward reads x and the N gradients once and writes gx.
//
// Decomposition: a wave owns 64*VEC consecutive channels of one batch row
// over a chunk of `chunk` steps (it re-reads the one row before its chunk);
// four waves per workgroup take consecutive chunks.  The host picks the
// chunk length (a power of two, 8 to 64 steps) so that the grid holds
// enough waves to keep loads in flight on every SIMD.  The mixing-vector
// gradient is reduced per wave in registers, written as per-(batch, chunk)
// partial sums and summed over them in fixed order by a second kernel
// (deterministic).
#include <type_traits>

#include "wkv_common.h"

namespace wkv {

constexpr int kTmMaxN = 3;

template <typename RAW>
struct Ptrs3 {
  RAW* p[kTmMaxN];
};

template <typename E, int VEC>
__device__ __forceinline__ void tm_load(float (&v)[VEC], const typename E::raw* p) {
  if constexpr (VEC == 1) {
    v[0] = load_scalar<E>(p);
  } else {
    Pack<E, VEC> pk;
    pk.load(p);
#pragma unroll
    for (int c = 0; c < VEC; ++c) v[c] = pk.get(c);
  }
}

template <typename E, int VEC>
__device__ __forceinline__ void tm_store(typename E::raw* p, const float (&v)[VEC]) {
  if constexpr (VEC == 1) {
    store_scalar<E>(p, v[0]);
  } else {
    store_vec<E, VEC>(p, v);
  }
}

// x: [B,T,C] (EI); mix: [N][C] fp32; out_j: [B,T,C] (EO).
template <typename EI, typename EO, int N, int VEC>
__global__ __launch_bounds__(256) void shift_mix_fwd_kernel(const typename EI::raw* __restrict__ x,
                                                            const float* __restrict__ mix,
                                                            Ptrs3<typename EO::raw> out, int B,
                                                            int T, int C, int chunk) {
  constexpr int U = 8;  // steps loaded ahead
  const int n_cg = (C + 64 * VEC - 1) / (64 * VEC);
  const int n_tc = (T + chunk - 1) / chunk;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + wave;  // (b, cg, tc), tc fastest
  const int tc = item % n_tc;
  const int rest = item / n_tc;
  const int cg = rest % n_cg;
  const int b = rest / n_cg;
  if (b >= B) return;  // the last workgroup may hold fewer than four items
  const int c0 = cg * 64 * VEC + lane * VEC;
  if (c0 >= C) return;
  const int t0 = tc * chunk;
  const int t1 = min(T, t0 + chunk);
  const size_t base = size_t(b) * T * C + c0;

  float mu[N][VEC], om[N][VEC];
#pragma unroll
  for (int j = 0; j < N; ++j)
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      mu[j][c] = mix[j * C + c0 + c];
      om[j][c] = 1.f - mu[j][c];
    }
  float prev[VEC];
  if (t0 > 0) {
    tm_load<EI, VEC>(prev, x + base + size_t(t0 - 1) * C);
  } else {
#pragma unroll
    for (int c = 0; c < VEC; ++c) prev[c] = 0.f;
  }
  for (int t = t0; t < t1; t += U) {
    float cur[U][VEC];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      if (t + i < t1) tm_load<EI, VEC>(cur[i], x + base + size_t(t + i) * C);
    }
#pragma unroll
    for (int i = 0; i < U; ++i) {
      if (t + i < t1) {
#pragma unroll
        for (int j = 0; j < N; ++j) {
          float o[VEC];
#pragma unroll
          for (int c = 0; c < VEC; ++c) {
            const float a = cur[i][c] * mu[j][c];
            const float s = prev[c] * om[j][c];
            o[c] = a + s;
          }
          tm_store<EO, VEC>(out.p[j] + base + size_t(t + i) * C, o);
        }
#pragma unroll
        for (int c = 0; c < VEC; ++c) prev[c] = cur[i][c];
      }
    }
  }
}

// g_j: [B,T,C] (EG); gx: [B,T,C] (EI); partial: [N][B*n_tc][C] fp32.
template <typename EI, typename EG, int N, int VEC>
__global__ __launch_bounds__(256) void shift_mix_bwd_kernel(const typename EI::raw* __restrict__ x,
                                                            const float* __restrict__ mix,
                                                            Ptrs3<const typename EG::raw> g,
                                                            typename EI::raw* __restrict__ gx,
                                                            float* __restrict__ partial, int B,
                                                            int T, int C, int chunk) {
  constexpr int U = 8;  // steps per block (measured: 2 and 4 no faster)
  const int n_cg = (C + 64 * VEC - 1) / (64 * VEC);
  const int n_tc = (T + chunk - 1) / chunk;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + wave;
  const int tc = item % n_tc;
  const int rest = item / n_tc;
  const int cg = rest % n_cg;
  const int b = rest / n_cg;
  if (b >= B) return;
  const int c0 = cg * 64 * VEC + lane * VEC;
  if (c0 >= C) return;
  const int t0 = tc * chunk;
  const int t1 = min(T, t0 + chunk);
  const size_t base = size_t(b) * T * C + c0;

  float mu[N][VEC], om[N][VEC], acc[N][VEC];
#pragma unroll
  for (int j = 0; j < N; ++j)
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      mu[j][c] = mix[j * C + c0 + c];
      om[j][c] = 1.f - mu[j][c];
      acc[j][c] = 0.f;
    }
  float prev[VEC];
  if (t0 > 0) {
    tm_load<EI, VEC>(prev, x + base + size_t(t0 - 1) * C);
  } else {
#pragma unroll
    for (int c = 0; c < VEC; ++c) prev[c] = 0.f;
  }
  // gcur[j] = g_j at the current step; the next step's gradient is loaded
  // with the batch (g at t = T is zero).
  float gn[N][VEC];
#pragma unroll
  for (int j = 0; j < N; ++j) tm_load<EG, VEC>(gn[j], g.p[j] + base + size_t(t0) * C);
  // A block of K steps (K = U, or 1 for the steps after the last whole
  // block): the loads of all K steps are issued first (16-bit gradients held
  // packed and converted where used), then the steps are computed and stored
  // in order.  No load sits under a branch (a load under a branch that joins
  // a constant gets a wait of its own): the gradient row after step T-1 is
  // read from row T-1 and replaced by zero.
  auto block = [&](int t, auto k_tag) {
    constexpr int K = decltype(k_tag)::value;
    Pack<EI, VEC> xs[K];
    Pack<EG, VEC> gs[K][N];
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const int tg = min(t + i + 1, T - 1);
      xs[i].load(x + base + size_t(t + i) * C);
#pragma unroll
      for (int j = 0; j < N; ++j) gs[i][j].load(g.p[j] + base + size_t(tg) * C);
    }
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const bool past_end = t + i + 1 >= T;
      float o[VEC];
#pragma unroll
      for (int c = 0; c < VEC; ++c) o[c] = 0.f;
#pragma unroll
      for (int j = 0; j < N; ++j) {
#pragma unroll
        for (int c = 0; c < VEC; ++c) {
          const float gc = gn[j][c];
          const float gnext = past_end ? 0.f : gs[i][j].get(c);
          o[c] = fmaf(gnext, om[j][c], fmaf(gc, mu[j][c], o[c]));
          acc[j][c] = fmaf(gc, xs[i].get(c) - prev[c], acc[j][c]);
          gn[j][c] = gnext;
        }
      }
      tm_store<EI, VEC>(gx + base + size_t(t + i) * C, o);
#pragma unroll
      for (int c = 0; c < VEC; ++c) prev[c] = xs[i].get(c);
    }
  };
  int t = t0;
  for (; t + U <= t1; t += U) block(t, std::integral_constant<int, U>{});
  for (; t < t1; ++t) block(t, std::integral_constant<int, 1>{});
  const size_t prow = size_t(b) * n_tc + tc;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    float* dst = partial + (size_t(j) * B * n_tc + prow) * C + c0;
#pragma unroll
    for (int c = 0; c < VEC; ++c) dst[c] = acc[j][c];
  }
}

}  // namespace wkv

// ------------------------------------------------------------ launchers ----
namespace wkv_host {

static int tm_vec(int C) { return C % 4 == 0 ? 4 : 1; }

// Steps per wave: the longest power-of-two chunk (64 down to 8) that still
// gives kTmMinWaves waves, two per SIMD.  Shorter chunks (more waves) were
// measured no faster at B=64, T=1024, C=512 and cost more partial sums.
// WKV_TM_CHUNK=8|16|32|64 in the environment overrides it (measurement).
constexpr int64_t kTmMinWaves = 2048;

static int tm_chunk(int64_t B, int64_t T, int64_t C) {
  static const int env = [] {
    const char* s = getenv("WKV_TM_CHUNK");
    const int v = s ? atoi(s) : 0;
    return (v == 8 || v == 16 || v == 32 || v == 64) ? v : 0;
  }();
  if (env) return env;
  const int64_t n_cg = (C + 64 * tm_vec(int(C)) - 1) / (64 * tm_vec(int(C)));
  int chunk = 64;
  while (chunk > 8 && B * n_cg * ((T + chunk - 1) / chunk) < kTmMinWaves) chunk /= 2;
  return chunk;
}

// Four waves per workgroup; wave items (b, cg, tc) enumerate tc fastest.
static dim3 tm_grid(int B, int T, int C, int vec, int chunk) {
  const int64_t n_cg = (C + 64 * vec - 1) / (64 * vec);
  const int64_t n_tc = (T + chunk - 1) / chunk;
  return dim3(unsigned((int64_t(B) * n_cg * n_tc + 3) / 4));
}

size_t shift_mix_partial_floats(int64_t N, int64_t B, int64_t T, int64_t C) {
  const int64_t chunk = tm_chunk(B, T, C);
  return size_t(N) * size_t(B) * size_t((T + chunk - 1) / chunk) * size_t(C);
}

template <typename EI, typename EO, int N, int VEC>
static int fwd_launch(const void* x, const float* mix, void* const* out, int B, int T, int C,
                      hipStream_t stream) {
  wkv::Ptrs3<typename EO::raw> o{};
  for (int j = 0; j < N; ++j) o.p[j] = static_cast<typename EO::raw*>(out[j]);
  const int chunk = tm_chunk(B, T, C);
  launch(wkv::shift_mix_fwd_kernel<EI, EO, N, VEC>, tm_grid(B, T, C, VEC, chunk), dim3(256), stream,
         true, static_cast<const typename EI::raw*>(x), mix, o, B, T, C, chunk);
  return check_launch("shift_mix_fwd_kernel");
}

template <typename EI, typename EO, int N>
static int fwd_vec(const void* x, const float* mix, void* const* out, int B, int T, int C,
                   hipStream_t stream) {
  return tm_vec(C) == 4 ? fwd_launch<EI, EO, N, 4>(x, mix, out, B, T, C, stream)
                        : fwd_launch<EI, EO, N, 1>(x, mix, out, B, T, C, stream);
}

template <typename EI, typename EO>
static int fwd_n(const void* x, const float* mix, void* const* out, int n, int B, int T, int C,
                 hipStream_t stream) {
  switch (n) {
    case 1: return fwd_vec<EI, EO, 1>(x, mix, out, B, T, C, stream);
    case 2: return fwd_vec<EI, EO, 2>(x, mix, out, B, T, C, stream);
    case 3: return fwd_vec<EI, EO, 3>(x, mix, out, B, T, C, stream);
    default: return fail(1, "token_shift_mix: 1 to 3 mixing vectors");
  }
}

int shift_mix_forward_impl(const void* x, int x_dtype, const float* mix, void* const* out,
                           int out_dtype, int n, int B, int T, int C, hipStream_t stream) {
  using namespace wkv;
  if (x_dtype == 0 && out_dtype == 0) return fwd_n<F32, F32>(x, mix, out, n, B, T, C, stream);
  if (x_dtype == 0 && out_dtype == 1) return fwd_n<F32, BF16>(x, mix, out, n, B, T, C, stream);
  if (x_dtype == 0 && out_dtype == 2) return fwd_n<F32, F16>(x, mix, out, n, B, T, C, stream);
  if (x_dtype == 1 && out_dtype == 1) return fwd_n<BF16, BF16>(x, mix, out, n, B, T, C, stream);
  if (x_dtype == 2 && out_dtype == 2) return fwd_n<F16, F16>(x, mix, out, n, B, T, C, stream);
  return fail(1, "token_shift_mix: unsupported input/output dtype pair");
}

template <typename EI, typename EG, int N, int VEC>
static int bwd_launch(const void* x, const float* mix, const void* const* g, void* gx,
                      float* partial, float* gmix, int B, int T, int C, hipStream_t stream) {
  wkv::Ptrs3<const typename EG::raw> gp{};
  for (int j = 0; j < N; ++j) gp.p[j] = static_cast<const typename EG::raw*>(g[j]);
  const int chunk = tm_chunk(B, T, C);
  launch(wkv::shift_mix_bwd_kernel<EI, EG, N, VEC>, tm_grid(B, T, C, VEC, chunk), dim3(256),
         stream, false, static_cast<const typename EI::raw*>(x), mix, gp,
         static_cast<typename EI::raw*>(gx), partial, B, T, C, chunk);
  int rc = check_launch("shift_mix_bwd_kernel");
  if (rc) return rc;
  const int P = B * ((T + chunk - 1) / chunk);
  launch(wkv::column_sum_kernel<16>, dim3(unsigned((C + 63) / 64), unsigned(N)), dim3(1024), stream,
         true, static_cast<const float*>(partial), gmix, P, C);
  return check_launch("column_sum_kernel");
}

template <typename EI, typename EG, int N>
static int bwd_vec(const void* x, const float* mix, const void* const* g, void* gx, float* partial,
                   float* gmix, int B, int T, int C, hipStream_t stream) {
  return tm_vec(C) == 4 ? bwd_launch<EI, EG, N, 4>(x, mix, g, gx, partial, gmix, B, T, C, stream)
                        : bwd_launch<EI, EG, N, 1>(x, mix, g, gx, partial, gmix, B, T, C, stream);
}

template <typename EI, typename EG>
static int bwd_n(const void* x, const float* mix, const void* const* g, void* gx, float* partial,
                 float* gmix, int n, int B, int T, int C, hipStream_t stream) {
  switch (n) {
    case 1: return bwd_vec<EI, EG, 1>(x, mix, g, gx, partial, gmix, B, T, C, stream);
    case 2: return bwd_vec<EI, EG, 2>(x, mix, g, gx, partial, gmix, B, T, C, stream);
    case 3: return bwd_vec<EI, EG, 3>(x, mix, g, gx, partial, gmix, B, T, C, stream);
    default: return fail(1, "token_shift_mix_backward: 1 to 3 mixing vectors");
  }
}

int shift_mix_backward_impl(const void* x, int x_dtype, const float* mix, const void* const* g,
                            int g_dtype, void* gx, float* partial, float* gmix, int n, int B,
                            int T, int C, hipStream_t stream) {
  using namespace wkv;
  if (x_dtype == 0 && g_dtype == 0)
    return bwd_n<F32, F32>(x, mix, g, gx, partial, gmix, n, B, T, C, stream);
  if (x_dtype == 0 && g_dtype == 1)
    return bwd_n<F32, BF16>(x, mix, g, gx, partial, gmix, n, B, T, C, stream);
  if (x_dtype == 0 && g_dtype == 2)
    return bwd_n<F32, F16>(x, mix, g, gx, partial, gmix, n, B, T, C, stream);
  if (x_dtype == 1 && g_dtype == 1)
    return bwd_n<BF16, BF16>(x, mix, g, gx, partial, gmix, n, B, T, C, stream);
  if (x_dtype == 2 && g_dtype == 2)
    return bwd_n<F16, F16>(x, mix, g, gx, partial, gmix, n, B, T, C, stream);
  return fail(1, "token_shift_mix_backward: unsupported input/gradient dtype pair");
}

}  // namespace wkv_host
