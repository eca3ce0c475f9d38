// Layer norm fused into the token-shift mix of a SpikeGPT block, for gfx950.
//
// The blocks feed each mixing half through a layer norm
// (src/spikegpt/language.py:1341-1356: self.att(self.ln1(x)),
// self.ffn(self.ln2(x))) and the token-shift mixes (:344-353, 1016-1018,
// 1190-1191).  Per row r = (b, t) of x [B, T, C] (fp32 residual stream):
//   mean_r = sum_c x / C,  rstd_r = 1 / sqrt(sum_c (x - mean)^2 / C + eps)
//   y[r,c] = (x[r,c] - mean_r) rstd_r w[c] + bias[c]                  (F.layer_norm)
//   out_j[b,t,c] = y[b,t,c] mu_j[c] + y[b,t-1,c] (1 - mu_j[c]),  y[b,-1,:] = 0
// rounded once to the output type.  Backward, with g_j the output gradients
// and xhat = (x - mean) rstd:
//   gy[b,t,c] = sum_j g_j[b,t,c] mu_j[c] + g_j[b,t+1,c] (1 - mu_j[c])
//   gmu_j[c]  = sum_{b,t} g_j[b,t,c] (y[b,t,c] - y[b,t-1,c])
//   gw[c] = sum gy xhat,  gbias[c] = sum gy
//   gx = rstd (a - mean_c(a) - xhat mean_c(a xhat)),  a = gy w.
//
// Eager, this is the layer norm (read x, write y in fp32; its backward reads
// x, y's gradient and writes two more fp32 passes plus the partial gamma/beta
// sums) followed by the mix; fused, the forward reads x once and writes the n
// outputs and two floats per row, the backward reads x and the n gradients
// once and writes gx.
//
// Decomposition: a wave owns one row at a time, all C channels (lane l holds
// channels 256 j + 4 l + e, j < J = C/256, e < 4: 16-byte fp32 pieces), and
// walks a chunk of kLnRows consecutive rows of one sequence carrying the
// previous row's y (and, backward, the current row's gradients) in registers;
// row sums are wave butterflies.  C is 256 or 512 (J = 1, 2): a wider row
// needs more than half the register file per lane (J = 3 takes 205-256
// VGPRs).  Four waves per workgroup take consecutive
// chunks of the same sequence; the backward adds their column partials in LDS
// and writes one partial row per workgroup, summed over workgroups in fixed
// order by column_sum_kernel (deterministic).
#include "wkv_common.h"

namespace wkv {

constexpr int kLnRows = 32;    // rows per wave chunk
constexpr int kLnWaves = 4;    // waves (chunks) per workgroup
constexpr int kLnMaxN = 3;

template <typename RAW>
struct LnPtrs {
  RAW* p[kLnMaxN];
};

__device__ __forceinline__ float ln_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ void ln_wave_sum2(float& a, float& b) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ta = __shfl_xor(a, off, 64);
    const float tb = __shfl_xor(b, off, 64);
    a += ta;
    b += tb;
  }
}

// Loads the lane's J x 4 fp32 values of one row.
template <int J>
__device__ __forceinline__ void ln_load_row(float (&v)[J][4], const float* __restrict__ row,
                                            int lane) {
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const float4 t = *reinterpret_cast<const float4*>(row + 256 * j + 4 * lane);
    v[j][0] = t.x; v[j][1] = t.y; v[j][2] = t.z; v[j][3] = t.w;
  }
}

template <typename E, int J>
__device__ __forceinline__ void ln_load_grad(float (&v)[J][4], const typename E::raw* row,
                                             int lane) {
#pragma unroll
  for (int j = 0; j < J; ++j) {
    Pack<E, 4> p;
    p.load(row + 256 * j + 4 * lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[j][e] = p.get(e);
  }
}

// Row statistics of the lane's values (two passes from registers).
template <int J>
__device__ __forceinline__ void ln_stats(const float (&x)[J][4], int C, float eps, float& mean,
                                         float& rstd) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) s += x[j][e];
  mean = ln_wave_sum(s) / float(C);
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = x[j][e] - mean;
      q = fmaf(d, d, q);
    }
  rstd = 1.f / sqrtf(ln_wave_sum(q) / float(C) + eps);
}

// x: [B,T,C] fp32; w, bias: [C]; mix: [N][C]; out_j: [B,T,C] (EO);
// mean, rstd: [B*T].  Grid: ceil(n_items / 4) workgroups of 4 waves, item =
// (b, chunk) with the chunk fastest.
template <typename EO, int N, int J>
__global__ __launch_bounds__(256) void ln_mix_fwd_kernel(const float* __restrict__ x,
                                                         const float* __restrict__ w,
                                                         const float* __restrict__ bias,
                                                         const float* __restrict__ mix,
                                                         LnPtrs<typename EO::raw> out,
                                                         float* __restrict__ mean_out,
                                                         float* __restrict__ rstd_out, int B,
                                                         int T, float eps) {
  constexpr int C = 256 * J;
  constexpr int U = 4;  // rows loaded ahead
  const int n_tc = (T + kLnRows - 1) / kLnRows;
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * kLnWaves + (threadIdx.x >> 6);
  const int b = item / n_tc;
  if (b >= B) return;
  const int t0 = (item % n_tc) * kLnRows;
  const int t1 = min(T, t0 + kLnRows);
  const size_t seq = size_t(b) * T;

  float wv[J][4], bv[J][4], mu[N][J][4];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 256 * j + 4 * lane + e;
      wv[j][e] = w[c];
      bv[j][e] = bias[c];
#pragma unroll
      for (int n = 0; n < N; ++n) mu[n][j][e] = mix[n * C + c];
    }
  float prev[J][4];
  if (t0 > 0) {
    float xp[J][4];
    ln_load_row<J>(xp, x + (seq + t0 - 1) * C, lane);
    float m, r;
    ln_stats<J>(xp, C, eps, m, r);
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) prev[j][e] = (xp[j][e] - m) * r * wv[j][e] + bv[j][e];
  } else {
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) prev[j][e] = 0.f;
  }
  for (int t = t0; t < t1; t += U) {
    float xs[U][J][4];
#pragma unroll
    for (int i = 0; i < U; ++i)
      if (t + i < t1) ln_load_row<J>(xs[i], x + (seq + t + i) * C, lane);
#pragma unroll
    for (int i = 0; i < U; ++i) {
      if (t + i >= t1) break;
      const size_t row = seq + t + i;
      float m, r;
      ln_stats<J>(xs[i], C, eps, m, r);
      if (lane == 0) {
        mean_out[row] = m;
        rstd_out[row] = r;
      }
#pragma unroll
      for (int j = 0; j < J; ++j) {
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (xs[i][j][e] - m) * r * wv[j][e] + bv[j][e];
#pragma unroll
        for (int n = 0; n < N; ++n) {
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a = y[e] * mu[n][j][e];
            const float s = prev[j][e] * (1.f - mu[n][j][e]);
            o[e] = a + s;
          }
          store_vec<EO, 4>(out.p[n] + row * C + 256 * j + 4 * lane, o);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) prev[j][e] = y[e];
      }
    }
  }
}

// g_j: [B,T,C] (EG); gx: [B,T,C] fp32; gadd (optional): [B,T,C] fp32 added
// to gx (the gradient x receives through its other use, the residual
// stream); partial: [N + 2][P][C] fp32 with P = number of workgroups (rows:
// gmu_0..gmu_{N-1}, gw, gbias).
template <typename EG, int N, int J>
__global__ __launch_bounds__(256) void ln_mix_bwd_kernel(
    const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias,
    const float* __restrict__ mix, const float* __restrict__ mean,
    const float* __restrict__ rstd, LnPtrs<const typename EG::raw> g, float* __restrict__ gx,
    const float* __restrict__ gadd, float* __restrict__ partial, int B, int T) {
  constexpr int C = 256 * J;
  constexpr int F = N + 2;  // column-sum fields
  __shared__ float acc_lds[F * C];
  const int n_tc = (T + kLnRows - 1) / kLnRows;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int item = blockIdx.x * kLnWaves + wave;
  const int b = item / n_tc;
  const bool active = b < B;  // inactive waves still join the barriers
  const int t0 = (item % n_tc) * kLnRows;
  const int t1 = active ? min(T, t0 + kLnRows) : t0;
  const size_t seq = size_t(active ? b : 0) * T;

  float wv[J][4], bv[J][4], mu[N][J][4];
  float acc[F][J][4];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 256 * j + 4 * lane + e;
      wv[j][e] = w[c];
      bv[j][e] = bias[c];
#pragma unroll
      for (int n = 0; n < N; ++n) mu[n][j][e] = mix[n * C + c];
#pragma unroll
      for (int f = 0; f < F; ++f) acc[f][j][e] = 0.f;
    }
  float prev[J][4];
  float gcur[N][J][4];
  if (active && t0 > 0) {
    float xp[J][4];
    ln_load_row<J>(xp, x + (seq + t0 - 1) * C, lane);
    const float m = mean[seq + t0 - 1], r = rstd[seq + t0 - 1];
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) prev[j][e] = (xp[j][e] - m) * r * wv[j][e] + bv[j][e];
  } else {
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) prev[j][e] = 0.f;
  }
  // Software pipeline: the row being computed (x, statistics, the next
  // row's gradients) was loaded one iteration ahead.
  float xr[J][4], gn[N][J][4];
  float m_r = 0.f, r_r = 0.f;
  auto load_or_zero = [&](float (&v)[J][4], const typename EG::raw* p, bool ok) {
    if (ok) {
      ln_load_grad<EG, J>(v, p, lane);
    } else {
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[j][e] = 0.f;
    }
  };
  if (active && t0 < t1) {
#pragma unroll
    for (int n = 0; n < N; ++n) ln_load_grad<EG, J>(gcur[n], g.p[n] + (seq + t0) * C, lane);
    ln_load_row<J>(xr, x + (seq + t0) * C, lane);
    m_r = mean[seq + t0];
    r_r = rstd[seq + t0];
#pragma unroll
    for (int n = 0; n < N; ++n) load_or_zero(gn[n], g.p[n] + (seq + t0 + 1) * C, t0 + 1 < T);
  }
  for (int t = t0; t < t1; ++t) {
    const size_t row = seq + t;
    const bool more = t + 1 < t1;
    float xn[J][4], gnn[N][J][4];
    float m_n = 0.f, r_n = 0.f;
    if (more) {
      ln_load_row<J>(xn, x + (row + 1) * C, lane);
      m_n = mean[row + 1];
      r_n = rstd[row + 1];
    } else {
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) xn[j][e] = 0.f;
    }
#pragma unroll
    for (int n = 0; n < N; ++n) load_or_zero(gnn[n], g.p[n] + (row + 2) * C, more && t + 2 < T);
    // The added gradient of this row, used only at the store.
    float ga[J][4];
    if (gadd) ln_load_row<J>(ga, gadd + row * C, lane);
    const float m = m_r, r = r_r;
    float xh[J][4], a[J][4];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xh[j][e] = (xr[j][e] - m) * r;
        const float y = xh[j][e] * wv[j][e] + bv[j][e];
        float gy = 0.f;
#pragma unroll
        for (int n = 0; n < N; ++n) {
          gy = fmaf(gcur[n][j][e], mu[n][j][e], gy);
          gy = fmaf(gn[n][j][e], 1.f - mu[n][j][e], gy);
          acc[n][j][e] = fmaf(gcur[n][j][e], y - prev[j][e], acc[n][j][e]);
          gcur[n][j][e] = gn[n][j][e];
        }
        prev[j][e] = y;
        acc[N][j][e] = fmaf(gy, xh[j][e], acc[N][j][e]);
        acc[N + 1][j][e] += gy;
        a[j][e] = gy * wv[j][e];
        s1 += a[j][e];
        s2 = fmaf(a[j][e], xh[j][e], s2);
      }
    ln_wave_sum2(s1, s2);
    const float m1 = s1 / float(C), m2 = s2 / float(C);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = r * (a[j][e] - m1 - xh[j][e] * m2);
      if (gadd) {
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] += ga[j][e];
      }
      store_vec<F32, 4>(gx + row * C + 256 * j + 4 * lane, o);
    }
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xr[j][e] = xn[j][e];
#pragma unroll
        for (int n = 0; n < N; ++n) gn[n][j][e] = gnn[n][j][e];
      }
    m_r = m_n;
    r_r = r_n;
  }
  // Column partials of the four waves, added in LDS in wave order.
#pragma unroll 1
  for (int wv_turn = 0; wv_turn < kLnWaves; ++wv_turn) {
    if (wave == wv_turn) {
#pragma unroll
      for (int f = 0; f < F; ++f)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float* s = &acc_lds[f * C + 256 * j + 4 * lane + e];
            *s = wv_turn == 0 ? acc[f][j][e] : *s + acc[f][j][e];
          }
    }
    __syncthreads();
  }
  const int P = gridDim.x;
  for (int i = threadIdx.x; i < F * C; i += blockDim.x) {
    const int f = i / C, c = i % C;
    partial[(size_t(f) * P + blockIdx.x) * C + c] = acc_lds[i];
  }
}

}  // namespace wkv

// ------------------------------------------------------------ launchers ----
namespace wkv_host {

static int64_t ln_items(int64_t B, int64_t T) {
  return B * ((T + wkv::kLnRows - 1) / wkv::kLnRows);
}

int64_t ln_mix_workgroups(int64_t B, int64_t T) {
  return (ln_items(B, T) + wkv::kLnWaves - 1) / wkv::kLnWaves;
}

template <typename EO, int N, int J>
static int ln_fwd_launch(const float* x, const float* w, const float* bias, const float* mix,
                         void* const* out, float* mean, float* rstd, int B, int T, float eps,
                         hipStream_t s) {
  wkv::LnPtrs<typename EO::raw> o{};
  for (int n = 0; n < N; ++n) o.p[n] = static_cast<typename EO::raw*>(out[n]);
  launch(wkv::ln_mix_fwd_kernel<EO, N, J>, dim3(unsigned(ln_mix_workgroups(B, T))), dim3(256), s,
         true, x, w, bias, mix, o, mean, rstd, B, T, eps);
  return check_launch("ln_mix_fwd_kernel");
}

template <typename EO, int N>
static int ln_fwd_j(int J, const float* x, const float* w, const float* bias, const float* mix,
                    void* const* out, float* mean, float* rstd, int B, int T, float eps,
                    hipStream_t s) {
  switch (J) {
    case 1: return ln_fwd_launch<EO, N, 1>(x, w, bias, mix, out, mean, rstd, B, T, eps, s);
    case 2: return ln_fwd_launch<EO, N, 2>(x, w, bias, mix, out, mean, rstd, B, T, eps, s);
    default: return fail(1, "layer_norm_shift_mix: C must be 256 or 512");
  }
}

template <typename EO>
static int ln_fwd_n(int n, int J, const float* x, const float* w, const float* bias,
                    const float* mix, void* const* out, float* mean, float* rstd, int B, int T,
                    float eps, hipStream_t s) {
  switch (n) {
    case 2: return ln_fwd_j<EO, 2>(J, x, w, bias, mix, out, mean, rstd, B, T, eps, s);
    case 3: return ln_fwd_j<EO, 3>(J, x, w, bias, mix, out, mean, rstd, B, T, eps, s);
    default: return fail(1, "layer_norm_shift_mix: 2 or 3 mixing vectors");
  }
}

int ln_mix_forward_impl(const float* x, const float* w, const float* bias, const float* mix,
                        int n, void* const* out, int out_dtype, float* mean, float* rstd, int B,
                        int T, int C, float eps, hipStream_t s) {
  const int J = C / 256;
  switch (out_dtype) {
    case 0: return ln_fwd_n<wkv::F32>(n, J, x, w, bias, mix, out, mean, rstd, B, T, eps, s);
    case 1: return ln_fwd_n<wkv::BF16>(n, J, x, w, bias, mix, out, mean, rstd, B, T, eps, s);
    case 2: return ln_fwd_n<wkv::F16>(n, J, x, w, bias, mix, out, mean, rstd, B, T, eps, s);
    default: return fail(1, "layer_norm_shift_mix: unknown output dtype");
  }
}

template <typename EG, int N, int J>
static int ln_bwd_launch(const float* x, const float* w, const float* bias, const float* mix,
                         const float* mean, const float* rstd, const void* const* g, float* gx,
                         const float* gadd, float* partial, float* sums, int B, int T,
                         hipStream_t s) {
  wkv::LnPtrs<const typename EG::raw> gp{};
  for (int n = 0; n < N; ++n) gp.p[n] = static_cast<const typename EG::raw*>(g[n]);
  const int64_t P = ln_mix_workgroups(B, T);
  launch(wkv::ln_mix_bwd_kernel<EG, N, J>, dim3(unsigned(P)), dim3(256), s, false, x, w, bias,
         mix, mean, rstd, gp, gx, gadd, partial, B, T);
  int rc = check_launch("ln_mix_bwd_kernel");
  if (rc) return rc;
  launch(wkv::column_sum_kernel<16>, dim3(unsigned(J * 4), unsigned(N + 2)), dim3(1024), s, true,
         static_cast<const float*>(partial), sums, int(P), 256 * J);
  return check_launch("column_sum_kernel");
}

template <typename EG, int N>
static int ln_bwd_j(int J, const float* x, const float* w, const float* bias, const float* mix,
                    const float* mean, const float* rstd, const void* const* g, float* gx,
                    const float* gadd, float* partial, float* sums, int B, int T, hipStream_t s) {
  switch (J) {
    case 1:
      return ln_bwd_launch<EG, N, 1>(x, w, bias, mix, mean, rstd, g, gx, gadd, partial, sums, B, T, s);
    case 2:
      return ln_bwd_launch<EG, N, 2>(x, w, bias, mix, mean, rstd, g, gx, gadd, partial, sums, B, T, s);
    default: return fail(1, "layer_norm_shift_mix_backward: C must be 256 or 512");
  }
}

template <typename EG>
static int ln_bwd_n(int n, int J, const float* x, const float* w, const float* bias,
                    const float* mix, const float* mean, const float* rstd, const void* const* g,
                    float* gx, const float* gadd, float* partial, float* sums, int B, int T,
                    hipStream_t s) {
  switch (n) {
    case 2: return ln_bwd_j<EG, 2>(J, x, w, bias, mix, mean, rstd, g, gx, gadd, partial, sums, B, T, s);
    case 3: return ln_bwd_j<EG, 3>(J, x, w, bias, mix, mean, rstd, g, gx, gadd, partial, sums, B, T, s);
    default: return fail(1, "layer_norm_shift_mix_backward: 2 or 3 mixing vectors");
  }
}

int ln_mix_backward_impl(const float* x, const float* w, const float* bias, const float* mix,
                         int n, const float* mean, const float* rstd, const void* const* g,
                         int g_dtype, float* gx, const float* gadd, float* partial, float* sums,
                         int B, int T, int C, hipStream_t s) {
  const int J = C / 256;
  switch (g_dtype) {
    case 0:
      return ln_bwd_n<wkv::F32>(n, J, x, w, bias, mix, mean, rstd, g, gx, gadd, partial, sums, B, T, s);
    case 1:
      return ln_bwd_n<wkv::BF16>(n, J, x, w, bias, mix, mean, rstd, g, gx, gadd, partial, sums, B, T, s);
    case 2:
      return ln_bwd_n<wkv::F16>(n, J, x, w, bias, mix, mean, rstd, g, gx, gadd, partial, sums, B, T, s);
    default: return fail(1, "layer_norm_shift_mix_backward: unknown gradient dtype");
  }
}

}  // namespace wkv_host
