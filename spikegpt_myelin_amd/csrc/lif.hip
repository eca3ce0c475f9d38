// Sequence LIF (leaky integrate-and-fire) activation of SpikeGPT, forward
// and backward, for gfx950.
//
// Math (src/spikegpt/language.py:813-840 and the time loop :910-918), per
// (batch b, channel c) lane, membrane m_0 = 0:
//   h_t = m_{t-1} * decay + x_t                    (decay = 1 - 1/tau)
//   c_t = slope * (h_t - threshold)
//   s_t = [c_t >= 0]                               (hard forward spike)
//   m_t = h_t * (1 - s_t) + reset * s_t
// with the arctan surrogate derivative in the backward:
//   ds_t/dh_t = slope * 0.5 / (1 + (pi/2 * c_t)^2).
// Backward (dL/ds_t = g_t from upstream, dL/dm_t = gm carried from t+1):
//   dL/dh_t = g_t ds/dh + gm ((1 - s_t) + (reset - h_t) ds/dh)
//   dL/dx_t = dL/dh_t,   gm <- decay * dL/dh_t.
// The reset path is differentiated (the spike is not detached from the
// membrane update), as autograd does through the reference's eager step.
//
// The recurrence is nonlinear (threshold and reset), so there is no
// parallelism over time: a lane owns VEC channels of one batch row for the
// whole sequence.  Work decomposition: one wave64 workgroup per (batch, 64*VEC
// channels); per step a wave reads and writes one contiguous row segment
// (128 or 256 bytes).  Time is walked in segments of S steps; the next
// segment's inputs are prefetched into registers (double-buffered) through
// buffer descriptors (steps past T read as zero).  Spikes are exact 0/1 in the
// element type.
//
// Checkpoints: the forward stores the membrane at the start of every block of
// kLifBlock steps ([B][ceil(T/kLifBlock)][C] fp32, 0.125 B per element); the
// backward walks the blocks last to first, recomputes each block's h_t from
// its record into registers and runs the reverse recurrence over it, so x is
// read once by each pass and no per-step state is stored.
#include "wkv_common.h"

namespace wkv {

constexpr int kLifBlock = 32;  // steps per membrane checkpoint (= backward segment)

struct LifParams {
  float decay, threshold, reset, slope;
};

// Loads S steps starting at t0 for the lane (buffer descriptor based at the
// segment; steps at or past T read as zero).
template <typename E, int VEC, int S>
__device__ __forceinline__ void lif_load(Pack<E, VEC> (&xb)[S], const typename E::raw* __restrict__ x,
                                         size_t row_base, size_t row_tail, unsigned lane_boff, int t0,
                                         int C) {
  using raw = typename E::raw;
  const uint32_t bytes = span_bytes(row_tail, t0, C, int(sizeof(raw)));
  const rsrc_t r = make_rsrc(x + row_base + size_t(t0) * C, bytes);
  const unsigned stride = unsigned(C) * unsigned(sizeof(raw));
#pragma unroll
  for (int i = 0; i < S; ++i) load_buf(xb[i], r, lane_boff, unsigned(i) * stride);
}

template <typename E, int VEC, int S>
__device__ __forceinline__ void lif_fwd_segment(const Pack<E, VEC> (&xb)[S], float (&m)[VEC],
                                                const LifParams& P, typename E::raw* __restrict__ spk,
                                                float* __restrict__ ck, size_t row_base,
                                                size_t row_tail, unsigned lane_boff, size_t ck_row,
                                                unsigned ck_boff, int t0, int T, int C, bool active) {
  static_assert(S % kLifBlock == 0, "segments hold whole checkpoint blocks");
  OutPack<E, VEC> o[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    if (i % kLifBlock == 0 && ck != nullptr && active && t0 + i < T) {
      float* rec = ck + ck_row + size_t((t0 + i) / kLifBlock) * C;
      store_vec<F32, VEC>(byte_offset(rec, ck_boff), m);
    }
    float sv[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const float h = m[c] * P.decay + xb[i].get(c);
      const float s = P.slope * (h - P.threshold) >= 0.f ? 1.f : 0.f;
      m[c] = h * (1.f - s) + P.reset * s;
      sv[c] = s;
    }
    o[i].set(sv);
  }
  if (active) {
    // Steps past T fall outside the descriptor and are dropped.
    const rsrc_t r = make_rsrc(spk + row_base + size_t(t0) * C,
                               span_bytes(row_tail, t0, C, int(sizeof(typename E::raw))));
    const unsigned stride = unsigned(C) * unsigned(sizeof(typename E::raw));
#pragma unroll
    for (int i = 0; i < S; ++i) store_buf(o[i], r, lane_boff, unsigned(i) * stride);
  }
}

// ck may be null (no records).
template <typename E, int VEC, int S>
__global__ __launch_bounds__(64) void lif_fwd_kernel(const typename E::raw* __restrict__ x,
                                                     typename E::raw* __restrict__ spk,
                                                     float* __restrict__ ck, int T, int C,
                                                     LifParams P) {
  constexpr int CPW = 64 * VEC;
  const int n_cg = (C + CPW - 1) / CPW;
  const int b = blockIdx.x / n_cg;
  const int cg = blockIdx.x - b * n_cg;
  const int lane = threadIdx.x;
  const bool active = cg * CPW + lane * VEC < C;
  const size_t row_base = size_t(b) * T * C + size_t(cg) * CPW;
  const size_t row_tail = size_t(T) * C - size_t(cg) * CPW;
  const unsigned lane_boff = active ? unsigned(lane * VEC * sizeof(typename E::raw)) : 0u;
  const int nblk = (T + kLifBlock - 1) / kLifBlock;
  const size_t ck_row = size_t(b) * nblk * C + size_t(cg) * CPW;
  const unsigned ck_boff = active ? unsigned(lane * VEC * sizeof(float)) : 0u;

  float m[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) m[c] = 0.f;
  const int nseg = (T + S - 1) / S;
  Pack<E, VEC> xa[S], xb[S];
  lif_load<E, VEC, S>(xa, x, row_base, row_tail, lane_boff, 0, C);
  for (int seg = 0; seg < nseg; seg += 2) {
    // The next segment is loaded on every path (past the end the descriptor
    // is empty), so the wait before a segment only covers its own loads.
    lif_load<E, VEC, S>(xb, x, row_base, row_tail, lane_boff, (seg + 1) * S, C);
    lif_fwd_segment<E, VEC, S>(xa, m, P, spk, ck, row_base, row_tail, lane_boff, ck_row, ck_boff,
                               seg * S, T, C, active);
    if (seg + 1 >= nseg) break;
    lif_load<E, VEC, S>(xa, x, row_base, row_tail, lane_boff, (seg + 2) * S, C);
    lif_fwd_segment<E, VEC, S>(xb, m, P, spk, ck, row_base, row_tail, lane_boff, ck_row, ck_boff,
                               (seg + 1) * S, T, C, active);
  }
}

// One backward block (kLifBlock steps from t0): recompute h from the block's
// membrane record, then the reverse recurrence writing dL/dx.  Steps past T
// read x = 0 and g = 0, so they leave the carry at zero.
template <typename E, int VEC>
__device__ __forceinline__ void lif_bwd_block(const Pack<E, VEC> (&xb)[kLifBlock],
                                              const Pack<E, VEC> (&gb)[kLifBlock],
                                              float (&gm)[VEC], const LifParams& P,
                                              const float* __restrict__ ck,
                                              typename E::raw* __restrict__ gx, size_t row_base,
                                              size_t row_tail, unsigned lane_boff, size_t ck_row,
                                              unsigned ck_boff, int t0, int C, bool active) {
  constexpr int S = kLifBlock;
  constexpr float kHalfPi = 1.5707963267948966f;
  Pack<F32, VEC> m0;
  m0.load(byte_offset(ck + ck_row + size_t(t0 / S) * C, ck_boff));
  float h[S][VEC];
  float m[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) m[c] = active ? m0.x[c] : 0.f;
#pragma unroll
  for (int i = 0; i < S; ++i) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const float hh = m[c] * P.decay + xb[i].get(c);
      const float s = P.slope * (hh - P.threshold) >= 0.f ? 1.f : 0.f;
      m[c] = hh * (1.f - s) + P.reset * s;
      h[i][c] = hh;
    }
  }
  OutPack<E, VEC> o[S];
#pragma unroll
  for (int i = S - 1; i >= 0; --i) {
    float gv[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const float hh = h[i][c];
      const float cc = P.slope * (hh - P.threshold);
      const float s = cc >= 0.f ? 1.f : 0.f;
      const float q = kHalfPi * cc;
      const float dsdh = P.slope * (0.5f / (1.f + q * q));
      const float gh = gb[i].get(c) * dsdh + gm[c] * ((1.f - s) + (P.reset - hh) * dsdh);
      gv[c] = gh;
      gm[c] = P.decay * gh;
    }
    o[i].set(gv);
  }
  if (active) {
    const rsrc_t r = make_rsrc(gx + row_base + size_t(t0) * C,
                               span_bytes(row_tail, t0, C, int(sizeof(typename E::raw))));
    const unsigned stride = unsigned(C) * unsigned(sizeof(typename E::raw));
#pragma unroll
    for (int i = S - 1; i >= 0; --i) store_buf(o[i], r, lane_boff, unsigned(i) * stride);
  }
}

template <typename E, int VEC>
__global__ __launch_bounds__(64) void lif_bwd_kernel(const typename E::raw* __restrict__ x,
                                                     const typename E::raw* __restrict__ gs,
                                                     const float* __restrict__ ck,
                                                     typename E::raw* __restrict__ gx, int T,
                                                     int C, LifParams P) {
  constexpr int CPW = 64 * VEC;
  constexpr int S = kLifBlock;
  const int n_cg = (C + CPW - 1) / CPW;
  const int b = blockIdx.x / n_cg;
  const int cg = blockIdx.x - b * n_cg;
  const int lane = threadIdx.x;
  const bool active = cg * CPW + lane * VEC < C;
  const size_t row_base = size_t(b) * T * C + size_t(cg) * CPW;
  const size_t row_tail = size_t(T) * C - size_t(cg) * CPW;
  const unsigned lane_boff = active ? unsigned(lane * VEC * sizeof(typename E::raw)) : 0u;
  const int nblk = (T + S - 1) / S;
  const size_t ck_row = size_t(b) * nblk * C + size_t(cg) * CPW;
  const unsigned ck_boff = active ? unsigned(lane * VEC * sizeof(float)) : 0u;

  float gm[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) gm[c] = 0.f;
  Pack<E, VEC> xa[S], ga[S], xb[S], gb[S];
  const int last = nblk - 1;
  lif_load<E, VEC, S>(xa, x, row_base, row_tail, lane_boff, last * S, C);
  lif_load<E, VEC, S>(ga, gs, row_base, row_tail, lane_boff, last * S, C);
  for (int blk = last; blk >= 0; blk -= 2) {
    // Block 0 prefetches itself again (a cache hit) so that the same loads
    // are issued on every path.
    const int p1 = max(blk - 1, 0), p2 = max(blk - 2, 0);
    lif_load<E, VEC, S>(xb, x, row_base, row_tail, lane_boff, p1 * S, C);
    lif_load<E, VEC, S>(gb, gs, row_base, row_tail, lane_boff, p1 * S, C);
    lif_bwd_block<E, VEC>(xa, ga, gm, P, ck, gx, row_base, row_tail, lane_boff, ck_row, ck_boff,
                          blk * S, C, active);
    if (blk - 1 < 0) break;
    lif_load<E, VEC, S>(xa, x, row_base, row_tail, lane_boff, p2 * S, C);
    lif_load<E, VEC, S>(ga, gs, row_base, row_tail, lane_boff, p2 * S, C);
    lif_bwd_block<E, VEC>(xb, gb, gm, P, ck, gx, row_base, row_tail, lane_boff, ck_row, ck_boff,
                          (blk - 1) * S, C, active);
  }
}

}  // namespace wkv

// ------------------------------------------------------------ launchers ----
namespace wkv_host {

size_t lif_checkpoint_floats(int64_t B, int64_t T, int64_t C) {
  return size_t(B) * size_t((T + wkv::kLifBlock - 1) / wkv::kLifBlock) * size_t(C);
}

// 16-bit types: two channels per lane (256-byte rows) when C is even and
// that still leaves at least 256 waves; else one.  fp32: one channel per lane
// (256-byte rows already).
static int lif_vec(int64_t B, int64_t C, int elem_bytes) {
  if (elem_bytes == 4 || C % 2 != 0) return 1;
  return B * ((C + 127) / 128) >= 256 ? 2 : 1;
}

template <typename E, int VEC>
static int lif_fwd_launch(const void* x, void* spk, float* ck, int B, int T, int C,
                          const wkv::LifParams& P, hipStream_t stream) {
  using raw = typename E::raw;
  // Forward segment: two checkpoint blocks for 16-bit types, one for fp32
  // (register budget of the double-buffered inputs).
  constexpr int S = sizeof(raw) == 2 ? 2 * wkv::kLifBlock : wkv::kLifBlock;
  const int n_cg = (C + 64 * VEC - 1) / (64 * VEC);
  launch(wkv::lif_fwd_kernel<E, VEC, S>, dim3(unsigned(B) * unsigned(n_cg)), dim3(64), stream,
         true, static_cast<const raw*>(x), static_cast<raw*>(spk), ck, T, C, P);
  return check_launch("lif_fwd_kernel");
}

template <typename E, int VEC>
static int lif_bwd_launch(const void* x, const void* gs, const float* ck, void* gx, int B, int T,
                          int C, const wkv::LifParams& P, hipStream_t stream) {
  using raw = typename E::raw;
  const int n_cg = (C + 64 * VEC - 1) / (64 * VEC);
  launch(wkv::lif_bwd_kernel<E, VEC>, dim3(unsigned(B) * unsigned(n_cg)), dim3(64), stream, true,
         static_cast<const raw*>(x), static_cast<const raw*>(gs), ck, static_cast<raw*>(gx), T, C,
         P);
  return check_launch("lif_bwd_kernel");
}

template <typename E>
static int lif_fwd_dispatch(const void* x, void* spk, float* ck, int B, int T, int C,
                            const wkv::LifParams& P, hipStream_t stream) {
  return lif_vec(B, C, int(sizeof(typename E::raw))) == 2 ? lif_fwd_launch<E, 2>(x, spk, ck, B, T, C, P, stream)
                            : lif_fwd_launch<E, 1>(x, spk, ck, B, T, C, P, stream);
}

template <typename E>
static int lif_bwd_dispatch(const void* x, const void* gs, const float* ck, void* gx, int B,
                            int T, int C, const wkv::LifParams& P, hipStream_t stream) {
  return lif_vec(B, C, int(sizeof(typename E::raw))) == 2 ? lif_bwd_launch<E, 2>(x, gs, ck, gx, B, T, C, P, stream)
                            : lif_bwd_launch<E, 1>(x, gs, ck, gx, B, T, C, P, stream);
}

int lif_forward_impl(const void* x, void* spk, float* ck, int B, int T, int C, float decay,
                     float threshold, float reset, float slope, int dtype, hipStream_t stream) {
  const wkv::LifParams P{decay, threshold, reset, slope};
  switch (dtype) {
    case 0: return lif_fwd_dispatch<wkv::F32>(x, spk, ck, B, T, C, P, stream);
    case 1: return lif_fwd_dispatch<wkv::BF16>(x, spk, ck, B, T, C, P, stream);
    case 2: return lif_fwd_dispatch<wkv::F16>(x, spk, ck, B, T, C, P, stream);
    default: return fail(1, "lif_forward: unknown dtype");
  }
}

int lif_backward_impl(const void* x, const void* gs, const float* ck, void* gx, int B, int T,
                      int C, float decay, float threshold, float reset, float slope, int dtype,
                      hipStream_t stream) {
  const wkv::LifParams P{decay, threshold, reset, slope};
  switch (dtype) {
    case 0: return lif_bwd_dispatch<wkv::F32>(x, gs, ck, gx, B, T, C, P, stream);
    case 1: return lif_bwd_dispatch<wkv::BF16>(x, gs, ck, gx, B, T, C, P, stream);
    case 2: return lif_bwd_dispatch<wkv::F16>(x, gs, ck, gx, B, T, C, P, stream);
    default: return fail(1, "lif_backward: unknown dtype");
  }
}

}  // namespace wkv_host
