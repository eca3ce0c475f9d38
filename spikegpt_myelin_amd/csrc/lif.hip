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
#include <algorithm>
#include <cstdlib>

#include "wkv_common.h"

namespace wkv {

constexpr int kLifBlock = 32;  // steps per membrane checkpoint (= backward segment)

struct LifParams {
  float decay, threshold, reset, slope;
};

// One reverse step of the LIF backward: dL/dh_t for the incoming gradient
// g of s_t and the carried gradient gm (dL/dm_t), at h = h_t and
// c = slope (h_t - threshold), with the arctan surrogate derivative
// ds/dh = slope * 0.5 / (1 + (pi/2 c)^2):
//   dL/dh = g ds/dh + gm ((1 - s) + (reset - h) ds/dh)
//         = (slope/2) rcp(1 + q^2) (g + gm (reset - h)) + (s ? 0 : gm)
// with q = (pi/2) c, the hardware reciprocal (1 ulp) in place of an IEEE
// division, and fused multiply-adds (9 instructions instead of 14).  lif_bwd_scale gives (slope/2) rcp(1 + q^2) and
// lif_bwd_dh the rest, so that two carries at one step share the scale.
__device__ __forceinline__ float lif_bwd_scale(float cc, float slope) {
  const float q = 1.5707963267948966f * cc;
  return __builtin_amdgcn_rcpf(fmaf(q, q, 1.f)) * (0.5f * slope);
}
__device__ __forceinline__ float lif_bwd_dh(float g, float gm, float h, float cc, float scale,
                                            float reset) {
  return fmaf(scale, fmaf(gm, reset - h, g), cc >= 0.f ? 0.f : gm);
}

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
      const float gh = lif_bwd_dh(gb[i].get(c), gm[c], hh, cc, lif_bwd_scale(cc, P.slope),
                                  P.reset);
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

// --------------------------------------------------- staged wide I/O ----
// The kernels above issue one load per step per lane, so a wave has at most
// ~63 row reads in flight (the vector-memory counter), about 4 MB over the
// whole chip at B*C = 32768 -- too little to cover HBM latency.  The staged
// kernels below keep one channel per lane for the arithmetic but move data
// in 16-byte pieces: one wave instruction reads SPI consecutive steps of the
// wave's 64-channel row (1 KiB), the pieces of P blocks ahead wait in
// registers, and each 32-step block goes through LDS once to turn
// [step][piece] into [channel][step] order (and back for the outputs).  A
// wave then has P blocks (128-192 steps) in flight.  Requires C to be a
// multiple of 16 / sizeof(element) (a piece never straddles two rows).
// Byte offset beyond any descriptor the staged kernels build (their spans
// are below 2^31 bytes, checked on the host): accesses there read zero and
// stores are dropped.
constexpr unsigned kOutOfRange = 0x80000000u;

template <typename E>
struct Staged {
  using raw = typename E::raw;
  static constexpr int kEs = int(sizeof(raw));
  static constexpr int kLps = 4 * kEs;           // lanes (16-byte pieces) per step row
  static constexpr int kSpi = 64 / kLps;         // steps per wave instruction
  static constexpr int kInstr = kLifBlock / kSpi;  // instructions per block
  // Blocks in flight (the vector-memory counter caps a wave at 63
  // outstanding operations: per block the forward issues 2*kInstr + 1 and
  // the backward 3*kInstr + 1).
  static constexpr int kPf = kEs == 2 ? 6 : 3;
  static constexpr int kPb = kEs == 2 ? 4 : 2;

  // Per-lane byte offset of the lane's piece inside an instruction's span;
  // pieces past the last channel get an out-of-range offset, so that their
  // loads read zero and their stores are dropped by the descriptor check.
  __device__ static __forceinline__ unsigned lane_off(int lane, int C, int cg) {
    if (cg * 64 + (lane % kLps) * (16 / kEs) >= C) return kOutOfRange;
    return unsigned(lane / kLps) * unsigned(C) * unsigned(kEs) + unsigned(lane % kLps) * 16u;
  }

  // Loads the kInstr pieces of block `blk` (steps past T, and blocks outside
  // [lo, nblk), read as zero).
  __device__ static __forceinline__ void load(u32x4 (&st)[kInstr], const raw* __restrict__ p,
                                              size_t row_base, size_t row_tail, unsigned loff,
                                              int blk, int nblk, int C, int lo = 0) {
    const bool in = blk >= lo && blk < nblk;
    const int t0 = in ? blk * kLifBlock : 0;
    const uint32_t bytes = in ? span_bytes(row_tail, t0, C, kEs) : 0u;
    const rsrc_t r = make_rsrc(p + row_base + size_t(t0) * C, bytes);
    const unsigned stride = unsigned(kSpi) * unsigned(C) * unsigned(kEs);
#pragma unroll
    for (int j = 0; j < kInstr; ++j)
      st[j] = __builtin_amdgcn_raw_buffer_load_b128(r, loff, unsigned(j) * stride, 0);
  }

  __device__ static __forceinline__ void to_lds(u32x4* __restrict__ lds, const u32x4 (&st)[kInstr],
                                                int lane) {
#pragma unroll
    for (int j = 0; j < kInstr; ++j) lds[j * 64 + lane] = st[j];
  }

  __device__ static __forceinline__ float get(const u32x4* __restrict__ lds, int s, int c) {
    const raw v = reinterpret_cast<const raw*>(lds)[s * 64 + c];
    if constexpr (__is_same(E, F32)) {
      return v;
    } else if constexpr (__is_same(E, BF16)) {
      return bf16_bits_to_float(v);
    } else {
      return f16_bits_to_float(v);
    }
  }

  __device__ static __forceinline__ void put(u32x4* __restrict__ lds, int s, int c, float v) {
    store_scalar<E>(reinterpret_cast<raw*>(lds) + s * 64 + c, v);
  }

  // Writes block `blk` of an output from LDS (steps past T and pieces past
  // C fall outside the descriptor and are dropped; with `emit` false the
  // descriptor is empty and every store is dropped, so that every block
  // issues the same instructions).
  __device__ static __forceinline__ void store(raw* __restrict__ p, const u32x4* __restrict__ lds,
                                               size_t row_base, size_t row_tail, unsigned loff,
                                               int blk, int C, int lane, bool emit = true) {
    const int t0 = blk * kLifBlock;
    const rsrc_t r = make_rsrc(p + row_base + size_t(t0) * C,
                               emit ? span_bytes(row_tail, t0, C, kEs) : 0u);
    const unsigned stride = unsigned(kSpi) * unsigned(C) * unsigned(kEs);
#pragma unroll
    for (int j = 0; j < kInstr; ++j)
      __builtin_amdgcn_raw_buffer_store_b128(lds[j * 64 + lane], r, loff, unsigned(j) * stride,
                                             kAuxNT);
  }
};

// ------------------------------------------- forward split over time ----
// The membrane forgets its past at every spike (m is set to `reset`) and
// decays by `decay` otherwise, so two runs of the recurrence from different
// membranes over the same inputs become bit-identical after a few dozen
// steps and then stay identical.  The forward therefore splits the sequence
// into G.nseg segments of G.bps blocks and runs them at the same time: the
// workgroups of segment k > 0 start G.wb blocks before the segment from a
// zero membrane (warm-up: nothing written), then write the segment's
// outputs and records as the sequential kernel does.  Each publishes the
// membrane it holds at its segment's start (G.start) and after its last
// block (G.fin).  lif_fwd_fixup_kernel then walks the boundaries in order
// with the exact membrane; where the speculated one differs bit for bit, it
// reruns the segment from the exact membrane beside the speculated one,
// rewriting outputs and records that differ, until the two coincide (or to
// the segment's end).  The results are bit-identical to the sequential
// kernel for any input; the repair is short when the runs converge within
// the warm-up, as they do unless |decay| is close to 1 and no spike resets
// them.
struct LifSeg {
  int nseg;      // time segments (1: one pass over the whole sequence)
  int bps;       // checkpoint blocks per segment
  int wb;        // warm-up blocks before a segment's first block
  float* start;  // [nseg-1][B][C]: the membrane at the start of segment k+1 as speculated
  float* fin;    // [nseg-1][B][C]: the membrane after segment k (k < nseg-1) as computed
};

// This workgroup's segment: output blocks [lo, hi), processing from block
// `first` (warm-up blocks [first, lo)).  Grid: nseg x B x n_cg workgroups.
struct LifSegPos {
  int seg, b, cg, lo, hi, first;
  __device__ __forceinline__ LifSegPos(const LifSeg& G, int n_cg, int nblk) {
    const int rows = int(gridDim.x) / G.nseg;
    seg = int(blockIdx.x) / rows;
    const int rid = int(blockIdx.x) - seg * rows;
    b = rid / n_cg;
    cg = rid - b * n_cg;
    lo = seg * G.bps;
    hi = min(nblk, lo + G.bps);
    first = seg == 0 ? 0 : max(0, lo - G.wb);
  }
};

template <typename E, bool CK>
__global__ __launch_bounds__(64) void lif_fwd_staged_kernel(const typename E::raw* __restrict__ x,
                                                            typename E::raw* __restrict__ spk,
                                                            float* __restrict__ ck, int T, int C,
                                                            LifParams P, LifSeg G) {
  using S = Staged<E>;
  constexpr int PF = S::kPf;
  __shared__ u32x4 xs[S::kInstr * 64];
  __shared__ u32x4 os[S::kInstr * 64];
  const int n_cg = (C + 63) / 64;
  const int nblk = (T + kLifBlock - 1) / kLifBlock;
  const LifSegPos sp_(G, n_cg, nblk);
  const int b = sp_.b, cg = sp_.cg, lo = sp_.lo, hi = sp_.hi;
  const int lane = threadIdx.x;
  const size_t row_base = size_t(b) * T * C + size_t(cg) * 64;
  const size_t row_tail = size_t(T) * C - size_t(cg) * 64;
  const unsigned loff = S::lane_off(lane, C, cg);
  const bool lane_ok = cg * 64 + lane < C;
  // Membrane records through a descriptor over this group's records; lanes
  // past C get an out-of-range offset (their stores are dropped).
  const size_t ck_base = size_t(b) * nblk * C + size_t(cg) * 64;
  const rsrc_t rck = make_rsrc(CK ? ck + ck_base : ck, CK ? uint32_t(((size_t(nblk) - 1) * C + 64) * 4) : 0u);
  const unsigned ck_off = lane_ok ? unsigned(lane) * 4u : kOutOfRange;
  // The speculated membrane at this segment's start (segments after the first).
  const size_t bc = size_t(gridDim.x / G.nseg / n_cg) * C;
  const rsrc_t rst = make_rsrc(sp_.seg > 0 ? G.start + size_t(sp_.seg - 1) * bc + size_t(b) * C + cg * 64 : nullptr,
                               sp_.seg > 0 ? 256u : 0u);

  float m = 0.f;
  // Inputs P blocks ahead wait in registers; every block issues the same
  // loads and stores (past the segment's end, and for warm-up blocks, the
  // descriptors or offsets are empty), so the compiler's wait before a
  // block's LDS write covers only that block.
  auto block = [&](u32x4 (&st)[S::kInstr], int blk) {
    const bool emit = blk >= lo;
    S::to_lds(xs, st, lane);
    S::load(st, x, row_base, row_tail, loff, blk + PF, hi, C);
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m), rst,
                                          blk == lo && lane_ok ? unsigned(lane) * 4u : kOutOfRange,
                                          0, 0);
    if constexpr (CK)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m), rck, emit ? ck_off : kOutOfRange,
                                            unsigned(blk) * unsigned(C) * 4u, kAuxNT);
#pragma unroll
    for (int s = 0; s < kLifBlock; ++s) {
      const float h = m * P.decay + S::get(xs, s, lane);
      const float sp = P.slope * (h - P.threshold) >= 0.f ? 1.f : 0.f;
      m = h * (1.f - sp) + P.reset * sp;
      S::put(os, s, lane, sp);
    }
    S::store(spk, os, row_base, row_tail, loff, blk, C, lane, emit);
  };

  const int first = sp_.first;
  const int nb = hi - first;
  u32x4 st[PF][S::kInstr];
#pragma unroll
  for (int q = 0; q < PF; ++q) S::load(st[q], x, row_base, row_tail, loff, first + q, hi, C);
  const int nfull = nb - nb % PF;
  for (int base = 0; base < nfull; base += PF) {
#pragma unroll
    for (int q = 0; q < PF; ++q) block(st[q], first + base + q);
  }
#pragma unroll
  for (int q = 0; q < PF - 1; ++q)
    if (nfull + q < nb) block(st[q], first + nfull + q);
  if (sp_.seg < G.nseg - 1 && lane_ok)
    G.fin[size_t(sp_.seg) * bc + size_t(b) * C + cg * 64 + lane] = m;
}

// Forward with the residual add of the block (language.py:1326-1330,
// residual + spike): writes out = residual + s_t in fp32 instead of the
// spikes, from fp32 residual rows staged like x.  out may alias residual
// (each block is written after its own residual was read) when the
// sequence is not split (G.nseg = 1).
template <typename E>
__global__ __launch_bounds__(64) void lif_fwd_residual_kernel(const typename E::raw* __restrict__ x,
                                                              const float* res, float* out,
                                                              float* __restrict__ ck, int T,
                                                              int C, LifParams P, LifSeg G) {
  using S = Staged<E>;
  using SF = Staged<F32>;
  constexpr int PF = 3;  // blocks in flight (x and the wider residual pieces)
  __shared__ u32x4 xs[S::kInstr * 64];
  __shared__ u32x4 rs[SF::kInstr * 64];
  const int n_cg = (C + 63) / 64;
  const int nblk = (T + kLifBlock - 1) / kLifBlock;
  const LifSegPos sp_(G, n_cg, nblk);
  const int b = sp_.b, cg = sp_.cg, lo = sp_.lo, hi = sp_.hi;
  const int lane = threadIdx.x;
  const size_t row_base = size_t(b) * T * C + size_t(cg) * 64;
  const size_t row_tail = size_t(T) * C - size_t(cg) * 64;
  const unsigned loff = S::lane_off(lane, C, cg);
  const unsigned loffr = SF::lane_off(lane, C, cg);
  const bool lane_ok = cg * 64 + lane < C;
  const rsrc_t rck = make_rsrc(ck + size_t(b) * nblk * C + size_t(cg) * 64,
                               uint32_t(((size_t(nblk) - 1) * C + 64) * 4));
  const unsigned ck_off = lane_ok ? unsigned(lane) * 4u : kOutOfRange;
  const size_t bc = size_t(gridDim.x / G.nseg / n_cg) * C;
  const rsrc_t rst = make_rsrc(sp_.seg > 0 ? G.start + size_t(sp_.seg - 1) * bc + size_t(b) * C + cg * 64 : nullptr,
                               sp_.seg > 0 ? 256u : 0u);

  float m = 0.f;
  auto block = [&](u32x4 (&st)[S::kInstr], u32x4 (&sr)[SF::kInstr], int blk) {
    const bool emit = blk >= lo;
    S::to_lds(xs, st, lane);
    SF::to_lds(rs, sr, lane);
    S::load(st, x, row_base, row_tail, loff, blk + PF, hi, C);
    // (warm-up blocks need no residual: those read as zero, moving nothing)
    SF::load(sr, res, row_base, row_tail, loffr, blk + PF, hi, C, lo);
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m), rst,
                                          blk == lo && lane_ok ? unsigned(lane) * 4u : kOutOfRange,
                                          0, 0);
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m), rck, emit ? ck_off : kOutOfRange,
                                          unsigned(blk) * unsigned(C) * 4u, kAuxNT);
#pragma unroll
    for (int s = 0; s < kLifBlock; ++s) {
      const float h = m * P.decay + S::get(xs, s, lane);
      const float sp = P.slope * (h - P.threshold) >= 0.f ? 1.f : 0.f;
      m = h * (1.f - sp) + P.reset * sp;
      SF::put(rs, s, lane, SF::get(rs, s, lane) + sp);
    }
    SF::store(out, rs, row_base, row_tail, loffr, blk, C, lane, emit);
  };

  const int first = sp_.first;
  const int nb = hi - first;
  u32x4 st[PF][S::kInstr], sr[PF][SF::kInstr];
#pragma unroll
  for (int q = 0; q < PF; ++q) {
    S::load(st[q], x, row_base, row_tail, loff, first + q, hi, C);
    SF::load(sr[q], res, row_base, row_tail, loffr, first + q, hi, C, lo);
  }
  const int nfull = nb - nb % PF;
  for (int base = 0; base < nfull; base += PF) {
#pragma unroll
    for (int q = 0; q < PF; ++q) block(st[q], sr[q], first + base + q);
  }
#pragma unroll
  for (int q = 0; q < PF - 1; ++q)
    if (nfull + q < nb) block(st[q], sr[q], first + nfull + q);
  if (sp_.seg < G.nseg - 1 && lane_ok)
    G.fin[size_t(sp_.seg) * bc + size_t(b) * C + cg * 64 + lane] = m;
}

// Repair pass of the split forward: one wave per (batch, 64 channels), one
// lane per channel, boundaries in time order.  RES: `out` = residual +
// spike in fp32 (`res` must not alias `out`), else `spk` = spike.
constexpr int kLifMaxSeg = 16;
constexpr int kLifFixChunk = 16;  // steps loaded at once while rerunning

template <typename E, bool CK, bool RES>
__global__ __launch_bounds__(64) void lif_fwd_fixup_kernel(const typename E::raw* __restrict__ x,
                                                           const float* __restrict__ res,
                                                           typename E::raw* __restrict__ spk,
                                                           float* __restrict__ out,
                                                           float* __restrict__ ck, int B, int T,
                                                           int C, LifParams P, LifSeg G) {
  const int n_cg = (C + 63) / 64;
  const int b = int(blockIdx.x) / n_cg;
  const int cg = int(blockIdx.x) - b * n_cg;
  const int c = cg * 64 + int(threadIdx.x);
  const bool ok = c < C;
  const int nblk = (T + kLifBlock - 1) / kLifBlock;
  const size_t bc = size_t(B) * C;
  const size_t at = size_t(b) * C + size_t(ok ? c : 0);
  // Fast path: when every segment's speculated start equals the membrane
  // the previous segment ended with, each segment ran from the exact
  // membrane (by induction from segment 0, which starts at m = 0), and
  // nothing needs repair.  All boundary values are loaded at once.
  // (No short-circuit: the loads of all boundaries are issued together.)
  // The values are kept in LDS for the general path, which indexes them by a
  // run-time boundary number.
  __shared__ float lst[kLifMaxSeg - 1][64], lfi[kLifMaxSeg - 1][64];
  const int lane = int(threadIdx.x);
  // Every slot loads (past the last boundary it re-reads the last one), so
  // the loads form one straight run with a single wait.
  unsigned differ = 0;
#pragma unroll
  for (int k = 0; k < kLifMaxSeg - 1; ++k) {
    const int kk = min(k, G.nseg - 2);
    const float s0 = G.start[size_t(kk) * bc + at];
    const float f0 = G.fin[size_t(kk) * bc + at];
    differ |= __float_as_uint(s0) ^ __float_as_uint(f0);
    lst[k][lane] = s0;
    lfi[k][lane] = f0;
  }
  const bool verified = differ == 0;
  if (!__any(ok && !verified)) return;
  // General path: boundaries in order with the exact membrane.  (One wave
  // per workgroup: the LDS values above are this wave's own, in order.)
  float carry = lfi[0][lane];  // segment 0 starts from the exact membrane
  for (int k = 1; k < G.nseg; ++k) {
    const float spec = lst[k - 1][lane];
    bool todo = ok && __float_as_uint(carry) != __float_as_uint(spec);
    float m = carry, ms = spec;
    const int t_lo = k * G.bps * kLifBlock;
    const int t_hi = min(T, t_lo + G.bps * kLifBlock);
    for (int t0 = t_lo; t0 < t_hi && __any(todo); t0 += kLifFixChunk) {
      float xv[kLifFixChunk], rv[kLifFixChunk];
#pragma unroll
      for (int j = 0; j < kLifFixChunk; ++j) {
        const int t = t0 + j;
        const size_t i = (size_t(b) * T + size_t(t)) * C + size_t(c);
        xv[j] = todo && t < t_hi ? load_scalar<E>(x + i) : 0.f;
        rv[j] = RES && todo && t < t_hi ? res[i] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < kLifFixChunk; ++j) {
        const int t = t0 + j;
        // Steps past the segment leave every value unchanged (todo is off).
        const bool live = todo && t < t_hi;
        if (CK && live && t % kLifBlock == 0) ck[(size_t(b) * nblk + t / kLifBlock) * C + c] = m;
        const float h = m * P.decay + xv[j];
        const float s = P.slope * (h - P.threshold) >= 0.f ? 1.f : 0.f;
        const float mn = h * (1.f - s) + P.reset * s;
        const float hs = ms * P.decay + xv[j];
        const float ss = P.slope * (hs - P.threshold) >= 0.f ? 1.f : 0.f;
        const float msn = hs * (1.f - ss) + P.reset * ss;
        if (live && s != ss) {
          const size_t i = (size_t(b) * T + size_t(t)) * C + size_t(c);
          if constexpr (RES) {
            out[i] = rv[j] + s;
          } else {
            store_scalar<E>(spk + i, s);
          }
        }
        if (t < t_hi) {
          m = mn;
          ms = msn;
        }
        if (live && __float_as_uint(m) == __float_as_uint(ms)) todo = false;
      }
    }
    // Into segment k+1: the computed membrane after segment k is exact
    // unless this lane never coincided with the speculated run.
    if (k < G.nseg - 1) carry = todo ? m : lfi[k][lane];
  }
}

// G is the type of the incoming gradient: E, or fp32 when the spikes were
// added into an fp32 residual (lif_fwd_residual_kernel), whose gradient
// arrives in fp32.
//
// Split over time (G.nseg > 1), the mirror of the forward's: the carried
// gradient gm obeys a linear recurrence, gm <- decay (g ds/dh + gm A_t) with
// A_t = (1 - s_t) + (reset - h_t) ds/dh, whose factor |decay A_t| is at most
// about 0.51 for any membrane (the surrogate derivative is at most slope/2
// and falls off as 1/h^2), so runs from different carries coincide bit for
// bit after a few dozen steps.  Segment k (output blocks [lo, hi)) starts
// G.wb blocks after its end from gm = 0, runs those warm-up blocks without
// writing, publishes the carry it then holds (G.start[k], k < nseg-1), runs
// its own blocks last to first and publishes the carry it hands to earlier
// time (G.fin[k-1], k > 0).  lif_bwd_fixup_kernel repairs the boundaries
// from the last to the first.
template <typename E, typename G>
__global__ __launch_bounds__(64) void lif_bwd_staged_kernel(const typename E::raw* __restrict__ x,
                                                            const typename G::raw* __restrict__ gs,
                                                            const float* __restrict__ ck,
                                                            typename E::raw* __restrict__ gx,
                                                            int T, int C, LifParams P, LifSeg Sg) {
  using S = Staged<E>;
  using SG = Staged<G>;
  // Blocks in flight: one fewer when the gradient pieces are wider than x's.
  constexpr int PB = sizeof(typename G::raw) > sizeof(typename E::raw) ? S::kPb - 1 : S::kPb;
  __shared__ u32x4 xs[S::kInstr * 64];
  __shared__ u32x4 gl[SG::kInstr * 64];
  __shared__ u32x4 os[S::kInstr * 64];
  const int n_cg = (C + 63) / 64;
  const int nblk = (T + kLifBlock - 1) / kLifBlock;
  const LifSegPos sp_(Sg, n_cg, nblk);
  const int b = sp_.b, cg = sp_.cg, lo = sp_.lo, hi = sp_.hi, seg = sp_.seg;
  // Blocks processed: [lo, top], the warm-up ones (after hi - 1) first.
  const int top = min(nblk, hi + (seg == Sg.nseg - 1 ? 0 : Sg.wb)) - 1;
  const int lane = threadIdx.x;
  const size_t row_base = size_t(b) * T * C + size_t(cg) * 64;
  const size_t row_tail = size_t(T) * C - size_t(cg) * 64;
  const unsigned loff = S::lane_off(lane, C, cg);
  const unsigned loffg = SG::lane_off(lane, C, cg);
  const bool lane_ok = cg * 64 + lane < C;
  // Membrane records (lanes past C read as zero and never store).
  const rsrc_t rck = make_rsrc(ck + size_t(b) * nblk * C + size_t(cg) * 64,
                               uint32_t(((size_t(nblk) - 1) * C + 64) * 4));
  const unsigned ck_off = lane_ok ? unsigned(lane) * 4u : kOutOfRange;
  auto rec = [&](int blk) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        rck, ck_off, unsigned(max(blk, 0)) * unsigned(C) * 4u, 0));
  };
  const size_t bc = size_t(gridDim.x / Sg.nseg / n_cg) * C;
  const rsrc_t rst = make_rsrc(seg < Sg.nseg - 1 ? Sg.start + size_t(seg) * bc + size_t(b) * C + cg * 64 : nullptr,
                               seg < Sg.nseg - 1 ? 256u : 0u);

  float gm = 0.f;
  // Blocks are visited last to first; the inputs PB blocks ahead (earlier in
  // time) wait in registers.  Blocks before lo read as zero.
  auto block = [&](u32x4 (&sx)[S::kInstr], u32x4 (&sg)[SG::kInstr], float& sm, int blk) {
    const bool emit = blk < hi;
    S::to_lds(xs, sx, lane);
    SG::to_lds(gl, sg, lane);
    float m = sm;
    S::load(sx, x, row_base, row_tail, loff, blk - PB, nblk, C, lo);
    SG::load(sg, gs, row_base, row_tail, loffg, blk - PB, nblk, C, lo);
    sm = rec(blk - PB);
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(gm), rst,
                                          blk == hi - 1 && lane_ok ? unsigned(lane) * 4u : kOutOfRange,
                                          0, 0);
    // Recompute the block's pre-spike membranes h and c = slope (h - theta)
    // (the forward's operations, so the spikes are the forward's; the wave
    // is alone on its SIMD, so the 64 registers cost no occupancy).
    float h[kLifBlock], cs[kLifBlock];
#pragma unroll
    for (int s = 0; s < kLifBlock; ++s) {
      const float hh = m * P.decay + S::get(xs, s, lane);
      const float cc = P.slope * (hh - P.threshold);
      const float sp = cc >= 0.f ? 1.f : 0.f;
      m = hh * (1.f - sp) + P.reset * sp;
      h[s] = hh;
      cs[s] = cc;
    }
    // Reverse recurrence; steps past T have x = g = 0 and a zero carry.
#pragma unroll
    for (int s = kLifBlock - 1; s >= 0; --s) {
      const float cc = cs[s];
      const float gh = lif_bwd_dh(SG::get(gl, s, lane), gm, h[s], cc,
                                  lif_bwd_scale(cc, P.slope), P.reset);
      gm = P.decay * gh;
      S::put(os, s, lane, gh);
    }
    S::store(gx, os, row_base, row_tail, loff, blk, C, lane, emit);
  };

  const int nb = top - lo + 1;
  u32x4 sx[PB][S::kInstr], sg[PB][SG::kInstr];
  float sm[PB];
#pragma unroll
  for (int q = 0; q < PB; ++q) {
    const int blk = top - q;
    S::load(sx[q], x, row_base, row_tail, loff, blk, nblk, C, lo);
    SG::load(sg[q], gs, row_base, row_tail, loffg, blk, nblk, C, lo);
    sm[q] = rec(blk);
  }
  const int nfull = nb - nb % PB;
  int blk = top;
  for (int i = 0; i < nfull; i += PB) {
#pragma unroll
    for (int q = 0; q < PB; ++q) block(sx[q], sg[q], sm[q], blk - q);
    blk -= PB;
  }
#pragma unroll
  for (int q = 0; q < PB - 1; ++q)
    if (q < nb - nfull) block(sx[q], sg[q], sm[q], blk - q);
  if (seg > 0 && lane_ok) Sg.fin[size_t(seg - 1) * bc + size_t(b) * C + cg * 64 + lane] = gm;
}

// Repair pass of the split backward: one wave per (batch, 64 channels), one
// lane per channel, boundaries from the last to the first.  Boundary j lies
// between segments j and j + 1: the exact carry there is what segment j + 1
// handed on (G.fin[j], exact when segment j + 1 is), the speculated one
// G.start[j].  A rerun recomputes each block's membranes from its record and
// runs the exact and the speculated carries side by side, rewriting dL/dx
// where they differ, until the carries coincide.
template <typename E, typename G>
__global__ __launch_bounds__(64) void lif_bwd_fixup_kernel(const typename E::raw* __restrict__ x,
                                                           const typename G::raw* __restrict__ gs,
                                                           const float* __restrict__ ck,
                                                           typename E::raw* __restrict__ gx,
                                                           int B, int T, int C, LifParams P,
                                                           LifSeg Sg) {
  const int n_cg = (C + 63) / 64;
  const int b = int(blockIdx.x) / n_cg;
  const int cg = int(blockIdx.x) - b * n_cg;
  const int c = cg * 64 + int(threadIdx.x);
  const bool ok = c < C;
  const int nblk = (T + kLifBlock - 1) / kLifBlock;
  const size_t bc = size_t(B) * C;
  const size_t at = size_t(b) * C + size_t(ok ? c : 0);
  __shared__ float lst[kLifMaxSeg - 1][64], lfi[kLifMaxSeg - 1][64];
  const int lane = int(threadIdx.x);
  // Fast path: every speculated carry equals the one handed on (all loads
  // issued together; past the last boundary a slot re-reads the last one).
  unsigned differ = 0;
#pragma unroll
  for (int k = 0; k < kLifMaxSeg - 1; ++k) {
    const int kk = min(k, Sg.nseg - 2);
    const float s0 = Sg.start[size_t(kk) * bc + at];
    const float f0 = Sg.fin[size_t(kk) * bc + at];
    differ |= __float_as_uint(s0) ^ __float_as_uint(f0);
    lst[k][lane] = s0;
    lfi[k][lane] = f0;
  }
  if (!__any(ok && differ != 0)) return;
  // General path (one wave per workgroup: the LDS values are its own).
  float carry = lfi[Sg.nseg - 2][lane];  // the last segment starts from the exact zero
  for (int j = Sg.nseg - 2; j >= 0; --j) {
    const float spec = lst[j][lane];
    bool todo = ok && __float_as_uint(carry) != __float_as_uint(spec);
    float gm = carry, gms = spec;
    const int lo = j * Sg.bps;
    const int hi = min(nblk, lo + Sg.bps);
    for (int blk = hi - 1; blk >= lo && __any(todo); --blk) {
      const int t0 = blk * kLifBlock;
      float xv[kLifBlock], gv[kLifBlock];
#pragma unroll
      for (int s = 0; s < kLifBlock; ++s) {
        const int t = t0 + s;
        const size_t i = (size_t(b) * T + size_t(t)) * C + size_t(c);
        xv[s] = todo && t < T ? load_scalar<E>(x + i) : 0.f;
        gv[s] = todo && t < T ? load_scalar<G>(gs + i) : 0.f;
      }
      float m = todo ? ck[(size_t(b) * nblk + blk) * C + c] : 0.f;
      float h[kLifBlock];
#pragma unroll
      for (int s = 0; s < kLifBlock; ++s) {
        const float hh = m * P.decay + xv[s];
        const float sp = P.slope * (hh - P.threshold) >= 0.f ? 1.f : 0.f;
        m = hh * (1.f - sp) + P.reset * sp;
        h[s] = hh;
      }
#pragma unroll
      for (int s = kLifBlock - 1; s >= 0; --s) {
        const int t = t0 + s;
        const bool live = todo && t < T;
        const float cc = P.slope * (h[s] - P.threshold);
        const float scale = lif_bwd_scale(cc, P.slope);
        const float gh = lif_bwd_dh(gv[s], gm, h[s], cc, scale, P.reset);
        const float ghs = lif_bwd_dh(gv[s], gms, h[s], cc, scale, P.reset);
        if (live && __float_as_uint(gh) != __float_as_uint(ghs))
          store_scalar<E>(gx + (size_t(b) * T + size_t(t)) * C + size_t(c), gh);
        if (t < T) {
          gm = P.decay * gh;
          gms = P.decay * ghs;
        }
        if (live && __float_as_uint(gm) == __float_as_uint(gms)) todo = false;
      }
    }
    // Into boundary j - 1: the carry segment j hands on is exact unless this
    // lane never coincided with the speculated run.
    if (j > 0) carry = todo ? gm : lfi[j - 1][lane];
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

// The staged kernels need whole 16-byte pieces per row (C a multiple of
// 16 / element size) and per-batch spans below 2^31 bytes (their
// out-of-range offset); other shapes take the per-step kernels.
template <typename E>
static bool lif_staged_ok(int T, int C) {
  const size_t span = size_t(T) * size_t(C) * sizeof(typename E::raw);
  return C % (16 / int(sizeof(typename E::raw))) == 0 && span < (size_t(1) << 31);
}

// Time segments of the split passes for these sizes (1: no split): doubled
// while the waves stay below `waves` and every segment keeps at least
// `min_blocks` blocks; `env` overrides (measurement).
static int lif_nseg(int64_t B, int64_t T, int64_t C, const char* env, int64_t waves,
                    int64_t min_blocks) {
  const int64_t nblk = (T + wkv::kLifBlock - 1) / wkv::kLifBlock;
  const int64_t rows = B * ((C + 63) / 64);
  if (nblk <= 1 || rows <= 0) return 1;  // empty or one block: nothing to split
  int64_t n = 1;
  if (const char* e = getenv(env)) {
    n = std::min<int64_t>(std::max(atoi(e), 1), wkv::kLifMaxSeg);
  } else {
    while (n < wkv::kLifMaxSeg && rows * n < waves && 2 * n * min_blocks <= nblk) n *= 2;
  }
  n = std::min<int64_t>(n, nblk);
  const int64_t bps = (nblk + n - 1) / n;  // >= 1
  return int((nblk + bps - 1) / bps);
}

// The four passes and their rules, from measurements on MI355X (bf16, T =
// 1024, two-block warm-up; one pass -> split, microseconds):
//  * forward (4 B per element): ~4096 waves, segments >= 4 blocks.  B=64
//    C=512: 56.6 -> 40.1 / 33.5 / 31.8 at 2 / 4 / 8 segments.
//  * backward (6 B): ~2048 waves, segments >= 8 blocks (its blocks cost
//    more, so the warm-up weighs more on short segments).  B=64 C=512: 90.1
//    -> 54.4 / 65.2 / 78.0 at 4 / 8 / 16 segments.
//  * forward with the residual add (10 B): one pass from 384 rows of 64
//    channels on (the one pass already moves ~5.8 TB/s: B=64 C=512 57.7,
//    split 65-67), else ~2048 waves (B=16 C=768: 53.1 -> 26.9 at 8).
//  * backward with the fp32 residual gradient (8 B): ~1024 waves, >= 8
//    blocks (B=64 C=512: 79.0 -> 56.2 at 2, 61.8 at 4; B=16 C=768: 74.7 ->
//    34.4 at 4).
enum class LifPass { kForward, kBackward, kResidualForward, kResidualBackward };

static int lif_nseg(int64_t B, int64_t T, int64_t C, LifPass pass) {
  switch (pass) {
    case LifPass::kForward: return lif_nseg(B, T, C, "WKV_LIF_SEGS", 4096, 4);
    case LifPass::kBackward: return lif_nseg(B, T, C, "WKV_LIF_BWD_SEGS", 2048, 8);
    case LifPass::kResidualForward:
      if (B * ((C + 63) / 64) >= 384 && getenv("WKV_LIF_SEGS") == nullptr) return 1;
      return lif_nseg(B, T, C, "WKV_LIF_SEGS", 2048, 4);
    case LifPass::kResidualBackward: return lif_nseg(B, T, C, "WKV_LIF_BWD_SEGS", 1024, 8);
  }
  return 1;
}

// Warm-up blocks of a speculated segment (`env` overrides).  Two (64
// steps): with one, enough channels still differ at the boundary that the
// forward's repair costs more than the second block (B=64 T=1024 C=512, 4
// segments: repair 10.8 us after one block, 4.6 us after two or three).
static int lif_warmup(const char* env) {
  if (const char* e = getenv(env)) return std::min(std::max(atoi(e), 0), 8);
  return 2;
}

static size_t lif_seg_bytes(int64_t B, int64_t T, int64_t C, LifPass pass) {
  const int n = lif_nseg(B, T, C, pass);
  if (n <= 1) return 0;
  return size_t(2) * size_t(n - 1) * size_t(B) * size_t(C) * sizeof(float);
}

// One workspace query per direction serves both variants (the larger need).
size_t lif_fwd_workspace_bytes_impl(int64_t B, int64_t T, int64_t C) {
  return std::max(lif_seg_bytes(B, T, C, LifPass::kForward),
                  lif_seg_bytes(B, T, C, LifPass::kResidualForward));
}

size_t lif_bwd_workspace_bytes_impl(int64_t B, int64_t T, int64_t C) {
  return std::max(lif_seg_bytes(B, T, C, LifPass::kBackward),
                  lif_seg_bytes(B, T, C, LifPass::kResidualBackward));
}

// The split's layout for this pass and these sizes when `ws` holds enough
// bytes, else one segment (the one-pass kernel).
static wkv::LifSeg lif_seg(void* ws, size_t ws_bytes, int B, int T, int C, LifPass pass) {
  const int nblk = (T + wkv::kLifBlock - 1) / wkv::kLifBlock;
  wkv::LifSeg G{1, nblk, 0, nullptr, nullptr};
  const size_t need = lif_seg_bytes(B, T, C, pass);
  if (need == 0 || ws == nullptr || ws_bytes < need) return G;
  const int n = lif_nseg(B, T, C, pass);
  const bool backward = pass == LifPass::kBackward || pass == LifPass::kResidualBackward;
  G.nseg = n;
  G.bps = (nblk + n - 1) / n;
  G.wb = lif_warmup(backward ? "WKV_LIF_BWD_WARMUP" : "WKV_LIF_WARMUP");
  G.start = static_cast<float*>(ws);
  G.fin = G.start + size_t(n - 1) * size_t(B) * size_t(C);
  return G;
}

template <typename E>
static int lif_fwd_dispatch(const void* x, void* spk, float* ck, void* ws, size_t ws_bytes, int B,
                            int T, int C, const wkv::LifParams& P, hipStream_t stream) {
  using raw = typename E::raw;
  if (lif_staged_ok<E>(T, C)) {
    const wkv::LifSeg G = lif_seg(ws, ws_bytes, B, T, C, LifPass::kForward);
    const unsigned rows = unsigned(B) * unsigned((C + 63) / 64);
    const dim3 grid(rows * unsigned(G.nseg));
    const bool last = G.nseg == 1;
    if (ck != nullptr) {
      launch(wkv::lif_fwd_staged_kernel<E, true>, grid, dim3(64), stream, last,
             static_cast<const raw*>(x), static_cast<raw*>(spk), ck, T, C, P, G);
    } else {
      launch(wkv::lif_fwd_staged_kernel<E, false>, grid, dim3(64), stream, last,
             static_cast<const raw*>(x), static_cast<raw*>(spk), ck, T, C, P, G);
    }
    if (const int rc = check_launch("lif_fwd_staged_kernel")) return rc;
    if (G.nseg > 1) {
      if (ck != nullptr) {
        launch(wkv::lif_fwd_fixup_kernel<E, true, false>, dim3(rows), dim3(64), stream, true,
               static_cast<const raw*>(x), static_cast<const float*>(nullptr),
               static_cast<raw*>(spk), static_cast<float*>(nullptr), ck, B, T, C, P, G);
      } else {
        launch(wkv::lif_fwd_fixup_kernel<E, false, false>, dim3(rows), dim3(64), stream, true,
               static_cast<const raw*>(x), static_cast<const float*>(nullptr),
               static_cast<raw*>(spk), static_cast<float*>(nullptr), ck, B, T, C, P, G);
      }
      return check_launch("lif_fwd_fixup_kernel");
    }
    return 0;
  }
  return lif_vec(B, C, int(sizeof(typename E::raw))) == 2 ? lif_fwd_launch<E, 2>(x, spk, ck, B, T, C, P, stream)
                            : lif_fwd_launch<E, 1>(x, spk, ck, B, T, C, P, stream);
}

// Split backward: the segmented kernel, then the repair pass.
template <typename E, typename G>
static int lif_bwd_staged(const void* x, const void* gs, const float* ck, void* gx, void* ws,
                          size_t ws_bytes, int B, int T, int C, const wkv::LifParams& P,
                          LifPass pass, hipStream_t stream) {
  using raw = typename E::raw;
  using graw = typename G::raw;
  const wkv::LifSeg S = lif_seg(ws, ws_bytes, B, T, C, pass);
  const unsigned rows = unsigned(B) * unsigned((C + 63) / 64);
  launch(wkv::lif_bwd_staged_kernel<E, G>, dim3(rows * unsigned(S.nseg)), dim3(64), stream,
         S.nseg == 1, static_cast<const raw*>(x), static_cast<const graw*>(gs), ck,
         static_cast<raw*>(gx), T, C, P, S);
  if (const int rc = check_launch("lif_bwd_staged_kernel")) return rc;
  if (S.nseg > 1) {
    launch(wkv::lif_bwd_fixup_kernel<E, G>, dim3(rows), dim3(64), stream, true,
           static_cast<const raw*>(x), static_cast<const graw*>(gs), ck, static_cast<raw*>(gx), B,
           T, C, P, S);
    return check_launch("lif_bwd_fixup_kernel");
  }
  return 0;
}

template <typename E>
static int lif_bwd_dispatch(const void* x, const void* gs, const float* ck, void* gx, void* ws,
                            size_t ws_bytes, int B, int T, int C, const wkv::LifParams& P,
                            hipStream_t stream) {
  if (lif_staged_ok<E>(T, C))
    return lif_bwd_staged<E, E>(x, gs, ck, gx, ws, ws_bytes, B, T, C, P, LifPass::kBackward,
                                stream);
  return lif_vec(B, C, int(sizeof(typename E::raw))) == 2 ? lif_bwd_launch<E, 2>(x, gs, ck, gx, B, T, C, P, stream)
                            : lif_bwd_launch<E, 1>(x, gs, ck, gx, B, T, C, P, stream);
}

// Residual variants: staged kernels only (the caller checks lif_residual_ok).
// The split needs `out` and `res` disjoint (the repair reads the residual).
template <typename E>
static int lif_residual_fwd(const void* x, const float* res, float* out, float* ck, void* ws,
                            size_t ws_bytes, int B, int T, int C, const wkv::LifParams& P,
                            hipStream_t stream) {
  using raw = typename E::raw;
  const size_t n = size_t(B) * size_t(T) * size_t(C);
  const bool disjoint = out + n <= res || res + n <= out;
  const wkv::LifSeg G =
      lif_seg(disjoint ? ws : nullptr, ws_bytes, B, T, C, LifPass::kResidualForward);
  const unsigned rows = unsigned(B) * unsigned((C + 63) / 64);
  launch(wkv::lif_fwd_residual_kernel<E>, dim3(rows * unsigned(G.nseg)), dim3(64), stream,
         G.nseg == 1, static_cast<const raw*>(x), res, out, ck, T, C, P, G);
  if (const int rc = check_launch("lif_fwd_residual_kernel")) return rc;
  if (G.nseg > 1) {
    launch(wkv::lif_fwd_fixup_kernel<E, true, true>, dim3(rows), dim3(64), stream, true,
           static_cast<const raw*>(x), res, static_cast<raw*>(nullptr), out, ck, B, T, C, P, G);
    return check_launch("lif_fwd_fixup_kernel");
  }
  return 0;
}

template <typename E>
static int lif_residual_bwd(const void* x, const float* g, const float* ck, void* gx, void* ws,
                            size_t ws_bytes, int B, int T, int C, const wkv::LifParams& P,
                            hipStream_t stream) {
  return lif_bwd_staged<E, wkv::F32>(x, g, ck, gx, ws, ws_bytes, B, T, C, P,
                                     LifPass::kResidualBackward, stream);
}

bool lif_residual_ok(int64_t T, int64_t C, int dtype) {
  const int es = dtype == 0 ? 4 : 2;
  // x pieces and the fp32 residual pieces both whole, both spans < 2^31.
  (void)es;
  return C % 8 == 0 && size_t(T) * size_t(C) * 4 < (size_t(1) << 31);
}

int lif_residual_forward_impl(const void* x, const float* res, float* out, float* ck, void* ws,
                              size_t ws_bytes, int B, int T, int C, float decay, float threshold,
                              float reset, float slope, int dtype, hipStream_t stream) {
  const wkv::LifParams P{decay, threshold, reset, slope};
  switch (dtype) {
    case 0: return lif_residual_fwd<wkv::F32>(x, res, out, ck, ws, ws_bytes, B, T, C, P, stream);
    case 1: return lif_residual_fwd<wkv::BF16>(x, res, out, ck, ws, ws_bytes, B, T, C, P, stream);
    case 2: return lif_residual_fwd<wkv::F16>(x, res, out, ck, ws, ws_bytes, B, T, C, P, stream);
    default: return fail(1, "lif_residual_forward: unknown dtype");
  }
}

int lif_residual_backward_impl(const void* x, const float* g, const float* ck, void* gx,
                               void* ws, size_t ws_bytes, int B, int T, int C, float decay,
                               float threshold, float reset, float slope, int dtype,
                               hipStream_t stream) {
  const wkv::LifParams P{decay, threshold, reset, slope};
  switch (dtype) {
    case 0: return lif_residual_bwd<wkv::F32>(x, g, ck, gx, ws, ws_bytes, B, T, C, P, stream);
    case 1: return lif_residual_bwd<wkv::BF16>(x, g, ck, gx, ws, ws_bytes, B, T, C, P, stream);
    case 2: return lif_residual_bwd<wkv::F16>(x, g, ck, gx, ws, ws_bytes, B, T, C, P, stream);
    default: return fail(1, "lif_residual_backward: unknown dtype");
  }
}

int lif_forward_impl(const void* x, void* spk, float* ck, void* ws, size_t ws_bytes, int B, int T,
                     int C, float decay, float threshold, float reset, float slope, int dtype,
                     hipStream_t stream) {
  const wkv::LifParams P{decay, threshold, reset, slope};
  switch (dtype) {
    case 0: return lif_fwd_dispatch<wkv::F32>(x, spk, ck, ws, ws_bytes, B, T, C, P, stream);
    case 1: return lif_fwd_dispatch<wkv::BF16>(x, spk, ck, ws, ws_bytes, B, T, C, P, stream);
    case 2: return lif_fwd_dispatch<wkv::F16>(x, spk, ck, ws, ws_bytes, B, T, C, P, stream);
    default: return fail(1, "lif_forward: unknown dtype");
  }
}

int lif_backward_impl(const void* x, const void* gs, const float* ck, void* gx, void* ws,
                      size_t ws_bytes, int B, int T, int C, float decay, float threshold,
                      float reset, float slope, int dtype, hipStream_t stream) {
  const wkv::LifParams P{decay, threshold, reset, slope};
  switch (dtype) {
    case 0: return lif_bwd_dispatch<wkv::F32>(x, gs, ck, gx, ws, ws_bytes, B, T, C, P, stream);
    case 1: return lif_bwd_dispatch<wkv::BF16>(x, gs, ck, gx, ws, ws_bytes, B, T, C, P, stream);
    case 2: return lif_bwd_dispatch<wkv::F16>(x, gs, ck, gx, ws, ws_bytes, B, T, C, P, stream);
    default: return fail(1, "lif_backward: unknown dtype");
  }
}

}  // namespace wkv_host
