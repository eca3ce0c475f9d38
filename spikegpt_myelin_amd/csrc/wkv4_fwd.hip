// RWKV-4 / SpikeGPT WKV forward for gfx950.
//
// Math (the reference's, src/spikegpt/wkv_triton.py:34-58 and
// src/spikegpt/language.py:399-449), per (batch b, channel c) lane with
// w = -exp(time_decay), u = time_first:
//   y_t = (A_t + e^{u+k_t} v_t) / (B_t + e^{u+k_t}),
//   A_{t+1} = e^w A_t + e^{k_t} v_t,  B_{t+1} = e^w B_t + e^{k_t}.
//
// Work decomposition (MI355X-first, not the reference's one-program-per-
// (b, 64 channels) serial scan):
//   * one workgroup of W wave64s owns a "row" = (b, 64*VEC consecutive
//     channels) for the whole sequence; lane l of every wave handles channels
//     [l*VEC, l*VEC+VEC) of the row, so each load/store instruction of a wave
//     touches 64*VEC contiguous elements of one [B,T,C] row;
//   * time is cut into chunks of L steps; wave w handles chunk s*W + w of
//     segment s, holding the chunk's k/v in registers (loaded one segment
//     ahead, double-buffered);
//   * exponents are kept in one fixed base-2 frame: the state is
//     (A, B) = (p, q) directly and e_i = 2^{k_i log2e} needs no running max,
//     which is exact arithmetic while |k log2e| <= 60 and |u log2e| <= 16 (see
//     the range guard below); joining chunks is linear: p <- p*e^{Lw} + p_j.
//     The per-step work is one exp2 and one reciprocal per element, with no
//     per-step max or select;
//   * phase 1: every wave reduces its chunk to (p_j, q_j) from a zero state
//     and publishes it in LDS; after the segment's one barrier each wave folds
//     the segment carry and its predecessors' summaries (Horner in LDS) into
//     its own carry-in; phase 2: every wave re-runs its chunk from registers
//     with that carry and writes y.  k and v are read from HBM exactly once
//     and y written once.
//
// Checkpoints: with a checkpoint buffer the kernel also stores, at the start
// of every block of 64 steps, the state in running-max form (o, p, q) with
// (A, B) = 2^o (p, q) ([3][B][ceil(T/64)][C] fp32).  Rows computed here have
// o = 0 everywhere; rows recomputed by the exact serial path start from
// o = -1e38 in block 0, which tells the backward kernel to take its own exact
// path for them.  The backward recomputes the forward from these records
// instead of re-reading the whole sequence; without y (y == nullptr) the
// kernel writes records only.
//
// Range guard: every element of a row must satisfy |k log2e| <= 60, and the
// row's |u log2e| <= 16.  A wave that finds a key out of range sets a sticky
// LDS flag before the segment's barrier; every wave reads it after the
// barrier, so the decision is workgroup-uniform, and a rejected row is
// recomputed by the reference's running-max recurrence, one channel per
// thread.  Inputs whose keys stay inside +-30 (the benchmark's clamp) never
// take that path.
#include <algorithm>

#include "wkv_common.h"
#include "wkv_impl.h"

namespace wkv {

template <typename E, int VEC, int L, int W, bool WY, bool GATE = false>
struct Fwd {
  using raw = typename E::raw;
  using PackT = Pack<E, VEC>;
  static constexpr int CPW = 64 * VEC;       // channels per row
  static constexpr int SEG = W * L;          // steps per segment
  static constexpr int CPB = kCkptBlock / L;  // chunks per checkpoint block
  static_assert(kCkptBlock % L == 0 && SEG % kCkptBlock == 0, "segment/block layout");

  // [VEC][W][64]: lane index fastest, so every LDS access of a wave is one
  // conflict-free row of 64 dwords.  The chunk summaries are double-buffered
  // by segment parity: a wave may publish segment s+1's summary while a
  // slower wave still folds segment s's.
  struct Smem {
    float p[2][VEC][W][64];
    float q[2][VEC][W][64];
    float carry[2][2][VEC][64];  // (p, q) of the segment carry, by segment parity
    int bad;                     // sticky: some key of the row is out of range
  };

  // Loads the chunk of L steps starting at t0 through buffer descriptors
  // based at the chunk (row_base is wave-uniform, lane_boff the lane's byte
  // offset).  Steps at or past T read as zero.
  // WITH_R: the receptance chunk rb as well (GATE).
  template <bool WITH_R = GATE>
  __device__ static __forceinline__ void load_chunk(const raw* __restrict__ k,
                                                    const raw* __restrict__ v,
                                                    const raw* __restrict__ r, size_t row_base,
                                                    size_t row_tail, unsigned lane_boff, int t0,
                                                    int C, PackT (&kb)[L], PackT (&vb)[L],
                                                    PackT (&rb)[L]) {
    const uint32_t bytes = span_bytes(row_tail, t0, C, int(sizeof(raw)));
    const size_t base = row_base + size_t(t0) * C;
    const rsrc_t rk = make_rsrc(k + base, bytes);
    const rsrc_t rv = make_rsrc(v + base, bytes);
    const unsigned stride = unsigned(C) * unsigned(sizeof(raw));
#pragma unroll
    for (int i = 0; i < L; ++i) {
      load_buf(kb[i], rk, lane_boff, unsigned(i) * stride);
      load_buf(vb[i], rv, lane_boff, unsigned(i) * stride);
    }
    if constexpr (WITH_R) load_r(r, row_base, row_tail, lane_boff, t0, C, rb);
  }

  // The receptance chunk alone (GATE).
  __device__ static __forceinline__ void load_r(const raw* __restrict__ r, size_t row_base,
                                                size_t row_tail, unsigned lane_boff, int t0,
                                                int C, PackT (&rb)[L]) {
    const rsrc_t rr = make_rsrc(r + row_base + size_t(t0) * C,
                                span_bytes(row_tail, t0, C, int(sizeof(raw))));
    const unsigned stride = unsigned(C) * unsigned(sizeof(raw));
#pragma unroll
    for (int i = 0; i < L; ++i) load_buf(rb[i], rr, lane_boff, unsigned(i) * stride);
  }

  // Phase 1 of a chunk (L steps from t0): e = 2^{k log2e} of every step
  // (zero past T) and the chunk's summary (ps, qs) from a zero state.
  // Returns whether a key of the chunk is outside the fixed frame's range.
  template <bool FULL>
  __device__ static __forceinline__ bool summarize(int t0, int T, const PackT (&kb)[L],
                                                   const PackT (&vb)[L], const float (&D)[VEC],
                                                   float (&s)[L][VEC], float (&ps)[VEC],
                                                   float (&qs)[VEC]) {
    float mk[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) { ps[c] = 0.f; qs[c] = 0.f; mk[c] = 0.f; }
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const bool valid = FULL || (t0 + i) < T;
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const float kk = kb[i].get(c);
        mk[c] = fmaxf(mk[c], fabsf(kk));
        float e = fast_exp2(kk * kLog2e);
        if (!FULL) e = valid ? e : 0.f;
        s[i][c] = e;
        ps[c] = fmaf(ps[c], D[c], e * vb[i].get(c));
        qs[c] = fmaf(qs[c], D[c], e);
      }
    }
    bool bad = false;
#pragma unroll
    for (int c = 0; c < VEC; ++c) bad |= mk[c] * kLog2e > kMaxK;
    return bad;
  }

  // Phase 2 of a chunk from its carry-in (pin, qin): the checkpoint record
  // when the chunk starts a 64-step block, then the outputs.
  __device__ static __forceinline__ void emit(
      int t0, int T, int C, int wave, bool active, size_t row_base, size_t row_tail,
      unsigned lane_boff, raw* __restrict__ y, float* __restrict__ ck, size_t ck_row,
      unsigned ck_boff, size_t ck_field, const float (&s)[L][VEC], const PackT (&vb)[L],
      const PackT (&rb)[L], const float (&D)[VEC], const float (&U)[VEC], float (&pin)[VEC],
      float (&qin)[VEC]) {
    if (ck != nullptr && wave % CPB == 0 && active && t0 < T) {
      const float zero[VEC] = {};
      float* rec = ck + ck_row + size_t(t0 / kCkptBlock) * C;
      store_vec<F32, VEC>(byte_offset(rec + 0 * ck_field, ck_boff), zero);
      store_vec<F32, VEC>(byte_offset(rec + 1 * ck_field, ck_boff), pin);
      store_vec<F32, VEC>(byte_offset(rec + 2 * ck_field, ck_boff), qin);
    }
    if constexpr (WY) {
      // GATE: each step's outputs are stored as soon as they are computed
      // (the gate's arithmetic leaves no room to hold the chunk's L packs);
      // otherwise the chunk's stores go out together after the last step.
      OutPack<E, VEC> yp[GATE ? 1 : L];
      const unsigned stride = unsigned(C) * unsigned(sizeof(raw));
      // (unused, hence dropped, without GATE)
      const rsrc_t ry_gate = make_rsrc(y + row_base + size_t(t0) * C,
                                       span_bytes(row_tail, t0, C, int(sizeof(raw))));
#pragma unroll
      for (int i = 0; i < L; ++i) {
        float yv[VEC];
#pragma unroll
        for (int c = 0; c < VEC; ++c) {
          const float e = s[i][c];
          const float vv = vb[i].get(c);
          const float e1 = e * U[c];
          yv[c] = fmaf(e1, vv, pin[c]) * fast_rcp(qin[c] + e1);
          // fma(e, v, p*D) rather than fma(p, D, e*v): keeps phase 1's e*v
          // products from being carried live into this phase.
          pin[c] = fmaf(e, vv, pin[c] * D[c]);
          qin[c] = fmaf(qin[c], D[c], e);
          // GATE: sigmoid(r) * y with the separate kernels' roundings (y
          // and sigmoid(r) each rounded to the element type, then the
          // product), language.py:1035.
          if constexpr (GATE)
            yv[c] = round_to<E>(gate_sigmoid<E>(rb[i].get(c))) * round_to<E>(yv[c]);
        }
        if constexpr (GATE) {
          yp[0].set(yv);
          if (active) store_buf(yp[0], ry_gate, lane_boff, unsigned(i) * stride);
        } else {
          yp[i].set(yv);
        }
      }
      if (!GATE && active) {
        // Steps past T fall outside the descriptor and are dropped.
        const rsrc_t ry = make_rsrc(y + row_base + size_t(t0) * C,
                                    span_bytes(row_tail, t0, C, int(sizeof(raw))));
#pragma unroll
        for (int i = 0; i < L; ++i) store_buf(yp[i], ry, lane_boff, unsigned(i) * stride);
      }
    }
  }

  // One segment.  FULL: every step of the segment is inside the sequence.
  // Returns true when the range guard rejects the row (workgroup-uniform).
  template <bool FULL>
  __device__ static __forceinline__ bool segment(
      Smem& sm, int seg, int T, int C, int wave, int lane, bool active, size_t row_base,
      size_t row_tail, unsigned lane_boff, raw* __restrict__ y, float* __restrict__ ck, size_t ck_row,
      unsigned ck_boff, size_t ck_field, const PackT (&kb)[L], const PackT (&vb)[L],
      const PackT (&rb)[L], const float (&D)[VEC], const float (&DL)[VEC],
      const float (&U)[VEC]) {
    const int t0 = seg * SEG + wave * L;
    const int par = seg & 1;
    float s[L][VEC];
    float ps[VEC], qs[VEC];
    const bool bad = summarize<FULL>(t0, T, kb, vb, D, s, ps, qs);
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      sm.p[par][c][wave][lane] = ps[c];
      sm.q[par][c][wave][lane] = qs[c];
    }
    if (__any(active && bad) && lane == 0) sm.bad = 1;
    __syncthreads();
    if (sm.bad) return true;

    // Carry-in of this chunk: segment carry, then the earlier chunks.
    float pin[VEC], qin[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      pin[c] = seg > 0 ? sm.carry[par ^ 1][0][c][lane] : 0.f;
      qin[c] = seg > 0 ? sm.carry[par ^ 1][1][c][lane] : 0.f;
    }
    for (int w = 0; w < wave; ++w) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        pin[c] = fmaf(pin[c], DL[c], sm.p[par][c][w][lane]);
        qin[c] = fmaf(qin[c], DL[c], sm.q[par][c][w][lane]);
      }
    }
    if (wave == W - 1) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        sm.carry[par][0][c][lane] = fmaf(pin[c], DL[c], ps[c]);
        sm.carry[par][1][c][lane] = fmaf(qin[c], DL[c], qs[c]);
      }
    }
    emit(t0, T, C, wave, active, row_base, row_tail, lane_boff, y, ck, ck_row, ck_boff, ck_field,
         s, vb, rb, D, U, pin, qin);
    return false;
  }
};

// Reference running-max recurrence for one channel over the whole sequence
// (wkv_triton.py:41-58 in base-2 units), writing y (if any) and the
// checkpoint records (if any).  Used for rows the range guard rejects.
template <typename E>
__device__ void wkv4_fwd_channel_serial(const typename E::raw* __restrict__ k,
                                        const typename E::raw* __restrict__ v,
                                        const typename E::raw* __restrict__ r,
                                        typename E::raw* __restrict__ y, float w2, float u2, int T,
                                        int C, size_t base, float* __restrict__ ck,
                                        size_t ck_lane, size_t ck_field) {
  float o = kNegHuge, p = 0.f, q = 0.f;
  for (int t = 0; t < T; ++t) {
    const size_t idx = base + size_t(t) * C;
    if (ck != nullptr && t % kCkptBlock == 0) {
      float* rec = ck + ck_lane + size_t(t / kCkptBlock) * C;
      rec[0 * ck_field] = o;
      rec[1 * ck_field] = p;
      rec[2 * ck_field] = q;
    }
    const float kk = load_scalar<E>(k + idx) * kLog2e;
    const float vv = load_scalar<E>(v + idx);
    if (y != nullptr) {
      const float uk = u2 + kk;
      const float no = fmaxf(o, uk);
      const float a = fast_exp2(o - no);
      const float bb = fast_exp2(uk - no);
      float yv = (a * p + bb * vv) / (a * q + bb);
      if (r != nullptr)
        yv = round_to<E>(gate_sigmoid<E>(load_scalar<E>(r + idx))) * round_to<E>(yv);
      store_scalar<E>(y + idx, yv);
    }
    const float wo = w2 + o;
    const float no = fmaxf(wo, kk);
    const float a = fast_exp2(wo - no);
    const float bb = fast_exp2(kk - no);
    p = a * p + bb * vv;
    q = a * q + bb;
    o = no;
  }
}

// decay: time_decay (decay_is_w == 0, w = -exp(decay)) or w itself.
// GATE: y = sigmoid(r) * wkv (r [B,T,C] in the element type), the time
// mix's receptance gate folded in.
template <typename E, int VEC, int L, int W, bool WY, bool GATE>
__global__ __launch_bounds__(W * 64) void wkv4_fwd_kernel(
    const typename E::raw* __restrict__ k, const typename E::raw* __restrict__ v,
    const float* __restrict__ decay, int decay_is_w, const float* __restrict__ time_first,
    const typename E::raw* __restrict__ r, typename E::raw* __restrict__ y,
    float* __restrict__ ck, int T, int C) {
  using F = Fwd<E, VEC, L, W, WY, GATE>;
  using PackT = typename F::PackT;
  __shared__ typename F::Smem sm;

  const int n_cg = (C + F::CPW - 1) / F::CPW;
  const int b = blockIdx.x / n_cg;
  const int cg = blockIdx.x - b * n_cg;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c0 = cg * F::CPW + lane * VEC;
  const bool active = c0 < C;
  const size_t row_base = size_t(b) * T * C + size_t(cg) * F::CPW;
  const size_t row_tail = size_t(T) * C - size_t(cg) * F::CPW;
  // Lanes past the last channel read channel 0 of the row (never stored).
  const unsigned lane_boff = active ? unsigned(lane * VEC * sizeof(typename E::raw)) : 0u;
  const int nblk = (T + kCkptBlock - 1) / kCkptBlock;
  const size_t ck_field = size_t(gridDim.x / n_cg) * nblk * C;  // B * nblk * C
  const size_t ck_row = size_t(b) * nblk * C + size_t(cg) * F::CPW;
  const unsigned ck_boff = active ? unsigned(lane * VEC * sizeof(float)) : 0u;

  float D[VEC], DL[VEC], U[VEC];
  bool u_ok = true;
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    const float dv = active ? decay[c0 + c] : 0.f;
    const float tf = active ? time_first[c0 + c] : 0.f;
    const float w2 = (decay_is_w ? dv : -expf(dv)) * kLog2e;
    const float u2 = tf * kLog2e;
    D[c] = fast_exp2(w2);
    DL[c] = fast_exp2(w2 * float(L));
    U[c] = fast_exp2(u2);
    u_ok &= fabsf(u2) <= kMaxU;
  }
  if (threadIdx.x == 0) sm.bad = 0;
  // |u log2e| is part of the guard: a row with any channel out of range goes
  // straight to the exact path.
  bool bad = __syncthreads_or(!u_ok) != 0;

  const int nseg = (T + F::SEG - 1) / F::SEG;
  const int nfull = T / F::SEG;
  PackT kA[L], vA[L], kB[L], vB[L];
  // GATE: the receptance of the segment being computed, loaded when that
  // segment starts (it is read only by the segment's second phase) and
  // before the next segment's prefetch, so that waiting for it never waits
  // for the prefetch; one buffer instead of two keeps the 16-wave tile
  // within its 128 registers.
  PackT rc[L];
  // The next segment is prefetched on every path (past the end the
  // descriptor is empty and the loads return zeros without touching memory):
  // with the same loads issued on every path, the compiler's wait before a
  // segment's arithmetic only covers the loads it consumes, not the prefetch
  // issued just before it.
  if (!bad)
    F::template load_chunk<false>(k, v, r, row_base, row_tail, lane_boff, wave * L, C, kA, vA, rc);
  for (int seg = 0; seg < nseg && !bad; seg += 2) {
    if constexpr (GATE)
      F::load_r(r, row_base, row_tail, lane_boff, seg * F::SEG + wave * L, C, rc);
    F::template load_chunk<false>(k, v, r, row_base, row_tail, lane_boff,
                                  (seg + 1) * F::SEG + wave * L, C, kB, vB, rc);
    bad = seg < nfull
              ? F::template segment<true>(sm, seg, T, C, wave, lane, active, row_base, row_tail, lane_boff, y,
                                          ck, ck_row, ck_boff, ck_field, kA, vA, rc, D, DL, U)
              : F::template segment<false>(sm, seg, T, C, wave, lane, active, row_base, row_tail, lane_boff,
                                           y, ck, ck_row, ck_boff, ck_field, kA, vA, rc, D, DL, U);
    if (bad || seg + 1 >= nseg) break;
    if constexpr (GATE)
      F::load_r(r, row_base, row_tail, lane_boff, (seg + 1) * F::SEG + wave * L, C, rc);
    F::template load_chunk<false>(k, v, r, row_base, row_tail, lane_boff,
                                  (seg + 2) * F::SEG + wave * L, C, kA, vA, rc);
    bad = seg + 1 < nfull
              ? F::template segment<true>(sm, seg + 1, T, C, wave, lane, active, row_base,
                                          row_tail, lane_boff, y, ck, ck_row, ck_boff, ck_field, kB, vB, rc, D,
                                          DL, U)
              : F::template segment<false>(sm, seg + 1, T, C, wave, lane, active, row_base,
                                           row_tail, lane_boff, y, ck, ck_row, ck_boff, ck_field, kB, vB, rc, D,
                                           DL, U);
  }
  if (bad) {
    // Workgroup-uniform: recompute the row with the running-max recurrence.
    __syncthreads();
    for (int ch = threadIdx.x; ch < F::CPW; ch += blockDim.x) {
      const int c = cg * F::CPW + ch;
      if (c >= C) continue;
      const float w2 = (decay_is_w ? decay[c] : -expf(decay[c])) * kLog2e;
      const float u2 = time_first[c] * kLog2e;
      wkv4_fwd_channel_serial<E>(k, v, GATE ? r : nullptr, WY ? y : nullptr, w2, u2, T, C,
                                 size_t(b) * T * C + c, ck,
                                 size_t(b) * nblk * C + c, ck_field);
    }
  }
}

// ----------------------------------------------------- split over time ----
// For few rows (B * ceil(C / 64) below the CU count) the one-row kernel
// leaves CUs idle.  Here a workgroup owns one segment (W chunks of L steps)
// of one row: blockIdx = segment * rows + row, so every row's segment s is
// dispatched before segment s+1.  The workgroup reduces its segment to its
// aggregate -- the state change over the segment from a zero state, the
// Horner fold of its chunk summaries -- and publishes it.  Its carry-in is
// the state at the segment's start,
//   carry_s = sum_{j<s} e^{(s-1-j) SEG w} agg_j = e^{K SEG w} incl_{s-K-1}
//             + sum_{j=s-K}^{s-1} e^{(s-1-j) SEG w} agg_j,
// taken from the K = kLbWindow previous segments' aggregates and the
// inclusive state incl_{s-K-1} (the state at the end of that segment), the
// same words on every run (lb_window_carry), so the result is deterministic.
// It then publishes incl_s = e^{SEG w} carry_s + agg_s and runs its segment
// from registers as the one-row kernel does.  k, v are read once, y written
// once; the carries are 16 bytes per channel and segment.  Waits only go to
// lower block indices, and every wait is bounded (kLbMaxPolls): a workgroup
// that gives up marks its row, and the fix-up kernel that follows recomputes
// marked rows exactly, as it does rows whose keys leave the fixed frame's
// range.
//
// Look-back words: lb[2][nseg][rows][64*VEC] (aggregates, then inclusive
// states), each word the pair (p, q) of one channel; status[rows] (kRowOk, or
// kRowRedo for a row the fix-up kernel recomputes).
template <typename E, int VEC, int L, int W, bool WY, bool GATE>
__global__ __launch_bounds__(W * 64) void wkv4_fwd_split_kernel(
    const typename E::raw* __restrict__ k, const typename E::raw* __restrict__ v,
    const float* __restrict__ decay, int decay_is_w, const float* __restrict__ time_first,
    const typename E::raw* __restrict__ r, typename E::raw* __restrict__ y,
    float* __restrict__ ck, uint64_t* __restrict__ lb, uint32_t* __restrict__ status, int rows,
    int T, int C, int max_polls) {
  using F = Fwd<E, VEC, L, W, WY, GATE>;
  using PackT = typename F::PackT;
  __shared__ typename F::Smem sm;

  const int nseg = (T + F::SEG - 1) / F::SEG;
  const int seg = __builtin_amdgcn_readfirstlane(int(blockIdx.x) / rows);
  const int row = int(blockIdx.x) - seg * rows;
  const int n_cg = (C + F::CPW - 1) / F::CPW;
  const int b = row / n_cg;
  const int cg = row - b * n_cg;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c0 = cg * F::CPW + lane * VEC;
  const bool active = c0 < C;
  const size_t row_base = size_t(b) * T * C + size_t(cg) * F::CPW;
  const size_t row_tail = size_t(T) * C - size_t(cg) * F::CPW;
  const unsigned lane_boff = active ? unsigned(lane * VEC * sizeof(typename E::raw)) : 0u;
  const int nblk = (T + kCkptBlock - 1) / kCkptBlock;
  const size_t ck_field = size_t(rows / n_cg) * nblk * C;  // B * nblk * C
  const size_t ck_row = size_t(b) * nblk * C + size_t(cg) * F::CPW;
  const unsigned ck_boff = active ? unsigned(lane * VEC * sizeof(float)) : 0u;
  const int t0 = seg * F::SEG + wave * L;

  PackT kb[L], vb[L], rb[L];
  F::load_chunk(k, v, r, row_base, row_tail, lane_boff, t0, C, kb, vb, rb);

  float D[VEC], DL[VEC], DS[VEC], U[VEC];
  bool u_ok = true;
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    const float dv = active ? decay[c0 + c] : 0.f;
    const float tf = active ? time_first[c0 + c] : 0.f;
    const float w2 = (decay_is_w ? dv : -expf(dv)) * kLog2e;
    const float u2 = tf * kLog2e;
    D[c] = fast_exp2(w2);
    DL[c] = fast_exp2(w2 * float(L));
    DS[c] = fast_exp2(w2 * float(F::SEG));
    U[c] = fast_exp2(u2);
    u_ok &= fabsf(u2) <= kMaxU;
  }
  if (threadIdx.x == 0) sm.bad = 0;
  const bool u_bad = __syncthreads_or(!u_ok) != 0;

  float s[L][VEC];
  float ps[VEC], qs[VEC];
  const bool full = (seg + 1) * F::SEG <= T;
  const bool kbad = full ? F::template summarize<true>(t0, T, kb, vb, D, s, ps, qs)
                         : F::template summarize<false>(t0, T, kb, vb, D, s, ps, qs);
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    sm.p[0][c][wave][lane] = ps[c];
    sm.q[0][c][wave][lane] = qs[c];
  }
  if (__any(active && kbad) && lane == 0) sm.bad = 1;
  __syncthreads();
  const bool bad = u_bad || sm.bad != 0;

  const size_t plane = size_t(nseg) * rows * F::CPW;  // words per kind
  uint64_t* const mine = lb + (size_t(seg) * rows + row) * F::CPW + lane * VEC;
  if (wave == 0) {
    if (bad) {
      // Out of the fixed frame's range: publish placeholders (successors
      // must not wait) and leave the row to the fix-up kernel.
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        lb_store(mine + c, kLbNaN);
        lb_store(mine + plane + c, kLbNaN);
      }
      if (lane == 0) mark_row_redo(status, row);
    } else {
      float ap[VEC], aq[VEC];
#pragma unroll
      for (int c = 0; c < VEC; ++c) { ap[c] = 0.f; aq[c] = 0.f; }
      for (int w = 0; w < W; ++w) {
#pragma unroll
        for (int c = 0; c < VEC; ++c) {
          ap[c] = fmaf(ap[c], DL[c], sm.p[0][c][w][lane]);
          aq[c] = fmaf(aq[c], DL[c], sm.q[0][c][w][lane]);
        }
      }
#pragma unroll
      for (int c = 0; c < VEC; ++c) lb_store(mine + c, lb_pack(ap[c], aq[c]));
      float cp[VEC], cq[VEC];
      const uint64_t* base = lb + size_t(row) * F::CPW + lane * VEC;
      const bool gave_up = !lb_window_carry<VEC>(base, base + plane, size_t(rows) * F::CPW, seg,
                                                 nseg, +1, DS, cp, cq, max_polls);
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        lb_store(mine + plane + c, lb_pack(fmaf(cp[c], DS[c], ap[c]), fmaf(cq[c], DS[c], aq[c])));
        sm.carry[0][0][c][lane] = cp[c];
        sm.carry[0][1][c][lane] = cq[c];
      }
      if (__any(gave_up) && lane == 0) mark_row_redo(status, row);
    }
  }
  __syncthreads();
  if (bad) return;

  // Carry-in of this chunk: the segment's carry, then the earlier chunks.
  float pin[VEC], qin[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    pin[c] = sm.carry[0][0][c][lane];
    qin[c] = sm.carry[0][1][c][lane];
  }
  for (int w = 0; w < wave; ++w) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      pin[c] = fmaf(pin[c], DL[c], sm.p[0][c][w][lane]);
      qin[c] = fmaf(qin[c], DL[c], sm.q[0][c][w][lane]);
    }
  }
  F::emit(t0, T, C, wave, active, row_base, row_tail, lane_boff, y, ck, ck_row, ck_boff, ck_field,
          s, vb, rb, D, U, pin, qin);
}

// Rows a split forward marked (keys outside the fixed frame's range, or a
// look-back that gave up): recomputed with the running-max recurrence, one
// channel per thread, overwriting y and the records.  One wave per row; an
// unmarked row returns at once.
template <typename E, bool WY, bool GATE>
__global__ __launch_bounds__(64) void wkv4_fwd_fixup_kernel(
    const typename E::raw* __restrict__ k, const typename E::raw* __restrict__ v,
    const float* __restrict__ decay, int decay_is_w, const float* __restrict__ time_first,
    const typename E::raw* __restrict__ r, typename E::raw* __restrict__ y,
    float* __restrict__ ck, const uint32_t* __restrict__ status, int cpw, int n_cg, int T,
    int C) {
  const int row = blockIdx.x;
  if (status[row] == kRowOk) return;
  const int b = row / n_cg;
  const int cg = row - b * n_cg;
  const int nblk = (T + kCkptBlock - 1) / kCkptBlock;
  const size_t ck_field = size_t(gridDim.x / n_cg) * nblk * C;
  for (int ch = threadIdx.x; ch < cpw; ch += 64) {
    const int c = cg * cpw + ch;
    if (c >= C) continue;
    const float w2 = (decay_is_w ? decay[c] : -expf(decay[c])) * kLog2e;
    const float u2 = time_first[c] * kLog2e;
    wkv4_fwd_channel_serial<E>(k, v, GATE ? r : nullptr, WY ? y : nullptr, w2, u2, T, C,
                               size_t(b) * T * C + c, ck, size_t(b) * nblk * C + c, ck_field);
  }
}

}  // namespace wkv

// ------------------------------------------------------------ launcher ----
namespace wkv_host {

// Tile configurations compiled into the library (no VGPR spills at 64*W
// threads per workgroup).  SEG = W*L must be a multiple of the 64-step
// checkpoint block.
static constexpr TileCfg kFwdCfgs[] = {{2, 8, 16}, {1, 8, 16}, {2, 8, 8}, {1, 16, 8}, {1, 8, 8},
                                        {1, 16, 4}, {2, 16, 4}};

// fp32 tensors already give 4-byte lane loads at one channel per lane; the
// 16-bit types use two channels per lane when the batch fills the GPU.
static TileCfg pick_fwd_cfg(int64_t B, int64_t C, int elem_bytes) {
  int vec, L, W;
  if (env_cfg("WKV_FWD_CFG", vec, L, W)) {
    for (const TileCfg& c : kFwdCfgs)
      if (c.vec == vec && c.L == L && c.W == W && (vec == 1 || C % 2 == 0)) return c;
  }
  if (elem_bytes == 2 && pick_vec(B, C) == 2) return TileCfg{2, 8, 16};
  return TileCfg{1, 8, 16};
}

// ------------------------------------------------ split over time (host) --
// Tile configurations of the split kernel (SEG = W*L steps per workgroup,
// a multiple of the 64-step record block).
static constexpr TileCfg kFwdSplitCfgs[] = {{1, 8, 8}, {1, 8, 16}, {1, 16, 4}, {2, 8, 8},
                                             {1, 4, 16}, {2, 4, 16}};

// The split kernel runs when the one-row kernel would leave CUs idle: fewer
// than kSplitRows rows of 64 channels and at least two segments.
// WKV_SPLIT=0 / 1 forces it off / on (measurement); WKV_FWD_SPLIT_CFG picks
// the tile.  Returns {0, 0, 0} when the one-row kernel runs.
int split_mode() {
  const char* s = getenv("WKV_SPLIT");
  return s ? atoi(s) : -1;
}

static TileCfg pick_fwd_split_cfg(int64_t B, int64_t T, int64_t C) {
  TileCfg cfg{1, 16, 4};
  int vec, L, W;
  if (env_cfg("WKV_FWD_SPLIT_CFG", vec, L, W)) {
    for (const TileCfg& c : kFwdSplitCfgs)
      if (c.vec == vec && c.L == L && c.W == W && (vec == 1 || C % 2 == 0)) cfg = c;
  }
  const int64_t rows1 = B * ((C + 63) / 64);
  const int64_t nseg = (T + cfg.L * cfg.W - 1) / (cfg.L * cfg.W);
  const int mode = split_mode();
  const bool want = mode == 1 || (mode != 0 && rows1 < kSplitRows && nseg >= kSplitMinSegs &&
                                       B * T * C >= kSplitMinElems);
  if (!want || nseg < 2 || B == 0 || C == 0) return TileCfg{0, 0, 0};
  return cfg;
}

// Workspace of the split forward: look-back words, then the row status words.
static size_t split_fwd_bytes(const TileCfg& cfg, int64_t B, int64_t T, int64_t C) {
  const int64_t cpw = 64 * cfg.vec;
  const int64_t rows = B * ((C + cpw - 1) / cpw);
  const int64_t nseg = (T + cfg.L * cfg.W - 1) / (cfg.L * cfg.W);
  const size_t words = size_t(2) * size_t(nseg) * size_t(rows) * size_t(cpw);
  return words * 8 + ((size_t(rows) * 4 + 15) / 16) * 16;
}

size_t wkv4_fwd_workspace_bytes_impl(int64_t B, int64_t T, int64_t C) {
  const TileCfg cfg = pick_fwd_split_cfg(B, T, C);
  return cfg.vec == 0 ? 0 : split_fwd_bytes(cfg, B, T, C);
}

// Fills `bytes` (a multiple of 16) of look-back workspace with all ones.
int lb_fill(void* ws, size_t bytes, hipStream_t stream) {
  const size_t n16 = bytes / 16;
  const unsigned blocks = unsigned(std::min<size_t>((n16 + 255) / 256, 4096));
  launch(wkv::lb_fill_kernel<0>, dim3(blocks), dim3(256), stream, false,
         static_cast<wkv::u32x4*>(ws), n16);
  return check_launch("lb_fill_kernel");
}

template <typename E, int VEC, int L, int W>
static int launch_fwd_split(const void* k, const void* v, const float* decay, int decay_is_w,
                            const float* tf, const void* r, void* y, float* ck, void* ws,
                            size_t ws_bytes, int B, int T, int C, hipStream_t stream) {
  using raw = typename E::raw;
  constexpr int CPW = 64 * VEC;
  const int n_cg = (C + CPW - 1) / CPW;
  const int rows = B * n_cg;
  const int nseg = (T + L * W - 1) / (L * W);
  const size_t words = size_t(2) * nseg * rows * CPW;
  uint64_t* lb = static_cast<uint64_t*>(ws);
  uint32_t* status = reinterpret_cast<uint32_t*>(lb + words);
  if (int rc = lb_fill(ws, ws_bytes, stream)) return rc;
  const raw* kk = static_cast<const raw*>(k);
  const raw* vv = static_cast<const raw*>(v);
  const raw* rr = static_cast<const raw*>(r);
  raw* yy = static_cast<raw*>(y);
  const dim3 grid(unsigned(nseg) * unsigned(rows)), block(W * 64);
  if (r != nullptr) {
    launch(wkv::wkv4_fwd_split_kernel<E, VEC, L, W, true, true>, grid, block, stream, false, kk,
           vv, decay, decay_is_w, tf, rr, yy, ck, lb, status, rows, T, C, lb_poll_limit());
  } else if (y != nullptr) {
    launch(wkv::wkv4_fwd_split_kernel<E, VEC, L, W, true, false>, grid, block, stream, false, kk,
           vv, decay, decay_is_w, tf, rr, yy, ck, lb, status, rows, T, C, lb_poll_limit());
  } else {
    launch(wkv::wkv4_fwd_split_kernel<E, VEC, L, W, false, false>, grid, block, stream, false,
           kk, vv, decay, decay_is_w, tf, rr, yy, ck, lb, status, rows, T, C, lb_poll_limit());
  }
  if (int rc = check_launch("wkv4_fwd_split_kernel")) return rc;
  if (r != nullptr) {
    launch(wkv::wkv4_fwd_fixup_kernel<E, true, true>, dim3(rows), dim3(64), stream, true, kk, vv,
           decay, decay_is_w, tf, rr, yy, ck, status, CPW, n_cg, T, C);
  } else if (y != nullptr) {
    launch(wkv::wkv4_fwd_fixup_kernel<E, true, false>, dim3(rows), dim3(64), stream, true, kk, vv,
           decay, decay_is_w, tf, rr, yy, ck, status, CPW, n_cg, T, C);
  } else {
    launch(wkv::wkv4_fwd_fixup_kernel<E, false, false>, dim3(rows), dim3(64), stream, true, kk,
           vv, decay, decay_is_w, tf, rr, yy, ck, status, CPW, n_cg, T, C);
  }
  return check_launch("wkv4_fwd_fixup_kernel");
}

// r (GATE) requires y.
template <typename E, int VEC, int L, int W>
static int launch_fwd(const void* k, const void* v, const float* decay, int decay_is_w,
                      const float* tf, const void* r, void* y, float* ck, int B, int T, int C,
                      hipStream_t stream) {
  using raw = typename E::raw;
  const int n_cg = (C + 64 * VEC - 1) / (64 * VEC);
  const dim3 grid(unsigned(B) * unsigned(n_cg)), block(W * 64);
  const raw* kk = static_cast<const raw*>(k);
  const raw* vv = static_cast<const raw*>(v);
  const raw* rr = static_cast<const raw*>(r);
  if (r != nullptr) {
    launch(wkv::wkv4_fwd_kernel<E, VEC, L, W, true, true>, grid, block, stream, true, kk, vv,
           decay, decay_is_w, tf, rr, static_cast<raw*>(y), ck, T, C);
  } else if (y != nullptr) {
    launch(wkv::wkv4_fwd_kernel<E, VEC, L, W, true, false>, grid, block, stream, true, kk, vv,
           decay, decay_is_w, tf, rr, static_cast<raw*>(y), ck, T, C);
  } else {
    launch(wkv::wkv4_fwd_kernel<E, VEC, L, W, false, false>, grid, block, stream, true, kk, vv,
           decay, decay_is_w, tf, rr, static_cast<raw*>(nullptr), ck, T, C);
  }
  return check_launch("wkv4_fwd_kernel");
}

template <typename E>
static int dispatch_fwd(const void* k, const void* v, const float* decay, int decay_is_w,
                        const float* tf, const void* r, void* y, float* ck, void* ws,
                        size_t ws_bytes, int B, int T, int C, hipStream_t stream) {
  const TileCfg sc = pick_fwd_split_cfg(B, T, C);
  if (sc.vec != 0 && ws != nullptr && ws_bytes >= split_fwd_bytes(sc, B, T, C)) {
    const size_t need = split_fwd_bytes(sc, B, T, C);
#define WKV_FWD_SPLIT_CASE(V, LL, WW)                                                        \
  if (sc.vec == V && sc.L == LL && sc.W == WW)                                              \
    return launch_fwd_split<E, V, LL, WW>(k, v, decay, decay_is_w, tf, r, y, ck, ws, need, B, \
                                          T, C, stream);
    WKV_FWD_SPLIT_CASE(1, 8, 8)
    WKV_FWD_SPLIT_CASE(1, 8, 16)
    WKV_FWD_SPLIT_CASE(1, 16, 4)
    WKV_FWD_SPLIT_CASE(2, 8, 8)
    WKV_FWD_SPLIT_CASE(1, 4, 16)
    WKV_FWD_SPLIT_CASE(2, 4, 16)
#undef WKV_FWD_SPLIT_CASE
  }
  const TileCfg cfg = pick_fwd_cfg(B, C, int(sizeof(typename E::raw)));
#define WKV_FWD_CASE(V, LL, WW)                    \
  if (cfg.vec == V && cfg.L == LL && cfg.W == WW) \
    return launch_fwd<E, V, LL, WW>(k, v, decay, decay_is_w, tf, r, y, ck, B, T, C, stream);
  WKV_FWD_CASE(2, 8, 16)
  WKV_FWD_CASE(1, 8, 16)
  WKV_FWD_CASE(2, 8, 8)
  WKV_FWD_CASE(1, 16, 8)
  WKV_FWD_CASE(1, 8, 8)
  WKV_FWD_CASE(1, 16, 4)
  WKV_FWD_CASE(2, 16, 4)
#undef WKV_FWD_CASE
  return fail(1, "wkv4_forward: no kernel for the selected tile configuration");
}

static int forward_any(const void* k, const void* v, const float* decay, int decay_is_w,
                       const float* tf, const void* r, void* y, float* ck, void* ws,
                       size_t ws_bytes, int B, int T, int C, int dtype, hipStream_t stream) {
  switch (dtype) {
    case 0:
      return dispatch_fwd<wkv::F32>(k, v, decay, decay_is_w, tf, r, y, ck, ws, ws_bytes, B, T, C,
                                    stream);
    case 1:
      return dispatch_fwd<wkv::BF16>(k, v, decay, decay_is_w, tf, r, y, ck, ws, ws_bytes, B, T, C,
                                     stream);
    case 2:
      return dispatch_fwd<wkv::F16>(k, v, decay, decay_is_w, tf, r, y, ck, ws, ws_bytes, B, T, C,
                                    stream);
    default: return fail(1, "wkv4_forward: unknown dtype");
  }
}

// ws (may be null): workspace for the split kernel, wkv4_fwd_workspace_bytes_impl bytes.
int wkv4_forward_impl(const void* k, const void* v, const float* decay, int decay_is_w,
                      const float* tf, void* y, float* ck, void* ws, size_t ws_bytes, int B,
                      int T, int C, int dtype, hipStream_t stream) {
  return forward_any(k, v, decay, decay_is_w, tf, nullptr, y, ck, ws, ws_bytes, B, T, C, dtype,
                     stream);
}

// y = sigmoid(r) * wkv (the time mix's gate folded in); y must be given.
int wkv4_forward_gated_impl(const void* k, const void* v, const float* decay, const float* tf,
                            const void* r, void* y, float* ck, void* ws, size_t ws_bytes, int B,
                            int T, int C, int dtype, hipStream_t stream) {
  return forward_any(k, v, decay, 0, tf, r, y, ck, ws, ws_bytes, B, T, C, dtype, stream);
}

}  // namespace wkv_host
