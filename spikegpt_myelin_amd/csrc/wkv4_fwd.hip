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
#include "wkv_common.h"

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
  // GATE: the receptance chunk rb as well.
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
    if constexpr (GATE) {
      const rsrc_t rr = make_rsrc(r + base, bytes);
#pragma unroll
      for (int i = 0; i < L; ++i) load_buf(rb[i], rr, lane_boff, unsigned(i) * stride);
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
    // Phase 1: e = 2^{k log2e} and the chunk summary from a zero state.
    float s[L][VEC];
    float ps[VEC], qs[VEC], mk[VEC];
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
    for (int c = 0; c < VEC; ++c) {
      bad |= mk[c] * kLog2e > kMaxK;
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
    if (ck != nullptr && wave % CPB == 0 && active && t0 < T) {
      const float zero[VEC] = {};
      float* rec = ck + ck_row + size_t(t0 / kCkptBlock) * C;
      store_vec<F32, VEC>(byte_offset(rec + 0 * ck_field, ck_boff), zero);
      store_vec<F32, VEC>(byte_offset(rec + 1 * ck_field, ck_boff), pin);
      store_vec<F32, VEC>(byte_offset(rec + 2 * ck_field, ck_boff), qin);
    }
    if (wave == W - 1) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        sm.carry[par][0][c][lane] = fmaf(pin[c], DL[c], ps[c]);
        sm.carry[par][1][c][lane] = fmaf(qin[c], DL[c], qs[c]);
      }
    }

    // Phase 2: outputs.
    if constexpr (WY) {
      OutPack<E, VEC> yp[L];
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
            yv[c] = round_to<E>(sigmoid_ref(rb[i].get(c))) * round_to<E>(yv[c]);
        }
        yp[i].set(yv);
      }
      if (active) {
        // Steps past T fall outside the descriptor and are dropped.
        const rsrc_t ry = make_rsrc(y + row_base + size_t(t0) * C,
                                    span_bytes(row_tail, t0, C, int(sizeof(raw))));
        const unsigned stride = unsigned(C) * unsigned(sizeof(raw));
#pragma unroll
        for (int i = 0; i < L; ++i) store_buf(yp[i], ry, lane_boff, unsigned(i) * stride);
      }
    }
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
        yv = round_to<E>(sigmoid_ref(load_scalar<E>(r + idx))) * round_to<E>(yv);
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
  PackT rA[L], rB[L];  // receptance chunks (loaded and used only with GATE)
  // The next segment is prefetched on every path (past the end the
  // descriptor is empty and the loads return zeros without touching memory):
  // with the same loads issued on every path, the compiler's wait before a
  // segment's arithmetic only covers the loads it consumes, not the prefetch
  // issued just before it.
  if (!bad) F::load_chunk(k, v, r, row_base, row_tail, lane_boff, wave * L, C, kA, vA, rA);
  for (int seg = 0; seg < nseg && !bad; seg += 2) {
    F::load_chunk(k, v, r, row_base, row_tail, lane_boff, (seg + 1) * F::SEG + wave * L, C, kB, vB,
                  rB);
    bad = seg < nfull
              ? F::template segment<true>(sm, seg, T, C, wave, lane, active, row_base, row_tail, lane_boff, y,
                                          ck, ck_row, ck_boff, ck_field, kA, vA, rA, D, DL, U)
              : F::template segment<false>(sm, seg, T, C, wave, lane, active, row_base, row_tail, lane_boff,
                                           y, ck, ck_row, ck_boff, ck_field, kA, vA, rA, D, DL, U);
    if (bad || seg + 1 >= nseg) break;
    F::load_chunk(k, v, r, row_base, row_tail, lane_boff, (seg + 2) * F::SEG + wave * L, C, kA, vA,
                  rA);
    bad = seg + 1 < nfull
              ? F::template segment<true>(sm, seg + 1, T, C, wave, lane, active, row_base,
                                          row_tail, lane_boff, y, ck, ck_row, ck_boff, ck_field, kB, vB, rB, D,
                                          DL, U)
              : F::template segment<false>(sm, seg + 1, T, C, wave, lane, active, row_base,
                                           row_tail, lane_boff, y, ck, ck_row, ck_boff, ck_field, kB, vB, rB, D,
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

}  // namespace wkv

// ------------------------------------------------------------ launcher ----
namespace wkv_host {

struct TileCfg { int vec, L, W; };

// Tile configurations compiled into the library (no VGPR spills at 64*W
// threads per workgroup).  SEG = W*L must be a multiple of the 64-step
// checkpoint block.
static constexpr TileCfg kFwdCfgs[] = {{2, 8, 16}, {1, 8, 16}, {2, 8, 8}, {1, 16, 8}, {1, 8, 8},
                                        {1, 16, 4}, {2, 16, 4}};

int pick_vec(int64_t B, int64_t C);
bool env_cfg(const char* name, int& vec, int& L, int& W);

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
                        const float* tf, const void* r, void* y, float* ck, int B, int T, int C,
                        hipStream_t stream) {
  TileCfg cfg = pick_fwd_cfg(B, C, int(sizeof(typename E::raw)));
  // The gated kernel holds the receptance chunks as well: at 16 waves per
  // workgroup (128 VGPRs) the two-channel tile spills, so it runs 8 waves.
  if (r != nullptr && cfg.vec == 2 && cfg.W == 16) cfg = TileCfg{2, cfg.L, 8};
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
                       const float* tf, const void* r, void* y, float* ck, int B, int T, int C,
                       int dtype, hipStream_t stream) {
  switch (dtype) {
    case 0: return dispatch_fwd<wkv::F32>(k, v, decay, decay_is_w, tf, r, y, ck, B, T, C, stream);
    case 1: return dispatch_fwd<wkv::BF16>(k, v, decay, decay_is_w, tf, r, y, ck, B, T, C, stream);
    case 2: return dispatch_fwd<wkv::F16>(k, v, decay, decay_is_w, tf, r, y, ck, B, T, C, stream);
    default: return fail(1, "wkv4_forward: unknown dtype");
  }
}

int wkv4_forward_impl(const void* k, const void* v, const float* decay, int decay_is_w,
                      const float* tf, void* y, float* ck, int B, int T, int C, int dtype,
                      hipStream_t stream) {
  return forward_any(k, v, decay, decay_is_w, tf, nullptr, y, ck, B, T, C, dtype, stream);
}

// y = sigmoid(r) * wkv (the time mix's gate folded in); y must be given.
int wkv4_forward_gated_impl(const void* k, const void* v, const float* decay, const float* tf,
                            const void* r, void* y, float* ck, int B, int T, int C, int dtype,
                            hipStream_t stream) {
  return forward_any(k, v, decay, 0, tf, r, y, ck, B, T, C, dtype, stream);
}

}  // namespace wkv_host
