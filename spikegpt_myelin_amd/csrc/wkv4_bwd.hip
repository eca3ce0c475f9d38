// RWKV-4 / SpikeGPT WKV backward for gfx950.
//
// Gradients (the quantities the reference backward kernel produces,
// src/spikegpt/wkv_triton.py:60-142, derived here from the closed form).
// Per lane, with den_t = B_t + e^{u+k_t}, z_t = gy_t / den_t and the reverse
// sums over later steps
//   G_t  = sum_{s>t} e^{(s-1-t)w} z_s,          H_t  = sum_{s>t} e^{(s-1-t)w} z_s y_s,
//   G'_t = sum_{s>t} (s-1-t) e^{(s-1-t)w} z_s,   H'_t = likewise with z_s y_s,
// the gradients are
//   gv_t = z_t e^{u+k_t} + e^{k_t} G_t
//   gk_t = z_t e^{u+k_t} (v_t - y_t) + e^{k_t} (v_t G_t - H_t)
//   gu   = sum_t z_t e^{u+k_t} (v_t - y_t)
//   gw   = sum_t e^{k_t} (v_t G'_t - H'_t)        (d/dw of e^{(t-1-i)w})
// and the reverse sums obey G_{t-1} = e^w G_t + z_t,
// G'_{t-1} = e^w (G'_t + G_t) (same for H with z_t y_t).  G_t and -H_t are
// the adjoints of the forward state (A_{t+1}, B_{t+1}) of the recurrence
// A_{t+1} = e^w A_t + e^{k_t} v_t, so the w-gradient is also
//   gw   = e^w sum_t (G_t A_t - H_t B_t)
// (expand both sides: each pair i < s is counted s-1-i times).  The reverse
// sweep uses this form: it needs the forward states the sweep recomputes
// anyway and no G', H' sums.  The reference accumulates gw in its forward
// replay (dpdw/dqdw); accumulating it in the reverse sweep needs no extra
// forward state, so the forward can be recomputed from the small checkpoint
// records the forward kernel writes.
//
// One reverse sweep (segments last to first; rows, chunks and segments as in
// the forward kernel).  Per segment each wave:
//   * takes the forward state at the segment start from the records,
//     prefetched with the segment's k, v, gy;
//   * computes 2^{k log2e} and its chunk's forward summary; after one
//     barrier, an LDS Horner gives its chunk's forward carry;
//   * recomputes the chunk's forward keeping z = gy/den, z y and the states
//     (A_t, B_t) in registers and reduces its chunk's reverse sums from a zero
//     state; after a second barrier, a reverse LDS Horner
//     (G <- G_j + e^{Lw} G) gives the carry at its chunk's end;
//   * runs the reverse recurrence with that carry, writing gk and gv and
//     accumulating gw and gu.
// k, v, gy are read once and gk, gv written once.  gw/gu are reduced over the
// waves of the row into [B, C] partials that a second small kernel sums over
// B in fixed order (deterministic).
//
// All sums live in the forward kernel's fixed base-2 frame (e = 2^{k log2e},
// state (A, B) = (p, q)), which is exact while the forward kernel's range
// guard holds.  The forward kernel marks each row it recomputed with the
// exact serial path (record o = -1e38 at block 0 instead of 0); such rows are
// recomputed here one channel per thread with the reference's running-max
// recurrences.
#include <algorithm>

#include "wkv_common.h"
#include "wkv_impl.h"

namespace wkv {

// Serial recomputation of one channel with the reference's recurrences (base
// 2) from the checkpoint records.  Blocks of 64 steps are visited last to
// first and, inside each, sub-chunks of L steps last to first: the forward is
// replayed from the block record to the sub-chunk, the sub-chunk's y, 1/den
// and output exponent are kept, and the stabilised reverse recurrence
// (wkv_triton.py:120-142, extended by the G', H' sums for gw) runs over it.
// Quadratic within a block; only rows outside the shared-frame range take it.
// r, gr (both null, or both given): the forward was sigmoid(r) * wkv; gy is
// the gradient of that product and grad_r is written to gr.
template <typename E, int L>
__device__ void wkv4_bwd_channel_serial(const typename E::raw* __restrict__ gy,
                                        const typename E::raw* __restrict__ k,
                                        const typename E::raw* __restrict__ v,
                                        const typename E::raw* __restrict__ r,
                                        typename E::raw* __restrict__ gk,
                                        typename E::raw* __restrict__ gv,
                                        typename E::raw* __restrict__ gr, float w2, float u2,
                                        int T, int C, size_t base, const float* __restrict__ ck,
                                        size_t ck_lane, size_t ck_field, float& gw_out,
                                        float& gu_out) {
  const int nblk = (T + kCkptBlock - 1) / kCkptBlock;
  float orr = kNegHuge, G = 0.f, H = 0.f, Gp = 0.f, Hp = 0.f;
  float gw = 0.f, gu = 0.f;
  for (int j = nblk - 1; j >= 0; --j) {
    const int b0 = j * kCkptBlock;
    const int nsub = (min(T - b0, kCkptBlock) + L - 1) / L;
    const float* rec = ck + ck_lane + size_t(j) * C;
    for (int m = nsub - 1; m >= 0; --m) {
      float o = rec[0 * ck_field], p = rec[1 * ck_field], q = rec[2 * ck_field];
      const int t0 = b0 + m * L;
      for (int t = b0; t < t0; ++t) {
        const size_t idx = base + size_t(t) * C;
        const float kk = load_scalar<E>(k + idx) * kLog2e;
        const float vv = load_scalar<E>(v + idx);
        const float wo = w2 + o;
        const float no = fmaxf(wo, kk);
        const float a = fast_exp2(wo - no);
        const float bb = fast_exp2(kk - no);
        p = a * p + bb * vv;
        q = a * q + bb;
        o = no;
      }
      float ys[L], rs[L], nfs[L];
#pragma unroll
      for (int i = 0; i < L; ++i) {
        const int t = t0 + i;
        ys[i] = 0.f;
        rs[i] = 0.f;
        nfs[i] = 0.f;
        if (t < T) {
          const size_t idx = base + size_t(t) * C;
          const float kk = load_scalar<E>(k + idx) * kLog2e;
          const float vv = load_scalar<E>(v + idx);
          const float uk = u2 + kk;
          float no = fmaxf(o, uk);
          float a = fast_exp2(o - no);
          float bb = fast_exp2(uk - no);
          const float r = 1.f / (a * q + bb);
          ys[i] = (a * p + bb * vv) * r;
          rs[i] = r;
          nfs[i] = no;
          const float wo = w2 + o;
          no = fmaxf(wo, kk);
          a = fast_exp2(wo - no);
          bb = fast_exp2(kk - no);
          p = a * p + bb * vv;
          q = a * q + bb;
          o = no;
        }
      }
#pragma unroll
      for (int i = L - 1; i >= 0; --i) {
        const int t = t0 + i;
        if (t < T) {
          const size_t idx = base + size_t(t) * C;
          const float kk = load_scalar<E>(k + idx) * kLog2e;
          const float vv = load_scalar<E>(v + idx);
          float g = load_scalar<E>(gy + idx);
          if (r != nullptr) {
            float grad_r;
            g = gate_backward<E>(g, gate_sigmoid<E>(load_scalar<E>(r + idx)), round_to<E>(ys[i]),
                                 grad_r);
            store_scalar<E>(gr + idx, grad_r);
          }
          const float zr = g * rs[i];
          const float ze = zr * fast_exp2(u2 + kk - nfs[i]);
          const float bk = fast_exp2(kk + orr);
          const float gkd = ze * (vv - ys[i]);
          store_scalar<E>(gv + idx, ze + bk * G);
          store_scalar<E>(gk + idx, gkd + bk * (vv * G - H));
          gu += gkd;
          gw += bk * (vv * Gp - Hp);
          const float wo = w2 + orr;
          const float no = fmaxf(wo, -nfs[i]);
          const float a = fast_exp2(wo - no);
          const float bz = zr * fast_exp2(-nfs[i] - no);
          Gp = a * (Gp + G);
          Hp = a * (Hp + H);
          G = a * G + bz;
          H = a * H + bz * ys[i];
          orr = no;
        }
      }
    }
  }
  gw_out = gw;
  gu_out = gu;
}

template <typename E, int VEC, int L, int W, bool GATE = false>
struct Bwd {
  using raw = typename E::raw;
  using PackT = Pack<E, VEC>;
  static constexpr int CPW = 64 * VEC;
  static constexpr int SEG = W * L;
  static constexpr int BPS = SEG / kCkptBlock;  // checkpoint blocks per segment
  // The one-row kernel's (1, 8, 16) tile loads each segment when it starts
  // instead of one segment ahead (see wkv4_bwd_kernel).
  static constexpr bool kNoPrefetch = VEC == 1 && L == 8 && W == 16;
  static_assert(SEG % kCkptBlock == 0, "segment/block layout");

  struct Smem {
    float p[VEC][W][64];
    float q[VEC][W][64];
    float G[VEC][W][64];
    float H[VEC][W][64];
    float rcarry[2][2][VEC][64];  // reverse segment carry (G, H)
  };

  // Per channel: e^{iw} (d0[i-1]) for i = 1..L-1.
  struct Weights {
    float d0[L - 1][VEC];
  };

  // Forward state at a segment's start.
  struct Recs {
    float p[VEC], q[VEC];
  };

  // Loads the wave's chunk (L steps from t0) of segment seg through buffer
  // descriptors based at the chunk (row_base, ck_row wave-uniform; lane_boff,
  // ck_boff the lane's byte offsets); steps at or past T read as zero.
  // GATE: also the receptance chunk rb (g is then the gradient of the gated
  // output).
  __device__ static __forceinline__ void load(const raw* __restrict__ k, const raw* __restrict__ v,
                                              const raw* __restrict__ g, const raw* __restrict__ r,
                                              const float* __restrict__ ck, size_t ck_row,
                                              unsigned ck_boff, size_t ck_field, int seg,
                                              size_t row_base, size_t row_tail, unsigned lane_boff,
                                              int t0, int C, PackT (&kb)[L], PackT (&vb)[L],
                                              PackT (&gb)[L], PackT (&rb)[L], Recs& rc) {
    const uint32_t bytes = span_bytes(row_tail, t0, C, int(sizeof(raw)));
    const size_t base = row_base + size_t(t0) * C;
    const rsrc_t rk = make_rsrc(k + base, bytes);
    const rsrc_t rv = make_rsrc(v + base, bytes);
    const rsrc_t rg = make_rsrc(g + base, bytes);
    const unsigned stride = unsigned(C) * unsigned(sizeof(raw));
#pragma unroll
    for (int i = 0; i < L; ++i) {
      load_buf(kb[i], rk, lane_boff, unsigned(i) * stride);
      load_buf(vb[i], rv, lane_boff, unsigned(i) * stride);
      load_buf(gb[i], rg, lane_boff, unsigned(i) * stride);
    }
    if constexpr (GATE) {
      const rsrc_t rr = make_rsrc(r + base, bytes);
#pragma unroll
      for (int i = 0; i < L; ++i) load_buf(rb[i], rr, lane_boff, unsigned(i) * stride);
    }
    const float* rec = ck + ck_row + size_t(seg) * BPS * C;
    Pack<F32, VEC> a;
    a.load(byte_offset(rec + 1 * ck_field, ck_boff));
#pragma unroll
    for (int c = 0; c < VEC; ++c) rc.p[c] = a.x[c];
    a.load(byte_offset(rec + 2 * ck_field, ck_boff));
#pragma unroll
    for (int c = 0; c < VEC; ++c) rc.q[c] = a.x[c];
  }

  // e^{k} of the chunk's steps (zero past T) and the chunk's forward summary
  // from a zero state.
  template <bool FULL>
  __device__ static __forceinline__ void summarize(int t0, int T, const PackT (&kb)[L],
                                                   const PackT (&vb)[L], const float (&D)[VEC],
                                                   float (&ek)[L][VEC], float (&ps)[VEC],
                                                   float (&qs)[VEC]) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) { ps[c] = 0.f; qs[c] = 0.f; }
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const bool valid = FULL || (t0 + i) < T;
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        float e = fast_exp2(kb[i].get(c) * kLog2e);
        if (!FULL) e = valid ? e : 0.f;
        ek[i][c] = e;
        ps[c] = fmaf(ps[c], D[c], e * vb[i].get(c));
        qs[c] = fmaf(qs[c], D[c], e);
      }
    }
  }

  // Forward recompute of the chunk from its forward carry (P, Q): keeps
  // z = gy/den, z y (zero past the end) and the states (A_t, B_t) before
  // step t; GATE: the gate's backward, grad_r stored.  Then the chunk's
  // reverse summary (G, H) from a zero state at its end, as dot products
  // with the weights e^{iw} of step i: G = sum_i e^{iw} z_i (H with z y).
  template <bool FULL>
  __device__ static __forceinline__ void recompute(
      int t0, int T, int C, bool active, size_t row_base, size_t row_tail, unsigned lane_boff,
      const PackT (&vb)[L], const PackT (&gb)[L], const PackT (&rb)[L], const float (&ek)[L][VEC],
      const float (&D)[VEC], const float (&U)[VEC], const Weights& Wt, float (&P)[VEC],
      float (&Q)[VEC], float (&zz)[L][VEC], float (&zy)[L][VEC], float (&pa)[L][VEC],
      float (&qa)[L][VEC], raw* __restrict__ gr, float (&G)[VEC], float (&H)[VEC]) {
    OutPack<E, VEC> grp[GATE ? L : 1];
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const bool valid = FULL || (t0 + i) < T;
      float grv[VEC];
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const float vv = vb[i].get(c);
        const float e = ek[i][c];
        const float e1 = e * U[c];
        const float r = fast_rcp(Q[c] + e1);
        const float y = fmaf(e1, vv, P[c]) * r;
        float gyv = gb[i].get(c);
        if constexpr (GATE) {
          // The gate's backward as the separate kernels compute it: its
          // input gradient round(g s) feeds the recurrence, and grad_r
          // comes from round(g y) with y rounded as the forward stored it.
          gyv = gate_backward<E>(gyv, gate_sigmoid<E>(rb[i].get(c)), round_to<E>(y), grv[c]);
        }
        const float z = gyv * r;
        zz[i][c] = FULL || valid ? z : 0.f;
        zy[i][c] = FULL || valid ? z * y : 0.f;
        pa[i][c] = P[c];
        qa[i][c] = Q[c];
        P[c] = fmaf(e, vv, P[c] * D[c]);
        Q[c] = fmaf(Q[c], D[c], e);
      }
      if constexpr (GATE) grp[i].set(grv);
    }
    if constexpr (GATE) {
      if (active) {
        // Steps past T fall outside the descriptor and are dropped.
        const rsrc_t rgr = make_rsrc(gr + row_base + size_t(t0) * C,
                                     span_bytes(row_tail, t0, C, int(sizeof(raw))));
        const unsigned stride = unsigned(C) * unsigned(sizeof(raw));
#pragma unroll
        for (int i = 0; i < L; ++i) store_buf(grp[i], rgr, lane_boff, unsigned(i) * stride);
      }
    }
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      G[c] = zz[0][c];
      H[c] = zy[0][c];
    }
#pragma unroll
    for (int i = 1; i < L; ++i) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        G[c] = fmaf(zz[i][c], Wt.d0[i - 1][c], G[c]);
        H[c] = fmaf(zy[i][c], Wt.d0[i - 1][c], H[c]);
      }
    }
  }

  // Reverse pass of the chunk from the carry (G, H) at its end: gk, gv
  // stored (together, after the pass), gw and gu accumulated; (G, H) leaves
  // as the carry at the chunk's start.
  __device__ static __forceinline__ void reverse(
      int t0, int C, bool active, size_t row_base, size_t row_tail, unsigned lane_boff,
      const PackT (&vb)[L], const float (&ek)[L][VEC], const float (&zz)[L][VEC],
      const float (&zy)[L][VEC], const float (&pa)[L][VEC], const float (&qa)[L][VEC],
      const float (&D)[VEC], const float (&U)[VEC], float (&G)[VEC], float (&H)[VEC],
      raw* __restrict__ gk, raw* __restrict__ gv, float (&gw)[VEC], float (&gu)[VEC]) {
    OutPack<E, VEC> gko_p[L], gvo_p[L];
#pragma unroll
    for (int i = L - 1; i >= 0; --i) {
      float gko[VEC], gvo[VEC];
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const float vv = vb[i].get(c);
        const float e = ek[i][c];
        const float z = zz[i][c];
        // With a = e^u z + G and b = e^u z y + H:
        //   gv = e a,  gk = e (v a - b) = e^{u+k} z (v - y) + e^k (v G - H),
        // and gu accumulates e (z v - z y) (times e^u once at the end).
        const float a = fmaf(U[c], z, G[c]);
        const float bb = fmaf(U[c], zy[i][c], H[c]);
        gvo[c] = e * a;
        gko[c] = e * fmaf(vv, a, -bb);
        gu[c] = fmaf(e, fmaf(z, vv, -zy[i][c]), gu[c]);
        // gw accumulates G_t A_t - H_t B_t (times e^w once at the end).
        gw[c] = fmaf(G[c], pa[i][c], fmaf(-H[c], qa[i][c], gw[c]));
        G[c] = fmaf(G[c], D[c], z);
        H[c] = fmaf(H[c], D[c], zy[i][c]);
      }
      gko_p[i].set(gko);
      gvo_p[i].set(gvo);
    }
    if (active) {
      // Steps past T fall outside the descriptors and are dropped.
      const uint32_t bytes = span_bytes(row_tail, t0, C, int(sizeof(raw)));
      const size_t base = row_base + size_t(t0) * C;
      const rsrc_t rgk = make_rsrc(gk + base, bytes);
      const rsrc_t rgv = make_rsrc(gv + base, bytes);
      const unsigned stride = unsigned(C) * unsigned(sizeof(raw));
#pragma unroll
      for (int i = L - 1; i >= 0; --i) {
        store_buf(gko_p[i], rgk, lane_boff, unsigned(i) * stride);
        store_buf(gvo_p[i], rgv, lane_boff, unsigned(i) * stride);
      }
    }
  }

  // One segment (visited last to first).  FULL: every step is inside the
  // sequence.
  template <bool FULL>
  __device__ static __forceinline__ void segment(
      Smem& sm, int seg, int nseg, int T, int C, int wave, int lane, bool active, size_t row_base,
      size_t row_tail, unsigned lane_boff, const PackT (&kb)[L], const PackT (&vb)[L], const PackT (&gb)[L],
      const PackT (&rb)[L], const Recs& rc, const float (&D)[VEC], const float (&DL)[VEC],
      const float (&U)[VEC], const Weights& Wt, raw* __restrict__ gk, raw* __restrict__ gv,
      raw* __restrict__ gr, float (&gw)[VEC], float (&gu)[VEC]) {
    const int t0 = (seg * W + wave) * L;
    float P[VEC], Q[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      P[c] = rc.p[c];
      Q[c] = rc.q[c];
    }
    float ek[L][VEC];
    float ps[VEC], qs[VEC];
    summarize<FULL>(t0, T, kb, vb, D, ek, ps, qs);
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      sm.p[c][wave][lane] = ps[c];
      sm.q[c][wave][lane] = qs[c];
    }
    __syncthreads();
    for (int w = 0; w < wave; ++w) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        P[c] = fmaf(P[c], DL[c], sm.p[c][w][lane]);
        Q[c] = fmaf(Q[c], DL[c], sm.q[c][w][lane]);
      }
    }
    float zz[L][VEC], zy[L][VEC], pa[L][VEC], qa[L][VEC];
    float G[VEC], H[VEC];
    recompute<FULL>(t0, T, C, active, row_base, row_tail, lane_boff, vb, gb, rb, ek, D, U, Wt, P,
                    Q, zz, zy, pa, qa, gr, G, H);
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      sm.G[c][wave][lane] = G[c];
      sm.H[c][wave][lane] = H[c];
    }
    __syncthreads();
    // Carry at this chunk's end: the later segment's carry, then the later
    // chunks of this segment, nearest last.
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const int sl = (seg + 1) & 1;
      const bool later = seg + 1 < nseg;
      G[c] = later ? sm.rcarry[sl][0][c][lane] : 0.f;
      H[c] = later ? sm.rcarry[sl][1][c][lane] : 0.f;
    }
    for (int w = W - 1; w > wave; --w) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        G[c] = fmaf(DL[c], G[c], sm.G[c][w][lane]);
        H[c] = fmaf(DL[c], H[c], sm.H[c][w][lane]);
      }
    }
    reverse(t0, C, active, row_base, row_tail, lane_boff, vb, ek, zz, zy, pa, qa, D, U, G, H, gk,
            gv, gw, gu);
    if (wave == 0) {
      const int sl = seg & 1;
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        sm.rcarry[sl][0][c][lane] = G[c];
        sm.rcarry[sl][1][c][lane] = H[c];
      }
    }
  }
};

// decay: time_decay (decay_is_w == 0, w = -exp(decay)) or w itself.
// GATE: the forward was y = sigmoid(r) * wkv; gy is the gradient of that y,
// and the kernel also writes grad_r (gr).
template <typename E, int VEC, int L, int W, bool GATE>
__global__ __launch_bounds__(W * 64) void wkv4_bwd_kernel(
    const typename E::raw* __restrict__ gy, const float* __restrict__ decay, int decay_is_w,
    const float* __restrict__ u_in, const typename E::raw* __restrict__ k,
    const typename E::raw* __restrict__ v, const typename E::raw* __restrict__ r,
    const float* __restrict__ ck, typename E::raw* __restrict__ gk,
    typename E::raw* __restrict__ gv, typename E::raw* __restrict__ gr,
    float* __restrict__ gw_part, float* __restrict__ gu_part, int T, int C) {
  using F = Bwd<E, VEC, L, W, GATE>;
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
  const int nseg = (T + F::SEG - 1) / F::SEG;
  const int nfull = T / F::SEG;
  const int nblk = (T + kCkptBlock - 1) / kCkptBlock;
  const size_t ck_field = size_t(gridDim.x / n_cg) * nblk * C;
  const size_t ck_row = size_t(b) * nblk * C + size_t(cg) * F::CPW;
  const unsigned ck_boff = active ? unsigned(lane * VEC * sizeof(float)) : 0u;

  float D[VEC], DL[VEC], U[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    const float dv = active ? decay[c0 + c] : 0.f;
    const float uv = active ? u_in[c0 + c] : 0.f;
    const float w2 = (decay_is_w ? dv : -expf(dv)) * kLog2e;
    D[c] = fast_exp2(w2);
    DL[c] = fast_exp2(w2 * float(L));
    U[c] = fast_exp2(uv * kLog2e);
  }
  typename F::Weights Wt;
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    float pw = D[c];
#pragma unroll
    for (int i = 1; i < L; ++i) {
      Wt.d0[i - 1][c] = pw;
      pw *= D[c];
    }
  }
  // Rows the forward kernel recomputed with its exact serial path carry
  // o != 0 in their block-0 records; this row then takes the exact path too.
  bool serial = false;
  {
    Pack<F32, VEC> o;
    o.load(byte_offset(ck + ck_row, ck_boff));
#pragma unroll
    for (int c = 0; c < VEC; ++c) serial |= active && o.x[c] != 0.f;
  }
  const bool bad = __syncthreads_or(serial) != 0;

  float gw[VEC], gu[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) { gw[c] = 0.f; gu[c] = 0.f; }
  if (!bad) {
    PackT kA[L], vA[L], gA[L], kB[L], vB[L], gB[L];
    PackT xA[L], xB[L];  // receptance chunks (loaded and used only with GATE)
    typename F::Recs rA, rB;
    const int last = nseg - 1;
    if constexpr (F::kNoPrefetch) {
      // Sixteen waves of one channel per lane: no segment is fetched ahead
      // (the second register buffer would not fit the 128 VGPRs that four
      // waves per SIMD leave); the other waves on each SIMD cover the wait.
      for (int seg = last; seg >= 0; --seg) {
        F::load(k, v, gy, r, ck, ck_row, ck_boff, ck_field, seg, row_base, row_tail, lane_boff,
                seg * F::SEG + wave * L, C, kA, vA, gA, xA, rA);
        if (seg < nfull) {
          F::template segment<true>(sm, seg, nseg, T, C, wave, lane, active, row_base, row_tail,
                                    lane_boff, kA, vA, gA, xA, rA, D, DL, U, Wt, gk, gv, gr, gw,
                                    gu);
        } else {
          F::template segment<false>(sm, seg, nseg, T, C, wave, lane, active, row_base, row_tail,
                                     lane_boff, kA, vA, gA, xA, rA, D, DL, U, Wt, gk, gv, gr, gw,
                                     gu);
        }
      }
    } else {
    F::load(k, v, gy, r, ck, ck_row, ck_boff, ck_field, last, row_base, row_tail, lane_boff,
            last * F::SEG + wave * L, C, kA, vA, gA, xA, rA);
    // The next segment is prefetched on every path (segment 0 prefetches
    // itself again, a cache hit), so that the wait before a segment's
    // arithmetic only covers the loads it consumes.  Steps past T read as
    // zero (outside the buffer descriptors).
    for (int seg = last; seg >= 0; seg -= 2) {
      const int s1 = max(seg - 1, 0), s2 = max(seg - 2, 0);
      F::load(k, v, gy, r, ck, ck_row, ck_boff, ck_field, s1, row_base, row_tail, lane_boff,
              s1 * F::SEG + wave * L, C, kB, vB, gB, xB, rB);
      if (seg < nfull) {
        F::template segment<true>(sm, seg, nseg, T, C, wave, lane, active, row_base, row_tail, lane_boff,
                                  kA, vA, gA, xA, rA, D, DL, U, Wt, gk, gv, gr, gw, gu);
      } else {
        F::template segment<false>(sm, seg, nseg, T, C, wave, lane, active, row_base, row_tail, lane_boff,
                                   kA, vA, gA, xA, rA, D, DL, U, Wt, gk, gv, gr, gw, gu);
      }
      if (seg - 1 < 0) break;
      F::load(k, v, gy, r, ck, ck_row, ck_boff, ck_field, s2, row_base, row_tail, lane_boff,
              s2 * F::SEG + wave * L, C, kA, vA, gA, xA, rA);
      if (seg - 1 < nfull) {
        F::template segment<true>(sm, seg - 1, nseg, T, C, wave, lane, active, row_base,
                                  row_tail, lane_boff, kB, vB, gB, xB, rB, D, DL, U, Wt, gk, gv, gr, gw, gu);
      } else {
        F::template segment<false>(sm, seg - 1, nseg, T, C, wave, lane, active, row_base,
                                   row_tail, lane_boff, kB, vB, gB, xB, rB, D, DL, U, Wt, gk, gv, gr, gw, gu);
      }
    }
    }
  }

  if (!bad) {
    // Reduce gw/gu over the waves of the row (reusing the summary arrays).
    __syncthreads();
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      sm.G[c][wave][lane] = gw[c] * D[c];
      sm.H[c][wave][lane] = gu[c] * U[c];
    }
    __syncthreads();
    for (int ch = threadIdx.x; ch < F::CPW; ch += blockDim.x) {
      const int c = cg * F::CPW + ch;
      if (c >= C) continue;
      // channel ch of the row lives in lane ch / VEC, slot ch % VEC
      const int l = ch / VEC, s = ch - l * VEC;
      float sw = 0.f, su = 0.f;
      for (int w = 0; w < W; ++w) {
        sw += sm.G[s][w][l];
        su += sm.H[s][w][l];
      }
      gw_part[size_t(b) * C + c] = sw;
      gu_part[size_t(b) * C + c] = su;
    }
  } else {
    for (int ch = threadIdx.x; ch < F::CPW; ch += blockDim.x) {
      const int c = cg * F::CPW + ch;
      if (c >= C) continue;
      const float w2 = (decay_is_w ? decay[c] : -expf(decay[c])) * kLog2e;
      float sw, su;
      wkv4_bwd_channel_serial<E, 8>(gy, k, v, GATE ? r : nullptr, gk, gv, GATE ? gr : nullptr,
                                    w2, u_in[c] * kLog2e, T, C,
                                    size_t(b) * T * C + c, ck, size_t(b) * nblk * C + c,
                                    ck_field, sw, su);
      gw_part[size_t(b) * C + c] = sw;
      gu_part[size_t(b) * C + c] = su;
    }
  }
}

// ----------------------------------------------------- split over time ----
// For few rows: one workgroup per (segment, row), blockIdx = (nseg - 1 -
// segment) * rows + row, so that later segments are dispatched first.  The
// forward state at the segment's start comes from the records; the reverse
// carry at its end (G, H from all later steps) comes from the later
// segments' words, mirroring the forward split kernel (lb_window_carry over
// the K nearest later segments and one inclusive word):
//   R_s = sum_{j>s} e^{(j-s-1) SEG w} agg_j,   incl_s = e^{SEG w} R_s + agg_s,
// with agg_s the segment's reverse sums from a zero state at its end (the
// fold of its chunks' sums) and incl_s the reverse state at its start.  gw
// and gu are reduced per (batch, segment) into [B * nseg][C] partials, which
// wkv4_bwd_fixup_kernel sums over the segments into [B][C] for
// wkv4_param_grad_kernel.  Rows that the forward recomputed exactly, and rows
// whose look-back gave up, are left to wkv4_bwd_fixup_kernel.
//
// Look-back words: lb[2][nseg][rows][64*VEC] (aggregates, then inclusive
// states), each word the pair (G, H) of one channel; status[rows].
template <typename E, int VEC, int L, int W, bool GATE>
__global__ __launch_bounds__(W * 64) void wkv4_bwd_split_kernel(
    const typename E::raw* __restrict__ gy, const float* __restrict__ decay, int decay_is_w,
    const float* __restrict__ u_in, const typename E::raw* __restrict__ k,
    const typename E::raw* __restrict__ v, const typename E::raw* __restrict__ r,
    const float* __restrict__ ck, typename E::raw* __restrict__ gk,
    typename E::raw* __restrict__ gv, typename E::raw* __restrict__ gr,
    float* __restrict__ gw_part, float* __restrict__ gu_part, uint64_t* __restrict__ lb,
    uint32_t* __restrict__ status, int rows, int T, int C, int max_polls) {
  using F = Bwd<E, VEC, L, W, GATE>;
  using PackT = typename F::PackT;
  __shared__ typename F::Smem sm;

  const int nseg = (T + F::SEG - 1) / F::SEG;
  const int seg = nseg - 1 - __builtin_amdgcn_readfirstlane(int(blockIdx.x) / rows);
  const int row = int(blockIdx.x) - (nseg - 1 - seg) * rows;
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
  const size_t ck_field = size_t(rows / n_cg) * nblk * C;
  const size_t ck_row = size_t(b) * nblk * C + size_t(cg) * F::CPW;
  const unsigned ck_boff = active ? unsigned(lane * VEC * sizeof(float)) : 0u;
  const int t0 = (seg * W + wave) * L;

  // Rows the forward kernels recomputed with their exact path carry o != 0
  // in their block-0 records: the fix-up kernel handles them.
  bool serial = false;
  {
    Pack<F32, VEC> o;
    o.load(byte_offset(ck + ck_row, ck_boff));
#pragma unroll
    for (int c = 0; c < VEC; ++c) serial |= active && o.x[c] != 0.f;
  }
  if (__syncthreads_or(serial) != 0) return;

  PackT kb[L], vb[L], gb[L], xb[L];
  typename F::Recs rc;
  F::load(k, v, gy, r, ck, ck_row, ck_boff, ck_field, seg, row_base, row_tail, lane_boff, t0, C,
          kb, vb, gb, xb, rc);

  float D[VEC], DL[VEC], DS[VEC], U[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    const float dv = active ? decay[c0 + c] : 0.f;
    const float uv = active ? u_in[c0 + c] : 0.f;
    const float w2 = (decay_is_w ? dv : -expf(dv)) * kLog2e;
    D[c] = fast_exp2(w2);
    DL[c] = fast_exp2(w2 * float(L));
    DS[c] = fast_exp2(w2 * float(F::SEG));
    U[c] = fast_exp2(uv * kLog2e);
  }
  typename F::Weights Wt;
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    float pw = D[c];
#pragma unroll
    for (int i = 1; i < L; ++i) {
      Wt.d0[i - 1][c] = pw;
      pw *= D[c];
    }
  }

  const bool full = (seg + 1) * F::SEG <= T;
  float P[VEC], Q[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    P[c] = rc.p[c];
    Q[c] = rc.q[c];
  }
  float ek[L][VEC];
  float ps[VEC], qs[VEC];
  if (full)
    F::template summarize<true>(t0, T, kb, vb, D, ek, ps, qs);
  else
    F::template summarize<false>(t0, T, kb, vb, D, ek, ps, qs);
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    sm.p[c][wave][lane] = ps[c];
    sm.q[c][wave][lane] = qs[c];
  }
  __syncthreads();
  for (int w = 0; w < wave; ++w) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      P[c] = fmaf(P[c], DL[c], sm.p[c][w][lane]);
      Q[c] = fmaf(Q[c], DL[c], sm.q[c][w][lane]);
    }
  }
  float zz[L][VEC], zy[L][VEC], pa[L][VEC], qa[L][VEC];
  float G[VEC], H[VEC];
  if (full)
    F::template recompute<true>(t0, T, C, active, row_base, row_tail, lane_boff, vb, gb, xb, ek, D,
                                U, Wt, P, Q, zz, zy, pa, qa, gr, G, H);
  else
    F::template recompute<false>(t0, T, C, active, row_base, row_tail, lane_boff, vb, gb, xb, ek,
                                 D, U, Wt, P, Q, zz, zy, pa, qa, gr, G, H);
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    sm.G[c][wave][lane] = G[c];
    sm.H[c][wave][lane] = H[c];
  }
  __syncthreads();

  if (wave == 0) {
    const size_t plane = size_t(nseg) * rows * F::CPW;  // words per kind
    uint64_t* const mine = lb + (size_t(seg) * rows + row) * F::CPW + lane * VEC;
    // This segment's reverse sums from a zero state at its end.
    float ag[VEC], ah[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) { ag[c] = 0.f; ah[c] = 0.f; }
    for (int w = W - 1; w >= 0; --w) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        ag[c] = fmaf(DL[c], ag[c], sm.G[c][w][lane]);
        ah[c] = fmaf(DL[c], ah[c], sm.H[c][w][lane]);
      }
    }
#pragma unroll
    for (int c = 0; c < VEC; ++c) lb_store(mine + c, lb_pack(ag[c], ah[c]));
    float rg[VEC], rh[VEC];
    const uint64_t* base = lb + size_t(row) * F::CPW + lane * VEC;
    const bool gave_up = !lb_window_carry<VEC>(base, base + plane, size_t(rows) * F::CPW, seg,
                                               nseg, -1, DS, rg, rh, max_polls);
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      lb_store(mine + plane + c, lb_pack(fmaf(DS[c], rg[c], ag[c]), fmaf(DS[c], rh[c], ah[c])));
      sm.rcarry[0][0][c][lane] = rg[c];
      sm.rcarry[0][1][c][lane] = rh[c];
    }
    if (__any(gave_up) && lane == 0) mark_row_redo(status, row);
  }
  __syncthreads();

  // Carry at this chunk's end: the segment's carry, then the later chunks.
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    G[c] = sm.rcarry[0][0][c][lane];
    H[c] = sm.rcarry[0][1][c][lane];
  }
  for (int w = W - 1; w > wave; --w) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      G[c] = fmaf(DL[c], G[c], sm.G[c][w][lane]);
      H[c] = fmaf(DL[c], H[c], sm.H[c][w][lane]);
    }
  }
  float gw[VEC], gu[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) { gw[c] = 0.f; gu[c] = 0.f; }
  F::reverse(t0, C, active, row_base, row_tail, lane_boff, vb, ek, zz, zy, pa, qa, D, U, G, H, gk,
             gv, gw, gu);

  // gw, gu of this (batch, segment) reduced over the waves.
  __syncthreads();
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    sm.G[c][wave][lane] = gw[c] * D[c];
    sm.H[c][wave][lane] = gu[c] * U[c];
  }
  __syncthreads();
  const size_t slot = (size_t(b) * nseg + seg) * C;
  for (int ch = threadIdx.x; ch < F::CPW; ch += blockDim.x) {
    const int c = cg * F::CPW + ch;
    if (c >= C) continue;
    const int l = ch / VEC, s = ch - l * VEC;
    float sw = 0.f, su = 0.f;
    for (int w = 0; w < W; ++w) {
      sw += sm.G[s][w][l];
      su += sm.H[s][w][l];
    }
    gw_part[slot + c] = sw;
    gu_part[slot + c] = su;
  }
}

// After the split backward: per row, its gw, gu summed over the segments in
// a fixed order into the [B][C] partials (gw_b, gu_b) that
// wkv4_param_grad_kernel sums over the batch.  Rows the split kernel left
// (the forward's exact rows, and rows whose look-back gave up) are first
// recomputed with the exact serial path, which writes gk, gv (and grad_r)
// over the whole row and gives the row's sums directly.  One wave per row.
template <typename E, bool GATE>
__global__ __launch_bounds__(64) void wkv4_bwd_fixup_kernel(
    const typename E::raw* __restrict__ gy, const float* __restrict__ decay, int decay_is_w,
    const float* __restrict__ u_in, const typename E::raw* __restrict__ k,
    const typename E::raw* __restrict__ v, const typename E::raw* __restrict__ r,
    const float* __restrict__ ck, typename E::raw* __restrict__ gk,
    typename E::raw* __restrict__ gv, typename E::raw* __restrict__ gr,
    const float* __restrict__ gw_seg, const float* __restrict__ gu_seg,
    float* __restrict__ gw_b, float* __restrict__ gu_b, const uint32_t* __restrict__ status,
    int cpw, int n_cg, int nseg, int T, int C) {
  const int row = blockIdx.x;
  const int b = row / n_cg;
  const int cg = row - b * n_cg;
  const int nblk = (T + kCkptBlock - 1) / kCkptBlock;
  const size_t ck_field = size_t(gridDim.x / n_cg) * nblk * C;
  bool redo = status[row] != kRowOk;
  for (int ch = threadIdx.x; ch < cpw; ch += 64) {
    const int c = cg * cpw + ch;
    if (c < C) redo |= ck[size_t(b) * nblk * C + c] != 0.f;
  }
  redo = __any(redo);
  for (int ch = threadIdx.x; ch < cpw; ch += 64) {
    const int c = cg * cpw + ch;
    if (c >= C) continue;
    float sw = 0.f, su = 0.f;
    if (redo) {
      const float w2 = (decay_is_w ? decay[c] : -expf(decay[c])) * kLog2e;
      wkv4_bwd_channel_serial<E, 8>(gy, k, v, GATE ? r : nullptr, gk, gv, GATE ? gr : nullptr,
                                    w2, u_in[c] * kLog2e, T, C, size_t(b) * T * C + c, ck,
                                    size_t(b) * nblk * C + c, ck_field, sw, su);
    } else {
      const float* pw = gw_seg + size_t(b) * nseg * C + c;
      const float* pu = gu_seg + size_t(b) * nseg * C + c;
#pragma unroll 8
      for (int sg = 0; sg < nseg; ++sg) {
        sw += pw[size_t(sg) * C];
        su += pu[size_t(sg) * C];
      }
    }
    gw_b[size_t(b) * C + c] = sw;
    gu_b[size_t(b) * C + c] = su;
  }
}

// grad_time_decay[c] = sum_b gw[b,c] * w[c] (chain rule through
// w = -exp(time_decay), applied per batch element as the reference does,
// wkv_triton.py:117,194); grad_time_first[c] = sum_b gu[b,c].  A block
// covers 64 channels with 16 threads per channel, each summing every 16th
// batch row; the 16 partials are added in a fixed tree order
// (deterministic).
__global__ __launch_bounds__(1024) void wkv4_param_grad_kernel(
    const float* __restrict__ gw_part, const float* __restrict__ gu_part,
    const float* __restrict__ decay, int decay_is_w, float* __restrict__ gtd,
    float* __restrict__ gtf, int B, int C) {
  constexpr int G = 16;
  __shared__ float sw[G][64], su[G][64];
  const int lane = threadIdx.x & 63;
  const int grp = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  float aw = 0.f, au = 0.f;
  if (c < C) {
    const float wc = decay_is_w ? decay[c] : -expf(decay[c]);
#pragma unroll 4
    for (int b = grp; b < B; b += G) {
      aw += gw_part[size_t(b) * C + c] * wc;
      au += gu_part[size_t(b) * C + c];
    }
  }
  sw[grp][lane] = aw;
  su[grp][lane] = au;
  __syncthreads();
  for (int h = G / 2; h > 0; h >>= 1) {
    if (grp < h) {
      sw[grp][lane] += sw[grp + h][lane];
      su[grp][lane] += su[grp + h][lane];
    }
    __syncthreads();
  }
  if (grp == 0 && c < C) {
    gtd[c] = sw[0][lane];
    gtf[c] = su[0][lane];
  }
}

// Fills the [C] parameter gradients with zeros (empty batch or sequence).
__global__ void wkv4_zero2_kernel(float* a, float* b, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) { a[i] = 0.f; b[i] = 0.f; }
}

}  // namespace wkv

// ------------------------------------------------------------ launcher ----
namespace wkv_host {

// Tile configurations compiled into the library (selectable with
// WKV_BWD_CFG="vec,L,W" for measurement).  SEG = W*L must be a multiple of
// the 64-step checkpoint block.  Defaults: (2,8,8) for 16-bit tensors with
// enough rows of 128 channels to fill the chip; for one channel per lane,
// (1,8,16) when at most one workgroup per CU exists (256 rows of 64
// channels or fewer: four waves per SIMD without the segment prefetch,
// 4-9 % faster than (1,8,8) at B=16 C=768 and B=24 T=3072), else (1,8,8)
// (1 % faster at 512 rows).  The other W=16 configurations are capped at
// 128 VGPRs and spill.
static constexpr TileCfg kBwdCfgs[] = {{2, 8, 8}, {1, 8, 16}, {2, 4, 16}, {1, 16, 8}, {1, 8, 8},
                                        {1, 16, 4}, {2, 16, 4}};
// Tile configurations of the split kernel (WKV_BWD_SPLIT_CFG).
static constexpr TileCfg kBwdSplitCfgs[] = {{1, 8, 8}, {1, 16, 4}, {1, 8, 16}, {2, 8, 8},
                                             {1, 4, 16}, {2, 4, 16}};

static TileCfg pick_bwd_cfg(int64_t B, int64_t C, int elem_bytes) {
  int vec, L, W;
  if (env_cfg("WKV_BWD_CFG", vec, L, W)) {
    for (const TileCfg& c : kBwdCfgs)
      if (c.vec == vec && c.L == L && c.W == W && (vec == 1 || C % 2 == 0)) return c;
  }
  if (elem_bytes == 2 && pick_vec(B, C) == 2) return TileCfg{2, 8, 8};
  return B * ((C + 63) / 64) <= 256 ? TileCfg{1, 8, 16} : TileCfg{1, 8, 8};
}

// The split kernel runs on the same condition as the forward's (few rows,
// at least two segments); {0, 0, 0} when the one-row kernel runs.
static TileCfg pick_bwd_split_cfg(int64_t B, int64_t T, int64_t C) {
  TileCfg cfg{1, 16, 4};
  int vec, L, W;
  if (env_cfg("WKV_BWD_SPLIT_CFG", vec, L, W)) {
    for (const TileCfg& c : kBwdSplitCfgs)
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

size_t wkv4_checkpoint_floats(int64_t B, int64_t T, int64_t C) {
  return size_t(wkv::kCkptFields) * size_t(B) * size_t((T + wkv::kCkptBlock - 1) / wkv::kCkptBlock) *
         size_t(C);
}

size_t wkv4_partials_floats(int64_t B, int64_t C) { return 2 * size_t(B) * size_t(C); }

static size_t round16(size_t n) { return (n + 15) / 16 * 16; }

// Workspace of the split backward: [2][B][C] and [2][B * nseg][C] fp32
// partials, then the look-back words and the row status words.
static size_t split_bwd_bytes(const TileCfg& cfg, int64_t B, int64_t T, int64_t C) {
  const int64_t cpw = 64 * cfg.vec;
  const int64_t rows = B * ((C + cpw - 1) / cpw);
  const int64_t nseg = (T + cfg.L * cfg.W - 1) / (cfg.L * cfg.W);
  const size_t words = size_t(2) * size_t(nseg) * size_t(rows) * size_t(cpw);
  return round16(wkv4_partials_floats(B, C) * 4) + round16(wkv4_partials_floats(B * nseg, C) * 4) +
         words * 8 + round16(size_t(rows) * 4);
}

// Workspace of a backward from records: the split kernel's when it runs,
// else the [2][B][C] partials.
size_t wkv4_bwd_ck_workspace_bytes_impl(int64_t B, int64_t T, int64_t C) {
  const TileCfg sc = pick_bwd_split_cfg(B, T, C);
  const size_t plain = round16(wkv4_partials_floats(B, C) * 4);
  return sc.vec == 0 ? plain : std::max(plain, split_bwd_bytes(sc, B, T, C));
}

// r, gr (both null or both given): the gated backward (forward y = sigmoid(r)
// * wkv, grad_r written to gr).
template <typename E, int VEC, int L, int W>
static int launch_bwd(const void* gy, const float* decay, int decay_is_w, const float* u,
                      const void* k, const void* v, const void* r, const float* ck, void* gk,
                      void* gv, void* gr, float* gtd, float* gtf, float* partials, int B, int T,
                      int C, hipStream_t stream) {
  using raw = typename E::raw;
  float* gw_part = partials;
  float* gu_part = partials + size_t(B) * C;
  const int n_cg = (C + 64 * VEC - 1) / (64 * VEC);
  const dim3 grid(unsigned(B) * n_cg), block(W * 64);
  const raw* g_ = static_cast<const raw*>(gy);
  const raw* k_ = static_cast<const raw*>(k);
  const raw* v_ = static_cast<const raw*>(v);
  const raw* r_ = static_cast<const raw*>(r);
  if (r != nullptr) {
    launch(wkv::wkv4_bwd_kernel<E, VEC, L, W, true>, grid, block, stream, false, g_, decay,
           decay_is_w, u, k_, v_, r_, ck, static_cast<raw*>(gk), static_cast<raw*>(gv),
           static_cast<raw*>(gr), gw_part, gu_part, T, C);
  } else {
    launch(wkv::wkv4_bwd_kernel<E, VEC, L, W, false>, grid, block, stream, false, g_, decay,
           decay_is_w, u, k_, v_, r_, ck, static_cast<raw*>(gk), static_cast<raw*>(gv),
           static_cast<raw*>(nullptr), gw_part, gu_part, T, C);
  }
  int rc = check_launch("wkv4_bwd_kernel");
  if (rc) return rc;
  launch(wkv::wkv4_param_grad_kernel, dim3((C + 63) / 64), dim3(1024), stream, true,
                     gw_part, gu_part, decay, decay_is_w, gtd, gtf, B, C);
  return check_launch("wkv4_param_grad_kernel");
}

template <typename E, int VEC, int L, int W>
static int launch_bwd_split(const void* gy, const float* decay, int decay_is_w, const float* u,
                            const void* k, const void* v, const void* r, const float* ck,
                            void* gk, void* gv, void* gr, float* gtd, float* gtf, void* ws, int B,
                            int T, int C, hipStream_t stream) {
  using raw = typename E::raw;
  constexpr int CPW = 64 * VEC;
  const int n_cg = (C + CPW - 1) / CPW;
  const int rows = B * n_cg;
  const int nseg = (T + L * W - 1) / (L * W);
  const size_t b_bytes = round16(wkv4_partials_floats(B, C) * 4);
  const size_t seg_bytes = round16(wkv4_partials_floats(int64_t(B) * nseg, C) * 4);
  float* gw_b = static_cast<float*>(ws);
  float* gu_b = gw_b + size_t(B) * C;
  float* gw_part = reinterpret_cast<float*>(static_cast<char*>(ws) + b_bytes);
  float* gu_part = gw_part + size_t(B) * nseg * C;
  uint64_t* lb = reinterpret_cast<uint64_t*>(static_cast<char*>(ws) + b_bytes + seg_bytes);
  const size_t words = size_t(2) * nseg * rows * CPW;
  uint32_t* status = reinterpret_cast<uint32_t*>(lb + words);
  if (int rc = lb_fill(lb, words * 8 + round16(size_t(rows) * 4), stream)) return rc;
  const raw* g_ = static_cast<const raw*>(gy);
  const raw* k_ = static_cast<const raw*>(k);
  const raw* v_ = static_cast<const raw*>(v);
  const raw* r_ = static_cast<const raw*>(r);
  raw* gk_ = static_cast<raw*>(gk);
  raw* gv_ = static_cast<raw*>(gv);
  raw* gr_ = static_cast<raw*>(gr);
  const dim3 grid(unsigned(nseg) * unsigned(rows)), block(W * 64);
  if (r != nullptr) {
    launch(wkv::wkv4_bwd_split_kernel<E, VEC, L, W, true>, grid, block, stream, false, g_, decay,
           decay_is_w, u, k_, v_, r_, ck, gk_, gv_, gr_, gw_part, gu_part, lb, status, rows, T, C,
           lb_poll_limit());
  } else {
    launch(wkv::wkv4_bwd_split_kernel<E, VEC, L, W, false>, grid, block, stream, false, g_, decay,
           decay_is_w, u, k_, v_, r_, ck, gk_, gv_, static_cast<raw*>(nullptr), gw_part, gu_part,
           lb, status, rows, T, C, lb_poll_limit());
  }
  if (int rc = check_launch("wkv4_bwd_split_kernel")) return rc;
  if (r != nullptr) {
    launch(wkv::wkv4_bwd_fixup_kernel<E, true>, dim3(rows), dim3(64), stream, false, g_, decay,
           decay_is_w, u, k_, v_, r_, ck, gk_, gv_, gr_, gw_part, gu_part, gw_b, gu_b, status,
           CPW, n_cg, nseg, T, C);
  } else {
    launch(wkv::wkv4_bwd_fixup_kernel<E, false>, dim3(rows), dim3(64), stream, false, g_, decay,
           decay_is_w, u, k_, v_, r_, ck, gk_, gv_, static_cast<raw*>(nullptr), gw_part, gu_part,
           gw_b, gu_b, status, CPW, n_cg, nseg, T, C);
  }
  if (int rc = check_launch("wkv4_bwd_fixup_kernel")) return rc;
  launch(wkv::wkv4_param_grad_kernel, dim3((C + 63) / 64), dim3(1024), stream, true, gw_b, gu_b,
         decay, decay_is_w, gtd, gtf, B, C);
  return check_launch("wkv4_param_grad_kernel");
}

// ws: the workspace (at least the [2][B][C] partials); the split kernel runs
// when it is eligible and ws holds its workspace.
template <typename E>
static int dispatch_bwd(const void* gy, const float* decay, int decay_is_w, const float* u,
                        const void* k, const void* v, const void* r, const float* ck, void* gk,
                        void* gv, void* gr, float* gtd, float* gtf, void* ws, size_t ws_bytes,
                        int B, int T, int C, hipStream_t stream) {
  const TileCfg sc = pick_bwd_split_cfg(B, T, C);
  if (sc.vec != 0 && ws_bytes >= split_bwd_bytes(sc, B, T, C)) {
#define WKV_BWD_SPLIT_CASE(V, LL, WW)                                                        \
  if (sc.vec == V && sc.L == LL && sc.W == WW)                                              \
    return launch_bwd_split<E, V, LL, WW>(gy, decay, decay_is_w, u, k, v, r, ck, gk, gv, gr, \
                                          gtd, gtf, ws, B, T, C, stream);
    WKV_BWD_SPLIT_CASE(1, 8, 8)
    WKV_BWD_SPLIT_CASE(1, 16, 4)
    WKV_BWD_SPLIT_CASE(1, 8, 16)
    WKV_BWD_SPLIT_CASE(2, 8, 8)
    WKV_BWD_SPLIT_CASE(1, 4, 16)
    WKV_BWD_SPLIT_CASE(2, 4, 16)
#undef WKV_BWD_SPLIT_CASE
  }
  float* partials = static_cast<float*>(ws);
  const TileCfg cfg = pick_bwd_cfg(B, C, int(sizeof(typename E::raw)));
#define WKV_BWD_CASE(V, LL, WW)                                                                \
  if (cfg.vec == V && cfg.L == LL && cfg.W == WW)                                              \
    return launch_bwd<E, V, LL, WW>(gy, decay, decay_is_w, u, k, v, r, ck, gk, gv, gr, gtd, gtf, \
                                    partials, B, T, C, stream);
  WKV_BWD_CASE(2, 8, 8)
  WKV_BWD_CASE(1, 8, 16)
  WKV_BWD_CASE(2, 4, 16)
  WKV_BWD_CASE(1, 16, 8)
  WKV_BWD_CASE(1, 8, 8)
  WKV_BWD_CASE(1, 16, 4)
  WKV_BWD_CASE(2, 16, 4)
#undef WKV_BWD_CASE
  return fail(1, "wkv4_backward: no kernel for the selected tile configuration");
}

static int backward_any(const void* gy, const float* decay, int decay_is_w, const float* u,
                        const void* k, const void* v, const void* r, const float* ck, void* gk,
                        void* gv, void* gr, float* gtd, float* gtf, void* ws, size_t ws_bytes,
                        int B, int T, int C, int dtype, hipStream_t stream) {
  switch (dtype) {
    case 0:
      return dispatch_bwd<wkv::F32>(gy, decay, decay_is_w, u, k, v, r, ck, gk, gv, gr, gtd, gtf,
                                    ws, ws_bytes, B, T, C, stream);
    case 1:
      return dispatch_bwd<wkv::BF16>(gy, decay, decay_is_w, u, k, v, r, ck, gk, gv, gr, gtd, gtf,
                                     ws, ws_bytes, B, T, C, stream);
    case 2:
      return dispatch_bwd<wkv::F16>(gy, decay, decay_is_w, u, k, v, r, ck, gk, gv, gr, gtd, gtf,
                                    ws, ws_bytes, B, T, C, stream);
    default:
      return fail(1, "wkv4_backward: unknown dtype");
  }
}

// Backward from checkpoint records ck (written by the forward kernel).
int wkv4_backward_ck_impl(const void* gy, const float* decay, int decay_is_w, const float* u,
                          const void* k, const void* v, const float* ck, void* gk, void* gv,
                          float* gtd, float* gtf, void* ws, size_t ws_bytes, int B, int T, int C,
                          int dtype, hipStream_t stream) {
  return backward_any(gy, decay, decay_is_w, u, k, v, nullptr, ck, gk, gv, nullptr, gtd, gtf, ws,
                      ws_bytes, B, T, C, dtype, stream);
}

// The gated backward from checkpoint records: g is the gradient of
// y = sigmoid(r) * wkv; writes grad_r besides grad_k, grad_v and the
// parameter gradients.
int wkv4_backward_gated_ck_impl(const void* g, const float* decay, const float* u, const void* k,
                                const void* v, const void* r, const float* ck, void* gk,
                                void* gv, void* gr, float* gtd, float* gtf, void* ws,
                                size_t ws_bytes, int B, int T, int C, int dtype,
                                hipStream_t stream) {
  return backward_any(g, decay, 0, u, k, v, r, ck, gk, gv, gr, gtd, gtf, ws, ws_bytes, B, T, C,
                      dtype, stream);
}

// Workspace of wkv4_backward_impl: the checkpoint records, then what the
// forward (split) and the backward from the records need (used one after the
// other, so they share the space).  The minimum: records and the one-row
// kernels' partials.
size_t wkv4_bwd_workspace_bytes_impl(int64_t B, int64_t T, int64_t C, int dtype) {
  (void)dtype;
  return round16(wkv4_checkpoint_floats(B, T, C) * 4) +
         std::max(wkv4_fwd_workspace_bytes_impl(B, T, C), wkv4_bwd_ck_workspace_bytes_impl(B, T, C));
}

size_t wkv4_bwd_min_workspace_bytes_impl(int64_t B, int64_t T, int64_t C) {
  return round16(wkv4_checkpoint_floats(B, T, C) * 4) + round16(wkv4_partials_floats(B, C) * 4);
}

// Backward from the inputs alone: the forward kernel writes the checkpoint
// records (no y) into the workspace, then the reverse sweep runs.
int wkv4_backward_impl(const void* gy, const float* w, const float* u, const void* k,
                       const void* v, void* gk, void* gv, float* gtd, float* gtf, void* ws,
                       size_t ws_bytes, int B, int T, int C, int dtype, hipStream_t stream) {
  const size_t ck_bytes = round16(wkv4_checkpoint_floats(B, T, C) * 4);
  float* ck = static_cast<float*>(ws);
  void* rest = static_cast<char*>(ws) + ck_bytes;
  const size_t rest_bytes = ws_bytes - ck_bytes;
  // The forward stage does not end the call: it carries no stop event.
  CallEvents& ev = active_events();
  hipEvent_t stop = ev.stop;
  if (ev.kernel < 0) ev.stop = nullptr;
  int rc = wkv4_forward_impl(k, v, w, 1, u, nullptr, ck, rest, rest_bytes, B, T, C, dtype, stream);
  ev.stop = stop;
  if (rc) return rc;
  return wkv4_backward_ck_impl(gy, w, 1, u, k, v, ck, gk, gv, gtd, gtf, rest, rest_bytes, B, T, C,
                               dtype, stream);
}

int wkv4_zero_param_grads(float* gtd, float* gtf, int C, hipStream_t stream) {
  if (C <= 0) return 0;
  launch(wkv::wkv4_zero2_kernel, dim3((C + 255) / 256), dim3(256), stream, true, gtd,
                     gtf, C);
  return check_launch("wkv4_zero2_kernel");
}

}  // namespace wkv_host
