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
// G'_{t-1} = e^w (G'_t + G_t) (same for H with z_t y_t).  The reference
// accumulates gw in its forward replay (dpdw/dqdw); accumulating it in the
// reverse sweep instead needs no extra forward state, so the forward can be
// recomputed from one small checkpoint per segment.
//
// Decomposition (rows, chunks and segments as in the forward kernel):
//   sweep 1 (forward in time, reads k and v): per segment, the shared base-2
//     frame R, the chunk summaries and the segment-final state; the state at
//     every segment start (frame R, p, q) is written to a checkpoint buffer
//     (12 B per channel per segment of W*L steps);
//   sweep 2 (backward in time, reads k, v and gy): per segment, each wave
//     recomputes e^{k-R} and its chunk summary, gets its chunk's forward
//     carry by an LDS Horner from the segment checkpoint, recomputes the
//     chunk's forward keeping z~ = gy/den~ and y in registers, reduces its
//     chunk's reverse sums from a zero state, exchanges them in LDS (reverse
//     Horner: G <- G_j + e^{Lw} G,  G' <- G'_j + e^{Lw}(G' + L G)), then runs
//     the reverse recurrence with that carry, writing gk and gv and
//     accumulating gw, gu.  gw/gu are reduced over the waves of the row into
//     [B, C] partials that a second small kernel sums over B in fixed order.
//
// Reverse sums live in the segment frame: G~ = 2^R G, so that
// e^{k_t} G_t = 2^{k_t log2e - R} G~_t and 2^R z_t = gy_t / den~_t.
//
// Range guard as in the forward kernel but tighter (the reverse sums scale
// with 1/den); a rejected row is recomputed one channel per thread with the
// reference's running-max recurrences (forward replay + stabilised reverse).
#include "wkv_common.h"

namespace wkv {

constexpr float kBwdMaxSpread = 64.f;
constexpr float kBwdMaxJump = 64.f;
constexpr float kBwdMaxU = 16.f;

// Serial recomputation of one channel with the reference's recurrences (base
// 2).  Forward replay stores the state at every segment start; the reverse
// pass walks segments last to first and, inside each, sub-chunks of L steps
// last to first: it replays the forward from the segment checkpoint to the
// sub-chunk, keeps the sub-chunk's y, 1/den and output exponent, and runs the
// stabilised reverse recurrence (wkv_triton.py:120-142, extended by the G',
// H' sums for gw) over it.  Quadratic in the sub-chunks per segment; only
// rows outside the shared-frame range take it.
template <typename E, int L, int SEG>
__device__ void wkv4_bwd_channel_serial(const typename E::raw* __restrict__ gy,
                                        const typename E::raw* __restrict__ k,
                                        const typename E::raw* __restrict__ v,
                                        typename E::raw* __restrict__ gk,
                                        typename E::raw* __restrict__ gv, float w2, float u2,
                                        int T, int C, size_t base, float* ckR, float* ckP,
                                        float* ckQ, size_t ck_base, float& gw_out,
                                        float& gu_out) {
  const int nseg = (T + SEG - 1) / SEG;
  {
    float o = kNegHuge, p = 0.f, q = 0.f;
    for (int t = 0; t < T; ++t) {
      if (t % SEG == 0) {
        const size_t ci = ck_base + size_t(t / SEG) * C;
        ckR[ci] = o;
        ckP[ci] = p;
        ckQ[ci] = q;
      }
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
  }
  float orr = kNegHuge, G = 0.f, H = 0.f, Gp = 0.f, Hp = 0.f;
  float gw = 0.f, gu = 0.f;
  for (int j = nseg - 1; j >= 0; --j) {
    const int seg0 = j * SEG;
    const int nsub = (min(T - seg0, SEG) + L - 1) / L;
    for (int m = nsub - 1; m >= 0; --m) {
      const size_t ci = ck_base + size_t(j) * C;
      float o = ckR[ci], p = ckP[ci], q = ckQ[ci];
      const int t0 = seg0 + m * L;
      for (int t = seg0; t < t0; ++t) {
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
          const float g = load_scalar<E>(gy + idx);
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

template <typename E, int VEC, int L, int W>
struct Bwd {
  using raw = typename E::raw;
  using PackT = Pack<E, VEC>;
  static constexpr int CPW = 64 * VEC;
  static constexpr int SEG = W * L;

  struct Smem {
    float mx[W][CPW];
    float p[W][CPW];
    float q[W][CPW];
    float G[W][CPW];
    float H[W][CPW];
    float Gp[W][CPW];
    float Hp[W][CPW];
    float fcarry[2][3][CPW];  // forward segment carry (R, p, q)
    float rcarry[2][5][CPW];  // reverse segment carry (R, G, H, G', H')
  };

  // row_base is wave-uniform (SGPRs), lane_off the lane's 32-bit offset;
  // steps past the end re-read step T-1 (masked in the arithmetic).
  __device__ static __forceinline__ void load2(const raw* __restrict__ k, const raw* __restrict__ v,
                                               size_t row_base, unsigned lane_off, int t0, int T,
                                               int C, PackT (&kb)[L], PackT (&vb)[L]) {
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const size_t step = row_base + size_t(min(t0 + i, T - 1)) * C;
      kb[i].load((k + step) + lane_off);
      vb[i].load((v + step) + lane_off);
    }
  }

  __device__ static __forceinline__ void load3(const raw* __restrict__ k, const raw* __restrict__ v,
                                               const raw* __restrict__ g, size_t row_base,
                                               unsigned lane_off, int t0, int T, int C,
                                               PackT (&kb)[L], PackT (&vb)[L], PackT (&gb)[L]) {
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const size_t step = row_base + size_t(min(t0 + i, T - 1)) * C;
      kb[i].load((k + step) + lane_off);
      vb[i].load((v + step) + lane_off);
      gb[i].load((g + step) + lane_off);
    }
  }

  // Sweep 1, one segment: checkpoint of the segment's starting state and the
  // segment-final carry.  Returns true (workgroup-uniform) if the range guard
  // rejects the segment.
  __device__ static __forceinline__ bool sweep1_segment(
      Smem& sm, int seg, int T, int wave, int lane, bool active, const PackT (&kb)[L],
      const PackT (&vb)[L], const float (&D)[VEC], const float (&DL)[VEC], bool u_ok,
      float* __restrict__ ckR, float* __restrict__ ckP, float* __restrict__ ckQ, size_t ck_seg) {
    const int t0 = (seg * W + wave) * L;
    float s[L][VEC];
    float m[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) m[c] = kNegHuge;
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const bool valid = active && (t0 + i) < T;
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        s[i][c] = kb[i].get(c) * kLog2e;
        m[c] = valid ? fmaxf(m[c], s[i][c]) : m[c];
      }
    }
#pragma unroll
    for (int c = 0; c < VEC; ++c) sm.mx[wave][lane * VEC + c] = m[c];
    __syncthreads();

    float R[VEC], pin[VEC], qin[VEC];
    bool bad = !u_ok;
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      float r = kNegHuge;
#pragma unroll
      for (int w = 0; w < W; ++w) r = fmaxf(r, sm.mx[w][lane * VEC + c]);
      R[c] = (r == kNegHuge) ? 0.f : r;
      if (seg > 0) {
        const float Rc = sm.fcarry[(seg - 1) & 1][0][lane * VEC + c];
        const float d = Rc - R[c];
        bad |= active && (d > kBwdMaxJump || d < -kBwdMaxJump);
        const float f = fast_exp2(d);
        pin[c] = sm.fcarry[(seg - 1) & 1][1][lane * VEC + c] * f;
        qin[c] = sm.fcarry[(seg - 1) & 1][2][lane * VEC + c] * f;
      } else {
        pin[c] = 0.f;
        qin[c] = 0.f;
      }
    }
    if (wave == 0 && active) {
      store_vec<F32, VEC>(ckR + ck_seg, R);
      store_vec<F32, VEC>(ckP + ck_seg, pin);
      store_vec<F32, VEC>(ckQ + ck_seg, qin);
    }
    float ps[VEC], qs[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) { ps[c] = 0.f; qs[c] = 0.f; }
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const bool valid = active && (t0 + i) < T;
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const float x = s[i][c] - R[c];
        bad |= valid && (x < -kBwdMaxSpread);
        const float e = valid ? fast_exp2(x) : 0.f;
        ps[c] = fmaf(ps[c], D[c], e * vb[i].get(c));
        qs[c] = fmaf(qs[c], D[c], e);
      }
    }
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      sm.p[wave][lane * VEC + c] = ps[c];
      sm.q[wave][lane * VEC + c] = qs[c];
    }
    if (__syncthreads_or(bad)) return true;
    if (wave == W - 1) {
      // Segment-final state: fold every chunk of the segment into the carry.
      for (int w = 0; w < W; ++w) {
#pragma unroll
        for (int c = 0; c < VEC; ++c) {
          pin[c] = fmaf(pin[c], DL[c], sm.p[w][lane * VEC + c]);
          qin[c] = fmaf(qin[c], DL[c], sm.q[w][lane * VEC + c]);
        }
      }
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        sm.fcarry[seg & 1][0][lane * VEC + c] = R[c];
        sm.fcarry[seg & 1][1][lane * VEC + c] = pin[c];
        sm.fcarry[seg & 1][2][lane * VEC + c] = qin[c];
      }
    }
    return false;
  }

  // Sweep 2, one segment (segments visited last to first).
  __device__ static __forceinline__ void sweep2_segment(
      Smem& sm, int seg, int nseg, int T, int C, int wave, int lane, bool active, size_t row_base,
      unsigned lane_off, const PackT (&kb)[L], const PackT (&vb)[L], const PackT (&gb)[L],
      const float (&D)[VEC], const float (&DL)[VEC], const float (&U)[VEC],
      const float* __restrict__ ckR, const float* __restrict__ ckP,
      const float* __restrict__ ckQ, size_t ck_seg, raw* __restrict__ gk, raw* __restrict__ gv,
      float (&gw)[VEC], float (&gu)[VEC]) {
    const int t0 = (seg * W + wave) * L;
    float R[VEC], P[VEC], Q[VEC];
    {
      Pack<F32, VEC> a, b, c;
      a.load(ckR + ck_seg);
      b.load(ckP + ck_seg);
      c.load(ckQ + ck_seg);
#pragma unroll
      for (int j = 0; j < VEC; ++j) { R[j] = a.x[j]; P[j] = b.x[j]; Q[j] = c.x[j]; }
    }
    // e^{k-R} and this chunk's forward summary from a zero state.
    float ek[L][VEC];
    float ps[VEC], qs[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) { ps[c] = 0.f; qs[c] = 0.f; }
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const bool valid = active && (t0 + i) < T;
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const float e = valid ? fast_exp2(fmaf(kb[i].get(c), kLog2e, -R[c])) : 0.f;
        ek[i][c] = e;
        ps[c] = fmaf(ps[c], D[c], e * vb[i].get(c));
        qs[c] = fmaf(qs[c], D[c], e);
      }
    }
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      sm.p[wave][lane * VEC + c] = ps[c];
      sm.q[wave][lane * VEC + c] = qs[c];
    }
    __syncthreads();
    for (int w = 0; w < wave; ++w) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        P[c] = fmaf(P[c], DL[c], sm.p[w][lane * VEC + c]);
        Q[c] = fmaf(Q[c], DL[c], sm.q[w][lane * VEC + c]);
      }
    }
    // Forward recompute: keep z~ = gy/den~ and y (zero past the end).
    float zz[L][VEC], yy[L][VEC];
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const bool valid = active && (t0 + i) < T;
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const float vv = vb[i].get(c);
        const float e = ek[i][c];
        const float e1 = e * U[c];
        const float r = fast_rcp(Q[c] + e1);
        zz[i][c] = valid ? gb[i].get(c) * r : 0.f;
        yy[i][c] = valid ? fmaf(e1, vv, P[c]) * r : 0.f;
        P[c] = fmaf(e, vv, P[c] * D[c]);
        Q[c] = fmaf(Q[c], D[c], e);
      }
    }
    // Reverse summary of this chunk from a zero state at its end.
    float G[VEC], H[VEC], Gp[VEC], Hp[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) { G[c] = 0.f; H[c] = 0.f; Gp[c] = 0.f; Hp[c] = 0.f; }
#pragma unroll
    for (int i = L - 1; i >= 0; --i) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const float z = zz[i][c];
        Gp[c] = (Gp[c] + G[c]) * D[c];
        Hp[c] = (Hp[c] + H[c]) * D[c];
        G[c] = fmaf(G[c], D[c], z);
        H[c] = fmaf(H[c], D[c], z * yy[i][c]);
      }
    }
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      sm.G[wave][lane * VEC + c] = G[c];
      sm.H[wave][lane * VEC + c] = H[c];
      sm.Gp[wave][lane * VEC + c] = Gp[c];
      sm.Hp[wave][lane * VEC + c] = Hp[c];
    }
    __syncthreads();
    // Carry at this chunk's end: the later segment's carry (converted to this
    // frame), then the later chunks of this segment, nearest last.
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      if (seg + 1 < nseg) {
        const int sl = (seg + 1) & 1;
        const float f = fast_exp2(R[c] - sm.rcarry[sl][0][lane * VEC + c]);
        G[c] = sm.rcarry[sl][1][lane * VEC + c] * f;
        H[c] = sm.rcarry[sl][2][lane * VEC + c] * f;
        Gp[c] = sm.rcarry[sl][3][lane * VEC + c] * f;
        Hp[c] = sm.rcarry[sl][4][lane * VEC + c] * f;
      } else {
        G[c] = 0.f; H[c] = 0.f; Gp[c] = 0.f; Hp[c] = 0.f;
      }
    }
    for (int w = W - 1; w > wave; --w) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const int ch = lane * VEC + c;
        Gp[c] = fmaf(DL[c], fmaf(float(L), G[c], Gp[c]), sm.Gp[w][ch]);
        Hp[c] = fmaf(DL[c], fmaf(float(L), H[c], Hp[c]), sm.Hp[w][ch]);
        G[c] = fmaf(DL[c], G[c], sm.G[w][ch]);
        H[c] = fmaf(DL[c], H[c], sm.H[w][ch]);
      }
    }
    // Reverse pass with outputs.
#pragma unroll
    for (int i = L - 1; i >= 0; --i) {
      const int t = t0 + i;
      float gko[VEC], gvo[VEC];
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const float vv = vb[i].get(c);
        const float e = ek[i][c];
        const float z = zz[i][c];
        const float ze = z * (e * U[c]);
        const float gkd = ze * (vv - yy[i][c]);
        gvo[c] = fmaf(e, G[c], ze);
        gko[c] = fmaf(e, fmaf(vv, G[c], -H[c]), gkd);
        gu[c] += gkd;
        gw[c] = fmaf(e, fmaf(vv, Gp[c], -Hp[c]), gw[c]);
        Gp[c] = (Gp[c] + G[c]) * D[c];
        Hp[c] = (Hp[c] + H[c]) * D[c];
        G[c] = fmaf(G[c], D[c], z);
        H[c] = fmaf(H[c], D[c], z * yy[i][c]);
      }
      if (active && t < T) {
        const size_t step = row_base + size_t(t) * C;
        store_vec<E, VEC>((gk + step) + lane_off, gko);
        store_vec<E, VEC>((gv + step) + lane_off, gvo);
      }
    }
    if (wave == 0) {
      const int sl = seg & 1;
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        sm.rcarry[sl][0][lane * VEC + c] = R[c];
        sm.rcarry[sl][1][lane * VEC + c] = G[c];
        sm.rcarry[sl][2][lane * VEC + c] = H[c];
        sm.rcarry[sl][3][lane * VEC + c] = Gp[c];
        sm.rcarry[sl][4][lane * VEC + c] = Hp[c];
      }
    }
  }
};

template <typename E, int VEC, int L, int W>
__global__ __launch_bounds__(W * 64) void wkv4_bwd_kernel(
    const typename E::raw* __restrict__ gy, const float* __restrict__ w_in,
    const float* __restrict__ u_in, const typename E::raw* __restrict__ k,
    const typename E::raw* __restrict__ v, typename E::raw* __restrict__ gk,
    typename E::raw* __restrict__ gv, float* __restrict__ ckR, float* __restrict__ ckP,
    float* __restrict__ ckQ, float* __restrict__ gw_part, float* __restrict__ gu_part, int T,
    int C) {
  using F = Bwd<E, VEC, L, W>;
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
  // Lanes past the last channel read channel 0 of the row (never stored).
  const unsigned lane_off = active ? unsigned(lane * VEC) : 0u;
  const int nseg = (T + F::SEG - 1) / F::SEG;
  // Checkpoint of segment s for this lane: ck + ck_row + s * C.
  const size_t ck_row = size_t(b) * nseg * C + (active ? c0 : 0);

  float D[VEC], DL[VEC], U[VEC];
  bool u_ok = true;
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    const float wv = active ? w_in[c0 + c] : 0.f;
    const float uv = active ? u_in[c0 + c] : 0.f;
    const float w2 = wv * kLog2e;
    const float u2 = uv * kLog2e;
    D[c] = fast_exp2(w2);
    DL[c] = fast_exp2(w2 * float(L));
    U[c] = fast_exp2(u2);
    u_ok &= fabsf(u2) <= kBwdMaxU;
  }

  bool bad = false;
  {
    PackT kA[L], vA[L], kB[L], vB[L];
    F::load2(k, v, row_base, lane_off, wave * L, T, C, kA, vA);
    for (int seg = 0; seg < nseg; seg += 2) {
      if (seg + 1 < nseg)
        F::load2(k, v, row_base, lane_off, (seg + 1) * F::SEG + wave * L, T, C, kB, vB);
      if (F::sweep1_segment(sm, seg, T, wave, lane, active, kA, vA, D, DL, u_ok, ckR, ckP, ckQ,
                            ck_row + size_t(seg) * C)) {
        bad = true;
        break;
      }
      if (seg + 1 >= nseg) break;
      if (seg + 2 < nseg)
        F::load2(k, v, row_base, lane_off, (seg + 2) * F::SEG + wave * L, T, C, kA, vA);
      if (F::sweep1_segment(sm, seg + 1, T, wave, lane, active, kB, vB, D, DL, u_ok, ckR, ckP,
                            ckQ, ck_row + size_t(seg + 1) * C)) {
        bad = true;
        break;
      }
    }
  }

  if (!bad) {
    float gw[VEC], gu[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) { gw[c] = 0.f; gu[c] = 0.f; }
    PackT kA[L], vA[L], gA[L], kB[L], vB[L], gB[L];
    const int last = nseg - 1;
    F::load3(k, v, gy, row_base, lane_off, last * F::SEG + wave * L, T, C, kA, vA, gA);
    for (int seg = last; seg >= 0; seg -= 2) {
      if (seg - 1 >= 0)
        F::load3(k, v, gy, row_base, lane_off, (seg - 1) * F::SEG + wave * L, T, C, kB, vB, gB);
      F::sweep2_segment(sm, seg, nseg, T, C, wave, lane, active, row_base, lane_off, kA, vA, gA,
                        D, DL, U, ckR, ckP, ckQ, ck_row + size_t(seg) * C, gk, gv, gw, gu);
      if (seg - 1 < 0) break;
      if (seg - 2 >= 0)
        F::load3(k, v, gy, row_base, lane_off, (seg - 2) * F::SEG + wave * L, T, C, kA, vA, gA);
      F::sweep2_segment(sm, seg - 1, nseg, T, C, wave, lane, active, row_base, lane_off, kB, vB,
                        gB, D, DL, U, ckR, ckP, ckQ, ck_row + size_t(seg - 1) * C, gk, gv, gw,
                        gu);
    }
    // Reduce gw/gu over the waves of the row (reusing the summary arrays).
    __syncthreads();
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      sm.G[wave][lane * VEC + c] = gw[c];
      sm.H[wave][lane * VEC + c] = gu[c];
    }
    __syncthreads();
    for (int ch = threadIdx.x; ch < F::CPW; ch += blockDim.x) {
      const int c = cg * F::CPW + ch;
      if (c >= C) continue;
      float sw = 0.f, su = 0.f;
      for (int w = 0; w < W; ++w) {
        sw += sm.G[w][ch];
        su += sm.H[w][ch];
      }
      gw_part[size_t(b) * C + c] = sw;
      gu_part[size_t(b) * C + c] = su;
    }
  } else {
    for (int ch = threadIdx.x; ch < F::CPW; ch += blockDim.x) {
      const int c = cg * F::CPW + ch;
      if (c >= C) continue;
      float sw, su;
      wkv4_bwd_channel_serial<E, L, F::SEG>(gy, k, v, gk, gv, w_in[c] * kLog2e,
                                            u_in[c] * kLog2e, T, C, size_t(b) * T * C + c, ckR,
                                            ckP, ckQ, size_t(b) * nseg * C + c, sw, su);
      gw_part[size_t(b) * C + c] = sw;
      gu_part[size_t(b) * C + c] = su;
    }
  }
}

// grad_time_decay[c] = sum_b gw[b,c] * w[c] (chain rule through
// w = -exp(time_decay), applied per batch element as the reference does,
// wkv_triton.py:117,194); grad_time_first[c] = sum_b gu[b,c].  Fixed
// summation order: deterministic.
__global__ void wkv4_param_grad_kernel(const float* __restrict__ gw_part,
                                       const float* __restrict__ gu_part,
                                       const float* __restrict__ w, float* __restrict__ gtd,
                                       float* __restrict__ gtf, int B, int C) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const float wc = w[c];
  float sw = 0.f, su = 0.f;
  for (int b = 0; b < B; ++b) {
    sw += gw_part[size_t(b) * C + c] * wc;
    su += gu_part[size_t(b) * C + c];
  }
  gtd[c] = sw;
  gtf[c] = su;
}

// Fills the [C] parameter gradients with zeros (empty batch or sequence).
__global__ void wkv4_zero2_kernel(float* a, float* b, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) { a[i] = 0.f; b[i] = 0.f; }
}

}  // namespace wkv

// ------------------------------------------------------------ launcher ----
namespace wkv_host {

struct BwdCfg { int vec, L, W; };

// Tile configurations compiled into the library (VGPR use without spills at
// 64*W threads per workgroup).
static constexpr BwdCfg kBwdCfgs[] = {{1, 8, 16}, {2, 4, 16}, {2, 8, 8}, {1, 4, 16}, {1, 16, 8}};

int pick_vec(int64_t B, int64_t C);
bool env_cfg(const char* name, int& vec, int& L, int& W);

static BwdCfg pick_bwd_cfg(int64_t B, int64_t C, int elem_bytes) {
  int vec, L, W;
  if (env_cfg("WKV_BWD_CFG", vec, L, W)) {
    for (const BwdCfg& c : kBwdCfgs)
      if (c.vec == vec && c.L == L && c.W == W && (vec == 1 || C % 2 == 0)) return c;
  }
  if (elem_bytes == 4) return BwdCfg{1, 8, 16};
  return pick_vec(B, C) == 2 ? BwdCfg{2, 4, 16} : BwdCfg{1, 4, 16};
}

static int elem_bytes_of(int dtype) { return dtype == 0 ? 4 : 2; }

size_t wkv4_bwd_workspace_bytes_impl(int64_t B, int64_t T, int64_t C, int dtype) {
  const BwdCfg cfg = pick_bwd_cfg(B, C, elem_bytes_of(dtype));
  const int64_t seg = int64_t(cfg.L) * cfg.W;
  const int64_t nseg = (T + seg - 1) / seg;
  const int64_t floats = 3 * B * nseg * C + 2 * B * C;
  return size_t(floats) * sizeof(float) + 256;
}

template <typename E, int VEC, int L, int W>
static int launch_bwd(const void* gy, const float* w, const float* u, const void* k,
                      const void* v, void* gk, void* gv, float* gtd, float* gtf, float* ws,
                      int B, int T, int C, hipStream_t stream) {
  using raw = typename E::raw;
  const int nseg = (T + L * W - 1) / (L * W);
  float* ckR = ws;
  float* ckP = ckR + size_t(B) * nseg * C;
  float* ckQ = ckP + size_t(B) * nseg * C;
  float* gw_part = ckQ + size_t(B) * nseg * C;
  float* gu_part = gw_part + size_t(B) * C;
  const int n_cg = (C + 64 * VEC - 1) / (64 * VEC);
  hipLaunchKernelGGL((wkv::wkv4_bwd_kernel<E, VEC, L, W>), dim3(unsigned(B) * n_cg),
                     dim3(W * 64), 0, stream, static_cast<const raw*>(gy), w, u,
                     static_cast<const raw*>(k), static_cast<const raw*>(v),
                     static_cast<raw*>(gk), static_cast<raw*>(gv), ckR, ckP, ckQ, gw_part,
                     gu_part, T, C);
  int rc = check_launch("wkv4_bwd_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(wkv::wkv4_param_grad_kernel, dim3((C + 255) / 256), dim3(256), 0, stream,
                     gw_part, gu_part, w, gtd, gtf, B, C);
  return check_launch("wkv4_param_grad_kernel");
}

template <typename E>
static int dispatch_bwd(const void* gy, const float* w, const float* u, const void* k,
                        const void* v, void* gk, void* gv, float* gtd, float* gtf, float* ws,
                        int B, int T, int C, hipStream_t stream) {
  const BwdCfg cfg = pick_bwd_cfg(B, C, int(sizeof(typename E::raw)));
#define WKV_BWD_CASE(V, LL, WW)                                                          \
  if (cfg.vec == V && cfg.L == LL && cfg.W == WW)                                        \
    return launch_bwd<E, V, LL, WW>(gy, w, u, k, v, gk, gv, gtd, gtf, ws, B, T, C, stream);
  WKV_BWD_CASE(1, 8, 16)
  WKV_BWD_CASE(2, 4, 16)
  WKV_BWD_CASE(2, 8, 8)
  WKV_BWD_CASE(1, 4, 16)
  WKV_BWD_CASE(1, 16, 8)
#undef WKV_BWD_CASE
  return fail(1, "wkv4_backward: no kernel for the selected tile configuration");
}

int wkv4_backward_impl(const void* gy, const float* w, const float* u, const void* k,
                       const void* v, void* gk, void* gv, float* gtd, float* gtf, float* ws,
                       int B, int T, int C, int dtype, hipStream_t stream) {
  switch (dtype) {
    case 0: return dispatch_bwd<wkv::F32>(gy, w, u, k, v, gk, gv, gtd, gtf, ws, B, T, C, stream);
    case 1: return dispatch_bwd<wkv::BF16>(gy, w, u, k, v, gk, gv, gtd, gtf, ws, B, T, C, stream);
    case 2: return dispatch_bwd<wkv::F16>(gy, w, u, k, v, gk, gv, gtd, gtf, ws, B, T, C, stream);
    default: return fail(1, "wkv4_backward: unknown dtype");
  }
}

int wkv4_zero_param_grads(float* gtd, float* gtf, int C, hipStream_t stream) {
  if (C <= 0) return 0;
  hipLaunchKernelGGL(wkv::wkv4_zero2_kernel, dim3((C + 255) / 256), dim3(256), 0, stream, gtd,
                     gtf, C);
  return check_launch("wkv4_zero2_kernel");
}

}  // namespace wkv_host
