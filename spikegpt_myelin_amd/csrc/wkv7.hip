// RWKV-7 DPLR ("diagonal plus low rank") recurrence, forward and backward,
// for gfx950.
//
// Per (batch, head) with head size N = 64 and state S[i][j] (i: value index,
// j: key index), for each step t:
//   sa_t = S_{t-1} a_t,
//   S_t  = S_{t-1} diag(w_t) + sa_t b_t^T + v_t k_t^T,
//   y_t  = S_t r_t.
// Row i evolves as  S_i <- S_i * w + (S_i . a) b + v_i k :  the 64 rows are
// independent recurrences that share the step's vectors.
//
// Backward (G = dL/dS_t, accumulated from the last step to the first):
//   G     += dy_t r_t^T                      dr_t = S_t^T dy_t
//   c      = G b_t                           dv_t = G k_t
//   dk_t   = G^T v_t                         db_t = G^T sa_t
//   dw_t   = colsum(G o S_{t-1})             da_t = S_{t-1}^T c
//   G     <- G diag(w_t) + c a_t^T           (dL/dS_{t-1}; after step 0, dL/dS_0)
//
// Forward layout.  The rows of a (batch, head) are split over kSplit = 4
// workgroups of 256 threads; lane (rg, cg) of wave wv (rg = lane / 16 is the
// 16-lane DPP row, cg = lane % 16) holds one row, columns 4 cg .. +3.
//
// Backward layout.  One 256-thread workgroup (4 waves) owns one (batch,
// head): lane (rg, cg) of wave wv holds the 4x4 block of the state (and of
// its gradient) at rows 16 wv + 4 rg .. +3 and columns 4 cg .. +3.  Sums
// over j (S a, S r, G k, G b) are in-thread over 4 columns, then a DPP
// butterfly across the 16 lanes of a DPP row (no LDS).  Sums over i (the
// key-indexed gradients) are in-thread over 4 rows, then two gfx950 permlane
// swaps across the 4 DPP rows of the wave, then LDS across the 4 waves once
// per sub-chunk (collected while the next sub-chunk is recomputed).  The
// step vectors of KC = 16 steps are staged in LDS as fp32 (double-buffered;
// the next block is loaded into registers while the current one is
// computed).  Arithmetic is fp32 on the vector ALUs; no matrix cores.
//
// Checkpoints.  The forward can write a record per KS-step sub-chunk
// ([B*H][ceil(T/KS)][64 + KS][64] fp32): rows 0-63 hold the state at the
// sub-chunk's start (record 0: the initial state), row 64 + s holds sa_t of
// its step s.  The backward walks the blocks last to first and, inside each,
// the sub-chunks last to first; each sub-chunk's forward is recomputed from
// its own record (no replay; sa_t read, not recomputed), holding the states
// in registers, then the reverse recurrence runs over it.
//
// The reference's RWKV-7 code was deleted
// (benchmarks/results/optimizer_wkv_experiments_5090.md:3); the output
// convention here (y_t = S_t r_t on the post-update state, no scale) is this
// library's own.
#include "wkv_common.h"

namespace wkv {
namespace w7 {

constexpr int kN = 64;          // head size
constexpr int kThreads = 256;   // threads per workgroup
constexpr int kKC = 16;         // steps per staged block
constexpr int kKS = 8;          // steps per checkpoint / backward sub-chunk (registers)
constexpr int kNSub = kKC / kKS;
// A checkpoint record: the state at the start of its kKS steps (rows 0-63)
// and, for each of those steps, sa_t = S_{t-1} a_t (rows 64 ..).
constexpr int kRecRows = kN + kKS;
constexpr int kRecFloats = kRecRows * kN;

__device__ __forceinline__ float as_f(unsigned u) { return __uint_as_float(u); }

// s_waitcnt vmcnt(0) (gfx9 encoding: expcnt and lgkmcnt fields at their
// maximum).  Placed after a conditional load of the loop-carried state, so
// the compiler's wait analysis sees nothing pending at the loop header;
// otherwise it keeps a vmcnt(0) inside the loop, which then waits for the
// next block's prefetch every block.
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }
__device__ __forceinline__ unsigned as_u(float f) { return __float_as_uint(f); }

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over the 16 lanes of a DPP row; every lane of the row receives the
// same bits (each step adds a value and its mirror partner, which commute):
// xor 1, xor 2 (quad permutes), then half-row mirror and row mirror.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  x += dpp<0x140>(x);  // row_mirror
  return x;
}

// Sums four per-lane values over the wave's four 16-lane rows.  Row r of the
// result holds the total of value r.  v_permlane32_swap exchanges the upper
// half of its first operand with the lower half of its second;
// v_permlane16_swap exchanges the odd rows of the first with the even rows
// of the second.
__device__ __forceinline__ float rows4_sum(float v0, float v1, float v2, float v3) {
  // rows of s1: [v0_0+v0_2, v0_1+v0_3, v2_0+v2_2, v2_1+v2_3]
  const auto p = __builtin_amdgcn_permlane32_swap(as_u(v0), as_u(v2), false, false);
  const float s1 = as_f(p[0]) + as_f(p[1]);
  // rows of s2: likewise for v1, v3
  const auto q = __builtin_amdgcn_permlane32_swap(as_u(v1), as_u(v3), false, false);
  const float s2 = as_f(q[0]) + as_f(q[1]);
  // row 0: s1_0 + s1_1 = sum v0; row 1: s2_0 + s2_1 = sum v1;
  // row 2: s1_2 + s1_3 = sum v2; row 3: s2_2 + s2_3 = sum v3
  const auto r = __builtin_amdgcn_permlane16_swap(as_u(s1), as_u(s2), false, false);
  return as_f(r[0]) + as_f(r[1]);
}

template <typename E, int NV>
struct Vecs {
  const typename E::raw* p[NV];
  // q must be the same in every lane of the wave: it is moved to a scalar
  // register, so the choice is a scalar select.  A per-lane index would make
  // the compiler fetch the pointer from the argument block with a vector
  // load, and the wait for that load would also wait for every store the
  // wave still has in flight.
  __device__ __forceinline__ const typename E::raw* pick(int q) const {
    q = __builtin_amdgcn_readfirstlane(q);
    const typename E::raw* r = p[0];
#pragma unroll
    for (int i = 1; i < NV; ++i) r = (q == i) ? p[i] : r;
    return r;
  }
};

// Loads KC steps of NV step vectors of one (batch, head) in 16-byte pieces
// into registers, then writes them to LDS as fp32 [NV][KC][64].  Steps past
// the end re-read step T-1 (never used).
template <typename E, int NV>
struct Stager {
  using raw = typename E::raw;
  static constexpr int EPP = 16 / int(sizeof(raw));  // elements per piece
  static constexpr int PPV = kN / EPP;               // pieces per step vector
  static constexpr int NP = NV * kKC * PPV;
  static constexpr int PPT = (NP + kThreads - 1) / kThreads;
  static_assert((kKC * PPV) % 64 == 0, "a wave's pieces come from one step vector");
  uint4 buf[PPT];

  __device__ __forceinline__ void load(const Vecs<E, NV>& src, int bi, int h, int t0, int T,
                                       int H) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int p = int(threadIdx.x) + k * kThreads;
      if (NP % kThreads == 0 || p < NP) {
        const int q = p / (kKC * PPV);
        const int rem = p - q * (kKC * PPV);
        const int s = rem / PPV;
        const int pc = rem - s * PPV;
        const int t = min(t0 + s, T - 1);
        const raw* base = src.pick(q) + ((size_t(bi) * T + t) * H + h) * kN + pc * EPP;
        buf[k] = *reinterpret_cast<const uint4*>(base);
      }
    }
  }

  __device__ __forceinline__ void store(float* lds) const {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int p = int(threadIdx.x) + k * kThreads;
      if (NP % kThreads == 0 || p < NP) {
        const int q = p / (kKC * PPV);
        const int rem = p - q * (kKC * PPV);
        const int s = rem / PPV;
        const int pc = rem - s * PPV;
        float* dst = lds + (q * kKC + s) * kN + pc * EPP;
        const uint32_t w[4] = {buf[k].x, buf[k].y, buf[k].z, buf[k].w};
        if constexpr (EPP == 4) {
          *reinterpret_cast<float4*>(dst) =
              make_float4(as_f(w[0]), as_f(w[1]), as_f(w[2]), as_f(w[3]));
        } else {
          float f[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (__is_same(E, BF16)) {
              f[2 * e] = __uint_as_float(w[e] << 16);
              f[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
            } else {
              f[2 * e] = f16_bits_to_float(w[e] & 0xffffu);
              f[2 * e + 1] = f16_bits_to_float(w[e] >> 16);
            }
          }
          *reinterpret_cast<float4*>(dst) = make_float4(f[0], f[1], f[2], f[3]);
          *reinterpret_cast<float4*>(dst + 4) = make_float4(f[4], f[5], f[6], f[7]);
        }
      }
    }
  }
};

// Index of each step vector in the staged block.
enum { QR = 0, QW = 1, QK = 2, QV = 3, QA = 4, QB = 5, QDY = 6, QSA = 7 };
constexpr int kStageVecs = 8;  // the seven inputs, then sa_t from the records

__device__ __forceinline__ float4 lds4(const float* stage, int q, int s, int j) {
  return *reinterpret_cast<const float4*>(stage + (q * kKC + s) * kN + j);
}

struct Lane {
  int wv, rg, cg, i0, j0;
  __device__ __forceinline__ Lane() {
    wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
    const int lane = int(threadIdx.x) & 63;
    rg = lane >> 4;
    cg = lane & 15;
    i0 = 16 * wv + 4 * rg;
    j0 = 4 * cg;
  }
};

// Staged vectors of one recomputed forward step (w, b, k on the lane's
// columns; v and sa on its rows).
struct FwdVecs {
  float4 w, b, k, v, sa;
  __device__ __forceinline__ void load(const float* stage, int s, int i0, int j0) {
    w = lds4(stage, QW, s, j0);
    b = lds4(stage, QB, s, j0);
    k = lds4(stage, QK, s, j0);
    v = lds4(stage, QV, s, i0);
    sa = lds4(stage, QSA, s, i0);
  }
};

// One forward step on the lane's 4x4 block: the next state So from Si
// (separate arrays, so that an unrolled sequence of steps keeps every state
// in its own registers without copies), with sa (S_{t-1} a) per row taken
// from the records, where the forward kernel stored the value it used.  The
// update is the forward's expression, so both produce the same state bits.
__device__ __forceinline__ void fwd_step(const float (&Si)[4][4], float (&So)[4][4],
                                         const FwdVecs& x) {
  const float w[4] = {x.w.x, x.w.y, x.w.z, x.w.w};
  const float b[4] = {x.b.x, x.b.y, x.b.z, x.b.w};
  const float k[4] = {x.k.x, x.k.y, x.k.z, x.k.w};
  const float v[4] = {x.v.x, x.v.y, x.v.z, x.v.w};
  const float sa[4] = {x.sa.x, x.sa.y, x.sa.z, x.sa.w};
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) So[r][c] = fmaf(Si[r][c], w[c], fmaf(sa[r], b[c], v[r] * k[c]));
}

__device__ __forceinline__ size_t state_off(int bh, int i, int j) {
  return (size_t(bh) * kN + i) * kN + j;
}

__device__ __forceinline__ void load_state(float (&S)[4][4], const float* src, const Lane& L) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float4 x = *reinterpret_cast<const float4*>(src + (L.i0 + r) * kN + L.j0);
    S[r][0] = x.x; S[r][1] = x.y; S[r][2] = x.z; S[r][3] = x.w;
  }
}

__device__ __forceinline__ void store_state(float* dst, const float (&S)[4][4], const Lane& L) {
#pragma unroll
  for (int r = 0; r < 4; ++r)
    *reinterpret_cast<float4*>(dst + (L.i0 + r) * kN + L.j0) =
        make_float4(S[r][0], S[r][1], S[r][2], S[r][3]);
}

// ---- forward layout: the 64 rows of a (batch, head) split over kSplit
// workgroups.  Rows are independent in the forward, so a workgroup owns
// kRows of them and needs only its own kRows entries of v and y.  Lane
// (wave wv, DPP row rg, cg) holds one row, 4 columns:
//   row = kRows * split + 4 wv + rg,   columns 4 cg .. +3.
// The per-row sums are the same in-thread 4-column sum and 16-lane DPP
// butterfly as the backward's recomputation (fwd_step), so both produce the
// same state bits.  Four times the waves of a 4x4-block layout: at
// B = 16, H = 12 that is 768 workgroups, three waves on every SIMD.
constexpr int kSplit = 4;
constexpr int kRows = kN / kSplit;   // 16 rows per workgroup: 4 waves x 4 DPP rows
static_assert(kRows == 4 * (kThreads / 64), "one row per DPP row of each wave");

// Staged block: the key-side vectors r, w, k, a, b as fp32 [5][kKC][64],
// then the workgroup's slice of v as [kKC][kRows].
enum { KR = 0, KW = 1, KK = 2, KA = 3, KB = 4 };
constexpr int kRowStage = 5 * kKC * kN + kKC * kRows;

template <typename E>
struct RowStager {
  using raw = typename E::raw;
  static constexpr int EPP = 16 / int(sizeof(raw));  // elements per 16-byte piece
  static constexpr int PPV = kN / EPP;               // pieces per key-side vector
  static constexpr int PPR = kRows / EPP;            // pieces of v per step
  static constexpr int NK = 5 * kKC * PPV;
  static constexpr int NP = NK + kKC * PPR;
  static constexpr int PPT = (NP + kThreads - 1) / kThreads;
  static_assert((kKC * PPV) % 64 == 0, "a wave's pieces come from one step vector");
  uint4 buf[PPT];

  // Vecs order is (r, w, k, v, a, b): key-side vector q is input q, or q + 1 past v.
  __device__ __forceinline__ void load(const Vecs<E, 6>& src, int bi, int h, int i0, int t0,
                                       int T, int H) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int p = int(threadIdx.x) + k * kThreads;
      if (p < NK) {
        const int q = p / (kKC * PPV);
        const int rem = p - q * (kKC * PPV);
        const int s = rem / PPV;
        const int pc = rem - s * PPV;
        const int t = min(t0 + s, T - 1);
        const raw* base = src.pick(q < 3 ? q : q + 1) + ((size_t(bi) * T + t) * H + h) * kN +
                          pc * EPP;
        buf[k] = *reinterpret_cast<const uint4*>(base);
      } else if (p < NP) {
        const int s = (p - NK) / PPR;
        const int pc = (p - NK) - s * PPR;
        const int t = min(t0 + s, T - 1);
        const raw* base = src.p[3] + ((size_t(bi) * T + t) * H + h) * kN + i0 + pc * EPP;
        buf[k] = *reinterpret_cast<const uint4*>(base);
      }
    }
  }

  __device__ __forceinline__ void store(float* lds) const {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int p = int(threadIdx.x) + k * kThreads;
      float* dst;
      if (p < NK) {
        const int q = p / (kKC * PPV);
        const int rem = p - q * (kKC * PPV);
        const int s = rem / PPV;
        const int pc = rem - s * PPV;
        dst = lds + (q * kKC + s) * kN + pc * EPP;
      } else if (p < NP) {
        const int s = (p - NK) / PPR;
        const int pc = (p - NK) - s * PPR;
        dst = lds + 5 * kKC * kN + s * kRows + pc * EPP;
      } else {
        continue;
      }
      const uint32_t w[4] = {buf[k].x, buf[k].y, buf[k].z, buf[k].w};
      if constexpr (EPP == 4) {
        *reinterpret_cast<float4*>(dst) =
            make_float4(as_f(w[0]), as_f(w[1]), as_f(w[2]), as_f(w[3]));
      } else {
        float f[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (__is_same(E, BF16)) {
            f[2 * e] = __uint_as_float(w[e] << 16);
            f[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
          } else {
            f[2 * e] = f16_bits_to_float(w[e] & 0xffffu);
            f[2 * e + 1] = f16_bits_to_float(w[e] >> 16);
          }
        }
        *reinterpret_cast<float4*>(dst) = make_float4(f[0], f[1], f[2], f[3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(f[4], f[5], f[6], f[7]);
      }
    }
  }
};

// One staged block of a workgroup's rows over n steps.  FULL (n == kKC)
// drops the per-step guards, so the whole block is one basic block and the
// LDS reads of later steps are free to overlap earlier steps' arithmetic.
// CK: copy the state at each kKS-step record start to rec (stored by the
// caller after the block: no global store is in flight while the block's
// arithmetic waits on LDS, and the wait for the next block's staging loads
// finds only old stores ahead of it).
template <bool FULL, bool CK>
__device__ __forceinline__ void fwd_rows_block(float (&S)[4], const float* sg, float* yb,
                                               float& my_sa, int n, float (&rec)[kNSub][4],
                                               int lr, int j0) {
#pragma unroll
  for (int s = 0; s < kKC; ++s) {
    if (FULL || s < n) {
      if (CK && s % kKS == 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c) rec[s / kKS][c] = S[c];
      }
      const float4 a4 = lds4(sg, KA, s, j0);
      const float4 w4 = lds4(sg, KW, s, j0);
      const float4 b4 = lds4(sg, KB, s, j0);
      const float4 k4 = lds4(sg, KK, s, j0);
      const float v = sg[5 * kKC * kN + s * kRows + lr];
      const float a[4] = {a4.x, a4.y, a4.z, a4.w};
      const float w[4] = {w4.x, w4.y, w4.z, w4.w};
      const float b[4] = {b4.x, b4.y, b4.z, b4.w};
      const float k[4] = {k4.x, k4.y, k4.z, k4.w};
      float x = S[0] * a[0];
#pragma unroll
      for (int c = 1; c < 4; ++c) x = fmaf(S[c], a[c], x);
      const float sa = row16_sum(x);
      // Every lane of the DPP row holds the row's sa; lane cg keeps step cg's.
      if (CK) my_sa = (j0 == 4 * s) ? sa : my_sa;
#pragma unroll
      for (int c = 0; c < 4; ++c) S[c] = fmaf(S[c], w[c], fmaf(sa, b[c], v * k[c]));
      const float4 r4 = lds4(sg, KR, s, j0);
      const float rr[4] = {r4.x, r4.y, r4.z, r4.w};
      float yv = S[0] * rr[0];
#pragma unroll
      for (int c = 1; c < 4; ++c) yv = fmaf(S[c], rr[c], yv);
      // The 16 lanes of the DPP row hold the same sum and store it to the
      // same word (no exec-mask branch inside the block).
      yb[s * kRows + lr] = row16_sum(yv);
    }
  }
}

// Workgroup -> ((batch, head), split).  Consecutive workgroups go to
// different XCDs (round robin over 8); when the grid is a multiple of 8 the
// mapping puts the kSplit workgroups of one (batch, head), which read the
// same key-side vectors, on the same XCD and so the same L2.
__device__ __forceinline__ int xcd_local_block() {
  const int g = int(blockIdx.x);
  const int G = int(gridDim.x);
  return (G & 7) ? g : (g & 7) * (G >> 3) + (g >> 3);
}

}  // namespace w7

// ------------------------------------------------------------- forward ----
// kSplit workgroups per (batch, head), kRows state rows each.  ck (optional):
// one record per kKS-step sub-chunk, [B*H][ceil(T/kKS)][kRecRows][64]: the
// state at its start and sa_t of its steps (each workgroup writes its rows).
// y may be null (records only).
template <typename E, bool CK>
__global__ __launch_bounds__(w7::kThreads) void wkv7_fwd_kernel(
    w7::Vecs<E, 6> in, const float* __restrict__ s0, typename E::raw* __restrict__ y,
    float* __restrict__ s_out, float* __restrict__ ck, int T, int H) {
  using namespace w7;
  __shared__ float stage[2][kRowStage];
  __shared__ float ybuf[2][kKC * kRows];
  const int g = xcd_local_block();
  const int bh = g / kSplit;
  const int i0 = (g - bh * kSplit) * kRows;
  const int bi = bh / H;
  const int h = bh - bi * H;
  const int wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int lane = int(threadIdx.x) & 63;
  const int cg = lane & 15;
  const int lr = 4 * wv + (lane >> 4);   // row within the workgroup's slice
  const int row = i0 + lr;
  const int j0 = 4 * cg;

  float S[4];
  if (s0) {
    const float4 x = *reinterpret_cast<const float4*>(s0 + state_off(bh, row, j0));
    S[0] = x.x; S[1] = x.y; S[2] = x.z; S[3] = x.w;
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) S[c] = 0.f;
  }
  wait_vmem_all();
  const int nblk = (T + kKC - 1) / kKC;
  const int nrec = (T + kKS - 1) / kKS;
  RowStager<E> st;
  if (nblk > 0) {
    st.load(in, bi, h, i0, 0, T, H);
    st.store(stage[0]);
    __syncthreads();
  }
  for (int blk = 0; blk < nblk; ++blk) {
    const int t0 = blk * kKC;
    const int n = min(kKC, T - t0);
    if (blk + 1 < nblk) st.load(in, bi, h, i0, t0 + kKC, T, H);
    const float* sg = stage[blk & 1];
    float* yb = ybuf[blk & 1];
    float rec[kNSub][4];
    float my_sa = 0.f;  // sa of step cg of the block (row `row`)
    static_assert(kKC == 16, "one step of sa per lane of a 16-lane DPP row");
    if (n == kKC) {
      fwd_rows_block<true, CK>(S, sg, yb, my_sa, n, rec, lr, j0);
    } else {
      fwd_rows_block<false, CK>(S, sg, yb, my_sa, n, rec, lr, j0);
    }
    if (blk + 1 < nblk) st.store(stage[(blk + 1) & 1]);
    if (CK) {
      float* ckr = ck + (size_t(bh) * nrec + blk * kNSub) * kRecFloats + row * kN + j0;
#pragma unroll
      for (int m = 0; m < kNSub; ++m)
        if (m * kKS < n)
          *reinterpret_cast<float4*>(ckr + m * kRecFloats) =
              make_float4(rec[m][0], rec[m][1], rec[m][2], rec[m][3]);
      // sa of step s = cg of the block into row kN + s mod kKS of its record;
      // the rows of steps past T in the last record hold zeros (so that the
      // records are fully written).
      const int s = j0 / 4;
      if (blk * kNSub + s / kKS < nrec)
        ck[(size_t(bh) * nrec + blk * kNSub + s / kKS) * kRecFloats + (kN + s % kKS) * kN + row] =
            s < n ? my_sa : 0.f;
    }
    __syncthreads();
    if (y) {
      // kRows outputs per step: PPR 16-byte pieces at (bi, t0 + s, h, i0 ..),
      // one piece per thread.
      constexpr int EPP = RowStager<E>::EPP;
      constexpr int PPR = RowStager<E>::PPR;
      static_assert(kKC * PPR <= kThreads, "one y piece per thread");
      const int p = int(threadIdx.x);
      if (p < n * PPR) {
        const int s = p / PPR;
        const int pc = p - s * PPR;
        const float* src = yb + s * kRows + pc * EPP;
        float f[EPP];
#pragma unroll
        for (int e = 0; e < EPP; e += 4) {
          const float4 x = *reinterpret_cast<const float4*>(src + e);
          f[e] = x.x; f[e + 1] = x.y; f[e + 2] = x.z; f[e + 3] = x.w;
        }
        typename E::raw* dst = y + ((size_t(bi) * T + t0 + s) * H + h) * kN + i0 + pc * EPP;
        if constexpr (EPP == 4) {
          *reinterpret_cast<float4*>(dst) = make_float4(f[0], f[1], f[2], f[3]);
        } else {
          OutPack<E, 8> o;
          o.set(f);
          *reinterpret_cast<uint4*>(dst) = make_uint4(o.u[0], o.u[1], o.u[2], o.u[3]);
        }
      }
    }
  }
  if (s_out)
    *reinterpret_cast<float4*>(s_out + state_off(bh, row, j0)) = make_float4(S[0], S[1], S[2], S[3]);
}

// ------------------------------------------------------------ backward ----
namespace w7 {

// Row padding of the per-step reduction buffers: the reader's lanes walk
// 8 steps x 8 pieces, so a step stride that is a multiple of the bank count
// puts all 64 lanes of a read on a quarter of the banks; 4 extra floats per
// step spread them (and keep 16-byte alignment).
constexpr int kRedPad = 4;

// Staged vectors of one reverse step (r, w, k, a, b on the lane's columns;
// v, dy and sa on its rows; sa is read again rather than kept in registers
// from the recomputation).
struct RevVecs {
  float4 r, w, k, a, b, v, g, sa;
  __device__ __forceinline__ void load(const float* stage, int s, int i0, int j0) {
    r = lds4(stage, QR, s, j0);
    w = lds4(stage, QW, s, j0);
    k = lds4(stage, QK, s, j0);
    a = lds4(stage, QA, s, j0);
    b = lds4(stage, QB, s, j0);
    v = lds4(stage, QV, s, i0);
    g = lds4(stage, QDY, s, i0);
    sa = lds4(stage, QSA, s, i0);
  }
};

struct BwdSmem {
  float stage[2][kStageVecs * kKC * kN];
  // Per sub-chunk step: per-wave partial sums over the wave's 16 rows of the
  // five key-indexed gradients (dr, dk, dw, da, db) at [(wave * 5 + q) * kN
  // + column], and dv.
  // Double-buffered by sub-chunk parity: a sub-chunk writes one buffer while
  // slower threads may still read the previous sub-chunk's sums from the
  // other, so one barrier per sub-chunk suffices.
  float red[2][kKS][4 * 5 * kN + kRedPad];
  float dvb[2][kKS][kN + kRedPad];
  // Store target of the lanes that hold no dv value (one word per thread).
  float dv_sink[kThreads];
  // -0.0 x 4: the three missing partials of a dv output in GradStores
  // (adding -0.0 leaves every value, -0.0 included, unchanged).
  float neg_zero[4];
};

// Recompute + reverse over one sub-chunk of cnt steps starting at staged
// step sl, from the sub-chunk's state record S0 (FULL: cnt == kKS, no
// per-step guards).  Leaves the per-step partial sums in sm.red / sm.dvb and
// advances G to before the sub-chunk.
template <bool FULL, typename Pre>
__device__ __forceinline__ void bwd_subchunk(BwdSmem& sm, int rbuf, const float* sg,
                                             const float (&S0)[4][4],
                                             int sl, int cnt, const Lane& L, float (&G)[4][4],
                                             Pre&& pre) {
  constexpr int KS = kKS;
  // Work of the previous sub-chunk (its gradients' collection) issued in the
  // same basic block as this one's, so its LDS reads and sums interleave
  // with the recomputation below.
  pre();
  const int col = L.j0 + L.rg;  // column this lane holds after rows4_sum
  // dv of row i0 + cg is stored by lane cg < 4 of each DPP row (every lane of
  // the row holds the four rows' sums); the other lanes store to their own
  // sink word, so the store needs no exec mask (a mask per step splits the
  // sub-chunk into one basic block per step).
  const bool dv_lane = L.cg < 4;
  float* const dv_base = dv_lane ? &sm.dvb[rbuf][0][L.i0 + L.cg] : &sm.dv_sink[threadIdx.x];
  const int dv_stride = dv_lane ? kN + kRedPad : 0;
  // Recompute the sub-chunk: Sp[s] = S_{t-1} of step s, Sp[s+1] = S_t.  In a
  // full sub-chunk every step's LDS vectors are read one step ahead (the
  // last recomputed step reads the first reverse step's), so no step waits
  // for its own reads.
  float Sp[KS + 1][4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) Sp[0][r][c] = S0[r][c];
  FwdVecs fx;
  RevVecs rx;
  if (FULL) fx.load(sg, sl, L.i0, L.j0);
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if (FULL) {
      const FwdVecs cur = fx;
      if (s + 1 < KS) {
        fx.load(sg, sl + s + 1, L.i0, L.j0);
      } else {
        rx.load(sg, sl + KS - 1, L.i0, L.j0);
      }
      fwd_step(Sp[s], Sp[s + 1], cur);
    } else if (s < cnt) {
      FwdVecs cur;
      cur.load(sg, sl + s, L.i0, L.j0);
      fwd_step(Sp[s], Sp[s + 1], cur);
    }
  }
  // Reverse; the post-update state of step s (S_t) is Sp[s + 1].
#pragma unroll
  for (int s = KS - 1; s >= 0; --s) {
    if (FULL || s < cnt) {
      const float (&St)[4][4] = Sp[s + 1];
      RevVecs x;
      if (FULL) {
        x = rx;
        if (s > 0) rx.load(sg, sl + s - 1, L.i0, L.j0);
      } else {
        x.load(sg, sl + s, L.i0, L.j0);
      }
      const float rr[4] = {x.r.x, x.r.y, x.r.z, x.r.w};
      const float ww[4] = {x.w.x, x.w.y, x.w.z, x.w.w};
      const float kk[4] = {x.k.x, x.k.y, x.k.z, x.k.w};
      const float aa[4] = {x.a.x, x.a.y, x.a.z, x.a.w};
      const float bb[4] = {x.b.x, x.b.y, x.b.z, x.b.w};
      const float vv[4] = {x.v.x, x.v.y, x.v.z, x.v.w};
      const float gy[4] = {x.g.x, x.g.y, x.g.z, x.g.w};
      const float sa[4] = {x.sa.x, x.sa.y, x.sa.z, x.sa.w};
      float pr[4], pk[4], pw[4], pa[4], pb[4], dvr[4], cc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float x = St[0][c] * gy[0];
#pragma unroll
        for (int r = 1; r < 4; ++r) x = fmaf(St[r][c], gy[r], x);
        pr[c] = x;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) G[r][c] = fmaf(gy[r], rr[c], G[r][c]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = G[r][0] * kk[0], z = G[r][0] * bb[0];
#pragma unroll
        for (int c = 1; c < 4; ++c) {
          x = fmaf(G[r][c], kk[c], x);
          z = fmaf(G[r][c], bb[c], z);
        }
        dvr[r] = x;
        cc[r] = z;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        dvr[r] = row16_sum(dvr[r]);
        cc[r] = row16_sum(cc[r]);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float xk = G[0][c] * vv[0], xw = G[0][c] * Sp[s][0][c];
        float xa = Sp[s][0][c] * cc[0], xb = G[0][c] * sa[0];
#pragma unroll
        for (int r = 1; r < 4; ++r) {
          xk = fmaf(G[r][c], vv[r], xk);
          xw = fmaf(G[r][c], Sp[s][r][c], xw);
          xa = fmaf(Sp[s][r][c], cc[r], xa);
          xb = fmaf(G[r][c], sa[r], xb);
        }
        pk[c] = xk; pw[c] = xw; pa[c] = xa; pb[c] = xb;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) G[r][c] = fmaf(G[r][c], ww[c], cc[r] * aa[c]);
      float* rs = &sm.red[rbuf][s][L.wv * 5 * kN];
      rs[0 * kN + col] = rows4_sum(pr[0], pr[1], pr[2], pr[3]);
      rs[1 * kN + col] = rows4_sum(pk[0], pk[1], pk[2], pk[3]);
      rs[2 * kN + col] = rows4_sum(pw[0], pw[1], pw[2], pw[3]);
      rs[3 * kN + col] = rows4_sum(pa[0], pa[1], pa[2], pa[3]);
      rs[4 * kN + col] = rows4_sum(pb[0], pb[1], pb[2], pb[3]);
      {
        const float d01 = (L.cg & 1) ? dvr[1] : dvr[0];
        const float d23 = (L.cg & 1) ? dvr[3] : dvr[2];
        dv_base[s * dv_stride] = (L.cg & 2) ? d23 : d01;
      }
    }
  }
}

// The six gradients of one sub-chunk of kKS steps: 5 x kKS x 16 outputs of
// four columns summed over the four waves' partials in sm.red (dr, dk, dw,
// da, db), then kKS x 16 of dv from sm.dvb; 768 outputs, three per thread.
// collect() has no branch (the gradient an output belongs to is the same in
// every lane of a wave, and a dv output adds three -0.0 partials, which leave
// every value unchanged), so the caller can place it in the basic block of
// the next sub-chunk's work; the sums run in the order ((w0 + w1) + w2) + w3
// over the waves.  flush() writes the outputs of steps < cnt; the caller
// issues it after its next wait on a load.
template <typename E>
struct GradStores {
  using raw = typename E::raw;
  static constexpr int NO = 3;
  static_assert(6 * kKS * (kN / 4) == NO * kThreads, "three outputs per thread");
  static_assert(kKS * (kN / 4) % 64 == 0, "one gradient per wave and output slot");
  OutPack<E, 4> data[NO];

  // Gradient (0-4: dr, dk, dw, da, db; 5: dv), step and column group of
  // output slot k of this thread.
  __device__ static __forceinline__ int grad_of(int k) {
    return __builtin_amdgcn_readfirstlane((int(threadIdx.x) + k * kThreads) / (kKS * (kN / 4)));
  }
  __device__ static __forceinline__ int step_of(int k) {
    return ((int(threadIdx.x) + k * kThreads) / (kN / 4)) % kKS;
  }
  __device__ static __forceinline__ int col_of(int k) {
    return 4 * ((int(threadIdx.x) + k * kThreads) % (kN / 4));
  }

  __device__ __forceinline__ void collect(const BwdSmem& sm, int rbuf) {
#pragma unroll
    for (int k = 0; k < NO; ++k) {
      const int q = grad_of(k);
      const int s = step_of(k);
      const int c = col_of(k);
      const float* red = &sm.red[rbuf][s][(q < 5 ? q : 0) * kN + c];
      const bool sum = q < 5;
      const float* p0 = sum ? red : &sm.dvb[rbuf][s][c];
      const float* p1 = sum ? red + 5 * kN : sm.neg_zero;
      const float* p2 = sum ? red + 10 * kN : sm.neg_zero;
      const float* p3 = sum ? red + 15 * kN : sm.neg_zero;
      float4 x = *reinterpret_cast<const float4*>(p0);
      const float4 x1 = *reinterpret_cast<const float4*>(p1);
      const float4 x2 = *reinterpret_cast<const float4*>(p2);
      const float4 x3 = *reinterpret_cast<const float4*>(p3);
      x.x += x1.x; x.y += x1.y; x.z += x1.z; x.w += x1.w;
      x.x += x2.x; x.y += x2.y; x.z += x2.z; x.w += x2.w;
      x.x += x3.x; x.y += x3.y; x.z += x3.z; x.w += x3.w;
      const float f[4] = {x.x, x.y, x.z, x.w};
      data[k].set(f);
    }
  }

  // outs: dr, dk, dw, da, db, dv; t: first step of the sub-chunk.
  __device__ __forceinline__ void flush(raw* const (&outs)[6], int bi, int h, int t, int cnt,
                                        int T, int H) const {
#pragma unroll
    for (int k = 0; k < NO; ++k) {
      const int q = grad_of(k);
      const int s = step_of(k);
      raw* o = outs[0];
#pragma unroll
      for (int i = 1; i < 6; ++i) o = (q == i) ? outs[i] : o;
      raw* dst = o + ((size_t(bi) * T + t + s) * H + h) * kN + col_of(k);
      if (s < cnt) {
        if constexpr (sizeof(raw) == 4) {
          *reinterpret_cast<uint4*>(dst) =
              make_uint4(data[k].u[0], data[k].u[1], data[k].u[2], data[k].u[3]);
        } else {
          *reinterpret_cast<uint2*>(dst) = make_uint2(data[k].u[0], data[k].u[1]);
        }
      }
    }
  }
};

// Stages sa_t of one block's kKC steps (rows kN .. of its kNSub records)
// into LDS as step vector QSA: kKC * kN / 4 pieces of 16 bytes, one per
// thread.  Steps past T read the last record (never used).
struct SaStager {
  static_assert(kKC * kN / 4 == kThreads, "one sa piece per thread");
  float4 buf;

  __device__ __forceinline__ void load(const float* ckh, int blk, int nrec) {
    const int p = int(threadIdx.x);
    const int s = p / (kN / 4);
    const int pc = p - s * (kN / 4);
    const int rec = min(blk * kNSub + s / kKS, nrec - 1);
    buf = *reinterpret_cast<const float4*>(ckh + size_t(rec) * kRecFloats +
                                           (kN + s % kKS) * kN + pc * 4);
  }

  __device__ __forceinline__ void store(float* stage) const {
    const int p = int(threadIdx.x);
    const int s = p / (kN / 4);
    const int pc = p - s * (kN / 4);
    *reinterpret_cast<float4*>(stage + (QSA * kKC + s) * kN + pc * 4) = buf;
  }
};

}  // namespace w7

// One workgroup per (batch, head); blocks of kKC steps last to first, each
// in sub-chunks of kKS steps (last to first) recomputed from their
// checkpoint records.  ds_T (optional): gradient of the final state; ds0 (optional):
// gradient of the initial state.
template <typename E>
__global__ __launch_bounds__(w7::kThreads) void wkv7_bwd_kernel(
    w7::Vecs<E, 7> in, const float* __restrict__ ck, const float* __restrict__ ds_T,
    typename E::raw* __restrict__ dr, typename E::raw* __restrict__ dw,
    typename E::raw* __restrict__ dk, typename E::raw* __restrict__ dv,
    typename E::raw* __restrict__ da, typename E::raw* __restrict__ db, float* __restrict__ ds0,
    int T, int H) {
  using namespace w7;
  __shared__ BwdSmem sm;
  const int bh = blockIdx.x;
  const int bi = bh / H;
  const int h = bh - bi * H;
  const Lane L;

  float G[4][4];
  if (ds_T) {
    load_state(G, ds_T + state_off(bh, 0, 0), L);
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) G[r][c] = 0.f;
  }
  wait_vmem_all();
  const int nblk = (T + kKC - 1) / kKC;
  const int nrec = (T + kKS - 1) / kKS;
  const float* ckh = ck + size_t(bh) * nrec * kRecFloats;
  Stager<E, 7> st;
  SaStager sst;
  // Sub-chunks run last to first as one loop.  Loads and stores are ordered
  // so that no fresh store is in flight when a load is waited for (the
  // vector-memory counter counts both, so such a wait would also wait for
  // the store): the record of the next sub-chunk is fetched one sub-chunk
  // ahead, a block's staging loads are issued after its first record has
  // arrived, and each sub-chunk's gradients are held in registers and
  // stored two sub-chunks later, once that sub-chunk's record has arrived.
  float Sn[4][4];
  if (nblk > 0) {
    st.load(in, bi, h, (nblk - 1) * kKC, T, H);
    sst.load(ckh, nblk - 1, nrec);
    load_state(Sn, ckh + size_t(nrec - 1) * kRecFloats, L);
    st.store(sm.stage[(nblk - 1) & 1]);
    sst.store(sm.stage[(nblk - 1) & 1]);
    __syncthreads();
  }
  using raw = typename E::raw;
  if (threadIdx.x < 4) sm.neg_zero[threadIdx.x] = -0.f;
  raw* const outs[6] = {dr, dk, dw, da, db, dv};
  // The gradients of sub-chunk sc + 1 are collected during sub-chunk sc (in
  // its basic block, overlapping its recomputation) and stored at the start
  // of sub-chunk sc - 1.
  GradStores<E> out;
  for (int sc = nrec - 1; sc >= 0; --sc) {
    const int blk = sc / kNSub;
    const int m = sc - blk * kNSub;
    const int t0 = blk * kKC;
    const int n = min(kKC, T - t0);
    const int sl = m * kKS;
    const int cnt = min(kKS, n - sl);
    float S0[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) S0[r][c] = Sn[r][c];
    if (sc > 0) load_state(Sn, ckh + size_t(sc - 1) * kRecFloats, L);
    // Gradients of sub-chunk sc + 2 (none before the third sub-chunk).
    if (sc + 2 < nrec) out.flush(outs, bi, h, (sc + 2) * kKS, min(kKS, T - (sc + 2) * kKS), T, H);
    // First sub-chunk of this block to run: fetch the previous block.
    if (blk > 0 && (m == kNSub - 1 || sc == nrec - 1)) {
      st.load(in, bi, h, t0 - kKC, T, H);
      sst.load(ckh, blk - 1, nrec);
    }
    const float* sg = sm.stage[blk & 1];
    // Sub-chunk sc + 1's sums are in sm.red / sm.dvb [(sc + 1) & 1] since the
    // last barrier; in the first sub-chunk those buffers hold nothing yet
    // and the collected values are never stored.  Only the last sub-chunk of
    // the sequence (the first to run) can be partial.
    if (cnt == kKS) {
      bwd_subchunk<true>(sm, sc & 1, sg, S0, sl, cnt, L, G,
                         [&] { out.collect(sm, (sc + 1) & 1); });
    } else {
      bwd_subchunk<false>(sm, sc & 1, sg, S0, sl, cnt, L, G, [] {});
    }
    __syncthreads();
    if (m == 0 && blk > 0) {
      st.store(sm.stage[(blk - 1) & 1]);
      sst.store(sm.stage[(blk - 1) & 1]);
      __syncthreads();
    }
  }
  if (nrec > 1) out.flush(outs, bi, h, kKS, min(kKS, T - kKS), T, H);
  if (nrec > 0) {
    out.collect(sm, 0);
    out.flush(outs, bi, h, 0, min(kKS, T), T, H);
  }
  if (ds0) store_state(ds0 + state_off(bh, 0, 0), G, L);
}

}  // namespace wkv

namespace wkv_host {

size_t wkv7_checkpoint_floats(int64_t B, int64_t T, int64_t H) {
  return size_t(B) * size_t(H) * size_t((T + wkv::w7::kKS - 1) / wkv::w7::kKS) *
         wkv::w7::kRecFloats;
}

template <typename E>
static int launch_wkv7_fwd(const void* r, const void* w, const void* k, const void* v,
                           const void* a, const void* b, const float* s0, void* y, float* s_out,
                           float* ck, int B, int T, int H, hipStream_t stream) {
  using raw = typename E::raw;
  wkv::w7::Vecs<E, 6> in{{static_cast<const raw*>(r), static_cast<const raw*>(w),
                          static_cast<const raw*>(k), static_cast<const raw*>(v),
                          static_cast<const raw*>(a), static_cast<const raw*>(b)}};
  const dim3 grid(unsigned(B) * H * wkv::w7::kSplit);
  if (ck) {
    launch(wkv::wkv7_fwd_kernel<E, true>, grid, dim3(wkv::w7::kThreads), stream, true, in, s0,
           static_cast<raw*>(y), s_out, ck, T, H);
  } else {
    launch(wkv::wkv7_fwd_kernel<E, false>, grid, dim3(wkv::w7::kThreads), stream, true, in, s0,
           static_cast<raw*>(y), s_out, ck, T, H);
  }
  return check_launch("wkv7_fwd_kernel");
}

int wkv7_forward_impl(const void* r, const void* w, const void* k, const void* v, const void* a,
                      const void* b, const float* s0, void* y, float* s_out, float* ck, int B,
                      int T, int H, int dtype, hipStream_t stream) {
  switch (dtype) {
    case 0: return launch_wkv7_fwd<wkv::F32>(r, w, k, v, a, b, s0, y, s_out, ck, B, T, H, stream);
    case 1: return launch_wkv7_fwd<wkv::BF16>(r, w, k, v, a, b, s0, y, s_out, ck, B, T, H, stream);
    case 2: return launch_wkv7_fwd<wkv::F16>(r, w, k, v, a, b, s0, y, s_out, ck, B, T, H, stream);
    default: return fail(1, "wkv7_forward: unknown dtype");
  }
}

template <typename E>
static int launch_wkv7_bwd(const void* r, const void* w, const void* k, const void* v,
                           const void* a, const void* b, const void* dy, const float* ck,
                           const float* ds_T, void* dr, void* dw, void* dk, void* dv, void* da,
                           void* db, float* ds0, int B, int T, int H, hipStream_t stream) {
  using raw = typename E::raw;
  wkv::w7::Vecs<E, 7> in{{static_cast<const raw*>(r), static_cast<const raw*>(w),
                          static_cast<const raw*>(k), static_cast<const raw*>(v),
                          static_cast<const raw*>(a), static_cast<const raw*>(b),
                          static_cast<const raw*>(dy)}};
  launch(wkv::wkv7_bwd_kernel<E>, dim3(unsigned(B) * H), dim3(wkv::w7::kThreads),
                     stream, true, in, ck, ds_T, static_cast<raw*>(dr), static_cast<raw*>(dw),
                     static_cast<raw*>(dk), static_cast<raw*>(dv), static_cast<raw*>(da),
                     static_cast<raw*>(db), ds0, T, H);
  return check_launch("wkv7_bwd_kernel");
}

int wkv7_backward_ck_impl(const void* r, const void* w, const void* k, const void* v,
                          const void* a, const void* b, const void* dy, const float* ck,
                          const float* ds_T, void* dr, void* dw, void* dk, void* dv, void* da,
                          void* db, float* ds0, int B, int T, int H, int dtype,
                          hipStream_t stream) {
  switch (dtype) {
    case 0:
      return launch_wkv7_bwd<wkv::F32>(r, w, k, v, a, b, dy, ck, ds_T, dr, dw, dk, dv, da, db,
                                       ds0, B, T, H, stream);
    case 1:
      return launch_wkv7_bwd<wkv::BF16>(r, w, k, v, a, b, dy, ck, ds_T, dr, dw, dk, dv, da, db,
                                        ds0, B, T, H, stream);
    case 2:
      return launch_wkv7_bwd<wkv::F16>(r, w, k, v, a, b, dy, ck, ds_T, dr, dw, dk, dv, da, db,
                                       ds0, B, T, H, stream);
    default: return fail(1, "wkv7_backward: unknown dtype");
  }
}

}  // namespace wkv_host
