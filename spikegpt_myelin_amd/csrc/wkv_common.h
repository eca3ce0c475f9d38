// Shared device helpers for the gfx950 WKV kernels: element I/O for
// fp32/bf16/fp16 tensors, base-2 transcendentals, and the host-side error
// channel of the C ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace wkv {

// log2(e): every kernel keeps exponents in base 2 so that exp(x) is one
// v_exp_f32 of x * log2(e) folded into the operands once per element.
constexpr float kLog2e = 1.4426950408889634f;
// "Minus infinity" log-scale of an empty state, the value the reference
// kernels start from (wkv_triton.py:43), expressed in base-2 units.
constexpr float kNegHuge = -1e38f;
// Finite stand-in for +-infinity in running max/min reductions.
constexpr float kBig = 3.0e38f;

// Steps per checkpoint record of the forward state (see wkv4_fwd.hip).
constexpr int kCkptBlock = 64;
// Fields of a checkpoint record: state (A, B) = 2^o (p, q) at the block
// start.
constexpr int kCkptFields = 3;

// Range of the fixed-frame arithmetic (base-2 exponents): |k * log2(e)| of
// every element and |time_first * log2(e)| of every channel of a row.
// Outside it the row is recomputed with the reference running-max
// recurrences.
constexpr float kMaxK = 60.f;
constexpr float kMaxU = 16.f;

// p advanced by b bytes.  Spelled as a 32-bit byte offset added to a
// wave-uniform pointer so that loads and stores can use the scalar-base +
// 32-bit vector-offset address form (no per-lane 64-bit address arithmetic).
template <typename T>
__device__ __forceinline__ T* byte_offset(T* p, unsigned b) {
  // Opaque to the optimiser: keeps it from folding the lane offset into a
  // loop-invariant 64-bit per-lane pointer (which needs a 64-bit vector add
  // per access instead of the free scalar-base + offset form).
  asm volatile("" : "+v"(b));
  if constexpr (__is_const(T)) {
    return reinterpret_cast<T*>(reinterpret_cast<const char*>(p) + b);
  } else {
    return reinterpret_cast<T*>(reinterpret_cast<char*>(p) + b);
  }
}

// Clang vector types (the nontemporal builtins take these, not HIP's structs).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- math ----
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// ----------------------------------------------------------- element I/O --
// Element tags; storage is raw bits for the 16-bit types so that the kernels
// control conversions (bf16 widening is a shift; narrowing is round to
// nearest even via the hardware converter).
struct F32 { using raw = float; };
struct BF16 { using raw = uint16_t; };
struct F16 { using raw = uint16_t; };

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ uint16_t float_to_bf16_bits(float x) {
  __bf16 h = static_cast<__bf16>(x);  // RNE, NaN-preserving
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_float(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16));
  return static_cast<float>(h);
}

__device__ __forceinline__ uint16_t float_to_f16_bits(float x) {
  // The empty asm keeps x materialised as an fp32 value: without it the
  // compiler may fuse the multiply that produced x into the conversion
  // (one rounding straight to fp16), which would differ from rounding the
  // fp32 result -- what an fp32 computation followed by a cast produces.
  asm volatile("" : "+v"(x));
  _Float16 h = static_cast<_Float16>(x);  // RNE
  return __builtin_bit_cast(uint16_t, h);
}

// Rounds x to the element type and back (the value a 16-bit tensor holds).
template <typename E>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (__is_same(E, F32)) {
    return x;
  } else if constexpr (__is_same(E, BF16)) {
    return bf16_bits_to_float(float_to_bf16_bits(x));
  } else {
    return f16_bits_to_float(float_to_f16_bits(x));
  }
}

// sigmoid(r) as torch's fp32 kernel evaluates it (accurate expf, IEEE
// division), so values rounded from it agree with the eager path.
__device__ __forceinline__ float sigmoid_ref(float r) { return 1.f / (1.f + expf(-r)); }

// sigmoid(r) of the receptance gate, in fp32, for a gate tensor of element
// type E: sigmoid_ref for fp32 tensors.  For the 16-bit types the forward
// only ever uses the value rounded to the type, and the backward uses it at
// the 16-bit bar, so a short form is enough: e = 2^x with x = -|r| log2e,
// e in (0, 1], from the hardware exp2; sigmoid(|r|) = rcp(1 + e) and
// sigmoid(-|r|) = e * sigmoid(|r|).  Its error (a few fp32 ulp) moves the
// rounded value only where the exact sigmoid lies within that distance of a
// rounding midpoint.  bf16 keeps fp32's exponent range, so for it the fp32
// denormal range matters: below x = -126 the exponent is taken 64 higher
// and the result scaled back by a multiply (the hardware exp2 does not
// return denormals), and below x = -128, where the eager kernel's expf(-r)
// overflows and its 1 / (1 + inf) is 0, the value is 0 as there.  No
// branch: every lane runs the same instructions.
template <typename E>
__device__ __forceinline__ float gate_sigmoid(float r) {
  if constexpr (__is_same(E, F32)) {
    return sigmoid_ref(r);
  } else {
    const float x = -fabsf(r) * kLog2e;
    float e, sn;
    if constexpr (__is_same(E, BF16)) {
      const bool tiny = x < -126.f;
      e = fast_exp2(tiny ? x + 64.f : x);
      sn = e * fast_rcp(1.f + e);
      sn = tiny ? sn * 0x1p-64f : sn;
      sn = x < -128.f ? 0.f : sn;
    } else {
      // fp16: sigmoid(r) is below half the smallest fp16 denormal long
      // before e nears the fp32 denormal range, so no rescaling is needed.
      e = fast_exp2(x);
      sn = e * fast_rcp(1.f + e);
    }
    const float sp = fast_rcp(1.f + e);
    return r >= 0.f ? sp : sn;
  }
}

// Backward of out = round_E(s) * x, s = gate_sigmoid<E>(r), x the gated
// input as stored in E: grad_x = round_E(g s) (returned; it feeds the
// recurrence in the fused kernels) and grad_r = g s x (1 - s) (rounded at
// its store), the derivative taken through the unrounded s.
template <typename E>
__device__ __forceinline__ float gate_backward(float g, float s, float x, float& grad_r) {
  const float a = g * s;
  grad_r = a * x * (1.f - s);
  return round_to<E>(a);
}

// Vector of VEC consecutive channels as loaded by one lane in one
// instruction: raw bits held in 32-bit words.
template <typename E, int VEC> struct Pack;

template <int VEC> struct Pack<F32, VEC> {
  float x[VEC];
  __device__ __forceinline__ void load(const float* p) {
    if constexpr (VEC == 1) {
      x[0] = *p;
    } else if constexpr (VEC == 2) {
      float2 t = *reinterpret_cast<const float2*>(p);
      x[0] = t.x; x[1] = t.y;
    } else {
      static_assert(VEC == 4, "VEC");
      float4 t = *reinterpret_cast<const float4*>(p);
      x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int c = 0; c < VEC; ++c) x[c] = 0.f;
  }
  __device__ __forceinline__ float get(int c) const { return x[c]; }
};

template <int VEC> struct Pack<BF16, VEC> {
  static constexpr int W = (VEC + 1) / 2;
  uint32_t u[W];
  __device__ __forceinline__ void load(const uint16_t* p) {
    if constexpr (VEC == 1) {
      u[0] = *p;
    } else if constexpr (VEC == 2) {
      u[0] = *reinterpret_cast<const uint32_t*>(p);
    } else {
      static_assert(VEC == 4, "VEC");
      uint2 t = *reinterpret_cast<const uint2*>(p);
      u[0] = t.x; u[1] = t.y;
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < W; ++i) u[i] = 0u;
  }
  __device__ __forceinline__ float get(int c) const {
    const uint32_t w = u[c >> 1];
    return (c & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
  }
};

template <int VEC> struct Pack<F16, VEC> {
  static constexpr int W = (VEC + 1) / 2;
  uint32_t u[W];
  __device__ __forceinline__ void load(const uint16_t* p) {
    if constexpr (VEC == 1) {
      u[0] = *p;
    } else if constexpr (VEC == 2) {
      u[0] = *reinterpret_cast<const uint32_t*>(p);
    } else {
      static_assert(VEC == 4, "VEC");
      uint2 t = *reinterpret_cast<const uint2*>(p);
      u[0] = t.x; u[1] = t.y;
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < W; ++i) u[i] = 0u;
  }
  __device__ __forceinline__ float get(int c) const {
    const uint32_t w = u[c >> 1];
    return f16_bits_to_float((c & 1) ? (w >> 16) : (w & 0xffffu));
  }
};

// VEC floats already converted to the element type, held as 32-bit words
// until one vector store writes them.  Kernels convert each output as it is
// produced and issue a segment's stores together, under a single lane
// predicate.
template <typename E, int VEC> struct OutPack {
  static constexpr bool k32 = sizeof(typename E::raw) == 4;
  static constexpr int N = k32 ? VEC : (VEC + 1) / 2;
  uint32_t u[N];
  __device__ __forceinline__ void set(const float (&x)[VEC]) {
    if constexpr (k32) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) u[c] = __float_as_uint(x[c]);
    } else {
      uint16_t h[VEC];
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        if constexpr (__is_same(E, BF16)) {
          h[c] = float_to_bf16_bits(x[c]);
        } else {
          h[c] = float_to_f16_bits(x[c]);
        }
      }
      if constexpr (VEC == 1) {
        u[0] = h[0];
      } else {
#pragma unroll
        for (int i = 0; i < N; ++i) u[i] = uint32_t(h[2 * i]) | (uint32_t(h[2 * i + 1]) << 16);
      }
    }
  }
  // Non-temporal (streaming) stores: outputs are not re-read by the kernel
  // that writes them, and keeping them out of the L2 as dirty lines measured
  // 6-10% faster for both RWKV-4 kernels than ordinary stores.
  __device__ __forceinline__ void store(typename E::raw* p) const {
    if constexpr (k32) {
      if constexpr (VEC == 1) {
        __builtin_nontemporal_store(u[0], reinterpret_cast<uint32_t*>(p));
      } else if constexpr (VEC == 2) {
        __builtin_nontemporal_store(u32x2{u[0], u[1]}, reinterpret_cast<u32x2*>(p));
      } else {
        __builtin_nontemporal_store(u32x4{u[0], u[1], u[2], u[3]}, reinterpret_cast<u32x4*>(p));
      }
    } else {
      if constexpr (VEC == 1) {
        __builtin_nontemporal_store(static_cast<uint16_t>(u[0]), p);
      } else if constexpr (VEC == 2) {
        __builtin_nontemporal_store(u[0], reinterpret_cast<uint32_t*>(p));
      } else {
        __builtin_nontemporal_store(u32x2{u[0], u[1]}, reinterpret_cast<u32x2*>(p));
      }
    }
  }
};

// Store VEC floats as one vector store of the element type.
template <typename E, int VEC>
__device__ __forceinline__ void store_vec(typename E::raw* p, const float (&x)[VEC]) {
  if constexpr (sizeof(typename E::raw) == 4) {
    if constexpr (VEC == 1) {
      *p = x[0];
    } else if constexpr (VEC == 2) {
      *reinterpret_cast<float2*>(p) = make_float2(x[0], x[1]);
    } else {
      *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
    }
  } else {
    uint16_t h[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      if constexpr (__is_same(E, BF16)) {
        h[c] = float_to_bf16_bits(x[c]);
      } else {
        h[c] = float_to_f16_bits(x[c]);
      }
    }
    if constexpr (VEC == 1) {
      *p = h[0];
    } else if constexpr (VEC == 2) {
      *reinterpret_cast<uint32_t*>(p) = uint32_t(h[0]) | (uint32_t(h[1]) << 16);
    } else {
      *reinterpret_cast<uint2*>(p) = make_uint2(uint32_t(h[0]) | (uint32_t(h[1]) << 16),
                                                uint32_t(h[2]) | (uint32_t(h[3]) << 16));
    }
  }
}

template <typename E>
__device__ __forceinline__ float load_scalar(const typename E::raw* p) {
  if constexpr (__is_same(E, F32)) {
    return *p;
  } else if constexpr (__is_same(E, BF16)) {
    return bf16_bits_to_float(*p);
  } else {
    return f16_bits_to_float(*p);
  }
}

template <typename E>
__device__ __forceinline__ void store_scalar(typename E::raw* p, float x) {
  if constexpr (__is_same(E, F32)) {
    *p = x;
  } else if constexpr (__is_same(E, BF16)) {
    *p = float_to_bf16_bits(x);
  } else {
    *p = float_to_f16_bits(x);
  }
}

}  // namespace wkv

// ------------------------------------------------------------ host side ---
namespace wkv_host {
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

// Timing events of the entry point running on this thread.  Armed by
// wkv_time_next_call (kernel < 0): the first kernel dispatch of the call
// carries `start` and the dispatch that ends the call carries `stop`; or by
// wkv_time_next_kernel: dispatch number `kernel` of the call carries both.
// `count` numbers the call's dispatches.  All null outside a timed call.
struct CallEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
  int kernel = -1;
  int count = 0;
};
CallEvents& active_events();

// Kernel launch on `stream`; `ends_call` marks the last dispatch of an entry
// point.  During a timed call the events are bound to the dispatch packets
// themselves (hipExtLaunchKernel): the timestamps are the kernels' own start
// and end, and no marker packet is added to the stream.
template <typename... KArgs, typename... Args>
void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t stream, bool ends_call,
            Args... args) {
  CallEvents& ev = active_events();
  hipEvent_t start = nullptr, stop = nullptr;
  if (ev.kernel < 0) {
    start = ev.start;
    stop = ends_call ? ev.stop : nullptr;
    ev.start = nullptr;
  } else if (ev.count == ev.kernel) {
    start = ev.start;
    stop = ev.stop;
  }
  ++ev.count;
  if (start != nullptr || stop != nullptr) {
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0,
                          static_cast<KArgs>(args)...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, static_cast<KArgs>(args)...);
  }
}
}  // namespace wkv_host

namespace wkv {

// ------------------------------------------------------ buffer resources ----
// Raw (stride 0) buffer descriptor: base address in SGPRs, size in bytes.
// Loads at offsets >= bytes return 0 and stores there are dropped.  Every
// access is voffset (per lane, VGPR) + soffset (per step, SGPR), so address
// arithmetic stays on the scalar unit and no per-lane pointer is formed.
// Third dword: 32-bit data format, the raw-buffer setting on gfx9.
using rsrc_t = __amdgpu_buffer_rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}

// Cache-policy bits of a buffer instruction: non-temporal (streaming).
constexpr int kAuxNT = 2;

// Bytes from element `t0 * C` of a row to the end of its batch entry, where
// row_tail = T*C - (channel offset of the row); 0 when t0 >= T, saturated at
// 2^32 - 1 (a descriptor never needs more than one chunk's span).
__device__ __forceinline__ uint32_t span_bytes(size_t row_tail, int t0, int C, int esize) {
  const long long rem = (long long)row_tail - (long long)t0 * C;
  if (rem <= 0) return 0u;
  const unsigned long long b = (unsigned long long)rem * (unsigned long long)esize;
  return b > 0xFFFFFFFFull ? 0xFFFFFFFFu : uint32_t(b);
}

template <typename E, int VEC>
__device__ __forceinline__ void load_buf(Pack<E, VEC>& p, rsrc_t r, unsigned voff, unsigned soff) {
  constexpr int bytes = int(sizeof(typename E::raw)) * VEC;
  if constexpr (__is_same(E, F32)) {
    if constexpr (VEC == 1) {
      p.x[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
    } else if constexpr (VEC == 2) {
      const u32x2 t = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
      p.x[0] = __uint_as_float(t.x); p.x[1] = __uint_as_float(t.y);
    } else {
      const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
      p.x[0] = __uint_as_float(t.x); p.x[1] = __uint_as_float(t.y);
      p.x[2] = __uint_as_float(t.z); p.x[3] = __uint_as_float(t.w);
    }
  } else if constexpr (bytes == 2) {
    p.u[0] = __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
  } else if constexpr (bytes == 4) {
    p.u[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
  } else {
    const u32x2 t = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    p.u[0] = t.x; p.u[1] = t.y;
  }
}

// Non-temporal store of an OutPack (outputs are not re-read by the kernel
// that writes them; keeping them out of the L2 as dirty lines measured 6-10%
// faster for both RWKV-4 kernels than ordinary stores).
template <typename E, int VEC>
__device__ __forceinline__ void store_buf(const OutPack<E, VEC>& o, rsrc_t r, unsigned voff,
                                          unsigned soff) {
  constexpr int N = OutPack<E, VEC>::N;
  constexpr bool k16 = sizeof(typename E::raw) == 2;
  if constexpr (k16 && VEC == 1) {
    __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(o.u[0]), r, voff, soff, kAuxNT);
  } else if constexpr (N == 1) {
    __builtin_amdgcn_raw_buffer_store_b32(o.u[0], r, voff, soff, kAuxNT);
  } else if constexpr (N == 2) {
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{o.u[0], o.u[1]}, r, voff, soff, kAuxNT);
  } else {
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{o.u[0], o.u[1], o.u[2], o.u[3]}, r, voff, soff,
                                           kAuxNT);
  }
}

// out[r][c] = sum_p partial[r][p][c] over P partial rows in a fixed order:
// G threads per channel (G x 64 = the workgroup) each sum every G-th row,
// then a fixed LDS tree (the loop is unrolled so that a thread's loads are
// in flight together; the sums keep their order).  A template so that each
// translation unit that launches it holds its own copy.
template <int G>
__global__ __launch_bounds__(1024) void column_sum_kernel(const float* __restrict__ partial,
                                                          float* __restrict__ out, int P, int C) {
  __shared__ float sh[G][64];
  const int lane = threadIdx.x & 63;
  const int grp = threadIdx.x >> 6;
  const int r = blockIdx.y;
  const int c = blockIdx.x * 64 + lane;
  float a = 0.f;
  if (c < C) {
    const float* src = partial + size_t(r) * P * C + c;
#pragma unroll 8
    for (int p = grp; p < P; p += G) a += src[size_t(p) * C];
  }
  sh[grp][lane] = a;
  __syncthreads();
  for (int h = G / 2; h > 0; h >>= 1) {
    if (grp < h) sh[grp][lane] += sh[grp + h][lane];
    __syncthreads();
  }
  if (grp == 0 && c < C) out[size_t(r) * C + c] = sh[0][lane];
}

// ------------------------------------------------- look-back words ----
// Carries exchanged between workgroups of one kernel (the RWKV-4 kernels
// split over time): a pair of fp32 values (a, b) packed in one 64-bit word
// that is written and read with relaxed agent-scope atomics.  Such accesses
// are coherent across the chip's XCDs (their L2s are not) without any fence,
// and a 64-bit word is written in one piece, so the word is its own "ready"
// flag: the workspace is filled with kLbEmpty before the kernel, and a word
// that differs from it holds a published pair.  kLbEmpty is two NaNs with an
// all-ones payload, which arithmetic never produces (the hardware's NaN
// results are the canonical 0x7fc00000); a pair that still matches it (NaN
// inputs carrying that payload) is published as canonical NaNs instead.
constexpr uint64_t kLbEmpty = ~uint64_t(0);
constexpr uint64_t kLbNaN = (uint64_t(0x7fc00000u) << 32) | 0x7fc00000u;
// Polls of one word before a workgroup gives up waiting (the row is then
// recomputed by the exact path).  A published word arrives within
// microseconds; the bound only guarantees that every wave ends.  The kernels
// take the bound as an argument (at most this).
constexpr int kLbMaxPolls = 1 << 16;
// Marker values of the per-row status words (filled with all ones).
constexpr uint32_t kRowOk = ~uint32_t(0);
constexpr uint32_t kRowRedo = 0u;

__device__ __forceinline__ uint64_t lb_pack(float a, float b) {
  const uint64_t w = (uint64_t(__float_as_uint(b)) << 32) | __float_as_uint(a);
  return w == kLbEmpty ? kLbNaN : w;
}
__device__ __forceinline__ float lb_lo(uint64_t w) { return __uint_as_float(uint32_t(w)); }
__device__ __forceinline__ float lb_hi(uint64_t w) { return __uint_as_float(uint32_t(w >> 32)); }
__device__ __forceinline__ void lb_store(uint64_t* p, uint64_t w) {
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t lb_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Aggregates a split kernel folds before the inclusive word it waits for.
#ifndef WKV_LB_WINDOW
#define WKV_LB_WINDOW 4
#endif
constexpr int kLbWindow = WKV_LB_WINDOW;

// Carry of segment s of a row split over time, from look-back words.  dir =
// +1: the carry comes from the segments before s (forward), -1: from those
// after it (backward).  The K = kLbWindow nearest such segments contribute
// their aggregates and the next one out its inclusive word, folded by Horner
// from the farthest:  carry = (...(incl * DS + agg_far) * DS ...) * DS +
// agg_near, where DS is the decay over one segment.  The words read never
// depend on when they were published, so the carry (and the kernel's result)
// is the same on every run.  agg, incl: this lane's words of segment 0;
// segment j's are seg_stride words further.  Returns false, with a zero
// carry, when a word did not arrive within max_polls polls (at once,
// without reading, for max_polls < 0).
template <int VEC>
__device__ __forceinline__ bool lb_window_carry(const uint64_t* agg, const uint64_t* incl,
                                                size_t seg_stride, int s, int nseg, int dir,
                                                const float (&DS)[VEC], float (&ca)[VEC],
                                                float (&cb)[VEC], int max_polls) {
  constexpr int K = kLbWindow;
  uint64_t wa[K][VEC], wi[VEC];
  const int jo = s - dir * (K + 1);  // the inclusive word's segment
  const bool has_incl = jo >= 0 && jo < nseg;
#pragma unroll
  for (int c = 0; c < VEC; ++c) { ca[c] = 0.f; cb[c] = 0.f; }
  if (max_polls < 0) return false;
  for (int polls = 0;; ++polls) {
    bool ready = true;
#pragma unroll
    for (int d = 1; d <= K; ++d) {
      const int j = s - dir * d;
      if (j < 0 || j >= nseg) continue;
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        wa[d - 1][c] = lb_load(agg + size_t(j) * seg_stride + c);
        ready &= wa[d - 1][c] != kLbEmpty;
      }
    }
    if (has_incl) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        wi[c] = lb_load(incl + size_t(jo) * seg_stride + c);
        ready &= wi[c] != kLbEmpty;
      }
    }
    if (ready) break;
    if (polls >= max_polls) return false;
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    ca[c] = has_incl ? lb_lo(wi[c]) : 0.f;
    cb[c] = has_incl ? lb_hi(wi[c]) : 0.f;
  }
#pragma unroll
  for (int d = K; d >= 1; --d) {
    const int j = s - dir * d;
    if (j < 0 || j >= nseg) continue;
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      ca[c] = fmaf(ca[c], DS[c], lb_lo(wa[d - 1][c]));
      cb[c] = fmaf(cb[c], DS[c], lb_hi(wa[d - 1][c]));
    }
  }
  return true;
}

// Marks a row for recomputation by the exact path (read by a later kernel).
__device__ __forceinline__ void mark_row_redo(uint32_t* status, int row) {
  __hip_atomic_store(status + row, kRowRedo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Fills n16 pieces of 16 bytes with all ones (the look-back words and row
// status words of a split kernel, before it runs).  A template so that each
// translation unit that launches it holds its own copy.
template <int Unused = 0>
__global__ __launch_bounds__(256) void lb_fill_kernel(u32x4* __restrict__ p, size_t n16) {
  const u32x4 ones = {~0u, ~0u, ~0u, ~0u};
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n16; i += size_t(gridDim.x) * 256)
    p[i] = ones;
}

}  // namespace wkv
