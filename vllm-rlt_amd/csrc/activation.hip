// SiLU-and-Mul for the MLP step beside the attention path: out = silu(gate) * up.
//
// Reference contract: vllm_rlt/kernels/activation.py:9-33 and docs/kernels.md:
// equal shapes and dtypes (f32, f16, bf16), contiguous inputs whose storage
// offsets may be misaligned independently, SiLU rounded to the storage dtype
// before the multiply (torch's `F.silu(gate) * up`), product rounded to the
// dtype. tests/test_activation.py:360-430 demands bit-exact results over every
// 16-bit gate pattern.
//
// Rounding design (own): the value of silu(x) rounded to the dtype is computed
// exactly as the double-precision expression rounded first to fp32 and then
// to the dtype (torch's double -> bf16/f16 conversion path).
//  * bf16/f16: a compensated fp32 evaluation (error <= ~5 fp32 ulp) is
//    rounded; if y -/+ 8 ulp round to different dtype values (y lies near a
//    rounding boundary), or x is outside the fast path's range, the lane
//    recomputes in fp64. The fp32 -> dtype rounding has 13 (f16) or 16 (bf16)
//    spare bits, so the fallback is rare.
//  * f32: computed in fp64 and rounded once (CDNA's fp64 VALU runs at the fp32
//    rate, so this stays HBM-bound).
// The product of two dtype values is exact in fp32 (bf16/f16) or fp64 (f32),
// so one rounding gives torch's result.
//
// Memory layout: the vector body is aligned to the output; gate and up are read
// with aligned 16-byte loads and funnel-shifted (v_alignbyte) when their
// storage offset differs from the output's. Elements before the first aligned
// output vector and after the last are done one per thread.
#include <math.h>

#include <algorithm>

#include "common.h"

namespace vrh {
namespace {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

constexpr int kThreads = 256;
// One 16-byte vector per thread: measured at 5.9 TB/s on MI355X, ahead of a
// capped grid-stride loop (5.5-5.8), with next-step prefetch (5.3) or with
// non-temporal accesses (4.7-5.7). Larger inputs loop.
constexpr int kMaxBlocks = 1 << 20;
// fp32 ulps around a dtype rounding boundary that send a lane to fp64: above
// the fast evaluation's error bound (~5 ulp). silu depends only on the 16-bit
// gate, and every bf16 and f16 gate pattern has been checked to round as the
// fp64 expression does; 8 instead of 16 halves how often a wave takes the
// fp64 branch (8192 x 5632 bf16: 43 against 47 us).
constexpr int kWindow = 8;

// silu(x) in fp64, rounded to fp32 (the reference's double expression).
__device__ __forceinline__ float silu_ref(float xf) {
  const double x = xf;
  double y;
  if (x >= 0.0) {
    y = x / (1.0 + exp(-x));
  } else {
    const double t = exp(x);
    y = x * t / (1.0 + t);
  }
  return (float)y;
}

// Compensated fp32 silu, valid for x >= -87 (and +inf, NaN): t = e^-|x| from
// 2^p (1 + e ln 2) with p + e = -|x| log2(e) split by an FMA (p the rounded
// product, e its remainder), silu = (x >= 0 ? x : x t) / (1 + t). Tiny x give
// x / 2 exactly; +inf gives inf and NaN stays NaN.
__device__ __forceinline__ float silu_fast(float x) {
  constexpr float kLog2eHi = 1.44269502162933349609375f;         // log2(e) rounded to fp32
  constexpr float kLog2eLo = 1.925963033500011079e-8f;            // log2(e) - kLog2eHi
  constexpr float kLn2 = 0.693147180559945309f;
  const float z = __builtin_amdgcn_fmed3f(-fabsf(x), -87.0f, 0.0f);  // max(-|x|, -87)
  const float p = z * kLog2eHi;
  const float e = fmaf(z, kLog2eHi, -p) + z * kLog2eLo;
  const float b = __builtin_amdgcn_exp2f(p);
  const float t = fmaf(b, e * kLn2, b);          // e^z, ~2 ulp
  const float r = __builtin_amdgcn_rcpf(1.0f + t);
  return (x >= 0.0f ? x : x * t) * r;
}

template <typename T>
__device__ __forceinline__ T from_bits(uint32_t b);
template <>
__device__ __forceinline__ bf16_t from_bits<bf16_t>(uint32_t b) { return bf16_t{(uint16_t)b}; }
template <>
__device__ __forceinline__ f16_t from_bits<f16_t>(uint32_t b) {
  return __builtin_bit_cast(f16_t, (uint16_t)b);
}

template <typename T>
__device__ __forceinline__ uint32_t round_bits(float y);
template <>
__device__ __forceinline__ uint32_t round_bits<bf16_t>(float y) { return from_f32<bf16_t>(y).bits; }
template <>
__device__ __forceinline__ uint32_t round_bits<f16_t>(float y) {
  return __builtin_bit_cast(uint16_t, (f16_t)y);
}

// True when the fast value y cannot be trusted to round like the exact one:
// rounding |y| -/+ kWindow ulp to T differs (y is near a rounding boundary),
// or x lies below the fast path's range (x < -87, -inf).
template <typename T>
__device__ __forceinline__ bool needs_fp64(float x, float y) {
  const uint32_t mag = __float_as_uint(y) & 0x7fffffffu;
  const bool range = !(x >= -87.0f);
  if constexpr (__is_same(T, bf16_t)) {
    // bf16 keeps the top 16 bits: nearest-even boundaries sit at 0x8000 mod
    // 0x10000, so shift by 0x8000 and test for a carry out of the low half.
    const uint32_t lo = mag + (0x8000u - kWindow);
    return range || ((lo ^ (lo + 2 * kWindow)) >> 16) != 0;
  } else {
    return range || round_bits<T>(__uint_as_float(mag - kWindow)) !=
                        round_bits<T>(__uint_as_float(mag + kWindow));
  }
}

// silu(x) rounded to T, returned as fp32 (exactly representable in T).
template <typename T>
__device__ __forceinline__ float silu_rounded(float x) {
  float r = silu_fast(x);
  if (needs_fp64<T>(x, r)) {
    // A real (rarely taken) branch: without the empty asm the compiler
    // evaluates the fp64 path for every element and selects.
    asm volatile("");
    r = silu_ref(x);
  }
  return to_f32(from_bits<T>(round_bits<T>(r)));
}

// Element-wise result for one element (all dtypes), as the dtype's bits.
template <typename T>
__device__ __forceinline__ T silu_mul_one(T g, T u);
template <>
__device__ __forceinline__ float silu_mul_one<float>(float g, float u) {
  return silu_ref(g) * u;
}
template <>
__device__ __forceinline__ bf16_t silu_mul_one<bf16_t>(bf16_t g, bf16_t u) {
  return from_f32<bf16_t>(silu_rounded<bf16_t>(to_f32(g)) * to_f32(u));
}
template <>
__device__ __forceinline__ f16_t silu_mul_one<f16_t>(f16_t g, f16_t u) {
  return from_f32<f16_t>(silu_rounded<f16_t>(to_f32(g)) * to_f32(u));
}

// One 16-byte vector of results. The 16-bit types evaluate all eight fast
// values first and take one (rarely taken) branch for the fp64 fixups.
template <typename T>
__device__ __forceinline__ u32x4 silu_mul_vec(u32x4 g, u32x4 u) {
  u32x4 o;
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = __float_as_uint(silu_ref(__uint_as_float(g[i])) * __uint_as_float(u[i]));
  } else {
    float x[8], up[8], y[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (__is_same(T, bf16_t)) {
        x[2 * i] = __uint_as_float(g[i] << 16);
        x[2 * i + 1] = __uint_as_float(g[i] & 0xffff0000u);
        up[2 * i] = __uint_as_float(u[i] << 16);
        up[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
      } else {
        x[2 * i] = (float)__builtin_bit_cast(f16_t, (uint16_t)(g[i] & 0xffffu));
        x[2 * i + 1] = (float)__builtin_bit_cast(f16_t, (uint16_t)(g[i] >> 16));
        up[2 * i] = (float)__builtin_bit_cast(f16_t, (uint16_t)(u[i] & 0xffffu));
        up[2 * i + 1] = (float)__builtin_bit_cast(f16_t, (uint16_t)(u[i] >> 16));
      }
    }
    bool slow[8];
    bool any = false;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      y[k] = silu_fast(x[k]);
      slow[k] = needs_fp64<T>(x[k], y[k]);
      any = any || slow[k];
    }
    if (any) {
      asm volatile("");
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (slow[k]) y[k] = silu_ref(x[k]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a0 = to_f32(from_bits<T>(round_bits<T>(y[2 * i])));
      const float a1 = to_f32(from_bits<T>(round_bits<T>(y[2 * i + 1])));
      o[i] = pack2<T>(a0 * up[2 * i], a1 * up[2 * i + 1]);
    }
  }
  return o;
}

// Bytes [s, s + 16) of the 32-byte concatenation a || b (s uniform, 0..15).
__device__ __forceinline__ u32x4 funnel(u32x4 a, u32x4 b, int s) {
  const uint32_t w[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  const int r = s & 3;
  u32x4 o;
  switch (s >> 2) {
#define VRH_FUNNEL(Q)                                                              \
  case Q:                                                                          \
    for (int j = 0; j < 4; ++j) o[j] = __builtin_amdgcn_alignbyte(w[Q + j + 1], w[Q + j], r); \
    break;
    VRH_FUNNEL(0)
    VRH_FUNNEL(1)
    VRH_FUNNEL(2)
    VRH_FUNNEL(3)
#undef VRH_FUNNEL
  }
  return o;
}

struct SiluArgs {
  const char* gate;   // element `head` of gate (byte pointer, any alignment of its type)
  const char* up;
  char* out;          // element `head` of out: 16-byte aligned
  const char* gate0;  // element 0 of each tensor (scalar elements)
  const char* up0;
  char* out0;
  int64_t nvec;       // aligned output vectors
  int64_t head;       // scalar elements before the vector body
  int64_t tail;       // scalar elements after it
  int gshift, ushift; // byte offsets of gate / up from 16-byte alignment at `head`
};

template <typename T, bool GS, bool US>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(SiluArgs a) {
  constexpr int E = 16 / sizeof(T);
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const u32x4* gv = reinterpret_cast<const u32x4*>(a.gate - a.gshift);
  const u32x4* uv = reinterpret_cast<const u32x4*>(a.up - a.ushift);
  u32x4* ov = reinterpret_cast<u32x4*>(a.out);
  // Shifted inputs need the next aligned vector too; the body excludes the
  // last output vector in that case, so v + 1 stays inside the input. The
  // first loads are issued before the loop (this shape measured ~8 % faster
  // than loading at the top of each iteration).
  struct In { u32x4 g, g1, u, u1; };
  auto load = [&](int64_t v) {
    In r;
    r.g = gv[v];
    r.u = uv[v];
    if constexpr (GS) r.g1 = gv[v + 1];
    if constexpr (US) r.u1 = uv[v + 1];
    return r;
  };
  int64_t v = gid;
  In cur;
  if (v < a.nvec) cur = load(v);
  while (v < a.nvec) {
    u32x4 g = cur.g, u = cur.u;
    if constexpr (GS) g = funnel(g, cur.g1, a.gshift);
    if constexpr (US) u = funnel(u, cur.u1, a.ushift);
    ov[v] = silu_mul_vec<T>(g, u);
    v += stride;
    if (v < a.nvec) cur = load(v);
  }
  if (gid < a.head + a.tail) {
    const int64_t e = gid < a.head ? gid : a.head + a.nvec * E + (gid - a.head);
    const T g = reinterpret_cast<const T*>(a.gate0)[e];
    const T u = reinterpret_cast<const T*>(a.up0)[e];
    reinterpret_cast<T*>(a.out0)[e] = silu_mul_one<T>(g, u);
  }
}

template <typename T>
void launch_silu(const SiluArgs& a, hipStream_t s) {
  const int64_t work = std::max<int64_t>(a.nvec, a.head + a.tail);
  const int blocks = (int)std::min<int64_t>((work + kThreads - 1) / kThreads, kMaxBlocks);
  const bool gs = a.gshift != 0, us = a.ushift != 0;
  if (gs && us)
    hipLaunchKernelGGL((silu_mul_kernel<T, true, true>), dim3(blocks), dim3(kThreads), 0, s, a);
  else if (gs)
    hipLaunchKernelGGL((silu_mul_kernel<T, true, false>), dim3(blocks), dim3(kThreads), 0, s, a);
  else if (us)
    hipLaunchKernelGGL((silu_mul_kernel<T, false, true>), dim3(blocks), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((silu_mul_kernel<T, false, false>), dim3(blocks), dim3(kThreads), 0, s, a);
}

}  // namespace
}  // namespace vrh

using namespace vrh;

extern "C" int vrh_silu_and_mul(int dtype, void* out, const void* gate, const void* up,
                                int64_t count, vrh_stream_t stream) {
  VRH_CHECK_ARG(dtype == VRH_DTYPE_F32 || dtype == VRH_DTYPE_F16 || dtype == VRH_DTYPE_BF16,
                "vrh_silu_and_mul: supports float32, float16 and bfloat16");
  VRH_CHECK_ARG(count >= 0, "vrh_silu_and_mul: negative element count");
  if (count == 0) return VRH_OK;
  VRH_CHECK_ARG(out && gate && up, "vrh_silu_and_mul: null pointer");
  const int esz = dtype == VRH_DTYPE_F32 ? 4 : 2;
  const int E = 16 / esz;
  for (const void* p : {(const void*)out, gate, up})
    VRH_CHECK_ARG((uintptr_t)p % esz == 0, "vrh_silu_and_mul: pointer not aligned to its dtype");
  SiluArgs a;
  a.gate0 = static_cast<const char*>(gate);
  a.up0 = static_cast<const char*>(up);
  a.out0 = static_cast<char*>(out);
  const int64_t out_phase = (int64_t)(((uintptr_t)out % 16) / esz);
  a.head = std::min<int64_t>((E - out_phase) % E, count);
  a.gate = a.gate0 + a.head * esz;
  a.up = a.up0 + a.head * esz;
  a.out = a.out0 + a.head * esz;
  a.gshift = (int)((uintptr_t)a.gate % 16);
  a.ushift = (int)((uintptr_t)a.up % 16);
  a.nvec = (count - a.head) / E;
  // A shifted input reads the aligned vector after each body vector: leave
  // the last one to the scalar tail so no read passes the input's end.
  if ((a.gshift || a.ushift) && a.nvec > 0) a.nvec -= 1;
  a.tail = count - a.head - a.nvec * E;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == VRH_DTYPE_F32) launch_silu<float>(a, s);
  else if (dtype == VRH_DTYPE_F16) launch_silu<f16_t>(a, s);
  else launch_silu<bf16_t>(a, s);
  VRH_RETURN_LAUNCH("vrh_silu_and_mul");
}
