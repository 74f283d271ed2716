// Shared device helpers for the gfx950 paged-KV kernels.
//
// Storage types: float (f32), _Float16 (f16) and bf16 kept as raw uint16_t bits.
// Every kernel computes in fp32 and converts on load/store; bf16 stores round to
// nearest even (hardware v_cvt_pk_bf16_f32), as torch's `.to(torch.bfloat16)`.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

#include "vllm_rlt_hip.h"

namespace vrh {

struct bf16_t {
  uint16_t bits;
};
using f16_t = _Float16;

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16_t x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_t x) {
  return __uint_as_float(((uint32_t)x.bits) << 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ f16_t from_f32<f16_t>(float x) { return (f16_t)x; }
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
  // v_cvt_pk_bf16_f32: round to nearest even, NaN stays NaN.
  bf16_t r;
  r.bits = __builtin_bit_cast(uint16_t, (__bf16)x);
  return r;
}

// Two floats to packed 16-bit storage (low half = lo), one conversion.
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<bf16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
template <>
__device__ __forceinline__ uint32_t pack2<f16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, f16x2_t));
}

// v_exp_f32 (2^x) and v_rcp_f32 without library range handling: softmax
// arguments are <= 0 (or -inf -> 0) and the reciprocal's input is >= 1e-30.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// ---------------------------------------------------------------- raw vectors
// A VEC-element vector of T loaded/stored as one global instruction
// (16 B = global_load_dwordx4 when VEC * sizeof(T) == 16).
template <int BYTES>
struct RawVec;
template <>
struct RawVec<1> {
  using type = uint8_t;
};
template <>
struct RawVec<2> {
  using type = uint16_t;
};
template <>
struct RawVec<4> {
  using type = uint32_t;
};
template <>
struct RawVec<8> {
  using type = __attribute__((ext_vector_type(2))) uint32_t;
};
template <>
struct RawVec<16> {
  using type = __attribute__((ext_vector_type(4))) uint32_t;
};

template <int VB>
using raw_of = typename RawVec<VB>::type;

// Widest byte-copy vector (16, 8, 4, 2 or 1) dividing every size and pointer.
// Bytes per element of a storage dtype code (0 for an unknown code).
inline int dtype_bytes(int dtype) {
  return dtype == VRH_DTYPE_F32 ? 4 : (dtype == VRH_DTYPE_F16 || dtype == VRH_DTYPE_BF16) ? 2 : 0;
}

inline int pick_vb(std::initializer_list<int64_t> values, std::initializer_list<const void*> ptrs) {
  for (int vb = 16; vb > 1; vb >>= 1) {
    bool ok = true;
    for (int64_t s : values) ok = ok && (s % vb == 0);
    for (const void* p : ptrs) ok = ok && ((uintptr_t)p % vb == 0);
    if (ok) return vb;
  }
  return 1;
}

// Launch KERNEL<vb> for a runtime byte-vector width.
#define VRH_DISPATCH_VB(vb, KERNEL, grid, block, stream, args)                      \
  switch (vb) {                                                                     \
    case 16: hipLaunchKernelGGL(KERNEL<16>, grid, block, 0, stream, args); break;  \
    case 8: hipLaunchKernelGGL(KERNEL<8>, grid, block, 0, stream, args); break;    \
    case 4: hipLaunchKernelGGL(KERNEL<4>, grid, block, 0, stream, args); break;    \
    case 2: hipLaunchKernelGGL(KERNEL<2>, grid, block, 0, stream, args); break;    \
    default: hipLaunchKernelGGL(KERNEL<1>, grid, block, 0, stream, args); break;   \
  }

template <typename T, int VEC>
struct Vec {
  static constexpr int kBytes = VEC * (int)sizeof(T);
  using raw_t = typename RawVec<kBytes>::type;
  union {
    raw_t raw;
    T e[VEC];
  };
};

template <typename T, int VEC>
__device__ __forceinline__ typename Vec<T, VEC>::raw_t load_raw(const T* p) {
  return *reinterpret_cast<const typename Vec<T, VEC>::raw_t*>(p);
}

// Non-temporal variant for streams that are read exactly once (K/V tiles).
template <typename T, int VEC>
__device__ __forceinline__ typename Vec<T, VEC>::raw_t load_raw_stream(const T* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const typename Vec<T, VEC>::raw_t*>(p));
}

template <typename T, int VEC>
__device__ __forceinline__ void store_raw(T* p, typename Vec<T, VEC>::raw_t v) {
  *reinterpret_cast<typename Vec<T, VEC>::raw_t*>(p) = v;
}

template <typename T, int VEC>
__device__ __forceinline__ void unpack(typename Vec<T, VEC>::raw_t raw, float (&out)[VEC]) {
  Vec<T, VEC> v;
  v.raw = raw;
#pragma unroll
  for (int i = 0; i < VEC; ++i) out[i] = to_f32(v.e[i]);
}

template <typename T, int VEC>
__device__ __forceinline__ typename Vec<T, VEC>::raw_t pack(const float (&in)[VEC]) {
  Vec<T, VEC> v;
#pragma unroll
  for (int i = 0; i < VEC; ++i) v.e[i] = from_f32<T>(in[i]);
  return v.raw;
}

// ------------------------------------------------------- LDS-direct loads
// LDS byte offset of a __shared__ object.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)p;
}

// One 16-byte-per-lane load from global memory into LDS at m0 + 16 * lane
// (global_load_lds_dwordx4). Issued as inline assembly so that the compiler
// neither waits for it nor orders LDS reads behind it: the caller bounds it
// with vm_wait before reading the LDS it fills. The s_nop is the wait state an
// LDS-direct load needs after an M0 write (the compiler inserts it for the
// instructions it knows, not inside asm). sc1 (agent scope) reads the line
// from L2 without allocating it in the CU's L1: staged tiles are read once
// per workgroup, so L1 allocation only adds tag work to the gather path.
__device__ __forceinline__ void lds_dma16(const void* g, uint32_t m0) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off sc1" ::"v"(g), "{m0}"(m0) : "memory");
}

// The same load with a wave-uniform 64-bit base in SGPRs and a 32-bit byte
// offset per lane (the saddr form: no 64-bit per-lane address).
__device__ __forceinline__ void lds_dma16_s(const void* base, uint32_t lane_off, uint32_t m0) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 sc1" ::"v"(lane_off), "s"(base), "{m0}"(m0)
               : "memory");
}

// s_waitcnt vmcnt(N) (gfx9 encoding; expcnt and lgkmcnt not waited on).
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 16, "vmcnt");
  __builtin_amdgcn_s_waitcnt(N | (0x7 << 4) | (0xF << 8));
}

// ------------------------------------------------------------ wave reductions
// DPP control words (GCN/CDNA "row" = 16 lanes).
constexpr int kDppQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <-> 7-i within 8
constexpr int kDppRowMirror = 0x140;      // lane i <-> 15-i within 16

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float shfl_xor_f32(float x, int mask) {
  int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(x)));
}

__device__ __forceinline__ int shfl_i32(int x, int src_lane) {
  return __builtin_amdgcn_ds_bpermute(src_lane << 2, x);
}

// Sum over aligned groups of WIDTH lanes (WIDTH a power of two <= 64); every
// lane of the group receives the group total.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (WIDTH >= 2) x += dpp_f32<kDppQuadXor1>(x);
  if constexpr (WIDTH >= 4) x += dpp_f32<kDppQuadXor2>(x);
  if constexpr (WIDTH >= 8) x += dpp_f32<kDppRowHalfMirror>(x);
  if constexpr (WIDTH >= 16) x += dpp_f32<kDppRowMirror>(x);
  if constexpr (WIDTH >= 32) x += shfl_xor_f32(x, 16);
  if constexpr (WIDTH >= 64) x += shfl_xor_f32(x, 32);
  return x;
}

// Reductions across the lane groups that differ in bits [LOG_FROM, 6) of the
// lane id (i.e. across token groups when each group spans 1 << LOG_FROM lanes).
template <int FROM>
__device__ __forceinline__ float cross_group_max(float x) {
#pragma unroll
  for (int m = FROM; m < 64; m <<= 1) x = fmaxf(x, shfl_xor_f32(x, m));
  return x;
}
template <int FROM>
__device__ __forceinline__ float cross_group_sum(float x) {
#pragma unroll
  for (int m = FROM; m < 64; m <<= 1) x += shfl_xor_f32(x, m);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) x = fmaxf(x, shfl_xor_f32(x, m));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) x += shfl_xor_f32(x, m);
  return x;
}

__host__ __device__ __forceinline__ int64_t ceil_div64(int64_t a, int64_t b) {
  return (a + b - 1) / b;
}
__host__ __device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace vrh

// --------------------------------------------------------------- host helpers
// Last error text, per thread; set by every entry point that fails.
void vrh_set_error(const char* fmt, ...);

#define VRH_CHECK_ARG(cond, ...)     \
  do {                               \
    if (!(cond)) {                   \
      vrh_set_error(__VA_ARGS__);    \
      return VRH_ERROR_INVALID_ARG;  \
    }                                \
  } while (0)

#define VRH_RETURN_LAUNCH(what)                                                         \
  do {                                                                                  \
    hipError_t _e = hipGetLastError();                                                  \
    if (_e != hipSuccess) {                                                             \
      vrh_set_error("%s: kernel launch failed: %s", what, hipGetErrorString(_e));       \
      return VRH_ERROR_LAUNCH;                                                          \
    }                                                                                   \
    return VRH_OK;                                                                      \
  } while (0)
