// Shared device/host helpers for the minitp HIP library (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/minitp.h"

namespace minitp {

// ---------------------------------------------------------------------------
// Storage types. bf16 is kept as raw uint16 so every conversion (and its
// rounding) is explicit: float -> bf16 rounds to nearest even like
// torch's Tensor.to(torch.bfloat16); NaN maps to a quiet NaN.
struct bf16 {
  uint16_t bits;
};
// Operand type of the packed bf16 dot instructions.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// gfx950's v_cvt_pk_bf16_f32 rounds to nearest even, which is torch's
// float -> bfloat16 rounding: checked bit for bit against the integer form
// ((u + 0x7fff + lsb) >> 16) over every non-NaN fp32 pattern; NaN stays NaN.
typedef float f32x2_cvt __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_cvt __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_cvt v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_cvt));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return (uint16_t)pack_bf16x2(f, 0.f); }

// Round a float to the model's storage precision and back (identity for f32).
template <typename T>
__device__ __forceinline__ float round_to(float v);
template <>
__device__ __forceinline__ float round_to<float>(float v) { return v; }
template <>
__device__ __forceinline__ float round_to<bf16>(float v) { return bf16_to_f32(f32_to_bf16(v)); }

template <typename T>
__device__ __forceinline__ float load_f32(const T* p, int64_t i);
template <>
__device__ __forceinline__ float load_f32<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_f32<bf16>(const bf16* p, int64_t i) { return bf16_to_f32(p[i].bits); }

template <typename T>
__device__ __forceinline__ void store_f32(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void store_f32<float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void store_f32<bf16>(bf16* p, int64_t i, float v) { p[i].bits = f32_to_bf16(v); }

// 16-byte vector of elements: 8 bf16 or 4 f32.
template <typename T>
struct Vec;
template <>
struct Vec<bf16> {
  static constexpr int N = 8;
};
template <>
struct Vec<float> {
  static constexpr int N = 4;
};

// 16-byte weight load. Weights are read once per step; MINITP_NT_LOADS=1
// marks the loads non-temporal (a cache-policy hint), 0 issues plain loads.
#ifndef MINITP_NT_LOADS
#define MINITP_NT_LOADS 1
#endif
// The pointer is cast to the global address space: weight pointers read from
// memory (a device-side table) would otherwise compile to flat loads, which
// also count against the LDS counter and so make every LDS wait of the wave
// wait for its streamed weights.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 global_u32x4;
__device__ __forceinline__ uint4 load_stream16(const uint4* p) {
#if MINITP_NT_LOADS
  u32x4 v = __builtin_nontemporal_load((global_u32x4*)(p));
#else
  u32x4 v = *(global_u32x4*)(p);
#endif
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void unpack16(const uint4& v, float* out, bf16*) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void unpack16(const uint4& v, float* out, float*) {
  out[0] = __uint_as_float(v.x);
  out[1] = __uint_as_float(v.y);
  out[2] = __uint_as_float(v.z);
  out[3] = __uint_as_float(v.w);
}

// Separately rounded multiply and add, for the places where the reference
// rounds each elementwise op on its own. HIP's __fmul_rn / __fadd_rn are
// plain operators that the compiler may contract into an FMA, so contraction
// is switched off here (and for the whole library in the Makefile; every
// intended fused multiply-add is written as fmaf).
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// SwiGLU on values already rounded to the dtype (mlp.py:38):
// silu(g) = g / (1 + exp(-g)) in fp32, rounded to the dtype, times up, rounded.
__device__ __forceinline__ float silu_f32(float g) { return __fdiv_rn(g, add_rn(1.0f, expf(-g))); }
template <typename T>
__device__ __forceinline__ float swiglu(float g, float u) {
  return round_to<T>(mul_rn(round_to<T>(silu_f32(g)), u));
}

// ---------------------------------------------------------------------------
// Wave64 reductions on DPP (data-parallel primitives run in the VALU, no LDS
// crossbar): an inclusive row scan with row_shr 1/2/4/8 leaves each 16-lane
// row's total in its lane 15, row_bcast15 / row_bcast31 fold the rows into
// lane 63, and readlane broadcasts it. Masked-off rows and out-of-row sources
// read `identity`, so they contribute nothing.
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp_f32(float identity, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, identity),
                                                               __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                               BANK_MASK, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0x111>(0.f, v);          // row_shr:1
  v += dpp_f32<0x112>(0.f, v);          // row_shr:2
  v += dpp_f32<0x114>(0.f, v);          // row_shr:4
  v += dpp_f32<0x118>(0.f, v);          // row_shr:8
  v += dpp_f32<0x142, 0xa>(0.f, v);     // row_bcast:15 into rows 1, 3
  v += dpp_f32<0x143, 0xc>(0.f, v);     // row_bcast:31 into rows 2, 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
  const float ninf = -__builtin_inff();
  v = fmaxf(v, dpp_f32<0x111>(ninf, v));
  v = fmaxf(v, dpp_f32<0x112>(ninf, v));
  v = fmaxf(v, dpp_f32<0x114>(ninf, v));
  v = fmaxf(v, dpp_f32<0x118>(ninf, v));
  v = fmaxf(v, dpp_f32<0x142, 0xa>(ninf, v));
  v = fmaxf(v, dpp_f32<0x143, 0xc>(ninf, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum over aligned groups of 4 lanes (quad_perm xor 1, xor 2); every lane of
// the group ends with the group total.
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp_f32<0xB1>(0.f, v);  // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(0.f, v);  // quad_perm [2,3,0,1]
  return v;
}
__device__ __forceinline__ float pair_sum(float v) { return v + dpp_f32<0xB1>(0.f, v); }

// torch.argmax order: NaN beats any number; equal values (and two NaNs)
// resolve to the smaller index.
__device__ __forceinline__ bool argmax_better(float va, int64_t ia, float vb, int64_t ib) {
  bool na = va != va, nb = vb != vb;
  if (na || nb) return na && (!nb || ia < ib);
  return va > vb || (va == vb && ia < ib);
}

__device__ __forceinline__ void wave_argmax(float& v, int64_t& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(v, o, 64);
    int64_t oi = __shfl_xor(i, o, 64);
    if (argmax_better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// ---------------------------------------------------------------------------
// Host side: status plumbing.
void set_error(const char* fmt, ...);

#define MINITP_CHECK_ARG(cond, ...)                     \
  do {                                                  \
    if (!(cond)) {                                      \
      ::minitp::set_error(__VA_ARGS__);                 \
      return MINITP_ERR_ARG;                            \
    }                                                   \
  } while (0)

#define MINITP_RETURN_HIP(call)                                                      \
  do {                                                                               \
    hipError_t _e = (call);                                                          \
    if (_e != hipSuccess) {                                                          \
      ::minitp::set_error("%s failed: %s", #call, hipGetErrorString(_e));             \
      return MINITP_ERR_HIP;                                                         \
    }                                                                                \
  } while (0)

// Check the launch status right after a <<<>>> launch.
#define MINITP_LAUNCH_CHECK() MINITP_RETURN_HIP(hipGetLastError())

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Buffer resource over [base, base + bytes): a load at a lane offset past
// the end returns zeros without touching memory, so kernels issue their
// loads unconditionally (a load behind a branch leaves a value to merge with
// the branch-free default, and the compiler places that merge, and the wait
// it implies, before the next loads it issues). Built from wave-uniform
// values made explicitly uniform, so the resource lives in scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  const int n = (int)__builtin_amdgcn_readfirstlane(bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, n, 0x00020000);
}

// Split-K partial products, fp32 [S][M][N] in the forward's GEMM workspace
// (launch_gemm_partials), handed to the kernel that consumes the product.
struct Partials {
  const float* p;
  int S;
  int64_t M, N;
};

// Sum over the splits of elements (row, col .. col + 7), added in split
// order (the order gemm_reduce_kernel uses), the loads of four splits in
// flight at a time. col and N multiples of 4.
__device__ __forceinline__ void sum_partials8(const Partials& q, int64_t row, int64_t col, float* v) {
  const int64_t mn = q.M * q.N, off = row * q.N + col;
  auto ld = [&](int s, float* o) {
    const float4 a = *(const float4*)(q.p + s * mn + off), b = *(const float4*)(q.p + s * mn + off + 4);
    o[0] = a.x;
    o[1] = a.y;
    o[2] = a.z;
    o[3] = a.w;
    o[4] = b.x;
    o[5] = b.y;
    o[6] = b.z;
    o[7] = b.w;
  };
  ld(0, v);
  int s = 1;
  for (; s + 4 <= q.S; s += 4) {
    float t[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) ld(s + u, t[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] += t[u][e];
  }
  for (; s < q.S; ++s) {
    float t[8];
    ld(s, t);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] += t[e];
  }
}

}  // namespace minitp
