// Shared device helpers for the gfx950 kernels of the MoE verification path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "specfit_amd.h"

#define SF_WAVE 64

typedef __bf16 sf_bf16x8 __attribute__((ext_vector_type(8)));
typedef float sf_f32x4 __attribute__((ext_vector_type(4)));

// bf16 bit pattern -> fp32 (exact).
__device__ __forceinline__ float sf_bf16_to_f32(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// fp32 -> bf16 bit pattern, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t sf_f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float sf_round_bf16(float f) {
  return sf_bf16_to_f32(sf_f32_to_bf16(f));
}

// exp(x) for x <= 0, used by the router softmax.  Cody-Waite reduction
// x = n*ln2 + r with |r| <= ln2/2, degree-7 Taylor polynomial of e^r in
// Horner form with explicit fused multiply-adds, scale by 2^n built from the
// exponent bits.  Results that would be below 2^-126 return 0, so the
// function never produces a subnormal.  The CPU oracle evaluates the same
// operation sequence, so both sides produce identical bits.
__device__ __forceinline__ float sf_exp_nonpos(float x) {
  if (!(x > -87.0f)) return 0.0f;  // also maps NaN to 0
  float n = __builtin_rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.42860682030941723e-06f, r);
  float p = 1.98412698412698413e-04f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-03f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-03f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-02f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = static_cast<int>(n);
  if (ni <= -126) return 0.0f;
  float scale = __uint_as_float(static_cast<uint32_t>(ni + 127) << 23);
  return p * scale;
}

__device__ __forceinline__ float sf_silu(float x) {
  return x / (1.0f + __expf(-x));
}

// Value of x in the lane that DPP control CTRL selects (a register move
// across lanes, no LDS).
template <int CTRL>
__device__ __forceinline__ float sf_dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float sf_readlane(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Sum of the 64 lanes' x by the xor butterfly over distances 1, 2, 4, 8,
// 16, 32 (v[l] += v[l ^ d]), bit for bit, returned wave-uniform.  IEEE
// addition is commutative, so after distance d every aligned group of 2d
// lanes holds one value; the half-row and row mirrors (lane i <-> 7-i,
// i <-> 15-i) then deliver the same value as lane i ^ 4 and i ^ 8, and the
// four rows (r0..r3) finish as (r0 + r1) + (r2 + r3).
__device__ __forceinline__ float sf_wave_sum(float x) {
  x += sf_dpp<0xB1>(x);   // quad_perm [1,0,3,2]: lane ^ 1
  x += sf_dpp<0x4E>(x);   // quad_perm [2,3,0,1]: lane ^ 2
  x += sf_dpp<0x141>(x);  // row_half_mirror
  x += sf_dpp<0x140>(x);  // row_mirror
  return (sf_readlane(x, 0) + sf_readlane(x, 16)) + (sf_readlane(x, 32) + sf_readlane(x, 48));
}

// Maximum of the 64 lanes' x (fmaxf; exact in any order), wave-uniform.
__device__ __forceinline__ float sf_wave_max(float x) {
  x = fmaxf(x, sf_dpp<0xB1>(x));
  x = fmaxf(x, sf_dpp<0x4E>(x));
  x = fmaxf(x, sf_dpp<0x141>(x));
  x = fmaxf(x, sf_dpp<0x140>(x));
  return fmaxf(fmaxf(sf_readlane(x, 0), sf_readlane(x, 16)),
               fmaxf(sf_readlane(x, 32), sf_readlane(x, 48)));
}

// Maximum of the 64 lanes' x (signed integers), wave-uniform.
__device__ __forceinline__ int sf_wave_max_int(int x) {
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xf, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xf, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x141, 0xf, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x140, 0xf, 0xf, false));
  return max(max(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
             max(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

#define SF_HIP_CHECK(expr)                                        \
  do {                                                            \
    hipError_t sf_err__ = (expr);                                 \
    if (sf_err__ != hipSuccess) return SF_ERR_HIP_BASE + (int)sf_err__; \
  } while (0)

#define SF_LAUNCH_CHECK() SF_HIP_CHECK(hipGetLastError())
