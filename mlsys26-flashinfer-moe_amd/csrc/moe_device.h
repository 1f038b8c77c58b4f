// Device helpers shared by the gfx950 kernels of libmoe_fp8.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Logistic function sigma(x) = 1 / (1 + e^-x) as a fixed sequence of IEEE fp32
// operations (no contraction), so that a host restatement with the same operations
// reproduces it bit for bit. e^y uses Cody-Waite range reduction y = n*ln2 + r with
// |r| <= ln2/2 and the degree-7 Taylor polynomial of e^r; y is clamped to [-80, 80],
// which keeps every intermediate a normal number (sigma saturates beyond |x| = 80).
// Reference: tl.sigmoid in moe_routing_kernel, kernel.py:466.
__device__ __forceinline__ float sigmoid_f32(float x) {
#pragma clang fp contract(off)
  const float kLog2e = 1.44269502162933349609375f;     // fp32(log2(e))
  const float kLn2Hi = 0.693359375f;                   // 355/512, exact in 9 bits
  const float kLn2Lo = -2.12194440e-4f;                // fp32(ln2 - kLn2Hi)
  float y = -x;
  y = (y > 80.0f) ? 80.0f : y;
  y = (y < -80.0f) ? -80.0f : y;
  const float n = __builtin_rintf(y * kLog2e);
  const float r = (y - n * kLn2Hi) - n * kLn2Lo;
  float p = 1.98412701e-4f;                            // 1/5040
  p = p * r + 1.38888892e-3f;                          // 1/720
  p = p * r + 8.33333377e-3f;                          // 1/120
  p = p * r + 4.16666679e-2f;                          // 1/24
  p = p * r + 1.66666672e-1f;                          // 1/6
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  const float e = __builtin_ldexpf(p, (int)n);
  return __fdiv_rn(1.0f, 1.0f + e);
}

// fp32 -> bf16 with round-to-nearest-even (torch's Tensor.copy_ semantics), NaN -> quiet NaN
// keeping the sign and the top payload bits: gfx950's v_cvt_pk_bf16_f32, two values per
// instruction. Over all 2^32 fp32 inputs it gives the bits of the integer form
// (u + 0x7fff + ((u >> 16) & 1)) >> 16, with (u >> 16) | 0x40 for a NaN (an exhaustive GPU
// comparison found no difference).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

__device__ __forceinline__ uint2 pack_bf16x4(float a, float b, float c, float d) {
  uint2 r;
  r.x = pack_bf16x2(a, b);
  r.y = pack_bf16x2(c, d);
  return r;
}

// Four fp32 -> four OCP e4m3fn bytes (round to nearest even), little-endian order a,b,c,d.
__device__ __forceinline__ uint32_t pack_fp8x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// D[16x16] (+)= A[16x128] * B[128x16], fp8 e4m3 operands, fp32 accumulate.
// Lane l supplies row (A) / column (B) l%16 and the 32 K-bytes [(l/16)*32, +32).
// The result lane l holds D[4*(l/16)+i][l%16], i = 0..3.
__device__ __forceinline__ v4f mfma16x16x128_fp8(const v8i& a, const v8i& b, const v4f& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// D[32x32] (+)= A[32x64] * B[64x32], fp8 e4m3 operands, fp32 accumulate.
// Lane l supplies row (A) / column (B) l%32 and the 32 K-bytes [(l/32)*32, +32).
// The result lane l holds D[8*(i/4) + 4*(l/32) + i%4][l%32], i = 0..15.
__device__ __forceinline__ v16f mfma32x32x64_fp8(const v8i& a, const v8i& b, const v16f& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ v8i join(const v4i& lo, const v4i& hi) {
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

__device__ __forceinline__ v4i lo_half(const v8i& v) {
  v4i r;
  r[0] = v[0]; r[1] = v[1]; r[2] = v[2]; r[3] = v[3];
  return r;
}

__device__ __forceinline__ v4i hi_half(const v8i& v) {
  v4i r;
  r[0] = v[4]; r[1] = v[5]; r[2] = v[6]; r[3] = v[7];
  return r;
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

}  // namespace moe
