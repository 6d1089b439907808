// Device-side helpers shared by the EdgeCore gfx950 kernels.
//
// All kernel sources are compiled with -ffp-contract=off: a product written
// a*b + c stays a rounded multiply followed by a rounded add, which is what
// the reference CPU code computes (it is built with -std=c11, reference
// Makefile:3).  Fused multiply-adds are written out with __builtin_fmaf
// where the reference itself uses an FMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ec_expf.h"

namespace ec {

constexpr int kWave = 64;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// binary16 bits -> fp32 (exact, v_cvt_f32_f16)
__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
// bfloat16 bits -> fp32 (exact shift)
__device__ __forceinline__ float b2f(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
// fp32 -> binary16 bits, round to nearest even (v_cvt_f16_f32, default mode)
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <bool BF16>
__device__ __forceinline__ float w2f(uint16_t w) {
  if constexpr (BF16) return b2f(w); else return h2f(w);
}

// src/gpt2.c:587-590, with the reference's expf (ec_expf.h)
__device__ __forceinline__ float silu(float x) {
  float e = ec_expf_ref(-x);
  float den = 1.0f + e;
  return x / den;
}

// src/gpt2.c:393-396; tanh computed in double and rounded once (glibc's
// tanhf differs from that by one ulp on ~5% of inputs)
__device__ __forceinline__ float gelu_new(float x) {
  float x3 = ((0.044715f * x) * x) * x;
  float u = 0.7978845608028654f * (x + x3);
  float t = (float)tanh((double)u);
  float hx = 0.5f * x;
  return hx * (1.0f + t);
}

// ---- wave / block reductions (wave64) ----
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Block-wide reductions for blockDim.x == 256 (4 waves).  `red` is shared
// scratch of at least 4 elements of T.  Deterministic: fixed tree shape.
template <typename T>
__device__ __forceinline__ T block_sum256(T v, T *red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ float block_max256(float v, float *red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// int8 quantization of one activation with the row scale s
// (src/gpt2.c:456-459: lrintf(a / s) clamped to [-128, 127]).  On x86-64,
// lrintf of NaN or of a magnitude >= 2^63 returns LONG_MIN, which clamps to
// -128; every other value rounds half to even and clamps.
__device__ __forceinline__ int8_t quant1(float a, float s) {
  const float r = __builtin_rintf(a / s);
  if (!(fabsf(r) < 9.2233720368547758e18f)) return (int8_t)-128;
  return (int8_t)(int)fminf(fmaxf(r, -128.0f), 127.0f);
}

// row scale of src/gpt2.c:453
__device__ __forceinline__ float quant_scale(float maxa) {
  return maxa > 0.0f ? maxa / 127.0f : 1.0f;
}

// int8 GEMM epilogue of src/kernels.c:160-165: bias + ((float)dot * as) * bs
__device__ __forceinline__ float i8_epilogue(int dot, float as, float bs, float bv) {
  float t = (float)dot;
  t = t * as;
  t = t * bs;
  return bv + t;
}

}  // namespace ec
