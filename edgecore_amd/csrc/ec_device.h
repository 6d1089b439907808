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
#include "ec_quant.h"

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

// a * fp32(h) rounded once, for the binary16 h in the low (HI = 0) or high
// (HI = 1) half of w: one v_fma_mix_f32 with addend -0 instead of a convert
// and a multiply.  The fp16 operand converts exactly and x + (-0) == x for
// every x (signed zeros included), so the result equals a * h2f(h) bit for
// bit; written in asm because the compiler folds that fma back into the two
// instructions.
template <int HI>
__device__ __forceinline__ float mul_h(float a, uint32_t w) {
  const float mz = __builtin_bit_cast(float, 0x80000000u);
  float r;
  if constexpr (HI) asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(w), "v"(mz));
  else asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(w), "v"(mz));
  return r;
}

// s + a * fp32(h), the product rounded and then the add rounded (the
// reference's order, no fusion): mul_h and the add in one asm statement so
// that the product is consumed at once instead of being hoisted with all the
// others of a dot into registers
template <int HI>
__device__ __forceinline__ float mac_h(float s, float a, uint32_t w) {
  const float mz = __builtin_bit_cast(float, 0x80000000u);
  float p;
  if constexpr (HI)
    asm("v_fma_mix_f32 %1, %2, %3, %4 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\tv_add_f32 %0, %0, %1"
        : "+v"(s), "=&v"(p) : "v"(a), "v"(w), "v"(mz));
  else
    asm("v_fma_mix_f32 %1, %2, %3, %4 op_sel_hi:[0,1,0]\n\tv_add_f32 %0, %0, %1"
        : "+v"(s), "=&v"(p) : "v"(a), "v"(w), "v"(mz));
  return s;
}

// Two sequential dots at once: s0 += a[j] * fp32(k0[j]) and s1 += a[j] *
// fp32(k1[j]) for the eight binary16 elements j of the 16-byte chunks k0, k1
// (element j in the low (even j) or high half of dword j/2), in element
// order, each product rounded before its add (mul_h's product, then the add).
// One asm statement: the compiler pads every boundary between asm statements
// with a wait state, which per element would cost another instruction slot.
__device__ __forceinline__ void mac8x2(float &s0, float &s1, const float *a, v4u k0, v4u k1) {
  const float mz = __builtin_bit_cast(float, 0x80000000u);
  float t0, t1;
  asm(
      "v_fma_mix_f32 %[t0], %[a0], %[k00], %[mz] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[t1], %[a0], %[k10], %[mz] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_add_f32 %[s1], %[s1], %[t1]\n"
      "v_fma_mix_f32 %[t0], %[a1], %[k00], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[t1], %[a1], %[k10], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_add_f32 %[s1], %[s1], %[t1]\n"
      "v_fma_mix_f32 %[t0], %[a2], %[k01], %[mz] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[t1], %[a2], %[k11], %[mz] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_add_f32 %[s1], %[s1], %[t1]\n"
      "v_fma_mix_f32 %[t0], %[a3], %[k01], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[t1], %[a3], %[k11], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_add_f32 %[s1], %[s1], %[t1]\n"
      "v_fma_mix_f32 %[t0], %[a4], %[k02], %[mz] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[t1], %[a4], %[k12], %[mz] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_add_f32 %[s1], %[s1], %[t1]\n"
      "v_fma_mix_f32 %[t0], %[a5], %[k02], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[t1], %[a5], %[k12], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_add_f32 %[s1], %[s1], %[t1]\n"
      "v_fma_mix_f32 %[t0], %[a6], %[k03], %[mz] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[t1], %[a6], %[k13], %[mz] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_add_f32 %[s1], %[s1], %[t1]\n"
      "v_fma_mix_f32 %[t0], %[a7], %[k03], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[t1], %[a7], %[k13], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_add_f32 %[s1], %[s1], %[t1]\n"
      : [s0] "+v"(s0), [s1] "+v"(s1), [t0] "=&v"(t0), [t1] "=&v"(t1)
      : [a0] "v"(a[0]), [a1] "v"(a[1]), [a2] "v"(a[2]), [a3] "v"(a[3]), [a4] "v"(a[4]), [a5] "v"(a[5]),
        [a6] "v"(a[6]), [a7] "v"(a[7]), [k00] "v"(k0.x), [k01] "v"(k0.y), [k02] "v"(k0.z), [k03] "v"(k0.w),
        [k10] "v"(k1.x), [k11] "v"(k1.y), [k12] "v"(k1.z), [k13] "v"(k1.w), [mz] "v"(mz));
}
// one dot of mac8x2
__device__ __forceinline__ void mac8(float &s0, const float *a, v4u k0) {
  const float mz = __builtin_bit_cast(float, 0x80000000u);
  float t0;
  asm(
      "v_fma_mix_f32 %[t0], %[a0], %[k00], %[mz] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_fma_mix_f32 %[t0], %[a1], %[k00], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_fma_mix_f32 %[t0], %[a2], %[k01], %[mz] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_fma_mix_f32 %[t0], %[a3], %[k01], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_fma_mix_f32 %[t0], %[a4], %[k02], %[mz] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_fma_mix_f32 %[t0], %[a5], %[k02], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_fma_mix_f32 %[t0], %[a6], %[k03], %[mz] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      "v_fma_mix_f32 %[t0], %[a7], %[k03], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_add_f32 %[s0], %[s0], %[t0]\n"
      : [s0] "+v"(s0), [t0] "=&v"(t0)
      : [a0] "v"(a[0]), [a1] "v"(a[1]), [a2] "v"(a[2]), [a3] "v"(a[3]), [a4] "v"(a[4]), [a5] "v"(a[5]),
        [a6] "v"(a[6]), [a7] "v"(a[7]), [k00] "v"(k0.x), [k01] "v"(k0.y), [k02] "v"(k0.z), [k03] "v"(k0.w),
        [mz] "v"(mz));
}
// r[j] = a * fp32(h[j]) for the eight binary16 elements of the 16-byte chunk
// h (mul_h eight times, one asm statement)
__device__ __forceinline__ void mul8h(float *r, float a, v4u h) {
  const float mz = __builtin_bit_cast(float, 0x80000000u);
  asm(
      "v_fma_mix_f32 %[r0], %[a], %[h0], %[mz] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[r1], %[a], %[h0], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[r2], %[a], %[h1], %[mz] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[r3], %[a], %[h1], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[r4], %[a], %[h2], %[mz] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[r5], %[a], %[h2], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[r6], %[a], %[h3], %[mz] op_sel_hi:[0,1,0]\n"
      "v_fma_mix_f32 %[r7], %[a], %[h3], %[mz] op_sel:[0,1,0] op_sel_hi:[0,1,0]\n"
      : [r0] "=&v"(r[0]), [r1] "=&v"(r[1]), [r2] "=&v"(r[2]), [r3] "=&v"(r[3]), [r4] "=&v"(r[4]),
        [r5] "=&v"(r[5]), [r6] "=&v"(r[6]), [r7] "=&v"(r[7])
      : [a] "v"(a), [h0] "v"(h.x), [h1] "v"(h.y), [h2] "v"(h.z), [h3] "v"(h.w), [mz] "v"(mz));
}

template <bool BF16>
__device__ __forceinline__ float w2f(uint16_t w) {
  if constexpr (BF16) return b2f(w); else return h2f(w);
}

// src/gpt2.c:587-590, with the reference's expf (ec_expf.h); tab is the
// 2^(i/32) table (ec_exp2_32 or a copy of it in LDS)
__device__ __forceinline__ float silu(float x, const uint64_t *tab = ec_exp2_32) {
  float e = ec_expf_tab(-x, tab);
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

// Load of a value that is uniform across the block and not written while the
// kernel runs (positions, slots): through the constant address space, so the
// compiler emits a scalar load that needs no vector-memory wait.
template <typename T>
__device__ __forceinline__ T ld_uniform(const T *p) {
  return *(const __attribute__((address_space(4))) T *)(uintptr_t)p;
}

// The thread's index within the block, opaque to the compiler: values derived
// from it are not hoisted out of an enclosing loop (the persistent decode
// step runs whole kernels' bodies in a loop over layers, where hoisting every
// loop-invariant address computation exhausts the registers).
__device__ __forceinline__ int tid_opaque() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
// a wave-uniform int, likewise opaque
__device__ __forceinline__ int uniform_opaque(int v) {
  asm volatile("" : "+s"(v));
  return v;
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

// ---- DPP / readlane based reductions (every lane of the wave active) ----
// dpp_mov<CTRL>(v): v of the lane that the DPP control CTRL names
template <int CTRL, typename T>
__device__ __forceinline__ T dpp_mov(T v) {
  if constexpr (sizeof(T) == 8) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else {
    return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
  }
}
template <typename T>
__device__ __forceinline__ T readlane(T v, int l) {
  if constexpr (sizeof(T) == 8) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
  }
}
// sum over the wave: pairs, quads, rows of 8 and 16 by DPP, then the four
// rows of 16 in the order (r0 + r1) + (r2 + r3).  Every lane gets the result.
__device__ __forceinline__ double wave_sum_dpp(double v) {
  v = v + dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v = v + dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v = v + dpp_mov<0x141>(v);  // row_half_mirror
  v = v + dpp_mov<0x140>(v);  // row_mirror
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}
// Block reductions for blockDim.x == 256 with a single barrier.  `red` (4
// slots) must not be written by another reduction until every thread has
// passed one more barrier: callers alternate between slot sets or separate
// reuses with a barrier.
__device__ __forceinline__ double block_sum256_1b(double v, double *red) {
  v = wave_sum_dpp(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
// the same over NW waves (4 or 8), in a fixed pairwise order
template <int NW>
__device__ __forceinline__ double block_sum_1b(double v, double *red) {
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  v = wave_sum_dpp(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const double s4 = (red[0] + red[1]) + (red[2] + red[3]);
  if constexpr (NW == 4) return s4;
  else return s4 + ((red[4] + red[5]) + (red[6] + red[7]));
}
template <int NW>
__device__ __forceinline__ float block_max_1b(float v, float *red) {
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  v = wave_max_dpp(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float m4 = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  if constexpr (NW == 4) return m4;
  else return fmaxf(m4, fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7])));
}
__device__ __forceinline__ float block_max256_1b(float v, float *red) {
  v = wave_max_dpp(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// int8 quantization of one activation with the row scale s (ec_quant.h)
__device__ __forceinline__ int8_t quant1(float a, float s) { return ec_quant1(a, s); }

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
