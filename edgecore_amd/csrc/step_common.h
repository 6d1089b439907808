// Exchange primitives of the persistent decode steps (decode_step.hip,
// decode_step_gpt2.hip): blocks hand results to each other through tagged
// 64-bit words -- (float value, step tag) written with one device-coherent
// store -- and a reader polls, with a bounded number of polls, until the words
// carry this step's tag.  The tag changes every step, so no buffer is ever
// cleared between steps.
#pragma once

#include "ec_device.h"
#include "ec_kernels.h"

namespace ec {

namespace {

constexpr int kSpin = 1 << 18;  // polls before a wait gives up (~0.3 s)

__device__ __forceinline__ void put_word(unsigned long long *p, float v, unsigned tag) {
  __hip_atomic_store(p, ((unsigned long long)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// The layers' pointers come from a table in memory, so the compiler cannot
// tell that they point at global memory and would load through flat
// instructions, which count in the LDS counter as well: every LDS wait after
// them would then wait for the weight stream too.  Loads go through these
// global-space views instead.
template <class T>
using gptr = const __attribute__((address_space(1))) T *;
template <class T>
__device__ __forceinline__ gptr<T> gbl(const T *p) {
  return (gptr<T>)p;
}
__device__ __forceinline__ gptr<v4i> gbl16(const void *p) { return (gptr<v4i>)p; }

// The exchange words are read in pairs, each pair with one 16-byte
// device-coherent load (n even, buf 16-byte aligned): a block reads 16 bytes
// per load instead of 8, and the exchanges' time grows with the bytes all
// waiting blocks read.  Each word is still written by one 8-byte store, so
// each half of a pair is one consistent (value, tag) snapshot.
// (buf and n are block-uniform; readfirstlane puts the descriptor in scalar
// registers, or the compiler wraps every load in a loop over distinct
// descriptors)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t xch_rsrc(const unsigned long long *buf, int n) {
  const uint64_t v = (uint64_t)(uintptr_t)buf;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  void *p = (void *)(uintptr_t)(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, 0, __builtin_amdgcn_readfirstlane(n * 8),
                                           0x00020000);
}
__device__ __forceinline__ v4u get_pair(__amdgpu_buffer_rsrc_t r, int p) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, p * 16, 0, 16 /* sc1: device-coherent */);
}

// Wait until words [0, n) of buf carry `tag`; thread t owns the pairs
// p = t + kStepThreads * j (j < WP), words 2p and 2p + 1, and receives their
// values in x[j].  The loads are issued together and reissued only for the
// pairs still missing.  Returns the pairs received (bit j); a pair missing
// after a timed-out wait reads as zeros.
template <int WP>
__device__ __forceinline__ unsigned wait_pairs(const unsigned long long *buf, int n, unsigned tag, float (&x)[WP][2],
                                               int *err) {
  const int t = threadIdx.x;
  const __amdgpu_buffer_rsrc_t rs = xch_rsrc(buf, n);
  unsigned pending = 0;
#pragma unroll
  for (int j = 0; j < WP; j++) {
    x[j][0] = x[j][1] = 0.0f;
    if (t + kStepThreads * j < (n >> 1)) pending |= 1u << j;
  }
  const unsigned own = pending;
  v4u v[WP];
  for (int it = 0; pending; it++) {
#pragma unroll
    for (int j = 0; j < WP; j++)
      if ((pending >> j) & 1u) v[j] = get_pair(rs, t + kStepThreads * j);
#pragma unroll
    for (int j = 0; j < WP; j++) {
      if (((pending >> j) & 1u) && v[j].y == tag && v[j].w == tag) {
        x[j][0] = __uint_as_float(v[j].x);
        x[j][1] = __uint_as_float(v[j].z);
        pending &= ~(1u << j);
      }
    }
    if (!pending) break;
    if (it >= kSpin) {
      atomicOr(err, 1);
      break;
    }
    if ((it & 63) == 63 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
    __builtin_amdgcn_s_sleep(1);
  }
  return own;
}

// Wait for words [0, n) of buf and put their values into dst (LDS).  Every
// thread of the block calls it; it starts with a barrier (dst is still being
// read by the previous phase) and ends with one.
template <int WP>
__device__ void gather(const unsigned long long *buf, int n, unsigned tag, float *dst, int *err) {
  const int t = threadIdx.x;
  __syncthreads();
  float x[WP][2];
  const unsigned own = wait_pairs<WP>(buf, n, tag, x, err);
#pragma unroll
  for (int j = 0; j < WP; j++)
    if ((own >> j) & 1u) *reinterpret_cast<float2 *>(dst + 2 * (t + kStepThreads * j)) = make_float2(x[j][0], x[j][1]);
  __syncthreads();
}

// Plain fp32 words, kStepFfEmpty until written (each word by one 4-byte
// store): wait until words [0, n) of buf (n % 4 == 0, buf 16-byte aligned)
// are all written and put them into dst (LDS).  Thread t owns the quads t +
// kStepThreads * j (j < WQ), one 16-byte device-coherent load each, reissued
// only for the quads still incomplete; a 16-byte load brings 4 values where
// a tagged pair brings 2.  Every thread of the block calls it; it starts and
// ends with a barrier, as gather does.
template <int WQ>
__device__ void gather_plain(const float *buf, int n, float *dst, int *err) {
  const int t = threadIdx.x;
  __syncthreads();
  const uint64_t bp = (uint64_t)(uintptr_t)buf;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)bp), hi = __builtin_amdgcn_readfirstlane((uint32_t)(bp >> 32));
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(uintptr_t)(((uint64_t)hi << 32) | lo), 0, __builtin_amdgcn_readfirstlane(n * 4), 0x00020000);
  unsigned pending = 0;
#pragma unroll
  for (int j = 0; j < WQ; j++)
    if (t + kStepThreads * j < (n >> 2)) pending |= 1u << j;
  v4u v[WQ];
  for (int it = 0; pending; it++) {
#pragma unroll
    for (int j = 0; j < WQ; j++)
      if ((pending >> j) & 1u)
        v[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, (t + kStepThreads * j) * 16, 0, 16 /* sc1 */);
#pragma unroll
    for (int j = 0; j < WQ; j++) {
      if (((pending >> j) & 1u) && v[j].x != kStepFfEmpty && v[j].y != kStepFfEmpty && v[j].z != kStepFfEmpty &&
          v[j].w != kStepFfEmpty) {
        *reinterpret_cast<v4u *>(dst + 4 * (t + kStepThreads * j)) = v[j];
        pending &= ~(1u << j);
      }
    }
    if (!pending) break;
    if (it >= kSpin) {
      atomicOr(err, 1);
      break;
    }
    if ((it & 63) == 63 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
    __builtin_amdgcn_s_sleep(1);
  }
  __syncthreads();
}

__device__ __forceinline__ void put_plain(float *p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t *>(p), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

}  // namespace ec
