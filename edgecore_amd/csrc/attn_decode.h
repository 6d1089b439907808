// Decode attention of one (head, token) -- or one element slice of it --
// as a block-level device function, shared by the attention kernel
// (kernels.hip) and the persistent decode step (decode_step.hip).
#pragma once

#include "ec_device.h"
#include "ec_kernels.h"

#include <float.h>

namespace ec {

// One block per (head, token), reproducing the reference's arithmetic in its
// order: each score is one thread's sequential fp32 dot over head_dim (a
// rounded product, then a rounded add), scaled in double; max; e = expf(s -
// max) with the reference's expf; double sum; p = (float)(e * (1/sum)); each
// output element is a sequential fp32 sum over positions of the rounded
// products p*v.  The int8 path turns any last-bit difference here into
// different activation codes downstream, so the order is kept exactly.
//
// Work split: the products p*v of a tile of `vtile` positions are formed by
// all 256 threads into LDS, laid out [position/4][d][position%4] with the d
// index XOR-swizzled by the quad index (no bank conflicts on either side), so
// the thread owning output element d runs its sequential sum reading four
// positions per 16-byte LDS load.  With HD > 0 (head_dim fixed at compile
// time, 16-byte loads) the K rows of the first positions and the first V
// tile are read with coalesced loads (8 lanes per 128-byte row) issued at the
// start, unconditionally (indices clamped into the attended range), after the
// q/k/v elements: the hardware's in-order load counter then lets each phase
// wait for its own data only.  The K rows go through LDS (swizzled 16-byte
// chunks) so that each score is still one thread's sequential dot.  HD == 0
// is the generic path.
//
// FUSED: the block also rotates its q head and the token's new k (RoPE,
// src/gpt2.c:656-665, double cos/sin table) and uses the new k and v rounded
// to fp16 for the token's own position; the first query head of each KV group
// appends them to the cache (src/gpt2.c:726-741).  Only valid when no other
// token of the launch reads this token's slot.

// Sequential sum of the decode attention's output element: o += the four
// floats of each of 8*n8 quads (n8 >= 1), quad j at LDS byte address
// a + j*STRIDE, in order.  The loads of the next four quads are in flight
// while the current four are added, with one wait per two quads; the
// compiler's own schedule of this loop waits for every outstanding load at
// the top of each iteration.  Reads 4 quads past the end (values unused).
template <int STRIDE>
__device__ __forceinline__ float attn_chain8(float o, uint32_t a, int n8) {
  asm volatile(
      "ds_read_b128 v[224:227], %[a] offset:%[q0]\n"
      "ds_read_b128 v[228:231], %[a] offset:%[q1]\n"
      "ds_read_b128 v[232:235], %[a] offset:%[q2]\n"
      "ds_read_b128 v[236:239], %[a] offset:%[q3]\n"
      "L_attn_chain%=:\n"
      "ds_read_b128 v[240:243], %[a] offset:%[q4]\n"
      "ds_read_b128 v[244:247], %[a] offset:%[q5]\n"
      "ds_read_b128 v[248:251], %[a] offset:%[q6]\n"
      "ds_read_b128 v[252:255], %[a] offset:%[q7]\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_add_f32 %[o], %[o], v224\n"
      "v_add_f32 %[o], %[o], v225\n"
      "v_add_f32 %[o], %[o], v226\n"
      "v_add_f32 %[o], %[o], v227\n"
      "v_add_f32 %[o], %[o], v228\n"
      "v_add_f32 %[o], %[o], v229\n"
      "v_add_f32 %[o], %[o], v230\n"
      "v_add_f32 %[o], %[o], v231\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[o], %[o], v232\n"
      "v_add_f32 %[o], %[o], v233\n"
      "v_add_f32 %[o], %[o], v234\n"
      "v_add_f32 %[o], %[o], v235\n"
      "v_add_f32 %[o], %[o], v236\n"
      "v_add_f32 %[o], %[o], v237\n"
      "v_add_f32 %[o], %[o], v238\n"
      "v_add_f32 %[o], %[o], v239\n"
      "ds_read_b128 v[224:227], %[a] offset:%[q8]\n"
      "ds_read_b128 v[228:231], %[a] offset:%[q9]\n"
      "ds_read_b128 v[232:235], %[a] offset:%[q10]\n"
      "ds_read_b128 v[236:239], %[a] offset:%[q11]\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_add_f32 %[o], %[o], v240\n"
      "v_add_f32 %[o], %[o], v241\n"
      "v_add_f32 %[o], %[o], v242\n"
      "v_add_f32 %[o], %[o], v243\n"
      "v_add_f32 %[o], %[o], v244\n"
      "v_add_f32 %[o], %[o], v245\n"
      "v_add_f32 %[o], %[o], v246\n"
      "v_add_f32 %[o], %[o], v247\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[o], %[o], v248\n"
      "v_add_f32 %[o], %[o], v249\n"
      "v_add_f32 %[o], %[o], v250\n"
      "v_add_f32 %[o], %[o], v251\n"
      "v_add_f32 %[o], %[o], v252\n"
      "v_add_f32 %[o], %[o], v253\n"
      "v_add_f32 %[o], %[o], v254\n"
      "v_add_f32 %[o], %[o], v255\n"
      "v_add_u32 %[a], %[inc], %[a]\n"
      "s_sub_u32 %[n], %[n], 1\n"
      "s_cmp_lg_u32 %[n], 0\n"
      "s_cbranch_scc1 L_attn_chain%=\n"
      "s_waitcnt lgkmcnt(0)\n"
      : [o] "+v"(o), [a] "+v"(a), [n] "+s"(n8)
      : [inc] "v"(8 * STRIDE), [q0] "i"(0 * STRIDE), [q1] "i"(1 * STRIDE), [q2] "i"(2 * STRIDE), [q3] "i"(3 * STRIDE), [q4] "i"(4 * STRIDE), [q5] "i"(5 * STRIDE), [q6] "i"(6 * STRIDE), [q7] "i"(7 * STRIDE), [q8] "i"(8 * STRIDE), [q9] "i"(9 * STRIDE), [q10] "i"(10 * STRIDE), [q11] "i"(11 * STRIDE)
      : "v224", "v225", "v226", "v227", "v228", "v229", "v230", "v231", "v232", "v233", "v234", "v235", "v236", "v237", "v238", "v239", "v240", "v241", "v242", "v243", "v244", "v245", "v246", "v247", "v248", "v249", "v250", "v251", "v252", "v253", "v254", "v255", "scc", "memory");
  return o;
}

// As attn_chain8, 16 quads per iteration (n16 >= 1) in four register sets:
// the reads of the next 12 quads are in flight while the current four quads
// are added, one wait per four quads.  Reads 16 quads past the end (values
// unused).
template <int STRIDE>
__device__ __forceinline__ float attn_chain16(float o, uint32_t a, int n16) {
  static_assert(31 * STRIDE <= 65535, "ds_read offsets are 16-bit");
  asm volatile(
      "ds_read_b128 v[192:195], %[a] offset:%[q0]\n"
      "ds_read_b128 v[196:199], %[a] offset:%[q1]\n"
      "ds_read_b128 v[200:203], %[a] offset:%[q2]\n"
      "ds_read_b128 v[204:207], %[a] offset:%[q3]\n"
      "ds_read_b128 v[208:211], %[a] offset:%[q4]\n"
      "ds_read_b128 v[212:215], %[a] offset:%[q5]\n"
      "ds_read_b128 v[216:219], %[a] offset:%[q6]\n"
      "ds_read_b128 v[220:223], %[a] offset:%[q7]\n"
      "ds_read_b128 v[224:227], %[a] offset:%[q8]\n"
      "ds_read_b128 v[228:231], %[a] offset:%[q9]\n"
      "ds_read_b128 v[232:235], %[a] offset:%[q10]\n"
      "ds_read_b128 v[236:239], %[a] offset:%[q11]\n"
      "ds_read_b128 v[240:243], %[a] offset:%[q12]\n"
      "ds_read_b128 v[244:247], %[a] offset:%[q13]\n"
      "ds_read_b128 v[248:251], %[a] offset:%[q14]\n"
      "ds_read_b128 v[252:255], %[a] offset:%[q15]\n"
      "L_attn_chain16_%=:\n"
      "s_waitcnt lgkmcnt(12)\n"
      "v_add_f32 %[o], %[o], v192\n"
      "v_add_f32 %[o], %[o], v193\n"
      "v_add_f32 %[o], %[o], v194\n"
      "v_add_f32 %[o], %[o], v195\n"
      "v_add_f32 %[o], %[o], v196\n"
      "v_add_f32 %[o], %[o], v197\n"
      "v_add_f32 %[o], %[o], v198\n"
      "v_add_f32 %[o], %[o], v199\n"
      "v_add_f32 %[o], %[o], v200\n"
      "v_add_f32 %[o], %[o], v201\n"
      "v_add_f32 %[o], %[o], v202\n"
      "v_add_f32 %[o], %[o], v203\n"
      "v_add_f32 %[o], %[o], v204\n"
      "v_add_f32 %[o], %[o], v205\n"
      "v_add_f32 %[o], %[o], v206\n"
      "v_add_f32 %[o], %[o], v207\n"
      "ds_read_b128 v[192:195], %[a] offset:%[q16]\n"
      "ds_read_b128 v[196:199], %[a] offset:%[q17]\n"
      "ds_read_b128 v[200:203], %[a] offset:%[q18]\n"
      "ds_read_b128 v[204:207], %[a] offset:%[q19]\n"
      "s_waitcnt lgkmcnt(12)\n"
      "v_add_f32 %[o], %[o], v208\n"
      "v_add_f32 %[o], %[o], v209\n"
      "v_add_f32 %[o], %[o], v210\n"
      "v_add_f32 %[o], %[o], v211\n"
      "v_add_f32 %[o], %[o], v212\n"
      "v_add_f32 %[o], %[o], v213\n"
      "v_add_f32 %[o], %[o], v214\n"
      "v_add_f32 %[o], %[o], v215\n"
      "v_add_f32 %[o], %[o], v216\n"
      "v_add_f32 %[o], %[o], v217\n"
      "v_add_f32 %[o], %[o], v218\n"
      "v_add_f32 %[o], %[o], v219\n"
      "v_add_f32 %[o], %[o], v220\n"
      "v_add_f32 %[o], %[o], v221\n"
      "v_add_f32 %[o], %[o], v222\n"
      "v_add_f32 %[o], %[o], v223\n"
      "ds_read_b128 v[208:211], %[a] offset:%[q20]\n"
      "ds_read_b128 v[212:215], %[a] offset:%[q21]\n"
      "ds_read_b128 v[216:219], %[a] offset:%[q22]\n"
      "ds_read_b128 v[220:223], %[a] offset:%[q23]\n"
      "s_waitcnt lgkmcnt(12)\n"
      "v_add_f32 %[o], %[o], v224\n"
      "v_add_f32 %[o], %[o], v225\n"
      "v_add_f32 %[o], %[o], v226\n"
      "v_add_f32 %[o], %[o], v227\n"
      "v_add_f32 %[o], %[o], v228\n"
      "v_add_f32 %[o], %[o], v229\n"
      "v_add_f32 %[o], %[o], v230\n"
      "v_add_f32 %[o], %[o], v231\n"
      "v_add_f32 %[o], %[o], v232\n"
      "v_add_f32 %[o], %[o], v233\n"
      "v_add_f32 %[o], %[o], v234\n"
      "v_add_f32 %[o], %[o], v235\n"
      "v_add_f32 %[o], %[o], v236\n"
      "v_add_f32 %[o], %[o], v237\n"
      "v_add_f32 %[o], %[o], v238\n"
      "v_add_f32 %[o], %[o], v239\n"
      "ds_read_b128 v[224:227], %[a] offset:%[q24]\n"
      "ds_read_b128 v[228:231], %[a] offset:%[q25]\n"
      "ds_read_b128 v[232:235], %[a] offset:%[q26]\n"
      "ds_read_b128 v[236:239], %[a] offset:%[q27]\n"
      "s_waitcnt lgkmcnt(12)\n"
      "v_add_f32 %[o], %[o], v240\n"
      "v_add_f32 %[o], %[o], v241\n"
      "v_add_f32 %[o], %[o], v242\n"
      "v_add_f32 %[o], %[o], v243\n"
      "v_add_f32 %[o], %[o], v244\n"
      "v_add_f32 %[o], %[o], v245\n"
      "v_add_f32 %[o], %[o], v246\n"
      "v_add_f32 %[o], %[o], v247\n"
      "v_add_f32 %[o], %[o], v248\n"
      "v_add_f32 %[o], %[o], v249\n"
      "v_add_f32 %[o], %[o], v250\n"
      "v_add_f32 %[o], %[o], v251\n"
      "v_add_f32 %[o], %[o], v252\n"
      "v_add_f32 %[o], %[o], v253\n"
      "v_add_f32 %[o], %[o], v254\n"
      "v_add_f32 %[o], %[o], v255\n"
      "ds_read_b128 v[240:243], %[a] offset:%[q28]\n"
      "ds_read_b128 v[244:247], %[a] offset:%[q29]\n"
      "ds_read_b128 v[248:251], %[a] offset:%[q30]\n"
      "ds_read_b128 v[252:255], %[a] offset:%[q31]\n"
      "v_add_u32 %[a], %[inc], %[a]\n"
      "s_sub_u32 %[n], %[n], 1\n"
      "s_cmp_lg_u32 %[n], 0\n"
      "s_cbranch_scc1 L_attn_chain16_%=\n"
      "s_waitcnt lgkmcnt(0)\n"
      : [o] "+v"(o), [a] "+v"(a), [n] "+s"(n16)
      : [inc] "v"(16 * STRIDE), [q0] "i"(0 * STRIDE), [q1] "i"(1 * STRIDE), [q2] "i"(2 * STRIDE), [q3] "i"(3 * STRIDE), [q4] "i"(4 * STRIDE), [q5] "i"(5 * STRIDE), [q6] "i"(6 * STRIDE), [q7] "i"(7 * STRIDE), [q8] "i"(8 * STRIDE), [q9] "i"(9 * STRIDE), [q10] "i"(10 * STRIDE), [q11] "i"(11 * STRIDE), [q12] "i"(12 * STRIDE), [q13] "i"(13 * STRIDE), [q14] "i"(14 * STRIDE), [q15] "i"(15 * STRIDE), [q16] "i"(16 * STRIDE), [q17] "i"(17 * STRIDE), [q18] "i"(18 * STRIDE), [q19] "i"(19 * STRIDE), [q20] "i"(20 * STRIDE), [q21] "i"(21 * STRIDE), [q22] "i"(22 * STRIDE), [q23] "i"(23 * STRIDE), [q24] "i"(24 * STRIDE), [q25] "i"(25 * STRIDE), [q26] "i"(26 * STRIDE), [q27] "i"(27 * STRIDE), [q28] "i"(28 * STRIDE), [q29] "i"(29 * STRIDE), [q30] "i"(30 * STRIDE), [q31] "i"(31 * STRIDE)
      : "v192", "v193", "v194", "v195", "v196", "v197", "v198", "v199", "v200", "v201", "v202", "v203", "v204", "v205", "v206", "v207", "v208", "v209", "v210", "v211", "v212", "v213", "v214", "v215", "v216", "v217", "v218", "v219", "v220", "v221", "v222", "v223", "v224", "v225", "v226", "v227", "v228", "v229", "v230", "v231", "v232", "v233", "v234", "v235", "v236", "v237", "v238", "v239", "v240", "v241", "v242", "v243", "v244", "v245", "v246", "v247", "v248", "v249", "v250", "v251", "v252", "v253", "v254", "v255", "scc", "memory");
  return o;
}

// o += the four floats of each of the 4 quads at LDS byte address a + j*STRIDE,
// in order; the four reads are issued together (no read past the last quad)
template <int STRIDE>
__device__ __forceinline__ float attn_sum4(float o, uint32_t a) {
  asm volatile(
      "ds_read_b128 v[240:243], %[a]\n"
      "ds_read_b128 v[244:247], %[a] offset:%[q1]\n"
      "ds_read_b128 v[248:251], %[a] offset:%[q2]\n"
      "ds_read_b128 v[252:255], %[a] offset:%[q3]\n"
      "s_waitcnt lgkmcnt(3)\n"
      "v_add_f32 %[o], %[o], v240\n"
      "v_add_f32 %[o], %[o], v241\n"
      "v_add_f32 %[o], %[o], v242\n"
      "v_add_f32 %[o], %[o], v243\n"
      "s_waitcnt lgkmcnt(2)\n"
      "v_add_f32 %[o], %[o], v244\n"
      "v_add_f32 %[o], %[o], v245\n"
      "v_add_f32 %[o], %[o], v246\n"
      "v_add_f32 %[o], %[o], v247\n"
      "s_waitcnt lgkmcnt(1)\n"
      "v_add_f32 %[o], %[o], v248\n"
      "v_add_f32 %[o], %[o], v249\n"
      "v_add_f32 %[o], %[o], v250\n"
      "v_add_f32 %[o], %[o], v251\n"
      "s_waitcnt lgkmcnt(0)\n"
      "v_add_f32 %[o], %[o], v252\n"
      "v_add_f32 %[o], %[o], v253\n"
      "v_add_f32 %[o], %[o], v254\n"
      "v_add_f32 %[o], %[o], v255\n"
      : [o] "+v"(o)
      : [a] "v"(a), [q1] "i"(STRIDE), [q2] "i"(2 * STRIDE), [q3] "i"(3 * STRIDE)
      : "v240", "v241", "v242", "v243", "v244", "v245", "v246", "v247", "v248", "v249", "v250", "v251", "v252",
        "v253", "v254", "v255", "memory");
  return o;
}

template <int HD>
__device__ __forceinline__ float dot_k_row(const float *qs, const uint16_t *kp, int hd) {
  float s = 0.0f;
  if constexpr (HD > 0) {
    v4u kk[HD / 8];
#pragma unroll
    for (int c = 0; c < HD / 8; c++) kk[c] = *reinterpret_cast<const v4u *>(kp + 8 * c);
#pragma unroll
    for (int c = 0; c < HD / 8; c++) {
      const uint32_t wv[4] = {kk[c].x, kk[c].y, kk[c].z, kk[c].w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        s = mac_h<0>(s, qs[8 * c + 2 * j], wv[j]);
        s = mac_h<1>(s, qs[8 * c + 2 * j + 1], wv[j]);
      }
    }
  } else {
    for (int d = 0; d < hd; d++) {
      const float p0 = qs[d] * h2f(kp[d]);
      s = s + p0;
    }
  }
  return s;
}

// the own position's score from the fp16-rounded new k in LDS (one thread;
// unrolled with 16-byte reads, since every wave waits for it at the next
// barrier)
template <int HD>
__device__ __forceinline__ float dot_new_k(const float *qs, const float *kn, int hd) {
  float s = 0.0f;
  if constexpr (HD > 0) {
#pragma unroll
    for (int c = 0; c < HD / 4; c++) {
      const float4 q4 = *reinterpret_cast<const float4 *>(qs + 4 * c);
      const float4 k4 = *reinterpret_cast<const float4 *>(kn + 4 * c);
      const float p0 = q4.x * k4.x, p1 = q4.y * k4.y, p2 = q4.z * k4.z, p3 = q4.w * k4.w;
      s = s + p0;
      s = s + p1;
      s = s + p2;
      s = s + p3;
    }
  } else {
    for (int d = 0; d < hd; d++) {
      const float p0 = qs[d] * kn[d];
      s = s + p0;
    }
  }
  return s;
}

// stages of the decode attention's products for the largest tile (timed at
// 2, 3 and 6 stages for head_dim 64 at 504 positions: 8.0k, 7.6k and 8.4k
// cycles)
constexpr int kAttnStages = 3;

// 16-byte slots per quad of a slice's products (hs elements): 16 consecutive
// lanes of the writes and of the sums' reads hit distinct bank slots
__host__ __device__ constexpr inline int attn_spitch(int hs) { return hs <= 16 ? hs + 1 : attn_pitch(hs, 0); }
__host__ __device__ constexpr inline int attn_sswz(int hs) { return hs <= 16 ? 0 : attn_swz(hs, 0); }

// NS: element slices per head, one block each (1, or 2 / 4 for head_dim 64):
// every block of a head scores all positions, and forms the products and
// sums of its slice's elements only
// The body of one block: the attention of query head h (element slice
// `slice` of NS) of token m, reading the token's q row (qrow, head h) and new
// k / v rows (krow / vrow, its KV group) from global or shared memory;
// out(i, o) receives element i of the slice (i < hd / NS) from thread i.
// coff is added to every cache index (a layer's offset when a.kc / a.vc
// point at layer 0).
// Every thread of the block (NS > 1 ? 512 : 256) must call it.
// SCORED: steps 1-4 are skipped; the scores of (m, h) come from
// a.scores[(m * H + h) * sc_ld + i] (position lo + i), written by the scores
// pass with this body's arithmetic, and the cache already holds the token's k
// and v (FUSED must be false).
// PREK (the persistent step): the K rows of positions [lo, lo + min(n - 1,
// KQ)) are already in the K tile (attn_prefetch_k, waited for by the caller
// before its last barrier); the body loads and writes only the rest.
// mk(e) (optional) is called by every thread at phase boundaries, for a
// caller's timestamps: 0 the scores start, 1 the softmax starts, 2 the
// products and sums start, 3 and 4 the first tile's second and third stages
// start.
struct NoMark {
  __device__ void operator()(int) const {}
};
// The RoPE table entry that thread t's element uses (FUSED: rotated elements
// their pair's index, the others entry 0; rot = the rotated half or 0).
__device__ __forceinline__ int attn_rope_entry(int t, int hd, int rot) {
  const int tt = min(t, hd - 1);
  const bool rr = tt < 2 * rot;
  const int i0 = rr ? (tt < rot ? tt : tt - rot) : tt;
  return rr ? i0 : 0;
}
// Values a caller that runs the body for one token many times (the
// persistent step, once per layer) keeps in LDS: the 2^(i/32) table of
// ec_expf_tab, and thread t's (cos, sin) at the token's position, cs[t] =
// a.cs[pos * half + attn_rope_entry(t, hd, rot)] for t < hd.
struct AttnPre {
  const uint64_t *etab;
  const double2 *cs;
};
template <int HD, bool FUSED, int NS, bool SCORED = false, bool PREK = false, class Out, class Mark = NoMark>
__device__ __forceinline__ void attn_decode_block(const AttnArgs &a, int m, int h, int slice, const float *qrow,
                                                  const float *krow, const float *vrow, float *lds, Out &&out,
                                                  size_t coff = 0, Mark mk = Mark{}, const AttnPre *pre = nullptr) {
  static_assert(NS == 1 || (HD == 64 && (NS == 2 || NS == 4 || NS == 8)), "element slices: head_dim 64, 2 / 4 / 8");
  static_assert(!(SCORED && FUSED), "the scores pass appends the new k / v");
  // threads per block: 512 with element slices (one scored position per
  // thread up to 512 positions) and for the scored head_dim 128 body (six
  // product waves beside the two summing waves), else 256
  constexpr int NT = attn_threads(HD, NS, SCORED);
  // threads over which the softmax's double sum is partitioned (thread t:
  // positions t, t + SP, ...; then the fixed tree over SP / 64 waves): the
  // scored head_dim 128 body keeps the one-pass body's 256, so both give the
  // same sum bit for bit
  constexpr int SP = (SCORED && HD == 128) ? 256 : NT;
  constexpr int KU = NT == 512 ? kAttnUnits / 2 : kAttnUnits;  // K units per thread
  __shared__ float redf[NT / 64];
  __shared__ double redd[NT / 64];
  __shared__ uint64_t etab[32];  // expf table
  constexpr int CPR = HD > 0 ? HD / 8 : 1;         // 16-byte chunks per K/V row
  constexpr int HS = HD > 0 ? HD / NS : 0;  // elements of this block's slice
  constexpr int CPRV = HD > 0 ? CPR / NS : 1;  // 16-byte V chunks per slice
  const int t = tid_opaque();
  const int pos = ld_uniform(a.pos + m), slot = ld_uniform(a.slot + m);
  uint64_t et = 0;
  if (!pre) et = ec_exp2_32[t & 31];
  const uint64_t *etp = pre ? pre->etab : etab;
  const int kvh = h * a.KVH / a.H;
  int lo = 0;
  if (a.window > 0) {
    lo = pos - a.window + 1;
    if (lo < 0) lo = 0;
  }
  const int n = pos + 1 - lo;
  const int hd = HD > 0 ? HD : a.hd, T = a.vtile;
  const int hdp = (hd + 3) & ~3;
  float *qs = lds;
  float *kn = qs + hdp;  // FUSED: the new k, fp16-rounded
  float *vn = kn + hdp;  // FUSED: the new v, fp16-rounded
  float *sc = vn + hdp;
  float *prod = sc + ((a.max_npos + 3) & ~3);  // [T/4][P][4]
  const int PA = attn_pitch(hd, a.kv);        // 16-byte slots per quad of the product area
  const int P = NS > 1 ? attn_spitch(HS) : PA;  // slots per quad of this slice's products
  const size_t cbase = coff + (size_t)slot * a.C * a.kv + (size_t)kvh * hd;
  const uint16_t *K = a.kc + cbase + (size_t)lo * a.kv;
  const uint16_t *V = a.vc + cbase + (size_t)lo * a.kv;
  const int ncache = FUSED ? n - 1 : n;  // positions read from the cache
  const int last = ncache > 0 ? ncache - 1 : 0;  // clamp target of the unconditional loads

  // ---- 1. this thread's element of q (and of the new k and v) ----
  // Branch-free loads (index clamped into the head) so that every load of
  // steps 1-2 is issued before the first wait.
  const int rot = (FUSED && a.cs) ? a.half : 0;
  const int tt = min(t, hd - 1);
  const bool rr = tt < 2 * rot;  // element of the rotated part
  const int i0 = rr ? (tt < rot ? tt : tt - rot) : tt, i1 = rr ? i0 + rot : tt;
  const float qa = qrow[i0], qb = qrow[i1];
  float ka = 0.0f, kb = 0.0f, vv = 0.0f;
  double2 c2 = make_double2(1.0, 0.0);
  if constexpr (FUSED) {
    ka = krow[i0];
    kb = krow[i1];
    vv = vrow[tt];
    if (rot) c2 = pre ? pre->cs[tt] : a.cs[(size_t)pos * a.half + (rr ? i0 : 0)];
  }

  // ---- 2. K rows of the first KQ positions ----
  // unit = 4 positions x 8 elements (16 bytes each); KU per thread
  constexpr int KQMAX = HD > 0 ? NT * KU * 4 / CPR : 0;  // K positions staged
  constexpr int KP = CPR + 1;  // K tile row pitch in 16-byte chunks (odd: rows spread over the banks)
  // the K tile lives in the product area (T/4 * P slots of 16 bytes)
  const int KQ = min(KQMAX, (T / 4) * PA / KP);
  // V: the product threads (all but the first SWV waves, which hold the
  // output elements) keep the tile's V in registers in units of 4 positions x
  // 8 elements: QPU quads per unit index across the product threads, UPS units
  // per thread and stage of SQ quads, NSTG stages for the largest tile
  constexpr int SWV = HD > 64 ? HD / 64 : 1;
  constexpr int NPT = NT - 64 * SWV;
  constexpr int QPU = HD > 0 ? NPT / CPRV : 1;
  constexpr int MAXQ = HD > 0 ? (KQMAX < 512 ? KQMAX : 512) / 4 : 1;
  constexpr int UPS = (MAXQ + kAttnStages * QPU - 1) / (kAttnStages * QPU);
  constexpr int SQ = UPS * QPU;
  // The first stage is shorter (32 quads) when one unit per thread covers a
  // whole stage (element slices): its products are ready sooner and the sums
  // start earlier; stage s >= 1 covers quads [Q0 + SQ*(s-1), Q0 + SQ*s).
  constexpr int Q0 = (UPS == 1 && QPU >= 96) ? 32 : SQ;
  constexpr int NSTG = 1 + (MAXQ - Q0 + SQ - 1) / SQ;
  auto stage_lo = [](int s) { return s == 0 ? 0 : Q0 + SQ * (s - 1); };
  static_assert(HD == 0 || NPT % CPRV == 0, "product threads cover whole quads");
  const int pt = t - 64 * SWV;  // product thread index (negative in the summing waves)
  v4u vr[NSTG * UPS][4];
  // this product thread's V units of stage s of the tile at t0
  auto load_v_stage = [&](int t0, int s) {
    if (HD > 0 && pt >= 0) {
      const int qd0 = pt / CPRV, cd = pt - qd0 * CPRV;
#pragma unroll
      for (int u = 0; u < UPS; u++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int i = min(t0 + 4 * (stage_lo(s) + QPU * u + qd0) + e, last);
          vr[s * UPS + u][e] = *reinterpret_cast<const v4u *>(V + (size_t)i * a.kv + 8 * (CPRV * slice + cd));
        }
      }
    }
  };
  auto load_v = [&](int t0) {  // ... of every stage
#pragma unroll
    for (int s = 0; s < NSTG; s++) load_v_stage(t0, s);
  };
  // PREK with the whole context in one product tile: the product threads read
  // V from the V tile in LDS (attn_prefetch_v) instead of loading registers
  const bool vpre = PREK && HD == 64 && NS > 1 && n <= T;
  const v4u *vtl = reinterpret_cast<const v4u *>(reinterpret_cast<const char *>(prod) + step_vtile_off(T, a.kv));
  float mx = -FLT_MAX;
  if constexpr (SCORED) {
    // the scores into LDS and their maximum, 8 loads per thread in flight at
    // a time (unconditional, clamped into the row) with the first tile's V
    // issued behind the first batch: loaded one at a time behind V, C4's
    // 2080 scores took five round trips (~1.7-2.5 us before the softmax)
    if (!pre && t < 32) etab[t] = et;
    const float *src = a.scores + ((size_t)m * a.H + h) * a.sc_ld;
    constexpr int SB = 8;
    auto batch = [&](int base, float (&v)[SB]) {
#pragma unroll
      for (int k = 0; k < SB; k++) v[k] = src[min(base + t + NT * k, n - 1)];
    };
    auto keep = [&](int base, const float (&v)[SB]) {
#pragma unroll
      for (int k = 0; k < SB; k++) {
        const int i = base + t + NT * k;
        if (i < n) {
          sc[i] = v[k];
          mx = fmaxf(mx, v[k]);
        }
      }
    };
    {
      float v[SB];
      batch(0, v);
      load_v(0);
      keep(0, v);
    }
    for (int base = SB * NT; base < n; base += SB * NT) {
      float v[SB];
      batch(base, v);
      keep(base, v);
    }
  } else {
  v4u kr[HD > 0 ? KU : 1][4];
  if constexpr (HD > 0 && !PREK) {
#pragma unroll
    for (int u = 0; u < KU; u++) {
      const int unit = t + NT * u, qd = unit / CPR, cd = unit - qd * CPR;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int i = min(4 * qd + e, last);
        kr[u][e] = *reinterpret_cast<const v4u *>(K + (size_t)i * a.kv + 8 * cd);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- 3. RoPE, fp16 rounding of the new k/v, cache append ----
  if (!pre && t < 32) etab[t] = et;
  if (t < hd) {
    float qv = qa, kv_ = ka;
    if (rr) {
      // rotate-half: qa/ka hold element i0, qb/kb element i0 + half
      const double cr = c2.x, sr = c2.y;
      if (t < rot) {
        const double t1 = (double)qa * cr, t2 = (double)qb * sr, u1 = (double)ka * cr, u2 = (double)kb * sr;
        qv = (float)(t1 - t2);
        kv_ = (float)(u1 - u2);
      } else {
        const double t3 = (double)qa * sr, t4 = (double)qb * cr, u3 = (double)ka * sr, u4 = (double)kb * cr;
        qv = (float)(t3 + t4);
        kv_ = (float)(u3 + u4);
      }
    }
    qs[t] = qv;
    if constexpr (FUSED) {
      const uint16_t kh = f2h(kv_), vh = f2h(vv);
      kn[t] = h2f(kh);
      vn[t] = h2f(vh);
      // first query head of the group (its first slice)
      const bool writer = slice == 0 && (h == 0 || (h - 1) * a.KVH / a.H != kvh);
      if (writer) {
        const size_t woff = coff + ((size_t)slot * a.C + pos) * a.kv + (size_t)kvh * hd + t;
        a.kc_w[woff] = kh;
        a.vc_w[woff] = vh;
      }
      // the own position's row of the K tile takes the new k (its cache row
      // is read before the append), so the position is scored with the others
      if (HD > 0 && n - 1 < KQ)
        reinterpret_cast<uint16_t *>(prod)[((size_t)(n - 1) * KP + (t >> 3)) * 8 + (t & 7)] = kh;
    }
  }
  // K tile: row i, chunk c at 16-byte slot i*KP + c
  v4u *ktile = reinterpret_cast<v4u *>(prod);
  if constexpr (HD > 0 && !PREK) {
#pragma unroll
    for (int u = 0; u < KU; u++) {
      const int unit = t + NT * u, qd = unit / CPR, cd = unit - qd * CPR;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int i = 4 * qd + e;
        if (i < KQ && i < n && !(FUSED && i == n - 1)) ktile[i * KP + cd] = kr[u][e];
      }
    }
  }
  // Long contexts: the K rows of positions [k0, k0 + KQ) into kr (the next
  // K tile), loaded while the current tile is scored
  auto load_k = [&](int k0) {
    if constexpr (HD > 0) {
#pragma unroll
      for (int u = 0; u < KU; u++) {
        const int unit = t + NT * u, qd = unit / CPR, cd = unit - qd * CPR;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int i = min(k0 + 4 * qd + e, last);
          kr[u][e] = *reinterpret_cast<const v4u *>(K + (size_t)i * a.kv + 8 * cd);
        }
      }
    }
  };
  if (HD > 0 && n > KQ) load_k(KQ);
  // the product threads' V loads go out after the K rows are written, so no
  // wait before this point counts them; scores and softmax cover their latency
  if (!vpre) load_v(0);
  __syncthreads();

  mk(0);
  // ---- 4. scores ----
  auto put = [&](int i, float s) {
    s = (float)((double)s * a.inv_hd);
    sc[i] = s;
    mx = fmaxf(mx, s);
  };
  // the positions k0 + t + NT*r of the K tile (rows t + NT*r)
  auto score_tile = [&](int k0) {
    if constexpr (HD > 0) {
      // a wave whose positions all lie past n skips the dots (uniform)
      if (k0 + (t & ~63) >= n) return;
      // R positions per thread, their sequential dots interleaved
      constexpr int R = KQMAX / NT;
      float s[R];
#pragma unroll
      for (int r = 0; r < R; r++) s[r] = 0.0f;
#pragma unroll
      for (int c = 0; c < CPR; c++) {
        v4u kk[R];
#pragma unroll
        for (int r = 0; r < R; r++) kk[r] = ktile[min(t + NT * r, KQ - 1) * KP + c];
        float qv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) qv[j] = qs[8 * c + j];
#pragma unroll
        for (int r = 0; r + 1 < R; r += 2) mac8x2(s[r], s[r + 1], qv, kk[r], kk[r + 1]);
        if constexpr (R & 1) mac8(s[R - 1], qv, kk[R - 1]);
      }
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int i = k0 + t + NT * r;
        // past the first tile the own position (FUSED) is scored below
        if (i < n && t + NT * r < KQ && !(FUSED && k0 > 0 && i == n - 1)) put(i, s[r]);
      }
    }
  };
  if constexpr (HD > 0) {
    score_tile(0);
    // long contexts: further K tiles of KQ positions, each loaded into
    // registers while the previous one is scored
    for (int k0 = KQ; k0 < n; k0 += KQ) {
      __syncthreads();  // the previous tile is scored
#pragma unroll
      for (int u = 0; u < KU; u++) {
        const int unit = t + NT * u, qd = unit / CPR, cd = unit - qd * CPR;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int i = 4 * qd + e;
          if (i < KQ && k0 + i < n) ktile[i * KP + cd] = kr[u][e];
        }
      }
      if (k0 + KQ < n) load_k(k0 + KQ);
      __syncthreads();
      score_tile(k0);
    }
    if (FUSED && n - 1 >= KQ && t == 0) put(n - 1, dot_new_k<HD>(qs, kn, hd));
  } else {
    for (int i = t; i < n; i += NT)
      put(i, (FUSED && i == n - 1) ? dot_new_k<HD>(qs, kn, hd) : dot_k_row<HD>(qs, K + (size_t)i * a.kv, hd));
  }
  }  // !SCORED
  mk(1);
  mx = block_max_1b<NT / 64>(mx, redf);
  // e = expf(s - max) replaces each score in LDS; the sum's barrier publishes
  // them, and the threads that form the products turn them into the
  // probabilities p = (float)(e * (1 / sum)) as they read them (no separate
  // normalization pass and barrier)
  double sum = 0.0;
  if constexpr (SP == NT) {
    for (int i = t; i < n; i += NT) {
      const float e = ec_expf_tab(sc[i] - mx, etp);
      sc[i] = e;
      sum += (double)e;
    }
  } else {
    for (int i = t; i < n; i += NT) sc[i] = ec_expf_tab(sc[i] - mx, etp);
    __syncthreads();
    if (t < SP)
      for (int i = t; i < n; i += SP) sum += (double)sc[i];
  }
  // (threads t >= SP hold 0 and write slots the SP / 64-wave tree never reads)
  sum = block_sum_1b<SP / 64>(sum, redd);
  const double isum = 1.0 / sum;

  mk(2);
  // ---- 5. products p*v, and the sequential sums ----
  // element d of quad q sits in 16-byte slot q*P + swz(d) (below), P from
  // attn_pitch / attn_spitch
  const int sw = NS > 1 ? attn_sswz(HS) : attn_swz(hd, a.kv);
  const int hs = NS > 1 ? HS : hd;  // output elements of this block (summing lanes)
  // slot of element d within a quad: 16 consecutive lanes of the product
  // writes (units of 4 positions x 8 elements) and of the sums' reads
  // (consecutive d) touch 16 distinct bank slots; for head_dim 128 also each
  // 8 of them 8 distinct slots mod 8
  auto swz = [&](int d) {
    if constexpr (HD == 128 && NS == 1) return d ^ (((d >> 3) & 7) | (((d >> 6) & 1) << 3));
    else return d ^ ((d >> 4) & sw);
  };
  const float4 *pp = reinterpret_cast<const float4 *>(prod) + swz(t);
  float o = 0.0f;
  // sequential sum of the complete quads [qa, qe) of the tile into o
  auto sum_quads = [&](int qa, int qe) {
    const float4 *pq = pp + (size_t)qa * P;
    int nr = qe - qa;
    constexpr int STR = (NS > 1 ? attn_spitch(HD / NS) : attn_pitch(HD, 0)) * 16;  // bytes per quad
    if constexpr (HD > 0 && NS > 1) {
      // slices: the product area has room for 16 quads of look-ahead
      if (nr >= 16) {
        o = attn_chain16<STR>(o, (uint32_t)(uintptr_t)pq, nr >> 4);
        pq += (size_t)(nr & ~15) * P;
        nr &= 15;
      }
    }
    if constexpr (HD > 0) {
      if (nr >= 8) {
        o = attn_chain8<STR>(o, (uint32_t)(uintptr_t)pq, nr >> 3);
        pq += (size_t)(nr & ~7) * P;
        nr &= 7;
      }
      if (nr >= 4) {
        o = attn_sum4<STR>(o, (uint32_t)(uintptr_t)pq);
        pq += (size_t)4 * P;
        nr -= 4;
      }
    }
    for (; nr > 0; nr--, pq += P) {
      const float4 v = *pq;
      o = o + v.x;
      o = o + v.y;
      o = o + v.z;
      o = o + v.w;
    }
  };
  // the partial quad nq of a tile (cnt & 3 positions)
  auto sum_tail = [&](int nq, int cnt) {
    const float *tail = reinterpret_cast<const float *>(pp + (size_t)nq * P);
    for (int e = 0; e < (cnt & 3); e++) o = o + tail[e];
  };
  // the products of stage s (s < NSTG) of the tile at tt0 (tcnt positions):
  // this product thread's UPS units
  auto form = [&](int tt0, int tcnt, int s) {
#pragma unroll
    for (int u = 0; u < UPS; u++) {
      const int qd = stage_lo(s) + QPU * u + pt / CPRV, cd = pt % CPRV;
      v4u *vu = vr[s * UPS + u];
      if (4 * qd < tcnt && qd < stage_lo(s + 1)) {
        if (vpre) {
#pragma unroll
          for (int e = 0; e < 4; e++) vu[e] = vtl[(e * (T / 4) + qd) * CPRV + cd];
        }
        if (FUSED) {
          // the token's own position takes the fp16-rounded new v (one lane)
          const int en = n - 1 - tt0 - 4 * qd;
          if (en >= 0 && en < 4) {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
              w[j] = (uint32_t)f2h(vn[HS * slice + 8 * cd + 2 * j]) |
                     ((uint32_t)f2h(vn[HS * slice + 8 * cd + 2 * j + 1]) << 16);
            const v4u nv = {w[0], w[1], w[2], w[3]};
#pragma unroll
            for (int e = 0; e < 4; e++)
              if (e == en) vu[e] = nv;
          }
        }
        const float4 eq = *reinterpret_cast<const float4 *>(sc + tt0 + 4 * qd);
        const float pe[4] = {(float)((double)eq.x * isum), (float)((double)eq.y * isum),
                             (float)((double)eq.z * isum), (float)((double)eq.w * isum)};
        float pr[8][4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float r8[8];
          mul8h(r8, pe[e], vu[e]);
#pragma unroll
          for (int k = 0; k < 8; k++) pr[k][e] = r8[k];
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
          *reinterpret_cast<float4 *>(prod + ((size_t)qd * P + swz(8 * cd + k)) * 4) =
              make_float4(pr[k][0], pr[k][1], pr[k][2], pr[k][3]);
      }
    }
  };
  bool pre0 = false;  // this tile's stage-0 products were formed in the previous tile's last stage
  for (int t0 = 0; t0 < n; t0 += T) {
    const int cnt = min(T, n - t0);
    const int nq = cnt >> 2;  // complete quads
    if (t0 > 0) __syncthreads();  // the previous tile's last stage is done (the first tile: the sum's barrier)
    if constexpr (HD > 0) {
      // Stage s: the product threads form the products of their UPS units of
      // stage s (quads [stage_lo(s), stage_lo(s+1))) while the summing lanes
      // add the quads of stage s - 1; a barrier separates the stages.
      // (the V of tiles after the first is loaded during the previous tile's
      // stages)
      const int nqt = (cnt + 3) / 4;  // quads holding positions
      const int nst = nqt <= Q0 ? 1 : 1 + (nqt - Q0 + SQ - 1) / SQ;  // stages holding positions
      // The next tile's stage-0 products are formed during this tile's last
      // stage, beside its last sums, when that stage reads none of the quads
      // they overwrite (two stages or more): the next tile then starts with
      // its first sums instead of a stage of products alone.
      // (not in the persistent step, whose contexts mostly fit one tile:
      // there the extra code costs registers)
      const int cnt1 = min(T, n - t0 - T);  // the next tile's positions (<= 0: none)
      const bool pipe = !PREK && cnt1 > 0 && nst >= 2;
#pragma unroll
      for (int s = 0; s <= NSTG; s++) {
        if (s > nst || (s == 0 && pre0)) continue;  // uniform
        if (s == 1 || s == 2) mk(2 + s);
        if (pt >= 0) {
          if (s < nst) {
            form(t0, cnt, min(s, NSTG - 1));
            // the next tile's V of this stage into the registers the stage
            // has used up, so that its loads have the tile's later stages to
            // arrive in (loaded at the tile's end, each next tile began by
            // waiting for its V: about 1 us of the 2.4 us a 256-position tile
            // took at head_dim 128)
            if (t0 + T < n) load_v_stage(t0 + T, min(s, NSTG - 1));
          }
        } else if (t < hs && s > 0) {
          sum_quads(stage_lo(s - 1), min(stage_lo(s), nq));
          if (s == nst) sum_tail(nq, cnt);
        }
        if (s < nst) __syncthreads();
      }
      if (pipe && pt >= 0) {
        form(t0 + T, cnt1, 0);
        if (t0 + 2 * T < n) load_v_stage(t0 + 2 * T, 0);  // the V of the tile after next, stage 0
      }
      pre0 = pipe;
    } else {
      for (int e = t; e < cnt * hd; e += NT) {
        const int i = e / hd, d = e - i * hd;
        const float v = (FUSED && t0 + i == n - 1) ? vn[d] : h2f(V[(size_t)(t0 + i) * a.kv + d]);
        const float p = (float)((double)sc[t0 + i] * isum);
        prod[((size_t)(i >> 2) * P + (d ^ ((d >> 4) & sw))) * 4 + (i & 3)] = p * v;
      }
      __syncthreads();
      if (t < hd) {
        sum_quads(0, nq);
        sum_tail(nq, cnt);
      }
    }
  }
  if (t < hs) out(t, o);
}

// For attn_decode_block<HD, true, NS, false, true> (element slices, FUSED):
// load the K rows of positions [lo, lo + min(n - 1, KQ)) of token m's KV
// group (head h) straight from the cache into the K tile of lds, in the
// tile's layout (row i at 16-byte slot i * KP, chunk c at + c), one row per
// instruction (8 lanes of 16 bytes each).  Every thread of the block calls
// it; the loads complete asynchronously (vmcnt): the caller waits for them
// and then passes a barrier before the body reads the tile.
template <int HD, int NS>
__device__ __forceinline__ void attn_prefetch_k(const AttnArgs &a, int m, int h, float *lds, size_t coff = 0) {
  static_assert(HD == 64 && NS > 1, "element slices of head_dim 64");
  constexpr int NT = 512, KU = kAttnUnits / 2, CPR = HD / 8, KP = CPR + 1;
  constexpr int KQMAX = NT * KU * 4 / CPR;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int pos = ld_uniform(a.pos + m), slot = ld_uniform(a.slot + m);
  int lo = 0;
  if (a.window > 0) {
    lo = pos - a.window + 1;
    if (lo < 0) lo = 0;
  }
  const int n = pos + 1 - lo;
  const int KQ = min(KQMAX, (a.vtile / 4) * attn_pitch(HD, a.kv) / KP);
  const int rows = min(n - 1, KQ);
  const int kvh = h * a.KVH / a.H;
  const uint16_t *K = a.kc + coff + (size_t)slot * a.C * a.kv + (size_t)kvh * HD + (size_t)lo * a.kv;
  char *tile = reinterpret_cast<char *>(lds + 3 * HD + ((a.max_npos + 3) & ~3));
  typedef __attribute__((address_space(1))) void gvoid;
  typedef __attribute__((address_space(3))) void lvoid;
  if (lane < CPR) {
    for (int i = wave; i < rows; i += NT / 64)
      __builtin_amdgcn_global_load_lds((gvoid *)(K + (size_t)i * a.kv + 8 * lane), (lvoid *)(tile + (size_t)i * KP * 16),
                                       16, 0, 0);
  }
}

// For the same body: chunk c (c < 2) of this block's element slice of the V
// rows of positions [lo, lo + min(n - 1, T)) into the V tile (16-byte slot
// ((e * T / 4 + q) * 2 + c) for position 4 q + e, past the K tile and the
// products, step_vtile_off).  One instruction covers 32 quads of one e, each
// lane one chunk; lanes past the positions load nothing.  As
// attn_prefetch_k: every thread calls it, the caller waits and then passes a
// barrier.
template <int HD, int NS>
__device__ __forceinline__ void attn_prefetch_v(const AttnArgs &a, int m, int h, int slice, float *lds,
                                                size_t coff = 0) {
  static_assert(HD == 64 && NS == 4, "element slices of 16 of head_dim 64");
  constexpr int NT = 512, CPRV = HD / 8 / NS;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int pos = ld_uniform(a.pos + m), slot = ld_uniform(a.slot + m);
  int lo = 0;
  if (a.window > 0) {
    lo = pos - a.window + 1;
    if (lo < 0) lo = 0;
  }
  const int n = pos + 1 - lo, T = a.vtile, QM = T / 4;
  if (n > T) return;  // the body then loads V into registers
  const int rows = n - 1;
  const int kvh = h * a.KVH / a.H;
  const uint16_t *V = a.vc + coff + (size_t)slot * a.C * a.kv + (size_t)kvh * HD + (size_t)lo * a.kv;
  char *vt = reinterpret_cast<char *>(lds + 3 * HD + ((a.max_npos + 3) & ~3)) + step_vtile_off(T, a.kv);
  typedef __attribute__((address_space(1))) void gvoid;
  typedef __attribute__((address_space(3))) void lvoid;
  const int qd = lane / CPRV, cd = lane % CPRV;  // within an instruction's 32 quads
  for (int e = 0; e < 4; e++) {
    for (int q0 = 32 * wave; 4 * q0 + e < rows; q0 += 32 * (NT / 64)) {
      const int p = 4 * (q0 + qd) + e;
      if (p < rows)
        __builtin_amdgcn_global_load_lds((gvoid *)(V + (size_t)p * a.kv + 8 * (CPRV * slice + cd)),
                                         (lvoid *)(vt + (size_t)(e * QM + q0) * CPRV * 16), 16, 0, 0);
    }
  }
}

}  // namespace ec
