// gfx950 kernels of the EdgeCore transformer forward hot path.
//
// The fused decode GEMV lives in gemv_impl.h (instantiated per weight type in
// gemv_*.hip); this file holds the generic GEMV, norms, quantizer, embedding,
// RoPE/KV append, attention, argmax, elementwise math and the launchers.
#include "gemv_impl.h"

#include <float.h>

namespace ec {

hipEvent_t g_launch_ev[2] = {nullptr, nullptr};

static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// ---------------------------------------------------------------------------
// generic GEMV (any K, any alignment, every epilogue): one thread per output
// element, activations given as int8 rows + scales (PRO_I8) or fp32 rows
// (PRO_F32).  Used for shapes the vector kernels cannot read with 16-byte loads.
// ---------------------------------------------------------------------------

template <int WT, int EPI>
__global__ __launch_bounds__(256) void gemv_generic_kernel(GemvArgs a) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)a.M * a.N) return;
  const int m = (int)(idx / a.N), n = (int)(idx % a.N);
  float v, u = 0.0f;
  if constexpr (WT == WT_I8) {
    const int8_t *x = reinterpret_cast<const int8_t *>(a.A) + (size_t)m * a.lda;
    const int8_t *w = reinterpret_cast<const int8_t *>(a.W) + (size_t)n * a.K;
    int dot = 0;
    for (int k = 0; k < a.K; k++) dot += (int)x[k] * (int)w[k];
    v = i8_epilogue(dot, a.as[m], a.ws ? a.ws[n] : 1.0f,
                    (a.bias && EPI != EPI_SWIGLU) ? a.bias[n] : 0.0f);
    if constexpr (EPI == EPI_SWIGLU) {
      const int8_t *w2 = reinterpret_cast<const int8_t *>(a.W2) + (size_t)n * a.K;
      int d2 = 0;
      for (int k = 0; k < a.K; k++) d2 += (int)x[k] * (int)w2[k];
      u = i8_epilogue(d2, a.as[m], a.ws2 ? a.ws2[n] : 1.0f, 0.0f);
    }
  } else {
    const float *x = reinterpret_cast<const float *>(a.A) + (size_t)m * a.lda;
    const uint16_t *w = reinterpret_cast<const uint16_t *>(a.W) + (size_t)n * a.K;
    v = 0.0f;
    for (int k = 0; k < a.K; k++) v = __builtin_fmaf(x[k], w2f<WT == WT_BF16>(w[k]), v);
    if constexpr (EPI == EPI_SWIGLU) {
      const uint16_t *w2 = reinterpret_cast<const uint16_t *>(a.W2) + (size_t)n * a.K;
      for (int k = 0; k < a.K; k++) u = __builtin_fmaf(x[k], w2f<WT == WT_BF16>(w2[k]), u);
    }
    if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_RESID || EPI == EPI_BIAS_GELU) v = v + a.bias[n];
  }
  float *o = a.out + (size_t)m * a.ldo + n;
  if constexpr (EPI == EPI_SWIGLU) v = silu(v) * u;
  if constexpr (EPI == EPI_RESID || EPI == EPI_BIAS_RESID) v = *o + v;
  if constexpr (EPI == EPI_GELU || EPI == EPI_BIAS_GELU) v = gelu_new(v);
  *o = v;
}

// ---------------------------------------------------------------------------
// activation quantizer, norms, embedding
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void quant_kernel(const float *in, int ldi, int K, int8_t *q,
                                                    int ldq, float *s) {
  __shared__ float red[4];
  const int m = blockIdx.x;
  const float *x = in + (size_t)m * ldi;
  float mx = 0.0f;
  for (int k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(x[k]));
  mx = block_max256(mx, red);
  const float sc = quant_scale(mx);
  if (threadIdx.x == 0) s[m] = sc;
  int8_t *qr = q + (size_t)m * ldq;
  for (int k = threadIdx.x; k < K; k += 256) qr[k] = quant1(x[k], sc);
}

// src/gpt2.c:398-414 (LN) and 592-604 (RMS): double accumulation, fp32 output
template <bool LN, bool QUANT>
__global__ __launch_bounds__(256) void norm_kernel(const float *x, int E, const float *gamma,
                                                   const float *beta, double eps, float *h,
                                                   int ldh, int8_t *q, int ldq, float *qs) {
  extern __shared__ float row[];
  __shared__ double redd[4];
  __shared__ float redf[4];
  const int m = blockIdx.x;
  const float *xr = x + (size_t)m * E;
  double acc = 0.0;
  for (int i = threadIdx.x; i < E; i += 256) {
    const float v = xr[i];
    row[i] = v;
    acc += LN ? (double)v : (double)v * (double)v;
  }
  const double tot = block_sum256(acc, redd);
  double mean = 0.0, rstd;
  if constexpr (LN) {
    mean = tot / E;
    double a2 = 0.0;
    for (int i = threadIdx.x; i < E; i += 256) {
      const double d = (double)row[i] - mean;
      a2 += d * d;
    }
    const double var = block_sum256(a2, redd) / E;
    rstd = 1.0 / sqrt(var + eps);
  } else {
    rstd = 1.0 / sqrt(tot / E + eps);
  }
  float mx = 0.0f;
  for (int i = threadIdx.x; i < E; i += 256) {
    float t = LN ? (float)(((double)row[i] - mean) * rstd) : (float)((double)row[i] * rstd);
    t = t * gamma[i];
    if constexpr (LN) t = t + beta[i];
    if constexpr (QUANT) {
      row[i] = t;
      mx = fmaxf(mx, fabsf(t));
    } else {
      h[(size_t)m * ldh + i] = t;
    }
  }
  if constexpr (QUANT) {
    mx = block_max256(mx, redf);
    const float sc = quant_scale(mx);
    if (threadIdx.x == 0) qs[m] = sc;
    int8_t *qr = q + (size_t)m * ldq;
    for (int i = threadIdx.x; i < E; i += 256) qr[i] = quant1(row[i], sc);
  }
}

template <bool BF16>
__global__ __launch_bounds__(256) void embed_kernel(const uint16_t *wte, const uint16_t *wpe,
                                                    const int *tok, const int *pos, int E,
                                                    float *x) {
  const int m = blockIdx.x;
  const uint16_t *et = wte + (size_t)tok[m] * E;
  const uint16_t *ep = wpe ? wpe + (size_t)pos[m] * E : nullptr;
  for (int d = threadIdx.x; d < E; d += 256) {
    float v = w2f<BF16>(et[d]);
    if (ep) v = v + w2f<BF16>(ep[d]);
    x[(size_t)m * E + d] = v;
  }
}

// ---------------------------------------------------------------------------
// RoPE + KV append
// ---------------------------------------------------------------------------

// src/gpt2.c:656-665 (rotate-half in double) and :726-741 (fp16 append)
__global__ __launch_bounds__(256) void rope_kv_kernel(KvArgs a) {
  const int m = blockIdx.x;
  const int pos = a.pos[m], slot = a.slot[m];
  float *k = a.k + (size_t)m * a.ldk;
  const float *v = a.v + (size_t)m * a.ldk;
  if (a.cs) {
    float *q = a.q + (size_t)m * a.ldq;
    const double2 *cs = a.cs + (size_t)pos * a.half;
    const int tot = (a.H + a.KVH) * a.half;
    for (int idx = threadIdx.x; idx < tot; idx += 256) {
      const int hh = idx / a.half, i = idx - hh * a.half;
      float *p = hh < a.H ? q + (size_t)hh * a.hd : k + (size_t)(hh - a.H) * a.hd;
      const float x0 = p[i], x1 = p[i + a.half];
      const double c = cs[i].x, s = cs[i].y;
      const double t1 = x0 * c, t2 = x1 * s, t3 = x0 * s, t4 = x1 * c;
      p[i] = (float)(t1 - t2);
      p[i + a.half] = (float)(t3 + t4);
    }
    __syncthreads();
  }
  const size_t off = ((size_t)slot * a.C + pos) * a.kv;
  for (int d = threadIdx.x; d < a.kv; d += 256) {
    a.kc[off + d] = f2h(k[d]);
    a.vc[off + d] = f2h(v[d]);
  }
}

// ---------------------------------------------------------------------------
// attention (src/gpt2.c:527-557 and 744-777)
// ---------------------------------------------------------------------------
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
template <int HD, bool FUSED, int NS>
__global__ __launch_bounds__(NS > 1 ? 512 : 256) void attn_kernel(AttnArgs a) {
  static_assert(NS == 1 || (HD == 64 && (NS == 2 || NS == 4 || NS == 8)), "element slices: head_dim 64, 2 / 4 / 8");
  extern __shared__ __attribute__((aligned(16))) float lds[];
  // threads per block: 512 with element slices (one scored position per
  // thread up to 512 positions), else 256
  constexpr int NT = NS > 1 ? 512 : 256;
  constexpr int KU = NT == 512 ? kAttnUnits / 2 : kAttnUnits;  // K units per thread
  __shared__ float redf[NT / 64];
  __shared__ double redd[NT / 64];
  __shared__ uint64_t etab[32];  // expf table
  constexpr int CPR = HD > 0 ? HD / 8 : 1;         // 16-byte chunks per K/V row
  constexpr int HS = HD > 0 ? HD / NS : 0;  // elements of this block's slice
  constexpr int CPRV = HD > 0 ? CPR / NS : 1;  // 16-byte V chunks per slice
  const int m = blockIdx.y, t = threadIdx.x;
  int h = blockIdx.x, slice = 0;
  if (a.xcd_r) {
    // XCD-aware launch: blocks are dispatched to the 8 XCDs round-robin, so
    // block x runs on XCD x % 8 (gridDim.x is a multiple of 8); token m's
    // group g uses the blocks on XCD (m * KVH + g) % 8, x = that XCD + 8j, and
    // its heads (and their slices) share that XCD's L2 for the group's K/V
    // rows.  The tokens of a batch (their own slots' K/V) go to other XCDs.
    const int g = ((int)(blockIdx.x & 7) - m * a.KVH) & 7, j = blockIdx.x >> 3;
    if (g >= a.KVH || j >= a.xcd_r * NS) return;
    h = g * a.xcd_r + j / NS;
    slice = j % NS;
  } else if (NS > 1) {
    h = blockIdx.x / NS;
    slice = blockIdx.x % NS;
  }
  const int pos = ld_uniform(a.pos + m), slot = ld_uniform(a.slot + m);
  const uint64_t et = ec_exp2_32[t & 31];
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
  const size_t cbase = (size_t)slot * a.C * a.kv + (size_t)kvh * hd;
  const uint16_t *K = a.kc + cbase + (size_t)lo * a.kv;
  const uint16_t *V = a.vc + cbase + (size_t)lo * a.kv;
  const int ncache = FUSED ? n - 1 : n;  // positions read from the cache
  const int last = ncache > 0 ? ncache - 1 : 0;  // clamp target of the unconditional loads

  // ---- 1. this thread's element of q (and of the new k and v) ----
  // Branch-free loads (index clamped into the head) so that every load of
  // steps 1-2 is issued before the first wait.
  const float *qrow = a.q + (size_t)m * a.ldq + (size_t)h * hd;
  const float *krow = a.k + (size_t)m * a.ldk + (size_t)kvh * hd;
  const float *vrow = a.v + (size_t)m * a.ldk + (size_t)kvh * hd;
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
    if (rot) c2 = a.cs[(size_t)pos * a.half + (rr ? i0 : 0)];
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
  v4u kr[HD > 0 ? KU : 1][4], vr[NSTG * UPS][4];
  if constexpr (HD > 0) {
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
  auto load_v = [&](int t0) {  // this product thread's V units of the tile at t0
    if (HD > 0 && pt >= 0) {
      const int qd0 = pt / CPRV, cd = pt - qd0 * CPRV;
#pragma unroll
      for (int s = 0; s < NSTG; s++) {
#pragma unroll
        for (int u = 0; u < UPS; u++) {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int i = min(t0 + 4 * (stage_lo(s) + QPU * u + qd0) + e, last);
            vr[s * UPS + u][e] = *reinterpret_cast<const v4u *>(V + (size_t)i * a.kv + 8 * (CPRV * slice + cd));
          }
        }
      }
    }
  };
  __builtin_amdgcn_sched_barrier(0);

  // ---- 3. RoPE, fp16 rounding of the new k/v, cache append ----
  if (t < 32) etab[t] = et;
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
        const size_t woff = ((size_t)slot * a.C + pos) * a.kv + (size_t)kvh * hd + t;
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
  if constexpr (HD > 0) {
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
  load_v(0);
  __syncthreads();

  // ---- 4. scores ----
  float mx = -FLT_MAX;
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
  mx = block_max_1b<NT / 64>(mx, redf);
  // this thread's first two values stay in registers until the sum is known
  // (positions below 512); further ones go through LDS
  double sum = 0.0;
  float ev[2];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int i = t + NT * k;
    ev[k] = 0.0f;
    if (i < n) {
      ev[k] = ec_expf_tab(sc[i] - mx, etab);
      sum += (double)ev[k];
    }
  }
  for (int i = t + 2 * NT; i < n; i += NT) {
    const float e = ec_expf_tab(sc[i] - mx, etab);
    sc[i] = e;
    sum += (double)e;
  }
  sum = block_sum_1b<NT / 64>(sum, redd);
  const double isum = 1.0 / sum;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int i = t + NT * k;
    if (i < n) sc[i] = (float)((double)ev[k] * isum);
  }
  for (int i = t + 2 * NT; i < n; i += NT) sc[i] = (float)((double)sc[i] * isum);

  // ---- 5. products p*v, and the sequential sums ----
  // element d of quad q sits in 16-byte slot q*P + (d ^ ((d >> 4) & sw)); with
  // P and sw from attn_pitch/attn_swz every 16 consecutive lanes of the
  // product writes (units of 4 positions x 8 elements) and of the sums' reads
  // (consecutive d) touch 16 distinct bank slots
  const int sw = NS > 1 ? attn_sswz(HS) : attn_swz(hd, a.kv);
  const int hs = NS > 1 ? HS : hd;  // output elements of this block (summing lanes)
  const float4 *pp = reinterpret_cast<const float4 *>(prod) + (t ^ ((t >> 4) & sw));
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
  for (int t0 = 0; t0 < n; t0 += T) {
    const int cnt = min(T, n - t0);
    const int nq = cnt >> 2;  // complete quads
    __syncthreads();  // probabilities written / previous tile's sums done
    if constexpr (HD > 0) {
      // Stage s: the product threads form the products of their UPS units of
      // stage s (quads [stage_lo(s), stage_lo(s+1))) while the summing lanes
      // add the quads of stage s - 1; a barrier separates the stages.
      // (the V of tiles after the first is loaded during the previous tile's
      // last stage)
      const int nqt = (cnt + 3) / 4;  // quads holding positions
      const int nst = nqt <= Q0 ? 1 : 1 + (nqt - Q0 + SQ - 1) / SQ;  // stages holding positions
#pragma unroll
      for (int s = 0; s <= NSTG; s++) {
        if (s > nst) continue;  // uniform
        if (pt >= 0) {
#pragma unroll
          for (int u = 0; u < UPS; u++) {
            const int qd = stage_lo(s) + QPU * u + pt / CPRV, cd = pt % CPRV;
            v4u *vu = vr[min(s, NSTG - 1) * UPS + u];
            if (s < nst && 4 * qd < cnt && qd < stage_lo(s + 1)) {
              if (FUSED) {
                // the token's own position takes the fp16-rounded new v (one lane)
                const int en = n - 1 - t0 - 4 * qd;
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
              const float4 pq = *reinterpret_cast<const float4 *>(sc + t0 + 4 * qd);
              const float pe[4] = {pq.x, pq.y, pq.z, pq.w};
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
                *reinterpret_cast<float4 *>(prod + ((size_t)qd * P + ((8 * cd + k) ^ (((8 * cd + k) >> 4) & sw))) * 4) =
                    make_float4(pr[k][0], pr[k][1], pr[k][2], pr[k][3]);
            }
          }
          // the next tile's V into the registers this tile has used up
          if (s == nst - 1 && t0 + T < n) load_v(t0 + T);
        } else if (t < hs && s > 0) {
          sum_quads(stage_lo(s - 1), min(stage_lo(s), nq));
          if (s == nst) sum_tail(nq, cnt);
        }
        if (s < nst) __syncthreads();
      }
    } else {
      for (int e = t; e < cnt * hd; e += NT) {
        const int i = e / hd, d = e - i * hd;
        const float v = (FUSED && t0 + i == n - 1) ? vn[d] : h2f(V[(size_t)(t0 + i) * a.kv + d]);
        prod[((size_t)(i >> 2) * P + (d ^ ((d >> 4) & sw))) * 4 + (i & 3)] = sc[t0 + i] * v;
      }
      __syncthreads();
      if (t < hd) {
        sum_quads(0, nq);
        sum_tail(nq, cnt);
      }
    }
  }
  if (t < hs) a.out[(size_t)m * a.ldo + (size_t)h * hd + (size_t)hs * slice + t] = o;
}

// ---------------------------------------------------------------------------
// greedy argmax (first maximum wins; NaN never wins; a NaN at index 0 wins)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void argmax_kernel(const float *L, int V, int *out) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const float *l = L + (size_t)blockIdx.x * V;
  float bv = 0.0f;
  int bi = -1;
  for (int i = threadIdx.x; i < V; i += 256) {
    const float v = l[i];
    if (v == v && (bi < 0 || v > bv)) {
      bv = v;
      bi = i;
    }
  }
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      const int o = threadIdx.x + s;
      if (si[o] >= 0 && (si[threadIdx.x] < 0 || sv[o] > sv[threadIdx.x] ||
                         (sv[o] == sv[threadIdx.x] && si[o] < si[threadIdx.x]))) {
        sv[threadIdx.x] = sv[o];
        si[threadIdx.x] = si[o];
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float l0 = l[0];
    out[blockIdx.x] = (l0 != l0 || si[0] < 0) ? 0 : si[0];
  }
}

// argmax over the LM head's per-block candidates; logits[0] NaN -> 0 and no
// non-NaN logit -> 0, like the reference's strict '>' scan from index 0
__global__ __launch_bounds__(256) void argmax_finalize_kernel(const unsigned long long *cand, int ncand,
                                                              const float *logits, int ldl, int *out) {
  __shared__ unsigned long long red[4];
  const int r = blockIdx.x;
  unsigned long long b = 0ull;
  for (int i = threadIdx.x; i < ncand; i += 256) {
    const unsigned long long c = cand[(size_t)r * ncand + i];
    b = c > b ? c : b;
  }
  b = wave_max_u64(b);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; w++) b = red[w] > b ? red[w] : b;
    const float l0 = logits[(size_t)r * ldl];
    out[r] = (l0 != l0 || b == 0ull) ? 0 : (int)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFull));
  }
}

// ---------------------------------------------------------------------------
// elementwise device math, for checking the device arithmetic from tests
// ---------------------------------------------------------------------------

// plain copy of n4 16-byte elements (grid-stride): the reference kernel for
// HBM traffic counters and achievable bandwidth
__global__ __launch_bounds__(256) void copy_kernel(const v4u *in, v4u *out, size_t n4) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256)
    __builtin_nontemporal_store(__builtin_nontemporal_load(in + i), out + i);
}

__global__ __launch_bounds__(256) void math_kernel(int op, const void *in, void *out, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  if (op == MATH_F16_TO_F32) {
    reinterpret_cast<float *>(out)[i] = h2f(reinterpret_cast<const uint16_t *>(in)[i]);
    return;
  }
  const float x = reinterpret_cast<const float *>(in)[i];
  switch (op) {
  case MATH_EXPF: reinterpret_cast<float *>(out)[i] = ec_expf_ref(x); break;
  case MATH_SILU: reinterpret_cast<float *>(out)[i] = silu(x); break;
  case MATH_GELU: reinterpret_cast<float *>(out)[i] = gelu_new(x); break;
  case MATH_F32_TO_F16: reinterpret_cast<uint16_t *>(out)[i] = f2h(x); break;
  case MATH_QUANT1: reinterpret_cast<int8_t *>(out)[i] = quant1(x, 1.0f); break;
  case MATH_COPY: reinterpret_cast<float *>(out)[i] = x; break;
  default: break;
  }
}

hipError_t device_math(int op, const void *in, void *out, size_t n, hipStream_t st) {
  if (op < 0 || op > MATH_COPY) return hipErrorInvalidValue;
  if (op == MATH_COPY && n % 4 == 0 && al16(in) && al16(out)) {
    const size_t n4 = n / 4, blocks = (n4 + 255) / 256;
    klaunch(copy_kernel, dim3((unsigned)(blocks < 2048 ? blocks : 2048)), dim3(256), 0, st,
            reinterpret_cast<const v4u *>(in), reinterpret_cast<v4u *>(out), n4);
    return hipGetLastError();
  }
  klaunch(math_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, op, in, out, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------


static int g_gemv_max_blocks = 2048;
void gemv_set_max_blocks(int n) { g_gemv_max_blocks = n > 0 ? n : 2048; }
int gemv_max_blocks() { return g_gemv_max_blocks; }

int gemv_pick_mt(int M) { return M >= 5 ? 8 : M >= 3 ? 4 : M == 2 ? 2 : 1; }

// row shape: 4 rows per wave when a row fits one pass of 16 lanes, one row
// per wave otherwise (one pass up to 320 chunks, else the wide loop)
int gemv_pick_shape(int wt, int K) {
  const int nch = K / (wt == WT_I8 ? 16 : 8);
  if (nch <= 16 * (wt == WT_I8 ? 4 : 8)) return GS_NARROW;
  if (nch <= 64 * 5) return GS_MID;
  return GS_WIDE;
}

int gemv_grid_x(const GemvArgs &a, int wt, int epi) {
  (void)epi;
  const int rpb = gemv_pick_shape(wt, a.K) == GS_NARROW ? 16 : 4;
  const int ng = (a.N + rpb - 1) / rpb;
  return ng < g_gemv_max_blocks ? ng : g_gemv_max_blocks;
}

size_t gemv_lds_bytes(int wt, int pro, int MT, int K) {
  if (pro == PRO_F32) return 0;
  const int rows = gemv_wave_pro(pro, MT, K) ? 4 : MT;  // one row per wave, or the M tile
  if (wt == WT_I8) {
    const size_t kp = (size_t)(K + 15) / 16 * 16;
    return (rows * kp + 4 * rows + 15) / 16 * 16;  // codes, then one scale per row slot
  }
  const size_t kp = (size_t)(K + 7) / 8 * 8;
  return rows * kp * 4;
}

static int g_max_lds_bytes = 65536;

bool gemv_vector_ok(const GemvArgs &a, int wt, int pro) {
  const int chb = wt == WT_I8 ? 16 : 8;
  if (a.K <= 0 || a.K % chb || a.N <= 0 || !al16(a.W) || (a.W2 && !al16(a.W2))) return false;
  if (pro == PRO_I8 && (a.lda % 16 || !al16(a.A))) return false;
  if (pro != PRO_I8 && (a.lda % 4 || !al16(a.A))) return false;
  if (wt == WT_I8 && pro == PRO_F32) return false;
  if (wt != WT_I8 && (pro == PRO_I8 || pro == PRO_QUANT)) return false;
  // activation rows the prologue keeps in registers (float4 strips of 1024)
  if (pro == PRO_QUANT && a.K > 10 * 1024) return false;
  if (pro == PRO_RMS || pro == PRO_LN) {
    if (a.K > 4 * 1024 || !al16(a.gamma) || (pro == PRO_LN && !al16(a.beta))) return false;
  }
  return gemv_lds_bytes(wt, pro, gemv_pick_mt(a.M), a.K) <= (size_t)g_max_lds_bytes;
}

void gemv_set_max_lds(int bytes) { g_max_lds_bytes = bytes; }

hipError_t gemv(const GemvArgs &a, int wt, int epi, int pro, hipStream_t s) {
  if (wt == WT_I8) return gemv_i8_fused(a, epi, pro, s);
  if (wt == WT_BF16) return gemv_bf16_fused(a, epi, pro, s);
  return gemv_f16_fused(a, epi, pro, s);
}

template <int WT, int EPI>
static hipError_t launch_generic(const GemvArgs &a, hipStream_t s) {
  const size_t tot = (size_t)a.M * a.N;
  klaunch((gemv_generic_kernel<WT, EPI>), dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int WT>
static hipError_t generic_epi(const GemvArgs &a, int epi, hipStream_t s) {
  switch (epi) {
  case EPI_STORE: return launch_generic<WT, EPI_STORE>(a, s);
  case EPI_RESID: return launch_generic<WT, EPI_RESID>(a, s);
  case EPI_GELU: return launch_generic<WT, EPI_GELU>(a, s);
  case EPI_SWIGLU: return launch_generic<WT, EPI_SWIGLU>(a, s);
  case EPI_BIAS: return launch_generic<WT, EPI_BIAS>(a, s);
  case EPI_BIAS_RESID: return launch_generic<WT, EPI_BIAS_RESID>(a, s);
  case EPI_BIAS_GELU: return launch_generic<WT, EPI_BIAS_GELU>(a, s);
  default: return hipErrorInvalidValue;
  }
}

hipError_t gemv_generic(const GemvArgs &a, int wt, int epi, hipStream_t s) {
  if (wt == WT_I8) return generic_epi<WT_I8>(a, epi, s);
  if (wt == WT_BF16) return generic_epi<WT_BF16>(a, epi, s);
  return generic_epi<WT_F16>(a, epi, s);
}

hipError_t quant_rows(const float *in, int ldi, int M, int K, int8_t *q, int ldq, float *s,
                      hipStream_t st) {
  klaunch(quant_kernel, dim3(M), dim3(256), 0, st, in, ldi, K, q, ldq, s);
  return hipGetLastError();
}

hipError_t norm_rows(const float *x, int M, int E, const float *gamma, const float *beta,
                     double eps, float *h, int ldh, int8_t *q, int ldq, float *qs,
                     hipStream_t st) {
  const size_t lds = (size_t)E * sizeof(float);
  if (beta) {
    if (q) klaunch((norm_kernel<true, true>), dim3(M), dim3(256), lds, st, x, E, gamma, beta, eps, h, ldh, q, ldq, qs);
    else klaunch((norm_kernel<true, false>), dim3(M), dim3(256), lds, st, x, E, gamma, beta, eps, h, ldh, q, ldq, qs);
  } else {
    if (q) klaunch((norm_kernel<false, true>), dim3(M), dim3(256), lds, st, x, E, gamma, beta, eps, h, ldh, q, ldq, qs);
    else klaunch((norm_kernel<false, false>), dim3(M), dim3(256), lds, st, x, E, gamma, beta, eps, h, ldh, q, ldq, qs);
  }
  return hipGetLastError();
}

hipError_t embed(const uint16_t *wte, const uint16_t *wpe, bool bf16, const int *tok,
                 const int *pos, int M, int E, float *x, hipStream_t st) {
  if (bf16)
    klaunch(embed_kernel<true>, dim3(M), dim3(256), 0, st, wte, wpe, tok, pos, E, x);
  else
    klaunch(embed_kernel<false>, dim3(M), dim3(256), 0, st, wte, wpe, tok, pos, E, x);
  return hipGetLastError();
}

hipError_t rope_kv_append(const KvArgs &a, hipStream_t st) {
  klaunch(rope_kv_kernel, dim3(a.M), dim3(256), 0, st, a);
  return hipGetLastError();
}

size_t attention_lds_bytes(int max_npos, int hd, int vtile) {
  // q, new k, new v; scores; product tile of vtile/4 quads + 8 quads of slack
  return ((size_t)3 * ((hd + 3) & ~3) + (size_t)((max_npos + 3) & ~3) +
          (size_t)(vtile + 32) * attn_pitch(hd, 0)) * sizeof(float);
}

int attention_max_vtile(int hd, int kv) {
  if (!attn_vec(hd, kv)) return 512;
  const int t = 256 * kAttnUnits * 4 / (hd / 8);
  return t < 512 ? t : 512;
}

template <int HD>
static void launch_attn(AttnArgs a, size_t lds, hipStream_t st) {
  // grouped-query heads: one XCD per KV group (8 XCDs, block x -> XCD x % 8)
  const int r = a.H / a.KVH;
  a.xcd_r = (a.KVH <= 8 && a.H % a.KVH == 0 && r > 1) ? r : 0;
  // head_dim 64: four blocks per head (16 elements each), a quarter of the
  // products on each block's critical path.  With one XCD per KV group, the
  // 7 heads x 4 slices of a Qwen2-0.5B group fit that XCD's 32 CUs at once;
  // 8 slices took two rounds of blocks.
  constexpr int NS = HD == 64 ? 4 : 1;
  const dim3 grid((a.xcd_r ? 8 * r : a.H) * NS, a.M);
  const dim3 block(NS > 1 ? 512 : 256);
  if (a.fuse_kv) klaunch((attn_kernel<HD, true, NS>), grid, block, lds, st, a);
  else klaunch((attn_kernel<HD, false, NS>), grid, block, lds, st, a);
}

hipError_t attention(const AttnArgs &a, hipStream_t st) {
  if (a.vtile < 4 || (a.vtile & 3) || a.vtile > attention_max_vtile(a.hd, a.kv) || a.hd > 256)
    return hipErrorInvalidValue;
  const size_t lds = attention_lds_bytes(a.max_npos, a.hd, a.vtile);
  if (attn_vec(a.hd, a.kv) && a.hd == 64) launch_attn<64>(a, lds, st);
  else if (attn_vec(a.hd, a.kv) && a.hd == 128) launch_attn<128>(a, lds, st);
  else if (attn_vec(a.hd, a.kv) && a.hd == 32) launch_attn<32>(a, lds, st);
  else launch_attn<0>(a, lds, st);
  return hipGetLastError();
}

hipError_t argmax_finalize(const unsigned long long *cand, int ncand, const float *logits, int ldl, int rows,
                           int *out, hipStream_t st) {
  klaunch(argmax_finalize_kernel, dim3(rows), dim3(256), 0, st, cand, ncand, logits, ldl, out);
  return hipGetLastError();
}

hipError_t argmax_rows(const float *logits, int rows, int V, int *out, hipStream_t st) {
  klaunch(argmax_kernel, dim3(rows), dim3(256), 0, st, logits, V, out);
  return hipGetLastError();
}

}  // namespace ec
