// gfx950 kernels of the EdgeCore transformer forward hot path.
//
// Decode GEMV (M <= 8 rows per tile): weights stay in the reference layout
// [N][K] row-major.  A row is read by LPR lanes of one wave with 16-byte
// non-temporal loads (each instruction of a wave covers 64/LPR rows x LPR*16
// contiguous bytes), int8 rows are multiplied with v_dot4_i32_i8 into an exact
// int32 (any summation order gives the reference's int32), fp16/bf16 rows are
// widened to fp32 and accumulated with FMA.  The LPR partial sums are combined
// with a wave64 xor-shuffle tree and the epilogue (scales, bias, residual,
// GELU or SwiGLU) is applied in registers before the single store.
#include "gemv_impl.h"

#include <float.h>

namespace ec {

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
                                                    float *x, float *slots, int nslots, int ld) {
  const int m = blockIdx.x;
  if (slots)
    for (int j = threadIdx.x; j < nslots; j += 256) slots[(size_t)j * ld + m] = 0.0f;
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
// order: each score is one thread's sequential fp32 dot over head_dim, scaled
// in double; max; e = expf(s - max) with the reference's expf; double sum;
// p = (float)(e * (1/sum)); each output element is one thread's sequential
// fp32 sum over positions.  The int8 path turns any last-bit difference here
// into different activation codes downstream, so the order is kept exactly.
// The V rows of the attended positions are staged into LDS (tiles of vtile
// positions) with loads issued before the scores, so the sequential sums read
// LDS instead of waiting on memory.  HD > 0 fixes head_dim at compile time
// (whole K rows are loaded before each dot); HD == 0 is the generic path.
//
// FUSED: the block also rotates its q head and the token's new k (RoPE,
// src/gpt2.c:656-665, double cos/sin table) and uses the new k and v rounded
// to fp16 for the token's own position; the first query head of each KV group
// appends them to the cache (src/gpt2.c:726-741).  Only valid when no other
// token of the launch reads this token's slot.
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
        const float p0 = qs[8 * c + 2 * j] * h2f((uint16_t)(wv[j] & 0xffffu));
        s = s + p0;
        const float p1 = qs[8 * c + 2 * j + 1] * h2f((uint16_t)(wv[j] >> 16));
        s = s + p1;
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

template <int HD, bool FUSED>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  __shared__ float redf[4];
  __shared__ double redd[4];
  const int h = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
  const int pos = a.pos[m], slot = a.slot[m];
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
  float *kn = qs + hdp;  // FUSED: the new k (fp16-rounded), fp32
  float *sc = kn + (FUSED ? hdp : 0);
  uint16_t *vt = reinterpret_cast<uint16_t *>(sc + ((a.max_npos + 3) & ~3));
  const size_t cbase = (size_t)slot * a.C * a.kv + (size_t)kvh * hd;
  const uint16_t *K = a.kc + cbase + (size_t)lo * a.kv;
  const uint16_t *V = a.vc + cbase + (size_t)lo * a.kv;
  const bool vec = (hd & 7) == 0 && (a.kv & 7) == 0;
  const int ncache = FUSED ? n - 1 : n;  // positions read from the cache

  auto stage_v = [&](int t0) {  // cached V rows [t0, t0 + T) of the attended range -> vt
    const int cnt = min(T, ncache - t0);
    if (cnt <= 0) return;
    if (vec) {
      const int cpr = hd >> 3;
      for (int c = t; c < cnt * cpr; c += 256) {
        const int i = c / cpr, j = (c - i * cpr) << 3;
        *reinterpret_cast<v4u *>(vt + i * hd + j) = *reinterpret_cast<const v4u *>(V + (size_t)(t0 + i) * a.kv + j);
      }
    } else {
      for (int c = t; c < cnt * hd; c += 256) {
        const int i = c / hd, j = c - i * hd;
        vt[i * hd + j] = V[(size_t)(t0 + i) * a.kv + j];
      }
    }
  };

  const float *qrow = a.q + (size_t)m * a.ldq + (size_t)h * hd;
  if constexpr (FUSED) {
    const float *krow = a.k + (size_t)m * a.ldk + (size_t)kvh * hd;
    const float *vrow = a.v + (size_t)m * a.ldk + (size_t)kvh * hd;
    const bool writer = h == 0 || (h - 1) * a.KVH / a.H != kvh;  // first query head of the group
    const size_t woff = ((size_t)slot * a.C + pos) * a.kv + (size_t)kvh * hd;
    const int rot = a.cs ? a.half : 0;
    const double2 *cs = a.cs ? a.cs + (size_t)pos * a.half : nullptr;
    for (int i = t; i < hd; i += 256) {
      float qv, kvv;
      if (i < rot || (i >= rot && i < 2 * rot)) {
        const int i0 = i < rot ? i : i - rot;
        const double c = cs[i0].x, sn = cs[i0].y;
        const float q0 = qrow[i0], q1 = qrow[i0 + rot], k0 = krow[i0], k1 = krow[i0 + rot];
        if (i < rot) {
          const double t1 = q0 * c, t2 = q1 * sn, u1 = k0 * c, u2 = k1 * sn;
          qv = (float)(t1 - t2);
          kvv = (float)(u1 - u2);
        } else {
          const double t3 = q0 * sn, t4 = q1 * c, u3 = k0 * sn, u4 = k1 * c;
          qv = (float)(t3 + t4);
          kvv = (float)(u3 + u4);
        }
      } else {
        qv = qrow[i];
        kvv = krow[i];
      }
      qs[i] = qv;
      const uint16_t kh = f2h(kvv), vh = f2h(vrow[i]);
      kn[i] = h2f(kh);
      if (n - 1 < T) vt[(n - 1) * hd + i] = vh;  // own position lands in the first V tile
      if (writer) {
        a.kc_w[woff + i] = kh;
        a.vc_w[woff + i] = vh;
      }
    }
  } else {
    for (int d = t; d < hd; d += 256) qs[d] = qrow[d];
  }
  stage_v(0);
  __syncthreads();

  float mx = -FLT_MAX;
  for (int i = t; i < n; i += 256) {
    float s;
    if (FUSED && i == n - 1) {
      s = 0.0f;
      for (int d = 0; d < hd; d++) {
        const float p0 = qs[d] * kn[d];
        s = s + p0;
      }
    } else {
      s = dot_k_row<HD>(qs, K + (size_t)i * a.kv, hd);
    }
    s = (float)((double)s * a.inv_hd);
    sc[i] = s;
    mx = fmaxf(mx, s);
  }
  mx = block_max256(mx, redf);
  double sum = 0.0;
  for (int i = t; i < n; i += 256) {
    const float e = ec_expf_ref(sc[i] - mx);
    sc[i] = e;
    sum += (double)e;
  }
  sum = block_sum256(sum, redd);
  const double isum = 1.0 / sum;
  for (int i = t; i < n; i += 256) sc[i] = (float)((double)sc[i] * isum);
  __syncthreads();

  float o = 0.0f;
  for (int t0 = 0; t0 < n; t0 += T) {
    if (t0) {
      __syncthreads();
      stage_v(t0);
      if constexpr (FUSED) {
        if (n - 1 >= t0 && n - 1 < t0 + T) {  // own position lands in this tile
          const float *vrow = a.v + (size_t)m * a.ldk + (size_t)kvh * hd;
          for (int i = t; i < hd; i += 256) vt[(n - 1 - t0) * hd + i] = f2h(vrow[i]);
        }
      }
      __syncthreads();
    }
    if (t < hd) {
      const int cnt = min(T, n - t0);
      const uint16_t *vc = vt + t;
      const float *pp = sc + t0;
      int i = 0;
      for (; i + 8 <= cnt; i += 8) {
        float vv[8], pw[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
          vv[j] = h2f(vc[(i + j) * hd]);
          pw[j] = pp[i + j];
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const float pr = pw[j] * vv[j];
          o = o + pr;
        }
      }
      for (; i < cnt; i++) {
        const float pr = pp[i] * h2f(vc[i * hd]);
        o = o + pr;
      }
    }
  }
  if (t < hd) a.out[(size_t)m * a.ldo + (size_t)h * hd + t] = o;
  if (a.out_max) {  // row max |out| for the next linear's int8 quantization (NaN ignored)
    const float r = block_max256(t < hd ? fabsf(o) : 0.0f, redf);
    if (t == 0) atomicMax(reinterpret_cast<unsigned int *>(a.out_max + m), __float_as_uint(r));
  }
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
  default: break;
  }
}

hipError_t device_math(int op, const void *in, void *out, size_t n, hipStream_t st) {
  if (op < 0 || op > MATH_QUANT1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(math_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, op, in, out, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

static int g_gemv_max_blocks = 1024;
void gemv_set_max_blocks(int n) { g_gemv_max_blocks = n > 0 ? n : 1024; }
int gemv_max_blocks() { return g_gemv_max_blocks; }

int gemv_pick_mt(int M) { return M >= 5 ? 8 : M >= 3 ? 4 : M == 2 ? 2 : 1; }

// lanes per row: the narrow variant (4 or 2 rows per wave) when the whole
// row fits its register block and there are enough row groups to fill the
// chip, else one row per wave
int gemv_pick_lpr(int wt, int epi, int K, int N) {
  const int chb = wt == WT_I8 ? 16 : 8;
  const int narrow = wt == WT_I8 ? 16 : 32;
  const int nch = K / chb;
  const int rpb = (epi == EPI_SWIGLU ? 2 : 4) * (64 / narrow);
  if (nch <= narrow * lpr_cpl(narrow) && (N + rpb - 1) / rpb >= 256) return narrow;
  return 64;
}

int gemv_grid_x(const GemvArgs &a, int wt, int epi) {
  const int lpr = gemv_pick_lpr(wt, epi, a.K, a.N);
  const int rpb = (epi == EPI_SWIGLU ? 2 : 4) * (64 / lpr);
  const int ng = (a.N + rpb - 1) / rpb;
  return ng < g_gemv_max_blocks ? ng : g_gemv_max_blocks;
}

size_t gemv_lds_bytes(int wt, int pro, int MT, int K) {
  if (pro == PRO_F32) return 0;
  if (wt == WT_I8) {
    const size_t kp = (size_t)(K + 15) / 16 * 16;
    return (MT * kp + 4 * MT + 15) / 16 * 16;
  }
  const size_t kp = (size_t)(K + 7) / 8 * 8;
  return MT * kp * 4;
}

static int g_max_lds_bytes = 65536;

bool gemv_vector_ok(const GemvArgs &a, int wt, int pro) {
  const int chb = wt == WT_I8 ? 16 : 8;
  if (a.K <= 0 || a.K % chb || !al16(a.W) || (a.W2 && !al16(a.W2))) return false;
  if (pro == PRO_I8 && (a.lda % 16 || !al16(a.A))) return false;
  if (pro == PRO_F32 && (a.lda % 4 || !al16(a.A))) return false;
  if (wt == WT_I8 && pro == PRO_F32) return false;
  if (wt != WT_I8 && (pro == PRO_I8 || pro == PRO_QUANT)) return false;
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
  hipLaunchKernelGGL((gemv_generic_kernel<WT, EPI>), dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, a);
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
  hipLaunchKernelGGL(quant_kernel, dim3(M), dim3(256), 0, st, in, ldi, K, q, ldq, s);
  return hipGetLastError();
}

hipError_t norm_rows(const float *x, int M, int E, const float *gamma, const float *beta,
                     double eps, float *h, int ldh, int8_t *q, int ldq, float *qs,
                     hipStream_t st) {
  const size_t lds = (size_t)E * sizeof(float);
  if (beta) {
    if (q) hipLaunchKernelGGL((norm_kernel<true, true>), dim3(M), dim3(256), lds, st, x, E, gamma, beta, eps, h, ldh, q, ldq, qs);
    else hipLaunchKernelGGL((norm_kernel<true, false>), dim3(M), dim3(256), lds, st, x, E, gamma, beta, eps, h, ldh, q, ldq, qs);
  } else {
    if (q) hipLaunchKernelGGL((norm_kernel<false, true>), dim3(M), dim3(256), lds, st, x, E, gamma, beta, eps, h, ldh, q, ldq, qs);
    else hipLaunchKernelGGL((norm_kernel<false, false>), dim3(M), dim3(256), lds, st, x, E, gamma, beta, eps, h, ldh, q, ldq, qs);
  }
  return hipGetLastError();
}

hipError_t embed(const uint16_t *wte, const uint16_t *wpe, bool bf16, const int *tok,
                 const int *pos, int M, int E, float *x, float *slots, int nslots, int ld,
                 hipStream_t st) {
  if (bf16)
    hipLaunchKernelGGL(embed_kernel<true>, dim3(M), dim3(256), 0, st, wte, wpe, tok, pos, E, x, slots, nslots, ld);
  else
    hipLaunchKernelGGL(embed_kernel<false>, dim3(M), dim3(256), 0, st, wte, wpe, tok, pos, E, x, slots, nslots, ld);
  return hipGetLastError();
}

hipError_t rope_kv_append(const KvArgs &a, hipStream_t st) {
  hipLaunchKernelGGL(rope_kv_kernel, dim3(a.M), dim3(256), 0, st, a);
  return hipGetLastError();
}

size_t attention_lds_bytes(int max_npos, int hd, int vtile) {
  return ((size_t)((hd + 3) & ~3) + (size_t)((max_npos + 3) & ~3)) * sizeof(float) +
         (size_t)vtile * hd * sizeof(uint16_t);
}

template <int HD>
static void launch_attn(const AttnArgs &a, size_t lds, hipStream_t st) {
  if (a.fuse_kv) hipLaunchKernelGGL((attn_kernel<HD, true>), dim3(a.H, a.M), dim3(256), lds, st, a);
  else hipLaunchKernelGGL((attn_kernel<HD, false>), dim3(a.H, a.M), dim3(256), lds, st, a);
}

hipError_t attention(const AttnArgs &a, hipStream_t st) {
  const size_t lds = attention_lds_bytes(a.max_npos, a.hd, a.vtile) +
                     (a.fuse_kv ? (size_t)((a.hd + 3) & ~3) * sizeof(float) : 0);
  const bool vec = (a.kv & 7) == 0;
  if (vec && a.hd == 64) launch_attn<64>(a, lds, st);
  else if (vec && a.hd == 128) launch_attn<128>(a, lds, st);
  else if (vec && a.hd == 32) launch_attn<32>(a, lds, st);
  else launch_attn<0>(a, lds, st);
  return hipGetLastError();
}

hipError_t argmax_finalize(const unsigned long long *cand, int ncand, const float *logits, int ldl, int rows,
                           int *out, hipStream_t st) {
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(rows), dim3(256), 0, st, cand, ncand, logits, ldl, out);
  return hipGetLastError();
}

hipError_t argmax_rows(const float *logits, int rows, int V, int *out, hipStream_t st) {
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(256), 0, st, logits, V, out);
  return hipGetLastError();
}

}  // namespace ec
