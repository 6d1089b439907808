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
#include "ec_device.h"
#include "ec_kernels.h"

#include <float.h>

namespace ec {

// ---------------------------------------------------------------------------
// int8 GEMV
// ---------------------------------------------------------------------------

template <int LPR, int MT, int EPI>
__global__ __launch_bounds__(256) void gemv_i8_kernel(GemvI8Args a) {
  constexpr int RPW = kWave / LPR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = lane / LPR, sub = lane % LPR;
  int n, part = 0, rib;
  if constexpr (EPI == EPI_SWIGLU) {
    rib = (wave & 1) * RPW + grp;  // waves 0-1: gate rows, waves 2-3: up rows
    part = wave >> 1;
    n = blockIdx.x * (2 * RPW) + rib;
  } else {
    rib = wave * RPW + grp;
    n = blockIdx.x * (4 * RPW) + rib;
  }
  const int m0 = blockIdx.y * MT;
  const int mc = min(MT, a.M - m0);
  const bool valid = n < a.N;
  const int8_t *W = (EPI == EPI_SWIGLU && part) ? a.W2 : a.W;
  const int nch = a.K >> 4;

  int acc[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) acc[m] = 0;
  if (valid) {
    const v4i *wrow = reinterpret_cast<const v4i *>(W + (size_t)n * a.K);
#pragma unroll 4
    for (int c = sub; c < nch; c += LPR) {
      v4i w = __builtin_nontemporal_load(wrow + c);
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (m < mc) {
          v4i x = reinterpret_cast<const v4i *>(a.A + (size_t)(m0 + m) * a.lda)[c];
          int t = acc[m];
          t = __builtin_amdgcn_sdot4(x.x, w.x, t, false);
          t = __builtin_amdgcn_sdot4(x.y, w.y, t, false);
          t = __builtin_amdgcn_sdot4(x.z, w.z, t, false);
          t = __builtin_amdgcn_sdot4(x.w, w.w, t, false);
          acc[m] = t;
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MT; m++) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) acc[m] += __shfl_xor(acc[m], o, kWave);
  }

  if constexpr (EPI == EPI_SWIGLU) {
    __shared__ float up[MT][2 * RPW];
    if (sub == 0 && valid && part == 1) {
      const float bs = a.ws2 ? a.ws2[n] : 1.0f;
#pragma unroll
      for (int m = 0; m < MT; m++)
        if (m < mc) up[m][rib] = i8_epilogue(acc[m], a.as[m0 + m], bs, 0.0f);
    }
    __syncthreads();
    if (sub == 0 && valid && part == 0) {
      const float bs = a.ws ? a.ws[n] : 1.0f;
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (m < mc) {
          float g = i8_epilogue(acc[m], a.as[m0 + m], bs, 0.0f);
          float r = silu(g) * up[m][rib];
          a.out[(size_t)(m0 + m) * a.ldo + n] = r;
        }
      }
    }
  } else {
    if (sub == 0 && valid) {
      const float bs = a.ws ? a.ws[n] : 1.0f;
      const float bv = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (m < mc) {
          float v = i8_epilogue(acc[m], a.as[m0 + m], bs, bv);
          float *o = a.out + (size_t)(m0 + m) * a.ldo + n;
          if constexpr (EPI == EPI_RESID) v = *o + v;
          if constexpr (EPI == EPI_GELU) v = gelu_new(v);
          *o = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp16 / bf16 GEMV with fp32 activations
// ---------------------------------------------------------------------------

template <int LPR, int MT, int EPI, bool BF16>
__global__ __launch_bounds__(256) void gemv_w16_kernel(GemvW16Args a) {
  constexpr int RPW = kWave / LPR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = lane / LPR, sub = lane % LPR;
  int n, part = 0, rib;
  if constexpr (EPI == EPI_SWIGLU) {
    rib = (wave & 1) * RPW + grp;
    part = wave >> 1;
    n = blockIdx.x * (2 * RPW) + rib;
  } else {
    rib = wave * RPW + grp;
    n = blockIdx.x * (4 * RPW) + rib;
  }
  const int m0 = blockIdx.y * MT;
  const int mc = min(MT, a.M - m0);
  const bool valid = n < a.N;
  const uint16_t *W = (EPI == EPI_SWIGLU && part) ? a.W2 : a.W;
  const int nch = a.K >> 3;

  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) acc[m] = 0.0f;
  if (valid) {
    const v4u *wrow = reinterpret_cast<const v4u *>(W + (size_t)n * a.K);
#pragma unroll 4
    for (int c = sub; c < nch; c += LPR) {
      v4u w = __builtin_nontemporal_load(wrow + c);
      float wf[8];
      wf[0] = w2f<BF16>((uint16_t)(w.x & 0xffffu));
      wf[1] = w2f<BF16>((uint16_t)(w.x >> 16));
      wf[2] = w2f<BF16>((uint16_t)(w.y & 0xffffu));
      wf[3] = w2f<BF16>((uint16_t)(w.y >> 16));
      wf[4] = w2f<BF16>((uint16_t)(w.z & 0xffffu));
      wf[5] = w2f<BF16>((uint16_t)(w.z >> 16));
      wf[6] = w2f<BF16>((uint16_t)(w.w & 0xffffu));
      wf[7] = w2f<BF16>((uint16_t)(w.w >> 16));
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (m < mc) {
          const float4 *ap = reinterpret_cast<const float4 *>(a.A + (size_t)(m0 + m) * a.lda) + 2 * c;
          float4 x0 = ap[0], x1 = ap[1];
          float t = acc[m];
          t = __builtin_fmaf(x0.x, wf[0], t);
          t = __builtin_fmaf(x0.y, wf[1], t);
          t = __builtin_fmaf(x0.z, wf[2], t);
          t = __builtin_fmaf(x0.w, wf[3], t);
          t = __builtin_fmaf(x1.x, wf[4], t);
          t = __builtin_fmaf(x1.y, wf[5], t);
          t = __builtin_fmaf(x1.z, wf[6], t);
          t = __builtin_fmaf(x1.w, wf[7], t);
          acc[m] = t;
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MT; m++) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) acc[m] += __shfl_xor(acc[m], o, kWave);
  }

  if constexpr (EPI == EPI_SWIGLU) {
    __shared__ float up[MT][2 * RPW];
    if (sub == 0 && valid && part == 1) {
#pragma unroll
      for (int m = 0; m < MT; m++)
        if (m < mc) up[m][rib] = acc[m];
    }
    __syncthreads();
    if (sub == 0 && valid && part == 0) {
#pragma unroll
      for (int m = 0; m < MT; m++)
        if (m < mc) a.out[(size_t)(m0 + m) * a.ldo + n] = silu(acc[m]) * up[m][rib];
    }
  } else {
    if (sub == 0 && valid) {
      const float bv = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (m < mc) {
          float v = acc[m];
          float *o = a.out + (size_t)(m0 + m) * a.ldo + n;
          if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_RESID || EPI == EPI_BIAS_GELU) v = v + bv;
          if constexpr (EPI == EPI_RESID || EPI == EPI_BIAS_RESID) v = *o + v;
          if constexpr (EPI == EPI_GELU || EPI == EPI_BIAS_GELU) v = gelu_new(v);
          *o = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// generic GEMMs (any K, any alignment, every epilogue): one thread per output
// element.  Used for shapes the vector kernels cannot read with 16-byte loads.
// ---------------------------------------------------------------------------

template <int EPI>
__global__ __launch_bounds__(256) void gemm_i8_generic_kernel(GemvI8Args a) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)a.M * a.N) return;
  const int m = (int)(idx / a.N), n = (int)(idx % a.N);
  const int8_t *x = a.A + (size_t)m * a.lda, *w = a.W + (size_t)n * a.K;
  int dot = 0;
  for (int k = 0; k < a.K; k++) dot += (int)x[k] * (int)w[k];
  float v = i8_epilogue(dot, a.as[m], a.ws ? a.ws[n] : 1.0f, a.bias ? a.bias[n] : 0.0f);
  float *o = a.out + (size_t)m * a.ldo + n;
  if constexpr (EPI == EPI_SWIGLU) {
    const int8_t *w2 = a.W2 + (size_t)n * a.K;
    int d2 = 0;
    for (int k = 0; k < a.K; k++) d2 += (int)x[k] * (int)w2[k];
    const float u = i8_epilogue(d2, a.as[m], a.ws2 ? a.ws2[n] : 1.0f, 0.0f);
    v = silu(v) * u;
  }
  if constexpr (EPI == EPI_RESID) v = *o + v;
  if constexpr (EPI == EPI_GELU) v = gelu_new(v);
  *o = v;
}

template <int EPI, bool BF16>
__global__ __launch_bounds__(256) void gemm_w16_generic_kernel(GemvW16Args a) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)a.M * a.N) return;
  const int m = (int)(idx / a.N), n = (int)(idx % a.N);
  const float *x = a.A + (size_t)m * a.lda;
  const uint16_t *w = a.W + (size_t)n * a.K;
  float v = 0.0f;
  for (int k = 0; k < a.K; k++) v = __builtin_fmaf(x[k], w2f<BF16>(w[k]), v);
  float *o = a.out + (size_t)m * a.ldo + n;
  if constexpr (EPI == EPI_SWIGLU) {
    const uint16_t *w2 = a.W2 + (size_t)n * a.K;
    float u = 0.0f;
    for (int k = 0; k < a.K; k++) u = __builtin_fmaf(x[k], w2f<BF16>(w2[k]), u);
    v = silu(v) * u;
  }
  if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_RESID || EPI == EPI_BIAS_GELU) v = v + a.bias[n];
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

// One block per (head, token).  Each score is one thread's sequential fp32
// dot over head_dim in the reference order; max, exp (in double, rounded
// once), double sum and the normalisation follow the reference; each output
// element is one thread's sequential sum over positions in the reference
// order.  Scores live in LDS.
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
  extern __shared__ float lds[];
  __shared__ float redf[4];
  __shared__ double redd[4];
  const int h = blockIdx.x, m = blockIdx.y;
  const int pos = a.pos[m], slot = a.slot[m];
  const int kvh = h * a.KVH / a.H;
  int lo = 0;
  if (a.window > 0) {
    lo = pos - a.window + 1;
    if (lo < 0) lo = 0;
  }
  const int n = pos + 1 - lo;
  const int hd = a.hd;
  float *qs = lds;
  float *sc = lds + ((hd + 3) & ~3);
  const float *q = a.q + (size_t)m * a.ldq + (size_t)h * hd;
  for (int d = threadIdx.x; d < hd; d += 256) qs[d] = q[d];
  __syncthreads();
  const size_t cbase = (size_t)slot * a.C * a.kv + (size_t)kvh * hd;
  const uint16_t *K = a.kc + cbase + (size_t)lo * a.kv;
  const uint16_t *V = a.vc + cbase + (size_t)lo * a.kv;

  float mx = -FLT_MAX;
  const bool vec = (hd & 7) == 0 && (a.kv & 7) == 0;
  for (int i = threadIdx.x; i < n; i += 256) {
    const uint16_t *kp = K + (size_t)i * a.kv;
    float s = 0.0f;
    if (vec) {
      for (int d = 0; d < hd; d += 8) {
        const v4u kk = *reinterpret_cast<const v4u *>(kp + d);
        const uint32_t wv[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          float p0 = qs[d + 2 * j] * h2f((uint16_t)(wv[j] & 0xffffu));
          s = s + p0;
          float p1 = qs[d + 2 * j + 1] * h2f((uint16_t)(wv[j] >> 16));
          s = s + p1;
        }
      }
    } else {
      for (int d = 0; d < hd; d++) {
        float p0 = qs[d] * h2f(kp[d]);
        s = s + p0;
      }
    }
    s = (float)((double)s * a.inv_hd);
    sc[i] = s;
    mx = fmaxf(mx, s);
  }
  mx = block_max256(mx, redf);
  double sum = 0.0;
  for (int i = threadIdx.x; i < n; i += 256) {
    const float e = expf_d(sc[i] - mx);
    sc[i] = e;
    sum += (double)e;
  }
  sum = block_sum256(sum, redd);
  const double isum = 1.0 / sum;
  for (int i = threadIdx.x; i < n; i += 256) sc[i] = (float)((double)sc[i] * isum);
  __syncthreads();
  for (int d = threadIdx.x; d < hd; d += 256) {
    const uint16_t *vp = V + d;
    float o = 0.0f;
    int i = 0;
    for (; i + 8 <= n; i += 8) {
      float vv[8];
#pragma unroll
      for (int j = 0; j < 8; j++) vv[j] = h2f(vp[(size_t)(i + j) * a.kv]);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        float p = sc[i + j] * vv[j];
        o = o + p;
      }
    }
    for (; i < n; i++) {
      float p = sc[i] * h2f(vp[(size_t)i * a.kv]);
      o = o + p;
    }
    a.out[(size_t)m * a.ldo + (size_t)h * hd + d] = o;
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

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

bool gemv_i8_vector_ok(const GemvI8Args &a) {
  return a.K % 16 == 0 && a.lda % 16 == 0 && al16(a.A) && al16(a.W) && (!a.W2 || al16(a.W2));
}

bool gemv_w16_vector_ok(const GemvW16Args &a) {
  return a.K % 8 == 0 && a.lda % 4 == 0 && al16(a.A) && al16(a.W) && (!a.W2 || al16(a.W2));
}

static int pick_mt(int M) { return M >= 5 ? 8 : M >= 3 ? 4 : M == 2 ? 2 : 1; }
static int pick_lpr(int chunks) { return chunks >= 48 ? 64 : chunks >= 24 ? 32 : 16; }

template <int LPR, int MT, int EPI>
static hipError_t launch_i8(const GemvI8Args &a, hipStream_t s) {
  const int rpb = (EPI == EPI_SWIGLU ? 2 : 4) * (kWave / LPR);
  dim3 grid((a.N + rpb - 1) / rpb, (a.M + MT - 1) / MT);
  hipLaunchKernelGGL((gemv_i8_kernel<LPR, MT, EPI>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int LPR, int EPI>
static hipError_t launch_i8_mt(const GemvI8Args &a, hipStream_t s) {
  switch (pick_mt(a.M)) {
  case 1: return launch_i8<LPR, 1, EPI>(a, s);
  case 2: return launch_i8<LPR, 2, EPI>(a, s);
  case 4: return launch_i8<LPR, 4, EPI>(a, s);
  default: return launch_i8<LPR, 8, EPI>(a, s);
  }
}

template <int EPI>
static hipError_t launch_i8_lpr(const GemvI8Args &a, hipStream_t s) {
  switch (pick_lpr(a.K >> 4)) {
  case 64: return launch_i8_mt<64, EPI>(a, s);
  case 32: return launch_i8_mt<32, EPI>(a, s);
  default: return launch_i8_mt<16, EPI>(a, s);
  }
}

template <int EPI>
static hipError_t launch_i8_generic(const GemvI8Args &a, hipStream_t s) {
  const size_t tot = (size_t)a.M * a.N;
  hipLaunchKernelGGL(gemm_i8_generic_kernel<EPI>, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t gemm_i8_generic(const GemvI8Args &a, int epi, hipStream_t s) {
  switch (epi) {
  case EPI_STORE: return launch_i8_generic<EPI_STORE>(a, s);
  case EPI_RESID: return launch_i8_generic<EPI_RESID>(a, s);
  case EPI_GELU: return launch_i8_generic<EPI_GELU>(a, s);
  case EPI_SWIGLU: return launch_i8_generic<EPI_SWIGLU>(a, s);
  default: return hipErrorInvalidValue;
  }
}

hipError_t gemv_i8(const GemvI8Args &a, int epi, hipStream_t s) {
  if (a.K == 0 || !gemv_i8_vector_ok(a)) return gemm_i8_generic(a, epi, s);
  switch (epi) {
  case EPI_STORE: return launch_i8_lpr<EPI_STORE>(a, s);
  case EPI_RESID: return launch_i8_lpr<EPI_RESID>(a, s);
  case EPI_GELU: return launch_i8_lpr<EPI_GELU>(a, s);
  case EPI_SWIGLU: return launch_i8_lpr<EPI_SWIGLU>(a, s);
  default: return hipErrorInvalidValue;
  }
}

template <int LPR, int MT, int EPI, bool BF16>
static hipError_t launch_w16(const GemvW16Args &a, hipStream_t s) {
  const int rpb = (EPI == EPI_SWIGLU ? 2 : 4) * (kWave / LPR);
  dim3 grid((a.N + rpb - 1) / rpb, (a.M + MT - 1) / MT);
  hipLaunchKernelGGL((gemv_w16_kernel<LPR, MT, EPI, BF16>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int LPR, int EPI, bool BF16>
static hipError_t launch_w16_mt(const GemvW16Args &a, hipStream_t s) {
  switch (pick_mt(a.M)) {
  case 1: return launch_w16<LPR, 1, EPI, BF16>(a, s);
  case 2: return launch_w16<LPR, 2, EPI, BF16>(a, s);
  case 4: return launch_w16<LPR, 4, EPI, BF16>(a, s);
  default: return launch_w16<LPR, 8, EPI, BF16>(a, s);
  }
}

template <int EPI, bool BF16>
static hipError_t launch_w16_lpr(const GemvW16Args &a, hipStream_t s) {
  switch (pick_lpr(a.K >> 3)) {
  case 64: return launch_w16_mt<64, EPI, BF16>(a, s);
  case 32: return launch_w16_mt<32, EPI, BF16>(a, s);
  default: return launch_w16_mt<16, EPI, BF16>(a, s);
  }
}

template <bool BF16>
static hipError_t gemv_w16_t(const GemvW16Args &a, int epi, hipStream_t s) {
  switch (epi) {
  case EPI_STORE: return launch_w16_lpr<EPI_STORE, BF16>(a, s);
  case EPI_RESID: return launch_w16_lpr<EPI_RESID, BF16>(a, s);
  case EPI_SWIGLU: return launch_w16_lpr<EPI_SWIGLU, BF16>(a, s);
  case EPI_BIAS: return launch_w16_lpr<EPI_BIAS, BF16>(a, s);
  case EPI_BIAS_RESID: return launch_w16_lpr<EPI_BIAS_RESID, BF16>(a, s);
  case EPI_BIAS_GELU: return launch_w16_lpr<EPI_BIAS_GELU, BF16>(a, s);
  default: return hipErrorInvalidValue;
  }
}

template <int EPI, bool BF16>
static hipError_t launch_w16_generic(const GemvW16Args &a, hipStream_t s) {
  const size_t tot = (size_t)a.M * a.N;
  hipLaunchKernelGGL((gemm_w16_generic_kernel<EPI, BF16>), dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <bool BF16>
static hipError_t gemm_w16_generic_t(const GemvW16Args &a, int epi, hipStream_t s) {
  switch (epi) {
  case EPI_STORE: return launch_w16_generic<EPI_STORE, BF16>(a, s);
  case EPI_RESID: return launch_w16_generic<EPI_RESID, BF16>(a, s);
  case EPI_SWIGLU: return launch_w16_generic<EPI_SWIGLU, BF16>(a, s);
  case EPI_BIAS: return launch_w16_generic<EPI_BIAS, BF16>(a, s);
  case EPI_BIAS_RESID: return launch_w16_generic<EPI_BIAS_RESID, BF16>(a, s);
  case EPI_BIAS_GELU: return launch_w16_generic<EPI_BIAS_GELU, BF16>(a, s);
  default: return hipErrorInvalidValue;
  }
}

hipError_t gemm_w16_generic(const GemvW16Args &a, int epi, bool bf16, hipStream_t s) {
  return bf16 ? gemm_w16_generic_t<true>(a, epi, s) : gemm_w16_generic_t<false>(a, epi, s);
}

hipError_t gemv_w16(const GemvW16Args &a, int epi, bool bf16, hipStream_t s) {
  if (a.K == 0 || !gemv_w16_vector_ok(a)) return gemm_w16_generic(a, epi, bf16, s);
  return bf16 ? gemv_w16_t<true>(a, epi, s) : gemv_w16_t<false>(a, epi, s);
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
                 const int *pos, int M, int E, float *x, hipStream_t st) {
  if (bf16) hipLaunchKernelGGL(embed_kernel<true>, dim3(M), dim3(256), 0, st, wte, wpe, tok, pos, E, x);
  else hipLaunchKernelGGL(embed_kernel<false>, dim3(M), dim3(256), 0, st, wte, wpe, tok, pos, E, x);
  return hipGetLastError();
}

hipError_t rope_kv_append(const KvArgs &a, hipStream_t st) {
  hipLaunchKernelGGL(rope_kv_kernel, dim3(a.M), dim3(256), 0, st, a);
  return hipGetLastError();
}

size_t attention_lds_bytes(int max_npos, int hd) {
  return ((size_t)((hd + 3) & ~3) + (size_t)max_npos) * sizeof(float);
}

hipError_t attention(const AttnArgs &a, hipStream_t st) {
  const size_t lds = attention_lds_bytes(a.max_npos, a.hd);
  hipLaunchKernelGGL(attn_kernel, dim3(a.H, a.M), dim3(256), lds, st, a);
  return hipGetLastError();
}

hipError_t argmax_rows(const float *logits, int rows, int V, int *out, hipStream_t st) {
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(256), 0, st, logits, V, out);
  return hipGetLastError();
}

}  // namespace ec
