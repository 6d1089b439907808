// gfx950 kernels of the EdgeCore transformer forward hot path.
//
// The fused decode GEMV lives in gemv_impl.h (instantiated per weight type in
// gemv_*.hip); this file holds the generic GEMV, norms, quantizer, embedding,
// RoPE/KV append, attention, argmax, elementwise math and the launchers.
#include "attn_decode.h"
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

// the same for rows whose K is a multiple of 4 (16-byte aligned fp32 rows,
// 4-byte aligned int8 rows): each thread keeps its NV float4 of the row in
// registers between the max and the quantization
template <int NV>
__global__ __launch_bounds__(256) void quant_vec_kernel(const float *in, int ldi, int K, int8_t *q, int ldq,
                                                        float *s) {
  __shared__ float red[4];
  const int m = blockIdx.x, t = threadIdx.x, K4 = K / 4;
  const float4 *x = reinterpret_cast<const float4 *>(in + (size_t)m * ldi);
  float4 v[NV];
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = t + 256 * j;
    if (i < K4) {
      v[j] = x[i];
      mx = fmaxf(mx, fabsf(v[j].x));
      mx = fmaxf(mx, fabsf(v[j].y));
      mx = fmaxf(mx, fabsf(v[j].z));
      mx = fmaxf(mx, fabsf(v[j].w));
    }
  }
  mx = block_max256_1b(mx, red);
  const float sc = quant_scale(mx);
  if (t == 0) s[m] = sc;
  uint32_t *qr = reinterpret_cast<uint32_t *>(q + (size_t)m * ldq);
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = t + 256 * j;
    if (i < K4)
      qr[i] = (uint32_t)(uint8_t)quant1(v[j].x, sc) | ((uint32_t)(uint8_t)quant1(v[j].y, sc) << 8) |
              ((uint32_t)(uint8_t)quant1(v[j].z, sc) << 16) | ((uint32_t)(uint8_t)quant1(v[j].w, sc) << 24);
  }
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

// The same arithmetic per element for rows of E % 4 == 0 (16-byte aligned
// rows, gamma and beta): each thread loads its NV float4 of x, gamma and beta
// at the start and keeps them in registers (no LDS row, no dependent gamma
// load after the reductions), and each reduction takes one barrier.  The
// double sums run in another order than norm_kernel's (per thread over its
// float4s, then the block tree), which can move only their last bits.
template <bool LN, bool QUANT, int NV>
__global__ __launch_bounds__(256) void norm_vec_kernel(const float *x, int E, const float *gamma,
                                                       const float *beta, double eps, float *h, int ldh,
                                                       int8_t *q, int ldq, float *qs) {
  __shared__ double redd[8];
  __shared__ float redf[4];
  const int m = blockIdx.x, t = threadIdx.x, E4 = E / 4;
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)m * E);
  const float4 *g4 = reinterpret_cast<const float4 *>(gamma);
  const float4 *b4 = reinterpret_cast<const float4 *>(beta);
  float4 v[NV], g[NV], b[NV];
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = t + 256 * j;
    v[j] = g[j] = b[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < E4) {
      v[j] = xr[i];
      g[j] = g4[i];
      if constexpr (LN) b[j] = b4[i];
    }
  }
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const double d0 = v[j].x, d1 = v[j].y, d2 = v[j].z, d3 = v[j].w;
    acc += LN ? ((d0 + d1) + d2) + d3 : ((d0 * d0 + d1 * d1) + d2 * d2) + d3 * d3;
  }
  const double tot = block_sum256_1b(acc, redd);
  double mean = 0.0, rstd;
  if constexpr (LN) {
    mean = tot / E;
    double a2 = 0.0;
#pragma unroll
    for (int j = 0; j < NV; j++) {
      if (t + 256 * j < E4) {
        const double d0 = (double)v[j].x - mean, d1 = (double)v[j].y - mean, d2 = (double)v[j].z - mean,
                     d3 = (double)v[j].w - mean;
        a2 += ((d0 * d0 + d1 * d1) + d2 * d2) + d3 * d3;
      }
    }
    rstd = 1.0 / sqrt(block_sum256_1b(a2, redd + 4) / E + eps);
  } else {
    rstd = 1.0 / sqrt(tot / E + eps);
  }
  auto nrm = [&](float xv, float gv, float bv) {
    float r = LN ? (float)(((double)xv - mean) * rstd) : (float)((double)xv * rstd);
    r = r * gv;
    if constexpr (LN) r = r + bv;
    return r;
  };
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    v[j] = make_float4(nrm(v[j].x, g[j].x, b[j].x), nrm(v[j].y, g[j].y, b[j].y), nrm(v[j].z, g[j].z, b[j].z),
                       nrm(v[j].w, g[j].w, b[j].w));
    if (t + 256 * j < E4) {
      if constexpr (QUANT) {
        mx = fmaxf(mx, fabsf(v[j].x));
        mx = fmaxf(mx, fabsf(v[j].y));
        mx = fmaxf(mx, fabsf(v[j].z));
        mx = fmaxf(mx, fabsf(v[j].w));
      } else {
        reinterpret_cast<float4 *>(h + (size_t)m * ldh)[t + 256 * j] = v[j];
      }
    }
  }
  if constexpr (QUANT) {
    mx = block_max256_1b(mx, redf);
    const float sc = quant_scale(mx);
    if (t == 0) qs[m] = sc;
    uint32_t *qr = reinterpret_cast<uint32_t *>(q + (size_t)m * ldq);
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const int i = t + 256 * j;
      if (i < E4)
        qr[i] = (uint32_t)(uint8_t)quant1(v[j].x, sc) | ((uint32_t)(uint8_t)quant1(v[j].y, sc) << 8) |
                ((uint32_t)(uint8_t)quant1(v[j].z, sc) << 16) | ((uint32_t)(uint8_t)quant1(v[j].w, sc) << 24);
    }
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
// decode attention (src/gpt2.c:527-557 and 744-777): attn_decode.h
// ---------------------------------------------------------------------------
// One block per (head, token) -- NS blocks per head with element slices --
// running attn_decode_block (attn_decode.h) on the token's q row and new k/v
// rows in global memory.
template <int HD, bool FUSED, int NS, bool SCORED = false>
__global__ __launch_bounds__(attn_threads(HD, NS, SCORED)) void attn_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int m = blockIdx.y;
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
  const int hd = HD > 0 ? HD : a.hd, kvh = h * a.KVH / a.H;
  const float *qrow = a.q + (size_t)m * a.ldq + (size_t)h * hd;
  const float *krow = a.k + (size_t)m * a.ldk + (size_t)kvh * hd;
  const float *vrow = a.v + (size_t)m * a.ldk + (size_t)kvh * hd;
  float *orow = a.out + (size_t)m * a.ldo + (size_t)h * hd + (size_t)(hd / NS) * slice;
  float oabs = 0.0f;  // the largest |output| of this thread (NaN as 0)
  attn_decode_block<HD, FUSED, NS, SCORED>(a, m, h, slice, qrow, krow, vrow, lds, [&](int i, float o) {
    orow[i] = o;
    oabs = fmaxf(oabs, fabsf(o));
  });
  if (a.pmax) {  // uniform
    constexpr int NT = attn_threads(HD, NS, SCORED);
    __shared__ float red[NT / 64];
    const float mx = block_max_1b<NT / 64>(oabs, red);
    if (threadIdx.x == 0) a.pmax[(size_t)m * a.np + 4 * h + slice] = mx;
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

// first-stage argmax over chunks of csz logits: the orderable key (amax_key:
// larger value, then lower index) of each (row, chunk) into cand[row][chunk];
// NaN never wins, 0 stands for a chunk without a non-NaN value
__global__ __launch_bounds__(256) void argmax_chunk_kernel(const float *L, int V, int csz,
                                                           unsigned long long *cand) {
  __shared__ unsigned long long red[4];
  const int c = blockIdx.x, r = blockIdx.y, nc = gridDim.x;
  const float *l = L + (size_t)r * V;
  const int e = min(V, (c + 1) * csz);
  unsigned long long b = 0ull;
  for (int i = c * csz + threadIdx.x; i < e; i += 256) {
    const float v = l[i];
    if (v == v) {
      const unsigned long long k = amax_key(v, i);
      b = k > b ? k : b;
    }
  }
  b = wave_max_u64(b);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; w++) b = red[w] > b ? red[w] : b;
    cand[(size_t)r * nc + c] = b;
  }
}

// argmax over the LM head's per-block candidates; logits[0] NaN -> 0 and no
// non-NaN logit -> 0, like the reference's strict '>' scan from index 0
__global__ __launch_bounds__(256) void argmax_finalize_kernel(const unsigned long long *cand, int ncand,
                                                              const float *logits, int ldl, int *out,
                                                              int *chain_io, int *chain_out,
                                                              unsigned long long *chain_t) {
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
    const int id = (l0 != l0 || b == 0ull) ? 0 : (int)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFull));
    out[r] = id;
    if (chain_io) {  // a chained greedy step (one row): step_advance_kernel's work
      if (chain_t) chain_t[chain_io[6] + 1] = __builtin_amdgcn_s_memrealtime();
      chain_out[chain_io[6]] = id;
      chain_io[6] = chain_io[6] + 1;
      chain_io[0] = id;
      chain_io[1] = chain_io[1] + 1;
      chain_io[3] = (int)((unsigned)chain_io[3] + 1u);
    }
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
  const bool vec = K % 4 == 0 && ldi % 4 == 0 && ldq % 4 == 0 && ((uintptr_t)in & 15u) == 0 &&
                   ((uintptr_t)q & 3u) == 0 && K <= 256 * 4 * 16;
  if (vec) {
    const int nv = (K / 4 + 255) / 256;
    if (nv <= 1) klaunch(quant_vec_kernel<1>, dim3(M), dim3(256), 0, st, in, ldi, K, q, ldq, s);
    else if (nv <= 2) klaunch(quant_vec_kernel<2>, dim3(M), dim3(256), 0, st, in, ldi, K, q, ldq, s);
    else if (nv <= 4) klaunch(quant_vec_kernel<4>, dim3(M), dim3(256), 0, st, in, ldi, K, q, ldq, s);
    else if (nv <= 8) klaunch(quant_vec_kernel<8>, dim3(M), dim3(256), 0, st, in, ldi, K, q, ldq, s);
    else klaunch(quant_vec_kernel<16>, dim3(M), dim3(256), 0, st, in, ldi, K, q, ldq, s);
    return hipGetLastError();
  }
  klaunch(quant_kernel, dim3(M), dim3(256), 0, st, in, ldi, K, q, ldq, s);
  return hipGetLastError();
}

template <bool LN, bool QUANT>
static void launch_norm_vec(int nv, const float *x, int M, int E, const float *gamma, const float *beta, double eps,
                            float *h, int ldh, int8_t *q, int ldq, float *qs, hipStream_t st) {
  if (nv <= 1) klaunch((norm_vec_kernel<LN, QUANT, 1>), dim3(M), dim3(256), 0, st, x, E, gamma, beta, eps, h, ldh, q, ldq, qs);
  else if (nv <= 2) klaunch((norm_vec_kernel<LN, QUANT, 2>), dim3(M), dim3(256), 0, st, x, E, gamma, beta, eps, h, ldh, q, ldq, qs);
  else klaunch((norm_vec_kernel<LN, QUANT, 4>), dim3(M), dim3(256), 0, st, x, E, gamma, beta, eps, h, ldh, q, ldq, qs);
}

hipError_t norm_rows(const float *x, int M, int E, const float *gamma, const float *beta,
                     double eps, float *h, int ldh, int8_t *q, int ldq, float *qs,
                     hipStream_t st) {
  const bool vec = E % 4 == 0 && E <= 256 * 4 * 4 && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)gamma & 15u) == 0 &&
                   (!beta || ((uintptr_t)beta & 15u) == 0) &&
                   (q ? (ldq % 4 == 0 && ((uintptr_t)q & 3u) == 0) : (ldh % 4 == 0 && ((uintptr_t)h & 15u) == 0));
  if (vec) {
    const int nv = (E / 4 + 255) / 256;
    if (beta) {
      if (q) launch_norm_vec<true, true>(nv, x, M, E, gamma, beta, eps, h, ldh, q, ldq, qs, st);
      else launch_norm_vec<true, false>(nv, x, M, E, gamma, beta, eps, h, ldh, q, ldq, qs, st);
    } else {
      if (q) launch_norm_vec<false, true>(nv, x, M, E, gamma, beta, eps, h, ldh, q, ldq, qs, st);
      else launch_norm_vec<false, false>(nv, x, M, E, gamma, beta, eps, h, ldh, q, ldq, qs, st);
    }
    return hipGetLastError();
  }
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

// Reads weight matrices into the L2 of the XCDs that will use them: a
// prefill's matrix-core GEMMs wait on each stage's weight loads, and weights
// already in the XCD's L2 take a third off gate/up and down.  The GEMMs give
// XCD x a contiguous eighth of the weight rows (their tile order), so block b
// (on XCD b % 8) reads rows of the eighth b % 8.  The loads feed an xor that
// is stored only in the (practically never met) case that it equals a
// constant, so they cannot be dropped.
__global__ __launch_bounds__(256) void touch_kernel(TouchArgs a) {
  const int x = blockIdx.x & 7, sub = blockIdx.x >> 3, nsub = gridDim.x >> 3;
  unsigned acc = 0;
  for (int r = 0; r < a.n_ranges; r++) {
    const int rows8 = (a.rows[r] + 7) / 8;
    const int r0 = min(a.rows[r], x * rows8), r1 = min(a.rows[r], r0 + rows8);
    const uint4 *p = a.p[r] + (size_t)r0 * a.row16[r];
    const size_t n = (size_t)(r1 - r0) * a.row16[r], step = (size_t)nsub * 256;
    size_t i = (size_t)sub * 256 + threadIdx.x;
    for (; i + 3 * step < n; i += 4 * step) {
      const uint4 v0 = p[i], v1 = p[i + step], v2 = p[i + 2 * step], v3 = p[i + 3 * step];
      acc ^= v0.x ^ v1.y ^ v2.z ^ v3.w;
    }
    for (; i < n; i += step) acc ^= p[i].x;
  }
  if (acc == 0x9e3779b9u) *a.sink = acc;
}

hipError_t touch_ranges(const TouchArgs &a, int blocks, hipStream_t st) {
  if (a.n_ranges < 0 || a.n_ranges > kTouchRanges || !a.sink || blocks < 8 || blocks % 8) return hipErrorInvalidValue;
  klaunch(touch_kernel, dim3(blocks), dim3(256), 0, st, a);
  return hipGetLastError();
}

// After a chained greedy decode step (io: token, position, slot, tag, error,
// argmax id, ids written): the argmax id becomes the next step's token at the
// next position under the next tag, and is appended to out.
__global__ void step_advance_kernel(int *io, int *out, unsigned long long *stamps) {
  const int t = io[5];
  if (stamps) stamps[io[6] + 1] = __builtin_amdgcn_s_memrealtime();
  out[io[6]] = t;
  io[6] = io[6] + 1;
  io[0] = t;
  io[1] = io[1] + 1;
  io[3] = (int)((unsigned)io[3] + 1u);
}

// the constant 100 MHz clock into t[0]: the start of a run of chained steps
__global__ void chain_stamp_kernel(unsigned long long *t) { t[0] = __builtin_amdgcn_s_memrealtime(); }

hipError_t chain_stamp(unsigned long long *t, hipStream_t st) {
  klaunch(chain_stamp_kernel, dim3(1), dim3(1), 0, st, t);
  return hipGetLastError();
}

hipError_t step_advance(int *io, int *out, hipStream_t st, unsigned long long *stamps) {
  klaunch(step_advance_kernel, dim3(1), dim3(1), 0, st, io, out, stamps);
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

// ---------------------------------------------------------------------------
// Scores pass of a long decode context.  Block (chunk c of kScChunk
// positions, KV group g, token m); thread t scores relative position
// kScChunk * c + t for every query head of the group, each score a
// sequential fp32 dot over head_dim (rounded products, added in order) scaled
// in double -- attn_decode_block's arithmetic -- with the K row read once for
// all the group's heads.  FUSED: q and the new k are rotated here (RoPE in
// double, the body's formula), the new k and v rounded to fp16; the block
// holding the token's position appends them to the cache and scores that
// position from the rounded k.  The softmax / sums pass (attn_kernel with
// SCORED) runs after it.
constexpr int kScMaxHeads = 16;  // query heads per KV group

// element tt of a head row after RoPE (rotate-half, the (cos, sin) pair of
// the rotated index), as attn_decode_block computes it
__device__ __forceinline__ float rope_elem(const float *row, int tt, int rot, const double2 *cs_pos) {
  if (tt >= 2 * rot) return row[tt];
  const int i0 = tt < rot ? tt : tt - rot;
  const float xa = row[i0], xb = row[i0 + rot];
  const double2 c2 = cs_pos[i0];
  const double cr = c2.x, sr = c2.y;
  if (tt < rot) {
    const double t1 = (double)xa * cr, t2 = (double)xb * sr;
    return (float)(t1 - t2);
  }
  const double t3 = (double)xa * sr, t4 = (double)xb * cr;
  return (float)(t3 + t4);
}

// kScThreads threads over a chunk of CH positions: NT / CH per position,
// thread t scoring position t % CH for the group's heads r = t / CH, +
// NT / CH, ...  At 256 positions (two threads per position, two waves per
// SIMD instead of one, each thread's sequential dots half as many) C5's
// scores pass went 10.3 -> 8.9 us per layer (three per position 9.4 us,
// chunks of 128 positions 9.6 us: 320 blocks, more than one round).  Small
// grids take chunks of 128 (four threads per position, twice the blocks):
// C4's 4 tokens x 2 KV groups at 2080 positions are 72 blocks of 256.
constexpr int kScThreads = 512;
template <int HD, bool FUSED, int CH>
__global__ __launch_bounds__(kScThreads) void attn_scores_kernel(AttnArgs a) {
  constexpr int NT = kScThreads;
  constexpr int kScChunk = CH;
  constexpr int CPR = HD / 8;         // 16-byte chunks per K row
  constexpr int KP = CPR + 1;         // LDS row pitch in chunks (odd: a thread's row reads spread over the banks)
  constexpr int RPL = NT / CPR;       // rows per load instruction over the block
  __shared__ __attribute__((aligned(16))) float qs[kScMaxHeads][HD];
  __shared__ __attribute__((aligned(16))) uint16_t kn[HD];
  __shared__ v4u ktile[kScChunk * KP];
  const int c = blockIdx.x, g = blockIdx.y, m = blockIdx.z, t = threadIdx.x;
  const int R = a.H / a.KVH;
  const int pos = ld_uniform(a.pos + m), slot = ld_uniform(a.slot + m);
  int lo = 0;
  if (a.window > 0) {
    lo = pos - a.window + 1;
    if (lo < 0) lo = 0;
  }
  const int n = pos + 1 - lo, i0 = kScChunk * c;
  if (i0 >= n) return;  // uniform
  const int ncache = FUSED ? n - 1 : n;  // rows read from the cache
  const size_t cbase = ((size_t)slot * a.C) * a.kv + (size_t)g * HD;
  const uint16_t *K = a.kc + cbase + (size_t)lo * a.kv;
  // the chunk's K rows, coalesced (CPR lanes per row), clamped into the cache rows
  constexpr int KU = (kScChunk + RPL - 1) / RPL;  // rows per thread (the last ones guarded)
  v4u kr[KU];
#pragma unroll
  for (int u = 0; u < KU; u++) {
    const int r = min(RPL * u + t / CPR, kScChunk - 1), cc = t % CPR;
    const int i = min(i0 + r, ncache > 0 ? ncache - 1 : 0);
    kr[u] = *reinterpret_cast<const v4u *>(K + (size_t)i * a.kv + 8 * cc);
  }
  const int rot = (FUSED && a.cs) ? a.half : 0;
  const double2 *csp = rot ? a.cs + (size_t)pos * a.half : nullptr;
  for (int e = t; e < R * HD; e += NT) {
    const int r = e / HD, d = e - r * HD;
    const float *qrow = a.q + (size_t)m * a.ldq + (size_t)(g * R + r) * HD;
    qs[r][d] = rot ? rope_elem(qrow, d, rot, csp) : qrow[d];
  }
  if constexpr (FUSED) {
    if (t < HD) {
      const float *krow = a.k + (size_t)m * a.ldk + (size_t)g * HD;
      const float *vrow = a.v + (size_t)m * a.ldk + (size_t)g * HD;
      const uint16_t kh = f2h(rot ? rope_elem(krow, t, rot, csp) : krow[t]), vh = f2h(vrow[t]);
      kn[t] = kh;
      if (n - 1 < i0 + kScChunk) {  // this block holds the token's position: the append
        const size_t woff = cbase + (size_t)pos * a.kv + t;
        a.kc_w[woff] = kh;
        a.vc_w[woff] = vh;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < KU; u++) {
    const int r = RPL * u + t / CPR, cc = t % CPR;
    if (r < kScChunk) ktile[r * KP + cc] = kr[u];
  }
  __syncthreads();
  const int tp = t % kScChunk, i = i0 + tp;
  if (i >= n) return;
  // this thread's row: the own position (FUSED) takes the rounded new k
  const v4u *krow = (FUSED && i == n - 1) ? reinterpret_cast<const v4u *>(kn) : ktile + tp * KP;
  v4u kk[CPR];
#pragma unroll
  for (int cc = 0; cc < CPR; cc++) kk[cc] = krow[cc];
  float *dst = a.scores + ((size_t)m * a.H + (size_t)g * R) * a.sc_ld + i;
  for (int r = t / kScChunk; r < R; r += NT / kScChunk) {
    float s = 0.0f;
#pragma unroll
    for (int cc = 0; cc < CPR; cc++) {
      float qv[8];
#pragma unroll
      for (int j = 0; j < 8; j++) qv[j] = qs[r][8 * cc + j];
      mac8(s, qv, kk[cc]);
    }
    dst[(size_t)r * a.sc_ld] = (float)((double)s * a.inv_hd);
  }
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

template <int HD, int CH>
static void launch_attn_scores_ch(const AttnArgs &a, hipStream_t st) {
  const dim3 g1((a.max_npos + CH - 1) / CH, a.KVH, a.M);
  if (a.fuse_kv) klaunch((attn_scores_kernel<HD, true, CH>), g1, dim3(kScThreads), 0, st, a);
  else klaunch((attn_scores_kernel<HD, false, CH>), g1, dim3(kScThreads), 0, st, a);
}
template <int HD>
static void launch_attn_scores(const AttnArgs &a, hipStream_t st) {
  // chunks of 256 positions, or of 128 when that grid would fill half the CUs or less
  const long b256 = (long)((a.max_npos + 255) / 256) * a.KVH * a.M;
  if (b256 * 2 <= kStepBlocks) launch_attn_scores_ch<HD, 128>(a, st);
  else launch_attn_scores_ch<HD, 256>(a, st);
}

// the body on the scores pass's scores (the cache holds the new k / v)
template <int HD>
static void launch_attn_scored(AttnArgs a, hipStream_t st) {
  const int r = a.H / a.KVH;
  a.xcd_r = (a.KVH <= 8 && a.H % a.KVH == 0 && r > 1) ? r : 0;
  a.fuse_kv = 0;
  // one block per query head of 512 threads (two summing waves, six
  // product waves): 18.9 us per layer at C5's 1024-1290 positions against
  // 24.9 us with 256 threads (two product waves).  Element slices of head_dim
  // 128 (2 or 4 blocks per head) took 29 and 43 us against 24 us, their extra
  // blocks running in more rounds; one block per (token, KV group, 16
  // elements) for all six heads of a group, V read once per group, took 25
  // us: each block recomputes the six heads' softmax (six times the
  // exponentials of a per-head block).  head_dim 64 keeps the fused
  // kernel's four element slices of 16 (512 threads each).
  constexpr int NS = HD == 64 ? 4 : 1;
  const dim3 grid((a.xcd_r ? 8 * r : a.H) * NS, a.M);
  klaunch((attn_kernel<HD, false, NS, true>), grid, dim3(attn_threads(HD, NS, true)),
          attention_lds_bytes(a.max_npos, HD, a.vtile), st, a);
}

// the scores pass applies: a workspace, a long context, head_dim 128 (the
// one-block-per-head body, which re-scores nothing) or 64 (its four element
// slices, which otherwise each score every position again: C4's M = 4 steps
// at 2080 positions, 24.4 -> 5.3 + 17.2 us per layer), whole KV groups of at
// most kScMaxHeads heads.
bool attention_split_ok(const AttnArgs &a) {
  return a.scores && a.sc_ld >= a.max_npos && a.max_npos >= kAttnSplitMinPos && attn_vec(a.hd, a.kv) &&
         (a.hd == 128 || a.hd == 64) && a.H % a.KVH == 0 && a.H / a.KVH <= kScMaxHeads;
}

hipError_t attention(const AttnArgs &a, hipStream_t st) {
  if (a.vtile < 4 || (a.vtile & 3) || a.vtile > attention_max_vtile(a.hd, a.kv) || a.hd > 256)
    return hipErrorInvalidValue;
  const size_t lds = attention_lds_bytes(a.max_npos, a.hd, a.vtile);
  if (attention_split_ok(a)) {
    if (a.hd == 64) launch_attn_scores<64>(a, st);
    else launch_attn_scores<128>(a, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (a.hd == 64) launch_attn_scored<64>(a, st);
    else launch_attn_scored<128>(a, st);
    return hipGetLastError();
  }
  if (attn_vec(a.hd, a.kv) && a.hd == 64) launch_attn<64>(a, lds, st);
  else if (attn_vec(a.hd, a.kv) && a.hd == 128) launch_attn<128>(a, lds, st);
  else if (attn_vec(a.hd, a.kv) && a.hd == 32) launch_attn<32>(a, lds, st);
  else launch_attn<0>(a, lds, st);
  return hipGetLastError();
}

hipError_t attention_scores(const AttnArgs &a, hipStream_t st) {
  if (!attention_split_ok(a)) return hipErrorInvalidValue;
  if (a.hd == 64) launch_attn_scores<64>(a, st);
  else launch_attn_scores<128>(a, st);
  return hipGetLastError();
}

hipError_t attention_after_scores(const AttnArgs &a, hipStream_t st) {
  if (!attention_split_ok(a) || a.vtile < 4 || (a.vtile & 3) || a.vtile > attention_max_vtile(a.hd, a.kv))
    return hipErrorInvalidValue;
  if (a.hd == 64) launch_attn_scored<64>(a, st);
  else launch_attn_scored<128>(a, st);
  return hipGetLastError();
}

hipError_t argmax_finalize(const unsigned long long *cand, int ncand, const float *logits, int ldl, int rows,
                           int *out, hipStream_t st, int *chain_io, int *chain_out,
                           unsigned long long *chain_t) {
  if (chain_io && (rows != 1 || !chain_out)) return hipErrorInvalidValue;
  klaunch(argmax_finalize_kernel, dim3(rows), dim3(256), 0, st, cand, ncand, logits, ldl, out, chain_io, chain_out,
          chain_io ? chain_t : nullptr);
  return hipGetLastError();
}

hipError_t argmax_rows(const float *logits, int rows, int V, int *out, hipStream_t st) {
  klaunch(argmax_kernel, dim3(rows), dim3(256), 0, st, logits, V, out);
  return hipGetLastError();
}

hipError_t argmax_chunks(const float *logits, int rows, int V, unsigned long long *cand, int cap, int *nc_out,
                         hipStream_t st) {
  // chunks of at least 2048 logits, at most cap per row
  int nc = (V + 2047) / 2048;
  if (nc > cap) nc = cap;
  if (nc < 1) return hipErrorInvalidValue;
  const int csz = (V + nc - 1) / nc;
  nc = (V + csz - 1) / csz;
  *nc_out = nc;
  klaunch(argmax_chunk_kernel, dim3(nc, rows), dim3(256), 0, st, logits, V, csz, cand);
  return hipGetLastError();
}

hipError_t argmax_rows_chunked(const float *logits, int rows, int V, unsigned long long *cand, int cap, int *out,
                               hipStream_t st) {
  int nc = 0;
  const hipError_t e = argmax_chunks(logits, rows, V, cand, cap, &nc, st);
  if (e != hipSuccess) return e;
  return argmax_finalize(cand, nc, logits, V, rows, out, st);
}

}  // namespace ec
