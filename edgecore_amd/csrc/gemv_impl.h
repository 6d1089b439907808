// Decode / skinny GEMV kernels for gfx950 with fused prologues and epilogues.
//
//   out[m][n] = epilogue( dot( act[m][:], W[n][:] ) )       m < M (tiles of MT rows)
//
// Weights keep the reference layout [N][K] row-major (int8, fp16 or bf16).
// A row is read by LPR lanes of a wave with 16-byte non-temporal loads: one
// wave instruction covers 64/LPR rows x LPR*16 contiguous bytes.  A block of
// 256 threads (4 waves) owns a "row group" of 4*64/LPR output rows (2*64/LPR
// gate/up row pairs for SwiGLU) and walks the row groups grid-stride, so the
// activation prologue runs once per block, and the first row group's weights
// are already in flight (prefetched into registers) while it runs.
//
// Prologues (activation side; every block computes it, which at decode sizes
// is cheaper than another dependent launch):
//   PRO_I8    int8 rows + scales given (the gemm_int8 ABI)
//   PRO_F32   fp32 rows given, read from global (16-bit weights)
//   PRO_QUANT fp32 rows -> per-row int8 quantization (src/gpt2.c:446-461)
//   PRO_RMS   RMSNorm (src/gpt2.c:592-604), then quantize (int8) or keep fp32
//   PRO_LN    LayerNorm (src/gpt2.c:398-414), then quantize (int8) or keep fp32
// Norms accumulate in double like the reference; only the order of the double
// additions differs (a fixed tree).  int8 dots use v_dot4_i32_i8 into an exact
// int32, so the int8 epilogue bias + ((float)dot*as)*bs is bit-exact.  16-bit
// weights are widened to fp32 and accumulated with FMA.
#pragma once

#include "ec_device.h"
#include "ec_kernels.h"

#include <float.h>

namespace ec {

// orderable 64-bit argmax key: larger key = larger value, ties -> lower
// index; -0 folds onto +0 because the reference compares with '>'.
__device__ __forceinline__ unsigned long long amax_key(float v, int n) {
  v = v + 0.0f;
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)n);
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long w = __shfl_xor(v, o, kWave);
    v = w > v ? w : v;
  }
  return v;
}

constexpr int lpr_cpl(int lpr) { return lpr == 64 ? 10 : 4; }
constexpr int kStrips = 8;  // activation strips of 256 kept in registers by the prologue

// One fp32 activation row -> normalized (RMS/LN) and/or quantized into LDS.
// Thread t owns elements t + 256*j.  The first kStrips strips are kept in
// registers (every loop over them is unrolled, so they never spill to
// scratch); longer rows re-read the remaining strips from global memory.
template <int PRO, bool Q8>
__device__ __forceinline__ void prologue_row(const float *row, int K, int Kp, const float *gamma,
                                             const float *beta, double eps, const float *rowmax,
                                             int8_t *xq, float *xf, float *xs, double *redd,
                                             float *redf) {
  const int t = threadIdx.x;
  const int nstrip = (K + 255) >> 8;
  float v[kStrips];
#pragma unroll
  for (int j = 0; j < kStrips; j++) {
    const int i = t + 256 * j;
    v[j] = (i < K) ? row[i] : 0.0f;
  }
  double mean = 0.0, rstd = 1.0;
  if constexpr (PRO == PRO_RMS || PRO == PRO_LN) {
    double s1 = 0.0;
#pragma unroll
    for (int j = 0; j < kStrips; j++) {
      if (t + 256 * j < K) {
        const double d = (double)v[j];
        s1 += (PRO == PRO_LN) ? d : d * d;
      }
    }
    for (int j = kStrips; j < nstrip; j++) {
      const int i = t + 256 * j;
      if (i < K) {
        const double d = (double)row[i];
        s1 += (PRO == PRO_LN) ? d : d * d;
      }
    }
    s1 = block_sum256(s1, redd);
    if constexpr (PRO == PRO_LN) {
      mean = s1 / K;
      double s2 = 0.0;
#pragma unroll
      for (int j = 0; j < kStrips; j++) {
        if (t + 256 * j < K) {
          const double d = (double)v[j] - mean;
          s2 += d * d;
        }
      }
      for (int j = kStrips; j < nstrip; j++) {
        const int i = t + 256 * j;
        if (i < K) {
          const double d = (double)row[i] - mean;
          s2 += d * d;
        }
      }
      const double var = block_sum256(s2, redd) / K;
      rstd = 1.0 / sqrt(var + eps);
    } else {
      rstd = 1.0 / sqrt(s1 / K + eps);
    }
  }
  auto normed = [&](float x, int i) -> float {
    if constexpr (PRO == PRO_RMS) {
      x = (float)((double)x * rstd);
      x = x * gamma[i];
    } else if constexpr (PRO == PRO_LN) {
      x = (float)(((double)x - mean) * rstd);
      x = x * gamma[i];
      x = x + beta[i];
    }
    return x;
  };
  if constexpr (Q8) {
    float mx = 0.0f;
    if (PRO == PRO_QUANT && rowmax) {
      mx = *rowmax;  // max |row| published by the producing kernel
    } else {
#pragma unroll
      for (int j = 0; j < kStrips; j++) {
        const int i = t + 256 * j;
        if (i < K) {
          v[j] = normed(v[j], i);
          mx = fmaxf(mx, fabsf(v[j]));
        }
      }
      for (int j = kStrips; j < nstrip; j++) {
        const int i = t + 256 * j;
        if (i < K) mx = fmaxf(mx, fabsf(normed(row[i], i)));
      }
      mx = block_max256(mx, redf);
    }
    const float sc = quant_scale(mx);
#pragma unroll
    for (int j = 0; j < kStrips; j++) {
      const int i = t + 256 * j;
      if (i < Kp) xq[i] = (i < K) ? quant1(v[j], sc) : (int8_t)0;
    }
    for (int j = kStrips; j < (Kp + 255) / 256; j++) {
      const int i = t + 256 * j;
      if (i < Kp) xq[i] = (i < K) ? quant1(normed(row[i], i), sc) : (int8_t)0;
    }
    if (t == 0) *xs = sc;
  } else {
#pragma unroll
    for (int j = 0; j < kStrips; j++) {
      const int i = t + 256 * j;
      if (i < Kp) xf[i] = (i < K) ? normed(v[j], i) : 0.0f;
    }
    for (int j = kStrips; j < (Kp + 255) / 256; j++) {
      const int i = t + 256 * j;
      if (i < Kp) xf[i] = (i < K) ? normed(row[i], i) : 0.0f;
    }
  }
}

// WT: 0 int8, 1 fp16, 2 bf16
template <int WT, int LPR, int MT, int EPI, int PRO>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  constexpr bool Q8 = WT == 0;
  constexpr int CPL = lpr_cpl(LPR);
  constexpr int RPW = kWave / LPR;
  constexpr bool SWI = EPI == EPI_SWIGLU;
  constexpr int RPB = (SWI ? 2 : 4) * RPW;
  constexpr int CHB = Q8 ? 16 : 8;  // elements per 16-byte chunk
  constexpr bool LDS_ACT = PRO != PRO_F32;

  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  __shared__ double redd[4];
  __shared__ float redf[4];
  __shared__ float upx[SWI ? MT : 1][SWI ? 2 * RPW : 1];
  __shared__ unsigned long long keyred[4][MT];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = lane / LPR, sub = lane % LPR;
  const int part = SWI ? (wave >> 1) : 0;
  const int rib = SWI ? ((wave & 1) * RPW + grp) : (wave * RPW + grp);
  const int K = a.K;
  const int Kp = (K + CHB - 1) / CHB * CHB;
  const int nch = K / CHB;
  const int m0 = blockIdx.y * MT;
  const int mc = min(MT, a.M - m0);
  const int ngroups = (a.N + RPB - 1) / RPB;

  typedef typename std::conditional<Q8, v4i, v4u>::type vec_t;
  const void *Wsel = (SWI && part) ? a.W2 : a.W;
  vec_t w[CPL];
  auto load_w = [&](int rg, int kb) {
    const int n = rg * RPB + rib;
    const bool ok = n < a.N;
    const vec_t *wrow = reinterpret_cast<const vec_t *>(
        reinterpret_cast<const unsigned char *>(Wsel) + (size_t)n * K * (Q8 ? 1 : 2));
#pragma unroll
    for (int c = 0; c < CPL; c++) {
      const int ch = kb + sub + c * LPR;
      if (ok && ch < nch) w[c] = __builtin_nontemporal_load(wrow + ch);
    }
  };

  int rg = blockIdx.x;
  if (rg < ngroups) load_w(rg, 0);

  // ---- prologue: activation rows of this M tile into LDS ----
  int8_t *xq = reinterpret_cast<int8_t *>(lds);
  float *xf = reinterpret_cast<float *>(lds);
  float *xs = reinterpret_cast<float *>(lds + (size_t)MT * Kp);  // int8 path only
  if constexpr (PRO == PRO_I8) {
    for (int m = 0; m < mc; m++) {
      const int8_t *src = reinterpret_cast<const int8_t *>(a.A) + (size_t)(m0 + m) * a.lda;
      for (int i = threadIdx.x * 16; i < K; i += 256 * 16)
        *reinterpret_cast<v4i *>(xq + (size_t)m * Kp + i) = *reinterpret_cast<const v4i *>(src + i);
      if (threadIdx.x == 0) xs[m] = a.as[m0 + m];
    }
  } else if constexpr (PRO != PRO_F32) {
    for (int m = 0; m < mc; m++) {
      const float *row = reinterpret_cast<const float *>(a.A) + (size_t)(m0 + m) * a.lda;
      prologue_row<PRO, Q8>(row, K, Kp, a.gamma, a.beta, a.eps, a.in_max ? a.in_max + m0 + m : nullptr,
                            xq + (size_t)m * Kp, xf + (size_t)m * Kp, xs + m, redd, redf);
    }
  }
  __syncthreads();

  unsigned long long best[MT];
  float omax[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) {
    best[m] = 0ull;
    omax[m] = 0.0f;
  }

  for (; rg < ngroups; rg += gridDim.x) {
    const int n = rg * RPB + rib;
    const bool valid = n < a.N;
    typedef typename std::conditional<Q8, int, float>::type acc_t;
    acc_t acc[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) acc[m] = 0;
    for (int kb = 0; kb < nch; kb += LPR * CPL) {
      if (kb) load_w(rg, kb);
#pragma unroll
      for (int c = 0; c < CPL; c++) {
        const int ch = kb + sub + c * LPR;
        if (!valid || ch >= nch) continue;
        if constexpr (Q8) {
#pragma unroll
          for (int m = 0; m < MT; m++) {
            if (m < mc) {
              const v4i x = *reinterpret_cast<const v4i *>(xq + (size_t)m * Kp + (size_t)ch * 16);
              int s = acc[m];
              s = __builtin_amdgcn_sdot4(x.x, w[c].x, s, false);
              s = __builtin_amdgcn_sdot4(x.y, w[c].y, s, false);
              s = __builtin_amdgcn_sdot4(x.z, w[c].z, s, false);
              s = __builtin_amdgcn_sdot4(x.w, w[c].w, s, false);
              acc[m] = s;
            }
          }
        } else {
          float wf[8];
          const uint32_t wv[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
#pragma unroll
          for (int j = 0; j < 4; j++) {
            wf[2 * j] = w2f<WT == 2>((uint16_t)(wv[j] & 0xffffu));
            wf[2 * j + 1] = w2f<WT == 2>((uint16_t)(wv[j] >> 16));
          }
#pragma unroll
          for (int m = 0; m < MT; m++) {
            if (m < mc) {
              const float4 *xp =
                  LDS_ACT ? reinterpret_cast<const float4 *>(xf + (size_t)m * Kp + (size_t)ch * 8)
                          : reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(a.A) +
                                                             (size_t)(m0 + m) * a.lda + (size_t)ch * 8);
              const float4 x0 = xp[0], x1 = xp[1];
              float s = acc[m];
              s = __builtin_fmaf(x0.x, wf[0], s);
              s = __builtin_fmaf(x0.y, wf[1], s);
              s = __builtin_fmaf(x0.z, wf[2], s);
              s = __builtin_fmaf(x0.w, wf[3], s);
              s = __builtin_fmaf(x1.x, wf[4], s);
              s = __builtin_fmaf(x1.y, wf[5], s);
              s = __builtin_fmaf(x1.z, wf[6], s);
              s = __builtin_fmaf(x1.w, wf[7], s);
              acc[m] = s;
            }
          }
        }
      }
    }
    if (rg + (int)gridDim.x < ngroups) load_w(rg + gridDim.x, 0);  // prefetch the next group
#pragma unroll
    for (int m = 0; m < MT; m++) {
#pragma unroll
      for (int o = LPR / 2; o > 0; o >>= 1) acc[m] += __shfl_xor(acc[m], o, kWave);
    }

    // ---- epilogue ----
    float vals[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) {
      if constexpr (Q8) {
        const float as = xs[m];
        const float *wsc = (SWI && part) ? a.ws2 : a.ws;
        const float bs = (valid && wsc) ? wsc[n] : 1.0f;
        const float bv = (valid && a.bias && !SWI) ? a.bias[n] : 0.0f;
        vals[m] = i8_epilogue((int)acc[m], as, bs, bv);
      } else {
        vals[m] = (float)acc[m];
      }
    }
    if constexpr (SWI) {
      if (sub == 0 && valid && part == 1) {
#pragma unroll
        for (int m = 0; m < MT; m++)
          if (m < mc) upx[m][rib] = vals[m];
      }
      __syncthreads();
      if (sub == 0 && valid && part == 0) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
          if (m < mc) {
            const float r = silu(vals[m]) * upx[m][rib];
            a.out[(size_t)(m0 + m) * a.ldo + n] = r;
            omax[m] = fmaxf(omax[m], fabsf(r));
          }
        }
      }
      __syncthreads();
    } else {
      if (sub == 0 && valid) {
        const float bv = (!Q8 && a.bias) ? a.bias[n] : 0.0f;
#pragma unroll
        for (int m = 0; m < MT; m++) {
          if (m < mc) {
            float v = vals[m];
            float *o = a.out + (size_t)(m0 + m) * a.ldo + n;
            if constexpr (EPI == EPI_BIAS || EPI == EPI_BIAS_RESID || EPI == EPI_BIAS_GELU) v = v + bv;
            if constexpr (EPI == EPI_RESID || EPI == EPI_BIAS_RESID) v = *o + v;
            if constexpr (EPI == EPI_GELU || EPI == EPI_BIAS_GELU) v = gelu_new(v);
            *o = v;
            if constexpr (EPI == EPI_STORE) {
              if (a.cand && v == v) {
                const unsigned long long k = amax_key(v, n);
                best[m] = k > best[m] ? k : best[m];
              }
            }
          }
        }
      }
    }
  }

  if constexpr (SWI) {
    if (a.out_max) {  // row max |out| for the next linear's quantization
#pragma unroll
      for (int m = 0; m < MT; m++) {
        const float r = block_max256(omax[m], redf);
        if (threadIdx.x == 0 && m < mc)
          atomicMax(reinterpret_cast<unsigned int *>(a.out_max + m0 + m), __float_as_uint(r));
      }
    }
  }
  if constexpr (EPI == EPI_STORE) {
    if (a.cand) {  // one argmax candidate per (row, block)
#pragma unroll
      for (int m = 0; m < MT; m++) {
        const unsigned long long b = wave_max_u64(best[m]);
        if (lane == 0) keyred[wave][m] = b;
      }
      __syncthreads();
      if (threadIdx.x < MT && (int)threadIdx.x < mc) {
        const int m = threadIdx.x;
        unsigned long long b = keyred[0][m];
        for (int i = 1; i < 4; i++) b = keyred[i][m] > b ? keyred[i][m] : b;
        a.cand[(size_t)(m0 + m) * gridDim.x + blockIdx.x] = b;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host-side launch helpers (instantiated per weight type in gemv_*.hip)
// ---------------------------------------------------------------------------

template <int WT, int LPR, int MT, int EPI, int PRO>
hipError_t gemv_launch(const GemvArgs &a, hipStream_t s) {
  constexpr int RPW = kWave / LPR;
  constexpr int RPB = (EPI == EPI_SWIGLU ? 2 : 4) * RPW;
  const int ngroups = (a.N + RPB - 1) / RPB;
  const int gx = ngroups < gemv_max_blocks() ? ngroups : gemv_max_blocks();
  dim3 grid(gx, (a.M + MT - 1) / MT);
  const size_t lds = gemv_lds_bytes(WT, PRO, MT, a.K);
  hipLaunchKernelGGL((gemv_kernel<WT, LPR, MT, EPI, PRO>), grid, dim3(256), lds, s, a);
  return hipGetLastError();
}

template <int WT, int LPR, int EPI, int PRO>
hipError_t gemv_launch_mt(const GemvArgs &a, int mt, hipStream_t s) {
  switch (mt) {
  case 1: return gemv_launch<WT, LPR, 1, EPI, PRO>(a, s);
  case 2: return gemv_launch<WT, LPR, 2, EPI, PRO>(a, s);
  case 4: return gemv_launch<WT, LPR, 4, EPI, PRO>(a, s);
  default: return gemv_launch<WT, LPR, 8, EPI, PRO>(a, s);
  }
}

}  // namespace ec
