// Decode / skinny GEMV kernels for gfx950 with fused prologues and epilogues.
//
//   out[m][n] = epilogue( dot( act[m][:], W[n][:] ) )       m < M (tiles of MT rows)
//
// Weights keep the reference layout [N][K] row-major (int8, fp16 or bf16).
// A row is read by LPR lanes of a wave, CPL 16-byte non-temporal loads per
// lane per pass: one wave instruction covers 64/LPR rows x LPR*16 contiguous
// bytes.  A block of 256 threads (4 waves) owns a "row group" of 4*64/LPR
// output rows and walks the row groups grid-stride.  For SwiGLU a lane loads
// the matching gate and up rows, so both halves meet in the same lane.
//
// Load order is what makes the kernel fast at decode sizes: the activation
// row (and the norm weights) are loaded first, then the first row group's
// weights, scales, bias and residual, all unconditionally (indices clamped
// into range, results masked), so the hardware's in-order load counter lets
// the prologue wait for the activation alone while the weight stream is in
// flight.
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
#include "ec_quant.h"

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

// Row shapes of the fused kernel: (lanes per row, 16-byte chunks per lane).
// GS_NARROW: 4 rows per wave, rows up to 64 (int8) / 128 (16-bit) chunks;
// GS_MID: one row per wave, up to 320 chunks in one pass; GS_WIDE: one row
// per wave, 640 chunks per pass, any K.
enum { GS_NARROW = 0, GS_MID = 1, GS_WIDE = 2 };
template <int WT, int SHAPE>
struct GemvShape {
  static constexpr int LPR = SHAPE == GS_NARROW ? 16 : 64;
  static constexpr int CPL = SHAPE == GS_NARROW ? (WT == WT_I8 ? 4 : 8) : SHAPE == GS_MID ? 5 : 10;
};

// fp32 activation strips of 1024 (float4 per thread) kept in registers by the
// prologue: the quantizing prologue holds rows up to 10240, the norms up to
// 4096 (gemv_vector_ok enforces both).
template <int PRO>
struct ProStrips {
  static constexpr int NS = PRO == PRO_QUANT ? 10 : (PRO == PRO_RMS || PRO == PRO_LN) ? 4 : 0;
};

// Sum of the LPR lanes of each row group (LPR in {16, 64}); the result is
// valid in every lane of the group.  Integer sums are exact; fp32 sums use a
// fixed tree.
template <int LPR, typename T>
__device__ __forceinline__ T group_sum(T v) {
  v = v + dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v = v + dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v = v + dpp_mov<0x141>(v);  // row_half_mirror
  v = v + dpp_mov<0x140>(v);  // row_mirror
  if constexpr (LPR == 64) {
    const T r0 = readlane(v, 0), r1 = readlane(v, 16), r2 = readlane(v, 32), r3 = readlane(v, 48);
    v = (r0 + r1) + (r2 + r3);
  }
  return v;
}

template <int WT, int SHAPE, int MT, int EPI, int PRO, int WL>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  constexpr bool Q8 = WT == WT_I8;
  constexpr int LPR = GemvShape<WT, SHAPE>::LPR, CPL = GemvShape<WT, SHAPE>::CPL;
  constexpr int RPW = kWave / LPR;
  constexpr bool SWI = EPI == EPI_SWIGLU;
  constexpr bool RES = EPI == EPI_RESID || EPI == EPI_BIAS_RESID;
  constexpr int RPB = 4 * RPW;
  constexpr int CHB = Q8 ? 16 : 8;  // elements per 16-byte chunk
  constexpr bool LDS_ACT = PRO != PRO_F32;
  constexpr bool NORM = PRO == PRO_RMS || PRO == PRO_LN;
  constexpr int NS = ProStrips<PRO>::NS;
  static_assert(!WL || (MT <= 4 && (PRO == PRO_QUANT || NORM)), "wave-local prologue: up to 4 rows, fp32 input");
  static_assert(WL != 2 || (MT > 1 && PRO == PRO_QUANT), "wide wave-local prologue: quantized M tiles only");
  // WL with MT > 1: wave w computes row min(w, mc - 1) of the tile into LDS
  // slot w, and one block barrier precedes the dot
  constexpr bool WL1 = WL != 0 && MT == 1;

  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  __shared__ double redd[2][4];
  __shared__ float redf[4];
  __shared__ unsigned long long keyred[4][MT];
  __shared__ uint64_t etab[SWI ? 4 * 32 : 1];  // expf table of the SiLU, one copy per wave

  // every kernel argument into registers here: one wait on the argument
  // loads instead of one per first use
  asm volatile("" ::"s"(a.A), "s"(a.W), "s"(a.W2), "s"(a.ws), "s"(a.ws2), "s"(a.bias), "s"(a.out));
  asm volatile("" ::"s"(a.gamma), "s"(a.beta), "s"(a.as), "s"(a.cand), "s"(a.lda), "s"(a.ldo), "s"(a.M),
               "s"(a.K), "s"(a.N));

  const int t = threadIdx.x;
  uint64_t et = 0;
  if constexpr (SWI) et = ec_exp2_32[t & 31];
  const int lane = t & 63, wave = t >> 6;
  const int grp = lane / LPR, sub = lane % LPR;
  const int rib = wave * RPW + grp;
  const int K = a.K;
  const int Kp = (K + CHB - 1) / CHB * CHB;
  const int nch = K / CHB;
  const int m0 = blockIdx.y * MT;
  const int mc = min(MT, a.M - m0);
  const int ngroups = (a.N + RPB - 1) / RPB;

  typedef typename std::conditional<Q8, v4i, v4u>::type vec_t;
  constexpr size_t WB = Q8 ? 1 : 2;

  // Prologue layout: thread t owns activation elements 4t + 1024j; the block
  // reduces through LDS into one shared copy of the quantized / normalized row.
  const int nstrip = (K + 1023) >> 10;

  // ---- 1. activation row 0 of the tile (+ norm weights) ----
  float4 xv[NS > 0 ? NS : 1], gv[NORM ? NS : 1], bv[PRO == PRO_LN ? NS : 1];
  auto load_act = [&](int m) {
    const float *row = reinterpret_cast<const float *>(a.A) + (size_t)(m0 + m) * a.lda;
#pragma unroll
    for (int j = 0; j < NS; j++) {
      if (j < nstrip) {
        const int i = min(4 * t + 1024 * j, K - 4);
        xv[j] = *reinterpret_cast<const float4 *>(row + i);
        if constexpr (NORM) {
          if (m == 0) {
            gv[j] = *reinterpret_cast<const float4 *>(a.gamma + i);
            if constexpr (PRO == PRO_LN) bv[j] = *reinterpret_cast<const float4 *>(a.beta + i);
          }
        }
      }
    }
  };
  // WL: every wave holds a whole row, lane l elements 4l + 256j, and
  // computes the prologue alone: for one row (WL1) no block barrier, each
  // wave writing its own copy of the quantized / normalized row to LDS; for
  // an M tile of up to 4 rows, wave w takes row w.  WL 1: rows up to 1024;
  // WL 2: quantized rows of an M tile up to 5120 (all rows' loads in flight
  // at once and one block barrier, instead of one row after another through
  // block reductions).  The loads are unconditional (clamped into the row),
  // so the prologue's wait still leaves the weight loads in flight.
  constexpr int WLS = WL == 2 ? 20 : WL ? 4 : 1;
  float4 xw[WLS], gw[WL && NORM ? WLS : 1], bw[WL && PRO == PRO_LN ? WLS : 1];
  if constexpr (WL) {
    const int wr = MT > 1 ? min(wave, mc - 1) : 0;
    const float *row = reinterpret_cast<const float *>(a.A) + (size_t)(m0 + wr) * a.lda;
#pragma unroll
    for (int j = 0; j < WLS; j++) {
      const int i = min(4 * lane + 256 * j, K - 4);
      xw[j] = *reinterpret_cast<const float4 *>(row + i);
      if constexpr (NORM) gw[j] = *reinterpret_cast<const float4 *>(a.gamma + i);
      if constexpr (PRO == PRO_LN) bw[j] = *reinterpret_cast<const float4 *>(a.beta + i);
    }
    // the SiLU table and the row ahead of the weights: the stores of the
    // table would otherwise wait for the whole weight stream
    __builtin_amdgcn_sched_barrier(0);
  } else if constexpr (NS > 0) {
    load_act(0);
  }

  // ---- 2. first row group: weights, scales, bias, residual ----
  // All unconditional: absent scales / bias read a valid dummy address and
  // are replaced afterwards, so the number of loads after the activation is
  // the same on every path and the prologue waits for the activation only.
  const vec_t *Wv = reinterpret_cast<const vec_t *>(a.W);
  const vec_t *W2v = reinterpret_cast<const vec_t *>(a.W2);
  vec_t w[CPL], w2[SWI ? CPL : 1];
  auto load_w = [&](int rg, int kb) {
    const int n = min(rg * RPB + rib, a.N - 1);
    const size_t base = (size_t)n * K * WB / 16;
#pragma unroll
    for (int c = 0; c < CPL; c++) {
      const int ch = min(kb + sub + c * LPR, nch - 1);
      w[c] = __builtin_nontemporal_load(Wv + base + ch);
      if constexpr (SWI) w2[c] = __builtin_nontemporal_load(W2v + base + ch);
    }
  };
  const float *dummy = reinterpret_cast<const float *>(a.W);
  const float *wsp = a.ws ? a.ws : dummy, *ws2p = a.ws2 ? a.ws2 : dummy, *bp = a.bias ? a.bias : dummy;
  float bs = 1.0f, bs2 = 1.0f, bia = 0.0f, res[RES ? MT : 1];
  auto load_meta = [&](int rg) {
    const int n = min(rg * RPB + rib, a.N - 1);
    if constexpr (Q8) {
      bs = wsp[a.ws ? n : 0];
      if constexpr (SWI) bs2 = ws2p[a.ws2 ? n : 0];
    }
    bia = bp[a.bias ? n : 0];
    if constexpr (RES) {
#pragma unroll
      for (int m = 0; m < MT; m++) res[m] = a.out[(size_t)(m0 + min(m, mc - 1)) * a.ldo + n];
    }
  };
  auto fix_meta = [&](float &cbs, float &cbs2, float &cbia) {
    if (!a.ws) cbs = 1.0f;
    if (!a.ws2) cbs2 = 1.0f;
    if (!a.bias) cbia = 0.0f;
  };
  int rg = blockIdx.x;
  load_w(rg, 0);
  load_meta(rg);
  if constexpr (WL) __builtin_amdgcn_sched_barrier(0);  // every weight load out before the first wait

  // ---- 3. prologue: activation rows of this M tile into LDS ----
  // unconditional (lanes 32..63 repeat lanes 0..31): a conditional store
  // lets the compiler sink the table load behind the weight loads
  if constexpr (SWI) etab[32 * wave + (lane & 31)] = et;
  int8_t *xq = reinterpret_cast<int8_t *>(lds);
  float *xf = reinterpret_cast<float *>(lds);
  float *xs = reinterpret_cast<float *>(lds + (size_t)(WL ? 4 : MT) * Kp);  // int8 path only
  float xsw = 1.0f;  // WL: the row's scale (int8 path)
  if constexpr (WL) {
#pragma unroll
    for (int j = 0; j < WLS; j++) {
      if (4 * lane + 256 * j >= K) xw[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if constexpr (NORM) {
      double s1 = 0.0;
#pragma unroll
      for (int j = 0; j < WLS; j++) {
        const double d0 = xw[j].x, d1 = xw[j].y, d2 = xw[j].z, d3 = xw[j].w;
        if constexpr (PRO == PRO_LN) s1 += ((d0 + d1) + d2) + d3;
        else s1 += ((d0 * d0 + d1 * d1) + d2 * d2) + d3 * d3;
      }
      s1 = wave_sum_dpp(s1);
      double mean = 0.0, rstd;
      if constexpr (PRO == PRO_LN) {
        mean = s1 / K;
        double s2 = 0.0;
#pragma unroll
        for (int j = 0; j < WLS; j++) {
          if (4 * lane + 256 * j < K) {
            const double d0 = xw[j].x - mean, d1 = xw[j].y - mean, d2 = xw[j].z - mean, d3 = xw[j].w - mean;
            s2 += ((d0 * d0 + d1 * d1) + d2 * d2) + d3 * d3;
          }
        }
        rstd = 1.0 / sqrt(wave_sum_dpp(s2) / K + a.eps);
      } else {
        rstd = 1.0 / sqrt(s1 / K + a.eps);
      }
      auto nrm = [&](float x, float g, float b) -> float {
        if constexpr (PRO == PRO_RMS) {
          x = (float)((double)x * rstd);
          return x * g;
        } else {
          x = (float)(((double)x - mean) * rstd);
          x = x * g;
          return x + b;
        }
      };
#pragma unroll
      for (int j = 0; j < WLS; j++) {
        const float4 b = PRO == PRO_LN ? bw[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        xw[j].x = nrm(xw[j].x, gw[j].x, b.x);
        xw[j].y = nrm(xw[j].y, gw[j].y, b.y);
        xw[j].z = nrm(xw[j].z, gw[j].z, b.z);
        xw[j].w = nrm(xw[j].w, gw[j].w, b.w);
        if (4 * lane + 256 * j >= K) xw[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    if constexpr (Q8) {
      float mx = 0.0f;
#pragma unroll
      for (int j = 0; j < WLS; j++) {
        mx = fmaxf(mx, fabsf(xw[j].x));
        mx = fmaxf(mx, fabsf(xw[j].y));
        mx = fmaxf(mx, fabsf(xw[j].z));
        mx = fmaxf(mx, fabsf(xw[j].w));
      }
      mx = wave_max_dpp(mx);
      const float sc = quant_scale(mx);
      int8_t *q = xq + (size_t)wave * Kp;
      const bool fast = ec_quant_rcp_ok(sc);
      const float rcp = 1.0f / sc;
#pragma unroll
      for (int j = 0; j < WLS; j++) {
        const int i = 4 * lane + 256 * j;
        if (i < K) {
          uint32_t b0, b1, b2, b3;
          if (fast) {
            b0 = (uint8_t)ec_quant1_rcp(xw[j].x, sc, rcp);
            b1 = (uint8_t)ec_quant1_rcp(xw[j].y, sc, rcp);
            b2 = (uint8_t)ec_quant1_rcp(xw[j].z, sc, rcp);
            b3 = (uint8_t)ec_quant1_rcp(xw[j].w, sc, rcp);
          } else {
            b0 = (uint8_t)quant1(xw[j].x, sc);
            b1 = (uint8_t)quant1(xw[j].y, sc);
            b2 = (uint8_t)quant1(xw[j].z, sc);
            b3 = (uint8_t)quant1(xw[j].w, sc);
          }
          *reinterpret_cast<uint32_t *>(q + i) = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
        }
      }
      xsw = sc;
      if constexpr (MT > 1) {
        if (lane == 0) xs[wave] = sc;
      }
    } else {
      float *f = xf + (size_t)wave * Kp;
#pragma unroll
      for (int j = 0; j < WLS; j++) {
        const int i = 4 * lane + 256 * j;
        if (i < K) *reinterpret_cast<float4 *>(f + i) = xw[j];
      }
    }
  } else if constexpr (PRO == PRO_I8) {
    for (int m = 0; m < mc; m++) {
      const int8_t *src = reinterpret_cast<const int8_t *>(a.A) + (size_t)(m0 + m) * a.lda;
      for (int i = t * 16; i < K; i += 256 * 16)
        *reinterpret_cast<v4i *>(xq + (size_t)m * Kp + i) = *reinterpret_cast<const v4i *>(src + i);
      if (t == 0) xs[m] = a.as[m0 + m];
    }
  } else if constexpr (NS > 0) {
    for (int m = 0; m < mc; m++) {
      if (m) load_act(m);
      // lanes past the end of the row hold a clamped copy: zero them
#pragma unroll
      for (int j = 0; j < NS; j++) {
        if (j < nstrip && 4 * t + 1024 * j >= K) xv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
      double mean = 0.0, rstd = 1.0;
      if constexpr (NORM) {
        double s1 = 0.0;
#pragma unroll
        for (int j = 0; j < NS; j++) {
          if (j < nstrip) {
            const double d0 = xv[j].x, d1 = xv[j].y, d2 = xv[j].z, d3 = xv[j].w;
            if constexpr (PRO == PRO_LN) s1 += ((d0 + d1) + d2) + d3;
            else s1 += ((d0 * d0 + d1 * d1) + d2 * d2) + d3 * d3;
          }
        }
        s1 = block_sum256_1b(s1, redd[0]);
        if constexpr (PRO == PRO_LN) {
          mean = s1 / K;
          double s2 = 0.0;
#pragma unroll
          for (int j = 0; j < NS; j++) {
            if (j < nstrip && 4 * t + 1024 * j < K) {
              const double d0 = xv[j].x - mean, d1 = xv[j].y - mean, d2 = xv[j].z - mean, d3 = xv[j].w - mean;
              s2 += ((d0 * d0 + d1 * d1) + d2 * d2) + d3 * d3;
            }
          }
          const double var = block_sum256_1b(s2, redd[1]) / K;
          rstd = 1.0 / sqrt(var + a.eps);
        } else {
          rstd = 1.0 / sqrt(s1 / K + a.eps);
        }
        auto nrm = [&](float x, float g, float b) -> float {
          if constexpr (PRO == PRO_RMS) {
            x = (float)((double)x * rstd);
            return x * g;
          } else {
            x = (float)(((double)x - mean) * rstd);
            x = x * g;
            return x + b;
          }
        };
#pragma unroll
        for (int j = 0; j < NS; j++) {
          if (j < nstrip) {
            const float4 b = PRO == PRO_LN ? bv[j] : make_float4(0.f, 0.f, 0.f, 0.f);
            xv[j].x = nrm(xv[j].x, gv[j].x, b.x);
            xv[j].y = nrm(xv[j].y, gv[j].y, b.y);
            xv[j].z = nrm(xv[j].z, gv[j].z, b.z);
            xv[j].w = nrm(xv[j].w, gv[j].w, b.w);
            if (4 * t + 1024 * j >= K) xv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
      }
      if constexpr (Q8) {
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < NS; j++) {
          if (j < nstrip) {
            mx = fmaxf(mx, fabsf(xv[j].x));
            mx = fmaxf(mx, fabsf(xv[j].y));
            mx = fmaxf(mx, fabsf(xv[j].z));
            mx = fmaxf(mx, fabsf(xv[j].w));
          }
        }
        mx = block_max256_1b(mx, redf);
        const float sc = quant_scale(mx);
        int8_t *q = xq + (size_t)m * Kp;
        // the reference's rint(a / s) codes, from one reciprocal per row
        // (ec_quant.h) where the scale allows it
        const bool fast = ec_quant_rcp_ok(sc);
        const float rcp = 1.0f / sc;
#pragma unroll
        for (int j = 0; j < NS; j++) {
          const int i = 4 * t + 1024 * j;
          if (j < nstrip && i < Kp) {
            uint32_t b0, b1, b2, b3;
            if (fast) {
              b0 = (uint8_t)ec_quant1_rcp(xv[j].x, sc, rcp);
              b1 = (uint8_t)ec_quant1_rcp(xv[j].y, sc, rcp);
              b2 = (uint8_t)ec_quant1_rcp(xv[j].z, sc, rcp);
              b3 = (uint8_t)ec_quant1_rcp(xv[j].w, sc, rcp);
            } else {
              b0 = (uint8_t)quant1(xv[j].x, sc);
              b1 = (uint8_t)quant1(xv[j].y, sc);
              b2 = (uint8_t)quant1(xv[j].z, sc);
              b3 = (uint8_t)quant1(xv[j].w, sc);
            }
            *reinterpret_cast<uint32_t *>(q + i) = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
          }
        }
        if (t == 0) xs[m] = sc;
      } else {
        float *f = xf + (size_t)m * Kp;
#pragma unroll
        for (int j = 0; j < NS; j++) {
          const int i = 4 * t + 1024 * j;
          if (j < nstrip && i < Kp) *reinterpret_cast<float4 *>(f + i) = xv[j];
        }
      }
      // the two reductions of the next row reuse redd/redf: separate them
      if (m + 1 < mc) __syncthreads();
    }
  }
  if constexpr (!WL1) __syncthreads();

  unsigned long long best[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) best[m] = 0ull;

  for (; rg < ngroups; rg += gridDim.x) {
    const int n = rg * RPB + rib;
    const bool valid = n < a.N;
    typedef typename std::conditional<Q8, int, float>::type acc_t;
    acc_t acc[MT], acc2[SWI ? MT : 1];
#pragma unroll
    for (int m = 0; m < MT; m++) {
      acc[m] = 0;
      if constexpr (SWI) acc2[m] = 0;
    }
    for (int kb = 0; kb < nch; kb += LPR * CPL) {
      if (kb) load_w(rg, kb);
#pragma unroll
      for (int c = 0; c < CPL; c++) {
        const int ch = kb + sub + c * LPR;
        if (ch >= nch) continue;
        if constexpr (Q8) {
#pragma unroll
          for (int m = 0; m < MT; m++) {
            if (m < mc) {
              const v4i x = *reinterpret_cast<const v4i *>(xq + (size_t)(WL1 ? wave : m) * Kp + (size_t)ch * 16);
              int s = acc[m];
              s = __builtin_amdgcn_sdot4(x.x, w[c].x, s, false);
              s = __builtin_amdgcn_sdot4(x.y, w[c].y, s, false);
              s = __builtin_amdgcn_sdot4(x.z, w[c].z, s, false);
              s = __builtin_amdgcn_sdot4(x.w, w[c].w, s, false);
              acc[m] = s;
              if constexpr (SWI) {
                int u = acc2[m];
                u = __builtin_amdgcn_sdot4(x.x, w2[c].x, u, false);
                u = __builtin_amdgcn_sdot4(x.y, w2[c].y, u, false);
                u = __builtin_amdgcn_sdot4(x.z, w2[c].z, u, false);
                u = __builtin_amdgcn_sdot4(x.w, w2[c].w, u, false);
                acc2[m] = u;
              }
            }
          }
        } else {
          float wf[8], wf2[SWI ? 8 : 1];
          {
            const uint32_t wv[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
              wf[2 * j] = w2f<WT == WT_BF16>((uint16_t)(wv[j] & 0xffffu));
              wf[2 * j + 1] = w2f<WT == WT_BF16>((uint16_t)(wv[j] >> 16));
            }
          }
          if constexpr (SWI) {
            const uint32_t wv[4] = {w2[c].x, w2[c].y, w2[c].z, w2[c].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
              wf2[2 * j] = w2f<WT == WT_BF16>((uint16_t)(wv[j] & 0xffffu));
              wf2[2 * j + 1] = w2f<WT == WT_BF16>((uint16_t)(wv[j] >> 16));
            }
          }
#pragma unroll
          for (int m = 0; m < MT; m++) {
            if (m < mc) {
              const float4 *xp =
                  LDS_ACT ? reinterpret_cast<const float4 *>(xf + (size_t)(WL1 ? wave : m) * Kp + (size_t)ch * 8)
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
              if constexpr (SWI) {
                float u = acc2[m];
                u = __builtin_fmaf(x0.x, wf2[0], u);
                u = __builtin_fmaf(x0.y, wf2[1], u);
                u = __builtin_fmaf(x0.z, wf2[2], u);
                u = __builtin_fmaf(x0.w, wf2[3], u);
                u = __builtin_fmaf(x1.x, wf2[4], u);
                u = __builtin_fmaf(x1.y, wf2[5], u);
                u = __builtin_fmaf(x1.z, wf2[6], u);
                u = __builtin_fmaf(x1.w, wf2[7], u);
                acc2[m] = u;
              }
            }
          }
        }
      }
    }
    // this group's scales/bias/residual; then prefetch the next group
    float cbs = bs, cbs2 = bs2, cbia = bia;
    fix_meta(cbs, cbs2, cbia);
    float cres[RES ? MT : 1];
    if constexpr (RES) {
#pragma unroll
      for (int m = 0; m < MT; m++) cres[m] = res[m];
    }
    if (rg + (int)gridDim.x < ngroups) {
      load_w(rg + gridDim.x, 0);
      load_meta(rg + gridDim.x);
    }
#pragma unroll
    for (int m = 0; m < MT; m++) {
      acc[m] = group_sum<LPR>(acc[m]);
      if constexpr (SWI) acc2[m] = group_sum<LPR>(acc2[m]);
    }

    // ---- epilogue ----
    if (sub == 0 && valid) {
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (m < mc) {
          float v;
          if constexpr (Q8) {
            v = i8_epilogue((int)acc[m], WL1 ? xsw : xs[m], cbs, SWI ? 0.0f : cbia);
          } else {
            v = (float)acc[m];
          }
          float *o = a.out + (size_t)(m0 + m) * a.ldo + n;
          if constexpr (SWI) {
            const float u = Q8 ? i8_epilogue((int)acc2[m], WL1 ? xsw : xs[m], cbs2, 0.0f) : (float)acc2[m];
            v = silu(v, etab + 32 * wave) * u;
          } else {
            if constexpr (!Q8 && (EPI == EPI_BIAS || EPI == EPI_BIAS_RESID || EPI == EPI_BIAS_GELU)) v = v + cbia;
            if constexpr (RES) v = cres[m] + v;
            if constexpr (EPI == EPI_GELU || EPI == EPI_BIAS_GELU) v = gelu_new(v);
          }
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

  if constexpr (EPI == EPI_STORE) {
    if (a.cand) {  // one argmax candidate per (row, block)
#pragma unroll
      for (int m = 0; m < MT; m++) {
        const unsigned long long b = wave_max_u64(best[m]);
        if (lane == 0) keyred[wave][m] = b;
      }
      __syncthreads();
      if (t < MT && t < mc) {
        unsigned long long b = keyred[0][t];
        for (int i = 1; i < 4; i++) b = keyred[i][t] > b ? keyred[i][t] : b;
        a.cand[(size_t)(m0 + t) * gridDim.x + blockIdx.x] = b;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host-side launch helpers (instantiated per weight type in gemv_*.hip)
// ---------------------------------------------------------------------------

template <int WT, int SHAPE, int MT, int EPI, int PRO, int WL = 0>
hipError_t gemv_launch(const GemvArgs &a, hipStream_t s) {
  constexpr int RPB = 4 * (kWave / GemvShape<WT, SHAPE>::LPR);
  const int ngroups = (a.N + RPB - 1) / RPB;
  const int cap = gemv_max_blocks();
  const int gx = ngroups < cap ? ngroups : cap;
  dim3 grid(gx, (a.M + MT - 1) / MT);
  const size_t lds = gemv_lds_bytes(WT, PRO, MT, a.K);
  klaunch((gemv_kernel<WT, SHAPE, MT, EPI, PRO, WL>), grid, dim3(256), lds, s, a);
  return hipGetLastError();
}

// wave-local prologue of an M tile: rows up to 1024, or quantized rows up
// to 5120 (the wide form)
template <int WT, int SHAPE, int MT, int EPI, int PRO>
hipError_t gemv_wave_launch(const GemvArgs &a, hipStream_t s) {
  if constexpr (PRO == PRO_QUANT)
    if (a.K > 1024) return gemv_launch<WT, SHAPE, MT, EPI, PRO, 2>(a, s);
  return gemv_launch<WT, SHAPE, MT, EPI, PRO, 1>(a, s);
}

template <int WT, int EPI, int PRO>
hipError_t gemv_launch_shape(const GemvArgs &a, hipStream_t s) {
  const int shape = gemv_pick_shape(WT, a.K);
  const int mt = gemv_pick_mt(a.M);
#define EC_MT(SH)                                                   \
  switch (mt) {                                                     \
  case 1:                                                           \
    if constexpr (PRO == PRO_QUANT || PRO == PRO_RMS || PRO == PRO_LN) \
      if (gemv_wave_pro(PRO, 1, a.K)) return gemv_launch<WT, SH, 1, EPI, PRO, 1>(a, s);    \
    return gemv_launch<WT, SH, 1, EPI, PRO>(a, s);                  \
  case 2:                                                           \
    if constexpr (PRO == PRO_QUANT || PRO == PRO_RMS || PRO == PRO_LN) \
      if (gemv_wave_pro(PRO, 2, a.K)) return gemv_wave_launch<WT, SH, 2, EPI, PRO>(a, s);  \
    return gemv_launch<WT, SH, 2, EPI, PRO>(a, s);                  \
  case 4:                                                           \
    if constexpr (PRO == PRO_QUANT || PRO == PRO_RMS || PRO == PRO_LN) \
      if (gemv_wave_pro(PRO, 4, a.K)) return gemv_wave_launch<WT, SH, 4, EPI, PRO>(a, s);  \
    return gemv_launch<WT, SH, 4, EPI, PRO>(a, s);                  \
  default: return gemv_launch<WT, SH, 8, EPI, PRO>(a, s);           \
  }
  if (shape == GS_NARROW) {
    EC_MT(GS_NARROW)
  } else if (shape == GS_MID) {
    EC_MT(GS_MID)
  } else {
    EC_MT(GS_WIDE)
  }
#undef EC_MT
}

}  // namespace ec
