// The layer tail of a batched int8 Qwen2 decode (M <= kTailMaxM tokens, one
// slot each): everything of layer l after its attention, and the start of
// layer l + 1 before its attention, in one co-resident launch
// (src/gpt2.c:744-797 at M = batch, then :702-743 of the next layer):
//
//   o projection + residual     x_mid = x + o(quant(att))      :744-784
//   RMSNorm, gate/up, SiLU      h = silu(g(n)) * u(n)          :785-791
//   down projection + residual  x = x_mid + d(quant(h))        :792-796
//   next layer: RMSNorm, q|k|v  qkv = Wqkv n(x) + b            :702-713
//
// Why: the batched decode otherwise runs these as four GEMV launches per
// layer (q|k|v, o, gate/up, down) of 1-9 MB each, each starting from a cold
// weight stream behind a full kernel boundary; at C4's four tokens they took
// ~25 us per layer against ~10 us for the same phases inside the one-token
// persistent step.  The attention (two launches at long contexts) stays
// separate: this kernel runs between layer l's attention and layer l + 1's.
//
// Grid: kStepBlocks blocks of kStepThreads threads, all resident (a plain
// launch on an idle device, or a cooperative one).  Roles, by block index:
//
//   OD (E / 16 blocks, 16 rows each) -- o rows for every token (64 groups of
//      8 lanes: row r0 + g % 16, token g / 16), x_mid = x + o, publish
//      x_mid; then wait for the FFN rows' scales and codes, down rows (two
//      per wave, every token), x = x_mid + d: store x and publish.
//   G  (ceil(F / 64) blocks, 64 gate/up row pairs each) -- wait for x_mid,
//      RMSNorm + quantize (wave m: token m), gate and up rows for every
//      token, silu(g) * u; publish each token's maximum over the block's
//      values, wait for every block's, and quantize and publish the block's
//      values with the row scale (each FFN value is quantized once, by its
//      producer, instead of by every o/down block: that took 2.7 us there,
//      and codes cross the exchange in a quarter of the bytes).
//   Q  (ceil(NQ / 16) blocks, 16 rows each; none after the last layer) --
//      wait for x, the next layer's RMSNorm + quantize, q|k|v rows, store.
//
// Every block issues its weight loads before it waits, so the weight stream
// overlaps the wait.  Results go from block to block through tagged 64-bit
// words (step_common.h), polled by every thread of a waiting block (a
// counter of finished producers polled by one thread instead took 2.5-5 us
// to be seen, against 0.6-2 us for the words themselves); the tag is one
// counter for every launch, read at the start and advanced by the launch's
// last block to finish, so a graph replay needs nothing from the host and no
// buffer is ever cleared.
//
// The arithmetic is the batched GEMVs' (gemv_impl.h at M tiles of up to 4
// rows): the norms sum in double in the wave order (lane l holds elements
// 4l + 256j, then the DPP tree), the codes depend only on the row maximum,
// int8 dots are exact int32, and the epilogues are the same device
// functions, so the logits equal the kernel-per-op path's bit for bit.
//
// Waits are bounded (kSpin polls); a timed-out wait sets *err, the other
// waiting blocks see it within 64 polls and give up, and the host redoes the
// forward through the separate kernels.
#include "ec_device.h"
#include "ec_kernels.h"
#include "ec_quant.h"
#include "step_common.h"

namespace ec {

namespace {

constexpr int kTailRows = 16;                                      // rows of an OD or Q block
constexpr int kTailPairs = 64;                                     // row pairs of a G block
constexpr int kTailWP = (kTailMaxM * kTailMaxE / 2 + kStepThreads - 1) / kStepThreads;  // x words
constexpr int kTailMaxG = kTailMaxF / kTailPairs;                  // gate/up blocks at most
constexpr int kTailWQ = (kTailMaxM * kTailMaxF / 8 + 2 + kStepThreads - 1) / kStepThreads;  // FFN code pairs
// exchange areas (tagged words): x_mid [kTailMaxM][E], x [kTailMaxM][E],
// the gate/up blocks' per-token maxima (block gi's words for tokens m at
// 16 gi + m: one 128-byte line per block), the FFN codes four per word
// [M][F / 4] followed by the M rows' scales (kTailMaxM words)
constexpr int kMxLine = 16;  // words per 128-byte line
__device__ __forceinline__ unsigned long long *tail_mx(const BatchTailArgs &a) { return a.xch + 2 * kTailMaxM * a.E; }
__device__ __forceinline__ unsigned long long *tail_fq(const BatchTailArgs &a) {
  return a.xch + 2 * kTailMaxM * a.E + kMxLine * kTailMaxG;
}

// Wait for every gate/up block's maxima and form each token's row scale
// (quant_scale of the maximum over the whole FFN row: a maximum is exact in
// any order) into s_sf[m].  One wave polls, lane l the lines of blocks l
// and l + 64 (every thread of 132 blocks polling 19 shared lines took ~3 us
// to see them); every thread of a gate/up block calls it.
__device__ void wait_row_scales(const BatchTailArgs &a, int ngu, unsigned tag, float *s_sf) {
  const int t = threadIdx.x;
  if (t < 64) {
    const int M = a.M;
    const __amdgpu_buffer_rsrc_t rs = xch_rsrc(tail_mx(a), ngu * kMxLine);
    float mx[kTailMaxM] = {0.f, 0.f, 0.f, 0.f};
    unsigned pending = 0;
#pragma unroll
    for (int h = 0; h < 2; h++)
      if (t + 64 * h < ngu) pending |= 1u << h;
    for (int it = 0; pending; it++) {
      v4u w[2][2];
#pragma unroll
      for (int h = 0; h < 2; h++)
        if ((pending >> h) & 1u) {
          w[h][0] = get_pair(rs, (t + 64 * h) * (kMxLine / 2));
          w[h][1] = M > 2 ? get_pair(rs, (t + 64 * h) * (kMxLine / 2) + 1) : w[h][0];
        }
#pragma unroll
      for (int h = 0; h < 2; h++) {
        if (!((pending >> h) & 1u)) continue;
        const unsigned tg[4] = {w[h][0].y, w[h][0].w, w[h][1].y, w[h][1].w};
        bool ok = true;
#pragma unroll
        for (int m = 0; m < kTailMaxM; m++) ok = ok && (m >= M || tg[m] == tag);
        if (ok) {
          const uint32_t vv[4] = {w[h][0].x, w[h][0].z, w[h][1].x, w[h][1].z};
#pragma unroll
          for (int m = 0; m < kTailMaxM; m++)
            if (m < M) mx[m] = fmaxf(mx[m], __uint_as_float(vv[m]));
          pending &= ~(1u << h);
        }
      }
      if (!pending) break;
      if (it >= kSpin) {
        atomicOr(a.err, 1);
        break;
      }
      if ((it & 63) == 63 && __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int m = 0; m < kTailMaxM; m++) {
      const float r = wave_max_dpp(mx[m]);
      if (t == 0) s_sf[m] = quant_scale(r);
    }
  }
  __syncthreads();
}

// sum over the 8 lanes of each row group (exact int32)
__device__ __forceinline__ int tsum8(int v) {
  v = v + dpp_mov<0xB1>(v);
  v = v + dpp_mov<0x4E>(v);
  v = v + dpp_mov<0x141>(v);
  return v;
}

// sum over the wave (exact int32)
__device__ __forceinline__ int tsum64(int v) {
  v = v + dpp_mov<0xB1>(v);
  v = v + dpp_mov<0x4E>(v);
  v = v + dpp_mov<0x141>(v);
  v = v + dpp_mov<0x140>(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

__device__ __forceinline__ int tdot16(int s, v4i w, v4i x) {
  s = __builtin_amdgcn_sdot4(x.x, w.x, s, false);
  s = __builtin_amdgcn_sdot4(x.y, w.y, s, false);
  s = __builtin_amdgcn_sdot4(x.z, w.z, s, false);
  s = __builtin_amdgcn_sdot4(x.w, w.w, s, false);
  return s;
}

// A block's words for an exchange: stored, then waited for (the stores
// complete) before the block goes on, as the persistent steps do
__device__ __forceinline__ void published() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// One row of K <= 1024 fp32 values (K % 4 == 0) into int8 codes by one wave,
// as the GEMV's wave-local prologue does: lane l holds elements 4l + 256j
// (x, loaded by load_row; gamma g of the same elements, loaded by the
// caller, for the RMSNorm); NORM: RMSNorm first.  Returns the row scale.
__device__ __forceinline__ void load_row(const float *row, int K, float4 (&x)[4]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 4; j++) x[j] = *reinterpret_cast<const float4 *>(row + min(4 * lane + 256 * j, K - 4));
}
template <bool NORM>
__device__ float wave_codes(float4 (&x)[4], const float4 (&g)[4], int K, double eps, int8_t *q) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 4; j++)
    if (4 * lane + 256 * j >= K) x[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  if constexpr (NORM) {
    double s1 = 0.0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const double d0 = x[j].x, d1 = x[j].y, d2 = x[j].z, d3 = x[j].w;
      s1 += ((d0 * d0 + d1 * d1) + d2 * d2) + d3 * d3;
    }
    s1 = wave_sum_dpp(s1);
    const double rstd = 1.0 / sqrt(s1 / K + eps);
    auto nrm = [&](float v, float gv) -> float {
      v = (float)((double)v * rstd);
      return v * gv;
    };
#pragma unroll
    for (int j = 0; j < 4; j++) {
      x[j].x = nrm(x[j].x, g[j].x);
      x[j].y = nrm(x[j].y, g[j].y);
      x[j].z = nrm(x[j].z, g[j].z);
      x[j].w = nrm(x[j].w, g[j].w);
      if (4 * lane + 256 * j >= K) x[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; j++)
    mx = fmaxf(fmaxf(mx, fmaxf(fabsf(x[j].x), fabsf(x[j].y))), fmaxf(fabsf(x[j].z), fabsf(x[j].w)));
  mx = wave_max_dpp(mx);
  const float sc = quant_scale(mx);
  auto put = [&](auto q1) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = 4 * lane + 256 * j;
      if (i < K) {
        const uint32_t b0 = (uint8_t)q1(x[j].x), b1 = (uint8_t)q1(x[j].y), b2 = (uint8_t)q1(x[j].z),
                       b3 = (uint8_t)q1(x[j].w);
        *reinterpret_cast<uint32_t *>(q + i) = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
      }
    }
  };
  if (ec_quant_rcp_ok(sc)) {
    const float rcp = 1.0f / sc;
    put([&](float v) { return ec_quant1_rcp(v, sc, rcp); });
  } else {
    put([&](float v) { return quant1(v, sc); });
  }
  return sc;
}

// A row's 16-byte chunks sub + 8 c (c < 8) of a weight row of E int8: chunks
// past the row (c >= E / 128) load a clamped address and are zeroed, so the
// dot loops run all eight chunks without branches (a branch per chunk made
// each chunk's LDS read wait before its dot)
__device__ __forceinline__ void load_chunks(gptr<v4i> src, int sub, int ce, v4i (&w)[8]) {
#pragma unroll
  for (int c = 0; c < 8; c++) {
    const v4i v = __builtin_nontemporal_load(src + min(sub + 8 * c, 8 * ce - 1));
    w[c] = c < ce ? v : v4i{0, 0, 0, 0};
  }
}
// a dot of the eight chunks against the row's codes (LDS; the reads of the
// zeroed chunks past the row stay inside the codes area's padding)
__device__ __forceinline__ int dot_chunks(const v4i (&w)[8], const int8_t *q, int sub) {
  v4i x[8];
#pragma unroll
  for (int c = 0; c < 8; c++) x[c] = *reinterpret_cast<const v4i *>(q + 16 * (sub + 8 * c));
  int acc = 0;
#pragma unroll
  for (int c = 0; c < 8; c++) acc = tdot16(acc, w[c], x[c]);
  return acc;
}

// gamma of a lane's elements of the wave-local row (loaded ahead of a wait)
__device__ __forceinline__ void load_gamma(const float *g, int K, float4 (&gv)[4]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 4; j++) gv[j] = *reinterpret_cast<const float4 *>(g + min(4 * lane + 256 * j, K - 4));
}

// o / down rows [r0, r0 + 16) for every token
__device__ void tail_od(const BatchTailArgs &a, int gi, unsigned tag, int8_t *codes) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int grp = t >> 3, sub = t & 7;
  const int E = a.E, F = a.F, M = a.M, ce = E >> 7, nch = F >> 4;
  const int r0 = gi * kTailRows;
  const int ro = r0 + (grp & 15), mo = grp >> 4;
  const bool on_o = mo < M;
  unsigned long long *XM = a.xch, *X = a.xch + kTailMaxM * E;
  __shared__ float xm_own[kTailMaxM * kTailRows], x_own[kTailMaxM * kTailRows], s_sc[kTailMaxM], s_sf[kTailMaxM];

  // the attention rows first (on the critical path), then the weights: this
  // group's o row, this wave's two down rows
  float4 ax[4];
  if (wave < M) load_row(a.att + (size_t)wave * E, E, ax);
  v4i wo[8], wd[2][5];
  {
    load_chunks(gbl16(a.wo + (size_t)ro * E), sub, ce, wo);
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const auto sd = gbl16(a.wd + (size_t)(r0 + wave + 8 * h) * F);
#pragma unroll
      for (int c = 0; c < 5; c++) wd[h][c] = __builtin_nontemporal_load(sd + min(lane + 64 * c, nch - 1));
    }
  }
  const float wso = gbl(a.so)[ro], wsd0 = gbl(a.sd)[r0 + wave], wsd1 = gbl(a.sd)[r0 + wave + 8];
  const float bo = a.bo ? gbl(a.bo)[ro] : 0.0f, bd0 = a.bd ? gbl(a.bd)[r0 + wave] : 0.0f,
              bd1 = a.bd ? gbl(a.bd)[r0 + wave + 8] : 0.0f;
  const float xin = on_o && sub == 0 ? a.x[(size_t)mo * E + ro] : 0.0f;

  // ---- O: each token's attention row quantized by wave m ----
  if (wave < M) {
    const float4 none[4] = {};
    const float s = wave_codes<false>(ax, none, E, 0.0, codes + (size_t)wave * E);
    if (lane == 0) s_sc[wave] = s;
  }
  __syncthreads();
  if (on_o) {
    const int acc = tsum8(dot_chunks(wo, codes + (size_t)mo * E, sub));
    if (sub == 0) xm_own[mo * kTailRows + (grp & 15)] = xin + i8_epilogue(acc, s_sc[mo], wso, bo);
  }
  __syncthreads();
  // one wave stores the words, one instruction per 128-byte line (token m's 16 rows)
  if (t < M * kTailRows) put_word(XM + (size_t)(t >> 4) * E + r0 + (t & 15), xm_own[t], tag);
  published();

  // ---- D: the rows' scales from the gate/up blocks' maxima, then the FFN
  // codes (quantized by the gate/up blocks, four per word) into LDS ----
  // (the scales follow the codes, written by gate/up block 0: the o/down
  // blocks do not poll the maxima lines)
  {
    const int ncp = M * F / 8;  // code pairs
    float v[kTailWQ][2];
    const unsigned own = wait_pairs<kTailWQ>(tail_fq(a), M * F / 4 + kTailMaxM, tag, v, a.err);
#pragma unroll
    for (int j = 0; j < kTailWQ; j++) {
      const int p = t + kStepThreads * j;
      if ((own >> j) & 1u) {
        if (p < ncp) {
          *reinterpret_cast<uint2 *>(codes + 8 * p) = make_uint2(__float_as_uint(v[j][0]), __float_as_uint(v[j][1]));
        } else {
          s_sf[2 * (p - ncp)] = v[j][0];
          s_sf[2 * (p - ncp) + 1] = v[j][1];
        }
      }
    }
  }
  __syncthreads();
  float sc[kTailMaxM];
#pragma unroll
  for (int m = 0; m < kTailMaxM; m++) sc[m] = s_sf[m];
  // down rows r0 + wave and r0 + wave + 8, every token
  int acc[2][kTailMaxM] = {};
#pragma unroll
  for (int c = 0; c < 5; c++) {
    if (lane + 64 * c < nch) {
#pragma unroll
      for (int m = 0; m < kTailMaxM; m++) {
        if (m < M) {
          const v4i xq = *reinterpret_cast<const v4i *>(codes + (size_t)m * F + 16 * (lane + 64 * c));
          acc[0][m] = tdot16(acc[0][m], wd[0][c], xq);
          acc[1][m] = tdot16(acc[1][m], wd[1][c], xq);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kTailMaxM; m++) {
    if (m < M) {
      const int d0 = tsum64(acc[0][m]), d1 = tsum64(acc[1][m]);
      if (lane == 0) {
        x_own[m * kTailRows + wave] = xm_own[m * kTailRows + wave] + i8_epilogue(d0, sc[m], wsd0, bd0);
        x_own[m * kTailRows + wave + 8] = xm_own[m * kTailRows + wave + 8] + i8_epilogue(d1, sc[m], wsd1, bd1);
      }
    }
  }
  __syncthreads();
  if (t < M * kTailRows) {
    const size_t i = (size_t)(t >> 4) * E + r0 + (t & 15);
    a.x[i] = x_own[t];
    if (a.wqkv) put_word(X + i, x_own[t], tag);
  }
}

// gate/up row pairs [g0, g0 + 64) for every token
__device__ void tail_gu(const BatchTailArgs &a, int gi, unsigned tag, float *xs, int8_t *codes) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int grp = t >> 3, sub = t & 7;
  const int E = a.E, F = a.F, M = a.M, ce = E >> 7;
  const int g0 = gi * kTailPairs;
  const int pg = min(g0 + grp, F - 1);
  const unsigned long long *XM = a.xch;
  __shared__ float s_sc[kTailMaxM], stage[kTailMaxM * kTailPairs], s_sf[kTailMaxM], s_mx[kTailMaxM];
  __shared__ uint32_t qstage[kTailMaxM * kTailPairs / 4];  // the block's codes, four per word
  __shared__ uint64_t etab[32];  // the SiLU's 2^(i/32) table
  if (t < 32) etab[t] = ec_exp2_32[t];

  v4i wg[8], wu[8];
  {
    load_chunks(gbl16(a.wg + (size_t)pg * E), sub, ce, wg);
    load_chunks(gbl16(a.wu + (size_t)pg * E), sub, ce, wu);
  }
  const float bsg = gbl(a.sg)[pg], bsu = gbl(a.su)[pg];
  float4 gam[4];
  load_gamma(a.ln2_g, E, gam);

  gather<kTailWP>(XM, M * E, tag, xs, a.err);
  if (wave < M) {
    float4 xr[4];
    load_row(xs + (size_t)wave * E, E, xr);
    const float s = wave_codes<true>(xr, gam, E, a.eps, codes + (size_t)wave * E);
    if (lane == 0) s_sc[wave] = s;
  }
  __syncthreads();
  int ag[kTailMaxM] = {}, au[kTailMaxM] = {};
#pragma unroll
  for (int m = 0; m < kTailMaxM; m++) {
    if (m < M) {
      v4i x[8];
#pragma unroll
      for (int c = 0; c < 8; c++) x[c] = *reinterpret_cast<const v4i *>(codes + (size_t)m * E + 16 * (sub + 8 * c));
#pragma unroll
      for (int c = 0; c < 8; c++) {
        ag[m] = tdot16(ag[m], wg[c], x[c]);
        au[m] = tdot16(au[m], wu[c], x[c]);
      }
    }
  }
  // every lane of the group holds the sums; lane m takes token m's epilogue
  int dg = 0, du = 0;
#pragma unroll
  for (int m = 0; m < kTailMaxM; m++) {
    if (m < M) {
      const int sg = tsum8(ag[m]), su = tsum8(au[m]);
      if (sub == m) {
        dg = sg;
        du = su;
      }
    }
  }
  if (sub < M) {
    const float gv = i8_epilogue(dg, s_sc[sub], bsg, 0.0f), u = i8_epilogue(du, s_sc[sub], bsu, 0.0f);
    stage[sub * kTailPairs + grp] = silu(gv, etab) * u;
  }
  __syncthreads();
  // wave m: token m's maximum over this block's values, published; then,
  // with every block's maxima, the row scale and this block's codes
  const int ngu = (F + kTailPairs - 1) / kTailPairs;
  unsigned long long *MX = tail_mx(a), *FQ = tail_fq(a);
  const float hv = wave < M && g0 + lane < F ? stage[wave * kTailPairs + lane] : 0.0f;
  if (wave < M) {
    const float mx = wave_max_dpp(fabsf(hv));
    if (lane == 0) s_mx[wave] = mx;
  }
  __syncthreads();
  // the block's line of maxima, by one store instruction
  if (t < M) put_word(MX + (size_t)gi * kMxLine + t, s_mx[t], tag);
  wait_row_scales(a, ngu, tag, s_sf);
  if (wave < M) {
    const float sf = s_sf[wave];
    const int8_t c = ec_quant_rcp_ok(sf) ? ec_quant1_rcp(hv, sf, 1.0f / sf) : quant1(hv, sf);
    reinterpret_cast<int8_t *>(qstage)[wave * kTailPairs + lane] = c;
  }
  __syncthreads();
  // 16 words (64 codes) per token, stored by one wave; block 0 also stores
  // the rows' scales after the codes
  if (t < 16 * M) {
    const int m = t >> 4, k = t & 15;
    if (g0 + 4 * k < F)
      put_word(FQ + (size_t)m * (F / 4) + g0 / 4 + k, __uint_as_float(qstage[m * 16 + k]), tag);
  }
  if (gi == 0 && t >= 64 && t < 64 + kTailMaxM)
    put_word(FQ + (size_t)M * (F / 4) + (t - 64), t - 64 < M ? s_sf[t - 64] : 1.0f, tag);
}

// the next layer's q|k|v rows [q0, q0 + 16) for every token
__device__ void tail_qkv(const BatchTailArgs &a, int qi, unsigned tag, float *xs, int8_t *codes) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int grp = t >> 3, sub = t & 7;
  const int E = a.E, M = a.M, ce = E >> 7;
  const int rq = min(qi * kTailRows + (grp & 15), a.NQ - 1), mq = grp >> 4;
  const bool on_q = mq < M && qi * kTailRows + (grp & 15) < a.NQ;
  const unsigned long long *X = a.xch + kTailMaxM * E;
  __shared__ float s_sc[kTailMaxM];

  v4i wq[8];
  {
    load_chunks(gbl16(a.wqkv + (size_t)rq * E), sub, ce, wq);
  }
  const float wsq = gbl(a.sqkv)[rq], bq = a.bqkv ? gbl(a.bqkv)[rq] : 0.0f;
  float4 gam[4];
  load_gamma(a.ln1n_g, E, gam);

  gather<kTailWP>(X, M * E, tag, xs, a.err);
  if (wave < M) {
    float4 xr[4];
    load_row(xs + (size_t)wave * E, E, xr);
    const float s = wave_codes<true>(xr, gam, E, a.eps, codes + (size_t)wave * E);
    if (lane == 0) s_sc[wave] = s;
  }
  __syncthreads();
  if (on_q) {
    const int acc = tsum8(dot_chunks(wq, codes + (size_t)mq * E, sub));
    if (sub == 0) a.qkv[(size_t)mq * a.ldq + rq] = i8_epilogue(acc, s_sc[mq], wsq, bq);
  }
}

__global__ __launch_bounds__(kStepThreads) void batch_tail_kernel(BatchTailArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int b = blockIdx.x;
  const unsigned tag = ld_uniform(a.tag);
  const int nod = a.E / kTailRows, ngu = (a.F + kTailPairs - 1) / kTailPairs;
  const int nq = a.wqkv ? (a.NQ + kTailRows - 1) / kTailRows : 0;
  float *xs = lds;                                                      // [M][E] gathered rows
  int8_t *codes = reinterpret_cast<int8_t *>(lds + kTailMaxM * a.E);  // [M][max(E, F)]
  if (b < nod)
    tail_od(a, b, tag, codes);
  else if (b < nod + ngu)
    tail_gu(a, b - nod, tag, xs, codes);
  else if (b < nod + ngu + nq)
    tail_qkv(a, b - nod - ngu, tag, xs, codes);
  // the last block to finish advances the tag for the next launch (every
  // block read it at its start) and resets the counter
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    if (__hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1) {
      __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(a.tag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace

size_t batch_tail_lds(int E, int F) {
  // the codes area padded by the 1024 - E bytes that the dots' zeroed
  // chunks read past the last row
  return (size_t)kTailMaxM * E * sizeof(float) + (size_t)kTailMaxM * (E > F ? E : F) + kTailMaxE;
}

size_t batch_tail_xch_words(int E) {
  return (size_t)2 * kTailMaxM * E + (size_t)kMxLine * kTailMaxG + (size_t)kTailMaxM * kTailMaxF / 4 + kTailMaxM;
}

bool batch_tail_shape_ok(int E, int F, int NQ) {
  return E % 128 == 0 && E <= kTailMaxE && F % 16 == 0 && F >= 64 && F <= kTailMaxF && NQ >= 1 &&
         E / kTailRows + (F + kTailPairs - 1) / kTailPairs + (NQ + kTailRows - 1) / kTailRows <= kStepBlocks;
}

hipError_t batch_tail(const BatchTailArgs &a, bool cooperative, hipStream_t s) {
  if (a.M < 1 || a.M > kTailMaxM || !batch_tail_shape_ok(a.E, a.F, a.NQ)) return hipErrorInvalidValue;
  const size_t lds = batch_tail_lds(a.E, a.F);
  if (cooperative) {
    BatchTailArgs args = a;
    void *kargs[] = {&args};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void *>(batch_tail_kernel), dim3(kStepBlocks),
                                      dim3(kStepThreads), kargs, (unsigned)lds, s);
  }
  klaunch(batch_tail_kernel, dim3(kStepBlocks), dim3(kStepThreads), (uint32_t)lds, s, a);
  return hipGetLastError();
}

}  // namespace ec
