// Persistent decode step: every layer of the int8 Qwen2 forward for one token
// (M = 1) in one co-resident grid, for the greedy / sampled decode loop
// (src/runtime_main.c:335-352 over src/gpt2.c:667-797).
//
// Why: a decode step of separate kernels is ~120 dependent launches of
// 1-9 MB each; each launch starts with a cold weight stream and pays the
// dispatch between kernels.  Here one launch runs all layers.  Blocks hand
// their results to each other through tagged 64-bit words -- (float value,
// step tag) written with one device-coherent store; the FFN activation
// through plain fp32 words in a half of a double buffer (ff_rearm) -- and a
// consumer issues its phase's weight loads before it waits for the words of
// its input, so the weight stream overlaps the wait instead of following it.
//
// Grid: kStepBlocks blocks of kStepThreads threads, one per CU (a plain
// launch on an idle device, or a cooperative one: all blocks resident, so the
// waits can be satisfied).  Block b runs on XCD b % 8.  Per layer:
//
//   A  (56 attention blocks: query head h, element slice s; 4 per head, the
//      heads of KV group g on XCD g) -- wait for x; RMSNorm + int8 quantize
//      (ln1); the 64 q rows of head h and the 64 + 64 k / v rows of group g
//      (int8 dot, fp32 epilogue) into LDS; then the decode attention body
//      (attn_decode.h: RoPE, fp16 KV append, scores, softmax, p*v sums);
//      publish the slice of the attention output.
//   O  (E / 16 o / down blocks, 16 rows each) -- wait for the attention
//      output; quantize; o rows; x_mid = x + o (residual).
//   G  (ceil(F / 64) gate/up blocks, up to 64 row pairs each) -- wait for
//      x_mid; RMSNorm (ln2) + quantize; gate and up rows; silu(g) * u.
//   D  (the o / down blocks, the same rows as O) -- wait for the FFN
//      activation; quantize; down rows; x = x_mid + d.
//
// An o / down block's O rows are its D rows, so both residuals use values
// the block itself produced.  Every arithmetic step is the separate kernels':
// the norms accumulate in double in the decode GEMV's wave order (lane l
// holds elements 4l + 256j), the activation codes depend only on the row
// maximum, int8 dots are exact int32, and the epilogues are the same device
// functions -- so the step's results are bit-identical to the kernel-per-op
// path.
//
// A wait is bounded: past kSpin polls the block sets *err and goes on, and
// every other waiting block sees *err within 64 polls and gives up too; the
// step then finishes quickly with invalid results and the host reports the
// error.  Nothing here spins without an exit.
#include "attn_decode.h"
#include "ec_device.h"
#include "ec_kernels.h"
#include "step_common.h"

namespace ec {

namespace {

constexpr int kNW = kStepThreads / 64;  // waves per block
constexpr int kODRows = 2 * kNW;          // o / down rows per o / down block (two down rows per wave)
constexpr int kFMax = 5120;               // largest FFN width

// TRACE: thread 0 of every block records s_memrealtime (100 MHz) at each
// phase boundary into a.trace[block][layer][kStepEvents]
template <bool TRACE>
__device__ __forceinline__ void mark(const StepArgs &a, int b, int l, int e) {
  if (TRACE && threadIdx.x == 0) a.trace[((size_t)b * a.L + l) * kStepEvents + e] = __builtin_amdgcn_s_memrealtime();
}

// A block's words for an exchange are stored by one wave, one store
// instruction per 128-byte line (lines written piecewise by several waves
// reached the readers about 0.7 us later); published(): that wave waits until
// its stores have reached the device-coherent level and the block waits for
// it, before any wave issues more loads (a store left behind the next
// layer's weight loads reached the readers later still).
__device__ __forceinline__ void published() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// gather's wait, then the int8 quantization of the words (src/gpt2.c:446-461)
// straight from the registers that received them: the row maximum over the
// block, then each thread's codes into codes[] (LDS).  Returns the scale.
// TRACE: event ev of layer l is recorded once every thread has its words.
template <int WP, bool TRACE = false>
__device__ float gather_quant(const unsigned long long *buf, int n, unsigned tag, int8_t *codes, float *red,
                              int *err, const StepArgs *ta = nullptr, int l = 0, int ev = 0) {
  const int t = threadIdx.x;
  __syncthreads();  // codes are still read by the previous phase
  float x[WP][2];
  const unsigned own = wait_pairs<WP>(buf, n, tag, x, err);
  if constexpr (TRACE) {
    __syncthreads();
    mark<true>(*ta, blockIdx.x, l, ev);
  }
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < WP; j++) mx = fmaxf(mx, fmaxf(fabsf(x[j][0]), fabsf(x[j][1])));
  mx = block_max_1b<kNW>(mx, red);
  const float sc = quant_scale(mx);
  auto put = [&](auto q1) {
#pragma unroll
    for (int j = 0; j < WP; j++) {
      if (!((own >> j) & 1u)) continue;
      const int8_t c0 = q1(x[j][0]), c1 = q1(x[j][1]);
      *reinterpret_cast<uint16_t *>(codes + 2 * (t + kStepThreads * j)) =
          (uint16_t)((uint8_t)c0 | ((unsigned)(uint8_t)c1 << 8));
    }
  };
  // one branch per block (sc is uniform), not a select per element
  if (ec_quant_rcp_ok(sc)) {
    const float rcp = 1.0f / sc;
    put([&](float v) { return ec_quant1_rcp(v, sc, rcp); });
  } else {
    put([&](float v) { return quant1(v, sc); });
  }
  __syncthreads();
  return sc;
}


// The FFN activation: plain fp32 words, kStepFfEmpty until written (each
// word by one 4-byte store).  gather_quant_ff waits until words [0, n) of buf
// (n % 4 == 0, buf 16-byte aligned) are all written -- thread t owns the
// quads t + kStepThreads * j (j < WQ), one 16-byte device-coherent load each,
// reissued only for the quads still incomplete -- then quantizes them as
// gather_quant does.
template <int WQ>
__device__ float gather_quant_ff(const float *buf, int n, int8_t *codes, float *red, int *err) {
  const int t = threadIdx.x;
  __syncthreads();  // codes are still read by the previous phase
  const uint64_t bp = (uint64_t)(uintptr_t)buf;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)bp), hi = __builtin_amdgcn_readfirstlane((uint32_t)(bp >> 32));
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(uintptr_t)(((uint64_t)hi << 32) | lo), 0, __builtin_amdgcn_readfirstlane(n * 4), 0x00020000);
  unsigned pending = 0;
#pragma unroll
  for (int j = 0; j < WQ; j++)
    if (t + kStepThreads * j < (n >> 2)) pending |= 1u << j;
  const unsigned own = pending;
  v4u v[WQ];
  float x[WQ][4];
#pragma unroll
  for (int j = 0; j < WQ; j++) x[j][0] = x[j][1] = x[j][2] = x[j][3] = 0.0f;
  for (int it = 0; pending; it++) {
#pragma unroll
    for (int j = 0; j < WQ; j++)
      if ((pending >> j) & 1u)
        v[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, (t + kStepThreads * j) * 16, 0, 16 /* sc1 */);
#pragma unroll
    for (int j = 0; j < WQ; j++) {
      if (((pending >> j) & 1u) && v[j].x != kStepFfEmpty && v[j].y != kStepFfEmpty && v[j].z != kStepFfEmpty &&
          v[j].w != kStepFfEmpty) {
        x[j][0] = __uint_as_float(v[j].x);
        x[j][1] = __uint_as_float(v[j].y);
        x[j][2] = __uint_as_float(v[j].z);
        x[j][3] = __uint_as_float(v[j].w);
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
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < WQ; j++)
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x[j][0]), fabsf(x[j][1])), fmaxf(fabsf(x[j][2]), fabsf(x[j][3]))));
  mx = block_max_1b<kNW>(mx, red);
  const float sc = quant_scale(mx);
  auto put = [&](auto q1) {
#pragma unroll
    for (int j = 0; j < WQ; j++) {
      if (!((own >> j) & 1u)) continue;
      uint32_t c = 0;
#pragma unroll
      for (int e = 0; e < 4; e++) c |= (uint32_t)(uint8_t)q1(x[j][e]) << (8 * e);
      *reinterpret_cast<uint32_t *>(codes + 4 * (t + kStepThreads * j)) = c;
    }
  };
  // one branch per block (sc is uniform), not a select per element
  if (ec_quant_rcp_ok(sc)) {
    const float rcp = 1.0f / sc;
    put([&](float v) { return ec_quant1_rcp(v, sc, rcp); });
  } else {
    put([&](float v) { return quant1(v, sc); });
  }
  __syncthreads();
  return sc;
}

// sum over the 8 lanes of each row group (exact int32)
__device__ __forceinline__ int sum8(int v) {
  v = v + dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v = v + dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v = v + dpp_mov<0x141>(v);  // row_half_mirror
  return v;
}

// 16 int8 products of a weight chunk against the activation chunk x
__device__ __forceinline__ int dot16x(int s, v4i w, v4i x) {
  s = __builtin_amdgcn_sdot4(x.x, w.x, s, false);
  s = __builtin_amdgcn_sdot4(x.y, w.y, s, false);
  s = __builtin_amdgcn_sdot4(x.z, w.z, s, false);
  s = __builtin_amdgcn_sdot4(x.w, w.w, s, false);
  return s;
}

// 16 int8 products of a weight chunk against the activation chunk at q
__device__ __forceinline__ int dot16(int s, v4i w, const int8_t *q) {
  const v4i x = *reinterpret_cast<const v4i *>(q);
  s = __builtin_amdgcn_sdot4(x.x, w.x, s, false);
  s = __builtin_amdgcn_sdot4(x.y, w.y, s, false);
  s = __builtin_amdgcn_sdot4(x.z, w.z, s, false);
  s = __builtin_amdgcn_sdot4(x.w, w.w, s, false);
  return s;
}

}  // namespace

// Layout of the dynamic LDS outside the attention body: fp32 row (up to F
// floats), then the int8 codes (one copy per wave for rows <= 1024, one
// shared copy for the FFN row).
size_t decode_step_scratch_bytes(int E, int F) {
  const int K = E > F ? E : F;
  const size_t codes = (size_t)(kNW * 1024 > K ? kNW * 1024 : K);
  return (size_t)K * 4 + codes + 64;
}

// sum over the wave (exact int32): rows of 16 by DPP, then the four rows
__device__ __forceinline__ int sum64(int v) {
  v = v + dpp_mov<0xB1>(v);
  v = v + dpp_mov<0x4E>(v);
  v = v + dpp_mov<0x141>(v);
  v = v + dpp_mov<0x140>(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

// RMSNorm (gamma) of the fp32 row xs[K] (LDS, K <= 1024, K % 4 == 0) and
// its int8 quantization into codes (LDS, shared), by the whole block.  The
// sum of squares is formed in the decode GEMV's wave order (lane l holds
// elements 4l + 256j, then the DPP tree), by every wave; the normalization,
// the row maximum and the codes are element-wise and split over the block
// (thread t: elements t and t + kStepThreads).  g[] holds gamma of those
// elements, loaded by the caller.  Returns the row scale.
__device__ float block_norm_quant(const float *xs, int K, const float *g, double eps, int8_t *codes, float *red) {
  const int t = threadIdx.x, lane = t & 63;
  double s1 = 0.0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    float4 x = *reinterpret_cast<const float4 *>(xs + min(4 * lane + 256 * j, K - 4));
    if (4 * lane + 256 * j >= K) x = make_float4(0.f, 0.f, 0.f, 0.f);
    const double d0 = x.x, d1 = x.y, d2 = x.z, d3 = x.w;
    s1 += ((d0 * d0 + d1 * d1) + d2 * d2) + d3 * d3;
  }
  s1 = wave_sum_dpp(s1);
  const double rstd = 1.0 / sqrt(s1 / K + eps);
  float y[2];
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int i = t + kStepThreads * j;
    y[j] = 0.0f;
    if (i < K) {
      const float xn = (float)((double)xs[i] * rstd);
      y[j] = xn * g[j];
      mx = fmaxf(mx, fabsf(y[j]));
    }
  }
  mx = block_max_1b<kNW>(mx, red);
  const float sc = quant_scale(mx);
  // one branch per block (sc is uniform), not a select per element
  if (ec_quant_rcp_ok(sc)) {
    const float rcp = 1.0f / sc;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int i = t + kStepThreads * j;
      if (i < K) codes[i] = ec_quant1_rcp(y[j], sc, rcp);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int i = t + kStepThreads * j;
      if (i < K) codes[i] = quant1(y[j], sc);
    }
  }
  __syncthreads();
  return sc;
}


// The attention blocks' loop: per layer, the q/k/v rows of the head (weights
// loaded into registers one layer ahead, during the GEMV blocks' phases) and
// the attention; then the next layer's weights, and one touch of each 128-byte
// line of the next layer's K/V rows that this block's attention will read,
// so that they come from L2 when it runs.
template <bool TRACE>
__device__ void attention_loop(const StepArgs &a, int head, int slice, unsigned tag, int tok, float *lds,
                               float *qkv_s, float *red, const uint64_t *etab) {
  const int b = blockIdx.x;
  const int E = a.E, kv = 64 * a.KVH, kvh = head * a.KVH / a.H;
  const size_t S = (size_t)3 * E;
  float *xs = lds + a.norm_off;  // past the attention area
  int8_t *codes = reinterpret_cast<int8_t *>(xs + E);
  v4i w[3][7];
  float ws[3], gam[2];
  auto load_layer = [&](int l) {
    const StepLayer &W = a.layers[l];
    const int t = tid_opaque(), grp = t >> 3, sub = t & 7;
#pragma unroll
    for (int p = 0; p < 3; p++) {
      const int r = 64 * p + grp;
      const int n = p == 0 ? head * 64 + r : p == 1 ? E + kvh * 64 + (r - 64) : E + kv + kvh * 64 + (r - 128);
      const auto src = gbl16(W.wqkv + (size_t)n * E);
#pragma unroll
      for (int c = 0; c < 7; c++) w[p][c] = __builtin_nontemporal_load(src + sub + 8 * c);
      ws[p] = gbl(W.sqkv)[n];
    }
#pragma unroll
    for (int j = 0; j < 2; j++) gam[j] = gbl(W.ln1_g)[min(t + kStepThreads * j, E - 1)];
  };
  load_layer(0);
  attn_prefetch_k<64, kStepSlices>(a.attn, 0, uniform_opaque(head), lds, 0);
  attn_prefetch_v<64, kStepSlices>(a.attn, 0, uniform_opaque(head), uniform_opaque(slice), lds, 0);
  // the token's RoPE (cos, sin) per element, the same in every layer, kept in
  // LDS (the norm's barriers publish it before the first use); the exp
  // table is the block's copy of the SiLU table
  __shared__ double2 cs_s[64];
  {
    const int t = threadIdx.x, rot = a.attn.cs ? a.attn.half : 0;
    if (t < 64)
      cs_s[t] = rot ? a.attn.cs[(size_t)ld_uniform(a.attn.pos) * a.attn.half + attn_rope_entry(t, 64, rot)]
                    : make_double2(1.0, 0.0);
  }
  const AttnPre pre{etab, cs_s};
  for (int l = 0; l < a.L; l++) {
    mark<TRACE>(a, b, l, 0);
    const int t = tid_opaque(), grp = t >> 3, sub = t & 7;
    if (l == 0) {
      for (int i = t; i < E; i += kStepThreads) xs[i] = h2f(gbl(a.wte)[(size_t)tok * E + i]);
      __syncthreads();
    } else {
      gather<1>(a.xch + (size_t)(l - 1) * S, E, tag, xs, a.err);
    }
    // this wave's K-tile rows have landed; the norm's barriers publish them
    // to the block before the attention body reads the tile
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    mark<TRACE>(a, b, l, 1);
    const float sx = block_norm_quant(xs, E, gam, a.eps, codes, red);
    mark<TRACE>(a, b, l, 11);
#pragma unroll
    for (int p = 0; p < 3; p++) {
      int acc = 0;
#pragma unroll
      for (int c = 0; c < 7; c++) acc = dot16(acc, w[p][c], codes + 16 * (sub + 8 * c));
      acc = sum8(acc);
      if (sub == 0) qkv_s[64 * p + grp] = i8_epilogue(acc, sx, ws[p], 0.0f);
    }
    __syncthreads();
    mark<TRACE>(a, b, l, 2);
    const int hh = uniform_opaque(head), ss = uniform_opaque(slice);
    unsigned long long *att = a.xch + (size_t)l * S + 2 * E;
    const int o0 = hh * 64 + 16 * ss;
    attn_decode_block<64, true, kStepSlices, false, true>(a.attn, 0, hh, ss, qkv_s, qkv_s + 64, qkv_s + 128, lds,
                                             [&](int i, float o) { put_word(att + o0 + i, o, tag); },
                                             a.kv_layer * l, [&](int e) { mark<TRACE>(a, b, l, e < 3 ? 15 + e : 1 + e); }, &pre);
    mark<TRACE>(a, b, l, 8);
    published();  // (threads t < 16 stored the slice's words; the body's LDS is reused by the next layer)
    mark<TRACE>(a, b, l, 3);
    if (l + 1 < a.L) {
      load_layer(l + 1);
      // the next layer's K rows into the K tile (its first KQ positions) and
      // this slice's V rows into the V tile
      attn_prefetch_k<64, kStepSlices>(a.attn, 0, hh, lds, a.kv_layer * (l + 1));
      attn_prefetch_v<64, kStepSlices>(a.attn, 0, hh, ss, lds, a.kv_layer * (l + 1));
    }
  }
}

// The o / down blocks' loop (block gi): per layer the o rows [r0, r0 + kODRows)
// of E with the residual, then the down rows of the same indices with the
// residual.  Their weights (one 8-lane group per o row, one wave per two down
// rows) are loaded at the start of the layer, while the attention runs.
template <bool TRACE>
__device__ void od_loop(const StepArgs &a, int gi, unsigned tag, int tok, float *lds, float *xown, float *xmown,
                        float *red) {
  const int b = blockIdx.x;
  const int E = a.E, F = a.F;
  const size_t S = (size_t)3 * E;
  int8_t *codes = reinterpret_cast<int8_t *>(lds + (E > F ? E : F));
  if ((int)threadIdx.x < kODRows) xown[threadIdx.x] = h2f(gbl(a.wte)[(size_t)tok * E + gi * kODRows + threadIdx.x]);
  for (int l = 0; l < a.L; l++) {
    const StepLayer &W = a.layers[l];
    mark<TRACE>(a, b, l, 0);
    unsigned long long *X = a.xch + (size_t)l * S, *XM = X + E, *ATT = X + 2 * E;
    const float *FV = a.ffv + ((size_t)(tag & 1u) * a.L + l) * F;
    const int t = tid_opaque(), lane = t & 63, wave = t >> 6;
    const int grp = t >> 3, sub = t & 7;  // 64 row groups of 8 lanes (rows of E int8)
    const int r0 = uniform_opaque(gi) * kODRows;
    const bool on_o = grp < kODRows;
    const int no = r0 + (on_o ? grp : 0);
    const int nch = F / 16;
    constexpr int CD = 5;  // down chunks per lane (F <= 5120)
    v4i wo[7], wd[2][CD];
    {
      const auto so = gbl16(W.wo + (size_t)no * E);
      if (on_o) {
#pragma unroll
        for (int c = 0; c < 7; c++) wo[c] = __builtin_nontemporal_load(so + sub + 8 * c);
      }
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const auto sd = gbl16(W.wd + (size_t)(r0 + wave + 8 * h) * F);
#pragma unroll
        for (int c = 0; c < CD; c++) wd[h][c] = __builtin_nontemporal_load(sd + min(lane + 64 * c, nch - 1));
      }
    }
    const float wso = gbl(W.so)[no], wsd0 = gbl(W.sd)[r0 + wave], wsd1 = gbl(W.sd)[r0 + wave + 8];

    // ---------------- O: output projection + residual ----------------
    {
      const float sa = gather_quant<1, TRACE>(ATT, E, tag, codes, red, a.err, &a, l, 13);
      mark<TRACE>(a, b, l, 4);
      int acc = 0;
#pragma unroll
      for (int c = 0; c < 7; c++) acc = dot16(acc, wo[c], codes + 16 * (sub + 8 * c));
      acc = sum8(acc);
      if (on_o && sub == 0) xmown[grp] = xown[grp] + i8_epilogue(acc, sa, wso, 0.0f);
      __syncthreads();
      if ((int)threadIdx.x < kODRows) put_word(XM + r0 + threadIdx.x, xmown[threadIdx.x], tag);
      published();
      mark<TRACE>(a, b, l, 5);
    }

    // ---------------- D: down projection + residual ----------------
    {
      const float sf = gather_quant_ff<(kFMax / 4 + kStepThreads - 1) / kStepThreads>(FV, F, codes, red, a.err);
      mark<TRACE>(a, b, l, 12);
      mark<TRACE>(a, b, l, 8);
      int acc0 = 0, acc1 = 0;
#pragma unroll
      for (int c = 0; c < CD; c++) {
        if (lane + 64 * c < nch) {
          const v4i x = *reinterpret_cast<const v4i *>(codes + 16 * (lane + 64 * c));
          acc0 = dot16x(acc0, wd[0][c], x);
          acc1 = dot16x(acc1, wd[1][c], x);
        }
      }
      acc0 = sum64(acc0);
      acc1 = sum64(acc1);
      if (lane == 0) {
        xown[wave] = xmown[wave] + i8_epilogue(acc0, sf, wsd0, 0.0f);
        xown[wave + 8] = xmown[wave + 8] + i8_epilogue(acc1, sf, wsd1, 0.0f);
      }
      __syncthreads();
      if ((int)threadIdx.x < kODRows) {
        put_word(X + r0 + threadIdx.x, xown[threadIdx.x], tag);
        if (l + 1 == a.L) a.x_out[r0 + threadIdx.x] = xown[threadIdx.x];
      }
      published();  // (xown / codes are reused by the next layer)
      mark<TRACE>(a, b, l, 9);
    }
  }
}

// The gate/up blocks' loop (block gi of ng): per layer the gate/up row pairs
// [g0, g1) of F (at most 64: one 8-lane group each) with the SiLU gating,
// after the RMSNorm and quantization of x_mid.  etab: this wave's copy of
// the SiLU's 2^(i/32) table.
template <bool TRACE>
__device__ void gu_loop(const StepArgs &a, int gi, int ng, unsigned tag, float *lds, float *red, uint64_t *etab) {
  const int b = blockIdx.x;
  const int E = a.E, F = a.F;
  const size_t S = (size_t)3 * E;
  float *xs = lds;
  int8_t *codes = reinterpret_cast<int8_t *>(lds + (E > F ? E : F));
  for (int l = 0; l < a.L; l++) {
    const StepLayer &W = a.layers[l];
    mark<TRACE>(a, b, l, 0);
    unsigned long long *XM = a.xch + (size_t)l * S + E;
    float *FV = a.ffv + ((size_t)(tag & 1u) * a.L + l) * F;
    const int t = tid_opaque();
    const int grp = t >> 3, sub = t & 7;  // 64 row groups of 8 lanes (rows of E int8)
    const int g = uniform_opaque(gi);
    const int g0 = g * F / ng, g1 = (g + 1) * F / ng;
    const bool on_g = grp < g1 - g0;
    const int ngt = g0 + (on_g ? grp : 0);
    v4i wg[7], wu[7];
    {
      const auto sg = gbl16(W.wg + (size_t)ngt * E), su = gbl16(W.wu + (size_t)ngt * E);
#pragma unroll
      for (int c = 0; c < 7; c++) {
        wg[c] = __builtin_nontemporal_load(sg + sub + 8 * c);
        wu[c] = __builtin_nontemporal_load(su + sub + 8 * c);
      }
    }
    const float bsg = gbl(W.sg)[ngt], bsu = gbl(W.su)[ngt];
    float gam[2];
#pragma unroll
    for (int j = 0; j < 2; j++) gam[j] = gbl(W.ln2_g)[min(t + kStepThreads * j, E - 1)];

    gather<1>(XM, E, tag, xs, a.err);
    mark<TRACE>(a, b, l, 6);
    const float sx = block_norm_quant(xs, E, gam, a.eps, codes, red);
    mark<TRACE>(a, b, l, 10);
    int ag = 0, au = 0;
#pragma unroll
    for (int c = 0; c < 7; c++) {
      ag = dot16(ag, wg[c], codes + 16 * (sub + 8 * c));
      au = dot16(au, wu[c], codes + 16 * (sub + 8 * c));
    }
    ag = sum8(ag);
    au = sum8(au);
    __shared__ float stage[64];  // the block's FFN words
    if (on_g && sub == 0) {
      const float gv = i8_epilogue(ag, sx, bsg, 0.0f), u = i8_epilogue(au, sx, bsu, 0.0f);
      stage[grp] = silu(gv, etab) * u;
    }
    __syncthreads();
    if ((int)threadIdx.x < g1 - g0)
      __hip_atomic_store(reinterpret_cast<uint32_t *>(FV + g0 + threadIdx.x), __float_as_uint(stage[threadIdx.x]),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    published();
    mark<TRACE>(a, b, l, 7);
  }
}

// A block with no role (ib of nb): fill the FFN half that the next step
// (tag + 1) uses with kStepFfEmpty.  The previous step used it and has
// ended; the next one starts after this launch ends.
__device__ void ff_rearm(const StepArgs &a, int ib, int nb, unsigned tag) {
  const size_t nq = (size_t)a.L * a.F / 4;
  v4u *q = reinterpret_cast<v4u *>(a.ffv + (size_t)((tag + 1u) & 1u) * a.L * a.F);
  const v4u e = {kStepFfEmpty, kStepFfEmpty, kStepFfEmpty, kStepFfEmpty};
  for (size_t i = (size_t)ib * kStepThreads + threadIdx.x; i < nq; i += (size_t)nb * kStepThreads) q[i] = e;
}

template <bool TRACE>
__global__ __launch_bounds__(kStepThreads) void decode_step_kernel(StepArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  __shared__ __attribute__((aligned(16))) float qkv_s[3 * 64];  // q of head h, k and v of its group
  __shared__ float xown[kODRows], xmown[kODRows];  // an o / down block's rows of x and x_mid
  __shared__ float red[kNW];
  __shared__ uint64_t etab[kNW][32];  // the SiLU's 2^(i/32) table, one copy per wave

  const int b = blockIdx.x, t = threadIdx.x;
  const unsigned tag = ld_uniform(a.tag);
  const int tok = ld_uniform(a.tok);
  etab[t >> 6][t & 31] = ec_exp2_32[t & 31];

  // roles: the attention blocks of query head h, element slice s (the heads
  // of KV group g on XCD g, as the attention kernel's XCD-grouped launch);
  // the other blocks, numbered gi in block order: E / kODRows o / down
  // blocks, then ceil(F / 64) gate/up blocks; the rest have nothing to do.
  // Separate roles keep the number of blocks that read each exchange small.
  const int rpg = a.H / a.KVH, na = rpg * kStepSlices;
  const int xcd = b & 7, jx = b >> 3;
  if (xcd < a.KVH && jx < na) {
    attention_loop<TRACE>(a, xcd * rpg + jx / kStepSlices, jx % kStepSlices, tag, tok, lds, qkv_s, red, etab[0]);
  } else {
    int before = 0;  // attention blocks with a lower index
    for (int x = 0; x < a.KVH; x++) before += b > x ? min(na, (b - x + 7) / 8) : 0;
    const int gi = b - before, nod = a.E / kODRows, ngu = (a.F + 63) / 64;
    if (gi < nod)
      od_loop<TRACE>(a, gi, tag, tok, lds, xown, xmown, red);
    else if (gi < nod + ngu)
      gu_loop<TRACE>(a, gi - nod, ngu, tag, lds, red, etab[t >> 6]);
    else
      ff_rearm(a, gi - nod - ngu, kStepBlocks - a.KVH * na - nod - ngu, tag);
  }
}

hipError_t decode_step(const StepArgs &a, size_t lds, bool cooperative, hipStream_t s) {
  StepArgs args = a;
  void *kargs[] = {&args};
  const void *k = a.trace ? reinterpret_cast<const void *>(decode_step_kernel<true>)
                          : reinterpret_cast<const void *>(decode_step_kernel<false>);
  if (cooperative)
    return hipLaunchCooperativeKernel(k, dim3(kStepBlocks), dim3(kStepThreads), kargs, (unsigned)lds, s);
  return hipLaunchKernel(k, dim3(kStepBlocks), dim3(kStepThreads), kargs, (unsigned)lds, s);
}

}  // namespace ec
