// Persistent decode step: every layer of the int8 Qwen2 forward for one token
// (M = 1) in one co-resident grid, for the greedy / sampled decode loop
// (src/runtime_main.c:335-352 over src/gpt2.c:667-797).
//
// Why: a decode step of separate kernels is ~120 dependent launches of
// 1-9 MB each; each launch starts with a cold weight stream and pays the
// dispatch between kernels.  Here one launch runs all layers.  Blocks hand
// their results to each other through tagged 64-bit words -- (float value,
// step tag) written with one device-coherent store -- and a consumer issues
// its phase's weight loads before it waits for the words of its input, so
// the weight stream overlaps the wait instead of following it.
//
// Grid: kStepBlocks blocks of kStepThreads threads, one per CU (cooperative
// launch: all blocks are resident, so the waits can be satisfied).  Block b
// runs on XCD b % 8.  Per layer:
//
//   A  (attention blocks: query head h, element slice s; 4 per head, the
//      heads of KV group g on XCD g) -- wait for x; RMSNorm + int8 quantize
//      (ln1); the 64 q rows of head h and the 64 + 64 k / v rows of group g
//      (int8 dot, fp32 epilogue) into LDS; then the decode attention body
//      (attn_decode.h: RoPE, fp16 KV append, scores, softmax, p*v sums);
//      publish the slice of the attention output.
//   O  (every block, rows [b N / NB, (b+1) N / NB) of 896) -- wait for the
//      attention output; quantize; o rows; x_mid = x + o (residual).
//   G  (every block, 19 gate/up row pairs) -- wait for x_mid; RMSNorm (ln2)
//      + quantize; gate and up rows; silu(g) * u.
//   D  (every block, the same rows as O) -- wait for the FFN activation;
//      quantize; down rows; x = x_mid + d.
//
// A block's O rows are its D rows, so both residuals use values the block
// itself produced.  Every arithmetic step is the separate kernels': the
// norms accumulate in double in the decode GEMV's wave order (lane l holds
// elements 4l + 256j), the activation codes depend only on the row maximum,
// int8 dots are exact int32, and the epilogues are the same device functions
// -- so the step's results are bit-identical to the kernel-per-op path.
//
// A wait is bounded: past kSpin polls the block sets *err and goes on, and
// every other waiting block sees *err within 64 polls and gives up too; the
// step then finishes quickly with invalid results and the host reports the
// error.  Nothing here spins without an exit.
#include "attn_decode.h"
#include "ec_device.h"
#include "ec_kernels.h"

namespace ec {

namespace {

constexpr int kSpin = 1 << 18;  // polls before a wait gives up (~0.3 s)
constexpr int kNW = kStepThreads / 64;  // waves per block

__device__ __forceinline__ void put_word(unsigned long long *p, float v, unsigned tag) {
  __hip_atomic_store(p, ((unsigned long long)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long get_word(const unsigned long long *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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


// Wait until words [0, n) of buf carry `tag` and put their values into dst
// (LDS).  Thread t owns words t + kStepThreads * j (j < WMAX); its loads are
// issued together and reissued only for the words still missing.  Every
// thread of the block calls it; it starts with a barrier (dst is still being
// read by the previous phase) and ends with one.
template <int WMAX>
__device__ void gather(const unsigned long long *buf, int n, unsigned tag, float *dst, int *err) {
  const int t = threadIdx.x;
  __syncthreads();
  unsigned pending = 0;
#pragma unroll
  for (int j = 0; j < WMAX; j++)
    if (t + kStepThreads * j < n) pending |= 1u << j;
  unsigned long long v[WMAX];
  for (int it = 0; pending; it++) {
#pragma unroll
    for (int j = 0; j < WMAX; j++)
      if ((pending >> j) & 1u) v[j] = get_word(buf + t + kStepThreads * j);
#pragma unroll
    for (int j = 0; j < WMAX; j++) {
      if (((pending >> j) & 1u) && (unsigned)(v[j] >> 32) == tag) {
        dst[t + kStepThreads * j] = __uint_as_float((unsigned)v[j]);
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

// gather's wait, then the int8 quantization of the words (src/gpt2.c:446-461)
// straight from the registers that received them: the row maximum over the
// block, then each thread's codes into codes[] (LDS).  Returns the scale.
template <int WMAX>
__device__ float gather_quant(const unsigned long long *buf, int n, unsigned tag, int8_t *codes, float *red,
                              int *err) {
  const int t = threadIdx.x;
  __syncthreads();  // codes are still read by the previous phase
  unsigned pending = 0;
#pragma unroll
  for (int j = 0; j < WMAX; j++)
    if (t + kStepThreads * j < n) pending |= 1u << j;
  const unsigned own = pending;
  unsigned long long v[WMAX];
  float x[WMAX];
  for (int it = 0; pending; it++) {
#pragma unroll
    for (int j = 0; j < WMAX; j++)
      if ((pending >> j) & 1u) v[j] = get_word(buf + t + kStepThreads * j);
#pragma unroll
    for (int j = 0; j < WMAX; j++) {
      if (((pending >> j) & 1u) && (unsigned)(v[j] >> 32) == tag) {
        x[j] = __uint_as_float((unsigned)v[j]);
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
  for (int j = 0; j < WMAX; j++) {
    if (!((own >> j) & 1u)) continue;
    if ((pending >> j) & 1u) x[j] = 0.0f;  // a timed-out wait (results discarded)
    mx = fmaxf(mx, fabsf(x[j]));
  }
  mx = block_max_1b<kNW>(mx, red);
  const float sc = quant_scale(mx);
  const bool fast = ec_quant_rcp_ok(sc);
  const float rcp = 1.0f / sc;
#pragma unroll
  for (int j = 0; j < WMAX; j++)
    if ((own >> j) & 1u) codes[t + kStepThreads * j] = fast ? ec_quant1_rcp(x[j], sc, rcp) : quant1(x[j], sc);
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
  const bool fast = ec_quant_rcp_ok(sc);
  const float rcp = 1.0f / sc;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int i = t + kStepThreads * j;
    if (i < K) codes[i] = fast ? ec_quant1_rcp(y[j], sc, rcp) : quant1(y[j], sc);
  }
  __syncthreads();
  return sc;
}

// TRACE: thread 0 of every block records s_memrealtime (100 MHz) at each
// phase boundary into a.trace[block][layer][kStepEvents]
template <bool TRACE>
__device__ __forceinline__ void mark(const StepArgs &a, int b, int l, int e) {
  if (TRACE && threadIdx.x == 0) a.trace[((size_t)b * a.L + l) * kStepEvents + e] = __builtin_amdgcn_s_memrealtime();
}

// The attention blocks' loop: per layer, the q/k/v rows of the head (weights
// loaded into registers one layer ahead, during the GEMV blocks' phases) and
// the attention; then the next layer's weights, and one touch of each 128-byte
// line of the next layer's K/V rows that this block's attention will read,
// so that they come from L2 when it runs.
template <bool TRACE>
__device__ void attention_loop(const StepArgs &a, int head, int slice, unsigned tag, int tok, float *lds,
                               float *qkv_s, float *red) {
  const int b = blockIdx.x;
  const int E = a.E, F = a.F, kv = 64 * a.KVH, kvh = head * a.KVH / a.H;
  const size_t S = (size_t)3 * E + F;
  float *xs = lds;
  int8_t *codes = reinterpret_cast<int8_t *>(lds + (E > F ? E : F));
  v4i w[3][7];
  float ws[3], gam[2];
  int sink = 0;
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
  for (int l = 0; l < a.L; l++) {
    mark<TRACE>(a, b, l, 0);
    const int t = tid_opaque(), grp = t >> 3, sub = t & 7;
    if (l == 0) {
      for (int i = t; i < E; i += kStepThreads) xs[i] = h2f(gbl(a.wte)[(size_t)tok * E + i]);
      __syncthreads();
    } else {
      gather<2>(a.xch + (size_t)(l - 1) * S, E, tag, xs, a.err);
    }
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
    unsigned long long *orow = a.xch + (size_t)l * S + 2 * E + hh * 64 + 16 * ss;
    attn_decode_block<64, true, kStepSlices>(a.attn, 0, hh, ss, qkv_s, qkv_s + 64, qkv_s + 128, lds,
                                             [&](int i, float o) { put_word(orow + i, o, tag); },
                                             a.kv_layer * l);
    __syncthreads();  // the body's LDS is reused by the next layer
    mark<TRACE>(a, b, l, 3);
    if (l + 1 < a.L) {
      load_layer(l + 1);
      // K and V rows [0, pos) of the group in the next layer: one 4-byte
      // load per 128-byte line (a K row and a V row are 128 bytes each)
      const int pos = ld_uniform(a.attn.pos), slot = ld_uniform(a.attn.slot);
      const size_t base = a.kv_layer * (l + 1) + (size_t)slot * a.attn.C * kv + (size_t)kvh * 64;
      const auto kc = gbl(reinterpret_cast<const int *>(a.attn.kc + base));
      const auto vc = gbl(reinterpret_cast<const int *>(a.attn.vc + base));
      for (int p = t; p < pos; p += kStepThreads) sink ^= kc[(size_t)p * kv / 2] ^ vc[(size_t)p * kv / 2];
    }
  }
  if (sink == 0x7fffffff && tag == 0) red[0] = (float)sink;  // keeps the touches (tag is never 0)
}

// The GEMV blocks' loop (block gi of ng): per layer the o rows [r0, r1) of E
// with the residual, the gate/up rows [g0, g1) of F with the SiLU gating,
// and the down rows [r0, r1) with the residual.
template <bool TRACE>
__device__ void gemv_loop(const StepArgs &a, int gi, int ng, unsigned tag, int tok, float *lds, float *xown,
                          float *xmown, float *red, uint64_t *etab) {
  const int b = blockIdx.x;
  const int E = a.E, F = a.F;
  const size_t S = (size_t)3 * E + F;
  float *xs = lds;
  int8_t *codes = reinterpret_cast<int8_t *>(lds + (E > F ? E : F));
  {
    const int r0 = gi * E / ng, r1 = (gi + 1) * E / ng;
    if ((int)threadIdx.x < r1 - r0) xown[threadIdx.x] = h2f(gbl(a.wte)[(size_t)tok * E + r0 + threadIdx.x]);
  }
  for (int l = 0; l < a.L; l++) {
    const StepLayer &W = a.layers[l];
    mark<TRACE>(a, b, l, 0);
    unsigned long long *X = a.xch + (size_t)l * S, *XM = X + E, *ATT = X + 2 * E, *FF = X + 3 * E;
    const int t = tid_opaque(), lane = t & 63, wave = t >> 6;
    const int grp = t >> 3, sub = t & 7;  // 64 row groups of 8 lanes (rows of E int8)
    const int g = uniform_opaque(gi);
    const int r0 = g * E / ng, r1 = (g + 1) * E / ng;  // o / down rows
    const int g0 = g * F / ng, g1 = (g + 1) * F / ng;  // gate/up rows

    // every weight of the layer's three phases, loaded while the attention
    // blocks run (the block waits for nothing else meanwhile): the o rows,
    // the gate/up rows and the down rows (one wave per row), with scales
    const bool on_o = grp < r1 - r0, on_g = grp < g1 - g0, on_d = wave < r1 - r0;
    const int no = r0 + (on_o ? grp : 0), ngt = g0 + (on_g ? grp : 0), nd = r0 + (on_d ? wave : 0);
    const int nch = F / 16;
    constexpr int CD = 5;  // down chunks per lane (F <= 5120)
    v4i wo[7], wg[7], wu[7], wd[CD];
    {
      const auto so = gbl16(W.wo + (size_t)no * E), sg = gbl16(W.wg + (size_t)ngt * E),
                 su = gbl16(W.wu + (size_t)ngt * E), sd = gbl16(W.wd + (size_t)nd * F);
#pragma unroll
      for (int c = 0; c < 7; c++) wo[c] = __builtin_nontemporal_load(so + sub + 8 * c);
#pragma unroll
      for (int c = 0; c < 7; c++) {
        wg[c] = __builtin_nontemporal_load(sg + sub + 8 * c);
        wu[c] = __builtin_nontemporal_load(su + sub + 8 * c);
      }
#pragma unroll
      for (int c = 0; c < CD; c++) wd[c] = __builtin_nontemporal_load(sd + min(lane + 64 * c, nch - 1));
    }
    const float wso = gbl(W.so)[no], bsg = gbl(W.sg)[ngt], bsu = gbl(W.su)[ngt], wsd = gbl(W.sd)[nd];
    float gam[2];
#pragma unroll
    for (int j = 0; j < 2; j++) gam[j] = gbl(W.ln2_g)[min(t + kStepThreads * j, E - 1)];

    // ---------------- O: output projection + residual ----------------
    {
      const float sa = gather_quant<2>(ATT, E, tag, codes, red, a.err);
      mark<TRACE>(a, b, l, 4);
      int acc = 0;
#pragma unroll
      for (int c = 0; c < 7; c++) acc = dot16(acc, wo[c], codes + 16 * (sub + 8 * c));
      acc = sum8(acc);
      if (on_o && sub == 0) {
        const float v = xown[grp] + i8_epilogue(acc, sa, wso, 0.0f);
        xmown[grp] = v;
        put_word(XM + no, v, tag);
      }
      mark<TRACE>(a, b, l, 5);
    }

    // ---------------- G: gate/up + SiLU gating ----------------
    {
      gather<2>(XM, E, tag, xs, a.err);
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
      if (on_g && sub == 0) {
        const float gv = i8_epilogue(ag, sx, bsg, 0.0f), u = i8_epilogue(au, sx, bsu, 0.0f);
        put_word(FF + ngt, silu(gv, etab + 32 * wave) * u, tag);
      }
      mark<TRACE>(a, b, l, 7);
    }

    // ---------------- D: down projection + residual ----------------
    {
      const float sf = gather_quant<10>(FF, F, tag, codes, red, a.err);
      mark<TRACE>(a, b, l, 8);
      int acc = 0;
#pragma unroll
      for (int c = 0; c < CD; c++)
        if (lane + 64 * c < nch) acc = dot16(acc, wd[c], codes + 16 * (lane + 64 * c));
      acc = sum64(acc);
      if (on_d && lane == 0) {
        const float v = xmown[wave] + i8_epilogue(acc, sf, wsd, 0.0f);
        xown[wave] = v;
        put_word(X + nd, v, tag);
        if (l + 1 == a.L) a.x_out[nd] = v;
      }
      __syncthreads();  // xown / codes reused by the next layer
      mark<TRACE>(a, b, l, 9);
    }
  }
}

template <bool TRACE>
__global__ __launch_bounds__(kStepThreads) void decode_step_kernel(StepArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  __shared__ __attribute__((aligned(16))) float qkv_s[3 * 64];  // q of head h, k and v of its group
  __shared__ float xown[8], xmown[8];  // this block's rows of x and x_mid
  __shared__ float red[kNW];
  __shared__ uint64_t etab[kNW][32];  // the SiLU's 2^(i/32) table, one copy per wave

  const int b = blockIdx.x, t = threadIdx.x;
  const unsigned tag = ld_uniform(a.tag);
  const int tok = ld_uniform(a.tok);
  etab[t >> 6][t & 31] = ec_exp2_32[t & 31];

  // roles: the attention blocks of query head h, element slice s (the heads
  // of KV group g on XCD g, as the attention kernel's XCD-grouped launch);
  // the other blocks, numbered gi in block order, run the GEMV phases
  const int rpg = a.H / a.KVH, na = rpg * kStepSlices;
  const int xcd = b & 7, jx = b >> 3;
  if (xcd < a.KVH && jx < na) {
    attention_loop<TRACE>(a, xcd * rpg + jx / kStepSlices, jx % kStepSlices, tag, tok, lds, qkv_s, red);
  } else {
    int before = 0;  // attention blocks with a lower index
    for (int x = 0; x < a.KVH; x++) before += b > x ? min(na, (b - x + 7) / 8) : 0;
    gemv_loop<TRACE>(a, b - before, kStepBlocks - a.KVH * na, tag, tok, lds, xown, xmown, red, etab[t >> 6]);
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
