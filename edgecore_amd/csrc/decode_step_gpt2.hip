// Persistent decode step of the fp16 GPT-2 forward for one token (M = 1):
// every layer of src/gpt2.c:470-574 (GPT-2 small: d_model 768, 12 heads of
// head_dim 64, GELU FFN 3072, LayerNorm, biases) in one co-resident grid, for
// the decode loop (src/runtime_main.c:335-352).
//
// The same scheme as the int8 Qwen2 step (decode_step.hip): blocks hand
// results to each other through tagged words (step_common.h), and each block
// issues its phase's weight loads before it waits for the words of its input.
// 256 blocks of 512 threads, one per CU; block b runs on XCD b % 8.  Per layer:
//
//   Q  (48 q|k|v blocks, 48 of the 3 E rows each) -- wait for x; LayerNorm
//      (ln_1); 48 rows of fp16 weights against the normalized row (fp32
//      products and sums); + bias; publish.
//   A  (48 attention blocks: head h, element slice s; the 4 slices of a head
//      on one XCD) -- wait for the head's 64 q, 64 k and 64 v words (with
//      the K and V rows already in registers); fp16 KV append, scores,
//      softmax, p*v sums (gpt2_attn, no RoPE); publish the slice of the
//      output.
//   O  (48 o / down blocks, 16 rows each) -- wait for the attention output;
//      o rows + bias; x_mid = x + (o + bias); publish.
//   F  (48 fc blocks, 64 rows each) -- wait for x_mid; LayerNorm (ln_2); fc
//      rows + bias; gelu_new; publish.
//   D  (the o / down blocks, the same rows as O) -- wait for the GELU
//      outputs; down rows + bias; x = x_mid + (d + bias); publish.
//
// An exchange costs about 2 us whatever its size (the store's trip to the
// device-coherent level, about 0.7 us, then the readers' next poll).  The
// attention blocks computing the head's q|k|v rows themselves (one exchange
// fewer) was slower: each slice block then does all 192 rows (2.3 us even on
// the matrix cores, against 1 us for a Q block's 48 rows) and pulls 295 KB
// of weights through its XCD's L2 every layer.
//
// Arithmetic: LayerNorm in two passes, each lane's sums in fp32 and the
// wave's in double (a fixed tree), the normalization in fp32; GELU is gelu_new
// (ec_device.h); the fp16 dots are fp32 fused multiply-adds in a fixed order
// (the reference's AVX2 order is eight interleaved FMA chains: the fp16 path
// is compared within a tolerance, not bit for bit).  The bias is added to the
// finished dot, then the residual, as src/gpt2.c:425-429 and 561-572 do.
//
// Waits are bounded as in decode_step.hip: past kSpin polls a block sets *err
// and goes on; the step then ends with invalid results and the host reports
// the error.
#include "attn_decode.h"
#include "ec_device.h"
#include "ec_kernels.h"
#include "step_common.h"

namespace ec {

namespace {

constexpr int E = kStep16E, F = kStep16F, HD = 64;
constexpr int kQRows = 48;             // q|k|v rows per Q block: 3 E / 48 = 48 blocks
constexpr int kFRows = 64;             // fc rows per F block: F / 64 = 48 blocks
constexpr int kODRows = 16;            // o / down rows per O/D block: E / 16 = 48 blocks
constexpr int kNQ = 3 * E / kQRows, kNOD = E / kODRows, kNF = F / kFRows;
constexpr int kHeads = E / HD;
constexpr int kNA = 4 * kHeads;  // attention blocks (4 slices per head)
static_assert(kNA + kNQ + kNOD + kNF <= kStepBlocks, "roles");
static_assert(kHeads <= 16, "heads 0-7 take j 0-3 of XCD h, heads 8-15 j 4-7 of XCD h - 8");

// exchange words per layer: X [E] | XM [E] | ATT [E] | QKV [3 E]; the GELU
// outputs are plain fp32 words in a.ffv
constexpr size_t kOffXM = E, kOffATT = 2 * E, kOffQKV = 3 * E;

// TRACE: thread 0 of every block records s_memrealtime (100 MHz) at each
// phase boundary into a.trace[block][layer][kStepEvents]: Q blocks events
// 0-3 (weights issued, x gathered, normalized, published), A blocks 4-6
// (waiting, q|k|v gathered, published), O/D blocks 7-11 (weights issued, attention gathered, x_mid published, GELU
// outputs gathered, x published), F blocks 12-15 (weights issued, x_mid
// gathered, normalized, published)
template <bool TRACE>
__device__ __forceinline__ void mark(const Step16Args &a, int l, int e) {
  if (TRACE && threadIdx.x == 0)
    a.trace[((size_t)blockIdx.x * a.L + l) * kStepEvents + e] = __builtin_amdgcn_s_memrealtime();
}

// Layer l's pointers, read with scalar loads: a vector load of them would
// make their first use wait for every earlier vector load of the block (the
// weight and K / V loads still in flight).
__device__ __forceinline__ Step16Layer layer_of(const Step16Args &a, int l) {
  const Step16Layer *p = a.layers + l;
  Step16Layer W;
  W.ln1_g = ld_uniform(&p->ln1_g);
  W.ln1_b = ld_uniform(&p->ln1_b);
  W.ln2_g = ld_uniform(&p->ln2_g);
  W.ln2_b = ld_uniform(&p->ln2_b);
  W.wqkv = ld_uniform(&p->wqkv);
  W.bqkv = ld_uniform(&p->bqkv);
  W.wo = ld_uniform(&p->wo);
  W.bo = ld_uniform(&p->bo);
  W.wfc = ld_uniform(&p->wfc);
  W.bfc = ld_uniform(&p->bfc);
  W.wd = ld_uniform(&p->wd);
  W.bd = ld_uniform(&p->bd);
  return W;
}

// A block's words for an exchange are staged in LDS and stored by one wave,
// one store instruction per 128-byte line: lines written piecewise by
// several instructions (each wave its own few words) reached the readers
// about 0.7 us later.  published(): then that wave waits until the stores
// have reached the device-coherent level, and the block waits for it, before
// it issues more loads -- a store left behind the next layer's weight loads
// (up to 120 KB a block) reached the readers about 1.4 us later still.
__device__ __forceinline__ void published() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// the 8 fp16 of a 16-byte chunk times the 8 floats at h (LDS), fused into acc
__device__ __forceinline__ float fma8(float acc, v4u w, const float *h) {
  const float4 h0 = *reinterpret_cast<const float4 *>(h), h1 = *reinterpret_cast<const float4 *>(h + 4);
  const float a[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    acc = __builtin_fmaf(a[2 * k], h2f((uint16_t)(ww[k] & 0xffffu)), acc);
    acc = __builtin_fmaf(a[2 * k + 1], h2f((uint16_t)(ww[k] >> 16)), acc);
  }
  return acc;
}

// sums over the 16 lanes of each DPP row (fixed tree; every lane of the row gets it)
__device__ __forceinline__ float sum16(float v) {
  v = v + dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v = v + dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v = v + dpp_mov<0x141>(v);  // row_half_mirror
  v = v + dpp_mov<0x140>(v);  // row_mirror
  return v;
}

// The dots of 2 R rows of a wave (acc[i]: lanes 0-31 row 2 i, lanes 32-63 row
// 2 i + 1, each a partial sum over the lane's chunks): each row's sum over its
// 32 lanes (the two DPP rows of its half, then their sum); lane k < 2 R
// receives the sum of row k.
template <int R>
__device__ __forceinline__ float finish_rows(const float (&acc)[R], int lane) {
  float v = 0.0f;
#pragma unroll
  for (int i = 0; i < R; i++) {
    const float s = sum16(acc[i]);
    const float r0 = readlane(s, 0) + readlane(s, 16), r1 = readlane(s, 32) + readlane(s, 48);
    v = lane == 2 * i ? r0 : v;
    v = lane == 2 * i + 1 ? r1 : v;
  }
  return v;
}

// LayerNorm of xs[E] (LDS; src/gpt2.c:398-414) by one wave into its own
// copy hw[E] (LDS), in two passes: lane l holds elements 4 l + 256 j, j < 3,
// sums them in fp32 in a fixed order, and the wave sums the lanes' partial
// sums in double (a fixed tree); mean, variance and 1 / sqrt(var + eps) in
// double, the normalization hw = (x - mean) * rstd * gamma + beta in fp32.
// Every wave computes the statistics itself, so the block passes no
// barrier: the wave reads only what it wrote.  g / b: gamma and beta of the
// lane's elements.  (The fp16 forward is compared within a tolerance.)
__device__ __forceinline__ void wave_layer_norm(const float *xs, const float4 (&g)[3], const float4 (&b)[3],
                                                double eps, float *hw) {
  const int lane = threadIdx.x & 63;
  float4 x[3];
#pragma unroll
  for (int j = 0; j < 3; j++) x[j] = *reinterpret_cast<const float4 *>(xs + 4 * lane + 256 * j);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 3; j++) s += (x[j].x + x[j].y) + (x[j].z + x[j].w);
  const double mean = wave_sum_dpp((double)s) / E;
  const float mf = (float)mean;
  float v = 0.0f;
#pragma unroll
  for (int j = 0; j < 3; j++) {
    const float d0 = x[j].x - mf, d1 = x[j].y - mf, d2 = x[j].z - mf, d3 = x[j].w - mf;
    v += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
  }
  const float rstd = (float)(1.0 / sqrt(wave_sum_dpp((double)v) / E + eps));
#pragma unroll
  for (int j = 0; j < 3; j++) {
    float4 h;
    h.x = ((x[j].x - mf) * rstd) * g[j].x + b[j].x;
    h.y = ((x[j].y - mf) * rstd) * g[j].y + b[j].y;
    h.z = ((x[j].z - mf) * rstd) * g[j].z + b[j].z;
    h.w = ((x[j].w - mf) * rstd) * g[j].w + b[j].w;
    *reinterpret_cast<float4 *>(hw + 4 * lane + 256 * j) = h;
  }
}

// gamma and beta of lane l's LayerNorm elements (wave_layer_norm)
__device__ __forceinline__ void ln_params(const float *gp, const float *bp, int lane, float4 (&g)[3],
                                          float4 (&b)[3]) {
  const gptr<v4u> g4 = (gptr<v4u>)gp, b4 = (gptr<v4u>)bp;
#pragma unroll
  for (int j = 0; j < 3; j++) {
    const v4u gv = g4[lane + 64 * j], bv = b4[lane + 64 * j];
    g[j] = make_float4(__uint_as_float(gv.x), __uint_as_float(gv.y), __uint_as_float(gv.z), __uint_as_float(gv.w));
    b[j] = make_float4(__uint_as_float(bv.x), __uint_as_float(bv.y), __uint_as_float(bv.z), __uint_as_float(bv.w));
  }
}

// x of the token at layer 0: fp32(wte[tok]) + fp32(wpe[pos]) (src/gpt2.c:489-499)
__device__ __forceinline__ float embed_x(const Step16Args &a, int tok, int pos, int i) {
  return h2f(gbl(a.wte)[(size_t)tok * E + i]) + h2f(gbl(a.wpe)[(size_t)pos * E + i]);
}

// Q blocks (block gi): rows [48 gi, 48 gi + 48) of q|k|v.  Wave w takes rows
// 6 w + 2 i + (lane >= 32), i < 3; a lane takes 16-byte chunks (lane & 31) +
// 32 c, c < 3, of those rows, so that it reads each chunk of the normalized
// row once for its three rows.
template <bool TRACE>
__device__ void q_loop(const Step16Args &a, int gi, unsigned tag, int tok, float *lds) {
  float *xs = lds;
  const int t = tid_opaque(), lane = t & 63, wave = t >> 6, half = lane >> 5, ln = lane & 31;
  const int pos = ld_uniform(a.attn.pos);
  for (int l = 0; l < a.L; l++) {
    const Step16Layer W = layer_of(a, l);
    const unsigned long long *X = a.xch + (size_t)(l - 1) * kStep16Words;
    unsigned long long *QKV = a.xch + (size_t)l * kStep16Words + kOffQKV;
    // rows n0 + 2 i (lanes 0-31) and n0 + 2 i + 1 (lanes 32-63)
    const int n0 = kQRows * uniform_opaque(gi) + 6 * wave;
    v4u w[3][3];
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const auto src = gbl16(W.wqkv + (size_t)(n0 + 2 * i + half) * E);
#pragma unroll
      for (int c = 0; c < 3; c++) w[i][c] = __builtin_bit_cast(v4u, __builtin_nontemporal_load(src + ln + 32 * c));
    }
    const float bias = gbl(W.bqkv)[n0 + min(lane, 5)];  // lane k < 6 finishes row n0 + k
    float4 g[3], b[3];
    ln_params(W.ln1_g, W.ln1_b, lane, g, b);
    mark<TRACE>(a, l, 0);
    if (l == 0) {
      for (int i = t; i < E; i += kStepThreads) xs[i] = embed_x(a, tok, pos, i);
      __syncthreads();
    } else {
      gather<1>(X, E, tag, xs, a.err);
    }
    mark<TRACE>(a, l, 1);
    float *hs = lds + E * (1 + wave);  // this wave's normalized row
    wave_layer_norm(xs, g, b, a.eps, hs);
    mark<TRACE>(a, l, 2);
    float acc[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < 3; c++) {
      const float *h = hs + 8 * (ln + 32 * c);
#pragma unroll
      for (int i = 0; i < 3; i++) acc[i] = fma8(acc[i], w[i][c], h);
    }
    const float v = finish_rows<3>(acc, lane);
    float *stage = lds + 9 * E;  // the block's 48 rows
    if (lane < 6) stage[6 * wave + lane] = v + bias;
    __syncthreads();
    if (t < kQRows) put_word(QKV + kQRows * uniform_opaque(gi) + t, stage[t], tag);
    published();
    mark<TRACE>(a, l, 3);
  }
}

// F blocks (block gi): fc rows [64 gi, 64 gi + 64), as the Q blocks' rows
// (wave w: rows 8 w + 2 i + (lane >= 32), i < 4).
template <bool TRACE>
__device__ void f_loop(const Step16Args &a, int gi, unsigned tag, float *lds) {
  float *xs = lds;
  const int t = tid_opaque(), lane = t & 63, wave = t >> 6, half = lane >> 5, ln = lane & 31;
  for (int l = 0; l < a.L; l++) {
    const Step16Layer W = layer_of(a, l);
    const unsigned long long *XM = a.xch + (size_t)l * kStep16Words + kOffXM;
    float *FF = a.ffv + ((size_t)(tag & 1u) * a.L + l) * F;
    const int n0 = kFRows * uniform_opaque(gi) + 8 * wave;
    v4u w[4][3];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const auto src = gbl16(W.wfc + (size_t)(n0 + 2 * i + half) * E);
#pragma unroll
      for (int c = 0; c < 3; c++) w[i][c] = __builtin_bit_cast(v4u, __builtin_nontemporal_load(src + ln + 32 * c));
    }
    const float bias = gbl(W.bfc)[n0 + min(lane, 7)];  // lane k < 8 finishes row n0 + k
    float4 g[3], b[3];
    ln_params(W.ln2_g, W.ln2_b, lane, g, b);
    mark<TRACE>(a, l, 12);
    gather<1>(XM, E, tag, xs, a.err);
    mark<TRACE>(a, l, 13);
    float *hs = lds + E * (1 + wave);  // this wave's normalized row
    wave_layer_norm(xs, g, b, a.eps, hs);
    mark<TRACE>(a, l, 14);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < 3; c++) {
      const float *h = hs + 8 * (ln + 32 * c);
#pragma unroll
      for (int i = 0; i < 4; i++) acc[i] = fma8(acc[i], w[i][c], h);
    }
    // the eight GELUs (a double tanh each) on eight lanes at once
    const float v = finish_rows<4>(acc, lane);
    float *stage = lds + 9 * E;  // the block's 64 rows
    if (lane < 8) stage[8 * wave + lane] = gelu_new(v + bias);
    __syncthreads();
    if (t < kFRows) put_plain(FF + kFRows * uniform_opaque(gi) + t, stage[t]);
    published();
    mark<TRACE>(a, l, 15);
  }
}

// O/D blocks (block gi): rows [16 gi, 16 gi + 16) of o and of down; wave w
// takes rows 2 w and 2 w + 1.  o: lanes 0-31 row 2 w, 32-63 row 2 w + 1, 3
// chunks each; down (K = F): every lane both rows, 6 chunks, each GELU
// chunk read once for the two rows.
template <bool TRACE>
__device__ void od_loop(const Step16Args &a, int gi, unsigned tag, int tok, float *lds, float *xown, float *xmown) {
  float *vs = lds;  // the attention output [E], then the GELU outputs [F]
  const int t = tid_opaque(), lane = t & 63, wave = t >> 6, half = lane >> 5, ln = lane & 31;
  const int pos = ld_uniform(a.attn.pos);
  const int r0 = kODRows * uniform_opaque(gi);
  if (t < kODRows) xown[t] = embed_x(a, tok, pos, r0 + t);
  for (int l = 0; l < a.L; l++) {
    const Step16Layer W = layer_of(a, l);
    unsigned long long *Xo = a.xch + (size_t)l * kStep16Words, *XM = Xo + kOffXM;
    const unsigned long long *ATT = Xo + kOffATT;
    const float *FFw = a.ffv + ((size_t)(tag & 1u) * a.L + l) * F;
    const int no = r0 + 2 * wave + half;
    v4u wo[3], wd[2][6];
    {
      const auto so = gbl16(W.wo + (size_t)no * E);
#pragma unroll
      for (int c = 0; c < 3; c++) wo[c] = __builtin_bit_cast(v4u, __builtin_nontemporal_load(so + ln + 32 * c));
#pragma unroll
      for (int r = 0; r < 2; r++) {
        const auto sd = gbl16(W.wd + (size_t)(r0 + 2 * wave + r) * F);
#pragma unroll
        for (int c = 0; c < 6; c++) wd[r][c] = __builtin_bit_cast(v4u, __builtin_nontemporal_load(sd + lane + 64 * c));
      }
    }
    const float bo0 = gbl(W.bo)[r0 + 2 * wave], bo1 = gbl(W.bo)[r0 + 2 * wave + 1];
    const float bd0 = gbl(W.bd)[r0 + 2 * wave], bd1 = gbl(W.bd)[r0 + 2 * wave + 1];

    // ---- o projection + residual ----
    mark<TRACE>(a, l, 7);
    gather<1>(ATT, E, tag, vs, a.err);
    mark<TRACE>(a, l, 8);
    {
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < 3; c++) acc = fma8(acc, wo[c], vs + 8 * (ln + 32 * c));
      const float s = sum16(acc);
      const float o0 = readlane(s, 0) + readlane(s, 16), o1 = readlane(s, 32) + readlane(s, 48);
      if (lane == 0) {
        xmown[2 * wave] = xown[2 * wave] + (o0 + bo0);
        xmown[2 * wave + 1] = xown[2 * wave + 1] + (o1 + bo1);
      }
      __syncthreads();
      if (t < kODRows) put_word(XM + r0 + t, xmown[t], tag);
      published();
    }

    // ---- down projection + residual ----
    mark<TRACE>(a, l, 9);
    gather_plain<(F / 4 + kStepThreads - 1) / kStepThreads>(FFw, F, vs, a.err);
    mark<TRACE>(a, l, 10);
    {
      float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
      for (int c = 0; c < 6; c++) {
        const float *h = vs + 8 * (lane + 64 * c);
        acc0 = fma8(acc0, wd[0][c], h);
        acc1 = fma8(acc1, wd[1][c], h);
      }
      const float s0 = sum16(acc0), s1 = sum16(acc1);
      const float d0 = (readlane(s0, 0) + readlane(s0, 16)) + (readlane(s0, 32) + readlane(s0, 48));
      const float d1 = (readlane(s1, 0) + readlane(s1, 16)) + (readlane(s1, 32) + readlane(s1, 48));
      if (lane == 0) {
        xown[2 * wave] = xmown[2 * wave] + (d0 + bd0);
        xown[2 * wave + 1] = xmown[2 * wave + 1] + (d1 + bd1);
      }
    }
    __syncthreads();
    if (t < kODRows) {
      put_word(Xo + r0 + t, xown[t], tag);
      if (l + 1 == a.L) a.x_out[r0 + t] = xown[t];
    }
    published();
    mark<TRACE>(a, l, 11);
  }
}

// Wait for the 64 q, 64 k and 64 v words of head h (words h*64.., E + h*64..,
// 2E + h*64.. of the q|k|v exchange) and put them into qkv_s[192] (LDS):
// threads t < 96 take one pair each.  Ends with a barrier.
__device__ void gather_head(const unsigned long long *QKV, int h, unsigned tag, float *qkv_s, int *err) {
  const int t = threadIdx.x;
  const __amdgpu_buffer_rsrc_t rs = xch_rsrc(QKV, 3 * E);
  if (t < 96) {
    const int r = t >> 5, w = r * E + h * HD + 2 * (t & 31);
    for (int it = 0;; it++) {
      const v4u v = get_pair(rs, w >> 1);
      if (v.y == tag && v.w == tag) {
        qkv_s[r * HD + 2 * (t & 31)] = __uint_as_float(v.x);
        qkv_s[r * HD + 2 * (t & 31) + 1] = __uint_as_float(v.z);
        break;
      }
      if (it >= kSpin) {
        atomicOr(err, 1);
        break;
      }
      if ((it & 63) == 63 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
}

// Attention of one head for the element slice s (16 of head_dim 64), fp16
// forward (src/gpt2.c:520-556 at M = 1): every position i < n = pos + 1 on
// thread i % 512 (at most kStep16MaxPos positions: two per thread), its K
// row and the slice's 16 V elements in registers, loaded by
// gpt2_attn_prefetch before the q|k|v words arrive (rows [0, pos) are final
// cache rows; the token's own row comes from the new k / v, rounded to fp16
// as the cache stores it).  The softmax's maximum and sum and the products'
// sums over positions are block reductions (fixed trees), not the
// reference's sequential sums: the fp16 forward is compared within a
// tolerance.  The slice-0 block appends the new k / v to the cache.
struct AttnRegs {
  v4u k[2][HD / 8];  // K rows t and t + 512
  v4u v[2][2];       // the slice's 16 V elements of those rows
};

__device__ __forceinline__ void gpt2_attn_prefetch(const AttnArgs &aa, size_t coff, int h, int slice, AttnRegs &r) {
  const int t = threadIdx.x;
  const int pos = ld_uniform(aa.pos), slot = ld_uniform(aa.slot);
  const size_t base = coff + (size_t)slot * aa.C * aa.kv + (size_t)h * HD;
  const auto K = gbl16(aa.kc + base), V = gbl16(aa.vc + base);
  const int last = pos > 0 ? pos - 1 : 0;  // the last cache row (clamp target of the unconditional loads)
  const int rc = aa.kv / 8;                // 16-byte chunks per cache row
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const int i = min(t + kStepThreads * q, last);
#pragma unroll
    for (int c = 0; c < HD / 8; c++) r.k[q][c] = __builtin_bit_cast(v4u, K[(size_t)i * rc + c]);
#pragma unroll
    for (int c = 0; c < 2; c++) r.v[q][c] = __builtin_bit_cast(v4u, V[(size_t)i * rc + 2 * slice + c]);
  }
}

// block reductions over the 8 waves (fixed trees); red: 8 floats of LDS,
// free until every thread has passed the next barrier
__device__ __forceinline__ float block_max8(float v, float *red) {
  v = wave_max_dpp(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7])));
}
__device__ __forceinline__ float wave_sum_f(float v) {
  v = sum16(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}
__device__ __forceinline__ float block_sum8(float v, float *red) {
  v = wave_sum_f(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
}

// qkv: q [64] | new k [64] | new v [64] (LDS); out(i, o) for the slice's 16
// outputs (threads t < 16, i = t); red: 16 + 16 x 512 floats of LDS.  What the next call writes to qkv and red is written after barriers
// that every thread passes only after this call's last reads.
template <class Out>
__device__ void gpt2_attn(const AttnArgs &aa, size_t coff, int h, int slice, const AttnRegs &r, const float *qkv,
                          float *red, Out &&out) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int pos = ld_uniform(aa.pos), slot = ld_uniform(aa.slot), n = pos + 1;
  const float *q = qkv, *kn = qkv + HD, *vn = qkv + 2 * HD;
  if (slice == 0 && t < HD) {  // append the new k / v (fp16) to the cache
    const size_t w = coff + ((size_t)slot * aa.C + pos) * aa.kv + (size_t)h * HD + t;
    aa.kc_w[w] = f2h(kn[t]);
    aa.vc_w[w] = f2h(vn[t]);
  }
  // scores; the token's own row (the new k, rounded to fp16) is scored by the
  // wave that holds its position, one element a lane
  const int il = n - 1, wl = (il % kStepThreads) >> 6;
  float dn = 0.0f;
  if (wave == wl) dn = wave_sum_f(q[lane] * h2f(f2h(kn[lane])));
  float sc[2], mx = -FLT_MAX;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int i = t + kStepThreads * k;
    float d = dn;
    if (i < il) {
      float d0 = 0.0f, d1 = 0.0f;  // two chains: even and odd chunks
#pragma unroll
      for (int c = 0; c < HD / 8; c += 2) {
        d0 = fma8(d0, r.k[k][c], q + 8 * c);
        d1 = fma8(d1, r.k[k][c + 1], q + 8 * c + 8);
      }
      d = d0 + d1;
    }
    sc[k] = (float)((double)d * aa.inv_hd);
    if (i < n) mx = fmaxf(mx, sc[k]);
  }
  mx = block_max8(mx, red);
  float e[2], es = 0.0f;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    e[k] = t + kStepThreads * k < n ? expf(sc[k] - mx) : 0.0f;
    es += e[k];
  }
  const float inv = 1.0f / block_sum8(es, red + 8);
  // products: the slice's 16 elements of p_i v_i for this thread's positions
  float o[16];
#pragma unroll
  for (int d = 0; d < 16; d++) o[d] = 0.0f;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int i = t + kStepThreads * k;
    const float p = e[k] * inv;
    if (i < il) {
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const uint32_t ww[4] = {r.v[k][c].x, r.v[k][c].y, r.v[k][c].z, r.v[k][c].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          o[8 * c + 2 * j] = __builtin_fmaf(p, h2f((uint16_t)(ww[j] & 0xffffu)), o[8 * c + 2 * j]);
          o[8 * c + 2 * j + 1] = __builtin_fmaf(p, h2f((uint16_t)(ww[j] >> 16)), o[8 * c + 2 * j + 1]);
        }
      }
    } else if (i == il) {
#pragma unroll
      for (int d = 0; d < 16; d++) o[d] = __builtin_fmaf(p, h2f(f2h(vn[16 * slice + d])), o[d]);
    }
  }
  // sums over the block through LDS: part[d][t], then thread t sums element
  // d = t / 32 over the threads j = t % 32 + 32 k, and the 32 lanes of its
  // half-wave add up (fixed trees throughout)
  float *part = red + 16;
#pragma unroll
  for (int d = 0; d < 16; d++) part[d * kStepThreads + t] = o[d];
  __syncthreads();
  float v = 0.0f;
#pragma unroll
  for (int k = 0; k < kStepThreads / 32; k++) v += part[(t >> 5) * kStepThreads + (t & 31) + 32 * k];
  v = sum16(v);
  const float v0 = readlane(v, 0) + readlane(v, 16), v1 = readlane(v, 32) + readlane(v, 48);
  // the 16 outputs leave through one store instruction (one 128-byte line):
  // stores to one line from several instructions reach the readers later
  if (lane == 0) {
    red[2 * wave] = v0;
    red[2 * wave + 1] = v1;
  }
  __syncthreads();
  if (t < 16) out(t, red[t]);
}

// A blocks: head h, element slice s of the attention, every layer; the next
// layer's K and V rows go into registers after each layer's attention, while
// the block waits for that layer's q|k|v words.
template <bool TRACE>
__device__ void attention_loop(const Step16Args &a, int head, int slice, unsigned tag, float *lds, float *qkv_s) {
  const int hh = uniform_opaque(head), ss = uniform_opaque(slice);
  AttnRegs r;
  gpt2_attn_prefetch(a.attn, 0, hh, ss, r);
  for (int l = 0; l < a.L; l++) {
    const unsigned long long *QKV = a.xch + (size_t)l * kStep16Words + kOffQKV;
    unsigned long long *att = a.xch + (size_t)l * kStep16Words + kOffATT;
    mark<TRACE>(a, l, 4);
    gather_head(QKV, hh, tag, qkv_s, a.err);
    mark<TRACE>(a, l, 5);
    const int o0 = hh * HD + 16 * ss;
    gpt2_attn(a.attn, a.kv_layer * l, hh, ss, r, qkv_s, lds, [&](int i, float o) { put_word(att + o0 + i, o, tag); });
    published();
    mark<TRACE>(a, l, 6);
    if (l + 1 < a.L) gpt2_attn_prefetch(a.attn, a.kv_layer * (l + 1), hh, ss, r);
  }
}

// The blocks with no role fill the half of ffv that the next step writes
// (tag + 1) with kStepFfEmpty: this step's half was filled during the step
// before, which has ended; the next step starts after this launch ends.
__device__ void ff_rearm(const Step16Args &a, int ib, int nb, unsigned tag) {
  const size_t nq = (size_t)a.L * F / 4;
  v4u *q = reinterpret_cast<v4u *>(a.ffv + (size_t)((tag + 1u) & 1u) * a.L * F);
  const v4u e = {kStepFfEmpty, kStepFfEmpty, kStepFfEmpty, kStepFfEmpty};
  for (size_t i = (size_t)ib * kStepThreads + threadIdx.x; i < nq; i += (size_t)nb * kStepThreads) q[i] = e;
}

template <bool TRACE>
__global__ __launch_bounds__(kStepThreads) void decode_step_gpt2_kernel(Step16Args a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  __shared__ __attribute__((aligned(16))) float qkv_s[3 * HD];
  __shared__ float xown[kODRows], xmown[kODRows];
  const int b = blockIdx.x;
  const unsigned tag = ld_uniform(a.tag);
  const int tok = ld_uniform(a.tok);
  // roles: attention blocks, head h < 8 on XCD h at slots j = b / 8 of 0-3,
  // head 8 + x on XCD x at j 4-7; then, numbered gi in block order, the Q,
  // O/D and F blocks; the rest have nothing to do
  const int xcd = b & 7, j = b >> 3;
  if (j < 4) {
    attention_loop<TRACE>(a, xcd, j, tag, lds, qkv_s);
    return;
  }
  if (j < 8 && xcd < kHeads - 8) {
    attention_loop<TRACE>(a, 8 + xcd, j - 4, tag, lds, qkv_s);
    return;
  }
  // attention blocks with a lower index: the 32 of j < 4, and of j 4-7 the
  // kHeads - 8 of each earlier row (and of this row, whose XCDs below this
  // one's all hold attention blocks)
  const int before = 32 + (j < 8 ? (j - 3) * (kHeads - 8) : 4 * (kHeads - 8));
  const int gi = b - before;
  if (gi < kNQ) q_loop<TRACE>(a, gi, tag, tok, lds);
  else if (gi < kNQ + kNOD) od_loop<TRACE>(a, gi - kNQ, tag, tok, lds, xown, xmown);
  else if (gi < kNQ + kNOD + kNF) f_loop<TRACE>(a, gi - kNQ - kNOD, tag, lds);
  else ff_rearm(a, gi - kNQ - kNOD - kNF, kStepBlocks - kNA - kNQ - kNOD - kNF, tag);
}

}  // namespace

// Q and F blocks: x, the eight waves' normalized rows and the staged rows;
// O/D blocks: the attention output or the GELU outputs; A blocks: the
// reductions' slots and the products' partial sums
size_t decode_step_gpt2_scratch_bytes() {
  const size_t a = (size_t)(9 * E + kFRows > F ? 9 * E + kFRows : F), b = 16 + 16 * (size_t)kStepThreads;
  return (a > b ? a : b) * sizeof(float);
}

hipError_t decode_step_gpt2(const Step16Args &a, size_t lds, bool cooperative, hipStream_t s) {
  Step16Args args = a;
  void *kargs[] = {&args};
  const void *k = a.trace ? reinterpret_cast<const void *>(decode_step_gpt2_kernel<true>)
                          : reinterpret_cast<const void *>(decode_step_gpt2_kernel<false>);
  if (cooperative)
    return hipLaunchCooperativeKernel(k, dim3(kStepBlocks), dim3(kStepThreads), kargs, (unsigned)lds, s);
  return hipLaunchKernel(k, dim3(kStepBlocks), dim3(kStepThreads), kargs, (unsigned)lds, s);
}

}  // namespace ec
