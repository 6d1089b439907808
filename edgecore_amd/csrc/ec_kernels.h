// Host-side launch interface of the gfx950 kernels.  Launchers check
// nothing: callers (runtime.hip) validate shapes and pointers first.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace ec {

// Per-launch timing: when a profiler sets g_launch_ev, the next kernel launch
// records its own start and stop timestamps on these two events
// (hipExtLaunchKernel, the dispatch packet's times) and clears them.  Every
// kernel of the library is launched through klaunch.
extern hipEvent_t g_launch_ev[2];
template <typename F, typename... Args>
inline void klaunch(F kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t s, Args... args) {
  if (g_launch_ev[0]) {
    hipEvent_t e0 = g_launch_ev[0], e1 = g_launch_ev[1];
    g_launch_ev[0] = g_launch_ev[1] = nullptr;
    hipExtLaunchKernelGGL(kernel, grid, block, lds, s, e0, e1, 0, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
  }
}

// GEMV/GEMM epilogues.  `out` has row stride ldo.
enum Epi {
  EPI_STORE = 0,       // out = v                   (+ optional argmax candidates)
  EPI_RESID = 1,       // out = out + v             (residual add, src/gpt2.c:782-784)
  EPI_GELU = 2,        // out = gelu_new(v)         (src/gpt2.c:568)
  EPI_SWIGLU = 3,      // out = silu(v_gate) * v_up (src/gpt2.c:790-791)
  EPI_BIAS = 4,        // out = v + bias            (16-bit linear bias pass, src/gpt2.c:425-429)
  EPI_BIAS_RESID = 5,  // out = out + (v + bias)
  EPI_BIAS_GELU = 6,   // out = gelu_new(v + bias)
};

// Activation prologues of the GEMV kernels (see gemv_impl.h).
enum Pro {
  PRO_I8 = 0,     // int8 rows + per-row scales
  PRO_F32 = 1,    // fp32 rows (16-bit weights)
  PRO_QUANT = 2,  // fp32 rows, quantized per row to int8
  PRO_RMS = 3,    // RMSNorm of fp32 rows (then quantized for int8 weights)
  PRO_LN = 4,     // LayerNorm of fp32 rows (then quantized for int8 weights)
};

struct GemvArgs {
  const void *A;  // [M][lda] int8 (PRO_I8) or fp32
  int lda;
  const float *as;  // PRO_I8 scales [M]
  const float *gamma, *beta;  // norm weights (PRO_RMS / PRO_LN)
  double eps;
  const void *W;   // [N][K] int8 / fp16 / bf16
  const void *W2;  // up weights (EPI_SWIGLU)
  const float *ws, *ws2;  // int8 per-row weight scales or null (1.0)
  const float *bias;      // [N] or null
  float *out;
  int ldo;
  int M, K, N;
  unsigned long long *cand;  // EPI_STORE: [M][gridDim.x] argmax candidate keys, or null
  // skinny int8 GEMM with the activation quantization fused (gemm_i8_skinny_q):
  // A is fp32 [M][lda] and row m's maximum |A| is the largest of the partial
  // maxima pmax[m * np + j], j < np (each >= 0, NaN counted as 0)
  const float *pmax;
  int np;
  // skinny GEMM: when set, each column group's block also writes, per output
  // row m, the largest |v| (NaN as 0) of its outputs to pmax_out[m * np_out +
  // group] (np_out >= the number of column groups)
  float *pmax_out;
  int np_out;
};

// Weight types
enum { WT_I8 = 0, WT_F16 = 1, WT_BF16 = 2 };

// Fused vector kernels; return hipErrorInvalidValue for an (epi, pro) pair
// that is not instantiated.  gemv_vector_ok tells whether a shape can use
// them (16-byte rows, LDS budget); gemv_generic runs any shape with PRO_I8 /
// PRO_F32 and every epilogue, one thread per output.
bool gemv_vector_ok(const GemvArgs &a, int wt, int pro);
hipError_t gemv(const GemvArgs &a, int wt, int epi, int pro, hipStream_t s);
hipError_t gemv_i8_fused(const GemvArgs &a, int epi, int pro, hipStream_t s);
hipError_t gemv_f16_fused(const GemvArgs &a, int epi, int pro, hipStream_t s);
hipError_t gemv_bf16_fused(const GemvArgs &a, int epi, int pro, hipStream_t s);
hipError_t gemv_generic(const GemvArgs &a, int wt, int epi, hipStream_t s);
// int8 matrix-core GEMM (gemm_mfma.hip) for M >= kGemmMinM: int8 A rows with
// scales as (PRO_I8 input), every epilogue but argmax candidates; the floats
// equal the vector GEMV's for the same rows.  gemm_i8_ok: shape and alignment
// (K % 16, lda % 16, 16-byte aligned A / W / W2).
constexpr int kGemmMinM = 16;
bool gemm_i8_ok(const GemvArgs &a, int epi);
hipError_t gemm_i8(const GemvArgs &a, int epi, hipStream_t s);
// the same with the row tile forced: bm 32, 64 or 128 (0: gemm_i8's choice)
hipError_t gemm_i8_tile(const GemvArgs &a, int epi, int bm, hipStream_t s);
// skinny int8 matrix-core GEMM for M <= 32 rows (batched decode): one block
// of wpb waves (0: the library's choice, at most 16) per 16 output columns,
// K split over the waves and summed exactly through LDS; for M <= 16, K >=
// 4096 and few column tiles, K is also split over up to 8 blocks per 64
// columns whose int32 tiles meet in a per-device workspace (launches that
// use it must not overlap on one device).  Same floats as gemm_i8.
hipError_t gemm_i8_skinny(const GemvArgs &a, int epi, int wpb, hipStream_t s);
// the skinny int8 GEMM on fp32 A rows, quantized as their fragments are read
// (src/gpt2.c:446-461: the row scale from the row's maximum |a|, given as
// partial maxima a.pmax / a.np, and the same codes as quant_rows); _ok: K a
// multiple of 16, 16-byte aligned rows, pmax set
bool gemm_i8_skinny_q_ok(const GemvArgs &a, int epi);
hipError_t gemm_i8_skinny_q(const GemvArgs &a, int epi, hipStream_t s);
// 16-bit-weight matrix-core GEMM (gemm_mfma.hip) for M >= kGemmMinM: fp32 A
// rows (lda), fp16 or bf16 weights, every epilogue but argmax candidates,
// no weight scales.  It first splits the rows into w16_parts(wt) 16-bit parts
// in `parts` ([M * parts][ldp] halves, ldp >= K, ldp % 8 == 0, 16-byte
// aligned) with per-row scales in rs[M].  gemm_w16_ok: K % 8, 16-byte aligned
// W / W2.
int w16_parts(int wt);
bool gemm_w16_ok(const GemvArgs &a, int wt, int epi);
hipError_t gemm_w16(const GemvArgs &a, int wt, int epi, uint16_t *parts, int ldp, float *rs, hipStream_t s);
hipError_t gemm_w16_tile(const GemvArgs &a, int wt, int epi, int bm, uint16_t *parts, int ldp, float *rs,
                         hipStream_t s);
// its two launches apart: the split of a.A's rows, then the GEMM on the parts
hipError_t split_rows16(const GemvArgs &a, int wt, uint16_t *parts, int ldp, float *rs, hipStream_t s);
hipError_t gemm_w16_parts(const GemvArgs &a, int wt, int epi, int bm, const uint16_t *parts, int ldp,
                          const float *rs, hipStream_t s);
// grid-size cap of the grid-stride GEMV (set from the CU count at init)
void gemv_set_max_blocks(int n);
int gemv_max_blocks();
// row shape (GS_* of gemv_impl.h) and M tile of the fused kernel for a launch
int gemv_pick_shape(int wt, int K);
int gemv_pick_mt(int M);
// prologue computed by every wave alone (activation rows of at most 1024
// fp32 elements, quantized or normalized; quantized rows of an M tile up to
// 5120): for one row, no block barrier and one LDS copy of the row per wave;
// for an M tile of up to 4 rows, one row per wave and one barrier
inline bool gemv_wave_pro(int pro, int MT, int K) {
  if (MT > 4) return false;
  if (pro == PRO_QUANT && MT > 1 && K <= 5120) return true;
  return K <= 1024 && (pro == PRO_QUANT || pro == PRO_RMS || pro == PRO_LN);
}
// LDS budget per block (device limit), checked by gemv_vector_ok
void gemv_set_max_lds(int bytes);
size_t gemv_lds_bytes(int wt, int pro, int MT, int K);
// number of x-blocks a gemv launch of this shape uses (sizes argmax candidates)
int gemv_grid_x(const GemvArgs &a, int wt, int epi);

// per-row activation quantizer: q[m][k], s[m]
hipError_t quant_rows(const float *in, int ldi, int M, int K, int8_t *q, int ldq, float *s,
                      hipStream_t st);

// LayerNorm (beta != null) or RMSNorm (beta == null) over rows of length E;
// writes fp32 rows to h (ldh) when q == null, else int8 rows + scales.
hipError_t norm_rows(const float *x, int M, int E, const float *gamma, const float *beta,
                     double eps, float *h, int ldh, int8_t *q, int ldq, float *qs,
                     hipStream_t st);

// x[m][:] = wte[tok[m]] (+ wpe[pos[m]])
hipError_t embed(const uint16_t *wte, const uint16_t *wpe, bool bf16, const int *tok,
                 const int *pos, int M, int E, float *x, hipStream_t st);

// Qwen2: rotate q heads and k heads of each token in place (rotate-half, double
// cos/sin table cs[pos][half] as (cos, sin) pairs), then append k and v to the
// fp16 cache at [layer][slot][pos].  GPT-2 (cs == null): append only.
struct KvArgs {
  float *q;  // token row m of q at q + m*ldq
  float *k;  // token row m of k at k + m*ldk
  const float *v;
  int ldq, ldk;  // v shares ldk
  int H, KVH, hd, kv;
  const double2 *cs;
  int half;
  const int *pos, *slot;
  uint16_t *kc, *vc;  // layer base of the caches
  int C;  // positions per slot
  int M;
};
hipError_t rope_kv_append(const KvArgs &a, hipStream_t st);
// reads up to kTouchRanges weight matrices (rows of row16 16-byte words)
// into the L2 of the XCDs whose GEMM blocks read them (see kernels.hip);
// blocks: a multiple of 8
constexpr int kTouchRanges = 6;
struct TouchArgs {
  const uint4 *p[kTouchRanges];
  int rows[kTouchRanges];
  int row16[kTouchRanges];
  int n_ranges;
  unsigned *sink;  // one device word, written only if the loaded xor equals a constant
};
hipError_t touch_ranges(const TouchArgs &a, int blocks, hipStream_t st);
// chained greedy decode: io[0..6] = token, position, slot, tag, error, argmax
// id, ids written; moves the argmax id into the next step's inputs and
// appends it to out[io[6]]; with stamps, the 100 MHz clock at that moment
// into stamps[io[6] + 1] (chain_stamp writes stamps[0] before the first step)
hipError_t step_advance(int *io, int *out, hipStream_t st, unsigned long long *stamps = nullptr);
hipError_t chain_stamp(unsigned long long *t, hipStream_t st);

// causal attention over the fp16 cache for every (head, token), in the
// reference's arithmetic order (see kernels.hip).  With `cs`/`fuse_kv` set it
// also applies RoPE to q and to the token's new k and appends k and v to the
// cache (decode batches whose tokens use distinct slots); otherwise q is
// already rotated and the cache already holds the new position.
struct AttnArgs {
  const float *q;
  int ldq;
  const uint16_t *kc, *vc;  // layer base
  float *out;
  int ldo;
  const int *pos, *slot;
  int H, KVH, hd, kv, C, window;
  double inv_hd;
  int M;
  int max_npos;  // upper bound of pos+1 over the batch (sizes the LDS score array)
  int vtile;     // positions per product tile in LDS (multiple of 4, <= attention_max_vtile)
  // fused RoPE + KV append
  int fuse_kv;
  const float *k, *v;  // token rows of the new k / v (row stride ldk)
  int ldk;
  const double2 *cs;   // RoPE table [pos][half] or null (GPT-2)
  int half;
  uint16_t *kc_w, *vc_w;  // writable views of kc / vc for the append
  int xcd_r;  // set by attention(): query heads per KV group when the launch is XCD-grouped, else 0
  // long decode contexts: scores [M][H][sc_ld] written by a scores pass (one
  // block per token, KV group and chunk of positions) and read by the
  // softmax / sums pass; null to score inside the attention blocks
  float *scores;
  int sc_ld;
  // decode launches (attn_kernel): when set, each block also writes the
  // largest |out| (NaN as 0) of its outputs to pmax[m * np + 4 h + slice]
  // (np >= 4 H), the partial row maxima of the o projection's fused
  // quantization
  float *pmax;
  int np;
};
// positions from which attention() splits a decode launch into the scores
// pass and the softmax / sums pass (when a.scores is set)
constexpr int kAttnSplitMinPos = 512;
hipError_t attention(const AttnArgs &a, hipStream_t st);
// the two launches attention() makes for a long decode context, apart
bool attention_split_ok(const AttnArgs &a);
hipError_t attention_scores(const AttnArgs &a, hipStream_t st);
hipError_t attention_after_scores(const AttnArgs &a, hipStream_t st);

// Persistent decode step (decode_step.hip): all layers of the int8 Qwen2
// forward for one token in one co-resident launch of kStepBlocks blocks of
// kStepThreads threads (d_model 896, head_dim 64, 4 attention blocks per
// query head, up to 8 query heads per KV group, FFN <= 5120).  Blocks exchange
// activations through tagged words (value, step tag) in `xch`, per layer
// [x after the layer: E][x after o: E][attention output: E], and the FFN
// activation through plain words in `ffv` (StepArgs).
constexpr int kStepBlocks = 256, kStepThreads = 512, kStepSlices = 4;
// phase timestamps per block and layer: 0 layer start, 1 x gathered (attention
// blocks), 2 q/k/v rows done, 3 attention done, 4 attention output gathered,
// 5 o done, 6 x_mid gathered, 7 gate/up done, 8 FFN activation gathered,
// 9 down done, 10 x_mid normalized and quantized, 11 x normalized and
// quantized (attention blocks), 12 FFN activation received and quantized,
// 13 attention output received (before its quantization), 14 unused, 15-17
// inside the attention body: scores start, softmax starts, products start
constexpr int kStepEvents = 18;
struct StepLayer {
  const float *ln1_g, *ln2_g;
  const int8_t *wqkv;  // [E + 2 kv][E]: q | k | v rows
  const float *sqkv;
  const int8_t *wo;
  const float *so;
  const int8_t *wg, *wu;
  const float *sg, *su;
  const int8_t *wd;  // [E][F]
  const float *sd;
};
struct StepArgs {
  const StepLayer *layers;  // device array [L]
  const uint16_t *wte;      // fp16 [V][E]
  int L, E, H, KVH, F;
  double eps;
  size_t kv_layer;  // elements per layer of one cache
  const int *tok;   // the token's id (its position and slot: attn.pos / attn.slot)
  const unsigned *tag;          // this step's tag (> 0, new every launch)
  unsigned long long *xch;      // tagged exchange words
  float *x_out;                 // x after the last layer [E] (the LM head's input)
  int *err;                     // set when a wait timed out (results invalid)
  unsigned long long *trace;    // null, or [blocks][L][kStepEvents] phase timestamps
  // the attention body's arguments for layer 0 (kc/vc, kc_w/vc_w at layer
  // 0, fused RoPE + append, M = 1); layer l adds l * kv_layer to the caches
  AttnArgs attn;
  // attention blocks: their fp32 row and int8 codes start this many floats
  // into the dynamic LDS, past the attention body's area (whose K tile is
  // filled for the next layer while they normalize)
  int norm_off;
  // the FFN activation, [2][L][F] floats: step tag t writes and reads half
  // t & 1 (plain values, kStepFfEmpty until written), and re-arms the other
  // half for the next step
  float *ffv;
};
// the FFN words' "not written" pattern: a signaling NaN, which arithmetic never
// produces (its NaN results are quiet)
constexpr uint32_t kStepFfEmpty = 0x7FA5A5A5u;

// The batched decode's layer tail (decode_tail.hip): layer l's o projection,
// RMSNorm, gate/up + SiLU and down (with their residuals), then layer l + 1's
// RMSNorm and q|k|v, for M <= kTailMaxM int8 Qwen2 tokens in one co-resident
// launch of kStepBlocks blocks of kStepThreads threads, between two
// attentions.  Shapes: E % 128 == 0, E <= kTailMaxE, F % 16 == 0,
// 64 <= F <= kTailMaxF, and E/16 + ceil(F/64) + ceil(NQ/16) blocks at most.
constexpr int kTailMaxM = 4, kTailMaxE = 1024, kTailMaxF = 5120;
struct BatchTailArgs {
  const int8_t *wo;                   // layer l: o [E][E], scales, bias (or null)
  const float *so, *bo;
  const float *ln2_g;                 // RMSNorm gamma before the MLP
  const int8_t *wg, *wu;              // gate / up [F][E] and their scales
  const float *sg, *su;
  const int8_t *wd;                   // down [E][F], scales, bias (or null)
  const float *sd, *bd;
  const float *ln1n_g;                // layer l + 1: RMSNorm gamma, q|k|v [NQ][E],
  const int8_t *wqkv;                 //   scales, bias (or null); wqkv null after
  const float *sqkv, *bqkv;           //   the last layer
  const float *att;                   // [M][E] layer l's attention output
  float *x;                           // [M][E] residual stream (in: x, out: x after layer l)
  float *qkv;                         // [M][ldq] layer l + 1's q|k|v
  int ldq, M, E, F, NQ;
  double eps;
  unsigned long long *xch;            // exchange words (batch_tail_xch_words of them)
  unsigned *tag, *done;               // launch tag, blocks finished
  int *err;                           // set when a wait times out
};
size_t batch_tail_lds(int E, int F);
size_t batch_tail_xch_words(int E);
bool batch_tail_shape_ok(int E, int F, int NQ);
hipError_t batch_tail(const BatchTailArgs &a, bool cooperative, hipStream_t s);
// dynamic LDS of the attention blocks' row and codes (d_model E)
constexpr inline size_t step_norm_bytes(int E) { return ((size_t)E * 5 + 15) & ~(size_t)15; }
size_t decode_step_scratch_bytes(int E, int F);
// cooperative: a cooperative launch (every block resident by contract);
// otherwise a plain launch of the same kStepBlocks blocks, one per CU, which the
// step's bounded waits turn into a reported error if a block never ran
hipError_t decode_step(const StepArgs &a, size_t lds, bool cooperative, hipStream_t s);

// Persistent decode step of the fp16 GPT-2 forward (decode_step_gpt2.hip):
// every layer for one token in one launch of kStepBlocks blocks of
// kStepThreads threads, for the GPT-2 small shape (d_model kStep16E, head_dim
// 64, FFN kStep16F).  Exchange words per layer (kStep16Words, tagged as in
// the int8 step): [x: E][x_mid: E][attention output: E][q|k|v: 3 E]; the GELU
// outputs go through ffv as the int8 step's FFN words do.
constexpr int kStep16E = 768, kStep16F = 3072;
constexpr int kStep16MaxPos = 2 * kStepThreads;  // positions the step's attention holds (two per thread)
constexpr size_t kStep16Words = 6 * (size_t)kStep16E;
struct Step16Layer {
  const float *ln1_g, *ln1_b, *ln2_g, *ln2_b;
  const uint16_t *wqkv;  // fp16 [3 E][E]: q | k | v rows
  const float *bqkv;
  const uint16_t *wo;
  const float *bo;
  const uint16_t *wfc;  // fp16 [F][E]
  const float *bfc;
  const uint16_t *wd;  // fp16 [E][F]
  const float *bd;
};
struct Step16Args {
  const Step16Layer *layers;   // device array [L]
  const uint16_t *wte, *wpe;   // fp16 [V][E], [n_ctx][E]
  int L;
  double eps;
  size_t kv_layer;             // elements per layer of one cache
  const int *tok;              // the token's id (position and slot: attn.pos / attn.slot)
  const unsigned *tag;         // this step's tag (> 0, new every launch)
  unsigned long long *xch;     // [L][kStep16Words] tagged exchange words
  float *x_out;                // x after the last layer [E]
  int *err;                    // set when a wait timed out (results invalid)
  unsigned long long *trace;   // null, or [blocks][L][kStepEvents] phase timestamps
  float *ffv;                  // GELU outputs [2][L][kStep16F]: half tag & 1, re-arming the other
  // the attention body's arguments for layer 0 (no RoPE: cs null); layer l
  // adds l * kv_layer to the caches
  AttnArgs attn;
};
// dynamic LDS of the step's non-attention blocks
size_t decode_step_gpt2_scratch_bytes();
hipError_t decode_step_gpt2(const Step16Args &a, size_t lds, bool cooperative, hipStream_t s);
// Prefill attention (attn_prefill.hip): the M tokens are one slot's run of
// consecutive positions whose k / v are already in the cache (fuse_kv 0);
// blocks of 16, 8 or 4 tokens per head.  _ok: head_dim 32/64/128, q rows
// 16-byte aligned, and the LDS of the scores (tokens per block x max_npos
// floats, window-bounded) within max_lds bytes.
bool attention_prefill_ok(const AttnArgs &a, int max_lds);
hipError_t attention_prefill(const AttnArgs &a, int max_lds, hipStream_t st);
// V units (4 positions x 8 elements) per thread held in registers
constexpr int kAttnUnits = 4;
// threads per block of the decode attention body: 512 with element slices
// and for the scored head_dim 128 body, else 256
__host__ __device__ constexpr inline int attn_threads(int hd, int ns, bool scored) {
  return (ns > 1 || (scored && hd == 128)) ? 512 : 256;
}
// head_dim with the 16-byte-load kernel (else the generic one)
__host__ __device__ inline bool attn_vec(int hd, int kv) {
  return (kv & 7) == 0 && (hd == 32 || hd == 64 || hd == 128);
}
// Product tile layout: 16-byte slots (4 positions of one element) per quad
// of positions, padded so that two (hd 64) or four (hd 32) quads written by
// one 16-lane group start on different banks; the element index is swizzled
// by d ^ ((d >> 4) & attn_swz) within its group of 16.  (kv is unused: the
// layout depends on head_dim only.)
__host__ __device__ constexpr inline int attn_pitch(int hd, int kv) {
  (void)kv;
  return (hd == 32 || hd == 64 || hd == 128) ? hd + (hd < 128 ? hd / 16 : 0) : hd;
}
__host__ __device__ constexpr inline int attn_swz(int hd, int kv) {
  (void)kv;
  return hd == 32 ? 1 : hd == 64 ? 3 : hd == 128 ? 7 : 0;
}

// The persistent step's attention body (head_dim 64, element slices of 16)
// keeps the V rows of its slice for the first product tile of T positions
// in LDS (attn_prefetch_v): 16-byte slot ((e * T / 4 + q) * 2 + c) holds
// chunk c of position 4 q + e.  Its offset in bytes from the product area's
// start: past the K tile's capacity (KQ rows of 144 bytes) and the slice
// products' extent (T / 4 + 32 quads of 17 slots).
__host__ __device__ constexpr inline size_t step_vtile_off(int T, int kv) {
  const int kq = (T / 4) * attn_pitch(64, kv) / 9;
  const size_t k = (size_t)(kq < 512 ? kq : 512) * 144, p = ((size_t)T / 4 + 32) * 17 * 16;
  return ((k > p ? k : p) + 255) & ~(size_t)255;
}
// dynamic LDS of a launch: q, new k, new v, max_npos scores, the product tile
size_t attention_lds_bytes(int max_npos, int hd, int vtile);
// largest vtile the kernel accepts for this head_dim / KV row length
int attention_max_vtile(int hd, int kv);

// greedy argmax per row (src/runtime_main.c:215-218 semantics): one block per
// row, or (chunked) per-chunk candidates into cand ([rows][<= cap]) and
// argmax_finalize
hipError_t argmax_rows(const float *logits, int rows, int V, int *out, hipStream_t st);
hipError_t argmax_rows_chunked(const float *logits, int rows, int V, unsigned long long *cand, int cap, int *out,
                               hipStream_t st);
// the chunked form's first launch alone; returns the chunk count in *nc
hipError_t argmax_chunks(const float *logits, int rows, int V, unsigned long long *cand, int cap, int *nc,
                         hipStream_t st);
// final reduction of the LM head's per-block argmax candidates; with
// chain_io (one row), also step_advance's work on chain_io / chain_out /
// chain_t
hipError_t argmax_finalize(const unsigned long long *cand, int ncand, const float *logits,
                           int ldl, int rows, int *out, hipStream_t st, int *chain_io = nullptr,
                           int *chain_out = nullptr, unsigned long long *chain_t = nullptr);

// top_k + 1 largest logits per row for sampling (topk.hip).  topk_select sorts
// chunks of 4096 logits into cand [rows][topk_chunks(V)][top_k + 1] keys and
// nan_flag [rows][topk_chunks(V)]; topk_merge writes vals/idx [rows][top_k + 1]
// (value descending, index ascending) and status [rows] (device pointers).
constexpr int kTopkMax = 128;
int topk_chunks(int V);
bool topk_ok(int V, int top_k);
hipError_t topk_select(const float *L, int rows, int V, int ld, int top_k, unsigned long long *cand,
                       unsigned char *nan_flag, hipStream_t st);
hipError_t topk_merge(const unsigned long long *cand, const unsigned char *nan_flag, int rows, int V, int top_k,
                      float *vals, int *idx, int *status, hipStream_t st);

// elementwise device math (ec_device_math)
enum { MATH_EXPF = 0, MATH_SILU = 1, MATH_GELU = 2, MATH_F32_TO_F16 = 3, MATH_F16_TO_F32 = 4, MATH_QUANT1 = 5, MATH_COPY = 6 };
hipError_t device_math(int op, const void *in, void *out, size_t n, hipStream_t st);

}  // namespace ec
