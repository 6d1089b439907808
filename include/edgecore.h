/*
 * edgecore.h -- C ABI of the MI355X (gfx950) EdgeCore library,
 * libedgecore_hip.so.
 *
 * The kernel and forward entry points keep the names, argument order,
 * layouts and meaning of the reference CPU runtime header (src/edgecore.h of
 * MaheshJakkala/EdgeCore), so a host written against that header links
 * against this library unchanged.  Each declaration names the reference
 * declaration it replaces.  Differences from the reference are listed at the
 * declaration they concern; the two that matter to callers are:
 *
 *   1. GPT2's weight, KV-cache and workspace pointers are DEVICE pointers
 *      (HBM on the GPU the library opened).  A host must not dereference or
 *      memset them; gpt2_kv_reset() replaces the reference driver's memset of
 *      k_cache/v_cache (src/runtime_main.c:312-316).
 *   2. The kernel ABI (gemm_*) takes host pointers exactly like the reference
 *      and stages through device memory; the ec_*_dev variants take device
 *      pointers and run on ec_stream().
 *
 * Everything runs on one GPU (device 0, or $EDGECORE_DEVICE) and one HIP
 * stream per process.  Like the reference, nothing here is re-entrant.
 */
#ifndef EDGECORE_H
#define EDGECORE_H

#include <stddef.h>
#include <stdint.h>
#include <string.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ECM_MAGIC "ECM1\n"

/* architecture ids of the .ecm meta `arch` field (src/edgecore.h:22-24) */
#define ARCH_GPT2 0
#define ARCH_QWEN2 1

/* rope scaling variants, meta `rope_type` (src/edgecore.h:27-28) */
#define ROPE_DEFAULT 0
#define ROPE_YARN 1

/* ------------------------------------------------------------------ */
/* host conversions (src/edgecore.h:34-109)                             */
/* ------------------------------------------------------------------ */

/* binary16 -> binary32, exact (replaces fp16_to_f32, src/edgecore.h:34) */
static inline float fp16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int sh = 0;
            while ((m & 0x400u) == 0) { m <<= 1; sh++; }
            bits = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13) | (m ? 0x400000u : 0u);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even, as the F16C path of the
 * reference (replaces f32_to_fp16, src/edgecore.h:64) */
static inline uint16_t f32_to_fp16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) {
        uint32_t r = ax - 0x38000000u, h = r >> 13, rem = r & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t e = ax >> 23;
    if (e < 102) return (uint16_t)sign;
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u, shift = 126u - e;
    uint32_t h = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* bfloat16 -> fp32 (src/edgecore.h:103) */
static inline float bf16_to_f32(uint16_t b)
{
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ------------------------------------------------------------------ */
/* kernel ABI (src/edgecore.h:115-136, semantics of src/kernels.c:129-168)*/
/* ------------------------------------------------------------------ */

/* C[M][N] = A[M][K] (fp32) . B[N][K]^T (fp16 weights, row-major [out][in]).
 * C is overwritten.  Host pointers.  Replaces gemm_fp16_fp32,
 * src/edgecore.h:119.  fp32 accumulation; the summation order differs from
 * the reference's 8-lane AVX2 order (results agree to fp32 rounding). */
void gemm_fp16_fp32(float *C, const float *A, const uint16_t *B, int M, int K, int N);

/* Same with bfloat16 weights.  Replaces gemm_bf16_fp32, src/edgecore.h:126. */
void gemm_bf16_fp32(float *C, const float *A, const uint16_t *B, int M, int K, int N);

/* C[m][n] = bias[n] + ((float)sum_k A[m][k]*B[n][k] * a_scale[m]) * b_scale[n]
 * with an exact int32 dot.  A int8 [M][K], B int8 [N][K]; b_scale and bias
 * may be NULL (1 and 0), a_scale may not.  Bit-exact with the reference.
 * Replaces gemm_int8, src/edgecore.h:134. */
void gemm_int8(float *C, const int8_t *A, const float *a_scale, const int8_t *B,
               const float *b_scale, const float *bias, int M, int K, int N);

/* Device-pointer variants (additions).  Enqueue on ec_stream() and return 0,
 * or a negative error code (message in ec_last_error()) without launching
 * anything when a shape or pointer is invalid. */
int ec_gemm_fp16_fp32_dev(float *C, const float *A, const uint16_t *B, int M, int K, int N);
int ec_gemm_bf16_fp32_dev(float *C, const float *A, const uint16_t *B, int M, int K, int N);
int ec_gemm_int8_dev(float *C, const int8_t *A, const float *a_scale, const int8_t *B,
                     const float *b_scale, const float *bias, int M, int K, int N);
/* The int8 matrix-core GEMM of the forward's prefill linears with its fused
 * epilogue, v = the gemm_int8 value of each output: epi 0 C = v, 1 C += v
 * (residual, src/gpt2.c:782-784), 2 C = gelu_new(v) (src/gpt2.c:568), 3 C =
 * silu(g) * u with g from B (b_scale, no bias) and u from B2 (b2_scale)
 * (src/gpt2.c:788-791).  bm forces the row tile (32, 64, 128; 0 = the
 * library's choice; 16 = the skinny kernel of batched decode, M <=
 * 32).  K a multiple of 16, A and B 16-byte aligned. */
int ec_gemm_int8_epi_dev(int epi, int bm, float *C, const int8_t *A, const float *a_scale, const int8_t *B,
                         const float *b_scale, const int8_t *B2, const float *b2_scale, const float *bias,
                         int M, int K, int N);
/* The 16-bit-weight matrix-core GEMM of the forward's prefill linears
 * (src/kernels.c:129-151 with the epilogues of src/gpt2.c), v = sum_k
 * A[m][k] * B[n][k] in fp32 from fp16 (wt 1) or bf16 (wt 2) weights: epi 0
 * C = v, 1 C += v, 2 C = gelu_new(v), 3 C = silu(v_B) * v_B2, 4 C = v +
 * bias, 5 C += v + bias, 6 C = gelu_new(v + bias).  The fp32 rows of A are
 * split into 16-bit parts first (2 for fp16 under a per-row power-of-two
 * scale, 3 for bf16), so the sums carry fp32-level accuracy.  bm forces the
 * row tile (32, 64, 128; 16 = the skinny kernel, M <= 32; 0 = the library's
 * choice).  K a multiple of 8, B and B2 16-byte aligned.  ec_gemm_fp16_fp32_dev / ec_gemm_bf16_fp32_dev take
 * this kernel for M >= 16. */
int ec_gemm_w16_epi_dev(int wt, int epi, int bm, float *C, const float *A, const uint16_t *B,
                        const uint16_t *B2, const float *bias, int M, int K, int N);
/* Activation quantizer of the reference linear() (src/gpt2.c:446-461):
 * per row s = max|a|/127 (1 for an all-zero row), q = clamp(rint(a/s)). */
int ec_quantize_rows_dev(const float *in, int M, int K, int8_t *q, float *s);

/* ------------------------------------------------------------------ */
/* tokenizer (src/edgecore.h:142-164)                                   */
/* ------------------------------------------------------------------ */

/* Byte-level BPE over the .ecm tokenizer blobs (src/tokenizer.c:500-1186):
 * GPT-2 (variant 0) or Qwen2 (variant 1) pre-tokenization, merges applied in
 * file order, <|...|> special tokens; tokenizer_encode returns the id count
 * or -1 when max_out is too small; tokenizer_decode returns a malloc'ed
 * string. */
typedef struct {
    char **id_to_token;
    int32_t *byte_to_id;
    int32_t *cp_to_byte;
    uint32_t *merge_l, *merge_r, *merge_m;
    int n_merges;
    int vocab_size;
    int variant;
    int eos_id;
    char **sp_tok;
    uint32_t *sp_len;
    int32_t *sp_id;
    int n_sp;
} Tokenizer;

int tokenizer_load(Tokenizer *t, const void *vocab_blob, size_t vocab_bytes,
                   const void *merges_blob, size_t merges_bytes, int vocab_size, int variant);
void tokenizer_free(Tokenizer *t);
int tokenizer_encode(const Tokenizer *t, const char *text, int *out, int max_out);
char *tokenizer_decode(const Tokenizer *t, const int *ids, int n);

/* ------------------------------------------------------------------ */
/* model (src/edgecore.h:170-273)                                       */
/* ------------------------------------------------------------------ */

/* Per-layer weights (src/edgecore.h:192-211): device pointers. */
struct LayerW {
    const float *ln1_g, *ln1_b;
    const void *attn_w;
    const float *attn_s, *attn_b;
    const void *proj_w;
    const float *proj_s, *proj_b;
    const float *ln2_g, *ln2_b;
    const void *fc_w;
    const float *fc_s, *fc_b;
    const void *fc2_w;
    const float *fc2_s, *fc2_b;

    const void *q_w, *k_w, *v_w, *o_w;
    const float *q_s, *k_s, *v_s, *o_s;
    const float *q_b, *k_b, *v_b, *o_b;
    const void *gate_w, *up_w, *down_w;
    const float *gate_s, *up_s, *down_s;
    const float *gate_b, *up_b, *down_b;
};

/* Field names and meaning follow src/edgecore.h:170-234.  All pointers below
 * `eos_token_id` point into device memory.  Qwen2 q/k/v weights (and scales)
 * are stored back to back, so q_w, k_w and v_w are each still a row-major
 * [out][in] matrix. */
typedef struct {
    char model_name[64];
    int n_layer, n_head, n_embd, n_ctx, vocab;
    int n_kv_head;
    int n_kv_embd;
    int intermediate;
    int head_dim;
    int arch;
    size_t n_params;
    double eps;

    double rope_theta;
    int rope_type;
    double yarn_factor, yarn_orig_max, yarn_attention_factor;
    int sliding_window;
    int tie_word_embeddings;
    int eos_token_id;

    const uint16_t *wte;
    const uint16_t *wpe;

    struct LayerW *lw; /* host array (n_layer) of device pointers */

    const float *lnf_g, *lnf_b;
    const uint16_t *lm_head;

    int precision; /* 0 = int8, 1 = fp16, 2 = bf16 (from the .ecm weight dtype) */

    uint16_t *k_cache, *v_cache; /* device, [n_layer][batch_cap][eff_ctx][n_kv_embd] fp16 */
    int batch_cap;
    int max_ctx;

    float *ws_x, *ws_tmp, *ws_qkv, *ws_attn, *ws_scores; /* device workspaces */
    int8_t *ws_q;
    float *ws_qs;
    size_t ws_q_cols;

    Tokenizer tok;

    void *file_data; /* host mapping of the .ecm file while loading, else NULL */
    size_t file_size;
    int file_mapped;
    /* The library keeps each model's device state in a table keyed by the
     * struct's address, so the layout is the reference's byte for byte: a
     * GPT2 must stay at one address from gpt2_load to gpt2_free. */
} GPT2;

typedef struct {
    char name[128];
    int dtype; /* 0 fp32, 1 fp16, 2 int8, 3 text, 4 bf16 */
    size_t nelems;
    size_t bytes;
    size_t offset;
    size_t dims[4];
    int ndims;
} EcmTensor;

/* Load an .ecm file, upload weights to HBM once and allocate the device KV
 * cache and workspaces for M up to max(eff_ctx, batch_cap).  0 ok, -1 fail
 * (message on stderr).  Replaces gpt2_load, src/edgecore.h:246. */
int gpt2_load(GPT2 *g, const char *path, int batch_cap, int max_ctx);

/* Replaces gpt2_free, src/edgecore.h:247. */
void gpt2_free(GPT2 *g);

/* Forward for M tokens (host tokens/positions/seqs, host logits [M][vocab]);
 * seqs NULL means token m goes to KV slot m.  Replaces gpt2_forward,
 * src/edgecore.h:259 (dispatches to the Qwen2 forward for arch qwen2).
 * Unlike the reference it checks its inputs: a token outside [0, vocab), a
 * position outside [0, eff_ctx) or M above the workspace prints a message
 * and exits with status 1, as the reference does on workspace overflow
 * (src/gpt2.c:442-445). */
void gpt2_forward(GPT2 *g, const int *tokens, const int *positions, const int *seqs,
                  int M, float *logits);

/* Replaces qwen2_forward, src/edgecore.h:263. */
void qwen2_forward(GPT2 *g, const int *tokens, const int *positions, const int *seqs,
                   int M, float *logits);

/* src/edgecore.h:267-269 */
static inline int gpt2_eff_ctx(const GPT2 *g)
{
    return (g->max_ctx > 0 && g->max_ctx < g->n_ctx) ? g->max_ctx : g->n_ctx;
}

/* Parse the .ecm text header and tensor table.  Returns the tensor count, or
 * -1.  Like the reference it fails once the table reaches `max` entries.
 * Replaces ecm_parse, src/edgecore.h:272. */
int ecm_parse(const void *data, size_t size, EcmTensor *out, int max, GPT2 *meta_out);

/* src/edgecore.h:279-280 (defined in the library rather than the driver) */
float peak_rss_gb(void);
double now_sec(void);

/* ------------------------------------------------------------------ */
/* additions                                                            */
/* ------------------------------------------------------------------ */

/* Zero the device KV cache (replaces the driver's memset of k_cache/v_cache,
 * src/runtime_main.c:312-316).  0 ok, <0 error. */
int gpt2_kv_reset(GPT2 *g);

/* Checked forward.  Computes the LM head only for rows [lm_from, M) (lm_from
 * = M skips it; every other result is the same as gpt2_forward).  If logits
 * is non-NULL it receives those rows ([M - lm_from][vocab], host).  If argmax
 * is non-NULL it receives, per row, the greedy token of src/runtime_main.c:
 * 215-218 (first maximum wins), computed on the GPU.  Returns 0 or a negative
 * error code (ec_last_error() has the message); nothing is launched when the
 * inputs are invalid. */
int gpt2_forward_ex(GPT2 *g, const int *tokens, const int *positions, const int *seqs,
                    int M, int lm_from, float *logits, int *argmax);

/* Forward whose LM-head rows [lm_from, M) return their top_k + 1 largest
 * logits instead of all vocab: vals/idx [M - lm_from][top_k + 1] (value
 * descending, index ascending) and status [M - lm_from]: 0 when the row has
 * no NaN and its top_k-th and (top_k+1)-th values differ, so that
 * ec_sample_candidates gives sample_token's token (src/runtime_main.c:213-248);
 * 1 otherwise (take the row from ec_last_logits and use ec_sample_full).
 * 0 < top_k < vocab, top_k <= ec_topk_max().  Replaces copying every logit
 * row back for sampled decoding.  0 or <0. */
int gpt2_forward_topk(GPT2 *g, const int *tokens, const int *positions, const int *seqs,
                      int M, int lm_from, int top_k, float *vals, int *idx, int *status);

/* Largest top_k of gpt2_forward_topk / ec_topk_dev. */
int ec_topk_max(void);

/* Greedy decode of n tokens in slot `slot`: `token` at position `pos` gives
 * out[0], out[0] at pos + 1 gives out[1], ... -- the ids of n single-token
 * gpt2_forward_ex steps with argmax (the greedy branch of the reference's
 * generation loop, src/runtime_main.c:338-348 with temp 0).  No counterpart in
 * the reference, whose loop reads each id on the host: with the persistent
 * decode step the steps are chained on the device (each argmax id becomes
 * the next step's token there) and the ids come back once.  Positions
 * pos..pos+n-1 must lie in the allocated context.  0 or <0. */
int ec_generate_greedy(GPT2 *g, int token, int pos, int slot, int n, int *out);

/* ec_generate_greedy that also reports each step's time in ms (step_ms [n],
 * nullable).  Chained steps take the times from the device: the GPU's
 * constant 100 MHz clock (s_memrealtime) is read by a one-thread kernel just
 * before the first step and by each step's argmax as it writes the id, and
 * step k's time is the difference of stamps k + 1 and k (step 0 includes the
 * launch of the first graph).  Steps run one forward at a time (no
 * persistent step for this model) are timed on the host around each forward.
 * No reference counterpart: the reference driver times each forward with the
 * host clock (src/runtime_main.c:337-342). */
int ec_generate_greedy_timed(GPT2 *g, int token, int pos, int slot, int n, int *out, double *step_ms);

/* Row `row` (counted from lm_from, < the LM-head chunk of the last forward,
 * which holds at least batch_cap rows) of the last forward's logits, into out
 * [vocab] (host).  0 or <0. */
int ec_last_logits(GPT2 *g, int row, float *out);

/* The device top-k selection alone: rows x vocab fp32 logits in device memory
 * (row stride ld) -> vals/idx/status as in gpt2_forward_topk (host). */
int ec_topk_dev(const float *logits, int rows, int vocab, int ld, int top_k, float *vals, int *idx,
                int *status);
/* ec_topk_dev without allocating: no reference counterpart; for callers that
 * cannot allocate device memory (code under stream capture, serving loops,
 * harnesses that forbid hipMalloc).  Its scratch is a 4 MiB device array of
 * the library, one per GPU for the life of the process; a call needing more
 * (about 40 KB per row at vocab 151936 and top_k 128) fails with a message.
 * Calls overlapping on one GPU share that array and race.  A first call into
 * the library may be this one: it then sets up only the device (no stream,
 * event or allocation) and runs on the null stream. */
int ec_topk_dev_noalloc(const float *logits, int rows, int vocab, int ld, int top_k, float *vals, int *idx,
                        int *status);

/* The forward's causal attention alone, on device memory, for checking it on
 * its own: head h of token m attends over positions [lo, pos[m]] of cache slot
 * slot[m] (lo = max(0, pos[m] - window + 1) when window > 0, else 0) with the
 * arithmetic of src/gpt2.c:527-557 (GPT-2, KVH = H) and 744-777 (Qwen2 GQA:
 * KV head h * KVH / H).  q [M][H*hd] fp32 (row stride ldq, 16-byte aligned
 * rows for path 0), kc / vc fp16 caches [nslots][C][KVH*hd], out [M][H*hd]
 * fp32 (row stride ldo); pos and slot are host arrays [M].  path 0: the
 * prefill kernel (one slot's consecutive positions pos[0] + m, as the forward
 * runs a prompt); path 1: the per-token kernel (any positions and slots, as
 * the forward runs decode steps); path 2: the forward's long-context decode
 * form (from 512 positions, head_dim 128; otherwise path 1): a scores pass
 * with one block per token, KV group and 256 positions, then the per-token
 * kernel's softmax and sums on those scores.  0 or <0. */
int ec_attention_dev(const float *q, int ldq, const uint16_t *kc, const uint16_t *vc, int nslots, int C, int H,
                     int KVH, int hd, const int *pos, const int *slot, int M, int window, float *out, int ldo,
                     int path);

/* Sampling of src/runtime_main.c:205-248.  ec_rng_next: the driver's LCG
 * (state advances, returns the top 31 bits).  ec_sample_full: sample_token on
 * a whole row (temp <= 0: greedy).  ec_sample_candidates: the same token from
 * the row's top_k + 1 candidates of a status-0 row; -1 when the arguments do
 * not allow it (temp <= 0, top_k outside (0, vocab), too few candidates). */
unsigned ec_rng_next(unsigned long long *state);
int ec_sample_full(const float *logits, int vocab, float temp, int top_k, unsigned long long *state);
int ec_sample_candidates(const float *vals, const int *idx, int ncand, int vocab, float temp, int top_k,
                         unsigned long long *state);

/* sizeof(GPT2) as compiled into the library (lets foreign-function hosts
 * check their mirror of the struct). */
size_t ec_gpt2_sizeof(void);

/* Error message of the last failing call on this thread ("" if none). */
const char *ec_last_error(void);

/* Opens the GPU on first use; 0 ok.  Every other entry point calls it
 * (ec_topk_dev_noalloc only its part that creates and allocates nothing). */
int ec_init(void);

/* Releases the library's streams, events and host-ABI staging buffers once
 * every model is freed; 0 ok, <0 while a model is still loaded.  The next
 * call sets the library up again.  No reference counterpart: the driver calls
 * it before it exits, so that nothing is left to the HIP runtime's teardown. */
int ec_release(void);

/* Device and pinned-host allocations the library has made so far (every one
 * goes through one counting helper); for tests of the no-allocation entry
 * point. */
long ec_alloc_count(void);

/* One-line JSON description of the GPU: name, gcnArchName, CUs, HBM bytes. */
int ec_device_info(char *buf, int len);

/* The library's HIP stream (hipStream_t) and a blocking wait on it. */
void *ec_stream(void);
int ec_sync(void);

/* Device memory helpers for hosts without a HIP runtime of their own. */
void *ec_dev_alloc(size_t bytes);
int ec_dev_free(void *p);
int ec_memcpy_h2d(void *dst, const void *src, size_t bytes);
int ec_memcpy_d2h(void *dst, const void *src, size_t bytes);
int ec_memset_dev(void *dst, int value, size_t bytes);

/* Per-kernel timing.  While enabled, every launch of a kernel whose family
 * name equals `filter` ("" = all) records its start and stop time on HIP
 * events (hipExtLaunchKernel: the dispatch's own timestamps, on the stream the
 * kernel runs on).  ec_prof_stop synchronises and writes a JSON
 * array of {"kernel", "launches", "total_us", "avg_us", "bytes_per_launch",
 * "gbps"} (bytes are the algorithmic bytes of each launch) into buf and
 * returns its length, or a negative error code. */
int ec_prof_start(const char *filter);
int ec_prof_stop(char *buf, int len);

/* Elementwise device arithmetic on n elements of device memory, for checking
 * it against the host: op 0 expf (the reference's expf), 1 SiLU
 * (src/gpt2.c:587-590), 2 GELU (src/gpt2.c:393-396), 3 fp32 -> fp16 bits
 * (round to nearest even), 4 fp16 bits -> fp32, 5 int8 quantization with
 * scale 1 (src/gpt2.c:456-459), 6 copy (16-byte loads and stores when n is a
 * multiple of 4 and both pointers are 16-byte aligned: the reference kernel
 * for HBM traffic counters).  fp32 in/out except as noted.  0 or <0. */
int ec_device_math(int op, const void *in, void *out, size_t n);

/* Diagnostics of the persistent decode step of one-token int8 Qwen2
 * forwards (a model loaded with EDGECORE_STEP_TRACE=1): the last step's
 * s_memrealtime (100 MHz) stamps at every block's phase boundaries,
 * [256 blocks][n_layer][10 events] (see ec_kernels.h, kStepEvents).
 * Returns the word count or <0. */
int ec_step_trace(GPT2 *g, unsigned long long *out, size_t n);

/* int8 weight packing of edgecore/ecm.py:50-59 (float64 max|w|/127, zero row
 * -> scale 1, round half to even, clip; a row holding NaN gets scale NaN and
 * codes -128, as numpy gives), used by the synthetic generator. */
void ec_quantize_int8_symmetric(const float *w, int rows, int cols, int8_t *q, float *scales);

/* fp32 -> bfloat16 bits of edgecore/ecm.py:27-41 (round to nearest even, NaN
 * -> 0x7fc0), used by the synthetic generator for bf16 weights. */
uint16_t ec_f32_to_bf16(float f);

#ifdef __cplusplus
}
#endif

#endif /* EDGECORE_H */
