/*
 * EdgeCore CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference CPU arithmetic for the transformer
 * forward hot path (src/kernels.c, src/gpt2.c, src/edgecore.h,
 * edgecore/ecm.py of the reference).  It is the checker the GPU library is
 * compared against and the CPU baseline that bench.py times.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product (libedgecore_hip.so, edgecore-runtime) never links or calls it.
 *
 * Every function cites the reference file:line it follows.  Parity status of
 * each function (what pins it) is recorded at the top of ec_oracle.c.
 */
#ifndef EC_ORACLE_H
#define EC_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions (src/edgecore.h:34-109, F16C path) ---- */
float    or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
float    or_bf16_to_f32(uint16_t b);
/* float32 -> bfloat16 RNE as edgecore/ecm.py:27-41 (NaN -> 0x7FC0) */
uint16_t or_f32_to_bf16(float f);

/* ---- weight packing (edgecore/ecm.py:50-59) ---- */
void or_quantize_int8_symmetric(const float *w, int rows, int cols,
                                int8_t *q, float *scales);

/* ---- activation quantizer inside linear() (src/gpt2.c:446-461) ---- */
void or_quantize_rows(const float *in, int M, int K, int8_t *q, float *s);

/* ---- GEMMs (src/kernels.c:129-168) ---- */
void or_gemm_fp16_fp32(float *C, const float *A, const uint16_t *B,
                       int M, int K, int N);
void or_gemm_bf16_fp32(float *C, const float *A, const uint16_t *B,
                       int M, int K, int N);
void or_gemm_int8(float *C, const int8_t *A, const float *a_scale,
                  const int8_t *B, const float *b_scale, const float *bias,
                  int M, int K, int N);

/* ---- row ops (src/gpt2.c:393-414, 587-604) ---- */
void  or_layernorm_rows(float *out, const float *in, const float *gamma,
                        const float *beta, int M, int N, double eps);
void  or_rmsnorm_rows(float *out, const float *in, const float *gamma,
                      int M, int N, double eps);
float or_gelu_new(float x);
float or_silu(float x);
/* RoPE inverse frequencies incl. the YaRN branch (src/gpt2.c:608-644) */
void  or_rope_inv_freq(double *inv_freq, int half, double theta, int yarn,
                       double yarn_factor, double yarn_orig_max);

/* ---- elementwise reference arithmetic over arrays (op codes of
 * ec_device_math in the library header) ---- */
void or_map(int op, const void *in, void *out, size_t n);

/* ---- whole model (src/gpt2.c:161-366 load, 470-805 forward) ---- */
typedef struct OrModel OrModel;

OrModel *or_load(const char *path, int batch_cap, int max_ctx);
void     or_free(OrModel *m);
/* zero the KV cache (what src/runtime_main.c:312-316 does with memset) */
void     or_kv_reset(OrModel *m);
int      or_vocab(const OrModel *m);
int      or_eff_ctx(const OrModel *m);
int      or_precision(const OrModel *m);   /* 0 int8, 1 fp16, 2 bf16 */
int      or_arch(const OrModel *m);        /* 0 gpt2, 1 qwen2 */
/* gpt2_forward/qwen2_forward semantics; logits [M][V].  Returns 0, or -1
 * when a position/slot/token is out of range or M exceeds the workspace. */
int      or_forward(OrModel *m, const int *tokens, const int *positions,
                    const int *seqs, int M, float *logits);
/* Attention rows alone on caller-given fp16 caches [nslots][C][KVH*hd]:
 * for each m in rows[0..nrows), every head, the forward's per-row attention
 * (src/gpt2.c:527-557, 744-777) over positions [lo, pos[m]] of slot slot[m];
 * q / out rows of stride ldq / ldo.  0 or -1. */
int or_attention_rows(const float *q, int ldq, const uint16_t *kc, const uint16_t *vc, int nslots, int C,
                      int H, int KVH, int hd, const int *pos, const int *slot, const int *rows, int nrows,
                      int window, float *out, int ldo);
/* or_forward with the LM head only for rows [lm_from, M) into logits
 * [M - lm_from][V]; the rest (KV cache included) unchanged.  0 or -1. */
int      or_forward_from(OrModel *m, const int *tokens, const int *positions,
                         const int *seqs, int M, int lm_from, float *logits);
/* greedy argmax, first maximum wins (src/runtime_main.c:213-219) */
int      or_argmax(const float *logits, int vocab);
/* gen_and_measure at batch 1, temp 0 (src/runtime_main.c:293-362): prefill
 * positions 0..n-1, then feed the last prompt token at position n and keep
 * the argmax.  out_ids gets n + n_gen ids.  step_logits (optional) gets the
 * [n_gen][V] logits of each decode step. */
int      or_generate(OrModel *m, const int *prompt, int n, int n_gen,
                     int *out_ids, float *step_logits);

#ifdef __cplusplus
}
#endif
#endif
