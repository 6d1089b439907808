// Host-side launch interface of the gfx950 kernels (kernels.hip).  Every
// launcher checks nothing: callers (runtime.hip) validate shapes first.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ec {

// GEMV/GEMM epilogues.  `out` has row stride ldo.
enum Epi {
  EPI_STORE = 0,       // out = v
  EPI_RESID = 1,       // out = out + v            (residual add, src/gpt2.c:782-784)
  EPI_GELU = 2,        // out = gelu_new(v)        (src/gpt2.c:568)
  EPI_SWIGLU = 3,      // out = silu(v_gate) * v_up (src/gpt2.c:790-791)
  EPI_BIAS = 4,        // out = v + bias            (fp16/bf16 linear bias pass, src/gpt2.c:425-429)
  EPI_BIAS_RESID = 5,  // out = out + (v + bias)
  EPI_BIAS_GELU = 6,   // out = gelu_new(v + bias)
};

struct GemvI8Args {
  const int8_t *A;  // [M][lda] int8 activations
  int lda;
  const float *as;  // [M] activation scales
  const int8_t *W;  // [N][K]
  const float *ws;  // [N] or null (1.0)
  const float *bias;  // [N] or null (0.0)
  const int8_t *W2;  // up weights for EPI_SWIGLU
  const float *ws2;
  float *out;
  int ldo;
  int M, K, N;
};

struct GemvW16Args {
  const float *A;  // [M][lda] fp32 activations
  int lda;
  const uint16_t *W;  // [N][K] fp16 or bf16
  const float *bias;  // [N] or null
  const uint16_t *W2;  // up weights for EPI_SWIGLU
  float *out;
  int ldo;
  int M, K, N;
};

// The vector kernels need K % 16 == 0 (int8) / K % 8 == 0 (16-bit) and
// 16-byte aligned rows; gemv_i8 / gemv_w16 fall back to the one-thread-per-
// output gemm_*_generic kernels (same epilogues) for anything else.
bool gemv_i8_vector_ok(const GemvI8Args &a);
bool gemv_w16_vector_ok(const GemvW16Args &a);
hipError_t gemv_i8(const GemvI8Args &a, int epi, hipStream_t s);
hipError_t gemv_w16(const GemvW16Args &a, int epi, bool bf16, hipStream_t s);
hipError_t gemm_i8_generic(const GemvI8Args &a, int epi, hipStream_t s);
hipError_t gemm_w16_generic(const GemvW16Args &a, int epi, bool bf16, hipStream_t s);

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

// causal attention over the fp16 cache for every (head, token)
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
  int max_npos;  // upper bound of pos+1 over the batch (sizes LDS)
};
hipError_t attention(const AttnArgs &a, hipStream_t st);
size_t attention_lds_bytes(int max_npos, int hd);

// greedy argmax per row (src/runtime_main.c:215-218 semantics)
hipError_t argmax_rows(const float *logits, int rows, int V, int *out, hipStream_t st);

}  // namespace ec
