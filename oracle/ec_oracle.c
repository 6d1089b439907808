/*
 * EdgeCore CPU oracle -- TEST INFRASTRUCTURE ONLY (see ec_oracle.h).
 *
 * Restates, in plain C11, the arithmetic of the reference CPU path so that the
 * MI355X library can be checked against it on the same seeded inputs.  Built
 * with -std=c11 (which implies -ffp-contract=off, exactly like the reference
 * Makefile:3), so every a*b+c below is a rounded multiply followed by a
 * rounded add unless fmaf() is written out, which is where the reference uses
 * _mm256_fmadd_ps.
 *
 * Parity pins (tests/test_oracle.py, tests/golden/):
 *   or_f32_to_f16 / or_f16_to_f32 : exhaustive vs the host F16C instruction
 *                                   (or_check_f16c below) + the reference build
 *   or_quantize_int8_symmetric     : tests/golden/packer.npz, whose codes come
 *                                   from exact rational arithmetic on the
 *                                   float64 definition (adversarial quotients
 *                                   a float32 packer rounds differently, ties,
 *                                   +-maxabs, zero/NaN/inf/subnormal rows)
 *   or_f32_to_bf16                 : all 2^32 inputs against round-to-nearest-
 *                                   even as a distance comparison
 *   or_quantize_rows               : closed-form ties / clamp cases + the
 *                                   reference build (through gpt2_forward)
 *   or_gemm_int8                   : brute-force int64 dot + adversarial
 *                                   (-128/127) rows + reference build vectors
 *                                   (tests/golden/kernels.npz)
 *   or_gemm_fp16_fp32 / bf16       : float64 brute force within gamma_K bound +
 *                                   bit-exact vs the reference build vectors
 *   norms, RoPE, attention, GELU,  : closed forms (constant row, pos 0 identity,
 *   SiLU, forward                    single-position attention = V row) + the
 *                                   reference build end to end (bit-exact
 *                                   logits and greedy tokens on seeded models)
 */
#define _GNU_SOURCE
#include "ec_oracle.h"

#include <fcntl.h>
#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__F16C__)
#include <immintrin.h>
#endif

/* ------------------------------------------------------------------ */
/* conversions                                                          */
/* ------------------------------------------------------------------ */

/* IEEE binary16 -> binary32, exact.  Follows the F16C path of
 * src/edgecore.h:34-38 (NaNs come back quiet, payload kept). */
float or_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int sh = 0;
            while ((m & 0x400u) == 0) { m <<= 1; sh++; }
            m &= 0x3ffu;
            bits = sign | ((uint32_t)(113 - sh) << 23) | (m << 13);
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

/* binary32 -> binary16 with round-to-nearest-even, overflow to infinity,
 * quiet NaN with the top payload bits.  Follows src/edgecore.h:64-68
 * (_mm_cvtps_ph(v, 0)); the reference's scalar fallback at :69-99 truncates
 * and is not what its AVX2 builds run. */
uint16_t or_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) /* NaN */
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) /* >= 65520 (incl. inf) rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) { /* result is a normal fp16 */
        uint32_t r = ax - 0x38000000u; /* rebias exponent by (127 - 15) << 23 */
        uint32_t h = r >> 13, rem = r & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    /* subnormal fp16 (or zero): value / 2^-24, rounded to nearest even */
    uint32_t e = ax >> 23;
    if (e < 102) return (uint16_t)sign; /* < 2^-25: rounds to zero */
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e; /* 14 .. 24 */
    uint32_t h = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float or_bf16_to_f32(uint16_t b)
{
    uint32_t bits = (uint32_t)b << 16; /* src/edgecore.h:103-109 */
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_f32_to_bf16(float f)
{
    uint32_t x; /* edgecore/ecm.py:27-41 */
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    uint64_t r = ((uint64_t)x + 0x7fffu + ((x >> 16) & 1u)) >> 16;
    return (uint16_t)r;
}

#if defined(__F16C__)
/* Exhaustive check of or_f32_to_f16 against the F16C instruction over the
 * input bit patterns [lo, hi).  Returns the number of mismatches. */
uint64_t or_check_f16c(uint32_t lo, uint32_t hi)
{
    uint64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t i = lo; i < (int64_t)hi; i++) {
        uint32_t b = (uint32_t)i;
        float f;
        memcpy(&f, &b, 4);
        uint16_t ref = (uint16_t)_mm_extract_epi16(_mm_cvtps_ph(_mm_set_ss(f), 0), 0);
        if (ref != or_f32_to_f16(f)) bad++;
    }
    return bad;
}

/* all 65536 fp16 -> fp32 against _mm_cvtph_ps (NaNs compared as NaN) */
uint64_t or_check_f16c_widen(void)
{
    uint64_t bad = 0;
    for (uint32_t h = 0; h < 65536u; h++) {
        float ref = _mm_cvtss_f32(_mm_cvtph_ps(_mm_cvtsi32_si128((int)h)));
        float got = or_f16_to_f32((uint16_t)h);
        if (isnan(ref) && isnan(got)) continue;
        if (memcmp(&ref, &got, 4) != 0) bad++;
    }
    return bad;
}
#endif

/* ------------------------------------------------------------------ */
/* quantizers                                                           */
/* ------------------------------------------------------------------ */

/* edgecore/ecm.py:50-59: float64 maxabs/127, zero scale -> 1.0, rint (ties
 * to even), clip to [-128, 127], scale stored as float32. */
void or_quantize_int8_symmetric(const float *w, int rows, int cols,
                                int8_t *q, float *scales)
{
    for (int r = 0; r < rows; r++) {
        const float *row = w + (size_t)r * cols;
        double maxabs = 0.0;
        for (int c = 0; c < cols; c++) {
            double a = fabs((double)row[c]);
            if (isnan(a)) maxabs = a; /* numpy's max propagates NaN */
            else if (a > maxabs) maxabs = a;
        }
        double s = maxabs / 127.0;
        if (s == 0.0) s = 1.0;
        for (int c = 0; c < cols; c++) {
            double v = rint((double)row[c] / s);
            /* numpy's float64 -> int32 cast of NaN is INT32_MIN on x86-64;
             * np.clip then gives -128 */
            if (isnan(v)) v = -128.0;
            if (v > 127.0) v = 127.0;
            if (v < -128.0) v = -128.0;
            q[(size_t)r * cols + c] = (int8_t)(int)v;
        }
        scales[r] = (float)s;
    }
}

/* src/gpt2.c:446-461: per-row float max|a|, s = max/127.0f (1.0f for an
 * all-zero row), q = clamp(lrintf(a / s)). */
void or_quantize_rows(const float *in, int M, int K, int8_t *q, float *s)
{
    for (int m = 0; m < M; m++) {
        const float *row = in + (size_t)m * K;
        float maxa = 0.0f;
        for (int k = 0; k < K; k++) {
            float a = fabsf(row[k]);
            if (a > maxa) maxa = a;
        }
        float sc = maxa > 0.0f ? maxa / 127.0f : 1.0f;
        s[m] = sc;
        for (int k = 0; k < K; k++) {
            long v = lrintf(row[k] / sc);
            if (v > 127) v = 127;
            if (v < -128) v = -128;
            q[(size_t)m * K + k] = (int8_t)v;
        }
    }
}

/* ------------------------------------------------------------------ */
/* GEMMs                                                                */
/* ------------------------------------------------------------------ */

static float g_f16_lut[65536];
static int g_f16_lut_ready;

static void f16_lut_init(void)
{
    if (g_f16_lut_ready) return;
    for (uint32_t h = 0; h < 65536u; h++) g_f16_lut[h] = or_f16_to_f32((uint16_t)h);
    g_f16_lut_ready = 1;
}

/* The reference dot (src/kernels.c:29-42 with hsum_ps at :5-15): eight fp32
 * FMA accumulators, lane j summing k = j (mod 8) over the largest multiple of
 * 8, reduced as ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)), then a scalar tail of
 * separate multiplies and adds. */
static inline float dot_w16(const float *a, const uint16_t *b, int K, int bf16)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int k = 0;
    for (; k + 8 <= K; k += 8) {
        for (int j = 0; j < 8; j++) {
            float bv = bf16 ? or_bf16_to_f32(b[k + j]) : g_f16_lut[b[k + j]];
            acc[j] = fmaf(a[k + j], bv, acc[j]);
        }
    }
    float res = ((acc[0] + acc[4]) + (acc[1] + acc[5])) +
                ((acc[2] + acc[6]) + (acc[3] + acc[7]));
    for (; k < K; k++) {
        float bv = bf16 ? or_bf16_to_f32(b[k]) : g_f16_lut[b[k]];
        float p = a[k] * bv;
        res = res + p;
    }
    return res;
}

static void gemm_w16(float *C, const float *A, const uint16_t *B, int M, int K,
                     int N, int bf16)
{
    f16_lut_init();
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        const uint16_t *brow = B + (size_t)n * K;
        for (int m = 0; m < M; m++)
            C[(size_t)m * N + n] = dot_w16(A + (size_t)m * K, brow, K, bf16);
    }
}

/* src/kernels.c:129-139 */
void or_gemm_fp16_fp32(float *C, const float *A, const uint16_t *B, int M,
                       int K, int N)
{
    gemm_w16(C, A, B, M, K, N, 0);
}

/* src/kernels.c:141-151 */
void or_gemm_bf16_fp32(float *C, const float *A, const uint16_t *B, int M,
                       int K, int N)
{
    gemm_w16(C, A, B, M, K, N, 1);
}

/* src/kernels.c:153-168: exact int32 dot (the AVX2 decomposition at :66-102
 * computes the exact sum), epilogue bias + ((float)dot * a_scale) * b_scale. */
void or_gemm_int8(float *C, const int8_t *A, const float *a_scale,
                  const int8_t *B, const float *b_scale, const float *bias,
                  int M, int K, int N)
{
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        const int8_t *brow = B + (size_t)n * K;
        float bs = b_scale ? b_scale[n] : 1.0f;
        float bv = bias ? bias[n] : 0.0f;
        for (int m = 0; m < M; m++) {
            const int8_t *arow = A + (size_t)m * K;
            int32_t dot = 0;
            for (int k = 0; k < K; k++) dot += (int32_t)arow[k] * (int32_t)brow[k];
            float t = (float)dot * a_scale[m];
            t = t * bs;
            C[(size_t)m * N + n] = bv + t;
        }
    }
}

/* ------------------------------------------------------------------ */
/* row ops                                                              */
/* ------------------------------------------------------------------ */

/* src/gpt2.c:398-414 */
void or_layernorm_rows(float *out, const float *in, const float *gamma,
                       const float *beta, int M, int N, double eps)
{
    for (int m = 0; m < M; m++) {
        const float *row = in + (size_t)m * N;
        float *o = out + (size_t)m * N;
        double mean = 0.0;
        for (int i = 0; i < N; i++) mean += row[i];
        mean /= N;
        double var = 0.0;
        for (int i = 0; i < N; i++) {
            double d = row[i] - mean;
            var += d * d;
        }
        var /= N;
        double rstd = 1.0 / sqrt(var + eps);
        for (int i = 0; i < N; i++) {
            float t = (float)(((double)row[i] - mean) * rstd);
            t = t * gamma[i];
            o[i] = t + beta[i];
        }
    }
}

/* src/gpt2.c:592-604 */
void or_rmsnorm_rows(float *out, const float *in, const float *gamma, int M,
                     int N, double eps)
{
    for (int m = 0; m < M; m++) {
        const float *row = in + (size_t)m * N;
        float *o = out + (size_t)m * N;
        double ms = 0.0;
        for (int i = 0; i < N; i++) ms += (double)row[i] * row[i];
        double rstd = 1.0 / sqrt(ms / N + eps);
        for (int i = 0; i < N; i++) {
            float t = (float)((double)row[i] * rstd);
            o[i] = t * gamma[i];
        }
    }
}

/* src/gpt2.c:393-396 */
float or_gelu_new(float x)
{
    float x3 = ((0.044715f * x) * x) * x;
    float u = 0.7978845608028654f * (x + x3);
    float hx = 0.5f * x;
    return hx * (1.0f + tanhf(u));
}

/* src/gpt2.c:587-590 */
float or_silu(float x)
{
    return x / (1.0f + expf(-x));
}

/* src/gpt2.c:608-644 (the nested corr_dim at :625-627 is inlined) */
void or_rope_inv_freq(double *inv_freq, int half, double theta, int yarn,
                      double yarn_factor, double yarn_orig_max)
{
    int dim = 2 * half;
    double inv_base = 1.0 / theta;
    for (int i = 0; i < half; i++)
        inv_freq[i] = pow(inv_base, (double)(2 * i) / (double)dim);
    if (!yarn) return;
    double pi2 = 6.28318530717958647692;
    double logbase = log(theta);
    double lo = floor((double)dim * log(yarn_orig_max / (32.0 * pi2)) / (2.0 * logbase));
    double hi = ceil((double)dim * log(yarn_orig_max / (1.0 * pi2)) / (2.0 * logbase));
    if (lo < 0.0) lo = 0.0;
    if (hi > (double)(dim - 1)) hi = (double)(dim - 1);
    double span = hi - lo;
    if (span < 1.0) span = 1.0;
    for (int i = 0; i < half; i++) {
        double ramp = ((double)i - lo) / span;
        if (ramp < 0.0) ramp = 0.0;
        if (ramp > 1.0) ramp = 1.0;
        double extrap = inv_freq[i];
        double interp = inv_freq[i] / yarn_factor;
        inv_freq[i] = interp * ramp + extrap * (1.0 - ramp);
    }
}

/* Elementwise reference arithmetic over arrays, op codes as ec_device_math:
 * 0 expf, 1 SiLU, 2 GELU, 3 fp32 -> fp16 bits, 4 fp16 bits -> fp32,
 * 5 lrintf quantization with scale 1 clamped to [-128, 127]. */
void or_map(int op, const void *in, void *out, size_t n)
{
    for (size_t i = 0; i < n; i++) {
        if (op == 4) {
            ((float *)out)[i] = or_f16_to_f32(((const uint16_t *)in)[i]);
            continue;
        }
        const float x = ((const float *)in)[i];
        switch (op) {
        case 0: ((float *)out)[i] = expf(x); break;
        case 1: ((float *)out)[i] = or_silu(x); break;
        case 2: ((float *)out)[i] = or_gelu_new(x); break;
        case 3: ((uint16_t *)out)[i] = or_f32_to_f16(x); break;
        case 5: {
            long v = lrintf(x);
            ((int8_t *)out)[i] = (int8_t)(v > 127 ? 127 : v < -128 ? -128 : v);
            break;
        }
        default: break;
        }
    }
}

/* ------------------------------------------------------------------ */
/* model                                                                */
/* ------------------------------------------------------------------ */

typedef struct {
    const void *w;
    const float *s, *b;
} OrLin;

typedef struct {
    const float *ln1_g, *ln1_b, *ln2_g, *ln2_b;
    OrLin attn, proj, fc, fc2;              /* gpt2 */
    OrLin q, k, v, o, gate, up, down;       /* qwen2 */
} OrLayer;

struct OrModel {
    int arch, precision;
    int L, H, KVH, E, C, V, F, hd, kv;
    double eps, rope_theta, yarn_factor, yarn_orig_max, yarn_attn;
    int rope_yarn, sliding_window, tie;
    const uint16_t *wte, *wpe, *lm_head;
    const float *lnf_g, *lnf_b;
    OrLayer *lw;
    int batch_cap, max_ctx, eff_ctx, mmax;
    uint16_t *kc, *vc;
    float *x, *h1, *qkv, *at;
    int8_t *qa;
    float *qs;
    void *map;
    size_t map_size;
};

typedef struct {
    char name[128];
    int dtype; /* 0 fp32 1 fp16 2 int8 3 text 4 bf16 */
    size_t bytes, offset;
} OrTensor;

static size_t or_dtype_size(int d)
{
    return d == 0 ? 4 : d == 1 ? 2 : d == 2 ? 1 : d == 4 ? 2 : 0;
}

/* .ecm header: magic, key=value lines to END_META, "name dtype dims..." lines
 * to END_TENSORS, then the blobs back to back (src/gpt2.c:34-136). */
static int or_parse(OrModel *g, const char *data, size_t size, OrTensor *t, int max)
{
    const char *p = data, *end = data + size;
    if (size < 5 || memcmp(p, "ECM1\n", 5) != 0) return -1;
    p += 5;
    char line[1024];
    int stage = 0, n = 0;
    while (p < end) {
        size_t k = 0;
        while (p < end && *p != '\n' && k + 1 < sizeof line) {
            if (*p != '\r') line[k++] = *p;
            p++;
        }
        line[k] = 0;
        if (p < end) p++;
        if (stage == 0) {
            if (!strcmp(line, "END_META")) { stage = 1; continue; }
            char *eq = strchr(line, '=');
            if (!eq) continue;
            *eq = 0;
            const char *key = line, *val = eq + 1;
            if (!strcmp(key, "n_layer")) g->L = atoi(val);
            else if (!strcmp(key, "n_head")) g->H = atoi(val);
            else if (!strcmp(key, "n_kv_head")) g->KVH = atoi(val);
            else if (!strcmp(key, "intermediate")) g->F = atoi(val);
            else if (!strcmp(key, "n_embd")) g->E = atoi(val);
            else if (!strcmp(key, "n_ctx")) g->C = atoi(val);
            else if (!strcmp(key, "vocab")) g->V = atoi(val);
            else if (!strcmp(key, "eps")) g->eps = atof(val);
            else if (!strcmp(key, "rope_theta")) g->rope_theta = atof(val);
            else if (!strcmp(key, "rope_type")) g->rope_yarn = !strcmp(val, "yarn");
            else if (!strcmp(key, "yarn_factor")) g->yarn_factor = atof(val);
            else if (!strcmp(key, "yarn_attention_factor")) g->yarn_attn = atof(val);
            else if (!strcmp(key, "yarn_orig_max")) g->yarn_orig_max = atof(val);
            else if (!strcmp(key, "sliding_window")) g->sliding_window = atoi(val);
            else if (!strcmp(key, "tie_word_embeddings")) g->tie = atoi(val);
            else if (!strcmp(key, "arch"))
                g->arch = (!strcmp(val, "qwen2") || !strcmp(val, "olmo3")) ? 1 : 0;
        } else {
            if (!strcmp(line, "END_TENSORS")) {
                size_t off = (size_t)(p - data);
                for (int i = 0; i < n; i++) {
                    t[i].offset = off;
                    off += t[i].bytes;
                }
                return off <= size ? n : -1;
            }
            char name[128], dt[16];
            if (sscanf(line, "%127s %15s", name, dt) < 2) continue;
            int d;
            if (!strcmp(dt, "fp32")) d = 0;
            else if (!strcmp(dt, "fp16")) d = 1;
            else if (!strcmp(dt, "int8")) d = 2;
            else if (!strcmp(dt, "text")) d = 3;
            else if (!strcmp(dt, "bf16")) d = 4;
            else continue;
            if (n >= max) return -1;
            OrTensor *tt = &t[n++];
            snprintf(tt->name, sizeof tt->name, "%s", name);
            tt->dtype = d;
            const char *q = line;
            for (int f = 0; f < 2; f++) { /* skip name and dtype */
                while (*q == ' ') q++;
                while (*q && *q != ' ') q++;
            }
            if (d == 3) {
                tt->bytes = (size_t)strtoull(q, NULL, 10);
            } else {
                size_t ne = 1;
                while (*q) {
                    while (*q == ' ') q++;
                    if (!*q) break;
                    char *e2;
                    ne *= (size_t)strtoull(q, &e2, 10);
                    if (e2 == q) break;
                    q = e2;
                }
                tt->bytes = ne * or_dtype_size(d);
            }
        }
    }
    return -1;
}

static const OrTensor *or_find(const OrTensor *t, int n, const char *name)
{
    for (int i = 0; i < n; i++)
        if (!strcmp(t[i].name, name)) return &t[i];
    return NULL;
}

OrModel *or_load(const char *path, int batch_cap, int max_ctx)
{
    OrModel *g = calloc(1, sizeof *g);
    if (!g) return NULL;
    g->batch_cap = batch_cap < 1 ? 1 : batch_cap;
    g->max_ctx = max_ctx > 0 ? max_ctx : 0;
    g->eps = 1e-5;
    int fd = open(path, O_RDONLY);
    if (fd < 0) { free(g); return NULL; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) { close(fd); free(g); return NULL; }
    void *map = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) { free(g); return NULL; }
    g->map = map;
    g->map_size = (size_t)st.st_size;
    OrTensor *t = calloc(1024, sizeof *t);
    int n = or_parse(g, map, g->map_size, t, 1024);
    const char *base = map;
#define OR_FAIL() do { free(t); or_free(g); return NULL; } while (0)
    if (n < 0) OR_FAIL();
    const OrTensor *wte = or_find(t, n, "wte"), *lnf = or_find(t, n, "ln_f.g");
    if (!wte || !lnf) OR_FAIL();
    g->wte = (const uint16_t *)(base + wte->offset);
    g->lnf_g = (const float *)(base + lnf->offset);
    const OrTensor *t0 = or_find(t, n, g->arch ? "blocks.0.q.w" : "blocks.0.attn.w");
    if (!t0) OR_FAIL();
    if (t0->dtype == 1) g->precision = 1;
    else if (t0->dtype == 2) g->precision = 0;
    else if (t0->dtype == 4) g->precision = 2;
    else OR_FAIL();
    if (g->arch == 1) { /* set_qwen2_defaults, src/gpt2.c:149-159 */
        if (g->KVH <= 0) g->KVH = g->H;
        g->hd = g->E / (g->H > 0 ? g->H : 1);
        g->kv = g->KVH * g->hd;
        if (g->F <= 0) g->F = 4 * g->E;
        if (g->rope_theta <= 0) g->rope_theta = 10000.0;
        if (g->yarn_orig_max <= 0) g->yarn_orig_max = g->C;
        if (g->yarn_factor <= 0) g->yarn_factor = 1.0;
        if (g->yarn_attn <= 0) g->yarn_attn = 1.0;
        const OrTensor *lm = or_find(t, n, "lm_head.w");
        if (lm && !g->tie) g->lm_head = (const uint16_t *)(base + lm->offset);
        else g->tie = 1;
    } else {
        const OrTensor *wpe = or_find(t, n, "wpe"), *lnb = or_find(t, n, "ln_f.b");
        if (!wpe || !lnb) OR_FAIL();
        g->wpe = (const uint16_t *)(base + wpe->offset);
        g->lnf_b = (const float *)(base + lnb->offset);
        g->kv = g->E;
        g->KVH = g->H;
        g->F = 4 * g->E;
        g->hd = g->E / g->H;
    }
    g->lw = calloc((size_t)g->L, sizeof *g->lw);
    char nm[256];
    for (int l = 0; l < g->L; l++) {
        OrLayer *W = &g->lw[l];
        const OrTensor *x;
#define OR_F32(field, suffix) \
        snprintf(nm, sizeof nm, "blocks.%d.%s", l, suffix); \
        x = or_find(t, n, nm); W->field = x ? (const float *)(base + x->offset) : NULL;
        OR_F32(ln1_g, "ln_1.g") OR_F32(ln1_b, "ln_1.b") OR_F32(ln2_g, "ln_2.g") OR_F32(ln2_b, "ln_2.b")
        const char *qs[7] = {"q", "k", "v", "o", "gate", "up", "down"};
        OrLin *ql[7] = {&W->q, &W->k, &W->v, &W->o, &W->gate, &W->up, &W->down};
        const char *gs[4] = {"attn", "proj", "fc", "fc2"};
        OrLin *gl[4] = {&W->attn, &W->proj, &W->fc, &W->fc2};
        int cnt = g->arch ? 7 : 4;
        for (int s = 0; s < cnt; s++) {
            const char *suf = g->arch ? qs[s] : gs[s];
            OrLin *lin = g->arch ? ql[s] : gl[s];
            snprintf(nm, sizeof nm, "blocks.%d.%s.w", l, suf);
            const OrTensor *tw = or_find(t, n, nm);
            snprintf(nm, sizeof nm, "blocks.%d.%s.s", l, suf);
            const OrTensor *ts = or_find(t, n, nm);
            snprintf(nm, sizeof nm, "blocks.%d.%s.b", l, suf);
            const OrTensor *tb = or_find(t, n, nm);
            if (!tw) OR_FAIL();
            if (!g->arch && !tb) OR_FAIL();
            if (!g->arch && g->precision == 0 && !ts) OR_FAIL();
            lin->w = base + tw->offset;
            lin->s = (g->precision == 0 && ts) ? (const float *)(base + ts->offset) : NULL;
            lin->b = tb ? (const float *)(base + tb->offset) : NULL;
        }
    }
    if (!or_find(t, n, "tokenizer.vocab") || !or_find(t, n, "tokenizer.merges")) OR_FAIL();
    free(t);
    g->eff_ctx = (g->max_ctx > 0 && g->max_ctx < g->C) ? g->max_ctx : g->C;
    size_t kvn = (size_t)g->L * g->batch_cap * g->eff_ctx * g->kv;
    g->kc = calloc(kvn, 2);
    g->vc = calloc(kvn, 2);
    size_t E = (size_t)g->E;
    g->mmax = g->eff_ctx > g->batch_cap ? g->eff_ctx : g->batch_cap;
    size_t Mx = (size_t)g->mmax;
    size_t cols = g->arch ? ((size_t)2 * g->F > E + 2 * (size_t)g->kv ? (size_t)2 * g->F : E + 2 * (size_t)g->kv)
                          : 4 * E;
    size_t qc = g->arch ? (E > (size_t)g->F ? E : (size_t)g->F) : 4 * E;
    g->x = malloc(Mx * E * 4);
    g->h1 = malloc(Mx * 4 * E * 4);
    g->qkv = malloc(Mx * cols * 4);
    g->at = malloc(Mx * E * 4);
    g->qa = malloc(Mx * qc);
    g->qs = malloc(Mx * 4);
    if (!g->kc || !g->vc || !g->x || !g->h1 || !g->qkv || !g->at || !g->qa || !g->qs) {
        or_free(g);
        return NULL;
    }
    return g;
#undef OR_FAIL
#undef OR_F32
}

void or_free(OrModel *g)
{
    if (!g) return;
    free(g->lw);
    free(g->kc); free(g->vc);
    free(g->x); free(g->h1); free(g->qkv); free(g->at); free(g->qa); free(g->qs);
    if (g->map) munmap(g->map, g->map_size);
    free(g);
}

void or_kv_reset(OrModel *g)
{
    size_t kvn = (size_t)g->L * g->batch_cap * g->eff_ctx * g->kv;
    memset(g->kc, 0, kvn * 2);
    memset(g->vc, 0, kvn * 2);
}

int or_vocab(const OrModel *g) { return g->V; }
int or_eff_ctx(const OrModel *g) { return g->eff_ctx; }
int or_precision(const OrModel *g) { return g->precision; }
int or_arch(const OrModel *g) { return g->arch; }

/* linear() of src/gpt2.c:420-464 */
static void or_linear(OrModel *g, const OrLin *lin, const float *bias, const float *in,
                      float *out, int M, int K, int N)
{
    if (g->precision == 0) {
        or_quantize_rows(in, M, K, g->qa, g->qs);
        or_gemm_int8(out, g->qa, g->qs, (const int8_t *)lin->w, lin->s, bias, M, K, N);
        return;
    }
    gemm_w16(out, in, (const uint16_t *)lin->w, M, K, N, g->precision == 2);
    if (bias)
        for (int m = 0; m < M; m++)
            for (int n = 0; n < N; n++) out[(size_t)m * N + n] += bias[n];
}

static inline float emb_val(const OrModel *g, uint16_t v)
{
    return g->precision == 2 ? or_bf16_to_f32(v) : or_f16_to_f32(v);
}

/* one attention row: head h of token m over cache positions [lo, pos]
 * (src/gpt2.c:527-557 and 744-777) */
static void or_attend(const float *q, const uint16_t *kb, const uint16_t *vb, int stride,
                      int hd, int lo, int pos, double inv_hd, float *sc, float *o)
{
    int npos = pos + 1;
    float maxs = -FLT_MAX;
    for (int p = lo; p < npos; p++) {
        const uint16_t *kp = kb + (size_t)p * stride;
        float s = 0.0f;
        for (int d = 0; d < hd; d++) {
            float pr = q[d] * g_f16_lut[kp[d]];
            s = s + pr;
        }
        s = (float)(s * inv_hd);
        sc[p] = s;
        if (s > maxs) maxs = s;
    }
    double sume = 0.0;
    for (int p = lo; p < npos; p++) {
        sc[p] = expf(sc[p] - maxs);
        sume += sc[p];
    }
    double isum = 1.0 / sume;
    for (int p = lo; p < npos; p++) sc[p] = (float)(sc[p] * isum);
    for (int d = 0; d < hd; d++) o[d] = 0.0f;
    for (int p = lo; p < npos; p++) {
        const uint16_t *vp = vb + (size_t)p * stride;
        float w = sc[p];
        for (int d = 0; d < hd; d++) {
            float pr = w * g_f16_lut[vp[d]];
            o[d] = o[d] + pr;
        }
    }
}

/* or_attend on caller-given caches [nslots][C][KVH*hd], for checking the
 * device attention kernels alone: the listed rows (tokens) m, every head h
 * (KV head h * KVH / H, src/gpt2.c:744-745), positions [lo, pos[m]] of slot
 * slot[m] with lo as the forward's (sliding window, src/gpt2.c:753-754).
 * 0, or -1 for arguments outside the caches. */
int or_attention_rows(const float *q, int ldq, const uint16_t *kc, const uint16_t *vc, int nslots, int C,
                      int H, int KVH, int hd, const int *pos, const int *slot, const int *rows, int nrows,
                      int window, float *out, int ldo)
{
    if (nslots < 1 || C < 1 || H < 1 || KVH < 1 || H % KVH || hd < 1 || nrows < 0) return -1;
    for (int r = 0; r < nrows; r++) {
        int m = rows[r];
        if (m < 0 || pos[m] < 0 || pos[m] >= C || slot[m] < 0 || slot[m] >= nslots) return -1;
    }
    f16_lut_init();
    const int kv = KVH * hd;
    const double inv_hd = 1.0 / sqrt((double)hd);
    int rc = 0;
#pragma omp parallel
    {
        float *sc = malloc((size_t)C * sizeof(float));
        if (!sc) rc = -1;
#pragma omp for collapse(2) schedule(static)
        for (int r = 0; r < nrows; r++) {
            for (int h = 0; h < H; h++) {
                if (!sc) continue;
                int m = rows[r];
                int lo = window > 0 ? pos[m] - window + 1 : 0;
                if (lo < 0) lo = 0;
                size_t cbase = (size_t)slot[m] * C * kv + (size_t)(h * KVH / H) * hd;
                or_attend(q + (size_t)m * ldq + (size_t)h * hd, kc + cbase, vc + cbase, kv, hd, lo, pos[m],
                          inv_hd, sc, out + (size_t)m * ldo + (size_t)h * hd);
            }
        }
        free(sc);
    }
    return rc;
}

static int or_check_inputs(const OrModel *g, const int *tokens, const int *positions, int M)
{
    if (M < 1 || M > g->mmax) return -1;
    for (int m = 0; m < M; m++) {
        if (tokens[m] < 0 || tokens[m] >= g->V) return -1;
        if (positions[m] < 0 || positions[m] >= g->eff_ctx) return -1;
        if (g->arch == 0 && positions[m] >= g->C) return -1;
    }
    return 0;
}

static inline int or_slot(const OrModel *g, const int *seqs, int m)
{
    int s = seqs ? seqs[m] : m;
    if (s >= g->batch_cap) s = g->batch_cap - 1;
    if (s < 0) s = 0;
    return s;
}

/* lm_from: first row whose logits are computed (rows before it are not
 * needed by the caller; every other result is unchanged). */
static int or_forward_rows(OrModel *g, const int *tokens, const int *positions,
                           const int *seqs, int M, float *logits, int lm_from)
{
    if (or_check_inputs(g, tokens, positions, M)) return -1;
    f16_lut_init();
    const int E = g->E, H = g->H, L = g->L, V = g->V, hd = g->hd, kv = g->kv;
    const int C = g->eff_ctx, F = g->F, B = g->batch_cap;
    const double inv_hd = 1.0 / sqrt((double)hd);
    float *x = g->x, *h1 = g->h1, *qkv = g->qkv, *at = g->at;

    for (int m = 0; m < M; m++) { /* embeddings, src/gpt2.c:489-499 / 690-700 */
        const uint16_t *et = g->wte + (size_t)tokens[m] * E;
        for (int d = 0; d < E; d++) {
            float v = emb_val(g, et[d]);
            if (g->arch == 0) v = v + emb_val(g, g->wpe[(size_t)positions[m] * E + d]);
            x[(size_t)m * E + d] = v;
        }
    }

    int half = hd / 2;
    if (half > 512) half = 512;
    double inv_freq[512];
    if (g->arch == 1)
        or_rope_inv_freq(inv_freq, half, g->rope_theta, g->rope_yarn, g->yarn_factor,
                         g->yarn_orig_max);

    for (int l = 0; l < L; l++) {
        const OrLayer *W = &g->lw[l];
        float *qbuf, *kbuf, *vbuf;
        int qstride, kvstride;
        if (g->arch == 0) {
            or_layernorm_rows(h1, x, W->ln1_g, W->ln1_b, M, E, g->eps);
            or_linear(g, &W->attn, W->attn.b, h1, qkv, M, E, 3 * E);
            qbuf = qkv; kbuf = qkv + E; vbuf = qkv + 2 * E;
            qstride = 3 * E; kvstride = 3 * E;
        } else {
            or_rmsnorm_rows(h1, x, W->ln1_g, M, E, g->eps);
            or_linear(g, &W->q, NULL, h1, qkv, M, E, E);
            or_linear(g, &W->k, NULL, h1, qkv + (size_t)M * E, M, E, kv);
            or_linear(g, &W->v, NULL, h1, qkv + (size_t)M * (E + kv), M, E, kv);
            qbuf = qkv; kbuf = qkv + (size_t)M * E; vbuf = qkv + (size_t)M * (E + kv);
            qstride = E; kvstride = kv;
            for (int m = 0; m < M; m++) { /* RoPE, src/gpt2.c:714-723 */
                double cs[512], sn[512];
                for (int i = 0; i < half; i++) {
                    double f = (double)positions[m] * inv_freq[i];
                    cs[i] = cos(f) * g->yarn_attn;
                    sn[i] = sin(f) * g->yarn_attn;
                }
                for (int hh = 0; hh < H + g->KVH; hh++) {
                    float *v = hh < H ? qbuf + (size_t)m * qstride + (size_t)hh * hd
                                      : kbuf + (size_t)m * kvstride + (size_t)(hh - H) * hd;
                    for (int i = 0; i < half; i++) {
                        float a = v[i], b = v[i + half];
                        double t1 = a * cs[i], t2 = b * sn[i];
                        double t3 = a * sn[i], t4 = b * cs[i];
                        v[i] = (float)(t1 - t2);
                        v[i + half] = (float)(t3 + t4);
                    }
                }
            }
        }
        /* KV store, src/gpt2.c:509-524 / 726-741 */
        size_t lstride = (size_t)B * C * kv;
        for (int m = 0; m < M; m++) {
            int slot = or_slot(g, seqs, m);
            size_t off = lstride * l + (size_t)slot * C * kv + (size_t)positions[m] * kv;
            for (int d = 0; d < kv; d++) {
                g->kc[off + d] = or_f32_to_f16(kbuf[(size_t)m * kvstride + d]);
                g->vc[off + d] = or_f32_to_f16(vbuf[(size_t)m * kvstride + d]);
            }
        }
        /* attention; each (h, m) row is independent, so the parallel loop
         * does not change any result */
#pragma omp parallel
        {
            float *sc = malloc((size_t)C * sizeof(float));
#pragma omp for collapse(2) schedule(static)
            for (int h = 0; h < H; h++) {
                for (int m = 0; m < M; m++) {
                    int slot = or_slot(g, seqs, m);
                    int pos = positions[m];
                    int kvh = g->arch ? h * g->KVH / H : h;
                    size_t cbase = ((size_t)l * B + slot) * (size_t)C * kv + (size_t)kvh * hd;
                    int lo = 0;
                    if (g->arch == 1 && g->sliding_window > 0) {
                        lo = pos - g->sliding_window + 1;
                        if (lo < 0) lo = 0;
                    }
                    or_attend(qbuf + (size_t)m * qstride + (size_t)h * hd, g->kc + cbase,
                              g->vc + cbase, kv, hd, lo, pos, inv_hd, sc,
                              at + (size_t)m * E + (size_t)h * hd);
                }
            }
            free(sc);
        }
        if (g->arch == 0) {
            or_linear(g, &W->proj, W->proj.b, at, h1, M, E, E);
            for (size_t i = 0; i < (size_t)M * E; i++) x[i] = x[i] + h1[i];
            or_layernorm_rows(h1, x, W->ln2_g, W->ln2_b, M, E, g->eps);
            or_linear(g, &W->fc, W->fc.b, h1, qkv, M, E, 4 * E);
            for (size_t i = 0; i < (size_t)M * 4 * E; i++) qkv[i] = or_gelu_new(qkv[i]);
            or_linear(g, &W->fc2, W->fc2.b, qkv, h1, M, 4 * E, E);
            for (size_t i = 0; i < (size_t)M * E; i++) x[i] = x[i] + h1[i];
        } else {
            or_linear(g, &W->o, NULL, at, h1, M, E, E);
            for (size_t i = 0; i < (size_t)M * E; i++) x[i] = x[i] + h1[i];
            or_rmsnorm_rows(h1, x, W->ln2_g, M, E, g->eps);
            or_linear(g, &W->gate, NULL, h1, qkv, M, E, F);
            or_linear(g, &W->up, NULL, h1, qkv + (size_t)M * F, M, E, F);
            for (size_t i = 0; i < (size_t)M * F; i++)
                qkv[i] = or_silu(qkv[i]) * qkv[(size_t)M * F + i];
            or_linear(g, &W->down, NULL, qkv, h1, M, F, E);
            for (size_t i = 0; i < (size_t)M * E; i++) x[i] = x[i] + h1[i];
        }
    }
    /* final norm + LM head, src/gpt2.c:576-580 / 799-804 */
    if (g->arch == 0) or_layernorm_rows(h1, x, g->lnf_g, g->lnf_b, M, E, g->eps);
    else or_rmsnorm_rows(h1, x, g->lnf_g, M, E, g->eps);
    if (lm_from < M && logits) {
        const uint16_t *lm = g->lm_head ? g->lm_head : g->wte;
        gemm_w16(logits, h1 + (size_t)lm_from * E, lm, M - lm_from, E, V, g->precision == 2);
    }
    return 0;
}

int or_forward(OrModel *g, const int *tokens, const int *positions, const int *seqs,
               int M, float *logits)
{
    return or_forward_rows(g, tokens, positions, seqs, M, logits, 0);
}

/* or_forward with the LM head only for rows [lm_from, M): logits gets
 * [M - lm_from][V] (may be NULL when lm_from == M); every other result, the
 * KV cache included, is the same (gpt2_forward_ex's lm_from) */
int or_forward_from(OrModel *g, const int *tokens, const int *positions, const int *seqs,
                    int M, int lm_from, float *logits)
{
    if (lm_from < 0 || lm_from > M) return -1;
    return or_forward_rows(g, tokens, positions, seqs, M, logits, lm_from);
}

int or_argmax(const float *logits, int vocab)
{
    int best = 0;
    for (int i = 1; i < vocab; i++)
        if (logits[i] > logits[best]) best = i;
    return best;
}

int or_generate(OrModel *g, const int *prompt, int n, int n_gen, int *out_ids,
                float *step_logits)
{
    if (n < 1 || n + n_gen > g->eff_ctx) return -1;
    int V = g->V;
    or_kv_reset(g);
    int *pos = malloc((size_t)n * sizeof(int)), *seq = calloc((size_t)n, sizeof(int));
    float *lg = malloc((size_t)V * sizeof(float));
    for (int i = 0; i < n; i++) pos[i] = i;
    memcpy(out_ids, prompt, (size_t)n * sizeof(int));
    /* the prefill logits are discarded by the reference driver; computing
     * them would not change anything below */
    int rc = or_forward_rows(g, prompt, pos, seq, n, NULL, n);
    int cur = prompt[n - 1], npos = n;
    for (int i = 0; rc == 0 && i < n_gen; i++) {
        rc = or_forward_rows(g, &cur, &npos, NULL, 1, lg, 0);
        if (rc) break;
        if (step_logits) memcpy(step_logits + (size_t)i * V, lg, (size_t)V * sizeof(float));
        cur = or_argmax(lg, V);
        out_ids[n + i] = cur;
        npos++;
    }
    free(pos); free(seq); free(lg);
    return rc;
}
