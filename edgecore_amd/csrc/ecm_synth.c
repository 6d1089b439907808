/*
 * ecm_synth -- seeded synthetic .ecm model and prompt generator.
 *
 * Writes GPT-2 or Qwen2 models in the .ecm layout of edgecore/ecm.py:62-100
 * (magic, key=value meta, tensor table, blobs) with random N(0, std) weights,
 * norm gains 1 and shifts 0 (the convention of scripts/make_synthetic.py),
 * int8 per-output-channel packing (edgecore/ecm.py:50-59) or fp16/bf16
 * round-to-nearest-even, and a 256-entry byte vocabulary with no merges.
 *
 * Random numbers: every tensor row has its own SplitMix64 stream keyed by
 * (seed, tensor index, row); uniforms are (x >> 11 + 1) * 2^-53 and normals
 * come from the Box-Muller transform, both outputs used.  Rows are independent
 * so the file is identical for any thread count.  Prompt ids are uniform in
 * [0, vocab) from one SplitMix64 stream seeded with --prompt-seed
 * (multiply-shift mapping).
 *
 * Presets follow the benchmark shapes: tiny-gpt2 (L2 E64 H2 ctx128 V50257
 * int8), gpt2-small (L12 E768 H12 ctx1024 V50257 fp16), qwen2-0.5b (L24 E896
 * H14/KV2 F4864 ctx32768 V151936 int8, tied), qwen2.5-1.5b (L28 E1536 H12/KV2
 * F8960 ctx32768 V151936 int8, tied), tiny-qwen2 (L2 E64 H4/KV2 F96 ctx128
 * V512 int8).
 */
#define _GNU_SOURCE
#include "edgecore.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
    const char *out, *name, *arch, *precision, *prompt_out, *rope_type;
    int L, E, H, KVH, F, C, V, tie, prompt_len, window, yarn_orig_max;
    double std, eps, theta, yarn_factor, yarn_attn;
    unsigned long long seed, prompt_seed;
} Opts;

static uint64_t sm64(uint64_t *s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t row_stream(uint64_t seed, uint64_t tensor, uint64_t row)
{
    uint64_t s = seed;
    uint64_t a = sm64(&s) ^ (tensor * 0xD1B54A32D192ED03ull);
    uint64_t b = sm64(&a) ^ (row * 0x8CB92BA72F3D8DD7ull);
    sm64(&b);
    return b;
}

static void normal_row(uint64_t state, float *dst, int n, double std)
{
    const double two_pi = 6.283185307179586476925286766559;
    for (int i = 0; i < n; i += 2) {
        double u1 = (double)((sm64(&state) >> 11) + 1) * 0x1.0p-53;
        double u2 = (double)((sm64(&state) >> 11) + 1) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        dst[i] = (float)(std * r * cos(two_pi * u2));
        if (i + 1 < n) dst[i + 1] = (float)(std * r * sin(two_pi * u2));
    }
}


typedef struct {
    char name[96];
    int kind; /* 0 random matrix, 1 ones, 2 zeros, 3 random vector, 4 scales of previous, 5 vocab, 6 merges */
    int dtype; /* 0 fp32 1 fp16 2 int8 3 text 4 bf16 */
    int rows, cols;
    size_t text_bytes;
    int rng_id;
} Tens;

static Tens g_t[4096];
static int g_n;
static int g_rng_next;

static void add(const char *name, int kind, int dtype, int rows, int cols)
{
    Tens *t = &g_t[g_n++];
    memset(t, 0, sizeof *t);
    snprintf(t->name, sizeof t->name, "%s", name);
    t->kind = kind;
    t->dtype = dtype;
    t->rows = rows;
    t->cols = cols;
    if (kind == 0 || kind == 3) t->rng_id = g_rng_next++;
}

static int prec_dtype(const char *p)
{
    return !strcmp(p, "int8") ? 2 : !strcmp(p, "bf16") ? 4 : 1;
}

static void add_linear(const char *prefix, int out, int in, int w_dtype, int bias)
{
    char nm[96];
    snprintf(nm, sizeof nm, "%s.w", prefix);
    add(nm, 0, w_dtype, out, in);
    if (w_dtype == 2) {
        snprintf(nm, sizeof nm, "%s.s", prefix);
        add(nm, 4, 0, out, 1);
    }
    if (bias) {
        snprintf(nm, sizeof nm, "%s.b", prefix);
        add(nm, 3, 0, 1, out);
    }
}

static size_t vocab_blob(uint8_t *dst)
{
    size_t o = 0;
    uint32_t v = 256;
    if (dst) memcpy(dst, &v, 4);
    o += 4;
    for (uint32_t i = 0; i < 256; i++) {
        uint32_t one = 1;
        if (dst) {
            memcpy(dst + o, &i, 4);
            memcpy(dst + o + 4, &one, 4);
            dst[o + 8] = (uint8_t)i;
        }
        o += 9;
    }
    return o;
}

static void build_table(const Opts *o)
{
    int wd = prec_dtype(o->precision);
    int ed = wd == 4 ? 4 : 1; /* embeddings and LM head: fp16 unless bf16 */
    char p[96], nm[128];
    g_n = 0;
    g_rng_next = 0;
    if (!strcmp(o->arch, "gpt2")) {
        add("wte", 0, ed, o->V, o->E);
        add("wpe", 0, ed, o->C, o->E);
        add("ln_f.g", 1, 0, 1, o->E);
        add("ln_f.b", 2, 0, 1, o->E);
        for (int l = 0; l < o->L; l++) {
            snprintf(p, sizeof p, "blocks.%d", l);
            snprintf(nm, sizeof nm, "%s.ln_1.g", p); add(nm, 1, 0, 1, o->E);
            snprintf(nm, sizeof nm, "%s.ln_1.b", p); add(nm, 2, 0, 1, o->E);
            snprintf(nm, sizeof nm, "%s.ln_2.g", p); add(nm, 1, 0, 1, o->E);
            snprintf(nm, sizeof nm, "%s.ln_2.b", p); add(nm, 2, 0, 1, o->E);
            snprintf(nm, sizeof nm, "%s.attn", p); add_linear(nm, 3 * o->E, o->E, wd, 1);
            snprintf(nm, sizeof nm, "%s.proj", p); add_linear(nm, o->E, o->E, wd, 1);
            snprintf(nm, sizeof nm, "%s.fc", p); add_linear(nm, 4 * o->E, o->E, wd, 1);
            snprintf(nm, sizeof nm, "%s.fc2", p); add_linear(nm, o->E, 4 * o->E, wd, 1);
        }
    } else {
        int hd = o->E / o->H, kv = o->KVH * hd;
        add("wte", 0, ed, o->V, o->E);
        if (!o->tie) add("lm_head.w", 0, ed, o->V, o->E);
        add("ln_f.g", 1, 0, 1, o->E);
        for (int l = 0; l < o->L; l++) {
            snprintf(p, sizeof p, "blocks.%d", l);
            snprintf(nm, sizeof nm, "%s.ln_1.g", p); add(nm, 1, 0, 1, o->E);
            snprintf(nm, sizeof nm, "%s.ln_2.g", p); add(nm, 1, 0, 1, o->E);
            snprintf(nm, sizeof nm, "%s.q", p); add_linear(nm, o->E, o->E, wd, 0);
            snprintf(nm, sizeof nm, "%s.k", p); add_linear(nm, kv, o->E, wd, 0);
            snprintf(nm, sizeof nm, "%s.v", p); add_linear(nm, kv, o->E, wd, 0);
            snprintf(nm, sizeof nm, "%s.o", p); add_linear(nm, o->E, o->E, wd, 0);
            snprintf(nm, sizeof nm, "%s.gate", p); add_linear(nm, o->F, o->E, wd, 0);
            snprintf(nm, sizeof nm, "%s.up", p); add_linear(nm, o->F, o->E, wd, 0);
            snprintf(nm, sizeof nm, "%s.down", p); add_linear(nm, o->E, o->F, wd, 0);
        }
    }
    add("tokenizer.vocab", 5, 3, 1, 1);
    g_t[g_n - 1].text_bytes = vocab_blob(NULL);
    add("tokenizer.merges", 6, 3, 1, 1);
    g_t[g_n - 1].text_bytes = 4;
}

static size_t dt_bytes(int d) { return d == 0 ? 4 : d == 2 ? 1 : d == 3 ? 1 : 2; }

/* %.17g, with ".0" appended to an integral value ("1.0", "4.0"), the form of
   the YaRN meta values in files written before these options existed */
static const char *fmt_real(char *buf, size_t n, double v)
{
    snprintf(buf, n, "%.17g", v);
    if (!strpbrk(buf, ".eEn")) strncat(buf, ".0", n - strlen(buf) - 1);
    return buf;
}

static int write_model(const Opts *o)
{
    char yf[40], ya[40];
    FILE *f = fopen(o->out, "wb");
    if (!f) { perror(o->out); return 1; }
    size_t n_params = 0;
    for (int i = 0; i < g_n; i++)
        if (g_t[i].kind != 4 && g_t[i].dtype != 3) n_params += (size_t)g_t[i].rows * g_t[i].cols;
    fputs(ECM_MAGIC, f);
    fprintf(f, "model_name=%s\nn_layer=%d\nn_head=%d\nn_embd=%d\nn_ctx=%d\nvocab=%d\n",
            o->name, o->L, o->H, o->E, o->C, o->V);
    fprintf(f, "eps=%.17g\narch=%s\n", o->eps, o->arch);
    if (!strcmp(o->arch, "qwen2"))
        fprintf(f, "n_kv_head=%d\nintermediate=%d\nrope_theta=%.17g\nrope_type=%s\n"
                   "yarn_factor=%s\nyarn_orig_max=%d\nyarn_attention_factor=%s\n"
                   "sliding_window=%d\ntie_word_embeddings=%d\neos_token_id=%d\n",
                o->KVH, o->F, o->theta, o->rope_type, fmt_real(yf, sizeof yf, o->yarn_factor),
                o->yarn_orig_max > 0 ? o->yarn_orig_max : o->C, fmt_real(ya, sizeof ya, o->yarn_attn),
                o->window, o->tie, o->V - 1);
    fprintf(f, "n_params=%zu\nEND_META\n", n_params);
    static const char *dn[] = {"fp32", "fp16", "int8", "text", "bf16"};
    for (int i = 0; i < g_n; i++) {
        Tens *t = &g_t[i];
        if (t->dtype == 3) fprintf(f, "%s text %zu\n", t->name, t->text_bytes);
        else if (t->rows == 1 || t->kind == 4) fprintf(f, "%s %s %d\n", t->name, dn[t->dtype], t->kind == 4 ? t->rows : t->cols);
        else fprintf(f, "%s %s %d %d\n", t->name, dn[t->dtype], t->rows, t->cols);
    }
    fputs("END_TENSORS\n", f);

    float *pending_scales = NULL;
    for (int i = 0; i < g_n; i++) {
        Tens *t = &g_t[i];
        if (t->kind == 5) {
            size_t nb = vocab_blob(NULL);
            uint8_t *b = (uint8_t *)malloc(nb);
            vocab_blob(b);
            fwrite(b, 1, nb, f);
            free(b);
            continue;
        }
        if (t->kind == 6) {
            uint32_t z = 0;
            fwrite(&z, 4, 1, f);
            continue;
        }
        if (t->kind == 4) {
            fwrite(pending_scales, 4, (size_t)t->rows, f);
            free(pending_scales);
            pending_scales = NULL;
            continue;
        }
        size_t ne = (size_t)t->rows * t->cols;
        if (t->kind == 1 || t->kind == 2) {
            float *v = (float *)malloc(ne * 4);
            for (size_t k = 0; k < ne; k++) v[k] = t->kind == 1 ? 1.0f : 0.0f;
            fwrite(v, 4, ne, f);
            free(v);
            continue;
        }
        void *buf = malloc(ne * dt_bytes(t->dtype));
        if (t->dtype == 2) pending_scales = (float *)malloc((size_t)t->rows * 4);
        if (!buf) { fclose(f); return 1; }
        int rows = t->kind == 3 ? 1 : t->rows;
        int cols = t->kind == 3 ? t->cols : t->cols;
#pragma omp parallel
        {
            float *tmp = (float *)malloc((size_t)cols * 4);
#pragma omp for schedule(static)
            for (int r = 0; r < rows; r++) {
                normal_row(row_stream(o->seed, (uint64_t)t->rng_id, (uint64_t)r), tmp, cols, o->std);
                size_t base = (size_t)r * cols;
                if (t->dtype == 0) memcpy((float *)buf + base, tmp, (size_t)cols * 4);
                else if (t->dtype == 1)
                    for (int c = 0; c < cols; c++) ((uint16_t *)buf)[base + c] = f32_to_fp16(tmp[c]);
                else if (t->dtype == 4)
                    for (int c = 0; c < cols; c++) ((uint16_t *)buf)[base + c] = ec_f32_to_bf16(tmp[c]);
                else
                    ec_quantize_int8_symmetric(tmp, 1, cols, (int8_t *)buf + base, pending_scales + r);
            }
            free(tmp);
        }
        fwrite(buf, dt_bytes(t->dtype), ne, f);
        free(buf);
    }
    if (fclose(f) != 0) return 1;
    return 0;
}

static int write_prompt(const Opts *o)
{
    FILE *f = fopen(o->prompt_out, "w");
    if (!f) { perror(o->prompt_out); return 1; }
    uint64_t s = o->prompt_seed;
    for (int i = 0; i < o->prompt_len; i++) {
        uint64_t x = sm64(&s);
        unsigned id = (unsigned)(((unsigned __int128)x * (unsigned)o->V) >> 64);
        fprintf(f, "%u%c", id, (i + 1) % 16 == 0 || i + 1 == o->prompt_len ? '\n' : ' ');
    }
    return fclose(f) != 0;
}

static int preset(Opts *o, const char *p)
{
    if (!strcmp(p, "tiny-gpt2")) {
        o->arch = "gpt2"; o->L = 2; o->E = 64; o->H = 2; o->C = 128; o->V = 50257; o->precision = "int8";
    } else if (!strcmp(p, "gpt2-small")) {
        o->arch = "gpt2"; o->L = 12; o->E = 768; o->H = 12; o->C = 1024; o->V = 50257; o->precision = "fp16";
    } else if (!strcmp(p, "qwen2-0.5b")) {
        o->arch = "qwen2"; o->L = 24; o->E = 896; o->H = 14; o->KVH = 2; o->F = 4864; o->C = 32768;
        o->V = 151936; o->precision = "int8"; o->tie = 1; o->eps = 1e-6; o->theta = 1e6;
    } else if (!strcmp(p, "qwen2.5-1.5b")) {
        o->arch = "qwen2"; o->L = 28; o->E = 1536; o->H = 12; o->KVH = 2; o->F = 8960; o->C = 32768;
        o->V = 151936; o->precision = "int8"; o->tie = 1; o->eps = 1e-6; o->theta = 1e6;
    } else if (!strcmp(p, "tiny-qwen2")) {
        o->arch = "qwen2"; o->L = 2; o->E = 64; o->H = 4; o->KVH = 2; o->F = 96; o->C = 128;
        o->V = 512; o->precision = "int8"; o->tie = 0; o->eps = 1e-6; o->theta = 1e6;
    } else {
        return -1;
    }
    o->name = p;
    return 0;
}

static void usage(void)
{
    fprintf(stderr,
            "usage: ecm_synth --out FILE [--preset tiny-gpt2|gpt2-small|qwen2-0.5b|qwen2.5-1.5b|tiny-qwen2]\n"
            "  [--arch gpt2|qwen2] [--layers N] [--embd E] [--heads H] [--kv-heads N] [--ffn F]\n"
            "  [--ctx C] [--vocab V] [--precision int8|fp16|bf16] [--tie 0|1] [--seed S]\n"
            "  [--std X] [--eps X] [--rope-theta X] [--name NAME]\n"
            "  [--sliding-window W] [--rope-type default|yarn] [--yarn-factor X]\n"
            "  [--yarn-orig-max N] [--yarn-attention-factor X]   (qwen2 only)\n"
            "  [--prompt-out FILE --prompt-len N [--prompt-seed S]]\n");
}

int main(int argc, char **argv)
{
    Opts o;
    memset(&o, 0, sizeof o);
    o.arch = "gpt2"; o.precision = "int8"; o.name = NULL;
    o.L = 2; o.E = 64; o.H = 2; o.C = 128; o.V = 256;
    o.std = 0.02; o.eps = 1e-5; o.theta = 1e6; o.seed = 0; o.prompt_seed = 1;
    o.rope_type = "default"; o.yarn_factor = 1.0; o.yarn_attn = 1.0;
    for (int i = 1; i < argc; i++) {
        const char *a = argv[i];
        const char *v = i + 1 < argc ? argv[i + 1] : NULL;
#define ARG(flag) (!strcmp(a, flag) && v && (i++, 1))
        if (ARG("--out")) o.out = v;
        else if (ARG("--preset")) { if (preset(&o, v)) { usage(); return 2; } }
        else if (ARG("--arch")) o.arch = v;
        else if (ARG("--layers")) o.L = atoi(v);
        else if (ARG("--embd")) o.E = atoi(v);
        else if (ARG("--heads")) o.H = atoi(v);
        else if (ARG("--kv-heads")) o.KVH = atoi(v);
        else if (ARG("--ffn")) o.F = atoi(v);
        else if (ARG("--ctx")) o.C = atoi(v);
        else if (ARG("--vocab")) o.V = atoi(v);
        else if (ARG("--precision")) o.precision = v;
        else if (ARG("--tie")) o.tie = atoi(v);
        else if (ARG("--seed")) o.seed = strtoull(v, NULL, 10);
        else if (ARG("--std")) o.std = atof(v);
        else if (ARG("--eps")) o.eps = atof(v);
        else if (ARG("--rope-theta")) o.theta = atof(v);
        else if (ARG("--name")) o.name = v;
        else if (ARG("--sliding-window")) o.window = atoi(v);
        else if (ARG("--rope-type")) o.rope_type = v;
        else if (ARG("--yarn-factor")) o.yarn_factor = atof(v);
        else if (ARG("--yarn-orig-max")) o.yarn_orig_max = atoi(v);
        else if (ARG("--yarn-attention-factor")) o.yarn_attn = atof(v);
        else if (ARG("--prompt-out")) o.prompt_out = v;
        else if (ARG("--prompt-len")) o.prompt_len = atoi(v);
        else if (ARG("--prompt-seed")) o.prompt_seed = strtoull(v, NULL, 10);
        else { usage(); return 2; }
#undef ARG
    }
    if (!o.out && !o.prompt_out) { usage(); return 2; }
    if (strcmp(o.arch, "gpt2") && strcmp(o.arch, "qwen2")) { usage(); return 2; }
    if (strcmp(o.precision, "int8") && strcmp(o.precision, "fp16") && strcmp(o.precision, "bf16")) { usage(); return 2; }
    if ((strcmp(o.rope_type, "default") && strcmp(o.rope_type, "yarn")) || o.window < 0) { usage(); return 2; }
    if (!strcmp(o.arch, "qwen2")) {
        if (o.KVH <= 0) o.KVH = o.H;
        if (o.F <= 0) o.F = 4 * o.E;
    }
    if (o.L < 1 || o.E < 1 || o.H < 1 || o.E % o.H || o.C < 1 || o.V < 1 ||
        (!strcmp(o.arch, "qwen2") && (o.H % o.KVH))) {
        fprintf(stderr, "ecm_synth: inconsistent shape\n");
        return 2;
    }
    if (!o.name) o.name = "synthetic";
    if (o.out) {
        build_table(&o);
        if (write_model(&o)) { fprintf(stderr, "ecm_synth: write failed\n"); return 1; }
    }
    if (o.prompt_out && o.prompt_len > 0 && write_prompt(&o)) return 1;
    return 0;
}
