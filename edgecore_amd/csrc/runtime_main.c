/*
 * edgecore-runtime: the command-line driver over libedgecore_hip.so.
 *
 * Contract kept from the reference driver (src/runtime_main.c), because the
 * reference's Python CLI parses it (edgecore/bench.py:124-152,
 * edgecore/verify.py:126-199, scripts/smoke_test.sh:17-86):
 *   - the flags and their defaults (:163-191, :600-640);
 *   - the JSON keys of each mode in the reference's order, with %.3f times,
 *     %.6g logits and null for non-finite values (:400-590);
 *   - the --logits-bin layout: int32 n, int32 vocab, int32 tokens[n],
 *     float32 logits[n][vocab] (:454-464);
 *   - exit codes: 0 ok, 1 load or prompt failure, 2 usage error or a
 *     --precision that differs from the file's weights (:610-662);
 *   - what is timed: TTFT is the prompt's forward, a step is one forward of
 *     `batch` tokens, tok/s and percentiles are computed as in :381-396 and
 *     :529-554; prompts are clamped to eff_ctx - 8 tokens;
 *   - sampling: the LCG seeded with --seed, one draw per batch row in row
 *     order; row 0's tokens are the generated ids.
 *
 * Everything else is this driver's own: a table of options that also prints
 * the help, core pinning from sysfs topology, a small JSON emitter, and a
 * Decoder object that owns the per-step buffers.  Differences in behaviour,
 * all additive or result-preserving: the KV cache is cleared on the device
 * (gpt2_kv_reset); greedy steps take the argmax on the GPU and copy back one
 * id per row; at batch 1 the greedy steps are chained on the GPU
 * (ec_generate_greedy_timed: each id becomes the next step's token there) and
 * each step's time is read from the GPU's clock, the ids coming back once
 * (key step_timing: "gpu-clock", else "host");
 * the prompt's forward computes the LM head of its last row only;
 * a prompt plus n-tokens beyond the context is refused (exit 2) instead of
 * writing past the cache; the JSON ends with extra keys (backend, device,
 * token_ids, tokens_per_sec_aggregate, decode_bytes_per_step, decode_gbps).
 */
#define _GNU_SOURCE
#include "edgecore.h"

#include <math.h>
#include <sched.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* configuration: one table drives parsing and the help text            */
/* ------------------------------------------------------------------ */

typedef struct {
    const char *model, *mode, *precision, *prompt, *tokens_file, *output, *affinity, *logits_bin;
    int threads, batch, n_tokens, warmup, iters, seed, top_k, logits_limit, max_ctx, no_print;
    double temp;
    double load_ms; /* measured, not a flag */
} Config;

enum { OPT_STR, OPT_INT, OPT_REAL, OPT_FLAG };

typedef struct {
    const char *flag;
    int kind;
    size_t at; /* offsetof(Config, field) */
    const char *arg, *help;
} Option;

static const Option kOptions[] = {
    {"--model", OPT_STR, offsetof(Config, model), "FILE", ".ecm model file (required)"},
    {"--mode", OPT_STR, offsetof(Config, mode), "M", "generate | logits | bench (generate)"},
    {"--precision", OPT_STR, offsetof(Config, precision), "P",
     "fp16 | bf16 | int8 | auto; must agree with the file's weights (auto)"},
    {"--threads", OPT_INT, offsetof(Config, threads), "N", "reported only: the forward runs on the GPU (1)"},
    {"--batch", OPT_INT, offsetof(Config, batch), "N", "sequences decoded together (1)"},
    {"--prompt", OPT_STR, offsetof(Config, prompt), "TEXT", "prompt text, encoded by the model's tokenizer"},
    {"--tokens-file", OPT_STR, offsetof(Config, tokens_file), "FILE", "prompt as whitespace-separated ids"},
    {"--n-tokens", OPT_INT, offsetof(Config, n_tokens), "N", "tokens to generate (32)"},
    {"--temp", OPT_REAL, offsetof(Config, temp), "T", "sampling temperature; 0 is greedy (0)"},
    {"--top-k", OPT_INT, offsetof(Config, top_k), "K", "sample among the K largest logits; 0 is all (0)"},
    {"--seed", OPT_INT, offsetof(Config, seed), "S", "sampling seed (42)"},
    {"--warmup", OPT_INT, offsetof(Config, warmup), "N", "untimed bench runs (1)"},
    {"--iters", OPT_INT, offsetof(Config, iters), "N", "timed bench runs (1)"},
    {"--logits-limit", OPT_INT, offsetof(Config, logits_limit), "N", "prompt tokens kept in logits mode (1024)"},
    {"--max-ctx", OPT_INT, offsetof(Config, max_ctx), "N", "context to allocate; 0 is the model's (0)"},
    {"--affinity", OPT_STR, offsetof(Config, affinity), "A",
     "none | auto | physical | CPU list such as 0,2,4 (none)"},
    {"--logits-bin", OPT_STR, offsetof(Config, logits_bin), "FILE", "also write raw logits (logits mode)"},
    {"--output", OPT_STR, offsetof(Config, output), "FILE", "write the JSON here instead of stdout"},
    {"--no-print", OPT_FLAG, offsetof(Config, no_print), NULL, "do not print the generated text"},
};
#define N_OPTIONS ((int)(sizeof kOptions / sizeof kOptions[0]))

static void print_help(const char *prog)
{
    fprintf(stderr, "usage: %s --model FILE [options]   (MI355X GPU forward; device 0 or $EDGECORE_DEVICE)\n", prog);
    for (int i = 0; i < N_OPTIONS; i++) {
        char left[48];
        snprintf(left, sizeof left, "%s%s%s", kOptions[i].flag, kOptions[i].arg ? " " : "",
                 kOptions[i].arg ? kOptions[i].arg : "");
        fprintf(stderr, "  %-22s %s\n", left, kOptions[i].help);
    }
}

static void config_defaults(Config *c)
{
    memset(c, 0, sizeof *c);
    c->mode = "generate";
    c->precision = "auto";
    c->affinity = "none";
    c->prompt = "The quick brown fox jumps over the lazy dog";
    c->threads = 1;
    c->batch = 1;
    c->n_tokens = 32;
    c->warmup = 1;
    c->iters = 1;
    c->seed = 42;
    c->logits_limit = 1024;
}

/* 0 ok; 2 usage error (message printed) */
static int config_parse(Config *c, int argc, char **argv)
{
    for (int i = 1; i < argc; i++) {
        const Option *o = NULL;
        for (int k = 0; k < N_OPTIONS && !o; k++)
            if (!strcmp(argv[i], kOptions[k].flag)) o = &kOptions[k];
        if (!o) {
            fprintf(stderr, "unknown arg: %s\n", argv[i]);
            print_help(argv[0]);
            return 2;
        }
        char *field = (char *)c + o->at;
        if (o->kind == OPT_FLAG) {
            *(int *)field = 1;
            continue;
        }
        if (i + 1 >= argc) {
            fprintf(stderr, "%s needs a value\n", o->flag);
            return 2;
        }
        const char *v = argv[++i];
        if (o->kind == OPT_STR) *(const char **)field = v;
        else if (o->kind == OPT_INT) *(int *)field = atoi(v);
        else *(double *)field = atof(v);
    }
    if (!c->model) {
        print_help(argv[0]);
        return 2;
    }
    if (c->batch < 1) c->batch = 1;
    if (c->n_tokens < 0) c->n_tokens = 0;
    return 0;
}

/* ------------------------------------------------------------------ */
/* CPU pinning                                                          */
/* ------------------------------------------------------------------ */

typedef struct {
    const char *policy;
    int applied;
    int ncpu;
    int cpu[1024];
} CpuPin;

/* the lowest CPU of a sysfs cpu list ("3", "3,67", "2-3,66-67") that is in
 * `allowed`, or -1 */
static int lowest_allowed(const char *path, const cpu_set_t *allowed)
{
    FILE *f = fopen(path, "r");
    if (!f) return -1;
    char buf[256];
    const int got = fgets(buf, sizeof buf, f) != NULL;
    fclose(f);
    if (!got) return -1;
    int best = -1;
    for (char *p = buf; *p && *p != '\n';) {
        char *end;
        long lo = strtol(p, &end, 10), hi = lo;
        if (end == p) break;
        if (*end == '-') {
            p = end + 1;
            hi = strtol(p, &end, 10);
        }
        for (long c = lo; c <= hi && c < CPU_SETSIZE; c++)
            if (CPU_ISSET((int)c, allowed) && (best < 0 || c < best)) best = (int)c;
        p = *end == ',' ? end + 1 : end;
    }
    return best;
}

/* one CPU per physical core: the lowest allowed CPU among each core's
 * hardware threads (sysfs topology/thread_siblings_list) */
static int cores_only(const cpu_set_t *allowed, cpu_set_t *out)
{
    CPU_ZERO(out);
    int n = 0;
    for (int c = 0; c < CPU_SETSIZE; c++) {
        if (!CPU_ISSET(c, allowed)) continue;
        char path[96];
        snprintf(path, sizeof path, "/sys/devices/system/cpu/cpu%d/topology/thread_siblings_list", c);
        const int lead = lowest_allowed(path, allowed);
        if (lead == c || lead < 0) {
            CPU_SET(c, out);
            n++;
        }
    }
    return n;
}

static int cpus_from_list(const char *s, cpu_set_t *out)
{
    CPU_ZERO(out);
    int n = 0;
    for (const char *p = s; *p;) {
        if (*p == ',' || *p == ' ') {
            p++;
            continue;
        }
        char *end;
        const long v = strtol(p, &end, 10);
        if (end == p || v < 0 || v >= CPU_SETSIZE) return -1;
        CPU_SET((int)v, out);
        n++;
        p = end;
    }
    return n > 0 ? 0 : -1;
}

static void pin_cpus(const char *policy, CpuPin *pin)
{
    memset(pin, 0, sizeof *pin);
    pin->policy = policy;
    cpu_set_t now, want;
    CPU_ZERO(&now);
    sched_getaffinity(0, sizeof now, &now);
    int have = 0;
    if (!strcmp(policy, "physical") || !strcmp(policy, "auto")) have = cores_only(&now, &want) > 0;
    else if (strcmp(policy, "none")) have = cpus_from_list(policy, &want) == 0;
    if (have && sched_setaffinity(0, sizeof want, &want) == 0) pin->applied = 1;
    CPU_ZERO(&now);
    sched_getaffinity(0, sizeof now, &now);
    for (int c = 0; c < CPU_SETSIZE && pin->ncpu < 1024; c++)
        if (CPU_ISSET(c, &now)) pin->cpu[pin->ncpu++] = c;
}

/* ------------------------------------------------------------------ */
/* JSON output                                                          */
/* ------------------------------------------------------------------ */

typedef struct {
    FILE *f;
    int fields;
} Json;

static void json_text(FILE *f, const char *s)
{
    fputc('"', f);
    for (const unsigned char *p = (const unsigned char *)s; *p; p++) {
        switch (*p) {
        case '"': fputs("\\\"", f); break;
        case '\\': fputs("\\\\", f); break;
        case '\n': fputs("\\n", f); break;
        case '\r': fputs("\\r", f); break;
        case '\t': fputs("\\t", f); break;
        default:
            if (*p < 0x20) fprintf(f, "\\u%04x", *p);
            else fputc(*p, f);
        }
    }
    fputc('"', f);
}

static void jkey(Json *j, const char *k)
{
    fprintf(j->f, "%s  \"%s\": ", j->fields++ ? ",\n" : "{\n", k);
}
static void jint(Json *j, const char *k, long long v) { jkey(j, k); fprintf(j->f, "%lld", v); }
static void jms(Json *j, const char *k, double v) { jkey(j, k); fprintf(j->f, "%.3f", v); }
static void jstr(Json *j, const char *k, const char *v) { jkey(j, k); json_text(j->f, v); }
static void jraw(Json *j, const char *k, const char *v) { jkey(j, k); fputs(v, j->f); }
static void jints(Json *j, const char *k, const int *v, int n)
{
    jkey(j, k);
    fputc('[', j->f);
    for (int i = 0; i < n; i++) fprintf(j->f, "%s%d", i ? "," : "", v[i]);
    fputc(']', j->f);
}
static void jclose(Json *j)
{
    fputs(j->fields ? "\n}\n" : "{}\n", j->f);
    fflush(j->f);
}

static void jpin(Json *j, const CpuPin *p)
{
    jstr(j, "affinity_requested", p->policy);
    jraw(j, "affinity_applied", p->applied ? "true" : "false");
    jints(j, "affinity_cpus", p->cpu, p->ncpu);
}

/* ------------------------------------------------------------------ */
/* statistics (percentile indices of src/runtime_main.c:388-396)        */
/* ------------------------------------------------------------------ */

typedef struct {
    double mean, p50, p95, p99, sum;
} Summary;

static int by_value(const void *a, const void *b)
{
    const double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}

static Summary summarize(const double *v, int n)
{
    Summary s = {0, 0, 0, 0, 0};
    if (n <= 0) return s;
    double *sorted = malloc((size_t)n * sizeof *sorted);
    memcpy(sorted, v, (size_t)n * sizeof *sorted);
    qsort(sorted, (size_t)n, sizeof *sorted, by_value);
    for (int i = 0; i < n; i++) s.sum += sorted[i];
    s.mean = s.sum / n;
    s.p50 = sorted[(n - 1) / 2];
    s.p95 = sorted[(int)(n * 0.95)];
    s.p99 = sorted[(int)(n * 0.99)];
    free(sorted);
    return s;
}

/* ------------------------------------------------------------------ */
/* decoding                                                             */
/* ------------------------------------------------------------------ */

/* the reference's sampling state (src/runtime_main.c:205-211); the draw
 * itself is ec_sample_full / ec_sample_candidates of the library */
static unsigned long long g_lcg;

typedef struct {
    GPT2 *g;
    int batch, top_k, ncand, use_topk;
    float temp;
    int *cur, *pos, *greedy;
    float *rows;               /* [batch][vocab] when sampling */
    float *cand_v;             /* [batch][top_k + 1] device top-k candidates */
    int *cand_i, *cand_status;
} Decoder;

static void fail_forward(void)
{
    fprintf(stderr, "forward failed: %s\n", ec_last_error());
    exit(1);
}

static void decoder_init(Decoder *d, GPT2 *g, int batch, float temp, int top_k)
{
    memset(d, 0, sizeof *d);
    d->g = g;
    d->batch = batch;
    d->temp = temp;
    d->top_k = top_k;
    const int V = g->vocab;
    /* sampled steps select the top_k + 1 largest logits on the GPU when k allows */
    d->use_topk = temp > 0.0f && top_k > 0 && top_k < V && top_k <= ec_topk_max();
    d->ncand = top_k + 1;
    d->cur = calloc((size_t)batch, sizeof(int));
    d->pos = calloc((size_t)batch, sizeof(int));
    d->greedy = calloc((size_t)batch, sizeof(int));
    if (temp > 0.0f) d->rows = malloc((size_t)batch * V * sizeof(float));
    if (d->use_topk) {
        d->cand_v = malloc((size_t)batch * d->ncand * sizeof(float));
        d->cand_i = malloc((size_t)batch * d->ncand * sizeof(int));
        d->cand_status = malloc((size_t)batch * sizeof(int));
    }
}

static void decoder_free(Decoder *d)
{
    free(d->cur); free(d->pos); free(d->greedy); free(d->rows);
    free(d->cand_v); free(d->cand_i); free(d->cand_status);
}

/* Fill every slot with the prompt (slot 0 timed: the TTFT), leaving each
 * slot's next input at the prompt's last token.  Returns the TTFT in ms. */
static double decoder_prefill(Decoder *d, const int *prompt, int n)
{
    int *at = malloc((size_t)n * sizeof(int)), *slot = malloc((size_t)n * sizeof(int));
    for (int i = 0; i < n; i++) at[i] = i;
    if (gpt2_kv_reset(d->g)) fail_forward();
    double ttft = 0.0;
    for (int b = 0; b < d->batch; b++) {
        for (int i = 0; i < n; i++) slot[i] = b;
        int first;
        const double t = now_sec();
        /* slot 0 computes its last row's LM head (and argmax), as the
         * reference's timed prompt forward does; the others skip it */
        if (gpt2_forward_ex(d->g, prompt, at, slot, n, b == 0 ? n - 1 : n, NULL, b == 0 ? &first : NULL))
            fail_forward();
        if (b == 0) ttft = (now_sec() - t) * 1000.0;
        d->cur[b] = prompt[n - 1];
        d->pos[b] = n;
    }
    free(at);
    free(slot);
    return ttft;
}

/* One decode step of every row; writes row 0's new token.  Returns ms. */
static double decoder_step(Decoder *d, int *row0_token)
{
    GPT2 *g = d->g;
    const int V = g->vocab, B = d->batch;
    const double t = now_sec();
    int rc;
    if (d->use_topk)
        rc = gpt2_forward_topk(g, d->cur, d->pos, NULL, B, 0, d->top_k, d->cand_v, d->cand_i, d->cand_status);
    else if (d->temp > 0.0f)
        rc = gpt2_forward_ex(g, d->cur, d->pos, NULL, B, 0, d->rows, NULL);
    else
        rc = gpt2_forward_ex(g, d->cur, d->pos, NULL, B, 0, NULL, d->greedy);
    if (rc) fail_forward();
    const double ms = (now_sec() - t) * 1000.0;
    for (int b = 0; b < B; b++) {
        int tok = d->greedy[b];
        if (d->use_topk && d->cand_status[b] == 0) {
            tok = ec_sample_candidates(d->cand_v + (size_t)b * d->ncand, d->cand_i + (size_t)b * d->ncand, d->ncand,
                                       V, d->temp, d->top_k, &g_lcg);
        } else if (d->temp > 0.0f) {
            float *row = d->rows + (size_t)b * V;
            /* NaN or a tie at the k-th place: draw from the whole row */
            if (d->use_topk && ec_last_logits(g, b, row)) fail_forward();
            tok = ec_sample_full(row, V, d->temp, d->top_k, &g_lcg);
        }
        d->cur[b] = tok;
        d->pos[b]++;
    }
    *row0_token = d->cur[0];
    return ms;
}

/* a prefill and n_gen steps: TTFT, per-step times and row 0's ids */
typedef struct {
    double ttft_ms;
    double *step_ms;
    int *ids; /* prompt followed by the generated tokens of row 0 */
    int n_ids;
    int gpu_timed; /* steps timed by the GPU's clock (chained greedy steps) */
} Run;

static void run_once(GPT2 *g, const Config *c, const int *prompt, int n, float temp, Run *r)
{
    Decoder d;
    decoder_init(&d, g, c->batch, temp, c->top_k);
    r->step_ms = malloc((size_t)(c->n_tokens > 0 ? c->n_tokens : 1) * sizeof(double));
    r->ids = malloc((size_t)(n + c->n_tokens) * sizeof(int));
    memcpy(r->ids, prompt, (size_t)n * sizeof(int));
    r->n_ids = n;
    r->gpu_timed = 0;
    r->ttft_ms = decoder_prefill(&d, prompt, n);
    if (c->batch == 1 && temp <= 0.0f && c->n_tokens > 0) {
        /* greedy at batch 1: the steps chained on the GPU (each id becomes the
         * next step's token there, the ids come back once), timed per step
         * by the GPU's clock */
        if (ec_generate_greedy_timed(g, d.cur[0], d.pos[0], 0, c->n_tokens, r->ids + r->n_ids, r->step_ms))
            fail_forward();
        r->n_ids += c->n_tokens;
        r->gpu_timed = 1;
    } else {
        for (int s = 0; s < c->n_tokens; s++) r->step_ms[s] = decoder_step(&d, &r->ids[r->n_ids++]);
    }
    decoder_free(&d);
}

static void run_free(Run *r)
{
    free(r->step_ms);
    free(r->ids);
}

/* ------------------------------------------------------------------ */
/* modes                                                                */
/* ------------------------------------------------------------------ */

/* the prompt as ids: --tokens-file if given, else --prompt through the
 * tokenizer; at most `cap` ids.  0 ok, -1 failure. */
static int prompt_ids(GPT2 *g, const Config *c, int *ids, int cap, int *n)
{
    *n = 0;
    if (!c->tokens_file) {
        const int k = tokenizer_encode(&g->tok, c->prompt, ids, cap);
        if (k < 0) return -1;
        *n = k;
        return 0;
    }
    FILE *f = fopen(c->tokens_file, "r");
    if (!f) {
        perror("tokens file");
        return -1;
    }
    int v;
    while (*n < cap && fscanf(f, "%d", &v) == 1) ids[(*n)++] = v;
    fclose(f);
    return 0;
}

#define PROMPT_CAP 4096

/* the prompt for generate/bench, clamped to eff_ctx - 8; 0 ok or an exit code */
static int decode_prompt(GPT2 *g, const Config *c, int *ids, int *n)
{
    if (prompt_ids(g, c, ids, PROMPT_CAP, n)) {
        fprintf(stderr, "prompt load failed\n");
        return 1;
    }
    if (*n < 1) {
        fprintf(stderr, "empty prompt\n");
        return 1;
    }
    const int ctx = gpt2_eff_ctx(g);
    if (*n > ctx - 8) *n = ctx - 8;
    if (*n < 1 || *n + c->n_tokens > ctx) {
        fprintf(stderr, "prompt (%d) + n-tokens (%d) exceeds the context (%d); raise --max-ctx\n", *n, c->n_tokens,
                ctx);
        return 2;
    }
    return 0;
}

static FILE *open_output(const Config *c)
{
    if (!c->output) return stdout;
    FILE *f = fopen(c->output, "w");
    if (!f) perror(c->output);
    return f;
}

static void device_json(char *buf, int len)
{
    if (ec_device_info(buf, len) < 0) snprintf(buf, (size_t)len, "null");
}

/* algorithmic HBM bytes of one decode step of `batch` tokens at mean
 * position p: every weight byte once (and int8 row scales), plus the fp16
 * K/V rows that attention reads */
static double step_bytes(const GPT2 *g, int batch, double p)
{
    const double E = g->n_embd, F = g->intermediate, kv = g->n_kv_embd, L = g->n_layer;
    const double lin = g->arch == ARCH_QWEN2 ? 2 * E * E + 2 * kv * E + 3 * F * E : 12 * E * E;
    const double weights = g->precision == 0 ? lin + 4 * (lin / E) : 2 * lin;
    return L * (weights + (p + 1) * kv * 4 * batch) + 2.0 * g->vocab * E;
}

static int mode_generate(GPT2 *g, const Config *c, const CpuPin *pin)
{
    int prompt[PROMPT_CAP], n;
    int rc = decode_prompt(g, c, prompt, &n);
    if (rc) return rc;
    g_lcg = (unsigned long long)(unsigned long)c->seed;
    Run r;
    run_once(g, c, prompt, n, (float)c->temp, &r);
    const Summary s = summarize(r.step_ms, c->n_tokens);
    const double wall = (s.sum + r.ttft_ms) / 1000.0;
    char *text = c->no_print ? NULL : tokenizer_decode(&g->tok, r.ids, r.n_ids);
    FILE *f = open_output(c);
    if (!f) return 1;
    char dev[512];
    device_json(dev, sizeof dev);
    Json j = {f, 0};
    jstr(&j, "mode", "generate");
    jstr(&j, "model", g->model_name);
    jstr(&j, "precision", c->precision);
    jint(&j, "threads", c->threads);
    jint(&j, "batch", c->batch);
    jms(&j, "load_time_ms", c->load_ms);
    jpin(&j, pin);
    jint(&j, "n_prompt_tokens", n);
    jint(&j, "n_generated_tokens", c->n_tokens);
    jms(&j, "ttft_ms", r.ttft_ms);
    jms(&j, "cold_start_ms", c->load_ms + r.ttft_ms);
    jms(&j, "tpot_avg_ms", s.mean);
    jms(&j, "tokens_per_sec", wall > 0 ? c->n_tokens / wall : 0.0);
    jms(&j, "p50_ms", s.p50);
    jms(&j, "p95_ms", s.p95);
    jms(&j, "p99_ms", s.p99);
    jms(&j, "peak_rss_gb", peak_rss_gb());
    if (text) jstr(&j, "text", text);
    jstr(&j, "backend", "hip-gfx950");
    jraw(&j, "device", dev);
    jstr(&j, "step_timing", r.gpu_timed ? "gpu-clock" : "host");
    jints(&j, "token_ids", r.ids + n, r.n_ids - n);
    jclose(&j);
    if (f != stdout) fclose(f);
    if (text) {
        printf("%s\n", text);
        free(text);
    }
    run_free(&r);
    return 0;
}

static int mode_logits(GPT2 *g, const Config *c, const CpuPin *pin)
{
    int toks[PROMPT_CAP], n;
    if (prompt_ids(g, c, toks, PROMPT_CAP, &n)) {
        fprintf(stderr, "prompt load failed\n");
        return 1;
    }
    if (n < 1) return 1;
    if (n > c->logits_limit) n = c->logits_limit;
    if (n > gpt2_eff_ctx(g)) {
        fprintf(stderr, "prompt (%d) exceeds the context (%d); raise --max-ctx\n", n, gpt2_eff_ctx(g));
        return 2;
    }
    const int V = g->vocab;
    int *at = malloc((size_t)n * sizeof(int)), *slot = calloc((size_t)n, sizeof(int));
    float *lg = malloc((size_t)n * V * sizeof(float));
    for (int i = 0; i < n; i++) at[i] = i;
    if (gpt2_kv_reset(g) || gpt2_forward_ex(g, toks, at, slot, n, 0, lg, NULL)) fail_forward();
    if (c->logits_bin) {
        FILE *b = fopen(c->logits_bin, "wb");
        if (!b) {
            perror("logits bin");
            return 1;
        }
        const int32_t head[2] = {n, V};
        fwrite(head, sizeof head, 1, b);
        fwrite(toks, sizeof(int32_t), (size_t)n, b);
        fwrite(lg, sizeof(float), (size_t)n * V, b);
        fclose(b);
    }
    FILE *f = open_output(c);
    if (!f) return 1;
    Json j = {f, 0};
    jstr(&j, "model", g->model_name);
    jstr(&j, "precision", c->precision);
    jint(&j, "threads", c->threads);
    jms(&j, "load_time_ms", c->load_ms);
    jpin(&j, pin);
    jint(&j, "n_tokens", n);
    jints(&j, "tokens", toks, n);
    jkey(&j, "logits");
    fputs("[\n", f);
    for (int i = 0; i < n; i++) {
        fputs("    [", f);
        const float *row = lg + (size_t)i * V;
        for (int v = 0; v < V; v++) {
            if (v) fputc(',', f);
            if (isfinite(row[v])) fprintf(f, "%.6g", row[v]);
            else fputs("null", f);
        }
        fprintf(f, "]%s\n", i + 1 < n ? "," : "");
    }
    fputs("  ]", f);
    jclose(&j);
    if (f != stdout) fclose(f);
    free(at);
    free(slot);
    free(lg);
    return 0;
}

static int mode_bench(GPT2 *g, const Config *c, const CpuPin *pin)
{
    int prompt[PROMPT_CAP], n;
    int rc = decode_prompt(g, c, prompt, &n);
    if (rc) return rc;
    const int iters = c->iters > 0 ? c->iters : 1, B = c->batch, nt = c->n_tokens;
    Run r;
    for (int w = 0; w < c->warmup; w++) {
        run_once(g, c, prompt, n, 0.0f, &r);
        run_free(&r);
    }
    /* every step's time counts once per row it decoded (src/runtime_main.c:521-526) */
    const int per_token = B * nt * iters;
    double *tok_ms = malloc((size_t)(per_token > 0 ? per_token : 1) * sizeof(double));
    double *ttft = malloc((size_t)iters * sizeof(double));
    double step_total = 0.0;
    int k = 0, gpu_timed = 0;
    for (int it = 0; it < iters; it++) {
        run_once(g, c, prompt, n, 0.0f, &r);
        ttft[it] = r.ttft_ms;
        gpu_timed = r.gpu_timed;
        for (int s = 0; s < nt; s++) {
            step_total += r.step_ms[s];
            for (int b = 0; b < B; b++) tok_ms[k++] = r.step_ms[s];
        }
        run_free(&r);
    }
    const Summary tok = summarize(tok_ms, k), first = summarize(ttft, iters);
    const double gen_s = tok.sum / 1000.0;
    const double bytes = step_bytes(g, B, n + (nt - 1) / 2.0);
    const double step_s = iters * nt > 0 ? step_total / 1000.0 / (iters * nt) : 0.0;
    FILE *f = open_output(c);
    if (!f) return 1;
    char dev[512];
    device_json(dev, sizeof dev);
    Json j = {f, 0};
    jstr(&j, "mode", "bench");
    jstr(&j, "model", g->model_name);
    jstr(&j, "precision", c->precision);
    jint(&j, "threads", c->threads);
    jint(&j, "batch", B);
    jms(&j, "load_time_ms", c->load_ms);
    jpin(&j, pin);
    jint(&j, "n_prompt_tokens", n);
    jint(&j, "n_generated_tokens", B * nt);
    jint(&j, "iterations", iters);
    jms(&j, "avg_token_ms", tok.mean);
    jms(&j, "p50_ms", tok.p50);
    jms(&j, "p95_ms", tok.p95);
    jms(&j, "p99_ms", tok.p99);
    jms(&j, "ttft_avg_ms", first.mean);
    jms(&j, "cold_start_ms", c->load_ms + first.mean);
    jms(&j, "ttft_p50_ms", first.p50);
    jms(&j, "ttft_p95_ms", first.p95);
    jms(&j, "ttft_p99_ms", first.p99);
    jms(&j, "tokens_per_sec", gen_s > 0 ? k / gen_s : 0.0);
    jms(&j, "total_generation_sec", gen_s);
    jms(&j, "peak_rss_gb", peak_rss_gb());
    jstr(&j, "backend", "hip-gfx950");
    jraw(&j, "device", dev);
    jstr(&j, "step_timing", gpu_timed ? "gpu-clock" : "host");
    jms(&j, "tokens_per_sec_aggregate", step_total > 0 ? (double)B * nt * iters / (step_total / 1000.0) : 0.0);
    jint(&j, "decode_bytes_per_step", (long long)bytes);
    jkey(&j, "decode_gbps");
    fprintf(f, "%.2f", step_s > 0 ? bytes / step_s / 1e9 : 0.0);
    jclose(&j);
    if (f != stdout) fclose(f);
    free(tok_ms);
    free(ttft);
    return 0;
}

/* ------------------------------------------------------------------ */

static const char *dtype_name(int precision) { return precision == 2 ? "bf16" : precision == 1 ? "fp16" : "int8"; }

int main(int argc, char **argv)
{
    Config c;
    config_defaults(&c);
    if (argc < 2) {
        print_help(argv[0]);
        return 2;
    }
    int rc = config_parse(&c, argc, argv);
    if (rc) return rc;
    static const char *const kDtypes[] = {"int8", "fp16", "bf16"};
    int want = -1;
    for (int p = 0; p < 3; p++)
        if (!strcmp(c.precision, kDtypes[p])) want = p;
    if (want < 0 && strcmp(c.precision, "auto")) {
        fprintf(stderr, "unknown precision: %s (use fp16|bf16|int8|auto)\n", c.precision);
        return 2;
    }
    CpuPin pin;
    pin_cpus(c.affinity, &pin);

    GPT2 g;
    const double t0 = now_sec();
    if (gpt2_load(&g, c.model, c.batch, c.max_ctx) != 0) {
        fprintf(stderr, "failed to load model\n");
        return 1;
    }
    c.load_ms = (now_sec() - t0) * 1000.0;
    if (want >= 0 && want != g.precision) {
        fprintf(stderr, "model file uses %s weights, but --precision %s was requested\n", dtype_name(g.precision),
                c.precision);
        gpt2_free(&g);
        ec_release();
        return 2;
    }
    c.precision = dtype_name(g.precision);

    if (!strcmp(c.mode, "generate")) rc = mode_generate(&g, &c, &pin);
    else if (!strcmp(c.mode, "logits")) rc = mode_logits(&g, &c, &pin);
    else if (!strcmp(c.mode, "bench")) rc = mode_bench(&g, &c, &pin);
    else {
        fprintf(stderr, "unknown mode: %s\n", c.mode);
        rc = 2;
    }
    gpt2_free(&g);
    /* the library's streams, events and buffers go before the process exits,
       not in the HIP runtime's own teardown */
    if (ec_release() != 0) fprintf(stderr, "edgecore: release: %s\n", ec_last_error());
    return rc;
}
