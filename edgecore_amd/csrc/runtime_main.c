/*
 * edgecore-runtime for the MI355X library: the command-line contract of the
 * reference driver (src/runtime_main.c) -- modes generate|logits|bench, the
 * same flags, JSON keys, --logits-bin layout and exit codes (0 ok, 1 load or
 * prompt failure, 2 usage error or precision mismatch) -- over the GPU
 * forward of libedgecore_hip.so.
 *
 * Differences from the reference, all additive or result-preserving:
 *   - the KV cache is cleared with gpt2_kv_reset() instead of a host memset;
 *   - greedy steps take the argmax on the GPU (same first-maximum rule) and
 *     copy back one id per sequence instead of the full logits row;
 *   - the prefill call computes the LM head of the last prompt row only (the
 *     reference computes all rows and then discards them);
 *   - n_prompt + n_tokens beyond the context is rejected (exit 2) instead of
 *     writing past the KV cache;
 *   - JSON gains "backend", "device", "tokens_per_sec_aggregate" and
 *     "decode_bytes_per_step" / "decode_gbps".
 */
#define _GNU_SOURCE
#include "edgecore.h"

#include <math.h>
#include <sched.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* CPU affinity (policy names of src/runtime_main.c:108-133)            */
/* ------------------------------------------------------------------ */

typedef struct {
    char requested[32];
    int cpus[256];
    int n;
    int applied;
    char error[96];
} Affinity;

static void cpuset_list(const cpu_set_t *set, int *cpus, int *n)
{
    *n = 0;
    for (int i = 0; i < CPU_SETSIZE && *n < 256; i++)
        if (CPU_ISSET(i, set)) cpus[(*n)++] = i;
}

static int parse_cpu_list(const char *s, cpu_set_t *set)
{
    CPU_ZERO(set);
    while (*s) {
        while (*s == ' ' || *s == ',') s++;
        if (!*s) break;
        char *end;
        long c = strtol(s, &end, 10);
        if (end == s || c < 0 || c >= CPU_SETSIZE) return -1;
        CPU_SET((int)c, set);
        s = end;
    }
    return 0;
}

/* first logical CPU of each (physical id, core id) pair in /proc/cpuinfo */
static int physical_cpuset(cpu_set_t *set)
{
    CPU_ZERO(set);
    FILE *f = fopen("/proc/cpuinfo", "r");
    if (!f) return -1;
    char line[256];
    int proc = -1, phys = -1, core = -1, n = 0;
    struct { int phys, core, cpu; } seen[512];
    while (fgets(line, sizeof line, f)) {
        int v;
        if (sscanf(line, "processor : %d", &v) == 1) { proc = v; phys = core = -1; }
        else if (sscanf(line, "physical id : %d", &v) == 1) phys = v;
        else if (sscanf(line, "core id : %d", &v) == 1) core = v;
        if (proc >= 0 && phys >= 0 && core >= 0) {
            int k = 0;
            while (k < n && !(seen[k].phys == phys && seen[k].core == core)) k++;
            if (k == n && n < 512) { seen[n].phys = phys; seen[n].core = core; seen[n].cpu = proc; n++; }
            else if (k < n && proc < seen[k].cpu) seen[k].cpu = proc;
            proc = -1;
        }
    }
    fclose(f);
    for (int k = 0; k < n; k++) CPU_SET(seen[k].cpu, set);
    return n > 0 ? 0 : -1;
}

static void affinity_apply(const char *policy, Affinity *a)
{
    memset(a, 0, sizeof *a);
    snprintf(a->requested, sizeof a->requested, "%s", policy);
    cpu_set_t set;
    int want = 0;
    if (!strcmp(policy, "physical") || !strcmp(policy, "auto")) {
        if (physical_cpuset(&set) == 0) want = 1;
        else snprintf(a->error, sizeof a->error, "physical core enumeration failed");
    } else if (strcmp(policy, "none")) {
        if (parse_cpu_list(policy, &set) == 0) want = 1;
        else snprintf(a->error, sizeof a->error, "bad cpu list");
    }
    if (want) {
        if (sched_setaffinity(0, sizeof set, &set) != 0) snprintf(a->error, sizeof a->error, "sched_setaffinity failed");
        else a->applied = 1;
    }
    cpu_set_t cur;
    CPU_ZERO(&cur);
    sched_getaffinity(0, sizeof cur, &cur);
    cpuset_list(&cur, a->cpus, &a->n);
}

static void json_str(FILE *o, const char *s)
{
    fputc('"', o);
    for (; *s; s++) {
        unsigned char c = (unsigned char)*s;
        if (c == '"') fputs("\\\"", o);
        else if (c == '\\') fputs("\\\\", o);
        else if (c == '\n') fputs("\\n", o);
        else if (c == '\t') fputs("\\t", o);
        else if (c == '\r') fputs("\\r", o);
        else if (c < 0x20) fprintf(o, "\\u%04x", c);
        else fputc(c, o);
    }
    fputc('"', o);
}

static void emit_affinity(FILE *o, const Affinity *a)
{
    fprintf(o, "  \"affinity_requested\": ");
    json_str(o, a->requested);
    fprintf(o, ",\n  \"affinity_applied\": %s,\n  \"affinity_cpus\": [", a->applied ? "true" : "false");
    for (int i = 0; i < a->n; i++) fprintf(o, "%s%d", i ? "," : "", a->cpus[i]);
    fprintf(o, "]");
}

/* ------------------------------------------------------------------ */
/* arguments                                                            */
/* ------------------------------------------------------------------ */

typedef struct {
    const char *model, *mode, *precision, *prompt, *tokens_file, *output, *affinity, *logits_bin;
    int threads, batch, n_tokens, warmup, iters, seed, top_k, logits_limit, no_print, max_ctx;
    float temp;
    double load_time_ms;
} Args;

static void usage(const char *prog)
{
    fprintf(stderr,
            "usage: %s --model FILE --mode {generate|logits|bench} [options]\n"
            "  --precision fp16|bf16|int8|auto (default auto; derived from .ecm weight dtype)\n"
            "  --threads N            (accepted; the forward runs on the GPU)\n"
            "  --batch N              (default 1)\n"
            "  --prompt TEXT          prompt for generate/logits (byte-level vocabularies)\n"
            "  --tokens-file FILE     token ids (whitespace separated) to use as prompt\n"
            "  --n-tokens N           tokens to generate (default 32)\n"
            "  --temp T               sampling temperature (default 0.0 = greedy)\n"
            "  --top-k N              top-k sampling (default 0 = off)\n"
            "  --seed N               rng seed\n"
            "  --warmup N / --iters N bench warmup / iterations\n"
            "  --logits-limit N       max prompt tokens for logits mode (default 1024)\n"
            "  --max-ctx N            max context length (default 0 = use model's n_ctx)\n"
            "  --affinity auto|none|physical|0[,2,..]  CPU affinity (default none)\n"
            "  --logits-bin FILE      write raw logits (n, vocab, tokens, logits f32)\n"
            "  --output FILE          JSON output file (default stdout)\n"
            "  --no-print             suppress generated text on stdout\n"
            "  GPU: device 0, or $EDGECORE_DEVICE\n",
            prog);
}

/* the LCG state of src/runtime_main.c:205-211; sample_token (:213-248) is
   ec_sample_full / ec_sample_candidates of the library */
static unsigned long long rng_state;

static int read_tokens(const char *path, int *out, int cap, int *n)
{
    FILE *f = fopen(path, "r");
    if (!f) { perror("tokens file"); return -1; }
    int v;
    *n = 0;
    while (fscanf(f, "%d", &v) == 1)
        if (*n < cap) out[(*n)++] = v;
    fclose(f);
    return 0;
}

static int load_prompt(GPT2 *g, const Args *a, int *toks, int cap, int *n)
{
    if (a->tokens_file) return read_tokens(a->tokens_file, toks, cap, n);
    int r = tokenizer_encode(&g->tok, a->prompt, toks, cap);
    if (r < 0) return -1;
    *n = r;
    return 0;
}

static void die_forward(void)
{
    fprintf(stderr, "forward failed: %s\n", ec_last_error());
    exit(1);
}

/* ------------------------------------------------------------------ */
/* prefill + decode (gen_and_measure, src/runtime_main.c:293-362)       */
/* ------------------------------------------------------------------ */

static void gen_and_measure(GPT2 *g, const int *prompt, int nprompt, int n_gen, int batch, float temp,
                            int top_k, double *tok_ms, int *out_ids, int *out_n, double *ttft_ms)
{
    int V = g->vocab;
    int *ids = malloc((size_t)(nprompt + n_gen + 8) * sizeof(int));
    memcpy(ids, prompt, (size_t)nprompt * sizeof(int));
    int n_ids = nprompt;
    int *ppos = malloc((size_t)nprompt * sizeof(int)), *pseq = malloc((size_t)nprompt * sizeof(int));
    for (int i = 0; i < nprompt; i++) { ppos[i] = i; pseq[i] = 0; }
    int *positions = malloc((size_t)batch * sizeof(int)), *cur = malloc((size_t)batch * sizeof(int));
    int *next = malloc((size_t)batch * sizeof(int));
    float *logits = temp > 0.0f ? malloc((size_t)batch * V * sizeof(float)) : NULL;
    /* sampled steps select the top_k + 1 logits on the GPU when top_k allows */
    const int use_topk = temp > 0.0f && top_k > 0 && top_k < V && top_k <= ec_topk_max();
    const int nc = top_k + 1;
    float *tk_vals = use_topk ? malloc((size_t)batch * nc * sizeof(float)) : NULL;
    int *tk_idx = use_topk ? malloc((size_t)batch * nc * sizeof(int)) : NULL;
    int *tk_status = use_topk ? malloc((size_t)batch * sizeof(int)) : NULL;
    int first;

    if (gpt2_kv_reset(g)) die_forward();
    double t0 = now_sec();
    if (gpt2_forward_ex(g, ids, ppos, pseq, nprompt, nprompt - 1, NULL, &first)) die_forward();
    *ttft_ms = (now_sec() - t0) * 1000.0;

    for (int b = 1; b < batch; b++) {
        for (int i = 0; i < nprompt; i++) pseq[i] = b;
        if (gpt2_forward_ex(g, ids, ppos, pseq, nprompt, nprompt, NULL, NULL)) die_forward();
    }
    for (int b = 0; b < batch; b++) cur[b] = ids[n_ids - 1];

    int npos = nprompt;
    for (int step = 0; step < n_gen; step++) {
        for (int b = 0; b < batch; b++) positions[b] = npos;
        double s0 = now_sec();
        int rc = use_topk ? gpt2_forward_topk(g, cur, positions, NULL, batch, 0, top_k, tk_vals, tk_idx, tk_status)
                 : temp > 0.0f ? gpt2_forward_ex(g, cur, positions, NULL, batch, 0, logits, NULL)
                               : gpt2_forward_ex(g, cur, positions, NULL, batch, 0, NULL, next);
        if (rc) die_forward();
        tok_ms[step] = (now_sec() - s0) * 1000.0;
        for (int b = 0; b < batch; b++) {
            int tok;
            if (use_topk && !tk_status[b]) {
                tok = ec_sample_candidates(tk_vals + (size_t)b * nc, tk_idx + (size_t)b * nc, nc, V, temp, top_k,
                                           &rng_state);
            } else if (use_topk) {  /* NaN or a tie at the top_k boundary: the whole row */
                if (ec_last_logits(g, b, logits + (size_t)b * V)) die_forward();
                tok = ec_sample_full(logits + (size_t)b * V, V, temp, top_k, &rng_state);
            } else {
                tok = temp > 0.0f ? ec_sample_full(logits + (size_t)b * V, V, temp, top_k, &rng_state) : next[b];
            }
            cur[b] = tok;
            if (b == 0) ids[n_ids++] = tok;
        }
        npos++;
    }
    *out_n = n_ids;
    memcpy(out_ids, ids, (size_t)n_ids * sizeof(int));
    free(ids); free(ppos); free(pseq); free(positions); free(cur); free(next); free(logits);
    free(tk_vals); free(tk_idx); free(tk_status);
}

static int cmp_double(const void *a, const void *b)
{
    double x = *(const double *)a, y = *(const double *)b;
    return x < y ? -1 : x > y;
}

/* percentiles of src/runtime_main.c:388-396 */
static void percentiles(const double *v, int n, double *p50, double *p95, double *p99)
{
    *p50 = *p95 = *p99 = 0.0;
    if (n <= 0) return;
    double *s = malloc((size_t)n * sizeof(double));
    memcpy(s, v, (size_t)n * sizeof(double));
    qsort(s, (size_t)n, sizeof(double), cmp_double);
    *p50 = s[(n - 1) / 2];
    *p95 = s[(int)(n * 0.95) < n ? (int)(n * 0.95) : n - 1];
    *p99 = s[(int)(n * 0.99) < n ? (int)(n * 0.99) : n - 1];
    free(s);
}

/* algorithmic HBM bytes of one decode step at batch b and mean position p:
 * every weight byte once, plus the K/V rows read by attention */
static double decode_bytes(const GPT2 *g, int batch, double mean_pos)
{
    double E = g->n_embd, F = g->intermediate, kv = g->n_kv_embd, V = g->vocab, L = g->n_layer;
    double wb = g->precision == 0 ? 1.0 : 2.0;
    double lin = g->arch == ARCH_QWEN2 ? (E * E * 2 + 2 * kv * E + 3 * F * E) : (12 * E * E);
    double per_layer = lin * wb + (g->precision == 0 ? 4.0 * (lin / E) : 0.0);
    double kvread = (mean_pos + 1.0) * kv * 2 * 2 * batch;
    return L * (per_layer + kvread) + V * E * 2.0;
}

static void emit_common(FILE *o, const GPT2 *g, const Args *a)
{
    char dev[512];
    if (ec_device_info(dev, sizeof dev) < 0) snprintf(dev, sizeof dev, "null");
    fprintf(o, "  \"model\": ");
    json_str(o, g->model_name);
    fprintf(o, ",\n  \"precision\": \"%s\",\n", a->precision);
    fprintf(o, "  \"backend\": \"hip-gfx950\",\n  \"device\": %s,\n", dev);
    fprintf(o, "  \"threads\": %d,\n", a->threads);
}

static int mode_generate(GPT2 *g, const Args *a, const Affinity *aff)
{
    int toks[4096], n;
    if (load_prompt(g, a, toks, 4096, &n)) { fprintf(stderr, "prompt load failed\n"); return 1; }
    if (n < 1) { fprintf(stderr, "empty prompt\n"); return 1; }
    int eff = gpt2_eff_ctx(g);
    if (n > eff - 8) n = eff - 8;
    if (n < 1 || n + a->n_tokens > eff) {
        fprintf(stderr, "prompt (%d) + n-tokens (%d) exceeds the context (%d); raise --max-ctx\n", n, a->n_tokens, eff);
        return 2;
    }
    int *ids = malloc((size_t)(n + a->n_tokens + 8) * sizeof(int));
    double *tok_ms = malloc((size_t)(a->n_tokens > 0 ? a->n_tokens : 1) * sizeof(double));
    double ttft = 0;
    int out_n = 0;
    gen_and_measure(g, toks, n, a->n_tokens, a->batch, a->temp, a->top_k, tok_ms, ids, &out_n, &ttft);
    double sum = 0;
    for (int i = 0; i < a->n_tokens; i++) sum += tok_ms[i];
    double tpot = a->n_tokens ? sum / a->n_tokens : 0;
    double total_s = (sum + ttft) / 1000.0;
    double tps = total_s > 0 ? a->n_tokens / total_s : 0;
    double p50, p95, p99;
    percentiles(tok_ms, a->n_tokens, &p50, &p95, &p99);
    char *text = a->no_print ? NULL : tokenizer_decode(&g->tok, ids, out_n);
    FILE *o = a->output ? fopen(a->output, "w") : stdout;
    if (!o) { perror(a->output); return 1; }
    fprintf(o, "{\n  \"mode\": \"generate\",\n");
    emit_common(o, g, a);
    fprintf(o, "  \"batch\": %d,\n  \"load_time_ms\": %.3f,\n", a->batch, a->load_time_ms);
    emit_affinity(o, aff);
    fprintf(o, ",\n  \"n_prompt_tokens\": %d,\n  \"n_generated_tokens\": %d,\n", n, a->n_tokens);
    fprintf(o, "  \"ttft_ms\": %.3f,\n  \"cold_start_ms\": %.3f,\n", ttft, a->load_time_ms + ttft);
    fprintf(o, "  \"tpot_avg_ms\": %.3f,\n  \"tokens_per_sec\": %.3f,\n", tpot, tps);
    fprintf(o, "  \"p50_ms\": %.3f,\n  \"p95_ms\": %.3f,\n  \"p99_ms\": %.3f,\n", p50, p95, p99);
    fprintf(o, "  \"token_ids\": [");
    for (int i = n; i < out_n; i++) fprintf(o, "%s%d", i > n ? "," : "", ids[i]);
    fprintf(o, "],\n  \"peak_rss_gb\": %.3f", peak_rss_gb());
    if (text) {
        fprintf(o, ",\n  \"text\": ");
        json_str(o, text);
    }
    fprintf(o, "\n}\n");
    if (a->output) fclose(o);
    if (text) { printf("%s\n", text); free(text); }
    free(ids);
    free(tok_ms);
    return 0;
}

static int mode_logits(GPT2 *g, const Args *a, const Affinity *aff)
{
    int toks[4096], n;
    if (load_prompt(g, a, toks, 4096, &n)) { fprintf(stderr, "prompt load failed\n"); return 1; }
    if (n < 1) return 1;
    if (n > a->logits_limit) n = a->logits_limit;
    if (n > gpt2_eff_ctx(g)) {
        fprintf(stderr, "prompt (%d) exceeds the context (%d); raise --max-ctx\n", n, gpt2_eff_ctx(g));
        return 2;
    }
    int V = g->vocab;
    int *pos = malloc((size_t)n * sizeof(int)), *seq = malloc((size_t)n * sizeof(int));
    float *logits = malloc((size_t)n * V * sizeof(float));
    for (int i = 0; i < n; i++) { pos[i] = i; seq[i] = 0; }
    if (gpt2_kv_reset(g) || gpt2_forward_ex(g, toks, pos, seq, n, 0, logits, NULL)) die_forward();
    if (a->logits_bin) {
        FILE *b = fopen(a->logits_bin, "wb");
        if (!b) { perror("logits bin"); return 1; }
        int32_t hdr[2] = {n, V};
        fwrite(hdr, 4, 2, b);
        fwrite(toks, 4, (size_t)n, b);
        fwrite(logits, 4, (size_t)n * V, b);
        fclose(b);
    }
    FILE *o = a->output ? fopen(a->output, "w") : stdout;
    if (!o) { perror(a->output); return 1; }
    fprintf(o, "{\n");
    emit_common(o, g, a);
    fprintf(o, "  \"load_time_ms\": %.3f,\n", a->load_time_ms);
    emit_affinity(o, aff);
    fprintf(o, ",\n  \"n_tokens\": %d,\n  \"tokens\": [", n);
    for (int i = 0; i < n; i++) fprintf(o, "%s%d", i ? "," : "", toks[i]);
    fprintf(o, "],\n  \"logits\": [\n");
    for (int i = 0; i < n; i++) {
        fprintf(o, "    [");
        for (int j = 0; j < V; j++) {
            float v = logits[(size_t)i * V + j];
            if (j) fputc(',', o);
            if (isfinite(v)) fprintf(o, "%.6g", v);
            else fputs("null", o);
        }
        fprintf(o, "]%s\n", i + 1 < n ? "," : "");
    }
    fprintf(o, "  ]\n}\n");
    if (a->output) fclose(o);
    free(pos); free(seq); free(logits);
    return 0;
}

static int mode_bench(GPT2 *g, const Args *a, const Affinity *aff)
{
    int toks[4096], n;
    if (load_prompt(g, a, toks, 4096, &n)) { fprintf(stderr, "prompt load failed\n"); return 1; }
    if (n < 1) { fprintf(stderr, "empty prompt\n"); return 1; }
    int eff = gpt2_eff_ctx(g);
    if (n > eff - 8) n = eff - 8;
    if (n < 1 || n + a->n_tokens > eff) {
        fprintf(stderr, "prompt (%d) + n-tokens (%d) exceeds the context (%d); raise --max-ctx\n", n, a->n_tokens, eff);
        return 2;
    }
    int nt = a->n_tokens;
    int total_gen = a->batch * nt;
    double *tok_ms = malloc((size_t)(nt > 0 ? nt : 1) * sizeof(double));
    int *ids = malloc((size_t)(n + nt + 8) * sizeof(int));
    for (int w = 0; w < a->warmup; w++) {
        double ttft; int out_n;
        gen_and_measure(g, toks, n, nt, a->batch, 0, 0, tok_ms, ids, &out_n, &ttft);
    }
    int iters = a->iters > 0 ? a->iters : 1;
    double *all_ms = malloc((size_t)(total_gen * iters + 1) * sizeof(double));
    double *ttfts = malloc((size_t)iters * sizeof(double));
    double step_sum = 0;
    int idx = 0;
    for (int it = 0; it < iters; it++) {
        double ttft; int out_n;
        gen_and_measure(g, toks, n, nt, a->batch, 0, 0, tok_ms, ids, &out_n, &ttft);
        ttfts[it] = ttft;
        for (int i = 0; i < nt; i++) {
            step_sum += tok_ms[i];
            for (int b = 0; b < a->batch; b++) all_ms[idx++] = tok_ms[i];
        }
    }
    int N = idx;
    double sum = 0;
    for (int i = 0; i < N; i++) sum += all_ms[i];
    double avg = N ? sum / N : 0, p50, p95, p99, t50, t95, t99;
    percentiles(all_ms, N, &p50, &p95, &p99);
    percentiles(ttfts, iters, &t50, &t95, &t99);
    double ttft_avg = 0;
    for (int i = 0; i < iters; i++) ttft_avg += ttfts[i] / iters;
    double gen_s = sum / 1000.0;
    double tps = gen_s > 0 ? N / gen_s : 0;
    double agg = step_sum > 0 ? (double)total_gen * iters / (step_sum / 1000.0) : 0;
    double dbytes = decode_bytes(g, a->batch, n + (nt - 1) / 2.0);
    double step_avg_s = iters * nt > 0 ? step_sum / 1000.0 / (iters * nt) : 0;
    FILE *o = a->output ? fopen(a->output, "w") : stdout;
    if (!o) { perror(a->output); return 1; }
    fprintf(o, "{\n  \"mode\": \"bench\",\n");
    emit_common(o, g, a);
    fprintf(o, "  \"batch\": %d,\n  \"load_time_ms\": %.3f,\n", a->batch, a->load_time_ms);
    emit_affinity(o, aff);
    fprintf(o, ",\n  \"n_prompt_tokens\": %d,\n  \"n_generated_tokens\": %d,\n  \"iterations\": %d,\n", n,
            total_gen, iters);
    fprintf(o, "  \"avg_token_ms\": %.3f,\n  \"p50_ms\": %.3f,\n  \"p95_ms\": %.3f,\n  \"p99_ms\": %.3f,\n", avg,
            p50, p95, p99);
    fprintf(o, "  \"ttft_avg_ms\": %.3f,\n  \"cold_start_ms\": %.3f,\n", ttft_avg, a->load_time_ms + ttft_avg);
    fprintf(o, "  \"ttft_p50_ms\": %.3f,\n  \"ttft_p95_ms\": %.3f,\n  \"ttft_p99_ms\": %.3f,\n", t50, t95, t99);
    fprintf(o, "  \"tokens_per_sec\": %.3f,\n  \"tokens_per_sec_aggregate\": %.3f,\n", tps, agg);
    fprintf(o, "  \"decode_bytes_per_step\": %.0f,\n  \"decode_gbps\": %.2f,\n", dbytes,
            step_avg_s > 0 ? dbytes / step_avg_s / 1e9 : 0.0);
    fprintf(o, "  \"total_generation_sec\": %.3f,\n  \"peak_rss_gb\": %.3f\n}\n", gen_s, peak_rss_gb());
    if (a->output) fclose(o);
    free(tok_ms); free(ids); free(all_ms); free(ttfts);
    return 0;
}

int main(int argc, char **argv)
{
    Args a;
    memset(&a, 0, sizeof a);
    a.mode = "generate"; a.precision = "auto"; a.affinity = "none";
    a.threads = 1; a.batch = 1; a.n_tokens = 32; a.warmup = 1; a.iters = 1; a.logits_limit = 1024;
    a.seed = 42;
    a.prompt = "The quick brown fox jumps over the lazy dog";
    if (argc < 2) { usage(argv[0]); return 2; }
    for (int i = 1; i < argc; i++) {
        const char *s = argv[i];
#define VAL() (i + 1 < argc ? argv[++i] : (fprintf(stderr, "missing value for %s\n", s), exit(2), ""))
        if (!strcmp(s, "--model")) a.model = VAL();
        else if (!strcmp(s, "--mode")) a.mode = VAL();
        else if (!strcmp(s, "--precision")) a.precision = VAL();
        else if (!strcmp(s, "--threads")) a.threads = atoi(VAL());
        else if (!strcmp(s, "--batch")) a.batch = atoi(VAL());
        else if (!strcmp(s, "--prompt")) a.prompt = VAL();
        else if (!strcmp(s, "--tokens-file")) a.tokens_file = VAL();
        else if (!strcmp(s, "--n-tokens")) a.n_tokens = atoi(VAL());
        else if (!strcmp(s, "--temp")) a.temp = (float)atof(VAL());
        else if (!strcmp(s, "--top-k")) a.top_k = atoi(VAL());
        else if (!strcmp(s, "--seed")) a.seed = atoi(VAL());
        else if (!strcmp(s, "--warmup")) a.warmup = atoi(VAL());
        else if (!strcmp(s, "--iters")) a.iters = atoi(VAL());
        else if (!strcmp(s, "--logits-limit")) a.logits_limit = atoi(VAL());
        else if (!strcmp(s, "--max-ctx")) a.max_ctx = atoi(VAL());
        else if (!strcmp(s, "--output")) a.output = VAL();
        else if (!strcmp(s, "--affinity")) a.affinity = VAL();
        else if (!strcmp(s, "--logits-bin")) a.logits_bin = VAL();
        else if (!strcmp(s, "--no-print")) a.no_print = 1;
        else { fprintf(stderr, "unknown arg: %s\n", s); usage(argv[0]); return 2; }
#undef VAL
    }
    if (!a.model) { usage(argv[0]); return 2; }
    if (a.batch < 1) a.batch = 1;
    if (a.n_tokens < 0) a.n_tokens = 0;
    rng_state = (unsigned long long)(unsigned long)a.seed;
    Affinity aff;
    affinity_apply(a.affinity, &aff);
    int want = -1;
    if (!strcmp(a.precision, "fp16")) want = 1;
    else if (!strcmp(a.precision, "bf16")) want = 2;
    else if (!strcmp(a.precision, "int8")) want = 0;
    else if (strcmp(a.precision, "auto")) {
        fprintf(stderr, "unknown precision: %s (use fp16|bf16|int8|auto)\n", a.precision);
        return 2;
    }
    GPT2 g;
    double t0 = now_sec();
    if (gpt2_load(&g, a.model, a.batch, a.max_ctx) != 0) {
        fprintf(stderr, "failed to load model\n");
        return 1;
    }
    a.load_time_ms = (now_sec() - t0) * 1000.0;
    const char *have = g.precision == 2 ? "bf16" : (g.precision ? "fp16" : "int8");
    if (want >= 0 && want != g.precision) {
        fprintf(stderr, "model file uses %s weights, but --precision %s was requested\n", have, a.precision);
        gpt2_free(&g);
        return 2;
    }
    a.precision = have;
    int rc;
    if (!strcmp(a.mode, "generate")) rc = mode_generate(&g, &a, &aff);
    else if (!strcmp(a.mode, "logits")) rc = mode_logits(&g, &a, &aff);
    else if (!strcmp(a.mode, "bench")) rc = mode_bench(&g, &a, &aff);
    else { fprintf(stderr, "unknown mode: %s\n", a.mode); rc = 2; }
    gpt2_free(&g);
    return rc;
}
