/*
 * Harness around the reference CPU runtime, built from the reference's own
 * sources (src/gpt2.c, src/kernels.c, src/tokenizer.c) into oracle/_ref/ by
 * oracle/Makefile -- TEST INFRASTRUCTURE ONLY, used to pin the oracle and to
 * write golden fixtures in the development container (the reference tree is
 * not present where the GPU runs).
 *
 * It drives gpt2_forward exactly the way src/runtime_main.c does:
 *   - refh_logits:   mode_logits (src/runtime_main.c:435-452)
 *   - refh_generate: gen_and_measure at batch 1, greedy (src/runtime_main.c:293-362)
 */
#include "edgecore.h" /* the reference header, from -I <reference>/src */

#define REFH_MAX 8
static GPT2 g_models[REFH_MAX];
static int g_used[REFH_MAX];

int refh_open(const char *path, int batch_cap, int max_ctx)
{
    for (int i = 0; i < REFH_MAX; i++) {
        if (g_used[i]) continue;
        if (gpt2_load(&g_models[i], path, batch_cap, max_ctx) != 0) return -1;
        g_used[i] = 1;
        return i;
    }
    return -1;
}

void refh_close(int h)
{
    if (h < 0 || h >= REFH_MAX || !g_used[h]) return;
    gpt2_free(&g_models[h]);
    g_used[h] = 0;
}

int refh_vocab(int h) { return g_models[h].vocab; }
int refh_eff_ctx(int h) { return gpt2_eff_ctx(&g_models[h]); }
int refh_precision(int h) { return g_models[h].precision; }

static void refh_kv_zero(GPT2 *g)
{
    size_t kv = (size_t)g->n_layer * (size_t)g->batch_cap * (size_t)gpt2_eff_ctx(g) *
                (size_t)g->n_kv_embd;
    memset(g->k_cache, 0, kv * sizeof(uint16_t));
    memset(g->v_cache, 0, kv * sizeof(uint16_t));
}

/* raw forward (caller manages the KV cache) */
void refh_forward(int h, const int *tokens, const int *positions, const int *seqs,
                  int M, float *logits)
{
    gpt2_forward(&g_models[h], tokens, positions, seqs, M, logits);
}

void refh_kv_reset(int h) { refh_kv_zero(&g_models[h]); }

int refh_logits(int h, const int *toks, int n, float *logits)
{
    GPT2 *g = &g_models[h];
    if (n < 1 || n > gpt2_eff_ctx(g)) return -1;
    int *pos = malloc((size_t)n * sizeof(int)), *seq = malloc((size_t)n * sizeof(int));
    for (int i = 0; i < n; i++) { pos[i] = i; seq[i] = 0; }
    refh_kv_zero(g);
    gpt2_forward(g, toks, pos, seq, n, logits);
    free(pos);
    free(seq);
    return 0;
}

int refh_generate(int h, const int *prompt, int n, int n_gen, int *out_ids,
                  float *step_logits)
{
    GPT2 *g = &g_models[h];
    int V = g->vocab;
    if (n < 1 || n + n_gen > gpt2_eff_ctx(g)) return -1;
    int *pos = malloc((size_t)n * sizeof(int)), *seq = malloc((size_t)n * sizeof(int));
    float *lg = malloc((size_t)n * V * sizeof(float));
    for (int i = 0; i < n; i++) { pos[i] = i; seq[i] = 0; }
    memcpy(out_ids, prompt, (size_t)n * sizeof(int));
    refh_kv_zero(g);
    gpt2_forward(g, prompt, pos, seq, n, lg);
    int cur = prompt[n - 1], npos = n;
    for (int i = 0; i < n_gen; i++) {
        gpt2_forward(g, &cur, &npos, NULL, 1, lg);
        if (step_logits) memcpy(step_logits + (size_t)i * V, lg, (size_t)V * sizeof(float));
        int best = 0; /* sample_token greedy, src/runtime_main.c:215-218 */
        for (int v = 1; v < V; v++)
            if (lg[v] > lg[best]) best = v;
        cur = best;
        out_ids[n + i] = cur;
        npos++;
    }
    free(pos);
    free(seq);
    free(lg);
    return 0;
}
