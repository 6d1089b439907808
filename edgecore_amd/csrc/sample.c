/*
 * Token sampling of the reference driver (src/runtime_main.c:205-248):
 * greedy argmax at temp <= 0, otherwise a top-k softmax at temperature temp
 * drawn with the driver's 64-bit LCG.
 *
 * ec_sample_full restates sample_token on a whole logits row.
 * ec_sample_candidates gives the same token, and advances the generator the
 * same way, from the row's top_k + 1 largest logits only (value descending,
 * index ascending), as the device selection returns them (ec_topk_dev).  That
 * is exact when the row has no NaN and the top_k-th and (top_k+1)-th values
 * differ (the device reports both); for other rows the caller uses the full
 * row.  The reference selects by a selection sort with swaps over an index
 * array, so among equal logits it takes the one at the smallest current
 * position, and each swap moves the element that sat at the front.  This
 * restatement tracks the positions of the candidates through those swaps:
 * under the two conditions above every pick is a candidate.
 */
#include "edgecore.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>

unsigned ec_rng_next(unsigned long long *state)
{
    *state = *state * 6364136223846793005ULL + 1442695040888963407ULL;
    return (unsigned)(*state >> 33);
}

/* softmax over the n picked logits (picked in selection order) and the draw */
static int draw(const float *lv, const int *li, int n, float temp, unsigned long long *state)
{
    const float maxl = lv[0];
    float *p = malloc((size_t)n * sizeof(float));
    if (!p) return li[n - 1];
    double sum = 0.0;
    for (int i = 0; i < n; i++) {
        const float d = (lv[i] - maxl) / temp;
        p[i] = expf(d);
        sum += p[i];
    }
    const double r = (double)ec_rng_next(state) / (double)0xffffffffu;
    double acc = 0.0;
    int pick = li[n - 1];
    for (int i = 0; i < n; i++) {
        acc += p[i] / sum;
        if (r < acc) {
            pick = li[i];
            break;
        }
    }
    free(p);
    return pick;
}

int ec_sample_full(const float *logits, int vocab, float temp, int top_k, unsigned long long *state)
{
    if (temp <= 0.0f) {
        int best = 0;
        for (int i = 1; i < vocab; i++)
            if (logits[i] > logits[best]) best = i;
        return best;
    }
    int *pos = malloc((size_t)vocab * sizeof(int));
    float *lv = malloc((size_t)vocab * sizeof(float));
    if (!pos || !lv) {
        free(pos);
        free(lv);
        return 0;
    }
    for (int i = 0; i < vocab; i++) pos[i] = i;
    for (int i = 0; i < top_k && i < vocab; i++) {
        int best = i;
        for (int j = i + 1; j < vocab; j++)
            if (logits[pos[j]] > logits[pos[best]]) best = j;
        const int t = pos[i];
        pos[i] = pos[best];
        pos[best] = t;
    }
    const int n = top_k > 0 && top_k < vocab ? top_k : vocab;
    for (int i = 0; i < n; i++) lv[i] = logits[pos[i]];
    const int pick = draw(lv, pos, n, temp, state);
    free(pos);
    free(lv);
    return pick;
}

int ec_sample_candidates(const float *vals, const int *idx, int ncand, int vocab, float temp, int top_k,
                         unsigned long long *state)
{
    if (temp <= 0.0f || top_k <= 0 || top_k >= vocab || ncand < top_k + 1) return -1;
    int *at = malloc((size_t)ncand * sizeof(int));  /* current position of each candidate */
    int *li = malloc((size_t)top_k * sizeof(int));
    float *lv = malloc((size_t)top_k * sizeof(float));
    if (!at || !li || !lv) {
        free(at);
        free(li);
        free(lv);
        return -1;
    }
    for (int c = 0; c < ncand; c++) at[c] = idx[c];
    for (int i = 0; i < top_k; i++) {
        /* the first position >= i holding the largest remaining value */
        int best = -1;
        for (int c = 0; c < ncand; c++) {
            if (at[c] < i) continue;
            if (best < 0 || vals[c] > vals[best] || (!(vals[best] > vals[c]) && at[c] < at[best])) best = c;
        }
        /* swap: the element at position i (a candidate or not) takes best's place */
        for (int c = 0; c < ncand; c++)
            if (at[c] == i) {
                at[c] = at[best];
                break;
            }
        at[best] = i;
        li[i] = idx[best];
        lv[i] = vals[best];
    }
    const int pick = draw(lv, li, top_k, temp, state);
    free(at);
    free(li);
    free(lv);
    return pick;
}
