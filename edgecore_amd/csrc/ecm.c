/*
 * Host side of the .ecm format and small host utilities of the library:
 * ecm_parse (src/gpt2.c:11-136 of the reference), the int8 weight packer
 * (edgecore/ecm.py:50-59), now_sec / peak_rss_gb (src/runtime_main.c:10-28).
 */
#define _GNU_SOURCE
#include "edgecore.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

double now_sec(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

float peak_rss_gb(void)
{
    FILE *f = fopen("/proc/self/status", "r");
    if (!f) return 0.0f;
    char line[256];
    unsigned long kb = 0;
    while (fgets(line, sizeof line, f))
        if (!strncmp(line, "VmHWM:", 6)) {
            sscanf(line + 6, "%lu", &kb);
            break;
        }
    fclose(f);
    return (float)kb / 1048576.0f;
}

/* ------------------------------------------------------------------ */
/* .ecm header                                                          */
/* ------------------------------------------------------------------ */

static size_t ecm_dtype_bytes(int dtype)
{
    switch (dtype) {
    case 0: return 4;
    case 1: return 2;
    case 2: return 1;
    case 4: return 2;
    default: return 0;
    }
}

/* Copies one line (without '\r' and '\n') into buf; returns the position
 * after it, or NULL at the end of the data with nothing read. */
static const char *ecm_line(const char *p, const char *end, char *buf, size_t cap)
{
    size_t n = 0;
    while (p < end && *p != '\n') {
        if (*p != '\r' && n + 1 < cap) buf[n++] = *p;
        p++;
    }
    buf[n] = 0;
    if (p < end) return p + 1;
    return n ? p : NULL;
}

static void ecm_meta(GPT2 *m, const char *key, const char *val)
{
    if (!strcmp(key, "model_name")) snprintf(m->model_name, sizeof m->model_name, "%s", val);
    else if (!strcmp(key, "n_layer")) m->n_layer = atoi(val);
    else if (!strcmp(key, "n_head")) m->n_head = atoi(val);
    else if (!strcmp(key, "n_kv_head")) m->n_kv_head = atoi(val);
    else if (!strcmp(key, "intermediate")) m->intermediate = atoi(val);
    else if (!strcmp(key, "n_embd")) m->n_embd = atoi(val);
    else if (!strcmp(key, "n_ctx")) m->n_ctx = atoi(val);
    else if (!strcmp(key, "vocab")) m->vocab = atoi(val);
    else if (!strcmp(key, "n_params")) m->n_params = (size_t)strtoull(val, NULL, 10);
    else if (!strcmp(key, "eps")) m->eps = atof(val);
    else if (!strcmp(key, "rope_theta")) m->rope_theta = atof(val);
    else if (!strcmp(key, "rope_type")) m->rope_type = !strcmp(val, "yarn") ? ROPE_YARN : ROPE_DEFAULT;
    else if (!strcmp(key, "yarn_factor")) m->yarn_factor = atof(val);
    else if (!strcmp(key, "yarn_attention_factor")) m->yarn_attention_factor = atof(val);
    else if (!strcmp(key, "yarn_orig_max")) m->yarn_orig_max = atof(val);
    else if (!strcmp(key, "sliding_window")) m->sliding_window = atoi(val);
    else if (!strcmp(key, "tie_word_embeddings")) m->tie_word_embeddings = atoi(val);
    else if (!strcmp(key, "eos_token_id")) m->eos_token_id = atoi(val);
    else if (!strcmp(key, "arch"))
        m->arch = (!strcmp(val, "qwen2") || !strcmp(val, "olmo3")) ? ARCH_QWEN2 : ARCH_GPT2;
}

int ecm_parse(const void *data, size_t size, EcmTensor *out, int max, GPT2 *meta)
{
    const char *p = (const char *)data, *end = p + size;
    char line[1024];
    if (size < 5 || memcmp(p, ECM_MAGIC, 5) != 0) {
        fprintf(stderr, "ecm: bad magic\n");
        return -1;
    }
    p += 5;
    for (;;) {
        p = ecm_line(p, end, line, sizeof line);
        if (!p) return -1;
        if (!strcmp(line, "END_META")) break;
        char *eq = strchr(line, '=');
        if (!eq) continue;
        *eq = 0;
        ecm_meta(meta, line, eq + 1);
    }
    int n = 0;
    for (;;) {
        p = ecm_line(p, end, line, sizeof line);
        if (!p) return -1;
        if (!strcmp(line, "END_TENSORS")) break;
        char name[128], dt[16];
        if (sscanf(line, "%127s %15s", name, dt) < 2) continue;
        int dtype;
        if (!strcmp(dt, "fp32")) dtype = 0;
        else if (!strcmp(dt, "fp16")) dtype = 1;
        else if (!strcmp(dt, "int8")) dtype = 2;
        else if (!strcmp(dt, "text")) dtype = 3;
        else if (!strcmp(dt, "bf16")) dtype = 4;
        else continue;
        EcmTensor *t = &out[n];
        memset(t, 0, sizeof *t);
        snprintf(t->name, sizeof t->name, "%s", name);
        t->dtype = dtype;
        const char *q = line;
        for (int f = 0; f < 2; f++) {
            while (*q == ' ') q++;
            while (*q && *q != ' ') q++;
        }
        if (dtype == 3) {
            t->ndims = 1;
            t->dims[0] = (size_t)strtoull(q, NULL, 10);
            t->nelems = t->bytes = t->dims[0];
        } else {
            t->nelems = 1;
            while (*q && t->ndims < 4) {
                while (*q == ' ') q++;
                if (!*q) break;
                char *e2;
                size_t d = (size_t)strtoull(q, &e2, 10);
                if (e2 == q) break;
                t->dims[t->ndims++] = d;
                t->nelems *= d;
                q = e2;
            }
            t->bytes = t->nelems * ecm_dtype_bytes(dtype);
        }
        /* the reference fails once the table holds `max` entries (src/gpt2.c:126) */
        if (++n >= max) return -1;
    }
    size_t off = (size_t)(p - (const char *)data);
    for (int i = 0; i < n; i++) {
        out[i].offset = off;
        off += out[i].bytes;
    }
    return n;
}

/* ------------------------------------------------------------------ */
/* weight packer                                                        */
/* ------------------------------------------------------------------ */

/* edgecore/ecm.py:50-59, in float64 as numpy computes it: max|w| (NaN
 * propagates, as numpy's max does), scale = max/127 (1.0 when 0), code =
 * clip(rint(w/scale)); numpy's float64 -> int32 cast gives INT32_MIN for a
 * NaN quotient on x86-64, which the clip turns into -128. */
void ec_quantize_int8_symmetric(const float *w, int rows, int cols, int8_t *q, float *scales)
{
    for (int r = 0; r < rows; r++) {
        const float *row = w + (size_t)r * cols;
        double maxabs = 0.0;
        for (int c = 0; c < cols; c++) {
            double a = fabs((double)row[c]);
            if (isnan(a)) { maxabs = a; break; }
            if (a > maxabs) maxabs = a;
        }
        double s = maxabs / 127.0;
        if (s == 0.0) s = 1.0;
        int8_t *qr = q + (size_t)r * cols;
        for (int c = 0; c < cols; c++) {
            double v = nearbyint((double)row[c] / s);
            qr[c] = (int8_t)(isnan(v) ? -128 : v > 127.0 ? 127 : v < -128.0 ? -128 : (int)v);
        }
        scales[r] = (float)s;
    }
}

/* edgecore/ecm.py:27-41: fp32 -> bfloat16 bits, round to nearest even,
 * every NaN to the quiet NaN 0x7fc0 */
uint16_t ec_f32_to_bf16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    const uint32_t lsb = (x >> 16) & 1u;
    return (uint16_t)(((uint64_t)x + 0x7fffu + lsb) >> 16);
}

