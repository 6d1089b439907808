/*
 * Byte-level BPE tokenizer of the .ecm files (src/tokenizer.c:500-1186 of the
 * reference; blobs written by edgecore/ecm.py:127-171).  Host code, used by
 * the driver for --prompt and for the decoded text.
 *
 *   vocab blob:  u32 count, then count x (u32 id, u32 len, len bytes)
 *   merges blob: u32 count, then count x (u32 len, bytes, u32 len, bytes)
 *
 * Behaviour kept from the reference:
 *   - every raw byte b is the token whose text is the UTF-8 form of GPT-2's
 *     bytes_to_unicode code point for b (printable Latin-1 bytes map to
 *     themselves, the other 68 to 256, 257, ... in byte order);
 *   - a merge is kept when both halves and their concatenation are in the
 *     vocabulary; encoding applies the kept merges in file order, each once
 *     over the whole piece, left to right, non-overlapping (not the
 *     lowest-rank-pair-first loop of other BPE implementations);
 *   - text is cut into pieces by a byte scanner approximating the GPT-2
 *     regex (variant 0) or Qwen2's (variant 1); every byte >= 0x80 counts as
 *     a letter;
 *   - vocabulary entries of the form <|...|> are special tokens: matched
 *     longest first before any piece is cut, and emitted verbatim by decode;
 *   - a byte with no token encodes as its own value; decode maps unknown ids
 *     to id 0 and unmapped code points to their low byte.
 */
#include "edgecore.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---- byte classes ------------------------------------------------------ */

static int is_ws(uint8_t b) { return b == ' ' || (b >= '\t' && b <= '\r'); }
static int is_nl(uint8_t b) { return b == '\n' || b == '\r'; }
static int is_alpha(uint8_t b) { return (b | 0x20) >= 'a' && (b | 0x20) <= 'z' ? 1 : b >= 0x80; }
static int is_num(uint8_t b) { return b >= '0' && b <= '9'; }
static int is_other(uint8_t b) { return !is_ws(b) && !is_alpha(b) && !is_num(b); }

static size_t run_of(const uint8_t *s, size_t n, size_t j, int (*cls)(uint8_t))
{
    while (j < n && cls(s[j])) j++;
    return j;
}

/* ---- pre-tokenizers: length of the piece that starts at s[i] ----------- */

static size_t piece_gpt2(const uint8_t *s, size_t n, size_t i)
{
    /* contractions 's 't 're 've 'm 'll 'd (case-sensitive) */
    if (s[i] == '\'' && i + 1 < n) {
        const uint8_t c = s[i + 1];
        if (c == 's' || c == 't' || c == 'm' || c == 'd') return 2;
        if (i + 2 < n && ((c == 'r' && s[i + 2] == 'e') || (c == 'v' && s[i + 2] == 'e') ||
                          (c == 'l' && s[i + 2] == 'l')))
            return 3;
    }
    /* an optional leading space, then a run of letters, digits or others */
    const size_t j = i + (s[i] == ' ' ? 1 : 0);
    if (j < n && (j > i || !is_ws(s[j]))) {
        if (is_alpha(s[j])) return run_of(s, n, j, is_alpha) - i;
        if (is_num(s[j])) return run_of(s, n, j, is_num) - i;
        if (!is_ws(s[j])) return run_of(s, n, j, is_other) - i;
    }
    return run_of(s, n, i, is_ws) - i;  /* whitespace */
}

static int lower(uint8_t c) { return c >= 'A' && c <= 'Z' ? c + 32 : c; }

static size_t piece_qwen2(const uint8_t *s, size_t n, size_t i)
{
    /* '(?i:[sdmt]|ll|ve|re) */
    if (s[i] == '\'') {
        const int c1 = i + 1 < n ? lower(s[i + 1]) : 0;
        if (c1 == 's' || c1 == 'd' || c1 == 'm' || c1 == 't') return 2;
        if (i + 2 < n) {
            const int c2 = lower(s[i + 2]);
            if ((c1 == 'l' && c2 == 'l') || (c1 == 'v' && c2 == 'e') || (c1 == 'r' && c2 == 'e')) return 3;
        }
    }
    /* [^\r\n\p{L}\p{N}]?\p{L}+ */
    if (!is_nl(s[i]) && !is_alpha(s[i]) && !is_num(s[i]) && i + 1 < n && is_alpha(s[i + 1]))
        return run_of(s, n, i + 1, is_alpha) - i;
    if (is_alpha(s[i])) return run_of(s, n, i, is_alpha) - i;
    /* \p{N}{1,3} */
    if (is_num(s[i])) {
        size_t j = i;
        while (j < n && j < i + 3 && is_num(s[j])) j++;
        return j - i;
    }
    /*  ?[^\s\p{L}\p{N}]+[\r\n]* */
    {
        const size_t j0 = i + (s[i] == ' ' ? 1 : 0);
        const size_t j = run_of(s, n, j0, is_other);
        if (j > j0) return run_of(s, n, j, is_nl) - i;
    }
    /* \s*[\r\n]+ : through the last newline of the whitespace run */
    const size_t w = run_of(s, n, i, is_ws);
    size_t k = w;
    while (k > i && !is_nl(s[k - 1])) k--;
    if (k > i) return k - i;
    /* \s+(?!\S): a run followed by a non-space leaves its last byte */
    if (w > i) {
        if (w >= n) return w - i;
        if (w > i + 1) return w - i - 1;
        return w - i;  /* \s+ */
    }
    return 1;
}

/* ---- string -> id map used while loading ------------------------------- */

typedef struct {
    const char *key;
    uint32_t len;
    int32_t id;
} Slot;

typedef struct {
    Slot *slot;
    size_t mask;
} Map;

static uint64_t hash_bytes(const char *p, uint32_t n)
{
    uint64_t h = 0xcbf29ce484222325ull;
    for (uint32_t i = 0; i < n; i++) h = (h ^ (uint8_t)p[i]) * 0x100000001b3ull;
    return h;
}

static int map_init(Map *m, size_t n)
{
    size_t cap = 64;
    while (cap < 2 * n + 2) cap <<= 1;
    m->slot = (Slot *)calloc(cap, sizeof(Slot));
    m->mask = cap - 1;
    return m->slot ? 0 : -1;
}

/* the first id given for a text wins */
static void map_put(Map *m, const char *key, uint32_t len, int32_t id)
{
    size_t h = (size_t)hash_bytes(key, len) & m->mask;
    while (m->slot[h].key) {
        if (m->slot[h].len == len && !memcmp(m->slot[h].key, key, len)) return;
        h = (h + 1) & m->mask;
    }
    m->slot[h].key = key;
    m->slot[h].len = len;
    m->slot[h].id = id;
}

static int32_t map_get(const Map *m, const char *key, uint32_t len)
{
    size_t h = (size_t)hash_bytes(key, len) & m->mask;
    while (m->slot[h].key) {
        if (m->slot[h].len == len && !memcmp(m->slot[h].key, key, len)) return m->slot[h].id;
        h = (h + 1) & m->mask;
    }
    return -1;
}

/* ---- load / free ------------------------------------------------------- */

static uint32_t get32(const uint8_t **p)
{
    uint32_t v;
    memcpy(&v, *p, 4);
    *p += 4;
    return v;
}

static int utf8_put(uint32_t cp, char *o)
{
    if (cp < 0x80) {
        o[0] = (char)cp;
        return 1;
    }
    if (cp < 0x800) {
        o[0] = (char)(0xC0 | (cp >> 6));
        o[1] = (char)(0x80 | (cp & 0x3F));
        return 2;
    }
    o[0] = (char)(0xE0 | (cp >> 12));
    o[1] = (char)(0x80 | ((cp >> 6) & 0x3F));
    o[2] = (char)(0x80 | (cp & 0x3F));
    return 3;
}

static int special_text(const char *s, size_t len)
{
    return len >= 4 && s[0] == '<' && s[1] == '|' && s[len - 2] == '|' && s[len - 1] == '>';
}

int tokenizer_load(Tokenizer *t, const void *vocab_blob, size_t vocab_bytes,
                   const void *merges_blob, size_t merges_bytes, int vocab_size, int variant)
{
    memset(t, 0, sizeof *t);
    t->vocab_size = vocab_size;
    t->variant = variant;
    t->eos_id = -1;
    if (vocab_size <= 0 || vocab_bytes < 4) return -1;
    t->id_to_token = (char **)calloc((size_t)vocab_size, sizeof(char *));
    t->byte_to_id = (int32_t *)malloc(256 * sizeof(int32_t));
    t->cp_to_byte = (int32_t *)malloc(512 * sizeof(int32_t));
    if (!t->id_to_token || !t->byte_to_id || !t->cp_to_byte) return -1;

    const uint8_t *p = (const uint8_t *)vocab_blob, *end = p + vocab_bytes;
    const uint32_t count = get32(&p);
    Map map;
    if (map_init(&map, count)) return -1;
    for (uint32_t i = 0; i < count && end - p >= 8; i++) {
        const uint32_t id = get32(&p), len = get32(&p);
        if ((size_t)(end - p) < len) break;
        if (id < (uint32_t)vocab_size) {
            char *txt = (char *)malloc((size_t)len + 1);
            if (!txt) break;
            memcpy(txt, p, len);
            txt[len] = 0;
            t->id_to_token[id] = txt;  /* a repeated id keeps its last text (earlier ones stay mapped) */
            map_put(&map, txt, len, (int32_t)id);
        }
        p += len;
    }

    /* merges kept when the halves and their concatenation are tokens */
    if (merges_bytes >= 4) {
        const uint8_t *q = (const uint8_t *)merges_blob, *qend = q + merges_bytes;
        const uint32_t nm = get32(&q);
        t->merge_l = (uint32_t *)malloc((size_t)(nm ? nm : 1) * sizeof(uint32_t));
        t->merge_r = (uint32_t *)malloc((size_t)(nm ? nm : 1) * sizeof(uint32_t));
        t->merge_m = (uint32_t *)malloc((size_t)(nm ? nm : 1) * sizeof(uint32_t));
        char *cat = NULL;
        size_t cat_cap = 0;
        if (t->merge_l && t->merge_r && t->merge_m) {
            for (uint32_t i = 0; i < nm && qend - q >= 4; i++) {
                const uint32_t la = get32(&q);
                if ((size_t)(qend - q) < la) break;
                const char *a = (const char *)q;
                q += la;
                if (qend - q < 4) break;
                const uint32_t lb = get32(&q);
                if ((size_t)(qend - q) < lb) break;
                const char *b = (const char *)q;
                q += lb;
                if ((size_t)la + lb > cat_cap) {
                    cat_cap = (size_t)la + lb;
                    char *nc = (char *)realloc(cat, cat_cap);
                    if (!nc) break;
                    cat = nc;
                }
                memcpy(cat, a, la);
                memcpy(cat + la, b, lb);
                const int32_t ia = map_get(&map, a, la), ib = map_get(&map, b, lb);
                const int32_t im = map_get(&map, cat, la + lb);
                if (ia >= 0 && ib >= 0 && im >= 0) {
                    t->merge_l[t->n_merges] = (uint32_t)ia;
                    t->merge_r[t->n_merges] = (uint32_t)ib;
                    t->merge_m[t->n_merges] = (uint32_t)im;
                    t->n_merges++;
                }
            }
        }
        free(cat);
    }

    /* bytes_to_unicode of GPT-2, and its inverse over code points < 512 */
    for (int c = 0; c < 512; c++) t->cp_to_byte[c] = -1;
    for (int b = 0, extra = 0; b < 256; b++) {
        const int kept = (b >= '!' && b <= '~') || (b >= 0xA1 && b <= 0xAC) || b >= 0xAE;
        const uint32_t cp = kept ? (uint32_t)b : 256u + (uint32_t)extra++;
        char u[4];
        const int ul = utf8_put(cp, u);
        t->byte_to_id[b] = map_get(&map, u, (uint32_t)ul);
        t->cp_to_byte[cp] = b;
    }
    t->eos_id = map_get(&map, "<|endoftext|>", 13);
    free(map.slot);

    /* special tokens, longest first (equal lengths in id order) */
    int ns = 0;
    for (int id = 0; id < vocab_size; id++)
        if (t->id_to_token[id] && special_text(t->id_to_token[id], strlen(t->id_to_token[id]))) ns++;
    if (ns) {
        t->sp_tok = (char **)malloc((size_t)ns * sizeof(char *));
        t->sp_len = (uint32_t *)malloc((size_t)ns * sizeof(uint32_t));
        t->sp_id = (int32_t *)malloc((size_t)ns * sizeof(int32_t));
        if (!t->sp_tok || !t->sp_len || !t->sp_id) return -1;
        for (int id = 0; id < vocab_size; id++) {
            char *txt = t->id_to_token[id];
            if (!txt) continue;
            const uint32_t len = (uint32_t)strlen(txt);
            if (!special_text(txt, len)) continue;
            int k = t->n_sp++;
            while (k > 0 && t->sp_len[k - 1] < len) {  /* stable insertion, by length descending */
                t->sp_tok[k] = t->sp_tok[k - 1];
                t->sp_len[k] = t->sp_len[k - 1];
                t->sp_id[k] = t->sp_id[k - 1];
                k--;
            }
            t->sp_tok[k] = txt;
            t->sp_len[k] = len;
            t->sp_id[k] = id;
        }
    }
    return 0;
}

void tokenizer_free(Tokenizer *t)
{
    if (t->id_to_token) {
        for (int i = 0; i < t->vocab_size; i++) free(t->id_to_token[i]);
        free(t->id_to_token);
    }
    free(t->byte_to_id);
    free(t->cp_to_byte);
    free(t->merge_l);
    free(t->merge_r);
    free(t->merge_m);
    free(t->sp_tok);
    free(t->sp_len);
    free(t->sp_id);
    memset(t, 0, sizeof *t);
}

/* ---- encode ------------------------------------------------------------ */

/* one piece: its bytes as tokens, then the merges in file order */
static int encode_piece(const Tokenizer *t, const uint8_t *s, size_t n, int *out, int max_out, int *total)
{
    int *ids = (int *)malloc((n ? n : 1) * sizeof(int));
    if (!ids) return -1;
    int m = 0;
    for (size_t i = 0; i < n; i++) {
        const int id = t->byte_to_id ? t->byte_to_id[s[i]] : -1;
        ids[m++] = id >= 0 ? id : s[i];
    }
    for (int r = 0; r < t->n_merges && m > 1; r++) {
        const int l = (int)t->merge_l[r], rt = (int)t->merge_r[r], mg = (int)t->merge_m[r];
        int w = 0;
        for (int i = 0; i < m;) {
            if (i + 1 < m && ids[i] == l && ids[i + 1] == rt) {
                ids[w++] = mg;
                i += 2;
            } else {
                ids[w++] = ids[i++];
            }
        }
        m = w;
    }
    int rc = 0;
    if (*total + m > max_out) {
        rc = -1;
    } else {
        memcpy(out + *total, ids, (size_t)m * sizeof(int));
        *total += m;
    }
    free(ids);
    return rc;
}

static int encode_span(const Tokenizer *t, const uint8_t *s, size_t n, int *out, int max_out, int *total)
{
    for (size_t i = 0; i < n;) {
        const size_t len = t->variant == 1 ? piece_qwen2(s, n, i) : piece_gpt2(s, n, i);
        if (encode_piece(t, s + i, len, out, max_out, total)) return -1;
        i += len;
    }
    return 0;
}

/* the special token starting at s[i], longest first, or -1 */
static int special_at(const Tokenizer *t, const uint8_t *s, size_t n, size_t i)
{
    for (int k = 0; k < t->n_sp; k++)
        if (i + t->sp_len[k] <= n && !memcmp(s + i, t->sp_tok[k], t->sp_len[k])) return k;
    return -1;
}

int tokenizer_encode(const Tokenizer *t, const char *text, int *out, int max_out)
{
    const uint8_t *s = (const uint8_t *)text;
    const size_t n = strlen(text);
    if (!strcmp(text, "<|endoftext|>")) {
        if (max_out < 1) return -1;
        out[0] = t->eos_id >= 0 ? t->eos_id : t->vocab_size - 1;
        return 1;
    }
    int total = 0;
    if (t->n_sp == 0) return encode_span(t, s, n, out, max_out, &total) ? -1 : total;
    for (size_t i = 0; i < n;) {
        const int k = special_at(t, s, n, i);
        if (k >= 0) {
            if (total + 1 > max_out) return -1;
            out[total++] = t->sp_id[k];
            i += t->sp_len[k];
            continue;
        }
        size_t next = i + 1;
        while (next < n && special_at(t, s, n, next) < 0) next++;
        if (encode_span(t, s + i, next - i, out, max_out, &total)) return -1;
        i = next;
    }
    return total;
}

/* ---- decode ------------------------------------------------------------ */

/* one UTF-8 code point (1..4 bytes; a malformed lead byte is taken alone) */
static size_t utf8_get(const uint8_t *s, size_t max, uint32_t *cp)
{
    const uint8_t c = s[0];
    if (c >= 0xC0 && c < 0xE0 && max >= 2 && (s[1] & 0xC0) == 0x80) {
        *cp = ((uint32_t)(c & 0x1F) << 6) | (s[1] & 0x3F);
        return 2;
    }
    if (c >= 0xE0 && c < 0xF0 && max >= 3 && (s[1] & 0xC0) == 0x80 && (s[2] & 0xC0) == 0x80) {
        *cp = ((uint32_t)(c & 0x0F) << 12) | ((uint32_t)(s[1] & 0x3F) << 6) | (s[2] & 0x3F);
        return 3;
    }
    if (c >= 0xF0 && c < 0xF8 && max >= 4 && (s[1] & 0xC0) == 0x80 && (s[2] & 0xC0) == 0x80 &&
        (s[3] & 0xC0) == 0x80) {
        *cp = ((uint32_t)(c & 0x07) << 18) | ((uint32_t)(s[1] & 0x3F) << 12) | ((uint32_t)(s[2] & 0x3F) << 6) |
              (s[3] & 0x3F);
        return 4;
    }
    *cp = c;
    return 1;
}

char *tokenizer_decode(const Tokenizer *t, const int *ids, int n)
{
    size_t cap = 1;
    for (int i = 0; i < n; i++) {
        const int id = ids[i] >= 0 && ids[i] < t->vocab_size && t->id_to_token[ids[i]] ? ids[i] : 0;
        if (t->id_to_token && t->id_to_token[id]) cap += strlen(t->id_to_token[id]);
    }
    char *out = (char *)malloc(cap);
    if (!out) return NULL;
    size_t o = 0;
    for (int i = 0; i < n; i++) {
        const int id = ids[i] >= 0 && ids[i] < t->vocab_size && t->id_to_token[ids[i]] ? ids[i] : 0;
        const char *tok = t->id_to_token ? t->id_to_token[id] : NULL;
        if (!tok) continue;
        const size_t len = strlen(tok);
        if (special_text(tok, len)) {
            memcpy(out + o, tok, len);
            o += len;
            continue;
        }
        for (size_t p = 0; p < len;) {
            uint32_t cp;
            p += utf8_get((const uint8_t *)tok + p, len - p, &cp);
            const int32_t b = cp < 512 && t->cp_to_byte ? t->cp_to_byte[cp] : -1;
            out[o++] = (char)(b >= 0 ? b : (int)(cp & 0xFF));
        }
    }
    out[o] = 0;
    return out;
}
