/* tokenizer.c - BPE tokenizer with the behaviour of runq.c:426-560. */
#include "tokenizer.h"

#include <ctype.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* The sort/bsearch below needs the piece table; qsort has no context
 * argument, so the table being sorted is held here for the comparator. */
static char** g_sort_pieces;

static int cmp_ids(const void* a, const void* b) {
    return strcmp(g_sort_pieces[*(const int*)a], g_sort_pieces[*(const int*)b]);
}

int tok_load(l2q_tokenizer* t, const char* path, int vocab_size, char* err, int errlen) {
    memset(t, 0, sizeof(*t));
    for (int i = 0; i < 256; i++) { t->byte_text[i][0] = (char)i; t->byte_text[i][1] = 0; }
    FILE* f = fopen(path, "rb");
    if (!f) { if (err) snprintf(err, errlen, "couldn't load %s", path); return -1; }
    t->vocab_size = vocab_size;
    t->pieces = (char**)calloc((size_t)vocab_size, sizeof(char*));
    t->scores = (float*)malloc((size_t)vocab_size * sizeof(float));
    if (!t->pieces || !t->scores) { fclose(f); if (err) snprintf(err, errlen, "malloc failed"); return -1; }
    if (fread(&t->max_token_length, 4, 1, f) != 1) goto bad;
    for (int i = 0; i < vocab_size; i++) {
        int32_t len;
        if (fread(&t->scores[i], 4, 1, f) != 1) goto bad;
        if (fread(&len, 4, 1, f) != 1 || len < 0) goto bad;
        t->pieces[i] = (char*)malloc((size_t)len + 1);
        if (!t->pieces[i]) goto bad;
        if (len && fread(t->pieces[i], (size_t)len, 1, f) != 1) goto bad;
        t->pieces[i][len] = 0;
    }
    fclose(f);
    return 0;
bad:
    fclose(f);
    if (err) snprintf(err, errlen, "failed read");
    tok_free(t);
    return -1;
}

void tok_free(l2q_tokenizer* t) {
    if (t->pieces)
        for (int i = 0; i < t->vocab_size; i++) free(t->pieces[i]);
    free(t->pieces);
    free(t->scores);
    free(t->by_text);
    memset(t, 0, sizeof(*t));
}

static void ensure_sorted(l2q_tokenizer* t) {
    if (t->by_text) return;
    t->by_text = (int*)malloc((size_t)t->vocab_size * sizeof(int));
    for (int i = 0; i < t->vocab_size; i++) t->by_text[i] = i;
    g_sort_pieces = t->pieces;
    qsort(t->by_text, (size_t)t->vocab_size, sizeof(int), cmp_ids);
}

/* Binary search over the text-sorted ids.  With duplicate piece texts any
 * matching id may be returned, as with bsearch in the reference. */
static int lookup_sorted(const l2q_tokenizer* t, const char* s) {
    int lo = 0, hi = t->vocab_size - 1;
    while (lo <= hi) {
        int mid = (lo + hi) >> 1;
        int c = strcmp(s, t->pieces[t->by_text[mid]]);
        if (c == 0) return t->by_text[mid];
        if (c < 0) hi = mid - 1; else lo = mid + 1;
    }
    return -1;
}

int tok_lookup(const l2q_tokenizer* t, const char* text) {
    ensure_sorted((l2q_tokenizer*)t);
    return lookup_sorted(t, text);
}

int tok_encode(l2q_tokenizer* t, const char* text, int bos, int eos, int* tokens) {
    if (text == NULL) return -1;
    ensure_sorted(t);
    size_t cap = (size_t)t->max_token_length * 2 + 3;
    char* buf = (char*)malloc(cap < 16 ? 16 : cap);
    int n = 0;
    if (bos) tokens[n++] = 1;
    if (text[0] != 0) tokens[n++] = lookup_sorted(t, " ");   /* dummy prefix */

    /* One token per UTF-8 code point (up to 4 bytes), byte fallback +3. */
    size_t len = 0;
    for (const char* c = text; *c; c++) {
        if ((*c & 0xC0) != 0x80) len = 0;
        buf[len++] = *c;
        buf[len] = 0;
        if ((c[1] & 0xC0) == 0x80 && len < 4) continue;
        int id = lookup_sorted(t, buf);
        if (id != -1) tokens[n++] = id;
        else for (size_t i = 0; i < len; i++) tokens[n++] = (unsigned char)buf[i] + 3;
        len = 0;
    }

    /* Merge the adjacent pair whose concatenation has the best score until
     * no pair is in the vocabulary (first best pair wins ties). */
    for (;;) {
        float best = -1e10f;
        int best_id = -1, at = -1;
        for (int i = 0; i + 1 < n; i++) {
            const char* a = t->pieces[tokens[i]];
            const char* b = t->pieces[tokens[i + 1]];
            size_t la = strlen(a), lb = strlen(b);
            if (la + lb + 1 > cap) continue;   /* longer than any vocab piece */
            memcpy(buf, a, la);
            memcpy(buf + la, b, lb + 1);
            int id = lookup_sorted(t, buf);
            if (id != -1 && t->scores[id] > best) { best = t->scores[id]; best_id = id; at = i; }
        }
        if (at < 0) break;
        tokens[at] = best_id;
        memmove(tokens + at + 1, tokens + at + 2, (size_t)(n - at - 2) * sizeof(int));
        n--;
    }
    if (eos) tokens[n++] = 2;
    free(buf);
    return n;
}

const char* tok_decode(const l2q_tokenizer* t, int prev, int token) {
    const char* p = t->pieces[token];
    if (prev == 1 && p[0] == ' ') p++;
    unsigned char byte;
    if (sscanf(p, "<0x%02hhX>", &byte) == 1) p = t->byte_text[byte];
    return p;
}

void tok_print_piece(const char* p) {
    if (p == NULL || p[0] == 0) return;
    if (p[1] == 0) {
        unsigned char b = (unsigned char)p[0];
        if (!(isprint(b) || isspace(b))) return;
    }
    printf("%s", p);
}

int tok_write(const char* path, char* const* pieces, const float* scores, int n) {
    FILE* f = fopen(path, "wb");
    if (!f) return -1;
    uint32_t maxlen = 0;
    for (int i = 0; i < n; i++) { uint32_t l = (uint32_t)strlen(pieces[i]); if (l > maxlen) maxlen = l; }
    int ok = fwrite(&maxlen, 4, 1, f) == 1;
    for (int i = 0; ok && i < n; i++) {
        int32_t l = (int32_t)strlen(pieces[i]);
        ok = fwrite(&scores[i], 4, 1, f) == 1 && fwrite(&l, 4, 1, f) == 1 &&
             (l == 0 || fwrite(pieces[i], (size_t)l, 1, f) == 1);
    }
    if (fclose(f) != 0) ok = 0;
    return ok ? 0 : -1;
}
