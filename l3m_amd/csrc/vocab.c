// The tokenizer section of a .l3m file (src/model.h:27-28): a 16-byte header {u32 n_tokens, i32 bos, i32 eos,
// u32 max_len}, then per token {f32 score, u16 len, len bytes}. The header is accepted under the reference's
// conditions (src/tokenizer.c:17-45): the count must fit the section at 6 bytes per token at least, and bos
// must be an id or negative (none).
//
// Decoding is the byte table. Encoding gives the reference's ids (tokenizer.c:103-170): the text is cut into
// pre-tokenizer pieces (SentencePiece: a word with its leading spaces, or the whole text; byte-level BPE: the
// GPT-2 pattern of contractions, letter, digit and punctuation runs with one optional leading space, and
// whitespace runs whose last space goes to the next word, digits one by one when the file says so). Each
// piece starts as its characters' pieces (UTF-8 characters for SentencePiece, bytes otherwise; a character
// without a piece falls back to its bytes, a byte without one is dropped), and then the adjacent pair whose
// concatenation is the highest-scoring piece (at most max_len bytes) is merged, the leftmost on equal scores,
// until no pair is a piece. Pieces are found through a hash of their bytes; a string held by several ids maps
// to the highest score, the lowest id on equal scores.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "host.h"

typedef struct {
    const uint8_t *at, *end;
} cursor;

static int take(cursor *c, void *dst, size_t n) {
    if ((size_t)(c->end - c->at) < n) return -1;
    if (dst) memcpy(dst, c->at, n);
    c->at += n;
    return 0;
}

static uint32_t fnv1a(const uint8_t *s, int n) {
    uint32_t h = 2166136261u;
    for (int i = 0; i < n; i++) h = (h ^ s[i]) * 16777619u;
    return h;
}

// The id whose piece is exactly s[0, n), or -1.
static int find(const l3m_vocab_table *t, const uint8_t *s, int n) {
    if (!t->slot || n < 1) return -1;
    for (uint32_t i = fnv1a(s, n) & t->mask;; i = (i + 1) & t->mask) {
        const int id = t->slot[i];
        if (id < 0) return -1;
        if (t->len[id] == n && !memcmp(t->bytes[id], s, (size_t)n)) return id;
    }
}

static int index_pieces(l3m_vocab_table *t) {
    unsigned cap = 16;
    while (cap < 2u * (unsigned)t->n + 16) cap <<= 1;
    t->slot = malloc(cap * sizeof *t->slot);
    if (!t->slot) return -1;
    t->mask = cap - 1;
    for (unsigned i = 0; i < cap; i++) t->slot[i] = -1;
    for (int id = 0; id < t->n; id++) {
        if (!t->len[id]) continue;
        for (uint32_t i = fnv1a(t->bytes[id], t->len[id]) & t->mask;; i = (i + 1) & t->mask) {
            const int o = t->slot[i];
            if (o < 0) { t->slot[i] = id; break; }
            if (t->len[o] == t->len[id] && !memcmp(t->bytes[o], t->bytes[id], t->len[id])) {
                if (t->score[id] > t->score[o]) t->slot[i] = id;   // the same bytes: the better score wins
                break;
            }
        }
    }
    return 0;
}

int l3m_vocab_init(l3m_vocab_table *t, const void *section, size_t size, unsigned flags) {
    memset(t, 0, sizeof *t);
    cursor c = {(const uint8_t *)section, (const uint8_t *)section + size};
    l3m_tok_header hdr;
    if (take(&c, &hdr, sizeof hdr)) return -1;
    const size_t room = (size_t)(c.end - c.at);
    if ((size_t)hdr.n_tokens > room / 6 || (int64_t)hdr.bos >= (int64_t)hdr.n_tokens) return -1;
    const size_t n = hdr.n_tokens;
    const uint8_t **bytes = calloc(n + 1, sizeof *bytes);
    uint16_t *len = calloc(n + 1, sizeof *len);
    float *score = calloc(n + 1, sizeof *score);
    t->bytes = bytes;
    t->len = len;
    t->score = score;
    if (!bytes || !len || !score) { l3m_vocab_free(t); return -1; }
    for (size_t i = 0; i < n; i++) {
        if (take(&c, &score[i], 4) || take(&c, &len[i], 2)) { l3m_vocab_free(t); return -1; }
        bytes[i] = c.at;
        if (take(&c, NULL, len[i])) { l3m_vocab_free(t); return -1; }
    }
    t->n = (int)n;
    t->bos = hdr.bos < 0 ? -1 : hdr.bos;
    t->eos = hdr.eos;
    t->max_len = (int)hdr.max_len;
    t->sp_prefix = (flags & L3M_F_SP_PREFIX) != 0;
    t->digits = (flags & L3M_F_DIGITS) != 0;
    // SentencePiece words split at spaces unless some piece holds a space after a non-space
    t->sp_words = t->sp_prefix;
    for (size_t i = 0; i < n && t->sp_words; i++)
        for (int j = 1; j < len[i]; j++)
            if (bytes[i][j] == ' ' && bytes[i][j - 1] != ' ') t->sp_words = 0;
    if (index_pieces(t)) { l3m_vocab_free(t); return -1; }
    return 0;
}

void l3m_vocab_free(l3m_vocab_table *t) {
    free((void *)t->bytes);
    free((void *)t->len);
    free(t->score);
    free(t->slot);
    memset(t, 0, sizeof *t);
}

// ------------------------------------------------------------------------------- pre-tokenizer

enum { C_SPACE, C_LETTER, C_DIGIT, C_PUNCT };

static int kind(uint8_t c) {                          // bytes >= 0x80 count as letters
    if (c == ' ' || (c >= '\t' && c <= '\r')) return C_SPACE;
    if (c >= '0' && c <= '9') return C_DIGIT;
    if (c >= 0x80 || ((c | 0x20) >= 'a' && (c | 0x20) <= 'z')) return C_LETTER;
    return C_PUNCT;
}

static int is_digit(const l3m_vocab_table *t, uint8_t c) { return t->digits && kind(c) == C_DIGIT; }

// Where the piece that starts at p ends.
static const uint8_t *cut(const l3m_vocab_table *t, const uint8_t *p) {
    if (t->sp_prefix) {                               // SentencePiece: leading spaces, then the word (or all)
        while (*p == ' ') p++;
        while (*p && (!t->sp_words || *p != ' ')) p++;
        return p;
    }
    if (*p == '\'') {                                 // 's 't 're 've 'm 'll 'd
        static const char *const tail[] = {"s", "t", "re", "ve", "m", "ll", "d"};
        for (size_t i = 0; i < sizeof tail / sizeof *tail; i++) {
            const size_t k = strlen(tail[i]);
            if (!strncmp((const char *)p + 1, tail[i], k)) return p + 1 + k;
        }
    }
    if (is_digit(t, *p)) return p + 1;                // digits one by one
    // one leading space joins a following non-space run (not a digit when digits go one by one)
    const uint8_t *q = p;
    if (*p == ' ' && p[1] && kind(p[1]) != C_SPACE && !is_digit(t, p[1])) q++;
    const int k = kind(*q);
    if (k != C_SPACE) {
        while (*q && kind(*q) == k) q++;
        return q;
    }
    while (*q && kind(*q) == C_SPACE) q++;
    // a whitespace run before a word leaves its last space to the word
    const int at_end = !*q || is_digit(t, *q);
    return q - p > 1 && !at_end ? q - 1 : q;
}

static int utf8_width(const uint8_t *p) {
    const int w = p[0] < 0x80 ? 1 : p[0] < 0xE0 ? 2 : p[0] < 0xF0 ? 3 : 4;
    for (int i = 1; i < w; i++)
        if ((p[i] & 0xC0) != 0x80) return 1;
    return w;
}

// ------------------------------------------------------------------------------------- merges

// A candidate merge of the symbols at positions left and right (adjacent when pushed), which held ids a
// and b then, into id (score its score). Stale candidates are recognized when popped.
typedef struct {
    float score;
    int   left, right, a, b, id;
} cand;

// Pops before: the higher score, then the leftmost.
static int first(const cand *x, const cand *y) { return x->score > y->score || (x->score == y->score && x->left < y->left); }

typedef struct {
    cand *h;
    int   n;
} heap;

static void heap_push(heap *q, cand c) {
    int i = q->n++;
    while (i > 0 && first(&c, &q->h[(i - 1) >> 1])) {
        q->h[i] = q->h[(i - 1) >> 1];
        i = (i - 1) >> 1;
    }
    q->h[i] = c;
}

static cand heap_pop(heap *q) {
    const cand top = q->h[0], last = q->h[--q->n];
    int i = 0;
    for (;;) {
        int c = 2 * i + 1;
        if (c >= q->n) break;
        if (c + 1 < q->n && first(&q->h[c + 1], &q->h[c])) c++;
        if (!first(&q->h[c], &last)) break;
        q->h[i] = q->h[c];
        i = c;
    }
    q->h[i] = last;
    return top;
}

// The candidate for the pair (left, right) of sym, if their concatenation is a piece of at most max_len bytes.
static void offer(const l3m_vocab_table *t, heap *q, const int32_t *sym, int left, int right) {
    uint8_t buf[512];
    const int a = sym[left], b = sym[right], n = t->len[a] + t->len[b];
    if (n > t->max_len || n > (int)sizeof buf) return;
    memcpy(buf, t->bytes[a], t->len[a]);
    memcpy(buf + t->len[a], t->bytes[b], t->len[b]);
    const int id = find(t, buf, n);
    if (id >= 0) heap_push(q, (cand){t->score[id], left, right, a, b, id});
}

// Merges the symbols sym[0, m) in place; returns how many remain.
static int merge(const l3m_vocab_table *t, int32_t *sym, int m) {
    if (m < 2) return m;
    int *nx = malloc((size_t)m * sizeof *nx), *pv = malloc((size_t)m * sizeof *pv);
    heap q = {malloc(3 * (size_t)m * sizeof(cand)), 0};   // m - 1 pairs, then at most two per merge
    if (!nx || !pv || !q.h) { free(nx); free(pv); free(q.h); return m; }
    for (int i = 0; i < m; i++) { nx[i] = i + 1; pv[i] = i - 1; }
    for (int i = 0; i + 1 < m; i++) offer(t, &q, sym, i, i + 1);
    while (q.n) {
        const cand c = heap_pop(&q);
        if (nx[c.left] != c.right || sym[c.left] != c.a || sym[c.right] != c.b) continue;
        sym[c.left] = c.id;
        sym[c.right] = -1;
        nx[c.left] = nx[c.right];
        if (nx[c.left] < m) pv[nx[c.left]] = c.left;
        if (pv[c.left] >= 0) offer(t, &q, sym, pv[c.left], c.left);
        if (nx[c.left] < m) offer(t, &q, sym, c.left, nx[c.left]);
    }
    int k = 0;
    for (int i = 0; i < m; i++)
        if (sym[i] >= 0) sym[k++] = sym[i];
    free(nx); free(pv); free(q.h);
    return k;
}

int l3m_vocab_encode(const l3m_vocab_table *t, const char *text, int add_bos, int32_t *out, int max) {
    int n = 0;
#define EMIT(id) do { if (n >= max) return -1; out[n++] = (id); } while (0)
    if (add_bos && t->bos >= 0) EMIT(t->bos);
    // the SentencePiece prefix space is emitted before the first piece's symbols and merges with them
    int lo = n;
    const int space = find(t, (const uint8_t *)" ", 1);
    if (t->sp_prefix && *text && space >= 0) EMIT(space);
    for (const uint8_t *p = (const uint8_t *)text; *p; lo = n) {
        const uint8_t *end = cut(t, p);
        while (p < end) {
            const int w = t->sp_prefix ? utf8_width(p) : 1, id = find(t, p, w);
            if (id >= 0) EMIT(id);
            else
                for (int i = 0; i < w; i++) {
                    const int b = find(t, p + i, 1);
                    if (b >= 0) EMIT(b);
                }
            p += w;
        }
        n = lo + merge(t, out + lo, n - lo);
    }
#undef EMIT
    return n;
}

const uint8_t *l3m_vocab_decode(const l3m_vocab_table *t, int32_t tok, int *len) {
    static const uint8_t empty[1] = {0};
    if (tok < 0 || tok >= t->n) {
        *len = 0;
        return empty;
    }
    *len = t->len[tok];
    return t->bytes[tok];
}
