// The tokenizer section of a .l3m file as a table of byte strings. Section layout (src/model.h:27-28):
// a 16-byte header {u32 n_tokens, i32 bos, i32 eos, u32 max_len}, then per token {f32 score, u16 len,
// len bytes}. The header is accepted under the reference's conditions (src/tokenizer.c:17-45): the
// count must fit the section at 6 bytes per token at least, and bos must be an id or negative (none).
//
// Decoding is exact. Encoding maps each input byte to its single-byte piece and applies no merges: text
// tokenization is not on the decode hot path, and for files whose pieces never merge (no piece of more
// than one byte, as in the synthetic models: the 256 bytes and empty pieces) it gives the reference's
// ids. A vocabulary with merge pieces is refused (-1, once with a message) rather than tokenized into
// ids the reference would not produce; such callers pass token ids.
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

int l3m_vocab_init(l3m_vocab_table *t, const void *section, size_t size) {
    memset(t, 0, sizeof *t);
    cursor c = {(const uint8_t *)section, (const uint8_t *)section + size};
    l3m_tok_header hdr;
    if (take(&c, &hdr, sizeof hdr)) return -1;
    const size_t room = (size_t)(c.end - c.at);
    if ((size_t)hdr.n_tokens > room / 6 || (int64_t)hdr.bos >= (int64_t)hdr.n_tokens) return -1;
    const size_t n = hdr.n_tokens;
    const uint8_t **bytes = calloc(n + 1, sizeof *bytes);
    uint16_t *len = calloc(n + 1, sizeof *len);
    t->bytes = bytes;
    t->len = len;
    if (!bytes || !len) { l3m_vocab_free(t); return -1; }
    for (size_t i = 0; i < n; i++) {
        if (take(&c, NULL, 4) || take(&c, &len[i], 2)) { l3m_vocab_free(t); return -1; }   // score unused
        bytes[i] = c.at;
        if (take(&c, NULL, len[i])) { l3m_vocab_free(t); return -1; }
    }
    t->n = (int)n;
    t->merges = 0;
    for (size_t i = 0; i < n; i++) t->merges |= len[i] > 1;
    t->bos = hdr.bos < 0 ? -1 : hdr.bos;
    t->eos = hdr.eos;
    t->max_len = (int)hdr.max_len;
    return 0;
}

void l3m_vocab_free(l3m_vocab_table *t) {
    free((void *)t->bytes);
    free((void *)t->len);
    memset(t, 0, sizeof *t);
}

static int piece_of_byte(const l3m_vocab_table *t, uint8_t b) {
    for (int id = 0; id < t->n; id++)
        if (t->len[id] == 1 && t->bytes[id][0] == b) return id;
    return -1;
}

int l3m_vocab_encode(const l3m_vocab_table *t, const char *text, int add_bos, int32_t *out, int max) {
    if (t->merges) {
        static int told;
        if (!told++) fprintf(stderr, "l3m: this vocabulary merges bytes into longer pieces, which this backend's byte-level "
                                     "encoder does not apply; pass token ids instead\n");
        return -1;
    }
    int n = 0;
    if (add_bos && t->bos >= 0) {
        if (max < 1) return -1;
        out[n++] = t->bos;
    }
    for (const char *p = text; *p; p++) {
        const int id = piece_of_byte(t, (uint8_t)*p);
        if (id < 0) continue;               // a byte with no piece of its own is dropped
        if (n >= max) return -1;
        out[n++] = id;
    }
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
