// The tokenizer section of a .l3m file as a byte table (format: src/model.h:27-28; header checks:
// src/tokenizer.c:17-45). Decoding is exact. Encoding maps each input byte to its single-byte piece and
// does not apply merges: text tokenization is not on the decode hot path, and for files whose pieces
// never merge (the synthetic models, whose pieces are the 256 bytes and empty strings) it gives the
// reference's ids.
#include <stdlib.h>
#include <string.h>
#include "host.h"

int l3m_vocab_init(l3m_vocab_table *t, const void *section, size_t size) {
    l3m_tok_header h;
    memset(t, 0, sizeof *t);
    if (size < sizeof h) return -1;
    memcpy(&h, section, sizeof h);
    if (h.n_tokens > (size - sizeof h) / 6 || h.bos >= (int64_t)h.n_tokens) return -1;
    t->n = (int)h.n_tokens; t->bos = h.bos < 0 ? -1 : h.bos; t->eos = h.eos; t->max_len = (int)h.max_len;
    t->bytes = malloc(((size_t)t->n + 1) * sizeof *t->bytes);
    uint16_t *len = malloc(((size_t)t->n + 1) * sizeof *len);
    t->len = len;
    if (!t->bytes || !len) { l3m_vocab_free(t); return -1; }
    const uint8_t *p = (const uint8_t *)section + sizeof h, *end = (const uint8_t *)section + size;
    for (int i = 0; i < t->n; i++) {
        if (end - p < 6) { l3m_vocab_free(t); return -1; }
        memcpy(&len[i], p + 4, 2);
        if (end - p - 6 < len[i]) { l3m_vocab_free(t); return -1; }
        t->bytes[i] = p + 6;
        p += 6 + len[i];
    }
    return 0;
}

void l3m_vocab_free(l3m_vocab_table *t) {
    free((void *)t->bytes);
    free((void *)t->len);
    memset(t, 0, sizeof *t);
}

static int single_byte_id(const l3m_vocab_table *t, uint8_t c) {
    for (int i = 0; i < t->n; i++) if (t->len[i] == 1 && t->bytes[i][0] == c) return i;
    return -1;
}

int l3m_vocab_encode(const l3m_vocab_table *t, const char *text, int add_bos, int32_t *out, int max) {
    int n = 0;
    if (add_bos && t->bos >= 0) { if (n == max) return -1; out[n++] = t->bos; }
    for (const uint8_t *p = (const uint8_t *)text; *p; p++) {
        int id = single_byte_id(t, *p);
        if (id < 0) continue;
        if (n == max) return -1;
        out[n++] = id;
    }
    return n;
}

const uint8_t *l3m_vocab_decode(const l3m_vocab_table *t, int32_t tok, int *len) {
    if (tok < 0 || tok >= t->n) { *len = 0; return (const uint8_t *)""; }
    *len = t->len[tok];
    return t->bytes[tok];
}
