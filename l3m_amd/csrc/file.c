// A mapped .l3m file, validated at open so that a malformed file is an error and never a bad read
// later. The rules are the reference's (src/file.c:26-98, 100-139): every tensor whole, aligned and in
// bounds; every canonical tensor present with the right shape; q, k, v sharing a dtype.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include "host.h"

#define MAX_DIM (1u << 24)

static int fail(l3m_mapped *f, const char *path, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "l3m: %s: ", path);
    vfprintf(stderr, fmt, ap);
    fputc('\n', stderr);
    va_end(ap);
    l3m_map_close(f);
    return -1;
}

static const char *tensor_problem(const l3m_mapped *f, const l3m_tensor *t) {
    if (!memchr(t->name, 0, sizeof t->name)) return "unterminated name";
    if (t->dtype >= L3M_NDTYPES || t->ndim < 1 || t->ndim > 2) return "bad dtype or ndim";
    uint64_t rows = t->ndim == 2 ? t->shape[0] : 1, cols = t->shape[t->ndim - 1];
    if (!rows || !cols || rows > MAX_DIM || cols > MAX_DIM) return "bad shape";
    if ((t->dtype >= L3M_Q8_0 && cols % L3M_QBLOCK) || (t->dtype == L3M_BF16 && cols % 2)) return "rows are not whole blocks";
    if (t->nbytes != rows * l3m_file_row_bytes((int)t->dtype, (int)cols)) return "nbytes does not match the shape";
    if (t->offset % 64 || t->offset > f->size || t->nbytes > f->size - t->offset) return "misaligned or past the end of the file";
    return NULL;
}

// 1 present and well-formed, 0 absent and optional, -1 otherwise (message printed). cols 0: a vector.
static int expect(const l3m_mapped *f, const char *path, const char *name, int required, int f32, uint64_t rows, uint64_t cols) {
    const l3m_tensor *t = l3m_map_tensor(f, name);
    if (!t) {
        if (required) fprintf(stderr, "l3m: %s: tensor %s missing\n", path, name);
        return required ? -1 : 0;
    }
    if (t->ndim != (cols ? 2u : 1u) || t->shape[0] != rows || (cols && t->shape[1] != cols) || (f32 && t->dtype != L3M_F32)) {
        fprintf(stderr, cols ? "l3m: %s: tensor %s: expected %s[%llu, %llu]\n" : "l3m: %s: tensor %s: expected %s[%llu]\n",
                path, name, f32 ? "f32 " : "", (unsigned long long)rows, (unsigned long long)cols);
        return -1;
    }
    return 1;
}

static int check_model(const l3m_mapped *f, const char *path) {
    const l3m_header *h = f->h;
    uint32_t dim = h->dim, ffn = h->ffn_dim, vocab = h->vocab;
    if (!dim || !ffn || !vocab || !h->ctx || !h->n_layers || !h->n_heads || !h->n_kv_heads || dim > MAX_DIM || ffn > MAX_DIM ||
        vocab > MAX_DIM || h->ctx > MAX_DIM || h->n_layers > MAX_DIM || dim % h->n_heads || h->n_heads % h->n_kv_heads ||
        dim / h->n_heads % 8) {
        fprintf(stderr, "l3m: %s: bad config: dim %u, heads %u, kv_heads %u (head_dim a multiple of 8), ffn %u, layers %u, vocab %u, ctx %u\n",
                path, dim, h->n_heads, h->n_kv_heads, ffn, h->n_layers, vocab, h->ctx);
        return -1;
    }
    uint32_t kv = dim / h->n_heads * h->n_kv_heads;
    int ln = (h->flags & L3M_F_LAYERNORM) != 0, gelu = (h->flags & L3M_F_GELU) != 0, bad = 0;
    bad |= expect(f, path, "embed", 1, 0, vocab, dim) < 0;
    if (!(h->flags & L3M_F_TIED)) bad |= expect(f, path, "lm_head", 1, 0, vocab, dim) < 0;
    bad |= expect(f, path, "pos_embed", (h->flags & L3M_F_LEARNED_POS) != 0, 1, h->ctx, dim) < 0;
    bad |= expect(f, path, "norm", 1, 1, dim, 0) < 0;
    bad |= expect(f, path, "norm_b", ln, 1, dim, 0) < 0;
    if (bad) return -1;
    char nm[80];
    for (uint32_t l = 0; l < h->n_layers; l++) {
#define B(s) (snprintf(nm, sizeof nm, "blk.%u.%s", l, s), nm)
        bad |= expect(f, path, B("attn_norm"), 1, 1, dim, 0) < 0;
        bad |= expect(f, path, B("attn_norm_b"), ln, 1, dim, 0) < 0;
        bad |= expect(f, path, B("ffn_norm"), 1, 1, dim, 0) < 0;
        bad |= expect(f, path, B("ffn_norm_b"), ln, 1, dim, 0) < 0;
        bad |= expect(f, path, B("wq"), 1, 0, dim, dim) < 0;
        bad |= expect(f, path, B("wk"), 1, 0, kv, dim) < 0;
        bad |= expect(f, path, B("wv"), 1, 0, kv, dim) < 0;
        bad |= expect(f, path, B("wo"), 1, 0, dim, dim) < 0;
        bad |= expect(f, path, B("w_up"), 1, 0, ffn, dim) < 0;
        bad |= expect(f, path, B("w_gate"), !gelu, 0, ffn, dim) < 0;
        bad |= expect(f, path, B("w_down"), 1, 0, dim, ffn) < 0;
        bad |= expect(f, path, B("bo"), 0, 1, dim, 0) < 0;
        bad |= expect(f, path, B("b_up"), 0, 1, ffn, 0) < 0;
        bad |= expect(f, path, B("b_down"), 0, 1, dim, 0) < 0;
        int bq = expect(f, path, B("bq"), 0, 1, dim, 0), bk = expect(f, path, B("bk"), 0, 1, kv, 0), bv = expect(f, path, B("bv"), 0, 1, kv, 0);
#undef B
        if (bad || bq < 0 || bk < 0 || bv < 0) return -1;
        const l3m_tensor *q = l3m_map_blk(f, (int)l, "wq"), *k = l3m_map_blk(f, (int)l, "wk"), *v = l3m_map_blk(f, (int)l, "wv");
        if (bq != bk || bq != bv || k->dtype != q->dtype || v->dtype != q->dtype) {
            fprintf(stderr, "l3m: %s: blk.%u: wq, wk, wv must share a dtype, and bq, bk, bv come together\n", path, l);
            return -1;
        }
    }
    return 0;
}

int l3m_map_open(l3m_mapped *f, const char *path) {
    memset(f, 0, sizeof *f);
    int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(f, path, "%s", strerror(errno));
    struct stat st;
    if (fstat(fd, &st) || !S_ISREG(st.st_mode) || (size_t)st.st_size < sizeof(l3m_header)) {
        close(fd);
        return fail(f, path, "not an l3m v%d file", L3M_VERSION);
    }
    f->size = (size_t)st.st_size;
    f->map = mmap(NULL, f->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (f->map == MAP_FAILED) { f->map = NULL; return fail(f, path, "mmap: %s", strerror(errno)); }
    const l3m_header *h = f->h = (const l3m_header *)f->map;
    if (!l3m_header_ok(h)) return fail(f, path, "not an l3m v%d file", L3M_VERSION);
    if (h->toc_offset % 8 || h->toc_offset > f->size || h->n_tensors > (f->size - h->toc_offset) / sizeof(l3m_tensor) ||
        h->tokenizer_offset > f->size)
        return fail(f, path, "truncated file");
    f->toc = (const l3m_tensor *)((const char *)f->map + h->toc_offset);
    for (uint32_t i = 0; i < h->n_tensors; i++) {
        const char *why = tensor_problem(f, &f->toc[i]);
        if (why) return fail(f, path, "tensor %u (%.64s): %s", i, f->toc[i].name, why);
    }
    if (check_model(f, path)) { l3m_map_close(f); return -1; }
    if (l3m_vocab_init(&f->tok, (const char *)f->map + h->tokenizer_offset, f->size - h->tokenizer_offset))
        return fail(f, path, "bad tokenizer section");
    if (f->tok.n > (int)h->vocab) return fail(f, path, "tokenizer has %d tokens, vocab only %u", f->tok.n, h->vocab);
    if (h->chat_offset) {
        int32_t im_start;
        const char *sys = (const char *)f->map + h->chat_offset + sizeof im_start;
        if (h->chat_offset > f->size - sizeof im_start || !memchr(sys, 0, f->size - h->chat_offset - sizeof im_start))
            return fail(f, path, "bad chat section");
        memcpy(&im_start, (const char *)f->map + h->chat_offset, sizeof im_start);
        if (im_start < 0 || im_start >= f->tok.n || f->tok.eos < 0 || f->tok.eos >= f->tok.n) return fail(f, path, "bad chat section");
        f->im_start = im_start;
        f->system = sys;
    }
    return 0;
}

void l3m_map_close(l3m_mapped *f) {
    l3m_vocab_free(&f->tok);
    if (f->map) munmap(f->map, f->size);
    memset(f, 0, sizeof *f);
}

const l3m_tensor *l3m_map_tensor(const l3m_mapped *f, const char *name) {
    for (uint32_t i = 0; i < f->h->n_tensors; i++)
        if (!strcmp(f->toc[i].name, name)) return &f->toc[i];
    return NULL;
}

const l3m_tensor *l3m_map_blk(const l3m_mapped *f, int layer, const char *name) {
    char b[80];
    snprintf(b, sizeof b, "blk.%d.%s", layer, name);
    return l3m_map_tensor(f, b);
}

const void *l3m_map_data(const l3m_mapped *f, const l3m_tensor *t) { return (const char *)f->map + t->offset; }
