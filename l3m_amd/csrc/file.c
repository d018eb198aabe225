// The .l3m reader. The file is mapped once and checked completely at open, so a malformed file is a
// load error and never an out-of-range read later. What is checked is what fpedd/l3m's reader checks
// (src/file.c:26-139), because a file either loads in both or in neither:
//   - the header: magic and version, a table of contents and tokenizer inside the file;
//   - every table entry: a terminated name, dtype and rank in range, whole 32-input blocks (bf16: an
//     even width), nbytes equal to rows x row bytes, a 64-byte aligned payload inside the file;
//   - the model: a sane geometry (head_dim a multiple of 8) and every tensor the architecture flags
//     call for, with its shape (norms and biases f32); wq, wk, wv of one dtype; bq, bk, bv together;
//   - the tokenizer and the optional chat section.
// The expected tensors are listed in one table below instead of being spelled out check by check.
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

#define DIM_LIMIT ((uint64_t)1 << 24)

typedef struct {
    char text[256];
} why;

static int because(why *w, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(w->text, sizeof w->text, fmt, ap);
    va_end(ap);
    return -1;
}

// One table-of-contents entry on its own.
static int entry_ok(const l3m_mapped *f, uint32_t i, why *w) {
    const l3m_tensor *t = &f->toc[i];
    if (strnlen(t->name, sizeof t->name) == sizeof t->name) return because(w, "table entry %u: name has no terminator", i);
    if (t->dtype >= L3M_NDTYPES) return because(w, "%s: unknown dtype %u", t->name, t->dtype);
    if (t->ndim != 1 && t->ndim != 2) return because(w, "%s: rank %u (1 or 2 expected)", t->name, t->ndim);
    const uint64_t width = t->shape[t->ndim - 1], height = t->ndim == 2 ? t->shape[0] : 1;
    if (width == 0 || height == 0 || width > DIM_LIMIT || height > DIM_LIMIT) return because(w, "%s: shape out of range", t->name);
    const int blocked = t->dtype == L3M_Q8_0 || t->dtype == L3M_Q4_0 || t->dtype == L3M_MXFP4;
    if ((blocked && width % L3M_QBLOCK != 0) || (t->dtype == L3M_BF16 && width % 2 != 0))
        return because(w, "%s: width %llu is not whole %s blocks", t->name, (unsigned long long)width, l3m_dtype_name((int)t->dtype));
    if (t->nbytes != height * l3m_file_row_bytes((int)t->dtype, (int)width))
        return because(w, "%s: %llu bytes do not match its shape", t->name, (unsigned long long)t->nbytes);
    if (t->offset % 64 != 0 || t->offset > f->size || f->size - t->offset < t->nbytes)
        return because(w, "%s: payload misaligned or outside the file", t->name);
    return 0;
}

// Symbolic sizes of the expected tensors.
enum { SZ_NONE, SZ_DIM, SZ_KV, SZ_FFN, SZ_VOCAB, SZ_CTX };
enum { NEED_ALWAYS, NEED_NEVER, NEED_IF_LN, NEED_UNLESS_GELU, NEED_UNLESS_TIED, NEED_IF_LEARNED_POS };
typedef struct {
    const char *name;       // per layer: the part after "blk.<l>."
    unsigned char need;     // when the tensor must be present (otherwise it is optional when present)
    unsigned char f32;      // must be f32 (norms, biases, position table)
    unsigned char rows, cols;   // cols SZ_NONE: a vector of `rows`
} expected;

static const expected MODEL_TENSORS[] = {
    {"embed", NEED_ALWAYS, 0, SZ_VOCAB, SZ_DIM},         {"lm_head", NEED_UNLESS_TIED, 0, SZ_VOCAB, SZ_DIM},
    {"pos_embed", NEED_IF_LEARNED_POS, 1, SZ_CTX, SZ_DIM}, {"norm", NEED_ALWAYS, 1, SZ_DIM, SZ_NONE},
    {"norm_b", NEED_IF_LN, 1, SZ_DIM, SZ_NONE},
};
static const expected LAYER_TENSORS[] = {
    {"attn_norm", NEED_ALWAYS, 1, SZ_DIM, SZ_NONE}, {"attn_norm_b", NEED_IF_LN, 1, SZ_DIM, SZ_NONE},
    {"ffn_norm", NEED_ALWAYS, 1, SZ_DIM, SZ_NONE},  {"ffn_norm_b", NEED_IF_LN, 1, SZ_DIM, SZ_NONE},
    {"wq", NEED_ALWAYS, 0, SZ_DIM, SZ_DIM},         {"wk", NEED_ALWAYS, 0, SZ_KV, SZ_DIM},
    {"wv", NEED_ALWAYS, 0, SZ_KV, SZ_DIM},          {"wo", NEED_ALWAYS, 0, SZ_DIM, SZ_DIM},
    {"w_up", NEED_ALWAYS, 0, SZ_FFN, SZ_DIM},       {"w_gate", NEED_UNLESS_GELU, 0, SZ_FFN, SZ_DIM},
    {"w_down", NEED_ALWAYS, 0, SZ_DIM, SZ_FFN},     {"bo", NEED_NEVER, 1, SZ_DIM, SZ_NONE},
    {"b_up", NEED_NEVER, 1, SZ_FFN, SZ_NONE},       {"b_down", NEED_NEVER, 1, SZ_DIM, SZ_NONE},
    {"bq", NEED_NEVER, 1, SZ_DIM, SZ_NONE},         {"bk", NEED_NEVER, 1, SZ_KV, SZ_NONE},
    {"bv", NEED_NEVER, 1, SZ_KV, SZ_NONE},
};

static uint64_t size_of(const l3m_header *h, int which) {
    switch (which) {
    case SZ_DIM: return h->dim;
    case SZ_KV: return (uint64_t)h->dim / h->n_heads * h->n_kv_heads;
    case SZ_FFN: return h->ffn_dim;
    case SZ_VOCAB: return h->vocab;
    case SZ_CTX: return h->ctx;
    }
    return 0;
}

static int required(const l3m_header *h, int need) {
    switch (need) {
    case NEED_ALWAYS: return 1;
    case NEED_IF_LN: return (h->flags & L3M_F_LAYERNORM) != 0;
    case NEED_UNLESS_GELU: return (h->flags & L3M_F_GELU) == 0;
    case NEED_UNLESS_TIED: return (h->flags & L3M_F_TIED) == 0;
    case NEED_IF_LEARNED_POS: return (h->flags & L3M_F_LEARNED_POS) != 0;
    }
    return 0;
}

// 1 present with the expected shape, 0 absent and optional, -1 otherwise.
static int tensor_ok(const l3m_mapped *f, const char *name, const expected *e, why *w) {
    const l3m_header *h = f->h;
    const l3m_tensor *t = l3m_map_tensor(f, name);
    if (!t) return required(h, e->need) ? because(w, "tensor %s missing", name) : 0;
    const uint64_t rows = size_of(h, e->rows), cols = size_of(h, e->cols);
    const int shape_ok = e->cols == SZ_NONE ? t->ndim == 1 && t->shape[0] == rows : t->ndim == 2 && t->shape[0] == rows && t->shape[1] == cols;
    if (!shape_ok || (e->f32 && t->dtype != L3M_F32)) {
        if (e->cols == SZ_NONE) return because(w, "tensor %s: expected %s[%llu]", name, e->f32 ? "f32 " : "", (unsigned long long)rows);
        return because(w, "tensor %s: expected %s[%llu, %llu]", name, e->f32 ? "f32 " : "", (unsigned long long)rows,
                       (unsigned long long)cols);
    }
    return 1;
}

static int model_ok(const l3m_mapped *f, why *w) {
    const l3m_header *h = f->h;
    const uint64_t dims[] = {h->dim, h->ffn_dim, h->vocab, h->ctx, h->n_layers, h->n_heads, h->n_kv_heads};
    int geometry = 1;
    for (size_t i = 0; i < sizeof dims / sizeof dims[0]; i++) geometry &= dims[i] > 0 && dims[i] <= DIM_LIMIT;
    if (geometry) geometry = h->dim % h->n_heads == 0 && h->n_heads % h->n_kv_heads == 0 && (h->dim / h->n_heads) % 8 == 0;
    if (!geometry)
        return because(w, "bad config: dim %u, heads %u, kv_heads %u (head_dim a multiple of 8), ffn %u, layers %u, vocab %u, ctx %u",
                       h->dim, h->n_heads, h->n_kv_heads, h->ffn_dim, h->n_layers, h->vocab, h->ctx);
    for (size_t i = 0; i < sizeof MODEL_TENSORS / sizeof MODEL_TENSORS[0]; i++)
        if (tensor_ok(f, MODEL_TENSORS[i].name, &MODEL_TENSORS[i], w) < 0) return -1;
    char name[96];
    for (uint32_t layer = 0; layer < h->n_layers; layer++) {
        int present[sizeof LAYER_TENSORS / sizeof LAYER_TENSORS[0]];
        for (size_t i = 0; i < sizeof LAYER_TENSORS / sizeof LAYER_TENSORS[0]; i++) {
            snprintf(name, sizeof name, "blk.%u.%s", layer, LAYER_TENSORS[i].name);
            if ((present[i] = tensor_ok(f, name, &LAYER_TENSORS[i], w)) < 0) return -1;
        }
        const int nb = sizeof LAYER_TENSORS / sizeof LAYER_TENSORS[0];   // bq, bk, bv are the last three
        const uint32_t dq = l3m_map_blk(f, (int)layer, "wq")->dtype;
        if (present[nb - 3] != present[nb - 2] || present[nb - 3] != present[nb - 1] || l3m_map_blk(f, (int)layer, "wk")->dtype != dq ||
            l3m_map_blk(f, (int)layer, "wv")->dtype != dq)
            return because(w, "blk.%u: wq, wk, wv must share a dtype, and bq, bk, bv come together", layer);
    }
    return 0;
}

static int open_checked(l3m_mapped *f, const char *path, why *w) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return because(w, "%s", strerror(errno));
    struct stat st;
    const int regular = fstat(fd, &st) == 0 && S_ISREG(st.st_mode);
    if (!regular || (uint64_t)st.st_size < sizeof(l3m_header)) {
        close(fd);
        return because(w, "not an l3m v%d file", L3M_VERSION);
    }
    f->size = (size_t)st.st_size;
    void *p = mmap(NULL, f->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) return because(w, "mmap: %s", strerror(errno));
    f->map = p;
    f->h = (const l3m_header *)p;
    const l3m_header *h = f->h;
    if (memcmp(h->magic, "l3m", 3) != 0 || h->version != L3M_VERSION) return because(w, "not an l3m v%d file", L3M_VERSION);
    const int toc_ok = h->toc_offset % 8 == 0 && h->toc_offset <= f->size &&
                       h->n_tensors <= (f->size - h->toc_offset) / sizeof(l3m_tensor) && h->tokenizer_offset <= f->size;
    if (!toc_ok) return because(w, "truncated file");
    f->toc = (const l3m_tensor *)((const uint8_t *)p + h->toc_offset);
    for (uint32_t i = 0; i < h->n_tensors; i++)
        if (entry_ok(f, i, w)) return -1;
    if (model_ok(f, w)) return -1;
    if (l3m_vocab_init(&f->tok, (const uint8_t *)p + h->tokenizer_offset, f->size - h->tokenizer_offset, h->flags))
        return because(w, "bad tokenizer section");
    if (f->tok.n > (int)h->vocab) return because(w, "tokenizer has %d tokens, vocab only %u", f->tok.n, h->vocab);
    if (h->chat_offset) {                  // [i32 im_start][system prompt, NUL-terminated]
        int32_t im_start;
        if (h->chat_offset > f->size - sizeof im_start) return because(w, "bad chat section");
        const char *sys = (const char *)p + h->chat_offset + sizeof im_start;
        if (!memchr(sys, 0, f->size - h->chat_offset - sizeof im_start)) return because(w, "bad chat section");
        memcpy(&im_start, (const uint8_t *)p + h->chat_offset, sizeof im_start);
        if (im_start < 0 || im_start >= f->tok.n || f->tok.eos < 0 || f->tok.eos >= f->tok.n) return because(w, "bad chat section");
        f->im_start = im_start;
        f->system = sys;
    }
    return 0;
}

int l3m_map_open(l3m_mapped *f, const char *path) {
    memset(f, 0, sizeof *f);
    why w = {{0}};
    if (open_checked(f, path, &w) == 0) return 0;
    fprintf(stderr, "l3m: %s: %s\n", path, w.text);
    l3m_map_close(f);
    return -1;
}

void l3m_map_close(l3m_mapped *f) {
    l3m_vocab_free(&f->tok);
    if (f->map) munmap(f->map, f->size);
    memset(f, 0, sizeof *f);
}

const l3m_tensor *l3m_map_tensor(const l3m_mapped *f, const char *name) {
    const l3m_tensor *t = f->toc, *end = f->toc + f->h->n_tensors;
    for (; t < end; t++)
        if (strcmp(t->name, name) == 0) return t;
    return NULL;
}

const l3m_tensor *l3m_map_blk(const l3m_mapped *f, int layer, const char *name) {
    char full[96];
    snprintf(full, sizeof full, "blk.%d.%s", layer, name);
    return l3m_map_tensor(f, full);
}

const void *l3m_map_data(const l3m_mapped *f, const l3m_tensor *t) { return (const uint8_t *)f->map + t->offset; }
