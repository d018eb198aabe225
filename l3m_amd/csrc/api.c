// The l3m model API (src/l3m.h) on one MI355X: load a .l3m file into device memory in the lane-tile
// layout, then run the reference's generate loop (engine.c:322-362, 549-561) with every forward pass on
// the GPU: runs of consecutive positions, each one launch of the persistent decode kernel (one captured
// graph per position where the persistent grid is not available). The host only feeds prompt ids, reads
// back the chosen ids per run, applies the stop rules and calls on_token.
#include <math.h>
#include <stdio.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include "dev.h"
#include "host.h"

#define MiB (1024.0 * 1024.0)
#define DEFAULT_CTX 512        // engine.c:22
#define NSLOTS 128             // logits slots = the most steps of one run (the last NSLOTS positions' logits stay readable)
#define HEAD_WGS 256           // workgroups of the head kernel
#define MAX_PARTS 64           // partial residual vectors a step kernel adds (head groups, FFN chunks)
#define BODY_CUS 32            // the CUs of one MI355X XCD (256 in 8), where the persistent kernel keeps the body
#define EVICT_BYTES (512u << 20)   // --cold: read before each forward pass, twice the 256 MiB Infinity Cache
#define SPIN_LIMIT 100000000ull    // a wait of the persistent kernel gives up after 1 s (100 MHz ticks)
#define LIVE_STEPS 8               // positions per run of steps when each token is handed over as it comes

// What the host reads back after a run of steps: the persistent launch's abort word, and the tokens the run
// produced (in order from its first position with a token).
typedef struct {
    unsigned           abort;
    unsigned           pad;
    unsigned long long waited;   // 100 MHz ticks attention group 0 waited for its inputs (persistent launches)
    int32_t            tok[NSLOTS];
} l3m_chunk_out;

struct l3m_model {
    l3m_mapped   f;
    int          reference, dtype;
    int          mx_wide;      // an mxfp4 body whose blocks all widen exactly: its step matrices are q8_0
    l3m_dmodel   dm;
    l3m_dlayer  *layers;
    void       **allocs;
    int          n_allocs, cap_allocs;
    l3m_graphs  *graphs;
    l3m_dlayer  *layers_dev;   // the layer descriptors in device memory (persistent kernel)
    l3m_dmodel  *dm_dev;       // dm in device memory
    // The call area, one device allocation and its pinned host image (call_host), in this order: the first
    // decoded position, the sampler state, the token ids [ctx + 1], then per run of steps in flight (slot)
    // its launch parameters and its sync words (zero in the image). A generate call's inputs and its first
    // run's parameters and zeroed sync words are one contiguous copy; each later run's, another.
    uint8_t     *call_dev, *call_host;
    size_t       call_samp, call_tok, call_slot[2];   // byte offsets in the call area
    l3m_run     *run_dev[2];   // the persistent kernel's launch parameters, one per run of steps in flight
    l3m_run     *run_host[2];  // their images
    unsigned    *sync[2];      // L3M_SYNC_WORDS flag, key and output words of the persistent kernel, per run in flight
    l3m_chunk_out *out_host;   // [2] pinned: what each run of steps in flight hands back
    void        *ev[2];        // the end of each run of steps in flight (its copies back included)
    int32_t     *stage_tok;    // the call's prompt ids in the image
    l3m_dsample *stage_smp;    // the call's sampler state in the image
    int         *stage_pos;    // the call's first decoded position in the image
    int          persist;      // decode with the persistent kernel (else one graph per step)
    int          grid, head_tpw, n_head, body_xcc;
    unsigned     lds_decode;
    double       work[3];      // persistent launches so far: steps, steps with the head, K/V rows read
    int          chunk_rows;   // FFN rows per chunk (the last chunk takes the rest)
    unsigned long long spin_limit;   // the persistent kernel's longest wait, 100 MHz ticks (1 s)
    float       *logits;       // [vocab], host copy of the last fed position's logits
    int          logits_pos;   // position whose logits l3m_logits returns, -1 before any generate
    float        temp;         // the running generate call's temperature (0: greedy)
    l3m_pflayer *pf;           // batched prompt prefill: per-layer full matrices, NULL when unavailable
    l3m_pfbuf    pfb;
    l3m_pfgraphs *pfg;         // the prefill's captured graphs (NULL: loose launches, L3M_PREFILL_GRAPH=0)
    int          prefill_min;  // prompts of at least this many tokens are prefilled (L3M_PREFILL_MIN)
    int          prefilled;    // positions the last generate call prefilled
    int          logits_fresh;
    double       tokens, ns;
    double       wait_ns;      // the persistent kernel's attention group 0 waiting for its inputs, since the last perf read
    int          cold;         // evict the caches before each forward pass (engine.c:330-338)
    void        *evict;        // EVICT_BYTES of device memory read to evict them
    double       cold_ns;      // host time spent evicting since the last perf read (not token time)
    double       cold_ns_all;  // the same since load
    double       weight_bytes, attn_bytes, ffn_bytes, head_bytes;
    char         desc[256];
};

static double now_ns(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec * 1e9 + (double)ts.tv_nsec;
}

static void *dalloc(l3m_model *m, size_t bytes) {
    if (m->n_allocs == m->cap_allocs) {
        int cap = m->cap_allocs ? 2 * m->cap_allocs : 64;
        void **a = realloc(m->allocs, (size_t)cap * sizeof *a);
        if (!a) return NULL;
        m->allocs = a;
        m->cap_allocs = cap;
    }
    void *p = l3m_dev_alloc(bytes);
    if (p) m->allocs[m->n_allocs++] = p;
    return p;
}

static void *dupload(l3m_model *m, const void *src, size_t bytes) {
    void *p = dalloc(m, bytes);
    if (p && l3m_dev_upload(p, src, bytes)) return NULL;
    return p;
}

// Pack rows (file pointers or NULL) into a device lane-tile matrix of dtype (f32 in reference mode).
static int upload_mat(l3m_model *m, l3m_dmat *out, int src_dtype, int rows, int k, const void *const *src) {
    int dt = m->reference ? L3M_F32 : src_dtype;
    size_t qs = l3m_lt_quant_size(dt, rows, k), ss = l3m_lt_scale_size(dt, rows, k);
    uint8_t *q = malloc(qs), *s = ss ? malloc(ss) : NULL;
    if (!q || (ss && !s)) { free(q); free(s); return -1; }
    if (m->reference) l3m_lt_pack_rows_f32(src_dtype, rows, k, src, q);
    else l3m_lt_pack_rows(dt, rows, k, src, q, s);
    out->q = dupload(m, q, qs);
    out->s = ss ? dupload(m, s, ss) : NULL;
    out->rows = rows; out->tiles = (rows + 15) / 16; out->nb = (k + 31) / 32; out->dtype = dt;
    free(q); free(s);
    m->weight_bytes += (double)(qs + ss);
    return out->q && (!ss || out->s) ? 0 : -1;
}

// A step kernel's matrix (q/k/v rows, Wo columns, gate/up rows, Wdown columns): stored in
// l3m_step_a_dtype(src_dtype). q4_0 rows widen exactly to q8_0 blocks (byte q - 8, the same scale); the
// bytes counted are the source's.
// The f16 bits of 2^e for -24 <= e <= 15 (the powers of two f16 holds), else -1.
static int f16_pow2(int e) {
    if (e < -24 || e > 15) return -1;
    return e >= -14 ? (e + 15) << 10 : 1 << (e + 24);
}

// An mxfp4 block as a q8_0 block with the same values: d = 2^(e - 128) and the doubled e2m1 codes
// (L3M_E2M1X2), exact when d is an f16 (104 <= e <= 143) or every code is zero. Returns 0 on success.
static int mxfp4_q8(const l3m_block_mxfp4 *in, l3m_block_q8_0 *o) {
    int any = 0;
    for (int j = 0; j < 16; j++) {
        o->qs[j] = L3M_E2M1X2[in->qs[j] & 15];
        o->qs[16 + j] = L3M_E2M1X2[in->qs[j] >> 4];
        any |= o->qs[j] | o->qs[16 + j];
    }
    const int h = f16_pow2((int)in->e - 128);
    if (h < 0 && any) return -1;
    o->d = h < 0 ? 0 : (uint16_t)h;
    return 0;
}

// Whether every block of the body's mxfp4 matrices widens exactly to q8_0 (mxfp4_q8).
static int mxfp4_body_widens(const l3m_mapped *f, int n_layers) {
    static const char *names[] = {"wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"};
    l3m_block_q8_0 tmp;
    for (int l = 0; l < n_layers; l++)
        for (int i = 0; i < 7; i++) {
            const l3m_tensor *t = l3m_map_blk(f, l, names[i]);
            if (!t || t->dtype != L3M_MXFP4 || t->shape[1] % 32) return 0;
            const l3m_block_mxfp4 *b = l3m_map_data(f, t);
            for (size_t n = (size_t)t->shape[0] * (size_t)(t->shape[1] / 32); n--; b++)
                if (mxfp4_q8(b, &tmp)) return 0;
        }
    return 1;
}

// q4_0 or mxfp4 file rows as q8_0 file rows of the same values (exact): q4_0 byte n - 8 with the same
// scale; mxfp4 the doubled e2m1 codes with d = 2^(e - 128). dst holds rows * (k / 32) q8_0 blocks; a NULL
// source row leaves its blocks zero. -1 when an mxfp4 block's scale is no f16 and its codes are not all
// zero (it does not widen exactly), or the dtype or k do not apply.
int l3m_widen_rows(int src_dtype, int rows, int k, const void *const *src, void *dst) {
    if ((src_dtype != L3M_Q4_0 && src_dtype != L3M_MXFP4) || k % 32 || rows < 0) return -1;
    const size_t nb = (size_t)k / 32;
    l3m_block_q8_0 *buf = dst;
    memset(buf, 0, (size_t)rows * nb * sizeof *buf);
    for (int r = 0; r < rows; r++) {
        if (!src[r]) continue;
        l3m_block_q8_0 *o = buf + (size_t)r * nb;
        if (src_dtype == L3M_MXFP4) {
            const l3m_block_mxfp4 *in = (const l3m_block_mxfp4 *)src[r];
            for (size_t b = 0; b < nb; b++)
                if (mxfp4_q8(in + b, o + b)) return -1;
        } else {
            const l3m_block_q4_0 *in = (const l3m_block_q4_0 *)src[r];
            for (size_t b = 0; b < nb; b++) {
                o[b].d = in[b].d;
                for (int j = 0; j < 16; j++) {
                    o[b].qs[j] = (int8_t)((in[b].qs[j] & 15) - 8);
                    o[b].qs[16 + j] = (int8_t)((in[b].qs[j] >> 4) - 8);
                }
            }
        }
    }
    return 0;
}

// Uploads q4_0 or mxfp4 rows as q8_0 rows of the same values (l3m_widen_rows; -1 if an mxfp4 block does
// not widen exactly). weight_bytes counts the source's bytes.
static int upload_widened(l3m_model *m, l3m_dmat *out, int src_dtype, int rows, int k, const void *const *src) {
    if ((src_dtype != L3M_Q4_0 && src_dtype != L3M_MXFP4) || k % 32) return -1;
    size_t nb = (size_t)k / 32;
    l3m_block_q8_0 *buf = malloc((size_t)rows * nb * sizeof *buf);
    const void **wide = malloc((size_t)rows * sizeof *wide);
    if (!buf || !wide || l3m_widen_rows(src_dtype, rows, k, src, buf)) { free(buf); free(wide); return -1; }
    for (int r = 0; r < rows; r++) wide[r] = src[r] ? buf + (size_t)r * nb : NULL;
    const double before = m->weight_bytes;
    int rc = upload_mat(m, out, L3M_Q8_0, rows, k, wide);
    m->weight_bytes = before + (double)(l3m_lt_quant_size(src_dtype, rows, k) + l3m_lt_scale_size(src_dtype, rows, k));
    free(buf); free(wide);
    return rc;
}

static int upload_step_mat(l3m_model *m, l3m_dmat *out, int src_dtype, int rows, int k, const void *const *src) {
    if (m->mx_wide && src_dtype == L3M_MXFP4) return upload_widened(m, out, src_dtype, rows, k, src);
    int dt = m->reference ? src_dtype : l3m_step_a_dtype(src_dtype);
    if (dt == src_dtype) return upload_mat(m, out, src_dtype, rows, k, src);
    if (src_dtype != L3M_Q4_0 || dt != L3M_Q8_0) return -1;
    return upload_widened(m, out, src_dtype, rows, k, src);
}

static const void *frow(const l3m_mapped *f, const l3m_tensor *t, int r) {
    return (const uint8_t *)l3m_map_data(f, t) + (size_t)r * l3m_file_row_bytes((int)t->dtype, (int)t->shape[1]);
}

// Layer l's f32 vector `name` on the device, or n zeros when the file leaves it out (optional biases).
static const float *vec_or_zero(l3m_model *m, const l3m_mapped *f, int l, const char *name, int n) {
    const l3m_tensor *t = l3m_map_blk(f, l, name);
    if (t) return dupload(m, l3m_map_data(f, t), (size_t)n * 4);
    float *z = calloc((size_t)n, 4);
    const float *d = z ? dupload(m, z, (size_t)n * 4) : NULL;
    free(z);
    return d;
}

// A prefill matrix: q8_0 lane tiles (q4_0 widened as the step matrices are; mxfp4 widened exactly).
static int upload_pf_mat(l3m_model *m, l3m_dmat *out, int src_dtype, int rows, int k, const void *const *src) {
    if (src_dtype == L3M_MXFP4 || src_dtype == L3M_Q4_0) return upload_widened(m, out, src_dtype, rows, k, src);
    return upload_step_mat(m, out, src_dtype, rows, k, src);
}

// The prefill matrices of layer l: the whole wq|wk|wv, wo, w_gate|w_up and w_down as q8_0 lane tiles. A second copy of the body, not counted in the bytes a decode
// step streams.
static int upload_prefill(l3m_model *m, const l3m_mapped *f, int l, int dt, const l3m_dlayer *L) {
    const l3m_dmodel *d = &m->dm;
    const int hd = d->hd, nq = d->n_heads * hd, nk = d->n_kv * hd;
    int cap = nq + 2 * nk;
    if (2 * d->ffn > cap) cap = 2 * d->ffn;
    if (d->dim > cap) cap = d->dim;
    const void **rows = malloc((size_t)cap * sizeof *rows);
    if (!rows) return -1;
    const l3m_tensor *wq = l3m_map_blk(f, l, "wq"), *wk = l3m_map_blk(f, l, "wk"), *wv = l3m_map_blk(f, l, "wv");
    const l3m_tensor *wo = l3m_map_blk(f, l, "wo"), *wg = l3m_map_blk(f, l, "w_gate"), *wu = l3m_map_blk(f, l, "w_up");
    const l3m_tensor *wd = l3m_map_blk(f, l, "w_down");
    l3m_pflayer *P = &m->pf[l];
    const double before = m->weight_bytes;
    int rc = 0, n = 0;
    for (int r = 0; r < nq; r++) rows[n++] = frow(f, wq, r);
    for (int r = 0; r < nk; r++) rows[n++] = frow(f, wk, r);
    for (int r = 0; r < nk; r++) rows[n++] = frow(f, wv, r);
    rc |= upload_pf_mat(m, &P->qkv, dt, n, d->dim, rows);
    for (int r = 0; r < d->dim; r++) rows[r] = frow(f, wo, r);
    rc |= upload_pf_mat(m, &P->wo, dt, d->dim, nq, rows);
    for (int r = 0; r < d->ffn; r++) { rows[r] = frow(f, wg, r); rows[d->ffn + r] = frow(f, wu, r); }
    rc |= upload_pf_mat(m, &P->gu, dt, 2 * d->ffn, d->dim, rows);
    for (int r = 0; r < d->dim; r++) rows[r] = frow(f, wd, r);
    rc |= upload_pf_mat(m, &P->down, dt, d->dim, d->ffn, rows);
    P->attn_norm = L->attn_norm;
    P->ffn_norm = L->ffn_norm;
    m->weight_bytes = before;
    free(rows);
    return rc || P->qkv.dtype != L3M_Q8_0 ? -1 : 0;
}

// The file row starting at input column c (whole 32-blocks for quantized rows).
static const void *col_slice(const void *row, int dtype, int c) {
    return (const uint8_t *)row + (dtype >= L3M_Q8_0 ? l3m_file_row_bytes(dtype, c) : (size_t)c * (dtype == L3M_BF16 ? 2 : 4));
}

static int upload_tensor(l3m_model *m, l3m_dmat *out, const l3m_tensor *t) {
    int rows = (int)t->shape[0], k = (int)t->shape[1];
    const void **src = malloc((size_t)rows * sizeof *src);
    if (!src) return -1;
    for (int r = 0; r < rows; r++) src[r] = frow(&m->f, t, r);
    int rc = upload_mat(m, out, (int)t->dtype, rows, k, src);
    free(src);
    return rc;
}

static l3m_model *fail(l3m_model *m, const char *msg) {
    if (msg) fprintf(stderr, "l3m: %s\n", msg);
    l3m_free(m);
    return NULL;
}

// The reference's angles (ops.c:31-32): angle = pos * powf(theta, -2i/hd), with the host libm.
void l3m_rope_table(float *table, int ctx, int hd, float theta) {
    for (int pos = 0; pos < ctx; pos++)
        for (int i = 0; i < hd / 2; i++) {
            float angle = pos * powf(theta, -2.0f * i / hd);
            table[((size_t)pos * (hd / 2) + i) * 2] = cosf(angle);
            table[((size_t)pos * (hd / 2) + i) * 2 + 1] = sinf(angle);
        }
}

l3m_model *l3m_load(const char *path, const l3m_opts *opts) {
    l3m_opts o = {0};
    if (opts) o = *opts;
    l3m_model *m = calloc(1, sizeof *m);
    if (!m) return NULL;
    m->logits_pos = -1;
    m->spin_limit = SPIN_LIMIT;
    if (l3m_map_open(&m->f, path)) { free(m); return NULL; }      // a bad file is reported as such first
    if (!l3m_hip_kernels_usable()) {
        fprintf(stderr, "l3m: no usable HIP device: %s\n", l3m_dev_error() ? l3m_dev_error() : "unknown");
        l3m_map_close(&m->f);
        free(m);
        return NULL;
    }
    const l3m_header *const h = m->f.h;
    const l3m_mapped *f = &m->f;
    // the GPT-2 variant runs as the whole family (LayerNorm with biases, learned positions, GELU MLP);
    // other mixes of those flags, or biases on a Llama model, are not on the GPU path
    const unsigned g2f = L3M_F_LAYERNORM | L3M_F_LEARNED_POS | L3M_F_GELU;
    const int gpt2 = (h->flags & g2f) == g2f;
    if ((h->flags & g2f) && !gpt2)
        return fail(m, "a mix of LayerNorm, GELU and learned positions other than the GPT-2 family is not on the GPU path");
    for (int l = 0; l < (int)h->n_layers && !gpt2; l++) {
        static const char *const bias[] = {"bq", "bk", "bv", "bo", "b_up", "b_down"};
        for (int i = 0; i < 6; i++)
            if (l3m_map_blk(f, l, bias[i])) return fail(m, "bias tensors on a Llama model are not on the GPU path");
    }
    l3m_dmodel *d = &m->dm;
    d->gpt2 = gpt2;
    m->reference = o.reference != 0;
    d->dim = (int)h->dim; d->n_heads = (int)h->n_heads; d->n_kv = (int)h->n_kv_heads; d->hd = d->dim / d->n_heads;
    d->kv_dim = d->hd * d->n_kv; d->ffn = (int)h->ffn_dim; d->vocab = (int)h->vocab;
    d->n_layers = (int)h->n_layers; d->eps = h->norm_eps; d->nslots = NSLOTS;
    d->ctx = (int)h->ctx < (o.ctx > 0 ? o.ctx : DEFAULT_CTX) ? (int)h->ctx : (o.ctx > 0 ? o.ctx : DEFAULT_CTX);
    if (d->hd > 256 || d->hd % 8) return fail(m, "the GPU attention kernel needs head_dim a multiple of 8, at most 256");
    if (d->dim % 4) return fail(m, "the GPU kernels need dim a multiple of 4");
    if (d->dim > 4096) return fail(m, "dim up to 4096 is supported by the GPU kernels");
    if (d->ctx > 8192) return fail(m, "ctx up to 8192 is supported by the GPU attention kernel");
    m->dtype = (int)l3m_map_blk(f, 0, "w_up")->dtype;
    // An mxfp4 body whose every block widens exactly (d = 2^(e-128) an f16, or all codes zero) runs its
    // step matrices as q8_0 blocks of the same values: the same integer dots and float operations as the
    // e2m1 path, without the per-code decode in the matvec loop (L3M_WIDEN=0 keeps the mxfp4 blocks).
    const char *wd_ = getenv("L3M_WIDEN");
    m->mx_wide = !m->reference && m->dtype == L3M_MXFP4 && (!wd_ || strcmp(wd_, "0")) && mxfp4_body_widens(f, (int)h->n_layers);

    // weights: per layer the head groups (q/k/v rows and Wo columns) and the FFN chunks (gate/up rows
    // and Wdown columns) of the two step kernels, then the head
    int quant = !m->reference && m->dtype >= L3M_Q8_0, hpk = d->n_heads / d->n_kv, nq = 1;
    while (quant && nq * d->hd % 32) nq++;                   // Wo slices of whole activation blocks
    if (d->n_heads % nq) nq = d->n_heads;
    d->n_groups = d->n_heads / nq;
    // FFN chunk (rows, a multiple of 32): at most the most rows whose gate/up rows (up rows only for GPT-2)
    // take at most one 16-row tile per wavefront and, with the Wdown columns, fit the weight slots a
    // workgroup holds in flight (one pass of loads covers the chunk). Every dtype takes the most rows that
    // do: fewer chunks, fewer partials for every attention prologue, at the same FFN time (stories15M bf16
    // +1.5% at 96 rows against 64, stories42M q8_0 at ctx 1024 +3.2% at 128 rows against 64; stories110M
    // q4_0 within 0.3% from 64 to 128 rows, 16% slower at 160). Then larger (more passes of loads) while
    // the body would not fit one XCD.
    int sdt = m->reference ? L3M_F32 : m->mx_wide ? L3M_Q8_0 : m->dtype, cap_a = 64 * l3m_step_slots(sdt, 0), cap_b = 64 * l3m_step_slots(sdt, 1);
    int nbd = (d->dim + 31) / 32, chunk = 32, gu = gpt2 ? 1 : 2;
    for (int c = 256; c >= 32; c -= 32)
        if (gu * c <= 16 * 16 && gu * c / 16 * nbd <= cap_a && (d->dim + 15) / 16 * (c / 32) <= cap_b) { chunk = c; break; }
    const char *ck_ = getenv("L3M_FFN_CHUNK");      // rows per FFN chunk (a multiple of 32), for measurement
    if (ck_ && atoi(ck_) >= 32 && atoi(ck_) % 32 == 0) chunk = atoi(ck_);
    while ((d->ffn + chunk - 1) / chunk > MAX_PARTS || (d->n_groups + (d->ffn + chunk - 1) / chunk > BODY_CUS && chunk < d->ffn)) chunk += 32;
    d->n_chunks = (d->ffn + chunk - 1) / chunk;
    m->chunk_rows = chunk;
    d->body_dtype = sdt;
    if (d->n_groups > MAX_PARTS || d->n_chunks > MAX_PARTS) return fail(m, "too many head groups or FFN chunks for the GPU kernels");
    l3m_model_layout(d);
    m->layers = calloc((size_t)d->n_layers, sizeof *m->layers);
    // batched prefill (q8_0 and q4_0 bodies, and mxfp4 bodies whose blocks widen exactly to q8_0; whole
    // 32-blocks): unless L3M_PREFILL=0
    const char *pe_ = getenv("L3M_PREFILL"), *pm_ = getenv("L3M_PREFILL_MIN");
    const int qb_ = d->dim % 32 == 0 && (d->n_heads * d->hd) % 32 == 0 && d->ffn % 32 == 0;
    if ((!pe_ || strcmp(pe_, "0")) && !m->reference && !gpt2 && qb_ && l3m_prefill_fits(d->dim, d->ffn, d->n_heads * d->hd, d->hd) &&
        (m->dtype == L3M_Q8_0 || m->dtype == L3M_Q4_0 || m->mx_wide || (m->dtype == L3M_MXFP4 && mxfp4_body_widens(f, d->n_layers))))
        m->pf = calloc((size_t)d->n_layers, sizeof *m->pf);
    m->prefill_min = pm_ ? atoi(pm_) : 8;
    l3m_dgroup *groups = calloc((size_t)d->n_groups, sizeof *groups);
    l3m_dchunk *chunks = calloc((size_t)d->n_chunks, sizeof *chunks);
    int max_rows = d->dim > 2 * chunk + 32 ? d->dim : 2 * chunk + 32;
    if ((nq + 2 * d->n_kv) * d->hd > max_rows) max_rows = (nq + 2 * d->n_kv) * d->hd;
    const void **rows = malloc((size_t)max_rows * sizeof *rows);
    if (!m->layers || !groups || !chunks || !rows) { free(groups); free(chunks); free(rows); return fail(m, "out of memory"); }
    unsigned lds_a = 0, lds_a0 = 0, lds_b = 0;
    for (int l = 0; l < d->n_layers; l++) {
        l3m_dlayer *L = &m->layers[l];
        const l3m_tensor *wq = l3m_map_blk(f, l, "wq"), *wk = l3m_map_blk(f, l, "wk"), *wv = l3m_map_blk(f, l, "wv");
        const l3m_tensor *wo = l3m_map_blk(f, l, "wo"), *wg = l3m_map_blk(f, l, "w_gate"), *wu = l3m_map_blk(f, l, "w_up");
        const l3m_tensor *wd = l3m_map_blk(f, l, "w_down");
        if (wo->dtype != wq->dtype || (wg && wg->dtype != wq->dtype) || wu->dtype != wq->dtype || wd->dtype != wq->dtype) {
            free(groups); free(chunks); free(rows);
            return fail(m, "every layer matrix must share one dtype on the GPU path");
        }
        int dt = (int)wq->dtype, rc = 0;
        double before = m->weight_bytes;
        // GPT-2 variant: the layer's norm biases and the biases added once per block, as device vectors
        // (a bias the file leaves out is zero)
        const float *b_up_dev = NULL;
        L->attn_norm_b = L->ffn_norm_b = L->bo = L->bdown = NULL;
        if (gpt2) {
            L->attn_norm_b = vec_or_zero(m, f, l, "attn_norm_b", d->dim);
            L->ffn_norm_b = vec_or_zero(m, f, l, "ffn_norm_b", d->dim);
            L->bo = vec_or_zero(m, f, l, "bo", d->dim);
            L->bdown = vec_or_zero(m, f, l, "b_down", d->dim);
            b_up_dev = vec_or_zero(m, f, l, "b_up", d->ffn);
            if (!L->attn_norm_b || !L->ffn_norm_b || !L->bo || !L->bdown || !b_up_dev) rc = -1;
        }
        for (int gi = 0; gi < d->n_groups; gi++) {
            l3m_dgroup *G = &groups[gi];
            G->q0 = gi * nq; G->nq = nq; G->kv0 = G->q0 / hpk; G->nkv = (G->q0 + nq - 1) / hpk - G->kv0 + 1;
            G->write_kv = 0;
            for (int k = 0; k < G->nkv; k++)
                if ((G->kv0 + k) * hpk >= G->q0 && (G->kv0 + k) * hpk < G->q0 + nq) G->write_kv |= 1u << k;
            int n = 0;
            for (int r = 0; r < nq * d->hd; r++) rows[n++] = frow(f, wq, G->q0 * d->hd + r);
            for (int r = 0; r < G->nkv * d->hd; r++) rows[n++] = frow(f, wk, G->kv0 * d->hd + r);
            for (int r = 0; r < G->nkv * d->hd; r++) rows[n++] = frow(f, wv, G->kv0 * d->hd + r);
            rc |= upload_step_mat(m, &G->qkv, dt, n, d->dim, rows);
            for (int r = 0; r < d->dim; r++) rows[r] = col_slice(frow(f, wo, r), dt, G->q0 * d->hd);
            rc |= upload_step_mat(m, &G->wo, dt, d->dim, nq * d->hd, rows);
            G->bqkv = NULL;
            if (gpt2) {                                  // [bq of the group's heads | bk | bv of its kv heads]
                float *b = calloc((size_t)n, sizeof *b);
                const l3m_tensor *bq = l3m_map_blk(f, l, "bq"), *bk = l3m_map_blk(f, l, "bk"), *bv = l3m_map_blk(f, l, "bv");
                if (!b) rc = -1;
                else {
                    if (bq) memcpy(b, (const float *)l3m_map_data(f, bq) + G->q0 * d->hd, (size_t)nq * d->hd * 4);
                    if (bk) memcpy(b + nq * d->hd, (const float *)l3m_map_data(f, bk) + G->kv0 * d->hd, (size_t)G->nkv * d->hd * 4);
                    if (bv) memcpy(b + (nq + G->nkv) * d->hd, (const float *)l3m_map_data(f, bv) + G->kv0 * d->hd, (size_t)G->nkv * d->hd * 4);
                    G->bqkv = dupload(m, b, (size_t)n * 4);
                    if (!G->bqkv) rc = -1;
                    free(b);
                }
            }
            l3m_group_layout(d->body_dtype, d->dim, d->ctx, d->hd, G);
            unsigned la = l3m_lds_attn(d->body_dtype, d->dim, d->ctx, d->hd, G, 1), la0 = l3m_lds_attn(d->body_dtype, d->dim, d->ctx, d->hd, G, 0);
            if (la > lds_a) lds_a = la;
            if (la0 > lds_a0) lds_a0 = la0;
        }
        double attn = m->weight_bytes - before;
        for (int ci = 0; ci < d->n_chunks; ci++) {
            l3m_dchunk *Cc = &chunks[ci];
            Cc->f0 = ci * chunk;
            Cc->nf = d->ffn - Cc->f0 < chunk ? d->ffn - Cc->f0 : chunk;
            int tiles = (Cc->nf + 15) / 16;
            Cc->bup = NULL;
            if (gpt2) {                                  // the up rows only (GELU MLP, no gate)
                for (int r = 0; r < 16 * tiles; r++) rows[r] = r < Cc->nf ? frow(f, wu, Cc->f0 + r) : NULL;
                rc |= upload_step_mat(m, &Cc->gate_up, dt, 16 * tiles, d->dim, rows);
                Cc->bup = b_up_dev ? b_up_dev + Cc->f0 : NULL;
            } else {
                for (int r = 0; r < 16 * tiles; r++) {       // gate row r, then up row r
                    rows[2 * r] = r < Cc->nf ? frow(f, wg, Cc->f0 + r) : NULL;
                    rows[2 * r + 1] = r < Cc->nf ? frow(f, wu, Cc->f0 + r) : NULL;
                }
                rc |= upload_step_mat(m, &Cc->gate_up, dt, 32 * tiles, d->dim, rows);
            }
            for (int r = 0; r < d->dim; r++) rows[r] = col_slice(frow(f, wd, r), dt, Cc->f0);
            rc |= upload_step_mat(m, &Cc->down, dt, d->dim, Cc->nf, rows);
            l3m_chunk_layout(d->body_dtype, d->dim, Cc);
            unsigned lb = l3m_lds_ffn(d->body_dtype, d->dim, Cc);
            if (lb > lds_b) lds_b = lb;
        }
        if (l == 0) { m->attn_bytes = attn; m->ffn_bytes = m->weight_bytes - before - attn; }
        L->groups = dupload(m, groups, (size_t)d->n_groups * sizeof *groups);
        L->chunks = dupload(m, chunks, (size_t)d->n_chunks * sizeof *chunks);
        L->attn_norm = dupload(m, l3m_map_data(f, l3m_map_blk(f, l, "attn_norm")), (size_t)d->dim * 4);
        L->ffn_norm = dupload(m, l3m_map_data(f, l3m_map_blk(f, l, "ffn_norm")), (size_t)d->dim * 4);
        if (rc || !L->groups || !L->chunks || !L->attn_norm || !L->ffn_norm) {
            free(groups); free(chunks); free(rows);
            return fail(m, "weight upload failed");
        }
        if (m->pf && upload_prefill(m, f, l, dt, L)) {
            free(groups); free(chunks); free(rows);
            return fail(m, "prefill weight upload failed");
        }
    }
    // The K/V window: every position of the context when it fits in LDS beside the rest of the attention
    // block, else the most positions (a multiple of 32) that fit; a step at a position past it reads K and V
    // from the cache. The offsets of l3m_group_layout do not depend on the window (it is the last region).
    int kv_win = d->ctx;
    for (;;) {
        unsigned need = 0;
        for (int gi = 0; gi < d->n_groups; gi++) {
            const unsigned la = l3m_lds_attn(d->body_dtype, d->dim, kv_win, d->hd, &groups[gi], 1);
            if (la > need) need = la;
        }
        lds_a = need;
        if (need <= l3m_dev_lds_max() || kv_win <= 32) break;
        kv_win = kv_win == d->ctx ? (d->ctx - 1) & ~31 : kv_win - 32;
    }
    free(groups); free(chunks); free(rows);
    const l3m_tensor *embed = l3m_map_tensor(f, "embed");
    double body = m->weight_bytes;
    if (upload_tensor(m, &d->embed, embed)) return fail(m, "embedding upload failed");
    if (h->flags & L3M_F_TIED) d->head = d->embed;
    else {
        m->weight_bytes = body;       // an untied embedding is one row per token, not streamed
        if (upload_tensor(m, &d->head, l3m_map_tensor(f, "lm_head"))) return fail(m, "lm_head upload failed");
    }
    m->head_bytes = m->weight_bytes - body;
    d->norm = dupload(m, l3m_map_data(f, l3m_map_tensor(f, "norm")), (size_t)d->dim * 4);
    d->norm_b = NULL; d->pos_embed = NULL;
    if (gpt2) {
        const l3m_tensor *nb = l3m_map_tensor(f, "norm_b"), *pe = l3m_map_tensor(f, "pos_embed");
        d->norm_b = nb ? dupload(m, l3m_map_data(f, nb), (size_t)d->dim * 4) : NULL;
        d->pos_embed = pe ? dupload(m, l3m_map_data(f, pe), (size_t)d->ctx * d->dim * 4) : NULL;
        if (!d->norm_b || !d->pos_embed) return fail(m, "GPT-2 norm bias or position table upload failed");
    }
    d->head_tiles_per_wg = (d->head.tiles + HEAD_WGS - 1) / HEAD_WGS;
    d->head_grid = (d->head.tiles + d->head_tiles_per_wg - 1) / d->head_tiles_per_wg;
    unsigned lds_max = l3m_dev_lds_max();
    d->kv_lds = lds_a <= lds_max;                // the K, V window in LDS when 32 positions fit beside the rest
    d->kv_win = d->kv_lds ? kv_win : 0;
    d->lds_a = d->kv_lds ? lds_a : lds_a0; d->lds_b = lds_b;
    d->lds_h = l3m_lds_head(d->head.dtype, d->dim, d->head.nb, d->head_tiles_per_wg);
    if (d->lds_a > lds_max || d->lds_b > lds_max || d->lds_h > lds_max || d->head_tiles_per_wg > 64)
        return fail(m, "model geometry needs more LDS per workgroup than this GPU has");

    // activations and state
    size_t kv = (size_t)d->n_layers * d->n_kv * d->ctx * d->hd * 2;
    // the call area (struct l3m_model): 256-byte aligned pieces
    m->call_samp = 256;
    m->call_tok = m->call_samp + (sizeof(l3m_dsample) + 255) / 256 * 256;
    m->call_slot[0] = m->call_tok + (((size_t)d->ctx + 1) * 4 + 255) / 256 * 256;
    m->call_slot[1] = m->call_slot[0] + 256 + (size_t)L3M_SYNC_WORDS * 4;
    const size_t call_bytes = m->call_slot[1] + 256 + (size_t)L3M_SYNC_WORDS * 4;
    _Static_assert(sizeof(l3m_run) <= 256, "launch parameters fit their 256 bytes");
    m->call_dev = dalloc(m, call_bytes);
    m->call_host = l3m_dev_host_alloc(call_bytes);
    if (!m->call_dev || !m->call_host) return fail(m, "device allocation failed");
    memset(m->call_host, 0, call_bytes);
    d->pos = (int *)m->call_dev;
    d->samp = (l3m_dsample *)(m->call_dev + m->call_samp);
    d->tokens = (int32_t *)(m->call_dev + m->call_tok);
    m->stage_pos = (int *)m->call_host;
    m->stage_smp = (l3m_dsample *)(m->call_host + m->call_samp);
    m->stage_tok = (int32_t *)(m->call_host + m->call_tok);
    for (int sl = 0; sl < 2; sl++) {
        m->run_dev[sl] = (l3m_run *)(m->call_dev + m->call_slot[sl]);
        m->run_host[sl] = (l3m_run *)(m->call_host + m->call_slot[sl]);
        m->sync[sl] = (unsigned *)(m->call_dev + m->call_slot[sl] + 256);
    }
    d->xa = dalloc(m, (size_t)d->dim * 4);
    d->xb = dalloc(m, (size_t)d->dim * 4);
    d->po = dalloc(m, (size_t)d->n_groups * d->dim * 4);
    d->pd = dalloc(m, (size_t)d->n_chunks * d->dim * 4);
    if (m->pf) {
        int mk = d->dim > d->n_heads * d->hd ? d->dim : d->n_heads * d->hd;
        if (d->ffn > mk) mk = d->ffn;
        const size_t kp = (size_t)(mk + 31) / 32 * 32, ctx = (size_t)d->ctx;
        m->pfb.astride = (int)((kp + 8 * (kp / 32) + 15) / 16 * 16);   // int8 values, f32 scales, i32 sums
        m->pfb.x = dalloc(m, ctx * d->dim * 4);
        m->pfb.act = dalloc(m, ctx * m->pfb.astride);
        m->pfb.qkv = dalloc(m, ctx * (size_t)(d->n_heads + 2 * d->n_kv) * d->hd * 4);
        m->pfb.att = dalloc(m, ctx * (size_t)d->n_heads * d->hd * 4);
        m->pfb.gu = dalloc(m, ctx * 2 * (size_t)d->ffn * 4);
        if (!m->pfb.x || !m->pfb.act || !m->pfb.qkv || !m->pfb.att || !m->pfb.gu) return fail(m, "out of device memory");
        const char *pg = getenv("L3M_PREFILL_GRAPH");  // 0: loose launches (for comparison)
        if ((!pg || strcmp(pg, "0")) && !(m->pfg = l3m_pfgraphs_new())) return fail(m, "out of host memory");
    }
    d->logits = dalloc(m, (size_t)NSLOTS * d->vocab * 4);
    // persistent kernel: one workgroup per CU (the LDS request keeps a second one off each CU); the body
    // (head groups, then FFN chunks) on the workgroups of one XCD, every other workgroup on head tiles.
    // Used when the grid fits on the device at once and one XCD holds the body.
    m->grid = l3m_dev_cus();
    const int n_body = d->n_groups + d->n_chunks;
    if (m->grid > n_body) {
        int spare = m->grid - n_body;
        if (spare > L3M_MAX_HEAD_WGS) spare = L3M_MAX_HEAD_WGS;
        m->head_tpw = (d->head.tiles + spare - 1) / spare;
        m->n_head = (d->head.tiles + m->head_tpw - 1) / m->head_tpw;
        unsigned lh = l3m_lds_head(d->head.dtype, d->dim, d->head.nb, m->head_tpw);
        m->lds_decode = d->lds_a > d->lds_b ? d->lds_a : d->lds_b;
        if (lh > m->lds_decode) m->lds_decode = lh;
        if (m->lds_decode < lds_max / 2 + 16) m->lds_decode = lds_max / 2 + 16;
        const char *pe = getenv("L3M_PERSIST");
        m->persist = (!pe || strcmp(pe, "0")) && l3m_decode_pair(d->body_dtype, d->head.dtype, gpt2) && d->n_groups <= 64 &&
                     d->n_chunks <= 64 && d->vocab <= 0x20000 && m->head_tpw <= 64 && m->lds_decode <= lds_max &&
                     l3m_decode_fits(d->body_dtype, d->head.dtype, gpt2, d->hd, m->grid, m->lds_decode);
        int *xcc = m->persist ? calloc((size_t)m->grid, sizeof *xcc) : NULL;
        if (xcc && !l3m_decode_placement(m->grid, m->lds_decode, xcc)) {
            int count[16] = {0};
            for (int b = 0; b < m->grid; b++) count[xcc[b] & 15]++;
            m->body_xcc = 0;
            for (int x = 1; x < 16; x++)
                if (count[x] > count[m->body_xcc]) m->body_xcc = x;
            m->persist = count[m->body_xcc] >= n_body;
        } else if (m->persist) {
            m->persist = 0;
            if (xcc) l3m_dev_clear_error();   // a refused probe only means no persistent kernel
        }
        free(xcc);
    }
    int parts = d->head_grid > m->grid ? d->head_grid : m->grid;
    d->part_val = dalloc(m, (size_t)parts * 4);
    d->part_idx = dalloc(m, (size_t)parts * 4);
    m->out_host = l3m_dev_host_alloc(2 * sizeof(l3m_chunk_out));
    m->ev[0] = l3m_dev_event_new();
    m->ev[1] = l3m_dev_event_new();
    m->dm_dev = dalloc(m, sizeof(l3m_dmodel));
    m->layers_dev = dupload(m, m->layers, (size_t)d->n_layers * sizeof *m->layers);
    d->done = dalloc(m, 4);
    d->kc = dalloc(m, kv);
    d->vc = dalloc(m, kv);
    float *rope = malloc((size_t)d->ctx * d->hd * sizeof(float));
    if (rope) l3m_rope_table(rope, d->ctx, d->hd, h->rope_theta);
    d->rope = rope ? dupload(m, rope, (size_t)d->ctx * d->hd * sizeof(float)) : NULL;
    free(rope);
    m->logits = calloc((size_t)d->vocab, sizeof *m->logits);
    if (!d->pos || !d->tokens || !d->xa || !d->xb || !d->po || !d->pd || !d->samp || !d->logits || !d->part_val || !d->part_idx || !d->done ||
        !d->kc || !d->vc || !d->rope || !d->norm || !m->logits || !m->layers_dev ||
        !m->out_host || !m->ev[0] || !m->ev[1] ||
        !m->dm_dev || l3m_dev_upload(m->dm_dev, d, sizeof *d))
        return fail(m, "device allocation failed");
    m->cold = o.cold != 0;
    if (m->cold && !(m->evict = dalloc(m, EVICT_BYTES))) return fail(m, "--cold: no device memory for the eviction buffer");
    const char *g = getenv("L3M_GRAPH");
    if (!g || strcmp(g, "0")) {
        m->graphs = l3m_graphs_build(d, m->layers);
        if (!m->graphs) return fail(m, "could not capture the decode step");
    }
    const char *base = strrchr(path, '/');
    base = base ? base + 1 : path;
    if (m->reference)
        snprintf(m->desc, sizeof m->desc, "%s: %s, %d layers, reference fp32 on 1 gpu (hip)", base, l3m_dtype_name(m->dtype), d->n_layers);
    else
        snprintf(m->desc, sizeof m->desc, "%s: %s, %d layers, %.1f MiB on 1 gpu (hip)%s", base, l3m_dtype_name(m->dtype), d->n_layers,
                 m->weight_bytes / MiB, m->mx_wide ? ", blocks widened exactly to q8_0" : "");
    if (o.verbose)
        fprintf(stderr, "l3m: %s, ctx %d, %s; %d head groups, %d ffn chunks, head %d x %d tiles, lds %u/%u/%u, kv in lds %d (%d positions); "
                "persistent %d (grid %d, body on xcd %d, head %d x %d tiles, lds %u)\n", m->desc, d->ctx, l3m_dev_name(), d->n_groups,
                d->n_chunks, d->head_grid, d->head_tiles_per_wg, d->lds_a, d->lds_b, d->lds_h, d->kv_lds, d->kv_win, m->persist, m->grid, m->body_xcc,
                m->n_head, m->head_tpw, m->lds_decode);
    return m;
}

void l3m_free(l3m_model *m) {
    if (!m) return;
    l3m_dev_sync();
    l3m_graphs_free(m->graphs);
    l3m_pfgraphs_free(m->pfg);
    l3m_dev_host_free(m->call_host);
    l3m_dev_host_free(m->out_host);
    l3m_dev_event_free(m->ev[0]);
    l3m_dev_event_free(m->ev[1]);
    for (int i = 0; i < m->n_allocs; i++) l3m_dev_free(m->allocs[i]);
    free(m->allocs); free(m->layers); free(m->logits); free(m->pf);
    if (m->f.map) l3m_map_close(&m->f);
    free(m);
}

static int step(l3m_model *m, int with_head) {
    return m->graphs ? l3m_graphs_launch(m->graphs, with_head, NULL) : l3m_step_enqueue(&m->dm, m->layers, with_head, NULL);
}

// Positions first..last queued as one run of steps (one persistent launch, or one graph per step; logits
// and a token from head_from on), then the copies of what the host reads back (the launch's abort word, the
// run's tokens) into slot's pinned area, then slot's event. Nothing waits: two runs can be in flight, each
// with its own sync area, launch parameters and pinned area. The sync words are zeroed and the parameters
// copied on the stream, behind the run that used slot before (which the host has waited for).
// from: the call-area byte offset the run's upload starts at (the slot's own parameters, or the start of
// the call area for a call's first run, whose inputs go with them); -1: nothing to upload.
static int chunk_enqueue(l3m_model *m, int first, int last, int head_from, int slot, long from) {
    const l3m_dmodel *d = &m->dm;
    l3m_chunk_out *out = &m->out_host[slot];
    const int f = first > head_from ? first : head_from, ntok = last >= f ? last - f + 1 : 0;
    if (m->persist) {
        // the parameters and the zeroed sync words in one copy from the image; the output span (abort word,
        // wait ticks, tokens) back in one copy
        unsigned *sync = m->sync[slot];
        const l3m_run r = {first, last - first + 1, head_from, m->head_tpw, m->n_head, m->body_xcc, sync, m->spin_limit, m->temp, 0};
        *m->run_host[slot] = r;
        const size_t end = m->call_slot[slot] + 256 + (size_t)L3M_SYNC_WORDS * 4;
        if (l3m_dev_upload_async(m->call_dev + from, m->call_host + from, end - (size_t)from) ||
            l3m_decode_launch(d->body_dtype, d->head.dtype, d->gpt2, d->hd, m->dm_dev, m->layers_dev, m->run_dev[slot], m->grid, m->lds_decode, NULL,
                              slot) ||
            l3m_dev_download_async(out, sync + L3M_SYNC_OUT, offsetof(l3m_chunk_out, tok) + (size_t)ntok * 4))
            return -1;
        for (int p = first; p <= last; p++) {
            m->work[0] += 1;
            m->work[1] += p >= head_from;
            m->work[2] += p + 1;                       // attention reads K, V rows 0..p of every kv head
        }
    } else {
        out->abort = 0;
        out->waited = 0;
        // a call's inputs: the position, the sampler state and the prompt's ids (head_from + 1 of them)
        if (from >= 0 && l3m_dev_upload_async(m->call_dev + from, m->call_host + from, m->call_tok - (size_t)from + (size_t)(head_from + 1) * 4))
            return -1;
        for (int p = first; p <= last; p++)
            if (step(m, p >= head_from)) return -1;
        if (ntok && l3m_dev_download_async(out->tok, d->tokens + f + 1, (size_t)ntok * 4)) return -1;
    }
    return l3m_dev_event_record(m->ev[slot]);
}

// Waits for slot's run of steps; -1 on a device error or a timed-out wait of the persistent kernel.
static int chunk_finish(l3m_model *m, int slot) {
    if (l3m_dev_event_wait(m->ev[slot]) || (m->persist && l3m_decode_timer_collect(slot))) return -1;
    m->wait_ns += 10.0 * (double)m->out_host[slot].waited;
    if (m->out_host[slot].abort) {
        fprintf(stderr, "l3m: decode kernel: a wait between phases timed out\n");
        return -1;
    }
    return 0;
}

// --cold (engine.c:330-338): the caches are emptied of the weights before a forward pass; the eviction is
// not token time. The queue is drained first, so the time counted is the eviction's alone.
static int evict(l3m_model *m) {
    if (l3m_dev_sync()) return -1;
    const double t0 = now_ns();
    if (l3m_dev_evict(m->evict, EVICT_BYTES, NULL) || l3m_dev_sync()) return -1;
    const double dt = now_ns() - t0;
    m->cold_ns += dt;
    m->cold_ns_all += dt;
    return 0;
}

// Run forward passes for positions 0..last (prompt, then greedy or sampled tokens); calls back per the
// reference's rules (engine.c:322-327, 342-362). temperature > 0 samples on the device from the generator
// seeded as engine.c:555 does. Returns the number generated, or -1 on a device error.
//
// The passes run in runs of steps queued on the stream, and the host reads each run's tokens back once it
// has finished. When something can stop the generation early (an on_token callback, or an EOS or BOS id
// the model has), the tokens are handed over as they come: the prompt's run ends at the first generated
// token, the later runs are LIVE_STEPS positions long, and two are kept in flight, so the next run computes
// while the host calls on_token for the last one's tokens; a stop leaves at most the rest of its run and the
// run behind it (under 2 LIVE_STEPS passes) computed in vain. Otherwise runs are NSLOTS positions long, also
// two in flight, so the next launch follows the last on the stream without waiting for the host. --cold
// runs one pass at a time (each after an eviction the host times).
static int run_steps(l3m_model *m, const int32_t *prompt, int n_prompt, int max_new, float temperature, uint64_t seed,
                     int (*on_token)(int32_t, void *), void *user) {
    l3m_dmodel *d = &m->dm;
    const int bos = m->f.tok.bos, eos = m->f.tok.eos;
    const int last = n_prompt - 1 + max_new < d->ctx - 1 ? n_prompt - 1 + max_new : d->ctx - 1;   // exhausted() at engine.c:322
    int n_gen = 0, stop = -1, rc = 0;
    l3m_dsample *smp = m->stage_smp;
    memset(smp, 0, sizeof *smp);
    smp->temp = temperature > 0 ? temperature : 0.0f;
    for (int h = 0; h < L3M_MAX_HEAD_WGS; h++) smp->rng[h] = seed * 0x9E3779B97F4A7C15ull + 1;   // engine.c:555
    m->temp = smp->temp;
    memcpy(m->stage_tok, prompt, (size_t)n_prompt * 4);
    // the image was last read by the previous call's copies, which its final wait covered
    // a long prompt: positions 0..n_prompt-2 in one batched pass, then decode from the last prompt token
    const int prefill = m->pf && n_prompt >= m->prefill_min && n_prompt - 1 >= 1;
    int next = prefill ? n_prompt - 1 : 0;
    *m->stage_pos = next;
    long from = 0;                                     // the first run takes the call's inputs with it
    m->prefilled = 0;
    if (prefill) {                                     // the prefill reads the prompt ids first
        if (l3m_dev_upload_async(m->call_dev, m->call_host, m->call_tok + (size_t)n_prompt * 4)) return -1;
        from = -1;
        if (m->cold && evict(m)) return -1;
        if (m->pfg ? l3m_prefill_graph(m->pfg, d, m->pf, &m->pfb, n_prompt - 1) : l3m_prefill(d, m->pf, &m->pfb, n_prompt - 1, NULL))
            return -1;
        m->prefilled = n_prompt - 1;
    }
    const int live = on_token != NULL || bos >= 0 || eos >= 0, depth = m->cold ? 1 : 2;
    int q_first[2], q_end[2], q_slot[2], nq = 0, slot = 0;
    for (;;) {
        while (!rc && stop < 0 && next <= last && nq < depth) {
            // --cold: one forward pass per run, each after an eviction
            int len = m->cold ? 1 : !live ? NSLOTS : next <= n_prompt - 1 ? n_prompt - next : LIVE_STEPS;
            if (len > NSLOTS) len = NSLOTS;
            const int end = next + len - 1 < last ? next + len - 1 : last;
            const long up = from >= 0 ? from : m->persist ? (long)m->call_slot[slot] : -1;
            from = -1;
            if ((m->cold && evict(m)) || chunk_enqueue(m, next, end, n_prompt - 1, slot, up)) {
                rc = -1;
                break;
            }
            q_first[nq] = next; q_end[nq] = end; q_slot[nq] = slot; nq++;
            slot ^= 1;
            next = end + 1;
        }
        if (!nq) break;
        const int first = q_first[0], end = q_end[0], s = q_slot[0];
        q_first[0] = q_first[1]; q_end[0] = q_end[1]; q_slot[0] = q_slot[1];
        nq--;
        if (chunk_finish(m, s)) rc = -1;               // the runs still in flight are waited for all the same
        if (rc || stop >= 0) continue;
        const int f = first > n_prompt - 1 ? first : n_prompt - 1;
        for (int p = f; p <= end && p < last; p++) {
            const int32_t tok = m->out_host[s].tok[p - f];
            if (tok == eos || tok == bos) { stop = p; break; }                 // accepted(), engine.c:323-327
            n_gen++;
            if (on_token && !on_token(tok, user)) { stop = p; break; }
        }
    }
    if (l3m_dev_sync() || rc) return -1;
    m->logits_pos = stop >= 0 ? stop : last;
    m->logits_fresh = 0;
    m->tokens += m->logits_pos + 1;
    return n_gen;
}

// run_steps, its time counted for l3m_perf (the generate calls and the bench loop alike).
static int run(l3m_model *m, const int32_t *prompt, int n_prompt, int max_new, float temperature, uint64_t seed,
               int (*on_token)(int32_t, void *), void *user) {
    const double t0 = now_ns();
    const int n = run_steps(m, prompt, n_prompt, max_new, temperature, seed, on_token, user);
    m->ns += now_ns() - t0;
    return n;
}

int l3m_generate(l3m_model *m, const int32_t *prompt, int n_prompt, int max_new, float temperature, uint64_t seed,
                 int (*on_token)(int32_t, void *), void *user) {
    if (n_prompt < 1 || n_prompt >= m->dm.ctx) return 0;
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= m->dm.vocab) { fprintf(stderr, "l3m: token %d out of range\n", prompt[i]); return -1; }
    const int n = run(m, prompt, n_prompt, max_new < 0 ? 0 : max_new, temperature, seed, on_token, user);
    if (n < 0) fprintf(stderr, "l3m: generate failed on the device: %s\n", l3m_dev_error() ? l3m_dev_error() : "?");
    return n;
}

const float *l3m_logits(const l3m_model *m) {
    l3m_model *mm = (l3m_model *)m;
    if (m->logits_pos >= 0 && !m->logits_fresh) {
        const float *slot = m->dm.logits + (size_t)(m->logits_pos % NSLOTS) * m->dm.vocab;
        if (!l3m_dev_download(mm->logits, slot, (size_t)m->dm.vocab * 4)) mm->logits_fresh = 1;
    }
    return m->logits;
}

int l3m_vocab(const l3m_model *m) { return m->dm.vocab; }
int l3m_ctx(const l3m_model *m) { return m->dm.ctx; }
const char *l3m_describe(const l3m_model *m) { return m->desc; }
int l3m_bos(const l3m_model *m) { return m->f.tok.bos; }
int l3m_eos(const l3m_model *m) { return m->f.tok.eos; }
const char *l3m_chatml(const l3m_model *m, int32_t *im_start) { *im_start = m->f.im_start; return m->f.system; }
int l3m_encode(const l3m_model *m, const char *text, int add_bos, int32_t *out, int max) {
    return l3m_vocab_encode(&m->f.tok, text, add_bos, out, max);
}
const char *l3m_decode(const l3m_model *m, int32_t tok, int *len) { return (const char *)l3m_vocab_decode(&m->f.tok, tok, len); }

// Counters since the last read (src/l3m.h:21-29): time per forward pass from the host clock around each
// generate call, less the --cold evictions (engine.c:584); weight bytes streamed per token; the CPU-side
// counters (L2 bytes, L3 misses, DRAM bytes, energy, LLC occupancy) have no GPU meaning here (NAN).
// ns_wait is the analogue of the ranks' barrier wait (engine.c:578-602): on the persistent kernel, the time
// its attention group 0 (on the step's critical chain) waited for the FFN flags and the head's token, per
// token; ns_compute is the rest. The one-graph-per-step path has no such waits (ns_wait NAN).
int l3m_perf_read(l3m_model *m, l3m_perf *out) {
    const double n = m->tokens, spent = m->ns - m->cold_ns, waited = m->wait_ns;
    m->tokens = m->ns = m->cold_ns = m->wait_ns = 0;
    *out = (l3m_perf){.l2_bytes = NAN, .l3_miss = NAN, .dram_bytes = NAN, .energy_j = NAN, .llc_occupancy = NAN};
    if (!(n > 0)) return -1;
    out->tokens = n;
    out->ns_token = spent / n;
    out->ns_wait = m->persist ? waited / n : NAN;
    out->ns_compute = m->persist ? out->ns_token - out->ns_wait : out->ns_token;
    out->bytes_token = m->reference ? 0 : m->weight_bytes;
    return 0;
}

// "0,2,4-7" -> ids; -1 when malformed or longer than max.
int l3m_parse_cpus(const char *list, int *cpus, int max) {
    if (!list || !*list) return -1;
    int count = 0;
    for (const char *s = list;;) {
        char *stop;
        const long lo = strtol(s, &stop, 10);
        if (stop == s || lo < 0) return -1;
        long hi = lo;
        if (*stop == '-') {
            s = stop + 1;
            hi = strtol(s, &stop, 10);
            if (stop == s || hi < lo) return -1;
        }
        if (hi - lo >= (long)max - count) return -1;
        for (long c = lo; c <= hi; ++c) cpus[count++] = (int)c;
        if (*stop == '\0') return count;
        if (*stop != ',' || stop[1] == '\0') return -1;
        s = stop + 1;
    }
}

void l3m_print_hw(FILE *out) {
    if (l3m_dev_init()) { fprintf(out, "no usable HIP device: %s\n", l3m_dev_error() ? l3m_dev_error() : "?"); return; }
    fprintf(out, "gpu 0: %s\n", l3m_dev_name());
}

double l3m_bench_decode_t(l3m_model *m, const int32_t *prompt, int n_prompt, int n_tokens, float temperature, uint64_t seed) {
    if (n_prompt < 1 || n_prompt >= m->dm.ctx) return -1;
    const double t0 = now_ns(), c0 = m->cold_ns_all;
    int done = 0;
    for (int tries = 0; done < n_tokens; tries++) {   // main.c:251: restart when the context is full
        int want = n_tokens - done, room = m->dm.ctx - n_prompt;
        int n = run(m, prompt, n_prompt, want < room ? want : room, temperature, seed + (uint64_t)tries, NULL, NULL);
        if (n < 0 || (n == 0 && (!(temperature > 0) || tries > 64))) return -1;   // a sampled EOS may end a run early
        done += n;
    }
    return (now_ns() - t0 - (m->cold_ns_all - c0)) / done;   // --cold: evictions are not token time
}

double l3m_bench_decode(l3m_model *m, const int32_t *prompt, int n_prompt, int n_tokens) {
    return l3m_bench_decode_t(m, prompt, n_prompt, n_tokens, 0.0f, 0);
}

double l3m_bench_kernel(l3m_model *m, int kind, int layer, int pos, int iters) {
    if (pos < 0 || pos >= m->dm.ctx || l3m_dev_upload(m->dm.pos, &pos, 4)) return -1;
    return l3m_time_step_kernel(&m->dm, m->layers, kind, layer, iters);
}

// Weight bytes one launch of a step kernel streams (rows x k x bytes per weight, the reference's
// bytes_token accounting): kind 0 the attention block, 1 the FFN block, 2 the head.
double l3m_kernel_bytes(const l3m_model *m, int kind, int pos) {
    (void)pos;
    return kind == 0 ? m->attn_bytes : kind == 1 ? m->ffn_bytes : m->head_bytes;
}

double l3m_weight_bytes(const l3m_model *m) { return m->weight_bytes; }

int l3m_decode_persistent(const l3m_model *m) { return m->persist; }

int l3m_prefill_positions(const l3m_model *m) { return m->prefilled; }

int l3m_decode_attention(const l3m_model *m) {
    return l3m_attention_mode(m->dm.kv_lds, m->dm.hd, m->dm.n_heads / m->dm.n_groups, m->dm.kv_win);
}

int l3m_decode_window(const l3m_model *m) { return m->dm.kv_win; }

int l3m_head_dim(const l3m_model *m) { return m->dm.hd; }

int l3m_kv_rows(const l3m_model *m, int layer, int kvh, int pos0, int n, uint16_t *k, uint16_t *v) {
    const l3m_dmodel *d = &m->dm;
    if (layer < 0 || layer >= d->n_layers || kvh < 0 || kvh >= d->n_kv || pos0 < 0 || n < 1 || pos0 + n > d->ctx) return -1;
    const size_t at = (((size_t)layer * d->n_kv + kvh) * d->ctx + pos0) * d->hd, bytes = (size_t)n * d->hd * 2;
    return l3m_dev_download(k, d->kc + at, bytes) || l3m_dev_download(v, d->vc + at, bytes) ? -1 : 0;
}

int l3m_logits_at(const l3m_model *m, int pos, float *out) {
    if (m->logits_pos < 0 || pos > m->logits_pos || pos <= m->logits_pos - NSLOTS || pos < 0) return -1;
    return l3m_dev_download(out, m->dm.logits + (size_t)(pos % NSLOTS) * m->dm.vocab, (size_t)m->dm.vocab * 4);
}

void l3m_decode_work(const l3m_model *m, double *out) {
    for (int i = 0; i < 3; i++) out[i] = m->work[i];
}

// The decode step's geometry: out[0] head groups, out[1] FFN chunks, out[2] query heads per group, out[3]
// rows per chunk (the last chunk takes what is left), out[4] head tiles per head workgroup.
void l3m_step_layout(const l3m_model *m, int *out) {
    const l3m_dmodel *d = &m->dm;
    out[0] = d->n_groups;
    out[1] = d->n_chunks;
    out[2] = d->n_heads / d->n_groups;
    out[3] = m->chunk_rows;
    out[4] = m->persist ? m->head_tpw : d->head_tiles_per_wg;
}

// One matvec of the decode step, on the matrix the step streams and through the form it runs (a parity
// hook; l3m_k_step_mv): which 0 the q/k/v rows of head group `index` in layer `layer`, 1 its Wo columns, 2
// the gate/up rows of FFN chunk `index` (gate row r, up row r), 3 its Wdown columns, 4 the head. x: the
// normalized input (host, k floats: dim, or the group's nq * hd, or the chunk's rows), y: one float per row
// of the matrix (host). 0 on success.
int l3m_step_matvec(const l3m_model *m, int which, int layer, int index, const float *x, float *y) {
    const l3m_dmodel *d = &m->dm;
    if (which < 0 || which > 4 || (which < 4 && (layer < 0 || layer >= d->n_layers))) return -1;
    if (d->gpt2 && (which == 1 || which == 3)) return -1;     // GPT-2 sums Wo and Wdown rows by rows_sum4
    l3m_dmat mat;
    int k = d->dim, form = 0, dtype = d->body_dtype;
    if (which <= 1) {
        l3m_dgroup G;
        if (index < 0 || index >= d->n_groups || l3m_dev_download(&G, m->layers[layer].groups + index, sizeof G)) return -1;
        mat = which ? G.wo : G.qkv;
        if (which) { k = G.nq * d->hd; form = 1; }
    } else if (which <= 3) {
        l3m_dchunk C;
        if (index < 0 || index >= d->n_chunks || l3m_dev_download(&C, m->layers[layer].chunks + index, sizeof C)) return -1;
        mat = which == 3 ? C.down : C.gate_up;
        if (which == 3) { k = C.nf; form = 2; }
    } else {
        mat = d->head;
        form = 3;
        dtype = d->head.dtype;
    }
    float *dx = l3m_dev_alloc((size_t)k * 4), *dy = l3m_dev_alloc((size_t)mat.rows * 4);
    int layout[5];
    l3m_step_layout(m, layout);
    int rc = !dx || !dy || l3m_dev_upload(dx, x, (size_t)k * 4) || l3m_k_step_mv(dtype, form, &mat, dx, k, dy, layout[4], NULL) ||
             l3m_dev_download(y, dy, (size_t)mat.rows * 4) ? -1 : 0;
    l3m_dev_free(dx);
    l3m_dev_free(dy);
    return rc;
}

// The persistent kernel's longest wait, in ticks of the 100 MHz clock (ticks < 0: the default, 1 s). A test
// hook: with 0 every wait that has to spin gives up at once, so a launch ends through the abort path.
void l3m_decode_spin_limit(l3m_model *m, long long ticks) { m->spin_limit = ticks < 0 ? SPIN_LIMIT : (unsigned long long)ticks; }

// l3m_encode on the tokenizer of the file at path, without a device (the host's part of l3m_load): the
// count, or -1 when the file is refused or the ids do not fit max.
int l3m_tokenize(const char *path, const char *text, int add_bos, int32_t *out, int max) {
    l3m_mapped f;
    if (l3m_map_open(&f, path)) return -1;
    const int n = l3m_vocab_encode(&f.tok, text, add_bos, out, max);
    l3m_map_close(&f);
    return n;
}
