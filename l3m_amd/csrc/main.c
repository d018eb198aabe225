// The l3m command line on the GPU backend (the reference's src/main.c:26-343): generate, check, bench,
// info and hw, plus gen, which writes the seeded synthetic models the benchmarks use. Prompts are text
// (-p) or token ids (--ids 1,2,3), or the seeded prompt of a synthetic model (--seed-prompt N).
#include <errno.h>
#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include "host.h"

#define MiB (1024.0 * 1024.0)
#define MIN(a, b) ((a) < (b) ? (a) : (b))
enum { MAX_IDS = 4096 };

typedef struct {
    const char *model, *prompt, *ids;
    const char *models[64];
    int n_models, md, seed_prompt;
    int max_new, ctx, ref, force, verbose, cold;
    float temperature;
    uint64_t seed;
} args;

_Noreturn static void usage(int code) {
    fprintf(code ? stderr : stdout,
        "usage: l3m generate|check|bench|info model.l3m [options]\n"
        "       l3m bench a.l3m b.l3m ... [--md]\n"
        "       l3m gen out.l3m --config stories15M|stories42M|stories110M|smollm2 [--dtype D] [--seed S]\n"
        "       l3m hw\n"
        "  -p \"prompt\"   --ids 1,2,3   --seed-prompt N (N ids from the model seed)   -n max_new (256)\n"
        "  -t temperature (0 on this backend)   -s seed   --ctx N   -v   --ref (fp32 reference path)\n");
    exit(code);
}

_Noreturn static void bad_arg(const char *what, const char *v) {
    fprintf(stderr, "l3m: bad %s %s\n", what, v);
    exit(2);
}

static long whole(const char *o, const char *v, long lo) {
    char *end;
    long x = strtol(v, &end, 10);
    if (end == v || *end || x < lo || x > INT_MAX) bad_arg(o, v);
    return x;
}

static args parse(int argc, char **argv, int first) {
    args a = { .max_new = 256, .temperature = 0.0f, .seed = (uint64_t)time(NULL) };
    for (int i = first; i < argc; i++) {
        const char *o = argv[i], *v = i + 1 < argc ? argv[i + 1] : NULL;
        char *end;
        if (o[0] != '-') {
            if (a.n_models == 64) bad_arg("model count, over 64:", o);
            a.models[a.n_models++] = o;
        }
        else if (!strcmp(o, "-p") && v) a.prompt = argv[++i];
        else if (!strcmp(o, "--ids") && v) a.ids = argv[++i];
        else if (!strcmp(o, "--seed-prompt") && v) a.seed_prompt = (int)whole(o, argv[++i], 1);
        else if (!strcmp(o, "-n") && v) a.max_new = (int)whole(o, argv[++i], 0);
        else if (!strcmp(o, "--ctx") && v) a.ctx = (int)whole(o, argv[++i], 2);
        else if (!strcmp(o, "--cores") && v) i++;                       // accepted, one GPU runs the model
        else if (!strcmp(o, "-t") && v) {
            a.temperature = strtof(argv[++i], &end);
            if (end == argv[i] || *end || !(a.temperature >= 0) || isinf(a.temperature)) bad_arg(o, argv[i]);
        }
        else if (!strcmp(o, "-s") && v) {
            a.seed = strtoull(argv[++i], &end, 10);
            if (end == argv[i] || *end || argv[i][0] == '-') bad_arg(o, argv[i]);
        }
        else if (!strcmp(o, "--ref")) a.ref = 1;
        else if (!strcmp(o, "--force")) a.force = 1;
        else if (!strcmp(o, "--cold")) a.cold = 1;
        else if (!strcmp(o, "--md")) a.md = 1;
        else if (!strcmp(o, "-v")) a.verbose = 1;
        else { fprintf(stderr, "l3m: unknown option %s%s\n", o, v ? "" : " (or missing value)"); usage(2); }
    }
    if (!a.n_models) usage(2);
    a.model = a.models[0];
    if (a.n_models > 1 && strcmp(argv[1], "bench")) { fprintf(stderr, "l3m: only bench takes several files\n"); exit(2); }
    return a;
}

static l3m_model *load(const args *a, int ref) {
    l3m_opts o = { .reference = ref, .force = a->force, .verbose = a->verbose, .ctx = a->ctx, .cold = a->cold };
    l3m_model *m = l3m_load(a->model, &o);
    if (!m) exit(1);
    return m;
}

// The prompt ids: --ids, --seed-prompt (from the file's name-independent seed given by -s), or -p text.
static int prompt_ids(l3m_model *m, const args *a, int32_t *ids, int max, const char *fallback) {
    int n = 0, fit = MIN(l3m_ctx(m), max);
    if (a->ids) {
        n = l3m_parse_cpus(a->ids, ids, max);                 // same "1,2-4" list syntax
        if (n < 1) { fprintf(stderr, "l3m: bad --ids %s\n", a->ids); return -1; }
    } else if (a->seed_prompt) {
        n = MIN(a->seed_prompt, max);
        l3m_gen_prompt(a->seed, l3m_vocab(m), n, ids);
    } else {
        n = l3m_encode(m, a->prompt ? a->prompt : fallback, 1, ids, max);
    }
    if (n >= 1 && n < fit) return n;
    if (n < 0) fprintf(stderr, "l3m: the prompt is over %d tokens\n", max);
    else fprintf(stderr, "l3m: the prompt is %d tokens, the limit is %d (--ctx %d)\n", n, fit - 1, l3m_ctx(m));
    return -1;
}

typedef struct { l3m_model *m; int32_t *toks; int n; int print; } sink;
static int on_token(int32_t tok, void *user) {
    sink *s = user;
    if (s->toks) s->toks[s->n] = tok;
    s->n++;
    if (s->print) {
        int len;
        const char *b = l3m_decode(s->m, tok, &len);
        if (len) fwrite(b, 1, (size_t)len, stdout);
        else printf("<%d>", tok);
        fflush(stdout);
    }
    return 1;
}

static void perf_line(l3m_model *m, FILE *out) {
    l3m_perf p;
    if (l3m_perf_read(m, &p)) return;
    fprintf(out, "%s\n%.0f tok/s  %.1f us/tok", l3m_describe(m), 1e9 / p.ns_token, p.ns_token / 1e3);
    if (p.bytes_token > 0) fprintf(out, "\nweights: %.1f MiB per token at %.0f GB/s", p.bytes_token / MiB, p.bytes_token / p.ns_token);
    fprintf(out, "\n");
}

static int cmd_generate(const args *a) {
    l3m_model *m = load(a, a->ref);
    int32_t ids[MAX_IDS];
    int n = prompt_ids(m, a, ids, MAX_IDS, "");
    if (n < 0) { l3m_free(m); return 1; }
    if (a->prompt && !a->ids && !a->seed_prompt) fputs(a->prompt, stdout);
    sink s = { m, NULL, 0, 1 };
    int made = l3m_generate(m, ids, n, a->max_new, a->temperature, a->seed, on_token, &s);
    printf("\n");
    fprintf(stderr, "\n[%d tokens] ", made);
    perf_line(m, stderr);
    l3m_free(m);
    return made < 0;
}

static void cell(double v, int prec) { if (isnan(v)) printf(" - |"); else printf(" %.*f |", prec, v); }

// As main.c:233-263: warm up with 16 tokens, then generate from BOS (or id 0) until -n tokens, restarting
// after each end of text or full context.
static int cmd_bench(const args *a) {
    if (a->max_new < 1) { fprintf(stderr, "l3m: bench needs -n 1 or more\n"); return 2; }
    int md = a->md || a->n_models > 1, failed = 0;
    if (md) {
        printf("| model | tok/s | us/tok | GB/s |\n");
        printf("|---|---:|---:|---:|\n");
    }
    for (int i = 0; i < a->n_models; i++) {
        args one = *a;
        one.model = a->models[i];
        l3m_opts o = { .reference = a->ref, .ctx = a->ctx };
        l3m_model *m = l3m_load(one.model, &o);
        if (!m) { if (md) printf("| %s | load failed |\n", one.model); failed = 1; continue; }
        int32_t bos = l3m_bos(m) < 0 ? 0 : l3m_bos(m);
        int32_t *out = malloc(sizeof(int32_t) * (size_t)(a->max_new + 16));
        sink s = { m, out, 0, 0 };
        l3m_perf p;
        l3m_generate(m, &bos, 1, 16, 0.f, 0, on_token, &s);
        l3m_perf_read(m, &p);
        s.n = 0;
        while (s.n < a->max_new && l3m_generate(m, &bos, 1, a->max_new - s.n, 0.f, 0, on_token, &s) > 0) {}
        if (!md) perf_line(m, stdout);
        else if (l3m_perf_read(m, &p)) printf("| %s | no tokens |\n", l3m_describe(m));
        else {
            printf("| %s | %.0f | %.1f |", l3m_describe(m), 1e9 / p.ns_token, p.ns_token / 1e3);
            cell(p.bytes_token > 0 ? p.bytes_token / p.ns_token : NAN, 0);
            printf("\n");
        }
        free(out);
        l3m_free(m);
    }
    return failed;
}

// KL(reference || fast) in nats (main.c:266-272).
static double kl(const float *lr, const float *lf, int n) {
    double mr = lr[0], mf = lf[0], zr = 0, zf = 0, sum = 0;
    for (int i = 1; i < n; i++) { if (lr[i] > mr) mr = lr[i]; if (lf[i] > mf) mf = lf[i]; }
    for (int i = 0; i < n; i++) { zr += exp(lr[i] - mr); zf += exp(lf[i] - mf); }
    for (int i = 0; i < n; i++) sum += exp(lr[i] - mr) / zr * ((lr[i] - mr - log(zr)) - (lf[i] - mf - log(zf)));
    return sum;
}

// Quantized path vs the fp32 reference path, both on the GPU: PASS iff argmax agrees and KL < 0.01 nats
// (main.c:274-304). Greedy agreement over 32 tokens is informational.
static int cmd_check(const args *a) {
    l3m_model *ref = load(a, 1), *fast = load(a, 0);
    int32_t ids[MAX_IDS], tr[64], tf[64];
    int n = prompt_ids(ref, a, ids, MAX_IDS, "Once upon a time"), vocab = l3m_vocab(ref);
    if (n < 0) { l3m_free(ref); l3m_free(fast); return 1; }
    l3m_generate(ref, ids, n, 0, 0.f, 0, NULL, NULL);
    l3m_generate(fast, ids, n, 0, 0.f, 0, NULL, NULL);
    float *lr = malloc((size_t)vocab * 4), *lf = malloc((size_t)vocab * 4);
    memcpy(lr, l3m_logits(ref), (size_t)vocab * 4);
    memcpy(lf, l3m_logits(fast), (size_t)vocab * 4);
    double maxerr = 0, d = kl(lr, lf, vocab);
    int ar = 0, af = 0;
    for (int i = 0; i < vocab; i++) {
        if (fabs(lr[i] - lf[i]) > maxerr) maxerr = fabs(lr[i] - lf[i]);
        if (lr[i] > lr[ar]) ar = i;
        if (lf[i] > lf[af]) af = i;
    }
    int ok = ar == af && d < 0.01;
    printf("logits after prompt: max-abs error %.3g, KL %.2g nats, argmax %s (%d vs %d)\n", maxerr, d, ar == af ? "agree" : "DIFFER", ar, af);
    sink sr = { ref, tr, 0, 0 }, sf = { fast, tf, 0, 0 };
    int nr = l3m_generate(ref, ids, n, 32, 0.f, 0, on_token, &sr);
    int nf = l3m_generate(fast, ids, n, 32, 0.f, 0, on_token, &sf);
    int same = 0;
    while (same < nr && same < nf && tr[same] == tf[same]) same++;
    printf("greedy tokens: %d of %d agree\n", same, nr);
    printf("%s\n", ok ? "PASS" : "FAIL");
    free(lr); free(lf);
    l3m_free(ref); l3m_free(fast);
    return !ok;
}

static int cmd_info(const args *a) {
    l3m_mapped f;
    if (l3m_map_open(&f, a->model)) return 1;
    const l3m_header *h = f.h;
    printf("%s  arch %.16s  flags 0x%x\n", a->model, h->arch, h->flags);
    printf("dim %u  layers %u  heads %u  kv_heads %u  ffn %u  vocab %u  ctx %u  rope_theta %g  eps %g\n",
           h->dim, h->n_layers, h->n_heads, h->n_kv_heads, h->ffn_dim, h->vocab, h->ctx, h->rope_theta, h->norm_eps);
    double total = 0;
    for (uint32_t i = 0; i < h->n_tensors; i++) {
        const l3m_tensor *t = &f.toc[i];
        char shape[48];
        snprintf(shape, sizeof shape, t->ndim > 1 ? "%llu x %llu" : "%llu", (unsigned long long)t->shape[0], (unsigned long long)t->shape[1]);
        printf("  %-24.64s %-6s %-14s %10llu bytes\n", t->name, l3m_dtype_name((int)t->dtype), shape, (unsigned long long)t->nbytes);
        total += (double)t->nbytes;
    }
    printf("%u tensors, %.1f MiB\n", h->n_tensors, total / MiB);
    l3m_map_close(&f);
    return 0;
}

// The benchmark configurations (2, 3, 4): random-init N(0, 0.02), norms 1, tied head
// of the body dtype, no BOS/EOS.
static int cmd_gen(int argc, char **argv) {
    const char *out = NULL, *cfg = NULL, *dt = NULL;
    uint64_t seed = 1;
    for (int i = 2; i < argc; i++) {
        if (!strcmp(argv[i], "--config") && i + 1 < argc) cfg = argv[++i];
        else if (!strcmp(argv[i], "--dtype") && i + 1 < argc) dt = argv[++i];
        else if (!strcmp(argv[i], "--seed") && i + 1 < argc) seed = strtoull(argv[++i], NULL, 10);
        else if (argv[i][0] != '-') out = argv[i];
        else usage(2);
    }
    if (!out || !cfg) usage(2);
    l3m_gen_spec s = { .arch = "llama", .rope_theta = 10000.0f, .norm_eps = 1e-5f, .tied = 1, .seed = seed, .std = 0.02f, .bos = -1, .eos = -1 };
    int dtype;
    if (!strcmp(cfg, "stories15M")) { s.dim = 288; s.n_layers = 6; s.n_heads = 6; s.n_kv_heads = 6; s.ffn_dim = 768; s.vocab = 32000; s.ctx = 256; dtype = L3M_BF16; }
    else if (!strcmp(cfg, "stories42M")) { s.dim = 512; s.n_layers = 8; s.n_heads = 8; s.n_kv_heads = 8; s.ffn_dim = 1376; s.vocab = 32000; s.ctx = 1024; dtype = L3M_Q8_0; }
    else if (!strcmp(cfg, "stories110M")) { s.dim = 768; s.n_layers = 12; s.n_heads = 12; s.n_kv_heads = 12; s.ffn_dim = 2048; s.vocab = 32000; s.ctx = 128; dtype = L3M_Q4_0; }
    else if (!strcmp(cfg, "smollm2")) { s.dim = 576; s.n_layers = 30; s.n_heads = 9; s.n_kv_heads = 3; s.ffn_dim = 1536; s.vocab = 49152; s.ctx = 256; dtype = L3M_Q8_0; }
    else { fprintf(stderr, "l3m: unknown --config %s\n", cfg); return 2; }
    if (dt) {
        dtype = -1;
        for (int d = 0; d < L3M_NDTYPES; d++) if (!strcmp(dt, l3m_dtype_name(d))) dtype = d;
        if (dtype < 0) { fprintf(stderr, "l3m: unknown --dtype %s\n", dt); return 2; }
    }
    s.dtype = s.head_dtype = dtype;
    return l3m_gen_write(&s, out) ? 1 : 0;
}

int main(int argc, char **argv) {
    for (int i = 1; i < argc; i++) if (!strcmp(argv[i], "-h") || !strcmp(argv[i], "--help")) usage(0);
    if (argc >= 2 && !strcmp(argv[1], "hw")) { l3m_print_hw(stdout); return 0; }
    if (argc >= 2 && !strcmp(argv[1], "gen")) return cmd_gen(argc, argv);
    if (argc < 2) usage(2);
    args a = parse(argc, argv, 2);
    const char *cmd = argv[1];
    if (!strcmp(cmd, "generate")) return cmd_generate(&a);
    if (!strcmp(cmd, "bench")) return cmd_bench(&a);
    if (!strcmp(cmd, "check")) return cmd_check(&a);
    if (!strcmp(cmd, "info")) return cmd_info(&a);
    fprintf(stderr, "l3m: unknown command %s\n", cmd);
    usage(2);
}
