// TEST AND BENCH INFRASTRUCTURE ONLY (never linked into the product): the reference's own matvec kernels
// timed on this host's cores, the CPU figures beside the GPU matvec numbers. Built by oracle/Makefile
// against _ref/libl3m_ref.so (fpedd/l3m compiled from its sources) and the reference's kernels.h, where
// the reference sources exist; bench.py loads it through ctypes.
//
// The method is the reference's tests/test_kernels.c:151-176 (tiles packed by l3m_pack_tile, x prepared
// by l3m_vec_prepare, the table's gemv looped for at least `seconds`, bytes = tiles x tile bytes), run on
// one core and on every listed core at once with contiguous tile ranges (the engine's row sharding,
// engine.c:88-93), each core looping on its own range.
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include "kernels.h"

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

// The widest table this CPU runs (dispatch.c's order): 2 avx512, 1 avx2, 0 scalar.
static const l3m_kernels *table(void) {
    if (l3m_kernels_usable(&l3m_kernels_avx512)) return &l3m_kernels_avx512;
    if (l3m_kernels_usable(&l3m_kernels_avx2)) return &l3m_kernels_avx2;
    return &l3m_kernels_scalar;
}
int cb_table(void) {
    const l3m_kernels *t = table();
    return t == &l3m_kernels_avx512 ? 2 : t == &l3m_kernels_avx2 ? 1 : 0;
}

typedef struct {
    const l3m_kernels *kt;
    int dtype, k, t0, t1, cpu;
    const uint8_t *tiles;
    size_t tile_bytes;
    const l3m_vec *x;
    float *y;
    atomic_int *go, *stop;
    long passes;
} worker;

static void *run(void *arg) {
    worker *w = arg;
    if (w->cpu >= 0) {
        cpu_set_t set;
        CPU_ZERO(&set);
        CPU_SET(w->cpu, &set);
        pthread_setaffinity_np(pthread_self(), sizeof set, &set);
    }
    while (!atomic_load(w->go)) {}
    const uint8_t *t = w->tiles + (size_t)w->t0 * w->tile_bytes;
    for (w->passes = 0; !atomic_load_explicit(w->stop, memory_order_relaxed); w->passes++)
        w->kt->gemv[w->dtype](w->y, t, w->t1 - w->t0, w->k, w->x);
    return NULL;
}

// GB/s of the table's gemv over an n x k matrix given as file rows (n a multiple of 16), on ncpu cores
// (cpus[i], or unpinned when cpus is NULL), looping for `seconds`. Negative on a setup failure.
double cb_gemv_gbs(int dtype, int n, int k, const uint8_t *rows, const float *x, const int *cpus, int ncpu, double seconds) {
    if (n % L3M_TILE || ncpu < 1 || ncpu > 256) return -1;
    const int ntiles = n / L3M_TILE;
    if (ncpu > ntiles) ncpu = ntiles;
    const size_t tb = l3m_tile_bytes(dtype, k), rb = l3m_row_bytes(dtype, k);
    uint8_t *tiles = aligned_alloc(64, (ntiles * tb + 63) / 64 * 64);
    float *y = calloc((size_t)n + 64, sizeof *y);
    void *scratch = malloc(2 * (size_t)k + 64);
    worker *ws = calloc((size_t)ncpu, sizeof *ws);
    pthread_t *th = calloc((size_t)ncpu, sizeof *th);
    if (!tiles || !y || !scratch || !ws || !th) { free(tiles); free(y); free(scratch); free(ws); free(th); return -1; }
    for (int t = 0; t < ntiles; t++) {
        const void *r[L3M_TILE];
        for (int c = 0; c < L3M_TILE; c++) r[c] = rows + ((size_t)t * L3M_TILE + c) * rb;
        l3m_pack_tile(tiles + (size_t)t * tb, dtype, r, k);
    }
    l3m_vec v;
    l3m_vec_prepare(&v, dtype, x, k, scratch);
    atomic_int go = 0, stop = 0;
    const l3m_kernels *kt = table();
    for (int i = 0; i < ncpu; i++) {
        ws[i] = (worker){kt, dtype, k, (int)((long)ntiles * i / ncpu), (int)((long)ntiles * (i + 1) / ncpu), cpus ? cpus[i] : -1,
                         tiles, tb, &v, y + (size_t)((long)ntiles * i / ncpu) * L3M_TILE, &go, &stop, 0};
        pthread_create(&th[i], NULL, run, &ws[i]);
    }
    const double t0 = now_s();
    atomic_store(&go, 1);
    while (now_s() - t0 < seconds) {
        struct timespec ts = {0, 1000000};
        nanosleep(&ts, NULL);
    }
    atomic_store(&stop, 1);
    double bytes = 0;
    for (int i = 0; i < ncpu; i++) {
        pthread_join(th[i], NULL);
        bytes += (double)ws[i].passes * (double)(ws[i].t1 - ws[i].t0) * (double)tb;
    }
    const double dt = now_s() - t0;
    free(tiles); free(y); free(scratch); free(ws); free(th);
    return bytes / dt * 1e-9;
}
