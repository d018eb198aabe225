// The boundary between the C host code and the HIP device code: device matrices in lane-tile layout,
// the device-resident model state, and the launchers (all return 0 or -1 and record a sticky error).
#pragma once
#include <stddef.h>
#include <stdint.h>
#include "l3m_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

// l3m_dmat (lane-tile device matrix, layout in host.h) is declared in l3m_hip.h.

typedef struct {
    l3m_dmat     qkv;            // [q rows (dim) | k rows (kv_dim) | v rows (kv_dim)] x dim
    l3m_dmat     wo;             // dim x dim
    l3m_dmat     gate_up;        // tiles interleaved: gate tile j, up tile j, ... (ffn padded to 16) x dim
    l3m_dmat     down;           // dim x ffn
    const float *attn_norm, *ffn_norm;
} l3m_dlayer;

typedef struct {
    int          dim, hd, n_heads, n_kv, kv_dim, ffn, ffn_pad, vocab, ctx, n_layers, nslots;
    float        eps;
    int         *pos;            // [1] position of the step being run
    int32_t     *tokens;         // [ctx + 1]: prompt ids, then each step's argmax at pos + 1
    float       *x, *q, *attn, *h;
    float       *logits;         // [nslots][vocab], slot = pos % nslots
    float       *part_val;       // per-workgroup argmax partials of the head
    int         *part_idx;
    unsigned    *done;           // workgroups finished in the head kernel
    const float *rope;           // [ctx][hd/2][2] cos, sin (host libm, the reference's angles)
    uint16_t    *kc, *vc;        // [layer][n_kv][ctx][hd] bf16
    l3m_dmat     embed, head;    // head may alias embed (tied)
    const float *norm;
} l3m_dmodel;

// ------------------------------------------------------------------ runtime
int         l3m_dev_init(void);                 // 0 when a gfx9 HIP device is usable
const char *l3m_dev_error(void);                // sticky: the first error seen, or NULL
void        l3m_dev_clear_error(void);
const char *l3m_dev_name(void);
void       *l3m_dev_alloc(size_t bytes);        // zeroed; NULL on failure
void        l3m_dev_free(void *p);
int         l3m_dev_upload(void *dst, const void *src, size_t bytes);
int         l3m_dev_download(void *dst, const void *src, size_t bytes);
int         l3m_dev_sync(void);
void       *l3m_dev_stream(void);

// ------------------------------------------------------------------ single kernels
size_t l3m_act_bytes(int dtype, int k);         // prepared activation: q8[kp] + scale[nb] + sum[nb], bf16[kp] or f32[kp]
int    l3m_k_prep(int dtype, const float *x, int k, void *act, void *stream);
int    l3m_k_gemv(const l3m_dmat *m, const void *act, int k, float *y, void *stream);
int    l3m_k_attend(float *out, const float *q, const uint16_t *k, const uint16_t *v, int pos, int hd, int stride, void *stream);
int    l3m_k_rmsnorm(float *y, const float *x, const float *w, int n, float eps, void *stream);
int    l3m_k_rope(float *v, int n_heads, int hd, int pos, const float *table, void *stream);
int    l3m_k_silu_mul(float *h, const float *g, int n, void *stream);
int    l3m_k_argmax(const float *x, int n, int32_t *out, void *stream);

// ------------------------------------------------------------------ decode step
// Enqueue one decode step at the device position: embedding, every layer, and when with_head, the final
// norm, the head, the argmax written to tokens[pos + 1]. Always advances pos.
int l3m_step_enqueue(const l3m_dmodel *m, const l3m_dlayer *layers, int with_head, void *stream);

// Timing (microseconds per launch, hipEvents on the library stream, after one untimed launch).
double l3m_time_gemv(const l3m_dmat *mats, int n_mats, const void *act, int k, float *y, int iters);
// kind: 0 qkv, 1 attention, 2 wo, 3 gate/up, 4 down, 5 head (which then does not advance the position)
double l3m_time_step_kernel(const l3m_dmodel *m, const l3m_dlayer *layers, int kind, int layer, int iters);

// Captured steps: graph 0 without the head (prompt), graph 1 with it.
typedef struct l3m_graphs l3m_graphs;
l3m_graphs *l3m_graphs_build(const l3m_dmodel *m, const l3m_dlayer *layers);
int         l3m_graphs_launch(l3m_graphs *g, int with_head, void *stream);
void        l3m_graphs_free(l3m_graphs *g);

#ifdef __cplusplus
}
#endif
