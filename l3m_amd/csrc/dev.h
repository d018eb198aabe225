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

// One head group of a layer's attention block: nq consecutive query heads (nq * hd a multiple of 32 for
// quantized weights, so the Wo slice is whole blocks) and the kv heads they read.
typedef struct {
    l3m_dmat qkv;                // rows [q of the nq heads | k of the nkv kv heads | v of them] x dim
    l3m_dmat wo;                 // dim rows x the group's nq * hd Wo columns
    int      q0, nq, kv0, nkv;   // first query head, count; first kv head, count
    unsigned write_kv;           // bit i: this group writes kv head kv0 + i into the cache
    int      att_wl;             // log2 of the most wavefronts one query head takes in the attention
    unsigned lds[10];            // LDS byte offsets of the attention block's regions (l3m_group_layout)
    const float *bqkv;           // GPT-2 variant: the biases of the qkv rows, in their order; else NULL
} l3m_dgroup;

// One chunk of a layer's FFN block: ffn rows [f0, f0 + nf), nf a multiple of 32.
typedef struct {
    l3m_dmat gate_up;            // 2 * nf rows: gate row r, up row r, ... x dim (GPT-2: the up rows only)
    l3m_dmat down;               // dim rows x the chunk's nf Wdown columns
    int      f0, nf;
    unsigned lds[5];             // LDS byte offsets of the FFN block's regions (l3m_chunk_layout)
    int      pad_;
    const float *bup;            // GPT-2 variant: b_up of rows f0.. (gate_up then holds the up rows only)
} l3m_dchunk;

typedef struct {
    const l3m_dgroup *groups;    // device arrays [n_groups], [n_chunks]
    const l3m_dchunk *chunks;
    const float      *attn_norm, *ffn_norm;
    const float      *attn_norm_b, *ffn_norm_b, *bo, *bdown;   // GPT-2 variant; else NULL
} l3m_dlayer;

typedef struct {
    int          dim, hd, n_heads, n_kv, kv_dim, ffn, vocab, ctx, n_layers, nslots;
    int          n_groups, n_chunks, head_grid, head_tiles_per_wg, body_dtype;
    int          kv_lds;         // attention copies the K, V rows of its kv heads into LDS (a window exists)
    int          kv_win;         // positions the LDS window holds (ctx, or the multiple of 32 that fits);
                                 // steps at pos >= kv_win read K and V from the cache
    float        eps;
    float        att_scale;      // 1 / sqrt(hd)
    int          hpk;            // query heads per kv head
    int          pro_groups[2], pro_per[2];   // prologue thread groups and parts per group: [0] over the
                                              // n_chunks FFN partials, [1] over the n_groups attention ones
    unsigned     lds_a, lds_b, lds_h;   // dynamic LDS bytes of the three step kernels
    int         *pos;            // [1] position of the step being run
    int32_t     *tokens;         // [ctx + 1]: prompt ids, then each step's argmax at pos + 1
    float       *xa, *xb;        // residual stream entering the attention block / the FFN block
    float       *po;             // [n_groups][dim] attention-block partials (Wo column slices)
    float       *pd;             // [n_chunks][dim] FFN partials (Wdown column slices)
    float       *logits;         // [nslots][vocab], slot = pos % nslots
    float       *part_val;       // [head_grid] argmax partials
    int         *part_idx;
    unsigned    *done;           // head workgroups finished this step
    const float *rope;           // [ctx][hd/2][2] cos, sin (host libm, the reference's angles)
    uint16_t    *kc, *vc;        // [layer][n_kv][ctx][hd] bf16
    l3m_dmat     embed, head;    // head may alias embed (tied)
    const float *norm;
    struct l3m_dsample *samp;    // temperature sampling: the generate call's temperature and random state
    const float *norm_b;         // GPT-2 variant (gpt2 != 0): the final LayerNorm's bias,
    const float *pos_embed;      // the learned position rows [ctx][dim]
    int          gpt2, pad_g2;
} l3m_dmodel;

// One launch of the persistent decode kernel: steps at positions pos0 .. pos0 + nsteps - 1; logits (and
// the argmax token at pos + 1) for positions >= head_from. The body runs on the workgroups of XCD
// body_xcc (at least n_groups + n_chunks of the grid land there); n_head workgroups take head_tpw tiles each.
typedef struct {
    int                pos0, nsteps, head_from;
    int                head_tpw, n_head, body_xcc;
    unsigned          *sync;           // L3M_SYNC_WORDS words: flags, tickets, argmax keys; zero at launch
    unsigned long long spin_limit;     // longest wait, in ticks of the 100 MHz clock
    float              temp;           // > 0: tokens are sampled at this temperature (samp holds the state)
    unsigned           pad;
} l3m_run;
#define L3M_MAX_HEAD_WGS 256                         // the key area holds this many keys, whatever n_head is
// Flag words, one 64-bit key per head workgroup, one 64-bit slice total per head workgroup (sampling),
// then the run's output span: the abort word, the wait ticks and the run's tokens, laid out as the host's
// l3m_chunk_out so that one copy brings all of it back.
#define L3M_SYNC_OUT (256 + 4 * L3M_MAX_HEAD_WGS)
#define L3M_SYNC_WORDS (L3M_SYNC_OUT + 256)
// Device-resident sampling state, set by the host at the start of each generate call. Every workgroup
// that takes part in sampling keeps its own copy of the xorshift64* state (engine.c:98-101) and advances
// it once per sampled token, so all copies stay equal: rng[h] for head workgroup h of the persistent
// kernel, rng[0] for the graph path's last head workgroup.
typedef struct l3m_dsample {
    float              temp;         // > 0: sample at this temperature; otherwise greedy
    unsigned           pad;
    unsigned long long rng[L3M_MAX_HEAD_WGS];
} l3m_dsample;
#define L3M_SYNC_ABORT L3M_SYNC_OUT                  // the word a timed-out wait sets
#define L3M_SYNC_WAIT (L3M_SYNC_OUT + 2)             // 64-bit: 100 MHz ticks attention group 0 waited for its inputs this launch
#define L3M_SYNC_TOK (L3M_SYNC_OUT + 4)              // the run's tokens, from its first position with a token (at most 128)

// ------------------------------------------------------------------ runtime
int         l3m_dev_init(void);                 // 0 when a gfx9 HIP device is usable
void        l3m_dev_shutdown(void);             // destroys the library's stream and events (host calls it before exit)
const char *l3m_dev_error(void);                // sticky: the first error seen, or NULL
void        l3m_dev_clear_error(void);
const char *l3m_dev_name(void);
void       *l3m_dev_alloc(size_t bytes);        // zeroed; NULL on failure
void        l3m_dev_free(void *p);
int         l3m_dev_upload_async(void *dst, const void *src_pinned, size_t bytes);   // queued, not waited for
int         l3m_dev_zero_async(void *dst, size_t bytes);
void       *l3m_dev_host_alloc(size_t bytes);   // pinned host memory
void        l3m_dev_host_free(void *p);
int         l3m_dev_upload(void *dst, const void *src, size_t bytes);
int         l3m_dev_download(void *dst, const void *src, size_t bytes);
int         l3m_dev_sync(void);
void       *l3m_dev_stream(void);

// ------------------------------------------------------------------ single kernels
size_t l3m_act_bytes(int dtype, int k);         // prepared activation: per 32-block values (q8_0 32 B, q4_0 nibble planes 32 B, mxfp4 f16 pairs 64 B) + scale[nb] + sum[nb] (mxfp4: + fp8 parts h, l 64 B per block), bf16[kp] or f32[kp]
int    l3m_k_prep(int dtype, const float *x, int k, void *act, void *stream);
int    l3m_k_gemv(const l3m_dmat *m, const void *act, int k, float *y, void *stream);
int    l3m_k_attend(float *out, const float *q, const uint16_t *k, const uint16_t *v, int pos, int hd, int stride, void *stream);
int    l3m_k_rmsnorm(float *y, const float *x, const float *w, int n, float eps, void *stream);
int    l3m_k_rope(float *v, int n_heads, int hd, int pos, const float *table, void *stream);
int    l3m_k_silu_mul(float *h, const float *g, int n, void *stream);
int    l3m_k_argmax(const float *x, int n, int32_t *out, void *stream);

// ------------------------------------------------------------------ decode step
// Enqueue one decode step at the device position: per layer the attention block (one workgroup per head
// group) and the FFN block (one per chunk); with_head adds the final norm, the head and the argmax written
// to tokens[pos + 1]. Always advances pos. LDS sizes in m must come from l3m_step_lds.
unsigned l3m_lds_attn(int dtype, int dim, int ctx, int hd, const l3m_dgroup *g, int kv_lds);
// Fill g->lds (region offsets, the same with or without the K/V window, which comes last) and g->att_wl;
// fill c->lds; fill m->pro_groups / pro_per / att_scale / hpk from the model's shape.
void     l3m_group_layout(int dtype, int dim, int ctx, int hd, l3m_dgroup *g);
void     l3m_chunk_layout(int dtype, int dim, l3m_dchunk *c);
void     l3m_model_layout(l3m_dmodel *m);
unsigned l3m_dev_lds_max(void);       // dynamic LDS one workgroup may use on this device
unsigned l3m_lds_ffn(int dtype, int dim, const l3m_dchunk *c);
unsigned l3m_lds_head(int dtype, int dim, int nb, int tiles_per_wg);
int      l3m_step_slots(int dtype, int which);   // weight slots per lane (matrix A / B of a step kernel), 64 pairs each
int      l3m_step_a_dtype(int dtype);            // storage dtype of a step kernel's matrix A for a body of dtype
int l3m_step_enqueue(const l3m_dmodel *m, const l3m_dlayer *layers, int with_head, void *stream);

// Batched prompt prefill: the full matrices of each layer as q8_0 lane-tile planes (q4_0 widened), and
// the activation buffers of up to ctx tokens.
typedef struct {
    l3m_dmat     qkv;            // (n_heads + 2 n_kv) hd rows (q, then k, then v) x dim
    l3m_dmat     wo;             // dim x n_heads hd
    l3m_dmat     gu;             // 2 ffn rows (gate, then up) x dim
    l3m_dmat     down;           // dim x ffn
    const float *attn_norm, *ffn_norm;
} l3m_pflayer;
typedef struct {
    float   *x;                  // [ctx][dim] residual stream
    uint8_t *act;                // [ctx][astride] int8 prep of each token's matrix input
    float   *qkv;                // [ctx][(n_heads + 2 n_kv) hd]
    float   *att;                // [ctx][n_heads hd]
    float   *gu;                 // [ctx][2 ffn]
    int      astride;
} l3m_pfbuf;
// K/V rows of positions 0..P-1 of every layer from the token ids on the device (m->tokens); the last
// layer's FFN is skipped (nothing reads it). -1 on a launch error.
int l3m_prefill(const l3m_dmodel *m, const l3m_pflayer *layers, const l3m_pfbuf *b, int P, void *stream);
// 1 when l3m_prefill takes a model of these sizes (nqd = n_heads * hd); the loader enables prefill only then.
int l3m_prefill_fits(int dim, int ffn, int nqd, int hd);
// The prefill of P positions as one captured graph per P (the launches' grids and arguments depend on P
// only; every buffer is the model's own), kept for the PF_GRAPHS most recently used lengths: a length seen
// before replays its graph, a new one is captured and instantiated first. -1 on a device error.
typedef struct l3m_pfgraphs l3m_pfgraphs;
l3m_pfgraphs *l3m_pfgraphs_new(void);
int           l3m_prefill_graph(l3m_pfgraphs *g, const l3m_dmodel *m, const l3m_pflayer *layers, const l3m_pfbuf *b, int P);
void          l3m_pfgraphs_free(l3m_pfgraphs *g);

// The persistent decode kernel (one cooperative launch for R->nsteps steps; layers_dev in device memory).
int l3m_dev_cus(void);
// The XCD each block of a cooperative grid of `grid` 1024-thread workgroups with lds bytes lands on
// (xcc[grid]); 0, or -1 on a device error.
int l3m_decode_placement(int grid, unsigned lds, int *xcc);
int l3m_decode_pair(int dtype, int head_dtype, int gpt2);    // 1 if the kernel is built for this (body, head, variant)
// hd: the model's head dimension (the kernel built for it as a constant when there is one, else the general one)
int l3m_decode_fits(int dtype, int head_dtype, int gpt2, int hd, int grid, unsigned lds);   // 1 if grid workgroups with lds bytes can all be resident
// m_dev, layers_dev, r_dev: device-memory copies (the kernel reads its parameters from there)
// slot (0 or 1): which of the two launches that may be in flight at once this is (its timing events).
int l3m_decode_launch(int dtype, int head_dtype, int gpt2, int hd, const l3m_dmodel *m_dev, const l3m_dlayer *layers_dev, const l3m_run *r_dev,
                      int grid, unsigned lds, void *stream, int slot);
// Adds slot's finished launch to l3m_decode_timer's total (after its stream work has been waited for).
int l3m_decode_timer_collect(int slot);
// Stream-ordered transfers and events on the library stream, for work kept in flight: a copy into pinned
// host memory without a wait; events (no timing) to wait for a point of the stream.
int   l3m_dev_download_async(void *dst_pinned, const void *src, size_t bytes);
void *l3m_dev_event_new(void);
void  l3m_dev_event_free(void *e);
int   l3m_dev_event_record(void *e);
int   l3m_dev_event_wait(void *e);

// Timing (microseconds per launch, hipEvents on the library stream, after one untimed launch).
double l3m_time_gemv(const l3m_dmat *mats, int n_mats, const void *act, int k, float *y, int iters);
// kind: 0 attention block, 1 FFN block, 2 head (which then does not advance the position)
double l3m_time_step_kernel(const l3m_dmodel *m, const l3m_dlayer *layers, int kind, int layer, int iters);

// Captured steps: graph 0 without the head (prompt), graph 1 with it.
typedef struct l3m_graphs l3m_graphs;
l3m_graphs *l3m_graphs_build(const l3m_dmodel *m, const l3m_dlayer *layers);
int         l3m_graphs_launch(l3m_graphs *g, int with_head, void *stream);
void        l3m_graphs_free(l3m_graphs *g);

#ifdef __cplusplus
}
#endif
