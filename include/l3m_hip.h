// l3m-mi355x: the C ABI of the MI355X (gfx950) backend for l3m's batch-1 decode hot path.
//
// Three layers of entry points, all extern "C" with plain pointers and sizes:
//  1. the model API, with the reference's names, types and contracts (src/l3m.h:10-58), so a caller of
//     libl3m.so (the CLI, python/l3m/__init__.py:31-50 via L3M_LIB) runs on the GPU unchanged;
//  2. the kernel table (src/kernels.h:24-46): l3m_kernels_hip, a drop-in next to the scalar/avx2/avx512
//     tables, taking the reference's host-side tile layout and prepared vector;
//  3. device-level entry points on device pointers (the kernels the engine fuses), for tests and benches.
#pragma once
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

// ============================================================================== 1. model API (l3m.h)

typedef struct l3m_model l3m_model;

// Replaces l3m_opts (src/l3m.h:10-19). cpus/n_cpus are accepted and ignored (one GPU runs the model);
// reference = 1 runs the same engine with every matrix widened to f32 and f32 activations (ref.c's math).
typedef struct {
    const int *cpus;
    int        n_cpus;
    int        ctx;        // KV cache length, 0 = min(model context, 512) (engine.c:22, 435)
    int        reference;
    int        force;
    int        verbose;
    int        cold;       // 1 = evict L2 and the Infinity Cache before each forward pass, one pass per launch;
                           // the eviction is not token time (engine.c:330-338, 584)
} l3m_opts;

// Replaces l3m_perf (src/l3m.h:21-29); counters the GPU path cannot read are NAN.
typedef struct {
    double tokens, ns_token, ns_compute, ns_wait, bytes_token, l2_bytes;
    double l3_miss, dram_bytes, energy_j, llc_occupancy;
} l3m_perf;

l3m_model   *l3m_load(const char *path, const l3m_opts *opts);                         // src/l3m.h:32, engine.c:425
void         l3m_free(l3m_model *m);                                                    // src/l3m.h:33, engine.c:533
int          l3m_generate(l3m_model *m, const int32_t *prompt, int n_prompt, int max_new, // src/l3m.h:40, engine.c:549
                          float temperature, uint64_t seed, int (*on_token)(int32_t tok, void *user), void *user);
const float *l3m_logits(const l3m_model *m);                                            // src/l3m.h:42, engine.c:563
int          l3m_vocab(const l3m_model *m);                                             // src/l3m.h:43
int          l3m_ctx(const l3m_model *m);                                               // src/l3m.h:44
const char  *l3m_describe(const l3m_model *m);                                          // src/l3m.h:45, engine.c:527
int          l3m_encode(const l3m_model *m, const char *text, int add_bos, int32_t *out, int max);  // src/l3m.h:48
const char  *l3m_decode(const l3m_model *m, int32_t tok, int *len);                     // src/l3m.h:49
int          l3m_bos(const l3m_model *m);                                               // src/l3m.h:50
int          l3m_eos(const l3m_model *m);                                               // src/l3m.h:51
const char  *l3m_chatml(const l3m_model *m, int32_t *im_start);                         // src/l3m.h:53
int          l3m_perf_read(l3m_model *m, l3m_perf *out);                                // src/l3m.h:55, engine.c:578
int          l3m_parse_cpus(const char *list, int *cpus, int max);                      // src/l3m.h:57
void         l3m_print_hw(FILE *out);                                                   // src/l3m.h:58

// ============================================================================ 2. kernel table (kernels.h)

enum { L3M_HIP_F32, L3M_HIP_BF16, L3M_HIP_Q8_0, L3M_HIP_Q4_0, L3M_HIP_MXFP4, L3M_HIP_NDTYPES };

typedef struct {                 // src/kernels.h:24-30
    const float    *f32;
    const uint16_t *bf16;
    const int8_t   *q8;
    const float    *scale;
    const int32_t  *sum;
} l3m_vec;

typedef void (*l3m_gemv_fn)(float *y, const void *tiles, int ntiles, int k, const l3m_vec *x);   // src/kernels.h:33

typedef struct {                 // src/kernels.h:35-40
    const char *name;
    l3m_gemv_fn gemv[L3M_HIP_NDTYPES];
    void (*attend)(float *out, const float *q, const uint16_t *k, const uint16_t *v, int pos, int head_dim, int stride);
} l3m_kernels;

extern const l3m_kernels l3m_kernels_hip;          // name "hip"; joins the tables of src/kernels.h:42
// 1 when a gfx950 GPU is usable from this process, else 0 (the reason in l3m_dev_error). The reference's
// dispatcher asks it before it selects l3m_kernels_hip (dispatch.c:23-36 with two added lines: in
// l3m_kernels_usable, `if (k == &l3m_kernels_hip) return l3m_hip_kernels_usable();`; in l3m_kernels_pick,
// `if (want && !strcmp(want, "hip") && l3m_hip_kernels_usable()) return &l3m_kernels_hip;`), and otherwise
// falls back to its own CPU table with its own message. This library defines no l3m_kernels_pick or
// l3m_kernels_usable of its own, so it never shadows the dispatcher's.
int                l3m_hip_kernels_usable(void);
const char        *l3m_hip_last_error(void);                   // the table's sticky error (its functions return void)
// No counterpart in the reference: l3m_kernels_hip.attend for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments
// (host pointers), same kernel, same result; it stages q, the K and V rows and the output through one
// fixed 4 MiB device array instead of buffers grown on demand: q and the output take 4 head_dim bytes
// each and K and V (pos * stride + head_dim) * 2 bytes each, every part rounded up to 256 bytes, so it
// refuses (-1, the reason and the bound on stderr) a call whose K (and V) part exceeds
// (4 MiB - 2 up256(4 head_dim)) / 2 bytes (2 MiB less 1 KiB at head_dim 256). Calls are serialized by a
// lock (two overlapping on one GPU would race on the array). 0 on success.
int l3m_hip_attend_noalloc(float *out, const float *q, const uint16_t *k, const uint16_t *v, int pos, int head_dim, int stride);

// ============================================================== 3. device-level (pointers are device memory)

typedef struct {
    const uint8_t *q, *s;        // lane-tile quant and scale planes
    int rows, tiles, nb, dtype;
} l3m_dmat;

int         l3m_dev_init(void);
void        l3m_dev_shutdown(void);   // the library's stream and events destroyed; later calls fail cleanly
const char *l3m_dev_error(void);
void        l3m_dev_clear_error(void);
const char *l3m_dev_name(void);
void       *l3m_dev_alloc(size_t bytes);
void        l3m_dev_free(void *p);
int         l3m_dev_upload(void *dst, const void *src, size_t bytes);
int         l3m_dev_download(void *dst, const void *src, size_t bytes);
int         l3m_dev_sync(void);
int         l3m_dev_copy(void *dst, const void *src, size_t bytes, void *stream);   // plain copy kernel (counter calibration)
void       *l3m_dev_stream(void);

// Lane-tile layout sizes and host-side packing (the GPU analogue of l3m_tile_bytes / l3m_pack_tile,
// src/kernels.h:49-50, pack.c:21-99).
int    l3m_lt_qbytes(int dtype);
int    l3m_lt_sbytes(int dtype);
size_t l3m_lt_quant_size(int dtype, int rows, int k);
size_t l3m_lt_scale_size(int dtype, int rows, int k);
void   l3m_lt_pack_rows(int dtype, int rows, int k, const void *const *rows_src, uint8_t *quant, uint8_t *scale);
void   l3m_lt_pack_ltiles(int dtype, int ntiles, int k, const void *tiles, uint8_t *quant, uint8_t *scale);

size_t l3m_act_bytes(int dtype, int k);
int    l3m_k_prep(int dtype, const float *x, int k, void *act, void *stream);             // l3m_vec_prepare, pack.c:101
int    l3m_k_gemv(const l3m_dmat *m, const void *act, int k, float *y, void *stream);    // gemv[dtype], kernels_scalar.c
int    l3m_k_attend(float *out, const float *q, const uint16_t *k, const uint16_t *v,    // l3m_attend, ops.c:58
                    int pos, int hd, int stride, void *stream);
int    l3m_k_rmsnorm(float *y, const float *x, const float *w, int n, float eps, void *stream);  // ops.c:13
int    l3m_k_rope(float *v, int n_heads, int hd, int pos, const float *table, void *stream);      // ops.c:29
int    l3m_k_silu_mul(float *h, const float *g, int n, void *stream);                            // ops.c:49
int    l3m_k_argmax(const float *x, int n, int32_t *out, void *stream);                          // engine.c:290-301
// The decode step's own pieces, alone (parity hooks):
// rows [row0, row0 + n) of m dequantized by the step's embedding lookup (l3m_dequant_row, pack.c:55-62)
// into out[n][32 * m->nb];
int    l3m_k_dequant(const l3m_dmat *m, int row0, int n, float *out, void *stream);
// which attention a decode step runs for a head group of nq query heads (2 matrix cores over the K/V
// window in LDS, for hd a multiple of 16; 1 VALU over the window; 0 VALU reading the cache; kv_lds: the
// window fits in LDS);
int    l3m_attention_mode(int kv_lds, int hd, int nq, int ctx);
// one head group's attention in that mode, exactly as the decode step runs it (l3m_attend, ops.c:58-73, for
// each query head; GQA head h reads kv head h / (nq / nkv)): q [nq][hd] f32, kc and vc [nkv][ctx][hd] bf16
// holding rows 0..pos, out [nq][hd].
int    l3m_k_attend_decode(int mode, float *out, const float *q, const uint16_t *kc, const uint16_t *vc, int nq, int nkv, int hd,
                           int ctx, int pos, void *stream);
// One of the decode step's matvecs alone, on device pointers: form 0 the wide form of the q/k/v and
// gate/up rows, 1 the Wo columns, 2 the Wdown columns, for a body of dtype `dtype` (m stored as the step
// stores it: q4_0 as q8_0 blocks of the same values); 3 the head of dtype `dtype`, tpw tiles per workgroup
// as the head workgroups take them. x: k f32 values (the step's normalized input), prepared in the kernel
// as the step prepares it; y: m->rows floats. The same device code as the step (tile_rows, slots_rows,
// mv with rows_sum4).
int    l3m_k_step_mv(int dtype, int form, const l3m_dmat *m, const float *x, int k, float *y, int tpw, void *stream);
// The same on a loaded model's own matrices (host x and y): which 0 the q/k/v rows of head group `index`
// of layer `layer` ([q rows of its nq heads | k rows of its kv heads | v rows]), 1 its Wo columns (k = nq
// hd), 2 the gate/up rows of FFN chunk `index` (gate row r, up row r; rows past the chunk zero), 3 its
// Wdown columns (k = the chunk's rows), 4 the head (vocab rows). -1 on a bad index or a device error.
int    l3m_step_matvec(const l3m_model *m, int which, int layer, int index, const float *x, float *y);
// out[5]: head groups, FFN chunks, query heads per group, rows per chunk (the last chunk takes the rest),
// head tiles per head workgroup. Group g holds query heads [g nq, (g + 1) nq) and kv heads
// [g nq / hpk, ((g + 1) nq - 1) / hpk]; chunk c holds FFN rows [c rows, min((c + 1) rows, ffn)).
void   l3m_step_layout(const l3m_model *m, int *out);
// Host: q4_0 or mxfp4 file rows as the q8_0 file rows of the same values the step matrices hold (q4_0:
// byte n - 8, the same f16 scale; mxfp4: the doubled e2m1 codes, d = 2^(e - 128)); dst rows * k / 32
// blocks of 34 bytes, NULL source rows zero. -1 when an mxfp4 block does not widen exactly.
int    l3m_widen_rows(int src_dtype, int rows, int k, const void *const *src, void *dst);
// One streaming read of bytes (16-byte multiple) at buf: with bytes above the Infinity Cache's size it
// evicts every cached weight (the --cold eviction, engine.c:330-338).
int    l3m_dev_evict(const void *buf, size_t bytes, void *stream);
void   l3m_rope_table(float *table, int ctx, int hd, float theta);   // host: [ctx][hd/2] (cos, sin), ops.c:31-32

// Benches. l3m_bench_decode: greedy tokens from prompt (restarting at a full context, main.c:251), ns per
// generated token. Timers use hipEvents on the library stream; microseconds per launch, <0 on error.
double l3m_bench_decode(l3m_model *m, const int32_t *prompt, int n_prompt, int n_tokens);
// The same with temperature sampling on the device (seed + i for the i-th run of the context).
double l3m_bench_decode_t(l3m_model *m, const int32_t *prompt, int n_prompt, int n_tokens, float temperature, uint64_t seed);
double l3m_time_gemv(const l3m_dmat *mats, int n_mats, const void *act, int k, float *y, int iters);
// Microseconds per launch of an empty kernel queued back to back: the launch interval, below which the
// figures of l3m_time_gemv and l3m_time_read are the launch rate, not the kernel's.
double l3m_time_launch_interval(int iters);
// The measured roofline beside it: one streaming read of `bytes` (a 16-byte multiple; the last 16 bytes
// are scratch) per launch, over bufs[i % n_bufs].
double l3m_time_read(void *const *bufs, int n_bufs, size_t bytes, int iters);
// One kernel of the decode step at position pos: kind 0 attention block, 1 FFN block, 2 head.
double l3m_bench_kernel(l3m_model *m, int kind, int layer, int pos, int iters);
// Timing of the persistent decode kernel's launches (hipEvents on the library stream around each launch):
// mode 1 clears and starts, 2 adds the last finished launch (the library calls it after each), 0 stops;
// every call reports the total microseconds and launches so far.
int    l3m_decode_timer(int mode, double *us, int *launches);
// What the persistent launches of m have processed so far: out[0] steps, out[1] steps with the head,
// out[2] K/V rows read per kv head and layer (sum of pos + 1).
void   l3m_decode_work(const l3m_model *m, double *out);
double l3m_kernel_bytes(const l3m_model *m, int kind, int pos);   // weight bytes one launch of that kernel reads
double l3m_weight_bytes(const l3m_model *m);                       // weight bytes streamed per token
// The persistent decode kernel's longest wait, in ticks of the 100 MHz clock; ticks < 0 restores the default
// (1 s). Past it a waiting workgroup raises the abort word, every workgroup leaves at its next wait, and
// l3m_generate returns -1 ("a wait between phases timed out"). A test hook for that path (no counterpart in
// the reference, whose barrier waits without bound, pool.c:111-123).
void   l3m_decode_spin_limit(l3m_model *m, long long ticks);
// Whether the mxfp4 matvecs of at least 128 tiles of 64-256 blocks (l3m_k_gemv) take the matrix cores (1,
// the default; L3M_GEMV_MX=0 in the environment starts at 0) or the VALU dots of the other dtypes' 8-wavefront
// matvec (0); on < 0 only reads it. Returns the setting before the call. A test and measurement hook (no
// counterpart in the reference): at 128 blocks per row both forms split a tile over 8 wavefronts and add
// each lane's blocks in the same order, so their results are bit-identical.
int    l3m_gemv_matrix_cores(int on);
// 1 when decode runs as one persistent cooperative kernel per chunk of steps (L3M_PERSIST=0 at load
// selects the one-graph-per-step path), 0 otherwise.
int    l3m_decode_persistent(const l3m_model *m);
// Per-phase timing of the persistent decode kernel, in the library built with L3M_PHASE_STAMPS
// (libl3m_hip_phases.so; -1 in the product build): mode 0 arms the stamps for layers (layer, layer + 1) at
// one position and clears them; mode 1 copies them out: out[2][3 * 64][16], per layer the 100 MHz clock at
// each phase boundary of attention group g (row g), FFN chunk c (row 64 + c) and head workgroup h (row
// 128 + h, on the last layer), 0 where unrecorded; mode 2 copies out the shader clock (s_memtime) at the
// same points.
int    l3m_phase_stamps(int mode, int pos, int layer, unsigned long long *out);
// The logits the last generate call computed at position pos (the prediction for pos + 1), into out
// [vocab]: positions within the last 128 that call ran; -1 otherwise. An inspection hook (the sampled and
// greedy tokens are checked against the logits they came from).
int    l3m_logits_at(const l3m_model *m, int pos, float *out);
// Prompt positions the last generate call ran as one batched prefill (0: token by token). Prompts of at
// least L3M_PREFILL_MIN (default 8) tokens on q8_0 and q4_0 bodies (and mxfp4 bodies whose blocks widen
// exactly to q8_0) are prefilled unless L3M_PREFILL=0.
int    l3m_prefill_positions(const l3m_model *m);
// The attention mode the decode step of m runs at positions inside its K/V window (l3m_attention_mode's
// codes); and the window's size in positions: ctx when every position fits in LDS, else the most (a
// multiple of 32) that fit, 0 when none. Steps at positions from l3m_decode_window on read the cache (mode 0).
int    l3m_decode_attention(const l3m_model *m);
int    l3m_decode_window(const l3m_model *m);
// K and V rows [pos0, pos0 + n) of kv head kvh in layer `layer` of m's cache (bf16 as the step writes them,
// engine.c:247-248), into k and v [n][hd]; -1 when out of range.
int    l3m_kv_rows(const l3m_model *m, int layer, int kvh, int pos0, int n, uint16_t *k, uint16_t *v);
int    l3m_head_dim(const l3m_model *m);   // hd of m: the row length of l3m_kv_rows

// Probes, the GPU analogues of the reference's bench/residency.c:31-97 and bench/exchange.c:22-44 (no
// counterpart in its library): bandwidth of workgroups streaming their own shards (per_xcd workgroups on
// each of the first xcds XCDs, bytes_per_wg each, warm, passes per launch), in GB/s; microseconds per
// exchange round of n workgroups (each writes its slice of a dim-float vector, flags, waits for all flags,
// reads the vector; on one XCD or across XCDs); microseconds per node of a hipGraph of empty kernels;
// shader clocks per dependent step inside one workgroup of `threads` threads (a power of two, 64-1024), for
// which = 0 an LDS hand-over (write, barrier, another lane's word read, barrier), 1 a dependent LDS read,
// 2 a 64-lane sum by DPP and permlane swaps, 3 a bf16 matrix-core product (16x16x32) into its own
// accumulator, 4 a barrier, 5 an LDS write and read-back, 6 expf.
int    l3m_probe_stream(size_t bytes_per_wg, int xcds, int per_xcd, int passes, double *gbs);
int    l3m_probe_exchange(int n, int same_xcd, int dim, int rounds, double *us_per_round);
int    l3m_probe_graph_node(int nodes, int reps, double *us_per_node);
int    l3m_probe_latency(int which, int threads, double *clocks);

// l3m_encode (src/l3m.h:48, tokenizer.c:156-170) on the tokenizer of the file at path, on the host alone (no
// device needed): the count, or -1 when the file is refused or the ids do not fit max.
int    l3m_tokenize(const char *path, const char *text, int add_bos, int32_t *out, int max);

// Synthetic .l3m models (seeded, host-independent bytes).
typedef struct {
    const char *arch;
    int      dim, n_layers, n_heads, n_kv_heads, ffn_dim, vocab, ctx;
    float    rope_theta, norm_eps;
    int      dtype, head_dtype, tied;
    uint64_t seed;
    float    std;
    float    norm_jitter;
    int      bos, eos;
} l3m_gen_spec;
int      l3m_gen_write(const l3m_gen_spec *spec, const char *path);
void     l3m_gen_prompt(uint64_t seed, int vocab, int n, int32_t *out);
uint64_t l3m_gen_u64(uint64_t stream, uint64_t i);
float    l3m_gen_normal(uint64_t stream, uint64_t i);
void     l3m_quantize_row(int dtype, void *dst, const float *x, int k);
uint16_t l3m_f32_to_f16(float f);

#ifdef __cplusplus
}
#endif
