// Host-side internals shared by the C files of the backend: the mapped .l3m file, block packing into the
// GPU lane-tile layout, the synthetic model generator and the tokenizer.
#pragma once
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include "format.h"
#include "l3m_hip.h"

#define L3M_EXPORT __attribute__((visibility("default")))

// ---------------------------------------------------------------- mapped file (reference file.h:17-22)
typedef struct {
    int             n, bos, eos, max_len;
    int             sp_prefix, sp_words, digits;   // SentencePiece prefix space, its words split at spaces, digits one by one
    const uint8_t **bytes;
    const uint16_t *len;
    float          *score;
    int            *slot;         // ids by their bytes (open addressing, mask + 1 entries, -1 empty)
    unsigned        mask;
} l3m_vocab_table;

typedef struct {
    void             *map;
    size_t            size;
    const l3m_header *h;
    const l3m_tensor *toc;
    l3m_vocab_table   tok;
    int               im_start;   // ChatML <|im_start|> id when system != NULL
    const char       *system;
} l3m_mapped;

int               l3m_map_open(l3m_mapped *f, const char *path);   // 0, or -1 with "l3m: <path>: <why>" on stderr
void              l3m_map_close(l3m_mapped *f);
const l3m_tensor *l3m_map_tensor(const l3m_mapped *f, const char *name);
const l3m_tensor *l3m_map_blk(const l3m_mapped *f, int layer, const char *name);
const void       *l3m_map_data(const l3m_mapped *f, const l3m_tensor *t);

// ---------------------------------------------------------------- lane-tile layout (GPU weights)
// A matrix of R rows x K inputs is stored as T = ceil(R/16) tiles of 16 rows and NB = ceil(K/32) blocks:
//   quant plane [T][NB][16 rows][QBYTES]   the row's 32-input block, in its file encoding
//   scale plane [T][NB][16 rows][SBYTES]   f16 d (q8_0, q4_0), e8m0 e (mxfp4), absent for bf16/f32
// QBYTES: f32 128, bf16 64, q8_0 32, q4_0 16, mxfp4 16. Missing rows and inputs past K are zero.
// A wavefront reads 4 consecutive blocks of one tile = 4*16*QBYTES contiguous bytes per step.
#define L3M_LT_ROWS 16
int    l3m_lt_qbytes(int dtype);
int    l3m_lt_sbytes(int dtype);
size_t l3m_lt_quant_size(int dtype, int rows, int k);
size_t l3m_lt_scale_size(int dtype, int rows, int k);
// rows[r] points at file row r (l3m_file_row_bytes each) or is NULL for a zero row.
void   l3m_lt_pack_rows(int dtype, int rows, int k, const void *const *rows_src, uint8_t *quant, uint8_t *scale);
// Same, with every row widened to f32 first (the fp32 reference mode): quant is f32 lane-tile.
void   l3m_lt_pack_rows_f32(int src_dtype, int rows, int k, const void *const *rows_src, uint8_t *quant);
// From the reference's 16-row tile layout (kernels.h:1-11, pack.c:64-99): ntiles tiles of k inputs.
void   l3m_lt_pack_ltiles(int dtype, int ntiles, int k, const void *tiles, uint8_t *quant, uint8_t *scale);
// Exact dequantization of one file row (pack.c:55-62).
void   l3m_row_to_f32(float *out, int dtype, const void *row, int k);

// ---------------------------------------------------------------- synthetic models
// l3m_gen_spec is declared in l3m_hip.h.

L3M_EXPORT int      l3m_gen_write(const l3m_gen_spec *spec, const char *path);   // 0 or -1
L3M_EXPORT void     l3m_gen_prompt(uint64_t seed, int vocab, int n, int32_t *out);
L3M_EXPORT uint64_t l3m_gen_u64(uint64_t stream, uint64_t i);                    // counter-based splitmix64
L3M_EXPORT float    l3m_gen_normal(uint64_t stream, uint64_t i);                 // ~N(0,1), IEEE basic ops only
// ggml round-to-nearest quantizers on one row of k inputs (k % 32 == 0), as the exporter writes them.
L3M_EXPORT void     l3m_quantize_row(int dtype, void *dst, const float *x, int k);
L3M_EXPORT uint16_t l3m_f32_to_f16(float f);

// ---------------------------------------------------------------- tokenizer (byte table)
int            l3m_vocab_init(l3m_vocab_table *t, const void *section, size_t size, unsigned flags);
void           l3m_vocab_free(l3m_vocab_table *t);
int            l3m_vocab_encode(const l3m_vocab_table *t, const char *text, int add_bos, int32_t *out, int max);
const uint8_t *l3m_vocab_decode(const l3m_vocab_table *t, int32_t tok, int *len);
