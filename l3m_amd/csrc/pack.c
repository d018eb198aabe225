// Host-side repacking of weights into the GPU lane-tile layout, done once at load.
//
// The reference repacks file rows into 16-row tiles with 4-byte lane groups for AVX (src/pack.c:64-99).
// The GPU layout keeps each row's 32-input block in its file encoding (so unpacking on the device is
// the ggml bit definition, model.h:58-60) and lays the blocks out block-major within a 16-row tile:
// a wavefront of 64 lanes = 16 rows x 4 consecutive blocks reads one contiguous 16*4*QBYTES run with
// 128-bit loads. Scales move to their own plane so the quant plane stays 16-byte aligned.
#include <stdlib.h>
#include <string.h>
#include "host.h"

#define QB L3M_QBLOCK
#define RT L3M_LT_ROWS

int l3m_lt_qbytes(int dtype) {
    switch (dtype) {
    case L3M_F32:  return 128;
    case L3M_BF16: return 64;
    case L3M_Q8_0: return 32;
    default:       return 16;
    }
}

int l3m_lt_sbytes(int dtype) { return dtype == L3M_Q8_0 || dtype == L3M_Q4_0 ? 2 : dtype == L3M_MXFP4 ? 1 : 0; }

static size_t tiles_of(int rows) { return ((size_t)rows + RT - 1) / RT; }
static size_t blocks_of(int k) { return ((size_t)k + QB - 1) / QB; }

size_t l3m_lt_quant_size(int dtype, int rows, int k) { return tiles_of(rows) * blocks_of(k) * RT * (size_t)l3m_lt_qbytes(dtype); }
size_t l3m_lt_scale_size(int dtype, int rows, int k) { return tiles_of(rows) * blocks_of(k) * RT * (size_t)l3m_lt_sbytes(dtype); }

// Copy block b of one file row into its lane-tile slots (the tail of a partial block stays zero).
static void put_block(int dtype, const void *row, int k, int b, uint8_t *qdst, uint8_t *sdst) {
    switch (dtype) {
    case L3M_F32: {
        int n = k - b * QB < QB ? k - b * QB : QB;
        memcpy(qdst, (const float *)row + (size_t)b * QB, (size_t)n * 4);
        break;
    }
    case L3M_BF16: {
        int n = k - b * QB < QB ? k - b * QB : QB;
        memcpy(qdst, (const uint16_t *)row + (size_t)b * QB, (size_t)n * 2);
        break;
    }
    case L3M_Q8_0: {
        const l3m_block_q8_0 *s = (const l3m_block_q8_0 *)row + b;
        memcpy(qdst, s->qs, 32);
        memcpy(sdst, &s->d, 2);
        break;
    }
    case L3M_Q4_0: {
        const l3m_block_q4_0 *s = (const l3m_block_q4_0 *)row + b;
        memcpy(qdst, s->qs, 16);
        memcpy(sdst, &s->d, 2);
        break;
    }
    case L3M_MXFP4: {
        const l3m_block_mxfp4 *s = (const l3m_block_mxfp4 *)row + b;
        memcpy(qdst, s->qs, 16);
        sdst[0] = s->e;
        break;
    }
    }
}

void l3m_lt_pack_rows(int dtype, int rows, int k, const void *const *src, uint8_t *quant, uint8_t *scale) {
    size_t nb = blocks_of(k), qb = (size_t)l3m_lt_qbytes(dtype), sb = (size_t)l3m_lt_sbytes(dtype);
    memset(quant, 0, l3m_lt_quant_size(dtype, rows, k));
    if (sb) memset(scale, 0, l3m_lt_scale_size(dtype, rows, k));
    for (int r = 0; r < rows; r++) {
        if (!src[r]) continue;
        size_t t = (size_t)r / RT, c = (size_t)r % RT;
        for (size_t b = 0; b < nb; b++) {
            size_t slot = (t * nb + b) * RT + c;
            put_block(dtype, src[r], k, (int)b, quant + slot * qb, sb ? scale + slot * sb : NULL);
        }
    }
}

// Exact widening of a file row (the unpacked values are exact in f32: pack.c:55-62 of the reference).
void l3m_row_to_f32(float *out, int dtype, const void *row, int k) {
    switch (dtype) {
    case L3M_F32: memcpy(out, row, (size_t)k * 4); return;
    case L3M_BF16: for (int i = 0; i < k; i++) out[i] = l3m_bf16_f32(((const uint16_t *)row)[i]); return;
    }
    for (int b = 0; b < k / QB; b++) {
        float d;
        int q[QB];
        if (dtype == L3M_Q8_0) {
            const l3m_block_q8_0 *s = (const l3m_block_q8_0 *)row + b;
            d = l3m_f16_f32(s->d);
            for (int i = 0; i < QB; i++) q[i] = s->qs[i];
        } else {
            const uint8_t *qs = dtype == L3M_Q4_0 ? ((const l3m_block_q4_0 *)row + b)->qs : ((const l3m_block_mxfp4 *)row + b)->qs;
            d = dtype == L3M_Q4_0 ? l3m_f16_f32(((const l3m_block_q4_0 *)row + b)->d) : l3m_e8m0_half(((const l3m_block_mxfp4 *)row + b)->e);
            for (int i = 0; i < QB / 2; i++) {
                int lo = qs[i] & 15, hi = qs[i] >> 4;
                q[i] = dtype == L3M_Q4_0 ? lo - 8 : L3M_E2M1X2[lo];
                q[i + QB / 2] = dtype == L3M_Q4_0 ? hi - 8 : L3M_E2M1X2[hi];
            }
        }
        for (int i = 0; i < QB; i++) out[b * QB + i] = d * (float)q[i];
    }
}

void l3m_lt_pack_rows_f32(int src_dtype, int rows, int k, const void *const *src, uint8_t *quant) {
    size_t nb = blocks_of(k);
    float *tmp = malloc((size_t)k * sizeof(float));
    memset(quant, 0, l3m_lt_quant_size(L3M_F32, rows, k));
    for (int r = 0; r < rows && tmp; r++) {
        if (!src[r]) continue;
        l3m_row_to_f32(tmp, src_dtype, src[r], k);
        size_t t = (size_t)r / RT, c = (size_t)r % RT;
        for (size_t b = 0; b < nb; b++) put_block(L3M_F32, tmp, k, (int)b, quant + ((t * nb + b) * RT + c) * 128, NULL);
    }
    free(tmp);
}

// From the reference's tile layout (kernels.h:1-11): per tile of 16 lanes and k inputs,
//   f32 [k][16]; bf16 [k/2][16][2]; quantized per 32 inputs: scales[16], then bytes where
//   q8: byte (i/4*16 + c)*4 + i%4 holds value+128; q4/mxfp4: byte (g*16 + c)*4 + j holds
//   element 8g+j in its low nibble and 8g+4+j in its high nibble.
void l3m_lt_pack_ltiles(int dtype, int ntiles, int k, const void *tiles, uint8_t *quant, uint8_t *scale) {
    int rows = ntiles * RT;
    size_t nb = blocks_of(k), qb = (size_t)l3m_lt_qbytes(dtype), sb = (size_t)l3m_lt_sbytes(dtype);
    memset(quant, 0, l3m_lt_quant_size(dtype, rows, k));
    if (sb) memset(scale, 0, l3m_lt_scale_size(dtype, rows, k));
    const uint8_t *src = tiles;
    size_t tile_bytes = dtype == L3M_F32 ? (size_t)k * RT * 4 : dtype == L3M_BF16 ? (size_t)k * RT * 2
                      : (size_t)k / QB * (dtype == L3M_Q8_0 ? 2 * RT + QB * RT : dtype == L3M_Q4_0 ? 2 * RT + QB * RT / 2 : RT + QB * RT / 2);
    for (int t = 0; t < ntiles; t++, src += tile_bytes) {
        for (int c = 0; c < RT; c++) {
            for (size_t b = 0; b < nb; b++) {
                size_t slot = ((size_t)t * nb + b) * RT + (size_t)c;
                uint8_t *qd = quant + slot * qb;
                if (dtype == L3M_F32 || dtype == L3M_BF16) {
                    int es = dtype == L3M_F32 ? 4 : 2;
                    for (int i = 0; i < QB && (int)b * QB + i < k; i++) {
                        int e = (int)b * QB + i;
                        size_t off = dtype == L3M_F32 ? ((size_t)e * RT + c) * 4 : (((size_t)e / 2 * RT + c) * 2 + e % 2) * 2;
                        memcpy(qd + (size_t)i * es, src + off, (size_t)es);
                    }
                    continue;
                }
                size_t blk_bytes = dtype == L3M_Q8_0 ? 2 * RT + QB * RT : dtype == L3M_Q4_0 ? 2 * RT + QB * RT / 2 : RT + QB * RT / 2;
                size_t scale_bytes = dtype == L3M_MXFP4 ? RT : 2 * RT;
                const uint8_t *blk = src + b * blk_bytes, *q = blk + scale_bytes;
                uint8_t *sd = scale + slot * sb;
                if (dtype == L3M_MXFP4) sd[0] = blk[c];
                else memcpy(sd, blk + 2 * c, 2);
                if (dtype == L3M_Q8_0) {
                    for (int i = 0; i < QB; i++) qd[i] = (uint8_t)(q[((size_t)i / 4 * RT + c) * 4 + i % 4] - 128);
                } else {
                    uint8_t nib[QB];
                    for (int g = 0; g < 4; g++)
                        for (int j = 0; j < 4; j++) {
                            uint8_t byte = q[((size_t)g * RT + c) * 4 + j];
                            nib[8 * g + j] = byte & 15;
                            nib[8 * g + 4 + j] = byte >> 4;
                        }
                    for (int i = 0; i < QB / 2; i++) qd[i] = (uint8_t)(nib[i] | nib[i + QB / 2] << 4);
                }
            }
        }
    }
}
