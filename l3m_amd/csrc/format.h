// The .l3m v1 on-disk format, byte-compatible with fpedd/l3m (src/model.h:1-70), plus the
// bit-level helpers every part of the backend shares (f16/bf16 conversion, block geometry).
//
// A file is [header 1024 B][tensors, each 64-B aligned][toc][tokenizer][chat, optional].
// Matrices are [rows = outputs][cols = inputs], row-major; quantized rows are runs of 32-input blocks
// whose bytes are ggml's (model.h:58-60).
#pragma once
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define L3M_VERSION 1
#define L3M_QBLOCK  32

enum l3m_dtype { L3M_F32, L3M_BF16, L3M_Q8_0, L3M_Q4_0, L3M_MXFP4, L3M_NDTYPES };

// Architecture flags (model.h:19-26).
enum l3m_flags {
    L3M_F_LAYERNORM   = 1 << 0,
    L3M_F_LEARNED_POS = 1 << 1,
    L3M_F_GELU        = 1 << 2,
    L3M_F_TIED        = 1 << 3,
    L3M_F_SP_PREFIX   = 1 << 4,
    L3M_F_DIGITS      = 1 << 5,
};

typedef struct {
    char     magic[4];            // "l3m\0"
    uint32_t version;
    char     arch[16];
    uint32_t flags;
    uint32_t dim, n_layers, n_heads, n_kv_heads, ffn_dim, vocab, ctx;
    float    rope_theta, norm_eps;
    uint32_t n_tensors, reserved;
    uint64_t toc_offset, tokenizer_offset, chat_offset;
    uint8_t  pad[1024 - 96];
} l3m_header;
_Static_assert(sizeof(l3m_header) == 1024, "l3m header is 1024 bytes");

typedef struct {
    char     name[64];
    uint32_t dtype, ndim;
    uint64_t shape[4];
    uint64_t offset, nbytes;
} l3m_tensor;
_Static_assert(sizeof(l3m_tensor) == 120, "toc entry is 120 bytes");

typedef struct { uint32_t n_tokens; int32_t bos, eos; uint32_t max_len; } l3m_tok_header;

// ggml blocks: q8_0 x = q*d; q4_0 nibble i low = x[i], high = x[i+16], x = (n-8)*d;
// mxfp4 same nibble order, x = e2m1(n) * 2^(e-127), e2m1 held doubled as an integer.
typedef struct { uint16_t d; int8_t  qs[32]; } l3m_block_q8_0;
typedef struct { uint16_t d; uint8_t qs[16]; } l3m_block_q4_0;
typedef struct { uint8_t  e; uint8_t qs[16]; } l3m_block_mxfp4;
_Static_assert(sizeof(l3m_block_q8_0) == 34 && sizeof(l3m_block_q4_0) == 18 && sizeof(l3m_block_mxfp4) == 17, "ggml blocks");

// Doubled e2m1 magnitudes with the sign in bit 3 (kernels.h:20).
static const int8_t L3M_E2M1X2[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

static inline const char *l3m_dtype_name(int dtype) {
    switch (dtype) {
    case L3M_F32: return "f32";
    case L3M_BF16: return "bf16";
    case L3M_Q8_0: return "q8_0";
    case L3M_Q4_0: return "q4_0";
    case L3M_MXFP4: return "mxfp4";
    }
    return "?";
}

// Bytes of one file row of k inputs (pack.c:10-19).
static inline size_t l3m_file_row_bytes(int dtype, int k) {
    static const unsigned per_block[L3M_NDTYPES] = {4 * L3M_QBLOCK, 2 * L3M_QBLOCK, sizeof(l3m_block_q8_0), sizeof(l3m_block_q4_0),
                                                    sizeof(l3m_block_mxfp4)};
    if (dtype < 0 || dtype >= L3M_NDTYPES) return 0;
    if (dtype <= L3M_BF16) return (size_t)k * (per_block[dtype] / L3M_QBLOCK);   // f32, bf16: any width
    return (size_t)(k / L3M_QBLOCK) * per_block[dtype];
}

static inline float l3m_bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t l3m_f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static inline float l3m_bf16_f32(uint16_t h) { return l3m_bits_f32((uint32_t)h << 16); }

// Round to nearest even; NaN is not special-cased, as in the reference (ops.h:6).
static inline uint16_t l3m_f32_bf16(float f) {
    uint32_t u = l3m_f32_bits(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// IEEE half to float, subnormals included (ops.c:5-11). Built from exact integer steps: a subnormal
// mantissa m is m * 2^-24, which is exact in float.
static inline float l3m_f16_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 0) {
        float v = (float)m * l3m_bits_f32(0x33800000u);   // 2^-24
        return sign ? -v : v;
    }
    if (e == 31) return l3m_bits_f32(sign | 0x7F800000u | m << 13);
    return l3m_bits_f32(sign | (e + 112) << 23 | m << 13);
}

// 2^(e-128) = the mxfp4 block scale 2^(e-127)/2 (pack.c:40), as exact float bits; e < 2 is subnormal.
static inline float l3m_e8m0_half(uint8_t e) {
    int x = (int)e - 128;                                  // -128 .. 127
    if (x >= -126) return l3m_bits_f32((uint32_t)(x + 127) << 23);
    return l3m_bits_f32(1u << (x + 149));                  // 2^-128 = bit 21, 2^-127 = bit 22
}
