// HIP kernels for the batch-1 decode hot path on CDNA4 (gfx950), and their launchers.
//
// Matrix-vector products read weights in the lane-tile layout (host.h): a workgroup of 4 wavefronts
// owns up to 4 tiles of 16 output rows; inside a wavefront lane = 16*sub + row, and the 4 subs walk
// consecutive 32-input blocks, so each step of a wavefront is one contiguous 1-4 KiB run of 128-bit
// loads. The activation vector is prepared once per workgroup into LDS (l3m's per-32-block int8
// quantization, or bf16, or f32) and broadcast from there. Per-block integer dots use v_dot4_i32_i8;
// q4_0 nibbles are masked in registers, mxfp4 e2m1 codes go through two v_perm_b32 byte tables.
// Reductions are fixed-order (wavefront shuffles, then LDS), so results are run-to-run identical.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include "dev.h"
#include "format.h"

namespace {

constexpr int RT = 16;    // rows per tile
constexpr int NT = 256;   // threads per workgroup

__host__ __device__ constexpr int qbytes(int dt) { return dt == L3M_F32 ? 128 : dt == L3M_BF16 ? 64 : dt == L3M_Q8_0 ? 32 : 16; }
__host__ __device__ constexpr int sbytes(int dt) { return dt == L3M_Q8_0 || dt == L3M_Q4_0 ? 2 : dt == L3M_MXFP4 ? 1 : 0; }
__host__ __device__ constexpr bool quantized(int dt) { return dt >= L3M_Q8_0; }
__host__ __device__ inline int kpad(int k) { return (k + 31) & ~31; }
__host__ __device__ inline size_t act_size(int dt, int k) {
    const int kp = kpad(k);
    return quantized(dt) ? (size_t)kp + 8 * (size_t)(kp / 32) : dt == L3M_BF16 ? 2 * (size_t)kp : 4 * (size_t)kp;
}
__host__ __device__ inline size_t align16(size_t n) { return (n + 15) & ~(size_t)15; }

// ------------------------------------------------------------------------------------------ scalars

__device__ __forceinline__ float f16_f32(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }
__device__ __forceinline__ float bf16_f32(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ uint16_t f32_bf16(float f) {       // nearest even, as the reference (ops.h:6)
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
// 2^(e-128): the mxfp4 block scale 2^(e-127)/2, exact; e < 2 gives an f32 subnormal.
__device__ __forceinline__ float e8m0_half(uint32_t e) {
    const int x = (int)e - 128;
    return x >= -126 ? __uint_as_float((uint32_t)(x + 127) << 23) : __uint_as_float(1u << (x + 149));
}
// Four e2m1 codes (one per byte, 0..15) to their doubled magnitudes + 16, i.e. 4..28 (kernels.h:21).
__device__ __forceinline__ uint32_t e2m1x2_plus16(uint32_t n) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(0x1C181614u, 0x13121110u, sel);   // 16 17 18 19 20 22 24 28
    const uint32_t neg = __builtin_amdgcn_perm(0x04080A0Cu, 0x0D0E0F10u, sel);   // 16 15 14 13 12 10  8  4
    const uint32_t m = ((n >> 3) & 0x01010101u) * 0xFFu;
    return (neg & m) | (pos & ~m);
}
__device__ __forceinline__ int dot4(uint32_t a, int b, int c) { return __builtin_amdgcn_sdot4((int)a, b, c, false); }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2bf(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// Element i of row r of a lane-tile matrix, exactly dequantized (the reference's dequant_row, pack.c:55-62).
__device__ float lt_elem(const l3m_dmat &m, int r, int i) {
    const size_t slot = ((size_t)(r >> 4) * m.nb + (i >> 5)) * RT + (r & 15);
    const int j = i & 31;
    switch (m.dtype) {
    case L3M_F32:  return ((const float *)m.q)[slot * 32 + j];
    case L3M_BF16: return bf16_f32(((const uint16_t *)m.q)[slot * 32 + j]);
    case L3M_Q8_0: return f16_f32(((const uint16_t *)m.s)[slot]) * (float)((const int8_t *)m.q)[slot * 32 + j];
    default: {
        const uint8_t byte = m.q[slot * 16 + (j & 15)];
        const int n = j < 16 ? byte & 15 : byte >> 4;
        if (m.dtype == L3M_Q4_0) return f16_f32(((const uint16_t *)m.s)[slot]) * (float)(n - 8);
        const int8_t e2m1x2[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
        return e8m0_half(m.s[slot]) * (float)e2m1x2[n];
    }
    }
}

// ------------------------------------------------------------------------------- workgroup helpers

// Sum over the workgroup in a fixed order; every thread gets the result. scratch: 4 floats of LDS.
__device__ float wg_sum(float v, float *scratch) {
    for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scratch[w] = v;
    __syncthreads();
    return ((scratch[0] + scratch[1]) + scratch[2]) + scratch[3];
}
__device__ float wg_max(float v, float *scratch) {
    for (int o = 32; o; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scratch[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(scratch[0], scratch[1]), fmaxf(scratch[2], scratch[3]));
}
// (value, index) maximum; ties and NaN go to the lower index, as the reference's strict '>' scan
// (engine.c:294, 300).
__device__ __forceinline__ void better(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i) || (v != v && v2 == v2)) { v = v2; i = i2; }
}
__device__ void wg_argmax(float &v, int &i, float *sv, int *si) {
    for (int o = 32; o; o >>= 1) {
        const float v2 = __shfl_xor(v, o);
        const int i2 = __shfl_xor(i, o);
        better(v, i, v2, i2);
    }
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { sv[w] = v; si[w] = i; }
    __syncthreads();
    v = sv[0]; i = si[0];
    for (int k = 1; k < 4; k++) better(v, i, sv[k], si[k]);
}

// x (k values, zero up to kp) into LDS xs, optionally RMS-normalized with weights nw (ops.c:13-18:
// s = 1/sqrt(sum x^2 / n + eps), y = x * s * w). src(i) yields x_i.
template <class Src>
__device__ void stage_x(float *xs, Src src, int k, int kp, const float *nw, float eps, float *scratch) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < kp; i += NT) {
        const float v = i < k ? src(i) : 0.f;
        xs[i] = v;
        ss = fmaf(v, v, ss);
    }
    if (nw) {
        const float tot = wg_sum(ss, scratch);
        const float s = 1.0f / sqrtf(tot / (float)k + eps);
        for (int i = threadIdx.x; i < k; i += NT) xs[i] = xs[i] * s * nw[i];
    }
    __syncthreads();
}

// Activation prep (pack.c:101-123): quantized -> per 32-block amax, inv = 127/amax, q = rint(x*inv),
// scale = amax/127, sum = sum(q); bf16 -> nearest even; f32 -> as is. 8 lanes per block.
template <int DT>
__device__ void prep_act(uint8_t *act, const float *xs, int kp) {
    if constexpr (quantized(DT)) {
        const int nb = kp / 32, g = threadIdx.x >> 3, l = threadIdx.x & 7;
        float *scale = (float *)(act + kp);
        int *sum = (int *)(act + kp + 4 * nb);
        for (int b = g; b < nb; b += NT / 8) {
            const float4 v = *(const float4 *)(xs + b * 32 + 4 * l);
            float am = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
            am = fmaxf(am, __shfl_xor(am, 1));
            am = fmaxf(am, __shfl_xor(am, 2));
            am = fmaxf(am, __shfl_xor(am, 4));
            const float inv = am > 0.f ? 127.0f / am : 0.f;
            const int q0 = (int)rintf(v.x * inv), q1 = (int)rintf(v.y * inv), q2 = (int)rintf(v.z * inv), q3 = (int)rintf(v.w * inv);
            *(uint32_t *)(act + b * 32 + 4 * l) = (uint32_t)(q0 & 255) | (uint32_t)(q1 & 255) << 8 | (uint32_t)(q2 & 255) << 16 | (uint32_t)(q3 & 255) << 24;
            int s = q0 + q1 + q2 + q3;
            s += __shfl_xor(s, 1);
            s += __shfl_xor(s, 2);
            s += __shfl_xor(s, 4);
            if (l == 0) { scale[b] = am / 127.0f; sum[b] = s; }
        }
    } else if constexpr (DT == L3M_BF16) {
        uint16_t *o = (uint16_t *)act;
        for (int i = threadIdx.x; i < kp; i += NT) o[i] = f32_bf16(xs[i]);
    } else {
        float *o = (float *)act;
        for (int i = threadIdx.x; i < kp; i += NT) o[i] = xs[i];
    }
    __syncthreads();
}

// ------------------------------------------------------------------------------------- matvec core

// One row-block: acc += (x.scale[b] * d) * (integer dot - offset * x.sum[b]) for the quantized dtypes
// (kernels_scalar.c:30-75), or the bf16 / f32 dot (kernels_scalar.c:9-28).
template <int DT>
__device__ __forceinline__ float block_fma(float acc, const uint4 *w, uint32_t sc, const uint8_t *act, int kp, int b) {
    if constexpr (quantized(DT)) {
        const int4 *xv = (const int4 *)(act + b * 32);
        const int4 x0 = xv[0], x1 = xv[1];
        const float xs = ((const float *)(act + kp))[b];
        int dot = 0;
        if constexpr (DT == L3M_Q8_0) {
            dot = dot4(w[0].x, x0.x, dot); dot = dot4(w[0].y, x0.y, dot);
            dot = dot4(w[0].z, x0.z, dot); dot = dot4(w[0].w, x0.w, dot);
            dot = dot4(w[1].x, x1.x, dot); dot = dot4(w[1].y, x1.y, dot);
            dot = dot4(w[1].z, x1.z, dot); dot = dot4(w[1].w, x1.w, dot);
            return fmaf(xs * f16_f32(sc), (float)dot, acc);
        } else {
            const int xsum = ((const int *)(act + kp + 4 * (kp / 32)))[b];
            const uint32_t v[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
            const int lo[4] = {x0.x, x0.y, x0.z, x0.w}, hi[4] = {x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t a = v[j] & 0x0F0F0F0Fu, c = (v[j] >> 4) & 0x0F0F0F0Fu;
                if constexpr (DT == L3M_MXFP4) { a = e2m1x2_plus16(a); c = e2m1x2_plus16(c); }
                dot = dot4(a, lo[j], dot);
                dot = dot4(c, hi[j], dot);
            }
            if constexpr (DT == L3M_Q4_0) return fmaf(xs * f16_f32(sc), (float)(dot - 8 * xsum), acc);
            else return fmaf(xs * e8m0_half(sc), (float)(dot - 16 * xsum), acc);
        }
    } else if constexpr (DT == L3M_BF16) {
        const uint4 *xv = (const uint4 *)(act + b * 64);
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const uint4 x = xv[v];
            acc = dot2bf(w[v].x, x.x, acc); acc = dot2bf(w[v].y, x.y, acc);
            acc = dot2bf(w[v].z, x.z, acc); acc = dot2bf(w[v].w, x.w, acc);
        }
        return acc;
    } else {
        const float4 *xv = (const float4 *)(act + b * 128);
#pragma unroll
        for (int v = 0; v < 8; v++) {
            const float4 x = xv[v];
            acc = fmaf(__uint_as_float(w[v].x), x.x, acc); acc = fmaf(__uint_as_float(w[v].y), x.y, acc);
            acc = fmaf(__uint_as_float(w[v].z), x.z, acc); acc = fmaf(__uint_as_float(w[v].w), x.w, acc);
        }
        return acc;
    }
}

// This lane's partial dot for row (lane & 15) of `tile`, over blocks b0 + sub, b0 + sub + 4, ... < b1.
template <int DT>
__device__ __forceinline__ float lane_dot(const l3m_dmat &m, int tile, int b0, int b1, const uint8_t *act, int kp, int lane) {
    constexpr int QBY = qbytes(DT), SBY = sbytes(DT), NV = QBY / 16;
    constexpr int U = DT == L3M_F32 ? 1 : DT == L3M_BF16 ? 2 : DT == L3M_Q8_0 ? 4 : 8;
    const int c = lane & 15, sub = lane >> 4;
    const size_t base = (size_t)tile * m.nb * RT + c;
    const uint8_t *__restrict__ qp = m.q + base * QBY;
    const uint8_t *__restrict__ sp = SBY ? m.s + base * SBY : nullptr;
    float acc = 0.f;
    for (int b = b0 + sub; b < b1; b += 4 * U) {
        uint4 w[U][NV];
        uint32_t sc[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int bb = b + 4 * u;
            sc[u] = 0;
            if (bb < b1) {
                const uint4 *src = (const uint4 *)(qp + (size_t)bb * RT * QBY);
#pragma unroll
                for (int v = 0; v < NV; v++) w[u][v] = src[v];
                if constexpr (SBY == 2) sc[u] = *(const uint16_t *)(sp + (size_t)bb * RT * 2);
                if constexpr (SBY == 1) sc[u] = sp[(size_t)bb * RT];
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (b + 4 * u < b1) acc = block_fma<DT>(acc, w[u], sc[u], act, kp, b + 4 * u);
    }
    return acc;
}

// The workgroup's 4/S tiles starting at tile0, each split over S wavefronts along the inputs.
// yv[t*16 + r] = output row r of tile tile0 + t. red: 64 floats of LDS.
template <int DT>
__device__ void wg_matvec(const l3m_dmat &m, int tile0, int S, const uint8_t *act, int kp, float *red, float *yv) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, tpw = 4 / S;
    const int t = wave / S, split = wave % S, tile = tile0 + t;
    const int b0 = split * m.nb / S, b1 = (split + 1) * m.nb / S;
    float acc = tile < m.tiles ? lane_dot<DT>(m, tile, b0, b1, act, kp, lane) : 0.f;
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (lane < 16) red[wave * 16 + lane] = acc;
    __syncthreads();
    if (tid < tpw * 16) {
        const int tt = tid >> 4, r = tid & 15;
        float y = red[(tt * S) * 16 + r];
        for (int s = 1; s < S; s++) y += red[(tt * S + s) * 16 + r];
        yv[tid] = y;
    }
    __syncthreads();
}

// LDS carve-up shared by the matvec kernels.
struct Smem {
    uint8_t *act;
    float *xs, *red, *yv, *scr;
    int *iscr;
};
__device__ Smem carve(uint8_t *base, int dt, int k) {
    Smem s;
    const int kp = kpad(k);
    s.act = base;
    s.xs = (float *)(base + align16(act_size(dt, k)));
    s.red = s.xs + kp;
    s.yv = s.red + 64;
    s.scr = s.yv + 64;
    s.iscr = (int *)(s.scr + 8);
    return s;
}
inline size_t smem_bytes(int dt, int k) { return align16(act_size(dt, k)) + 4 * (size_t)kpad(k) + 4 * (64 + 64 + 16); }
constexpr size_t LDS_MAX = 65536;   // dynamic LDS per workgroup without opting in to more

int pick_split(int nb) { return nb >= 16 ? 4 : nb >= 8 ? 2 : 1; }

// ------------------------------------------------------------------------------------------ kernels

extern "C" __global__ void __launch_bounds__(NT) k_dummy() {}

template <int DT>
__global__ void __launch_bounds__(NT) k_prep(const float *__restrict__ x, int k, uint8_t *__restrict__ out) {
    extern __shared__ __align__(16) uint8_t smem[];
    Smem s = carve(smem, DT, k);
    const int kp = kpad(k);
    stage_x(s.xs, [&](int i) { return x[i]; }, k, kp, nullptr, 0.f, s.scr);
    prep_act<DT>(s.act, s.xs, kp);
    const size_t n = act_size(DT, k);
    for (size_t i = threadIdx.x; i < n; i += NT) out[i] = s.act[i];
}

template <int DT>
__global__ void __launch_bounds__(NT) k_gemv(l3m_dmat m, const uint8_t *__restrict__ act_g, int k, float *__restrict__ y, int S) {
    extern __shared__ __align__(16) uint8_t smem[];
    Smem s = carve(smem, DT, k);
    const int kp = kpad(k);
    const size_t n4 = act_size(DT, k) / 4;   // 40 bytes per 32 inputs when quantized: whole words, not whole uint4
    for (size_t i = threadIdx.x; i < n4; i += NT) ((uint32_t *)s.act)[i] = ((const uint32_t *)act_g)[i];
    __syncthreads();
    const int tpw = 4 / S, tile0 = blockIdx.x * tpw;
    wg_matvec<DT>(m, tile0, S, s.act, kp, s.red, s.yv);
    if (threadIdx.x < tpw * 16) {
        const int r = (tile0 + (threadIdx.x >> 4)) * RT + (threadIdx.x & 15);
        if (r < m.rows) y[r] = s.yv[threadIdx.x];
    }
}

// One workgroup per query head (ops.c:58-73): scores q.K[t] / sqrt(hd) over t = 0..pos, softmax, sum of
// p[t] V[t]. K, V rows are `stride` elements apart; head h reads kv head h / hpk at k + kvh * kv_stride.
// dpos, when set, holds pos (device-resident step position).
__global__ void __launch_bounds__(NT) k_attend(float *__restrict__ out, const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                               const uint16_t *__restrict__ vc, int pos, const int *dpos, int hd, int stride,
                                               int hpk, size_t kv_stride) {
    extern __shared__ __align__(16) uint8_t smem[];
    if (dpos) pos = *dpos;
    const int h = blockIdx.x, n = pos + 1, tid = threadIdx.x;
    float *qs = (float *)smem, *sc = qs + hd, *part = sc + ((n + 3) & ~3), *scr = part + NT;
    const uint16_t *kh = kc + (size_t)(h / hpk) * kv_stride, *vh = vc + (size_t)(h / hpk) * kv_stride;
    for (int i = tid; i < hd; i += NT) qs[i] = q[(size_t)h * hd + i];
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)hd);
    float mx = -INFINITY;
    for (int t = tid; t < n; t += NT) {
        const uint4 *kr = (const uint4 *)(kh + (size_t)t * stride);
        float dot = 0.f;
        for (int v = 0; v < hd / 8; v++) {
            const uint4 kk = kr[v];
            const float *qq = qs + v * 8;
            dot = fmaf(qq[0], bf16_f32(kk.x & 0xFFFF), dot); dot = fmaf(qq[1], bf16_f32(kk.x >> 16), dot);
            dot = fmaf(qq[2], bf16_f32(kk.y & 0xFFFF), dot); dot = fmaf(qq[3], bf16_f32(kk.y >> 16), dot);
            dot = fmaf(qq[4], bf16_f32(kk.z & 0xFFFF), dot); dot = fmaf(qq[5], bf16_f32(kk.z >> 16), dot);
            dot = fmaf(qq[6], bf16_f32(kk.w & 0xFFFF), dot); dot = fmaf(qq[7], bf16_f32(kk.w >> 16), dot);
        }
        const float st = dot * scale;
        sc[t] = st;
        mx = fmaxf(mx, st);
    }
    mx = wg_max(mx, scr);
    float sum = 0.f;
    for (int t = tid; t < n; t += NT) {
        const float e = expf(sc[t] - mx);
        sc[t] = e;
        sum += e;
    }
    sum = wg_sum(sum, scr);
    for (int t = tid; t < n; t += NT) sc[t] = sc[t] / sum;
    __syncthreads();
    const int groups = NT / hd, i = tid % hd, g = tid / hd;
    float acc = 0.f;
    if (g < groups)
        for (int t = g; t < n; t += groups) acc = fmaf(sc[t], bf16_f32(vh[(size_t)t * stride + i]), acc);
    part[tid] = acc;
    __syncthreads();
    if (tid < hd) {
        float o = part[tid];
        for (int gg = 1; gg < groups; gg++) o += part[gg * hd + tid];
        out[(size_t)h * hd + tid] = o;
    }
}

__global__ void __launch_bounds__(NT) k_rmsnorm(float *y, const float *x, const float *w, int n, float eps) {
    extern __shared__ __align__(16) uint8_t smem[];
    float *xs = (float *)smem, *scr = xs + kpad(n);
    stage_x(xs, [&](int i) { return x[i]; }, n, kpad(n), w, eps, scr);
    for (int i = threadIdx.x; i < n; i += NT) y[i] = xs[i];
}

// Pairs (2i, 2i+1) of each head rotate by the table angle i (ops.c:29-40).
__device__ __forceinline__ float rope_one(float val, float partner, float c, float s, bool odd) {
    return odd ? partner * s + val * c : val * c - partner * s;
}

__global__ void __launch_bounds__(NT) k_rope(float *v, int n, int hd, const float *table) {
    const int r = blockIdx.x * NT + threadIdx.x;
    const float val = r < n ? v[r] : 0.f, partner = __shfl_xor(val, 1);
    if (r < n) {
        const int i = (r % hd) >> 1;
        v[r] = rope_one(val, partner, table[2 * i], table[2 * i + 1], r & 1);
    }
}

__device__ __forceinline__ float silu_mul(float up, float g) { return up * (g / (1.0f + expf(-g))); }

__global__ void __launch_bounds__(NT) k_silu_mul(float *h, const float *g, int n) {
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i < n) h[i] = silu_mul(h[i], g[i]);
}

__global__ void __launch_bounds__(NT) k_argmax(const float *x, int n, int32_t *out) {
    __shared__ float sv[4];
    __shared__ int si[4];
    float v = -INFINITY;
    int idx = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < n; i += NT) better(v, idx, x[i], i);
    wg_argmax(v, idx, sv, si);
    if (threadIdx.x == 0) *out = idx == 0x7FFFFFFF ? 0 : idx;
}

// ------------------------------------------------------------------------------ fused decode kernels

// Layer input x: the residual stream, or for layer 0 the embedding row of tokens[pos] (engine.c:236).
struct XIn {
    const float *x;
    l3m_dmat embed;
    int tok;
    __device__ float operator()(int i) const { return x ? x[i] : lt_elem(embed, tok, i); }
};

// RMSNorm + prep + qkv rows + RoPE on q and k + bf16 K, V into the cache at pos (engine.c:241-248).
template <int DT>
__global__ void __launch_bounds__(NT) k_qkv(l3m_dmodel M, l3m_dlayer L, int layer, int from_embed, int S) {
    extern __shared__ __align__(16) uint8_t smem[];
    Smem s = carve(smem, DT, M.dim);
    const int kp = kpad(M.dim), pos = *M.pos;
    XIn src{from_embed ? nullptr : M.x, M.embed, from_embed ? M.tokens[pos] : 0};
    if (from_embed && blockIdx.x == 0)
        for (int i = threadIdx.x; i < M.dim; i += NT) M.x[i] = src(i);
    stage_x(s.xs, src, M.dim, kp, L.attn_norm, M.eps, s.scr);
    prep_act<DT>(s.act, s.xs, kp);
    const int tpw = 4 / S, tile0 = blockIdx.x * tpw;
    wg_matvec<DT>(L.qkv, tile0, S, s.act, kp, s.red, s.yv);
    if (threadIdx.x < 64) {
        const int tid = threadIdx.x, r = (tile0 + (tid >> 4)) * RT + (tid & 15);
        const float val = tid < tpw * 16 ? s.yv[tid] : 0.f, partner = __shfl_xor(val, 1);
        if (tid < tpw * 16 && r < L.qkv.rows) {
            const int kvd = M.kv_dim;
            if (r < M.dim + kvd) {
                const int local = r < M.dim ? r : r - M.dim, i = (local % M.hd) >> 1;
                const float *cs = M.rope + ((size_t)pos * (M.hd >> 1) + i) * 2;
                const float o = rope_one(val, partner, cs[0], cs[1], local & 1);
                if (r < M.dim) M.q[r] = o;
                else M.kc[(((size_t)layer * M.n_kv + local / M.hd) * M.ctx + pos) * M.hd + local % M.hd] = f32_bf16(o);
            } else {
                const int local = r - M.dim - kvd;
                M.vc[(((size_t)layer * M.n_kv + local / M.hd) * M.ctx + pos) * M.hd + local % M.hd] = f32_bf16(val);
            }
        }
    }
}

// Prep of attn + wo rows + residual add (engine.c:256-259).
template <int DT>
__global__ void __launch_bounds__(NT) k_wo(l3m_dmodel M, l3m_dlayer L, int S) {
    extern __shared__ __align__(16) uint8_t smem[];
    Smem s = carve(smem, DT, M.dim);
    const int kp = kpad(M.dim);
    const float *a = M.attn;
    stage_x(s.xs, [&](int i) { return a[i]; }, M.dim, kp, nullptr, 0.f, s.scr);
    prep_act<DT>(s.act, s.xs, kp);
    const int tpw = 4 / S, tile0 = blockIdx.x * tpw;
    wg_matvec<DT>(L.wo, tile0, S, s.act, kp, s.red, s.yv);
    if (threadIdx.x < tpw * 16) {
        const int r = (tile0 + (threadIdx.x >> 4)) * RT + (threadIdx.x & 15);
        if (r < M.dim) M.x[r] += s.yv[threadIdx.x];
    }
}

// RMSNorm + prep + gate and up rows of the same outputs + h = up * silu(gate) (engine.c:261-268).
template <int DT>
__global__ void __launch_bounds__(NT) k_ffn(l3m_dmodel M, l3m_dlayer L, int S) {
    extern __shared__ __align__(16) uint8_t smem[];
    Smem s = carve(smem, DT, M.dim);
    const int kp = kpad(M.dim);
    const float *x = M.x;
    stage_x(s.xs, [&](int i) { return x[i]; }, M.dim, kp, L.ffn_norm, M.eps, s.scr);
    prep_act<DT>(s.act, s.xs, kp);
    const int tpw = 4 / S, tile0 = blockIdx.x * tpw;
    wg_matvec<DT>(L.gate_up, tile0, S, s.act, kp, s.red, s.yv);
    if (threadIdx.x < tpw * 8) {
        const int p = threadIdx.x >> 4, r16 = threadIdx.x & 15;
        const float g = s.yv[(2 * p) * 16 + r16], u = s.yv[(2 * p + 1) * 16 + r16];
        const int r = (tile0 / 2 + p) * RT + r16;
        if (r < M.ffn) M.h[r] = silu_mul(u, g);
    }
}

// Prep of h + down rows + residual add (engine.c:272-275). The last layer of a step without the head
// advances the position (nothing in this kernel reads it).
template <int DT>
__global__ void __launch_bounds__(NT) k_down(l3m_dmodel M, l3m_dlayer L, int S, int advance) {
    extern __shared__ __align__(16) uint8_t smem[];
    Smem s = carve(smem, DT, M.ffn);
    const int kp = kpad(M.ffn);
    const float *h = M.h;
    stage_x(s.xs, [&](int i) { return h[i]; }, M.ffn, kp, nullptr, 0.f, s.scr);
    prep_act<DT>(s.act, s.xs, kp);
    const int tpw = 4 / S, tile0 = blockIdx.x * tpw;
    wg_matvec<DT>(L.down, tile0, S, s.act, kp, s.red, s.yv);
    if (threadIdx.x < tpw * 16) {
        const int r = (tile0 + (threadIdx.x >> 4)) * RT + (threadIdx.x & 15);
        if (r < M.dim) M.x[r] += s.yv[threadIdx.x];
    }
    if (advance && blockIdx.x == 0 && threadIdx.x == 0) *M.pos += 1;
}

// Final RMSNorm + prep + head rows -> logits slot, then the greedy argmax (engine.c:277-301): each
// workgroup reduces its rows; the last workgroup to finish reduces the partials in index order,
// writes tokens[pos + 1], resets the counter and advances pos.
template <int DT>
__global__ void __launch_bounds__(NT) k_head(l3m_dmodel M, int S, int advance) {
    extern __shared__ __align__(16) uint8_t smem[];
    Smem s = carve(smem, DT, M.dim);
    const int kp = kpad(M.dim), pos = *M.pos;
    const float *x = M.x;
    stage_x(s.xs, [&](int i) { return x[i]; }, M.dim, kp, M.norm, M.eps, s.scr);
    prep_act<DT>(s.act, s.xs, kp);
    const int tpw = 4 / S, tile0 = blockIdx.x * tpw;
    wg_matvec<DT>(M.head, tile0, S, s.act, kp, s.red, s.yv);
    float *lg = M.logits + (size_t)(pos % M.nslots) * M.vocab;
    float v = -INFINITY;
    int idx = 0x7FFFFFFF;
    if (threadIdx.x < tpw * 16) {
        const int r = (tile0 + (threadIdx.x >> 4)) * RT + (threadIdx.x & 15);
        if (r < M.vocab) { lg[r] = s.yv[threadIdx.x]; v = s.yv[threadIdx.x]; idx = r; }
    }
    wg_argmax(v, idx, s.scr, s.iscr);
    __shared__ int last;
    if (threadIdx.x == 0) {
        M.part_val[blockIdx.x] = v;
        M.part_idx[blockIdx.x] = idx;
        __threadfence();
        last = atomicAdd(M.done, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    v = -INFINITY;
    idx = 0x7FFFFFFF;
    for (int w = threadIdx.x; w < (int)gridDim.x; w += NT) {
        const float pv = __hip_atomic_load(M.part_val + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int pi = __hip_atomic_load(M.part_idx + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        better(v, idx, pv, pi);
    }
    wg_argmax(v, idx, s.scr, s.iscr);
    if (threadIdx.x == 0) {
        if (advance) {
            M.tokens[pos + 1] = idx == 0x7FFFFFFF ? 0 : idx;
            *M.pos = pos + 1;
        }
        *M.done = 0;
    }
}

// ----------------------------------------------------------------------------------------- runtime

char g_err[512];
int g_has_err;
hipStream_t g_stream;
int g_ready = -1;
char g_name[128];

int fail(const char *what, hipError_t e) {
    if (!g_has_err) {
        snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e));
        g_has_err = 1;
        fprintf(stderr, "l3m: hip: %s\n", g_err);
    }
    return -1;
}
int fail_msg(const char *msg) {
    if (!g_has_err) {
        snprintf(g_err, sizeof g_err, "%s", msg);
        g_has_err = 1;
        fprintf(stderr, "l3m: hip: %s\n", g_err);
    }
    return -1;
}
#define CK(call) do { hipError_t e_ = (call); if (e_ != hipSuccess) return fail(#call, e_); } while (0)
#define CKL(what) do { hipError_t e_ = hipGetLastError(); if (e_ != hipSuccess) return fail(what, e_); } while (0)

hipStream_t as_stream(void *s) { return s ? (hipStream_t)s : g_stream; }

#define DISPATCH(dt, F, ...) \
    switch (dt) { \
    case L3M_F32: F<L3M_F32>(__VA_ARGS__); break; \
    case L3M_BF16: F<L3M_BF16>(__VA_ARGS__); break; \
    case L3M_Q8_0: F<L3M_Q8_0>(__VA_ARGS__); break; \
    case L3M_Q4_0: F<L3M_Q4_0>(__VA_ARGS__); break; \
    case L3M_MXFP4: F<L3M_MXFP4>(__VA_ARGS__); break; \
    default: return fail_msg("bad dtype"); }

template <int DT> void launch_prep(const float *x, int k, void *act, hipStream_t st) {
    hipLaunchKernelGGL(k_prep<DT>, dim3(1), dim3(NT), smem_bytes(DT, k), st, x, k, (uint8_t *)act);
}
template <int DT> void launch_gemv(const l3m_dmat &m, const void *act, int k, float *y, int S, hipStream_t st) {
    const int grid = (m.tiles + 4 / S - 1) / (4 / S);
    hipLaunchKernelGGL(k_gemv<DT>, dim3(grid), dim3(NT), smem_bytes(DT, k), st, m, (const uint8_t *)act, k, y, S);
}
template <int DT> void launch_qkv(const l3m_dmodel &M, const l3m_dlayer &L, int layer, hipStream_t st) {
    const int S = pick_split(L.qkv.nb), grid = (L.qkv.tiles + 4 / S - 1) / (4 / S);
    hipLaunchKernelGGL(k_qkv<DT>, dim3(grid), dim3(NT), smem_bytes(DT, M.dim), st, M, L, layer, layer == 0, S);
}
template <int DT> void launch_wo(const l3m_dmodel &M, const l3m_dlayer &L, hipStream_t st) {
    const int S = pick_split(L.wo.nb), grid = (L.wo.tiles + 4 / S - 1) / (4 / S);
    hipLaunchKernelGGL(k_wo<DT>, dim3(grid), dim3(NT), smem_bytes(DT, M.dim), st, M, L, S);
}
template <int DT> void launch_ffn(const l3m_dmodel &M, const l3m_dlayer &L, hipStream_t st) {
    const int S = L.gate_up.nb >= 8 ? 2 : 1, grid = L.gate_up.tiles / (4 / S) + (L.gate_up.tiles % (4 / S) ? 1 : 0);
    hipLaunchKernelGGL(k_ffn<DT>, dim3(grid), dim3(NT), smem_bytes(DT, M.dim), st, M, L, S);
}
template <int DT> void launch_down(const l3m_dmodel &M, const l3m_dlayer &L, int advance, hipStream_t st) {
    const int S = pick_split(L.down.nb), grid = (L.down.tiles + 4 / S - 1) / (4 / S);
    hipLaunchKernelGGL(k_down<DT>, dim3(grid), dim3(NT), smem_bytes(DT, M.ffn), st, M, L, S, advance);
}
template <int DT> void launch_head(const l3m_dmodel &M, int advance, hipStream_t st) {
    const int S = pick_split(M.head.nb), grid = (M.head.tiles + 4 / S - 1) / (4 / S);
    hipLaunchKernelGGL(k_head<DT>, dim3(grid), dim3(NT), smem_bytes(DT, M.dim), st, M, S, advance);
}
void launch_attend(const l3m_dmodel &M, int l, hipStream_t st) {
    const size_t sm = 4 * ((size_t)M.hd + ((M.ctx + 4) & ~3) + NT + 8);
    hipLaunchKernelGGL(k_attend, dim3(M.n_heads), dim3(NT), sm, st, M.attn, (const float *)M.q,
                       (const uint16_t *)(M.kc + (size_t)l * M.n_kv * M.ctx * M.hd),
                       (const uint16_t *)(M.vc + (size_t)l * M.n_kv * M.ctx * M.hd), 0, (const int *)M.pos, M.hd, M.hd,
                       M.n_heads / M.n_kv, (size_t)M.ctx * M.hd);
}

}  // namespace

// =============================================================================================== C ABI

struct l3m_graphs {
    hipGraph_t g[2];
    hipGraphExec_t e[2];
};

extern "C" {

int l3m_dev_init(void) {
    if (g_ready >= 0) return g_ready ? 0 : -1;
    g_ready = 0;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n < 1) { fail_msg("no HIP device"); return -1; }
    hipDeviceProp_t p;
    CK(hipGetDeviceProperties(&p, 0));
    snprintf(g_name, sizeof g_name, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    if (strncmp(p.gcnArchName, "gfx950", 6)) {
        char msg[256];
        snprintf(msg, sizeof msg, "device 0 is %s; this build targets gfx950", p.gcnArchName);
        return fail_msg(msg);
    }
    CK(hipSetDevice(0));
    CK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    hipLaunchKernelGGL(k_dummy, dim3(1), dim3(NT), 0, g_stream);
    CKL("first launch");
    CK(hipStreamSynchronize(g_stream));
    g_ready = 1;
    return 0;
}

const char *l3m_dev_error(void) { return g_has_err ? g_err : NULL; }
void l3m_dev_clear_error(void) { g_has_err = 0; g_err[0] = 0; }
const char *l3m_dev_name(void) { return g_name; }
void *l3m_dev_stream(void) { return (void *)g_stream; }

void *l3m_dev_alloc(size_t bytes) {
    void *p = NULL;
    if (l3m_dev_init()) return NULL;
    if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) { fail_msg("hipMalloc failed"); return NULL; }
    if (hipMemsetAsync(p, 0, bytes ? bytes : 16, g_stream) != hipSuccess || hipStreamSynchronize(g_stream) != hipSuccess) {
        (void)hipFree(p);
        fail_msg("hipMemset failed");
        return NULL;
    }
    return p;
}
void l3m_dev_free(void *p) { if (p) (void)hipFree(p); }
// Copies run on the library's stream, after the work already queued there, and complete before returning.
int l3m_dev_upload(void *dst, const void *src, size_t bytes) {
    if (l3m_dev_init()) return -1;
    CK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    CK(hipStreamSynchronize(g_stream));
    return 0;
}
int l3m_dev_download(void *dst, const void *src, size_t bytes) {
    if (l3m_dev_init()) return -1;
    CK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    CK(hipStreamSynchronize(g_stream));
    return 0;
}
int l3m_dev_sync(void) {
    if (l3m_dev_init()) return -1;
    CK(hipStreamSynchronize(g_stream));
    return 0;
}

size_t l3m_act_bytes(int dtype, int k) { return act_size(dtype, k); }

int l3m_k_prep(int dtype, const float *x, int k, void *act, void *stream) {
    if (k < 1 || dtype < 0 || dtype >= L3M_NDTYPES || smem_bytes(dtype, k) > LDS_MAX) return fail_msg("prep: k out of range for this dtype");
    hipStream_t st = as_stream(stream);
    DISPATCH(dtype, launch_prep, x, k, act, st);
    CKL("k_prep");
    return 0;
}

int l3m_k_gemv(const l3m_dmat *m, const void *act, int k, float *y, void *stream) {
    if (k < 1 || m->dtype < 0 || m->dtype >= L3M_NDTYPES || kpad(k) / 32 != m->nb || m->tiles != (m->rows + 15) / 16 || m->rows < 1)
        return fail_msg("gemv: shape does not match the matrix");
    if (smem_bytes(m->dtype, k) > LDS_MAX) return fail_msg("gemv: k too large for this dtype");
    hipStream_t st = as_stream(stream);
    const int S = pick_split(m->nb);
    DISPATCH(m->dtype, launch_gemv, *m, act, k, y, S, st);
    CKL("k_gemv");
    return 0;
}

int l3m_k_attend(float *out, const float *q, const uint16_t *k, const uint16_t *v, int pos, int hd, int stride, void *stream) {
    if (pos < 0 || hd < 8 || hd % 8 || hd > NT || stride < hd || stride % 8) return fail_msg("attend: bad shape");
    const size_t sm = 4 * ((size_t)hd + ((pos + 4) & ~3) + NT + 8);
    if (sm > LDS_MAX) return fail_msg("attend: pos too large");
    hipLaunchKernelGGL(k_attend, dim3(1), dim3(NT), sm, as_stream(stream), out, q, k, v, pos, (const int *)nullptr, hd, stride, 1, (size_t)0);
    CKL("k_attend");
    return 0;
}

int l3m_k_rmsnorm(float *y, const float *x, const float *w, int n, float eps, void *stream) {
    if (n < 1 || 4 * ((size_t)kpad(n) + 8) > LDS_MAX) return fail_msg("rmsnorm: n out of range");
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(NT), 4 * ((size_t)kpad(n) + 8), as_stream(stream), y, x, w, n, eps);
    CKL("k_rmsnorm");
    return 0;
}

int l3m_k_rope(float *v, int n_heads, int hd, int pos, const float *table, void *stream) {
    const int n = n_heads * hd;
    if (n < 2 || hd % 2) return fail_msg("rope: bad shape");
    hipLaunchKernelGGL(k_rope, dim3((n + NT - 1) / NT), dim3(NT), 0, as_stream(stream), v, n, hd, table + (size_t)pos * hd);
    CKL("k_rope");
    return 0;
}

int l3m_k_silu_mul(float *h, const float *g, int n, void *stream) {
    hipLaunchKernelGGL(k_silu_mul, dim3((n + NT - 1) / NT), dim3(NT), 0, as_stream(stream), h, g, n);
    CKL("k_silu_mul");
    return 0;
}

int l3m_k_argmax(const float *x, int n, int32_t *out, void *stream) {
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(NT), 0, as_stream(stream), x, n, out);
    CKL("k_argmax");
    return 0;
}

int l3m_step_enqueue(const l3m_dmodel *M, const l3m_dlayer *layers, int with_head, void *stream) {
    hipStream_t st = as_stream(stream);
    const int dt = layers[0].qkv.dtype;
    for (int l = 0; l < M->n_layers; l++) {
        const l3m_dlayer &L = layers[l];
        DISPATCH(dt, launch_qkv, *M, L, l, st);
        launch_attend(*M, l, st);
        DISPATCH(dt, launch_wo, *M, L, st);
        DISPATCH(dt, launch_ffn, *M, L, st);
        DISPATCH(dt, launch_down, *M, L, !with_head && l == M->n_layers - 1, st);
    }
    if (with_head) DISPATCH(M->head.dtype, launch_head, *M, 1, st);
    CKL("decode step");
    return 0;
}

l3m_graphs *l3m_graphs_build(const l3m_dmodel *M, const l3m_dlayer *layers) {
    l3m_graphs *g = (l3m_graphs *)calloc(1, sizeof *g);
    if (!g) return NULL;
    for (int w = 0; w < 2; w++) {
        if (hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal) != hipSuccess) { fail_msg("graph capture"); goto bad; }
        int rc = l3m_step_enqueue(M, layers, w, g_stream);
        if (hipStreamEndCapture(g_stream, &g->g[w]) != hipSuccess || rc) { fail_msg("graph capture"); goto bad; }
        if (hipGraphInstantiate(&g->e[w], g->g[w], NULL, NULL, 0) != hipSuccess) { fail_msg("graph instantiate"); goto bad; }
    }
    return g;
bad:
    l3m_graphs_free(g);
    return NULL;
}

int l3m_graphs_launch(l3m_graphs *g, int with_head, void *stream) {
    CK(hipGraphLaunch(g->e[with_head ? 1 : 0], as_stream(stream)));
    return 0;
}

// Average microseconds per launch over `iters` launches, timed with events on the library stream.
static double time_launches(int iters, int (*launch)(void *ctx, int i), void *ctx) {
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) { fail_msg("hipEventCreate"); return -1; }
    double us = -1;
    int rc = launch(ctx, 0);                                   // untimed first launch
    if (!rc && hipEventRecord(a, g_stream) == hipSuccess) {
        for (int i = 0; i < iters && !rc; i++) rc = launch(ctx, i);
        float ms = 0;
        if (!rc && hipEventRecord(b, g_stream) == hipSuccess && hipEventSynchronize(b) == hipSuccess &&
            hipEventElapsedTime(&ms, a, b) == hipSuccess)
            us = 1e3 * ms / iters;
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return rc ? -1 : us;
}

struct GemvCtx { const l3m_dmat *mats; int n; const void *act; int k; float *y; };
static int gemv_one(void *c, int i) {
    GemvCtx *g = (GemvCtx *)c;
    return l3m_k_gemv(&g->mats[i % g->n], g->act, g->k, g->y, g_stream);
}

double l3m_time_gemv(const l3m_dmat *mats, int n_mats, const void *act, int k, float *y, int iters) {
    if (l3m_dev_init() || n_mats < 1 || iters < 1) return -1;
    GemvCtx c{mats, n_mats, act, k, y};
    return time_launches(iters, gemv_one, &c);
}

struct StepCtx { const l3m_dmodel *M; const l3m_dlayer *L; int kind, layer; };
static int step_one(void *c, int) {
    StepCtx *s = (StepCtx *)c;
    const l3m_dmodel &M = *s->M;
    const l3m_dlayer &L = s->L[s->layer];
    const int dt = L.qkv.dtype;
    hipStream_t st = g_stream;
    switch (s->kind) {
    case 0: DISPATCH(dt, launch_qkv, M, L, s->layer, st); break;
    case 1: launch_attend(M, s->layer, st); break;
    case 2: DISPATCH(dt, launch_wo, M, L, st); break;
    case 3: DISPATCH(dt, launch_ffn, M, L, st); break;
    case 4: DISPATCH(dt, launch_down, M, L, 0, st); break;
    case 5: DISPATCH(M.head.dtype, launch_head, M, 0, st); break;
    default: return fail_msg("bad kernel kind");
    }
    CKL("timed kernel");
    return 0;
}

double l3m_time_step_kernel(const l3m_dmodel *M, const l3m_dlayer *layers, int kind, int layer, int iters) {
    if (l3m_dev_init() || layer < 0 || layer >= M->n_layers || iters < 1) return -1;
    StepCtx c{M, layers, kind, layer};
    return time_launches(iters, step_one, &c);
}

void l3m_graphs_free(l3m_graphs *g) {
    if (!g) return;
    for (int w = 0; w < 2; w++) {
        if (g->e[w]) (void)hipGraphExecDestroy(g->e[w]);
        if (g->g[w]) (void)hipGraphDestroy(g->g[w]);
    }
    free(g);
}

}  // extern "C"
