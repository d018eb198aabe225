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

// Reads through explicit global (address space 1) pointers: pointers taken from descriptors in device
// memory would otherwise be flat, and flat loads also count against the LDS wait counter, so every LDS
// barrier would wait for the weight stream in flight.
#define GLOBAL __attribute__((address_space(1)))
template <class T> __device__ __forceinline__ const GLOBAL T *gp(const void *p) { return (const GLOBAL T *)p; }
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldg16(const void *p, size_t i) {
    const u32x4 v = gp<u32x4>(p)[i];
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 ldg16f(const void *p, size_t i) {
    const f32x4 v = gp<f32x4>(p)[i];
    return make_float4(v.x, v.y, v.z, v.w);
}

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
    case L3M_F32:  return gp<float>(m.q)[slot * 32 + j];
    case L3M_BF16: return bf16_f32(gp<uint16_t>(m.q)[slot * 32 + j]);
    case L3M_Q8_0: return f16_f32(gp<uint16_t>(m.s)[slot]) * (float)gp<int8_t>(m.q)[slot * 32 + j];
    default: {
        const uint8_t byte = gp<uint8_t>(m.q)[slot * 16 + (j & 15)];
        const int n = j < 16 ? byte & 15 : byte >> 4;
        if (m.dtype == L3M_Q4_0) return f16_f32(gp<uint16_t>(m.s)[slot]) * (float)(n - 8);
        const int8_t e2m1x2[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
        return e8m0_half(gp<uint8_t>(m.s)[slot]) * (float)e2m1x2[n];
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

// ------------------------------------------------------------------------------ decode step kernels
//
// Per layer: kernel A (one workgroup per head group) = norm + prep + qkv rows + RoPE + KV write +
// attention + the group's Wo column slice; kernel B (one workgroup per FFN chunk) = norm + prep + gate/up
// rows + SiLU + prep + the chunk's Wdown column slice. Each writes a partial residual (po, pd); the next
// kernel adds the partials in a fixed order, so results are run-to-run identical.
//
// Every one of the 16 wavefronts of a workgroup runs the same sequence: issue its share of the loads of
// the incoming partial residuals, then issue its share of the weights (nothing depends on them), then
// wait for the partials only (loads complete in order), build the normalized activation in LDS, and
// only then consume the weights. So the weight stream overlaps the prologue instead of following it.

constexpr int NTE = 1024, NWE = NTE / 64;

// Weight slots per lane: a step kernel streams matrix A (qkv, gate/up, head rows) and matrix B (Wo,
// Wdown columns), each through its own register array; 64 (tile, block) pairs per slot and workgroup.
template <int DT> constexpr int nslot_a() { return DT == L3M_F32 ? 1 : DT == L3M_BF16 ? 2 : DT == L3M_Q8_0 ? 5 : 6; }
template <int DT> constexpr int nslot_b() { return DT == L3M_F32 ? 1 : DT == L3M_BF16 ? 1 : 3; }

template <int DT, int NS>
struct Pref {
    uint4 w[NS][qbytes(DT) / 16];
    uint32_t sc[NS];
};

// Slot s of this lane holds pair p = (wave + (s0 + s) * NWE) * 4 + sub of m, a pair being (tile, block)
// = (p / nb, p % nb) and the lane reading row (lane & 15) of it: 4 consecutive pairs = one contiguous
// 64 * QBYTES run per wavefront. Loads are unconditional (past the end they repeat the last pair) so that
// no branch ties a load to its use.
template <int DT, int NS>
__device__ __forceinline__ void pref_load(Pref<DT, NS> &pf, const l3m_dmat &m, int s0) {
    constexpr int QBY = qbytes(DT), SBY = sbytes(DT), NV = QBY / 16;
    const int wave = threadIdx.x >> 6, sub = (threadIdx.x >> 4) & 3, row = threadIdx.x & 15, n = m.tiles * m.nb;
    if (n <= 0) return;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        int p = (wave + (s0 + s) * NWE) * 4 + sub;
        p = p < n ? p : n - 1;
        const size_t slot = (size_t)p * 16 + row;
#pragma unroll
        for (int v = 0; v < NV; v++) pf.w[s][v] = ldg16(m.q, slot * NV + v);
        if constexpr (SBY == 2) pf.sc[s] = gp<uint16_t>(m.s)[slot];
        if constexpr (SBY == 1) pf.sc[s] = gp<uint8_t>(m.s)[slot];
        if constexpr (SBY == 0) pf.sc[s] = 0;
    }
}

// res[pair * 16 + row] for this lane's slots.
template <int DT, int NS>
__device__ __forceinline__ void pref_compute(Pref<DT, NS> &pf, const l3m_dmat &m, int s0, const uint8_t *act, int kp, float *res) {
    const int wave = threadIdx.x >> 6, sub = (threadIdx.x >> 4) & 3, row = threadIdx.x & 15, n = m.tiles * m.nb;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        // Pin the loaded registers here: otherwise the compiler hoists their first use (the f16 scale
        // conversion) up to the loads, and every wavefront stalls on its first load at entry.
        asm volatile("" : "+v"(pf.sc[s]));
#pragma unroll
        for (int v = 0; v < qbytes(DT) / 16; v++) asm volatile("" : "+v"(pf.w[s][v].x), "+v"(pf.w[s][v].y), "+v"(pf.w[s][v].z), "+v"(pf.w[s][v].w));
        const int p = (wave + (s0 + s) * NWE) * 4 + sub;
        if (p < n) res[p * 16 + row] = block_fma<DT>(0.f, pf.w[s], pf.sc[s], act, kp, p % m.nb);
    }
}

// All pairs of m: the prefetched batch, then any further batches (loaded here).
template <int DT, int NS>
__device__ void mv(Pref<DT, NS> &pf, const l3m_dmat &m, const uint8_t *act, int kp, float *res) {
    pref_compute<DT, NS>(pf, m, 0, act, kp, res);
    for (int s0 = NS; s0 * NWE * 4 < m.tiles * m.nb; s0 += NS) {
        pref_load<DT, NS>(pf, m, s0);
        pref_compute<DT, NS>(pf, m, s0, act, kp, res);
    }
}

// out[r] = sum over the row's blocks, in block order (all threads), for r < rows.
__device__ void rows_sum(const l3m_dmat &m, const float *res, float *out, int rows) {
    for (int i = threadIdx.x; i < rows; i += NTE) {
        const float *p = res + (size_t)(i >> 4) * m.nb * 16 + (i & 15);
        float y = p[0];
        for (int b = 1; b < m.nb; b++) y += p[b * 16];
        out[i] = y;
    }
}

// Workgroup-wide reductions in a fixed order; scr: 32 words of LDS.
__device__ float wge_sum(float v, float *scr) {
    for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scr[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = scr[0];
    for (int w = 1; w < NWE; w++) t += scr[w];
    return t;
}
__device__ float wge_max(float v, float *scr) {
    for (int o = 32; o; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scr[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = scr[0];
    for (int w = 1; w < NWE; w++) t = fmaxf(t, scr[w]);
    return t;
}
__device__ void wge_argmax(float &v, int &i, float *scr) {
    int *si = (int *)(scr + 16);
    for (int o = 32; o; o >>= 1) {
        const float v2 = __shfl_xor(v, o);
        const int i2 = __shfl_xor(i, o);
        better(v, i, v2, i2);
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { scr[threadIdx.x >> 6] = v; si[threadIdx.x >> 6] = i; }
    __syncthreads();
    v = scr[0]; i = si[0];
    for (int w = 1; w < NWE; w++) better(v, i, scr[w], si[w]);
}

// The incoming residual x = base + parts[0] + ... + parts[n-1] (or, for layer 0, the embedding row of
// tok). Thread t takes float4 column f = t % (dim/4) and the parts of group t / (dim/4); fill_load only
// issues its loads, fill_finish (after the weights are issued) adds them: group sums go through LDS and
// are added in group order.
constexpr int FILL_PER = 8;
struct Fill {
    float4 p[FILL_PER];
    float4 base;
    float e;
};
struct FillGeom {
    int n4, groups, per;
};
__device__ __forceinline__ FillGeom fill_geom(int dim, int nparts) {
    FillGeom g;
    g.n4 = dim / 4;
    g.groups = NTE / g.n4 < 1 ? 1 : NTE / g.n4;
    g.per = (nparts + g.groups - 1) / g.groups;
    if (g.per < 1) g.per = 1;
    return g;
}
// embed (by value: a pointer into the kernel's argument struct would move the whole struct to scratch)
// is read when use_embed is set.
__device__ __forceinline__ void fill_load(Fill &F, const float *base, const float *parts, int nparts, int dim, l3m_dmat embed, bool use_embed, int tok) {
    if (use_embed) {                                         // layer 0: x = dequant(embed[tok]) (engine.c:236)
        F.e = threadIdx.x < dim ? lt_elem(embed, tok, threadIdx.x) : 0.f;
        return;
    }
    const FillGeom G = fill_geom(dim, nparts);
    const int f = threadIdx.x % G.n4, grp = threadIdx.x / G.n4, j0 = grp * G.per;
    if (grp < G.groups && grp == 0) F.base = ldg16f(base, f);
#pragma unroll
    for (int j = 0; j < FILL_PER; j++)
        if (grp < G.groups && j < G.per && j0 + j < nparts) F.p[j] = ldg16f(parts + (size_t)(j0 + j) * dim, f);
}
// xs[0, dim) = x; also stored to keep when given. pbuf: LDS for the group sums (NTE float4). All threads call.
__device__ void fill_finish(Fill &F, float *xs, const float *parts, int nparts, int dim, float4 *pbuf, float *keep, bool embed) {
    if (embed) {
        if (threadIdx.x < dim) { xs[threadIdx.x] = F.e; if (keep) keep[threadIdx.x] = F.e; }
        __syncthreads();
        return;
    }
    const FillGeom G = fill_geom(dim, nparts);
    const int f = threadIdx.x % G.n4, grp = threadIdx.x / G.n4, j0 = grp * G.per;
    if (grp < G.groups) {
        float4 v = grp == 0 ? F.base : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < FILL_PER; j++)
            if (j < G.per && j0 + j < nparts) { v.x += F.p[j].x; v.y += F.p[j].y; v.z += F.p[j].z; v.w += F.p[j].w; }
        for (int j = FILL_PER; j < G.per && j0 + j < nparts; j++) {   // more parts than one batch: in order
            const float4 p = ldg16f(parts + (size_t)(j0 + j) * dim, f);
            v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
        }
        pbuf[grp * G.n4 + f] = v;
    }
    __syncthreads();
    if (threadIdx.x < G.n4) {
        float4 v = pbuf[threadIdx.x];
        for (int g = 1; g < G.groups; g++) {
            const float4 p = pbuf[g * G.n4 + threadIdx.x];
            v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
        }
        ((float4 *)xs)[threadIdx.x] = v;
        if (keep) ((float4 *)keep)[threadIdx.x] = v;
    }
    __syncthreads();
}

// Norm + prep of xs (x in [0, k)): RMSNorm with nw when given (ops.c:13-18), then the activation prep
// (pack.c:101-123) into act, padded to kp. All threads call it.
template <int DT>
__device__ void norm_prep(float *xs, uint8_t *act, int k, int kp, const float *nw, float eps, float *scr) {
    const int tid = threadIdx.x;
    for (int i = k + tid; i < kp; i += NTE) xs[i] = 0.f;
    if (nw) {
        float ss = 0.f;
        for (int i = tid; i < k; i += NTE) ss = fmaf(xs[i], xs[i], ss);
        const float tot = wge_sum(ss, scr);
        const float s = 1.0f / sqrtf(tot / (float)k + eps);
        for (int i = tid; i < k; i += NTE) xs[i] = xs[i] * s * nw[i];
    }
    __syncthreads();
    if constexpr (quantized(DT)) {
        const int nb = kp / 32, g = tid >> 3, l = tid & 7;
        float *scale = (float *)(act + kp);
        int *sum = (int *)(act + kp + 4 * nb);
        for (int b = g; b < nb; b += NTE / 8) {
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
        for (int i = tid; i < kp; i += NTE) ((uint16_t *)act)[i] = f32_bf16(xs[i]);
    } else {
        for (int i = tid; i < kp; i += NTE) ((float *)act)[i] = xs[i];
    }
    __syncthreads();
}

// LDS regions of the step kernels (byte offsets, 16-aligned) from the layer geometry. `work` holds the
// prologue's group sums, then the per-pair matvec results, then the attention partials.
struct LdsA { size_t xs, act, work, qkv, kv, sc, att, act2, scr, kvb, total; };
__host__ __device__ inline size_t work_bytes(size_t pairs) {
    const size_t w = 64 * pairs;
    return align16(w > 16 * (size_t)NTE ? w : 16 * (size_t)NTE);
}
__host__ __device__ inline LdsA lds_a(int dt, int dim, int ctx, int hd, const l3m_dgroup &g, int kv_lds) {
    LdsA L;
    size_t o = 0;
    const size_t pq = (size_t)g.qkv.tiles * g.qkv.nb, pw = (size_t)g.wo.tiles * g.wo.nb;
    L.xs = o;   o += align16(4 * (size_t)kpad(dim));
    L.act = o;  o += align16(act_size(dt, dim));
    L.work = o; o += work_bytes(pq > pw ? pq : pw);
    L.qkv = o;  o += align16(64 * (size_t)g.qkv.tiles);
    L.kv = o;   o += align16(8 * (size_t)g.nkv * hd);
    L.sc = o;   o += align16(4 * (size_t)(ctx + 4));
    L.att = o;  o += align16(4 * (size_t)kpad(g.nq * hd));
    L.act2 = o; o += align16(act_size(dt, g.nq * hd));
    L.scr = o;  o += 4 * 64;
    L.kvb = o;  o += kv_lds ? align16(4 * (size_t)g.nkv * ctx * hd) : 0;   // [K | V][nkv][ctx][hd] bf16
    L.total = o;
    return L;
}
struct LdsB { size_t xs, act, work, gu, h, act2, scr, total; };
__host__ __device__ inline LdsB lds_b(int dt, int dim, const l3m_dchunk &c) {
    LdsB L;
    size_t o = 0;
    const size_t pg = (size_t)c.gate_up.tiles * c.gate_up.nb, pw = (size_t)c.down.tiles * c.down.nb;
    L.xs = o;   o += align16(4 * (size_t)kpad(dim));
    L.act = o;  o += align16(act_size(dt, dim));
    L.work = o; o += work_bytes(pg > pw ? pg : pw);
    L.gu = o;   o += align16(64 * (size_t)c.gate_up.tiles);
    L.h = o;    o += align16(4 * (size_t)kpad(c.nf));
    L.act2 = o; o += align16(act_size(dt, c.nf));
    L.scr = o;  o += 4 * 64;
    L.total = o;
    return L;
}
struct LdsH { size_t xs, act, work, y, scr, total; };
__host__ __device__ inline LdsH lds_h(int dt, int dim, int nb, int tiles_per_wg) {
    LdsH L;
    size_t o = 0;
    L.xs = o;   o += align16(4 * (size_t)kpad(dim));
    L.act = o;  o += align16(act_size(dt, dim));
    L.work = o; o += work_bytes((size_t)tiles_per_wg * nb);
    L.y = o;    o += align16(64 * (size_t)tiles_per_wg);
    L.scr = o;  o += 4 * 64;
    L.total = o;
    return L;
}

// K and V rows 0..pos-1 of the group's kv heads, copied from the cache into LDS [K | V][nkv][ctx][hd] by
// the memory unit (global_load_lds_dwordx4: 64 lanes x 16 bytes into 1 KiB of LDS, no registers).
// Rows up to pos - 1 were written by earlier steps, so the copy can start at the top of the kernel.
__device__ void kv_window_dma(uint16_t *kvb, const l3m_dmodel &M, int layer, int kv0, int nkv, int pos) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const size_t win = (size_t)M.ctx * M.hd, total = (size_t)pos * M.hd * 2;     // bytes per head, K or V
    const int nch = (int)((total + 1023) / 1024), items = 2 * nkv * nch;
    for (int it = wave; it < items; it += NWE) {
        const int which = it / (nkv * nch), rem = it % (nkv * nch), j = rem / nch, c = rem % nch;
        const size_t byte = (size_t)c * 1024 + (size_t)lane * 16;
        const uint16_t *src = (which ? M.vc : M.kc) + ((size_t)layer * M.n_kv + kv0 + j) * win;
        uint8_t *dst = (uint8_t *)(kvb + ((size_t)which * nkv + j) * win) + (size_t)c * 1024;
        if (byte < total)
            __builtin_amdgcn_global_load_lds((const GLOBAL void *)((const uint8_t *)src + byte),
                                             (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
    }
}

// Kernel A: the attention block of one head group (engine.c:236-258).
template <int DT>
__global__ void __launch_bounds__(NTE) k_attn_block(l3m_dmodel M, l3m_dlayer Lw, int layer) {
    extern __shared__ __align__(16) uint8_t smem[];
    const l3m_dgroup G = Lw.groups[blockIdx.x];
    const int tid = threadIdx.x, pos = *M.pos, dim = M.dim, hd = M.hd, kp = kpad(dim);
    const LdsA L = lds_a(DT, dim, M.ctx, hd, G, M.kv_lds);
    float *xs = (float *)(smem + L.xs), *work = (float *)(smem + L.work), *qkv = (float *)(smem + L.qkv);
    float *kvc = (float *)(smem + L.kv), *sc = (float *)(smem + L.sc), *att = (float *)(smem + L.att), *scr = (float *)(smem + L.scr);
    uint8_t *act = smem + L.act, *act2 = smem + L.act2;

    Fill F;
    fill_load(F, M.xb, M.pd, M.n_chunks, dim, M.embed, layer == 0, layer ? 0 : M.tokens[pos]);
    Pref<DT, nslot_a<DT>()> pa;
    Pref<DT, nslot_b<DT>()> pb;
    pref_load<DT, nslot_a<DT>()>(pa, G.qkv, 0);
    pref_load<DT, nslot_b<DT>()>(pb, G.wo, 0);
    fill_finish(F, xs, M.pd, M.n_chunks, dim, (float4 *)work, blockIdx.x == 0 ? M.xa : nullptr, layer == 0);
    uint16_t *kvb = (uint16_t *)(smem + L.kvb);
    if (M.kv_lds) kv_window_dma(kvb, M, layer, G.kv0, G.nkv, pos);   // K, V rows 0..pos-1: no dependence on this step
    norm_prep<DT>(xs, act, dim, kp, Lw.attn_norm, M.eps, scr);

    mv<DT, nslot_a<DT>()>(pa, G.qkv, act, kp, work);
    __syncthreads();
    const int nqd = G.nq * hd, nkd = G.nkv * hd;
    rows_sum(G.qkv, work, qkv, nqd + 2 * nkd);
    __syncthreads();

    // RoPE on q and k: pairs (2i, 2i+1) of each head by the table angle i (ops.c:29-40)
    float rot = 0.f;
    if (tid < nqd + nkd) {
        const int local = tid < nqd ? tid : tid - nqd, i = (local % hd) >> 1;
        const float *cs = M.rope + ((size_t)pos * (hd >> 1) + i) * 2;
        const float a = qkv[tid], b = qkv[tid ^ 1];
        rot = (tid & 1) ? b * cs[1] + a * cs[0] : a * cs[0] - b * cs[1];
    }
    __syncthreads();
    if (tid < nqd + nkd) qkv[tid] = rot;
    __syncthreads();
    // k and v of this position, as the bf16 cache holds them (engine.c:247-248)
    for (int i = tid; i < 2 * nkd; i += NTE) {
        const uint16_t h = f32_bf16(qkv[nqd + i]);
        kvc[i] = bf16_f32(h);
        const int j = i < nkd ? i : i - nkd, kvl = j / hd;
        if (G.write_kv >> kvl & 1u) {
            uint16_t *c = i < nkd ? M.kc : M.vc;
            c[(((size_t)layer * M.n_kv + G.kv0 + kvl) * M.ctx + pos) * hd + j % hd] = h;
        }
    }
    __syncthreads();

    // attention of each query head over positions 0..pos (ops.c:58-73): rows before pos from the LDS
    // window (kv_lds) or from the cache, row pos from kvc
    if (M.kv_lds) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)hd);
    const int hpk = M.n_heads / M.n_kv, groups = NTE / hd, gi = tid / hd, ii = tid % hd, nv = hd / 8;
    const size_t win = (size_t)M.ctx * hd;
    for (int h = 0; h < G.nq; h++) {
        const int kvl = (G.q0 + h) / hpk - G.kv0;
        const float *q = qkv + h * hd;
        const uint16_t *kh = M.kv_lds ? kvb + kvl * win : M.kc + ((size_t)layer * M.n_kv + G.kv0 + kvl) * win;
        const uint16_t *vh = M.kv_lds ? kvb + (G.nkv + kvl) * win : M.vc + ((size_t)layer * M.n_kv + G.kv0 + kvl) * win;
        float mx = -INFINITY;
        for (int t = tid; t <= pos; t += NTE) {
            float dot = 0.f;
            if (t < pos) {
                const uint16_t *kr = kh + (size_t)t * hd;
                for (int v = 0; v < nv; v++) {
                    const uint4 kk = M.kv_lds ? ((const uint4 *)kr)[v] : ldg16(kr, v);
                    const float *qq = q + v * 8;
                    dot = fmaf(qq[0], bf16_f32(kk.x & 0xFFFF), dot); dot = fmaf(qq[1], bf16_f32(kk.x >> 16), dot);
                    dot = fmaf(qq[2], bf16_f32(kk.y & 0xFFFF), dot); dot = fmaf(qq[3], bf16_f32(kk.y >> 16), dot);
                    dot = fmaf(qq[4], bf16_f32(kk.z & 0xFFFF), dot); dot = fmaf(qq[5], bf16_f32(kk.z >> 16), dot);
                    dot = fmaf(qq[6], bf16_f32(kk.w & 0xFFFF), dot); dot = fmaf(qq[7], bf16_f32(kk.w >> 16), dot);
                }
            } else {
                const float *kr = kvc + kvl * hd;
                for (int i = 0; i < hd; i++) dot = fmaf(q[i], kr[i], dot);
            }
            sc[t] = dot * scale;
            mx = fmaxf(mx, dot * scale);
        }
        mx = wge_max(mx, scr);
        float sum = 0.f;
        for (int t = tid; t <= pos; t += NTE) {
            const float e = expf(sc[t] - mx);
            sc[t] = e;
            sum += e;
        }
        sum = wge_sum(sum, scr);
        for (int t = tid; t <= pos; t += NTE) sc[t] = sc[t] / sum;
        __syncthreads();
        float acc = 0.f;
        if (gi < groups)
            for (int t = gi; t <= pos; t += groups) {
                const float v = t == pos ? kvc[nkd + kvl * hd + ii]
                              : bf16_f32(M.kv_lds ? vh[(size_t)t * hd + ii] : gp<uint16_t>(vh)[(size_t)t * hd + ii]);
                acc = fmaf(sc[t], v, acc);
            }
        work[tid] = acc;
        __syncthreads();
        if (tid < hd) {
            float o = work[tid];
            for (int g = 1; g < groups; g++) o += work[g * hd + tid];
            att[h * hd + tid] = o;
        }
        __syncthreads();
    }
    // prep of the group's attention output, then its Wo columns -> the partial residual po[group]
    norm_prep<DT>(att, act2, nqd, kpad(nqd), nullptr, 0.f, scr);
    mv<DT, nslot_b<DT>()>(pb, G.wo, act2, kpad(nqd), work);
    __syncthreads();
    rows_sum(G.wo, work, M.po + (size_t)blockIdx.x * dim, dim);
}

// Kernel B: the FFN block of one chunk of ffn rows (engine.c:259-275). The last layer of a step without
// the head advances the position (nothing in this kernel reads it).
template <int DT>
__global__ void __launch_bounds__(NTE) k_ffn_block(l3m_dmodel M, l3m_dlayer Lw, int advance) {
    extern __shared__ __align__(16) uint8_t smem[];
    const l3m_dchunk C = Lw.chunks[blockIdx.x];
    const int tid = threadIdx.x, dim = M.dim, kp = kpad(dim);
    const LdsB L = lds_b(DT, dim, C);
    float *xs = (float *)(smem + L.xs), *work = (float *)(smem + L.work), *gu = (float *)(smem + L.gu);
    float *h = (float *)(smem + L.h), *scr = (float *)(smem + L.scr);
    uint8_t *act = smem + L.act, *act2 = smem + L.act2;

    Fill F;
    fill_load(F, M.xa, M.po, M.n_groups, dim, M.embed, false, 0);     // x += proj (engine.c:259)
    Pref<DT, nslot_a<DT>()> pa;
    Pref<DT, nslot_b<DT>()> pb;
    pref_load<DT, nslot_a<DT>()>(pa, C.gate_up, 0);
    pref_load<DT, nslot_b<DT>()>(pb, C.down, 0);
    fill_finish(F, xs, M.po, M.n_groups, dim, (float4 *)work, blockIdx.x == 0 ? M.xb : nullptr, false);
    norm_prep<DT>(xs, act, dim, kp, Lw.ffn_norm, M.eps, scr);
    mv<DT, nslot_a<DT>()>(pa, C.gate_up, act, kp, work);
    __syncthreads();
    rows_sum(C.gate_up, work, gu, C.gate_up.rows);
    __syncthreads();
    for (int i = tid; i < C.nf; i += NTE)                           // h = up * silu(gate) (ops.c:49-51)
        h[i] = silu_mul(gu[(2 * (i >> 4) + 1) * 16 + (i & 15)], gu[(2 * (i >> 4)) * 16 + (i & 15)]);
    __syncthreads();
    norm_prep<DT>(h, act2, C.nf, kpad(C.nf), nullptr, 0.f, scr);
    mv<DT, nslot_b<DT>()>(pb, C.down, act2, kpad(C.nf), work);
    __syncthreads();
    rows_sum(C.down, work, M.pd + (size_t)blockIdx.x * dim, dim);
    if (advance && blockIdx.x == 0 && tid == 0) *M.pos += 1;
}

// Final norm + head rows -> logits slot, then the greedy argmax (engine.c:277-301): each workgroup
// reduces its rows; the last workgroup to finish reduces the partials in index order, writes
// tokens[pos + 1], resets the counter and (advance) moves pos on.
template <int DT>
__global__ void __launch_bounds__(NTE) k_head_block(l3m_dmodel M, int advance) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, tpw = M.head_tiles_per_wg, t0 = blockIdx.x * tpw;
    l3m_dmat V = M.head;                                    // this workgroup's tiles of the head
    const int nt = t0 + tpw <= V.tiles ? tpw : V.tiles - t0;
    V.q += (size_t)t0 * V.nb * 16 * qbytes(DT);
    if (sbytes(DT)) V.s += (size_t)t0 * V.nb * 16 * sbytes(DT);
    V.tiles = nt;
    V.rows = nt * 16 < M.vocab - t0 * 16 ? nt * 16 : M.vocab - t0 * 16;
    const int pos = *M.pos, dim = M.dim, kp = kpad(dim);
    const LdsH L = lds_h(DT, dim, M.head.nb, tpw);
    float *xs = (float *)(smem + L.xs), *work = (float *)(smem + L.work), *y = (float *)(smem + L.y), *scr = (float *)(smem + L.scr);
    uint8_t *act = smem + L.act;

    Fill F;
    fill_load(F, M.xb, M.pd, M.n_chunks, dim, M.embed, false, 0);     // x += down (engine.c:275), last layer
    Pref<DT, nslot_a<DT>() + nslot_b<DT>()> pa;
    pref_load<DT, nslot_a<DT>() + nslot_b<DT>()>(pa, V, 0);
    fill_finish(F, xs, M.pd, M.n_chunks, dim, (float4 *)work, nullptr, false);
    norm_prep<DT>(xs, act, dim, kp, M.norm, M.eps, scr);
    mv<DT, nslot_a<DT>() + nslot_b<DT>()>(pa, V, act, kp, work);
    __syncthreads();
    rows_sum(V, work, y, V.rows);
    __syncthreads();
    float *lg = M.logits + (size_t)(pos % M.nslots) * M.vocab + (size_t)t0 * 16;
    float v = -INFINITY;
    int idx = 0x7FFFFFFF;
    if (tid < V.rows) { lg[tid] = y[tid]; v = y[tid]; idx = t0 * 16 + tid; }
    wge_argmax(v, idx, scr);
    __shared__ int last;
    if (tid == 0) {
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
    for (int w = tid; w < (int)gridDim.x; w += NTE) {
        const float pv = __hip_atomic_load(M.part_val + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int pi = __hip_atomic_load(M.part_idx + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        better(v, idx, pv, pi);
    }
    wge_argmax(v, idx, scr);
    if (tid == 0) {
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
unsigned g_lds_max = 65536;

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
// Kernels that take more than 64 KiB of dynamic LDS declare it once.
template <class K> void lds_opt_in(K kernel, unsigned bytes) {
    if (bytes > 65536) (void)hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}
template <int DT> void launch_attn(const l3m_dmodel &M, const l3m_dlayer &L, int layer, hipStream_t st) {
    lds_opt_in(k_attn_block<DT>, M.lds_a);
    hipLaunchKernelGGL(k_attn_block<DT>, dim3(M.n_groups), dim3(NTE), M.lds_a, st, M, L, layer);
}
template <int DT> void launch_ffn(const l3m_dmodel &M, const l3m_dlayer &L, int advance, hipStream_t st) {
    lds_opt_in(k_ffn_block<DT>, M.lds_b);
    hipLaunchKernelGGL(k_ffn_block<DT>, dim3(M.n_chunks), dim3(NTE), M.lds_b, st, M, L, advance);
}
template <int DT> void launch_head(const l3m_dmodel &M, int advance, hipStream_t st) {
    lds_opt_in(k_head_block<DT>, M.lds_h);
    hipLaunchKernelGGL(k_head_block<DT>, dim3(M.head_grid), dim3(NTE), M.lds_h, st, M, advance);
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
    int lds = 0;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, 0) == hipSuccess && lds > 0) g_lds_max = (unsigned)lds;
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
unsigned l3m_dev_lds_max(void) { return l3m_dev_init() ? 65536u : g_lds_max; }
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

unsigned l3m_lds_attn(int dtype, int dim, int ctx, int hd, const l3m_dgroup *g, int kv_lds) { return (unsigned)lds_a(dtype, dim, ctx, hd, *g, kv_lds).total; }
unsigned l3m_lds_ffn(int dtype, int dim, const l3m_dchunk *c) { return (unsigned)lds_b(dtype, dim, *c).total; }
unsigned l3m_lds_head(int dtype, int dim, int nb, int tiles_per_wg) { return (unsigned)lds_h(dtype, dim, nb, tiles_per_wg).total; }
int l3m_step_slots(int dtype, int which) {
    if (which) return dtype == L3M_F32 ? nslot_b<L3M_F32>() : dtype == L3M_BF16 ? nslot_b<L3M_BF16>() : dtype == L3M_Q8_0 ? nslot_b<L3M_Q8_0>() : nslot_b<L3M_Q4_0>();
    return dtype == L3M_F32 ? nslot_a<L3M_F32>() : dtype == L3M_BF16 ? nslot_a<L3M_BF16>() : dtype == L3M_Q8_0 ? nslot_a<L3M_Q8_0>() : nslot_a<L3M_Q4_0>();
}

int l3m_step_enqueue(const l3m_dmodel *M, const l3m_dlayer *layers, int with_head, void *stream) {
    hipStream_t st = as_stream(stream);
    for (int l = 0; l < M->n_layers; l++) {
        DISPATCH(M->body_dtype, launch_attn, *M, layers[l], l, st);
        DISPATCH(M->body_dtype, launch_ffn, *M, layers[l], !with_head && l == M->n_layers - 1, st);
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
    hipStream_t st = g_stream;
    switch (s->kind) {
    case 0: DISPATCH(M.body_dtype, launch_attn, M, s->L[s->layer], s->layer, st); break;
    case 1: DISPATCH(M.body_dtype, launch_ffn, M, s->L[s->layer], 0, st); break;
    case 2: DISPATCH(M.head.dtype, launch_head, M, 0, st); break;
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
