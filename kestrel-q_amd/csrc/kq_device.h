/*
 * kq_device.h — device helpers shared by the gfx950 kernels.
 *
 * Every kernel file is compiled with -ffp-contract=off: products and sums
 * that must match the CPU reference bit for bit (block decode, router dot,
 * softmax, top-k weights) are separately rounded; fused multiply-adds are
 * written explicitly (fmaf) only where the result is compared by tolerance.
 */
#ifndef KQ_DEVICE_H
#define KQ_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

/* Device status word bits (OR-ed by kernels, read by the host after sync). */
#define KQ_DEV_MALFORMED 1u  /* non-finite block scale -> MALFORMED_QUANTIZED_DATA */
#define KQ_DEV_NUMERIC 2u    /* non-finite result -> NUMERIC_DOMAIN */
#define KQ_DEV_INPUT 4u      /* non-finite input (checked first by the
                                reference) -> NUMERIC_DOMAIN */

#define KQ_WAVE 64

__device__ __forceinline__ void kq_flag(uint32_t *status, uint32_t bits) {
    atomicOr(status, bits);
}

__device__ __forceinline__ float kq_bits_f32(uint32_t u) {
    return __uint_as_float(u);
}

/* Exact binary16 -> binary32 (src/kq_numeric.c:58-82). A subnormal half
 * m * 2^-24 (m < 1024) is produced by one exact binary32 multiply; normal,
 * zero, Inf and NaN patterns by re-biasing the fields. */
__device__ __forceinline__ float kq_f16_to_f32(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t f = h & 0x3ffu;
    if (e == 0u) {
        float v = (float)f * 5.9604644775390625e-08f; /* 2^-24, exact */
        return __uint_as_float(__float_as_uint(v) | sign);
    }
    if (e == 31u) return __uint_as_float(sign | 0x7f800000u | (f << 13));
    return __uint_as_float(sign | ((e + 112u) << 23) | (f << 13));
}

__device__ __forceinline__ bool kq_isfinite(float v) {
    return (__float_as_uint(v) & 0x7f800000u) != 0x7f800000u;
}

/*
 * expf with the bits of glibc 2.35's x86-64 expf, which the reference calls
 * through libm (src/kq_numeric.c:628-638, :776-813). Method (ARM
 * optimized-routines): x*32/ln2 = k + r, 2^(k/32) from a 32-entry table, a
 * cubic in r, binary64 with fused multiply-adds (v_fma_f64 is IEEE fused on
 * gfx950, as fma() is on the host), one final rounding to binary32.
 */
__constant__ static const uint64_t kq_exp2_tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL,
    0x3fef9301d0125b51ULL, 0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL,
    0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL, 0x3fef06fe0a31b715ULL,
    0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL,
    0x3feea47eb03a5585ULL, 0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL,
    0x3feea11473eb0187ULL, 0x3feea589994cce13ULL, 0x3feeace5422aa0dbULL,
    0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL,
    0x3fef3720dcef9069ULL, 0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL,
    0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

__device__ __forceinline__ float kq_expf(float x) {
    uint32_t ux = __float_as_uint(x);
    uint32_t top = (ux >> 20) & 0x7ffu;
    if (top >= 0x42bu) {
        if (ux == 0xff800000u) return 0.0f;
        if (top >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    double xd = (double)x;
    double z = inv_ln2_n * xd;
    double kd = z + 0x1.8p+52;
    uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= 0x1.8p+52;
    double r = __fma_rn(inv_ln2_n, xd, -kd);
    uint64_t t = kq_exp2_tab[ki % 32u] + (ki << 47);
    double s = __longlong_as_double((long long)t);
    double p = __fma_rn(0x1.c6af84b912394p-5 / 32768.0, r, 0x1.ebfce50fac4f3p-3 / 1024.0);
    double r2 = r * r;
    double y = __fma_rn(0x1.62e42ff0c52d6p-1 / 32.0, r, 1.0);
    y = __fma_rn(p, r2, y);
    y = y * s;
    return (float)y;
}

/* src/kq_numeric.c:628-638: sign-stable logistic. */
__device__ __forceinline__ float kq_sigmoid(float x) {
    if (x >= 0.0f) {
        float e = kq_expf(-x);
        return 1.0f / (1.0f + e);
    }
    float e = kq_expf(x);
    return e / (1.0f + e);
}

/* src/kq_numeric.c:690-720: silu(g) = g * sigmoid(g), then * up. */
__device__ __forceinline__ float kq_swiglu(float g, float u) {
    float s = kq_sigmoid(g);
    float silu = g * s;
    return silu * u;
}

/* Q4_K/Q5_K 6-bit scale and min for sub-block j (src/kq_numeric.c:161-174),
 * from the 12 packed bytes held little-endian in three dwords. */
__device__ __forceinline__ uint32_t kq_byte(uint32_t w0, uint32_t w1,
                                            uint32_t w2, uint32_t i) {
    uint32_t w = i < 4u ? w0 : (i < 8u ? w1 : w2);
    return (w >> (8u * (i & 3u))) & 0xffu;
}

__device__ __forceinline__ void kq_k_scale(uint32_t j, uint32_t w0, uint32_t w1,
                                           uint32_t w2, uint32_t *sc,
                                           uint32_t *mn) {
    if (j < 4u) {
        *sc = kq_byte(w0, w1, w2, j) & 63u;
        *mn = kq_byte(w0, w1, w2, j + 4u) & 63u;
    } else {
        *sc = (kq_byte(w0, w1, w2, j + 4u) & 15u) |
              ((kq_byte(w0, w1, w2, j - 4u) >> 6) << 4);
        *mn = (kq_byte(w0, w1, w2, j + 4u) >> 4) |
              ((kq_byte(w0, w1, w2, j) >> 6) << 4);
    }
}

/*
 * Byte loads from addresses that are only 2-byte aligned (Q8_0 blocks are
 * 34 B and Q6_K blocks 210 B, so a block can start at 2 mod 4). The dwords
 * covering the span are read at 4-byte aligned addresses and re-aligned with
 * a byte funnel shift. `end` is one past the last valid byte of the buffer:
 * no dword that starts at or beyond it is read, and the final dword is
 * replaced by a 16-bit read when only two of its bytes are in bounds.
 */
__device__ __forceinline__ uint32_t kq_ld32_guard(const uint8_t *p,
                                                  const uint8_t *end) {
    if (p + 4 <= end) return *(const uint32_t *)p;
    if (p + 2 <= end) return (uint32_t)(*(const uint16_t *)p);
    return 0u;
}

__device__ __forceinline__ uint32_t kq_align2(uint32_t hi, uint32_t lo,
                                              uint32_t shift_bytes) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift_bytes);
}

/* 8 bytes at a 2-byte aligned address a (a < end). */
__device__ __forceinline__ uint2 kq_load8_u2a(const uint8_t *a,
                                              const uint8_t *end) {
    uintptr_t ua = (uintptr_t)a;
    const uint8_t *base = (const uint8_t *)(ua & ~(uintptr_t)3);
    uint32_t sh = (uint32_t)(ua & 3u);
    uint32_t d0 = *(const uint32_t *)base;
    uint32_t d1 = *(const uint32_t *)(base + 4);
    uint32_t d2 = sh ? kq_ld32_guard(base + 8, end) : 0u;
    uint2 r;
    r.x = kq_align2(d1, d0, sh);
    r.y = kq_align2(d2, d1, sh);
    return r;
}

/* 4 bytes at a 2-byte aligned address a. */
__device__ __forceinline__ uint32_t kq_load4_u2a(const uint8_t *a,
                                                 const uint8_t *end) {
    uintptr_t ua = (uintptr_t)a;
    const uint8_t *base = (const uint8_t *)(ua & ~(uintptr_t)3);
    uint32_t sh = (uint32_t)(ua & 3u);
    uint32_t d0 = *(const uint32_t *)base;
    uint32_t d1 = sh ? kq_ld32_guard(base + 4, end) : 0u;
    return kq_align2(d1, d0, sh);
}

/* Wave-wide sum over groups of G consecutive lanes (G power of two <= 64);
 * every lane of a group receives the group's sum. */
template <int G>
__device__ __forceinline__ float kq_group_sum(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, KQ_WAVE);
    return v;
}

#endif
