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
#define KQ_DEV_RANGE 8u      /* an index input out of range -> INVALID_ARGUMENT */

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

/* The same conversion in one v_cvt_f32_f16: exact for every finite input,
 * subnormals included (the kernels keep fp16 denormals: float denorm mode
 * 16/64 = 3), but a signalling NaN comes back quiet. For block scales on
 * tolerance-compared paths, where a non-finite scale only raises
 * MALFORMED; bit-exact decode keeps kq_f16_to_f32. */
__device__ __forceinline__ float kq_f16_to_f32_hw(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu));
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

/* The table may also be a copy in LDS (kq_expf_tab): a kernel that keeps
 * its own loads in flight across an activation then reads it without a
 * global load, and without the wait on every outstanding load that a
 * global load's use would bring. */
__device__ __forceinline__ float kq_expf_tab(float x, const uint64_t *tab) {
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
    uint64_t t = tab[ki % 32u] + (ki << 47);
    double s = __longlong_as_double((long long)t);
    double p = __fma_rn(0x1.c6af84b912394p-5 / 32768.0, r, 0x1.ebfce50fac4f3p-3 / 1024.0);
    double r2 = r * r;
    double y = __fma_rn(0x1.62e42ff0c52d6p-1 / 32.0, r, 1.0);
    y = __fma_rn(p, r2, y);
    y = y * s;
    return (float)y;
}

__device__ __forceinline__ float kq_expf(float x) { return kq_expf_tab(x, kq_exp2_tab); }

/* src/kq_numeric.c:628-638: sign-stable logistic. */
__device__ __forceinline__ float kq_sigmoid_tab(float x, const uint64_t *tab) {
    if (x >= 0.0f) {
        float e = kq_expf_tab(-x, tab);
        return 1.0f / (1.0f + e);
    }
    float e = kq_expf_tab(x, tab);
    return e / (1.0f + e);
}
__device__ __forceinline__ float kq_sigmoid(float x) { return kq_sigmoid_tab(x, kq_exp2_tab); }

/* src/kq_numeric.c:690-720: silu(g) = g * sigmoid(g), then * up. */
__device__ __forceinline__ float kq_swiglu_tab(float g, float u, const uint64_t *tab) {
    float s = kq_sigmoid_tab(g, tab);
    float silu = g * s;
    return silu * u;
}
__device__ __forceinline__ float kq_swiglu(float g, float u) { return kq_swiglu_tab(g, u, kq_exp2_tab); }

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

/* Scales and mins of Q4_K sub-blocks 2p and 2p+1 (p = 0..3), without
 * branches (p differs across lanes): the same 6-bit fields as kq_k_scale
 * (src/kq_numeric.c:161-174), from the 12 packed bytes q[0..11] in dwords
 * w0 = q[0..3], w1 = q[4..7], w2 = q[8..11]. */
__device__ __forceinline__ void kq_k_scale_pair(uint32_t p, uint32_t w0, uint32_t w1,
                                                uint32_t w2, uint32_t *s0, uint32_t *m0,
                                                uint32_t *s1, uint32_t *m1) {
    const uint32_t sh = 16u * (p & 1u);
    const uint32_t u = w0 >> sh; /* q[2(p&1)], q[2(p&1)+1] */
    const uint32_t z = w1 >> sh; /* q[4+2(p&1)], q[5+2(p&1)] */
    const uint32_t w = w2 >> sh; /* q[8+2(p&1)], q[9+2(p&1)] */
    /* all ones for sub-blocks 0..3; a bitwise select, which the compiler
     * keeps as v_bfi_b32 where a ?: becomes a divergent branch */
    const uint32_t lo = 0u - (uint32_t)(p < 2u);
    auto sel = [lo](uint32_t a, uint32_t b) { return (a & lo) | (b & ~lo); };
    *s0 = sel(u & 63u, (w & 15u) | ((u >> 2) & 0x30u));
    *s1 = sel((u >> 8) & 63u, ((w >> 8) & 15u) | ((u >> 10) & 0x30u));
    *m0 = sel(z & 63u, ((w >> 4) & 15u) | ((z >> 2) & 0x30u));
    *m1 = sel((z >> 8) & 63u, ((w >> 12) & 15u) | ((z >> 10) & 0x30u));
}

/* Workgroup barrier that orders LDS accesses only: global loads issued
 * before it stay in flight across it. The LDS-only release fence does not
 * make the compiler wait for the wave's own LDS writes (it takes LDS
 * operations as ordered across waves), and without the wait the last
 * ds_write before the barrier has been read stale by other waves: the
 * explicit lgkmcnt(0) completes them first. */
__device__ __forceinline__ void kq_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/*
 * Raw buffer loads: a 128-bit resource (base, byte count) in scalar
 * registers plus a 32-bit per-lane offset, so a row walk costs one 32-bit
 * add per row instead of 64-bit per-lane address arithmetic. Dwords whose
 * offset lies at or beyond the byte count read as zero without touching
 * memory. Word 3 = 0x00020000 is the raw-buffer format of the gfx9 family.
 */
template <int AUX>
struct KqBufA {
    __amdgpu_buffer_rsrc_t r;
};
/* AUX is the loads' cache policy: 0 the default, kKqNt non-temporal (nt:
 * the lines are marked for early eviction) */
using KqBuf = KqBufA<0>;
constexpr int kKqNt = 2;

template <int AUX = 0>
__device__ __forceinline__ KqBufA<AUX> kq_buf(const void *base, uint32_t bytes) {
    KqBufA<AUX> b;
    b.r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                            0x00020000);
    return b;
}

typedef unsigned int kq_u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int kq_u32x3 __attribute__((ext_vector_type(3)));
typedef unsigned int kq_u32x4 __attribute__((ext_vector_type(4)));

template <int A>
__device__ __forceinline__ uint4 kq_ld128(KqBufA<A> b, uint32_t voff, uint32_t soff) {
    const kq_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(b.r, (int)voff, (int)soff, A);
    return make_uint4(v.x, v.y, v.z, v.w);
}
template <int A>
__device__ __forceinline__ kq_u32x3 kq_ld96(KqBufA<A> b, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b96(b.r, (int)voff, (int)soff, A);
}
template <int A>
__device__ __forceinline__ kq_u32x2 kq_ld64(KqBufA<A> b, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b64(b.r, (int)voff, (int)soff, A);
}
template <int A>
__device__ __forceinline__ uint32_t kq_ld32(KqBufA<A> b, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(b.r, (int)voff, (int)soff, A);
}
template <int A>
__device__ __forceinline__ uint32_t kq_ld16(KqBufA<A> b, uint32_t voff, uint32_t soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(b.r, (int)voff, (int)soff, A);
}

/* a * b for operands below 2^24 with the full-rate 24-bit multiply: the
 * compiler emits the quarter-rate 32-bit one for a plain product (and for
 * __umul24) even when the operands are known to be small */
__device__ __forceinline__ uint32_t kq_mul_u24(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_mul_u32_u24 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

/*
 * Byte loads from addresses that are only 2-byte aligned (Q8_0 blocks are
 * 34 B and Q6_K blocks 210 B, so a block can start at 2 mod 4). The dwords
 * covering the span are read at 4-byte aligned addresses (the buffer start
 * is 4-byte aligned, so a - (a & 3) never precedes it) and re-aligned with
 * a byte funnel shift. The pointer arithmetic keeps the global address
 * space, so these stay global (not flat) loads.
 */
__device__ __forceinline__ uint32_t kq_align2(uint32_t hi, uint32_t lo,
                                              uint32_t shift_bytes) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift_bytes);
}

/* 4 bytes at a (a even), reading at most 2 bytes past a + 4. */
__device__ __forceinline__ uint32_t kq_load4_u2a(const uint8_t *a) {
    const uint32_t sh = (uint32_t)((uintptr_t)a & 3u);
    const uint32_t *base = (const uint32_t *)(a - sh);
    return kq_align2(base[sh ? 1 : 0], base[0], sh);
}

/* 4 bytes at a (a even), never reading at or past end (a + 4 <= end). */
__device__ __forceinline__ uint32_t kq_load4_u2a_end(const uint8_t *a, const uint8_t *end) {
    const uint32_t sh = (uint32_t)((uintptr_t)a & 3u);
    const uint32_t *base = (const uint32_t *)(a - sh);
    uint32_t d1 = base[0];
    if (sh) {
        if ((const uint8_t *)(base + 2) <= end)
            d1 = base[1];
        else
            d1 = (uint32_t)(*(const uint16_t *)(base + 1));
    }
    return kq_align2(d1, base[0], sh);
}

/* Wave-wide sum over groups of G consecutive lanes (G power of two <= 64);
 * every lane of a group receives the group's sum. */
template <int G>
__device__ __forceinline__ float kq_group_sum(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, KQ_WAVE);
    return v;
}

/* Bitwise AND the optimiser cannot split into per-byte field extracts, so
 * that byte-wise conversions of the result stay single v_cvt_f32_ubyteN
 * instructions. */
__device__ __forceinline__ uint32_t kq_and_0f(uint32_t a) {
    uint32_t r;
    asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ __forceinline__ uint32_t kq_and_f0(uint32_t a) {
    uint32_t r;
    asm("v_and_b32 %0, 0xf0f0f0f0, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ __forceinline__ uint32_t kq_xor_80(uint32_t a) {
    uint32_t r;
    asm("v_xor_b32 %0, 0x80808080, %1" : "=v"(r) : "v"(a));
    return r;
}

/* x from lane (l ^ mask) within rows of 16, through DPP: masks 1 and 2 are
 * quad permutes, 7 and 15 are the half-row and row mirrors. */
template <int MASK>
__device__ __forceinline__ uint32_t kq_dpp_pair(uint32_t x) {
    constexpr int ctrl = MASK == 1 ? 0xB1 : MASK == 2 ? 0x4E : MASK == 7 ? 0x141 : 0x140;
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, ctrl, 0xf, 0xf, false);
}
template <int MASK>
__device__ __forceinline__ float kq_dpp_pair(float x) {
    return __uint_as_float(kq_dpp_pair<MASK>(__float_as_uint(x)));
}

/* a(lane) + a(lane ^ 32) for lanes < 32 and b(lane ^ 32) + b(lane) for
 * lanes >= 32, with one v_permlane32_swap (gfx950). */
__device__ __forceinline__ float kq_fold32(float a, float b) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
/* The same across odd/even 16-lane rows (lane ^ 16), v_permlane16_swap. */
__device__ __forceinline__ float kq_fold16(float a, float b) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

/*
 * Transposed butterfly: every lane of a G-lane group (G = 1..64, power of
 * two, groups aligned in the wave) holds N partial sums; afterwards the
 * group's total of value j is held by lane j * G / N (N <= G, in v[0]) or by
 * lane j / (N / G) in v[j % (N / G)] (N > G). Each level halves the values a
 * lane keeps: the lane whose level bit is clear keeps the low half and
 * receives its partner's low half, the other keeps the high half. Levels run
 * from offset G/2 down; partners at a level differ in that level's bit and
 * agree in every higher bit (mirrors flip the lower bits too, which only
 * reorders lanes that later levels still combine).
 */
template <int G, int N, int O>
__device__ __forceinline__ void kq_reduce_level(float *v, uint32_t lane) {
    if constexpr (O >= 1) {
        constexpr int n = (N * O * 2 / G) > 0 ? (N * O * 2 / G) : 1; /* values at this level */
        if constexpr (n >= 2) {
            constexpr int h = n / 2;
            const bool upper = (lane & (uint32_t)O) != 0u;
#pragma unroll
            for (int i = 0; i < h; ++i) {
                const float lo = v[i], hi = v[i + h];
                if constexpr (O == 32) {
                    v[i] = kq_fold32(lo, hi);
                } else if constexpr (O == 16) {
                    v[i] = kq_fold16(lo, hi);
                } else {
                    const float keep = upper ? hi : lo;
                    const float send = upper ? lo : hi;
                    v[i] = keep + kq_dpp_pair<O == 8 ? 15 : O == 4 ? 7 : O>(send);
                }
            }
        } else {
            if constexpr (O == 32)
                v[0] = kq_fold32(v[0], v[0]);
            else if constexpr (O == 16)
                v[0] = kq_fold16(v[0], v[0]);
            else
                v[0] = v[0] + kq_dpp_pair<O == 8 ? 15 : O == 4 ? 7 : O>(v[0]);
        }
        kq_reduce_level<G, N, O / 2>(v, lane);
    }
}

template <int G, int N>
__device__ __forceinline__ void kq_group_reduce(float (&v)[N], uint32_t lane) {
    kq_reduce_level<G, N, G / 2>(v, lane);
}

/* ---- 64-bit values across a wave (all 64 lanes active) ---- */

/* x moved by one DPP control, as two 32-bit halves; lanes that the control
 * or the row mask leaves without a source receive 0.0. */
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double kq_dpp_f64(double x) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL,
                                                              ROW_MASK, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL,
                                                              ROW_MASK, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

/* Inclusive prefix sum over the wave: shifts by 1, 2, 4, 8 within rows of
 * 16 lanes, then row 0's total into row 1 and row 2's into row 3
 * (row_bcast:15), then rows 0-1's total into rows 2-3 (row_bcast:31). */
__device__ __forceinline__ double kq_wave_scan_f64(double x) {
    x += kq_dpp_f64<0x111>(x);
    x += kq_dpp_f64<0x112>(x);
    x += kq_dpp_f64<0x114>(x);
    x += kq_dpp_f64<0x118>(x);
    x += kq_dpp_f64<0x142, 0xa>(x);
    x += kq_dpp_f64<0x143, 0xc>(x);
    return x;
}

/* The value of lane l - 1 (0.0 in lane 0): wave_shr:1. */
__device__ __forceinline__ double kq_wave_shr1_f64(double x) {
    return kq_dpp_f64<0x138>(x);
}

__device__ __forceinline__ double kq_readlane_f64(double x, int lane) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

/* {x(l), x(l ^ 16)} or {x(l), x(l ^ 32)} (in either order, the same for
 * both halves) through v_permlane16_swap / v_permlane32_swap. */
template <int SPAN>
__device__ __forceinline__ void kq_swap_f64(double x, double &p, double &q) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
    auto rl = SPAN == 16 ? __builtin_amdgcn_permlane16_swap(lo, lo, false, false)
                         : __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    auto rh = SPAN == 16 ? __builtin_amdgcn_permlane16_swap(hi, hi, false, false)
                         : __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    p = __builtin_bit_cast(double, ((uint64_t)rh[0] << 32) | rl[0]);
    q = __builtin_bit_cast(double, ((uint64_t)rh[1] << 32) | rl[1]);
}

/* Maximum over the wave, in every lane: quad permutes, half-row and row
 * mirrors, then the two permlane swaps. NaN-free inputs. */
__device__ __forceinline__ double kq_wave_max_f64(double v) {
    v = fmax(v, kq_dpp_f64<0xB1>(v));
    v = fmax(v, kq_dpp_f64<0x4E>(v));
    v = fmax(v, kq_dpp_f64<0x141>(v));
    v = fmax(v, kq_dpp_f64<0x140>(v));
    double p, q;
    kq_swap_f64<16>(v, p, q);
    v = fmax(p, q);
    kq_swap_f64<32>(v, p, q);
    return fmax(p, q);
}

/* Sum over the wave, in every lane (the same butterfly as the maximum). */
__device__ __forceinline__ double kq_wave_sum_f64(double v) {
    v += kq_dpp_f64<0xB1>(v);
    v += kq_dpp_f64<0x4E>(v);
    v += kq_dpp_f64<0x141>(v);
    v += kq_dpp_f64<0x140>(v);
    double p, q;
    kq_swap_f64<16>(v, p, q);
    v = p + q;
    kq_swap_f64<32>(v, p, q);
    return p + q;
}

#endif
