/*
 * kq_rowdot.h — per-lane pieces of a dequant-fused row dot, shared by the
 * matvec, LM-head and MoE expert kernels.
 *
 * A row of C columns is split over C/32 lanes; each lane owns 32 weights
 * and holds the matching activations for batch columns 0..B-1 in registers
 * (load_x), streams its slice of every row it visits (load) and returns
 * its partial dot (dot). The decode of each format follows
 * src/kq_numeric.c:176-295 (Q8_0, Q4_K, Q5_1, Q5_K, IQ4_NL) and the GGML
 * Q6_K layout; the
 * per-sub-block scale is applied once to a sum of code*x products, and the
 * block offset (Q4_K dmin*m, Q6_K -32, Q8_0 +128 bias) is taken off with a
 * precomputed activation sum. Codes are converted with one
 * v_cvt_f32_ubyteN per weight (the masks are opaque to the optimiser).
 */
#ifndef KQ_ROWDOT_H
#define KQ_ROWDOT_H

#include <type_traits>

#include "kq_device.h"

namespace kq {

/* Activation sources. A lane takes its 32 activations per batch column as
 * 8 float4 chunks c = 0..7 in a fixed order (natural column k of chunk c is
 * Lane::xk(l, c)); a source returns batch column b's chunk. */
struct XGlobal {
    const float *x;
    uint32_t stride;
    __device__ __forceinline__ float4 operator()(int b, uint32_t k, int) const {
        return *(const float4 *)(x + (size_t)b * stride + k);
    }
};
/* LDS image [b][c][lpr] of float4 (XStage): consecutive lanes read
 * consecutive 16-byte words, lanes of one row position share a word */
struct XLds {
    const float4 *xs;
    uint32_t l, lpr;
    __device__ __forceinline__ float4 operator()(int b, uint32_t, int c) const {
        return xs[((uint32_t)b * 8u + (uint32_t)c) * lpr + l];
    }
};

/* chunks 2q and 2q + 1 (natural columns k .. k + 7) of every batch column */
template <int B, class X>
__device__ __forceinline__ bool load_x8(const X &src, uint32_t k, int q, float (&dst)[B][8]) {
    bool bad = false;
#pragma unroll
    for (int b = 0; b < B; ++b) {
        const float4 u = src(b, k, 2 * q), v = src(b, k + 4u, 2 * q + 1);
        dst[b][0] = u.x; dst[b][1] = u.y; dst[b][2] = u.z; dst[b][3] = u.w;
        dst[b][4] = v.x; dst[b][5] = v.y; dst[b][6] = v.z; dst[b][7] = v.w;
#pragma unroll
        for (int i = 0; i < 8; ++i) bad |= !kq_isfinite(dst[b][i]);
    }
    return bad;
}

/* 4 byte codes of w dotted with 4 activations, fp32 fused. */
__device__ __forceinline__ float dot4_u8(uint32_t w, const float *xv, float acc) {
    acc = fmaf((float)(w & 0xffu), xv[0], acc);
    acc = fmaf((float)((w >> 8) & 0xffu), xv[1], acc);
    acc = fmaf((float)((w >> 16) & 0xffu), xv[2], acc);
    acc = fmaf((float)(w >> 24), xv[3], acc);
    return acc;
}

template <int B>
__device__ __forceinline__ void sum8(const float (&v)[B][8], float (&s)[B]) {
#pragma unroll
    for (int b = 0; b < B; ++b) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) a += v[b][i];
        s[b] = a;
    }
}

/* ---------------- Q4_K: 144 B blocks of 256 ---------------- */
template <int B>
struct LaneQ4K {
    static constexpr uint32_t kBlockBytes = 144u;
    struct Raw {
        uint4 hd, qs;
    };
    uint32_t off;  /* byte offset of this lane's block within the row */
    uint32_t qoff; /* offset of its 16 qs bytes within the block */
    uint32_t gq, k0;
    float xl[B][16], xh[B][16], sxl[B], sxh[B];

    /* l = lane index within the row: block l/8, 16-byte qs slice l%8 */
    __device__ __forceinline__ void setup(uint32_t l) {
        const uint32_t bb = l >> 3, c = l & 7u, h = c & 1u;
        gq = c >> 1;
        off = kBlockBytes * bb;
        qoff = 16u + 32u * gq + 16u * h;
        k0 = 256u * bb + 64u * gq + 16u * h;
    }
    /* natural column of chunk c of lane l */
    __device__ static __forceinline__ uint32_t xk(uint32_t l, int c) {
        const uint32_t k = 256u * (l >> 3) + 64u * ((l & 7u) >> 1) + 16u * (l & 1u);
        return k + (c >= 4 ? 32u : 0u) + 8u * ((uint32_t)(c >> 1) & 1u) + 4u * ((uint32_t)c & 1u);
    }
    __device__ __forceinline__ bool load_x(const float *x, uint32_t stride) {
        return load_x(XGlobal{x, stride});
    }
    template <class X>
    __device__ __forceinline__ bool load_x(const X &src) {
        float t0[B][8], t1[B][8], s0[B], s1[B];
        bool bad = load_x8<B>(src, k0, 0, t0);
        bad |= load_x8<B>(src, k0 + 8u, 1, t1);
        sum8<B>(t0, s0);
        sum8<B>(t1, s1);
#pragma unroll
        for (int b = 0; b < B; ++b) {
#pragma unroll
            for (int i = 0; i < 8; ++i) { xl[b][i] = t0[b][i]; xl[b][8 + i] = t1[b][i]; }
            sxl[b] = s0[b] + s1[b];
        }
        bad |= load_x8<B>(src, k0 + 32u, 2, t0);
        bad |= load_x8<B>(src, k0 + 40u, 3, t1);
        sum8<B>(t0, s0);
        sum8<B>(t1, s1);
#pragma unroll
        for (int b = 0; b < B; ++b) {
#pragma unroll
            for (int i = 0; i < 8; ++i) { xh[b][i] = t0[b][i]; xh[b][8 + i] = t1[b][i]; }
            sxh[b] = s0[b] + s1[b];
        }
        return bad;
    }
    /* row_off: byte offset of the row in the buffer */
    template <int A>
    __device__ __forceinline__ Raw load(KqBufA<A> b, uint32_t row_off) const {
        Raw r;
        r.hd = kq_ld128(b, row_off + off, 0u);
        r.qs = kq_ld128(b, row_off + off + qoff, 0u);
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        r.hd = make_uint4(0, 0, 0, 0);
        r.qs = make_uint4(0, 0, 0, 0);
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float *acc, bool &malformed) const {
        const float d = kq_f16_to_f32_hw(r.hd.x);
        const float dmin = kq_f16_to_f32_hw(r.hd.x >> 16);
        malformed |= !kq_isfinite(d) || !kq_isfinite(dmin);
        uint32_t s0, m0, s1, m1;
        kq_k_scale_pair(gq, r.hd.y, r.hd.z, r.hd.w, &s0, &m0, &s1, &m1);
        const float dl = d * (float)s0, ml = dmin * (float)m0;
        /* high nibbles are converted in place (16 * code): fold 1/16 into
         * the sub-block scale (exact power of two) */
        const float dh = d * (float)s1 * 0.0625f, mh = dmin * (float)m1;
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            lo[w] = kq_and_0f(q[w]);
            hi[w] = kq_and_f0(q[w]);
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float sl = 0.0f, sh = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                sl = dot4_u8(lo[w], &xl[b][4 * w], sl);
                sh = dot4_u8(hi[w], &xh[b][4 * w], sh);
            }
            float v = dl * sl;
            v = fmaf(-ml, sxl[b], v);
            v = fmaf(dh, sh, v);
            v = fmaf(-mh, sxh[b], v);
            acc[b] = v;
        }
    }
};

/* ---------- integer dots over activation byte planes ----------
 * Digit lanes (LaneQ4KI, LaneQ6KI, LaneQ8I) keep the loads and lane layout
 * of their fp32 counterparts but take the activations staged as integers
 * (XStageI): per group of G consecutive columns (G = 16, 8, 32) one power
 * of two pw = 2^-k and X = rint(x * 2^k) with |X| <= 2^22, as three byte
 * planes X = D0 + 2^8 D1 + 2^16 D2, four columns per 32-bit word: for
 * unsigned codes (Q4_K, Q6_K) D0 and D1 are X's low bytes and D2 its
 * signed third byte; for signed codes (Q8_0) all three are balanced signed
 * digits in [-128, 127]. A word of four 8-bit codes meets each plane in one
 * v_dot4 (exact integer sums: u8 x u8 for unsigned digits, i8 x i8
 * otherwise); a group's sum
 * is rebuilt from the three plane sums, converted once and scaled by the
 * block scale times pw. Against fp32 products this moves each activation
 * by at most 2^-23 of the largest magnitude in its group, below the fp32
 * summation error the results are compared with. */

/* a lane's eight 16-byte slots per batch column from the staged image
 * [b][slot][lane] */
template <int B, int NS, bool BAL, bool ISUM = false, uint32_t HALF = 0u>
struct DigitSlots {
    static constexpr bool kDigits = true;
    static constexpr bool kBalanced = BAL; /* all three digits signed */
    static constexpr bool kIntSum = ISUM;  /* the record's sum is that of X, an int */
    uint4 sl[B][NS];
    /* slots in HALF (a bit mask) hold two words: only those are read */
    __device__ __forceinline__ void load_digits(const uint4 *img, uint32_t l, uint32_t lpr) {
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                const uint4 *p = img + ((uint32_t)b * 8u + (uint32_t)j) * lpr + l;
                if ((HALF >> j) & 1u) {
                    const uint2 h = *reinterpret_cast<const uint2 *>(p);
                    sl[b][j] = make_uint4(h.x, h.y, 0u, 0u);
                } else {
                    sl[b][j] = *p;
                }
            }
    }
    /* dword i of the lane's slots (i a compile-time constant) */
    __device__ __forceinline__ uint32_t word(int b, int i) const {
        const uint4 &s = sl[b][i >> 2];
        return (i & 3) == 0 ? s.x : (i & 3) == 1 ? s.y : (i & 3) == 2 ? s.z : s.w;
    }
};

/* sum of codes times X over one group from its three plane sums: exact in
 * int32 where |sum| < 2^31 */
__device__ __forceinline__ int digit_sum(int s0, int s1, int s2) {
    return (int)((uint32_t)s0 + ((uint32_t)s1 << 8) + ((uint32_t)s2 << 16));
}

/* Q4_K: groups of 16 columns, the low and the high nibbles' 16 columns of
 * a lane (|sum| <= 16 * 15 * 2^22 < 2^31). Record of a group: plane p word
 * w at 4p + w, pw at 12, the fp32 column sum at 13; slots 0..3 hold the
 * lane's low group, 4..7 its high one. */
template <int B>
struct LaneQ4KI : DigitSlots<B, 8, false, false, 0x88u> {
    static constexpr uint32_t kBlockBytes = 144u;
    static constexpr uint32_t kGroupCols = 16u;
    using Raw = typename LaneQ4K<B>::Raw;
    using DigitSlots<B, 8, false, false, 0x88u>::word;
    uint32_t off, qoff;
    uint32_t sel_a, sel_b, lo_mask;

    /* the lane of a row that reads column group g, and its first slot:
     * columns 256bb + 64gq + 16h + 0..15 are lane 8bb + 2gq + h's low
     * group, + 32 its high one */
    __device__ static __forceinline__ void home(uint32_t g, uint32_t &lane, uint32_t &slot) {
        const uint32_t r = g % 16u, t = r % 4u;
        lane = 8u * (g / 16u) + 2u * (r / 4u) + (t & 1u);
        slot = t < 2u ? 0u : 4u;
    }
    __device__ __forceinline__ void setup(uint32_t l) {
        const uint32_t bb = l >> 3, c = l & 7u, h = c & 1u, gq = c >> 1;
        off = kBlockBytes * bb;
        qoff = 16u + 32u * gq + 16u * h;
        /* scale bytes of sub-blocks 2gq, 2gq + 1 (src/kq_numeric.c:214-227):
         * q[2p], q[2p+1] and q[4+2p], q[5+2p] for p = gq & 1, in one word */
        const uint32_t p2 = 2u * (gq & 1u);
        sel_b = p2 | (p2 + 1u) << 8 | (p2 + 4u) << 16 | (p2 + 5u) << 24;
        sel_a = p2 | (p2 + 1u) << 8 | p2 << 16 | (p2 + 1u) << 24;
        lo_mask = gq < 2u ? 0xffffffffu : 0u;
    }
    template <int A>
    __device__ __forceinline__ Raw load(KqBufA<A> b, uint32_t row_off) const {
        Raw r;
        r.hd = kq_ld128(b, row_off + off, 0u);
        r.qs = kq_ld128(b, row_off + off + qoff, 0u);
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        r.hd = make_uint4(0, 0, 0, 0);
        r.qs = make_uint4(0, 0, 0, 0);
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float *acc, bool &malformed) const {
        const float d = kq_f16_to_f32_hw(r.hd.x);
        const float dmin = kq_f16_to_f32_hw(r.hd.x >> 16);
        malformed |= !kq_isfinite(d) || !kq_isfinite(dmin);
        /* [sc0, sc1, m0, m1] as bytes: 6-bit fields of q[0..7] for
         * sub-blocks 0..3, else the low/high nibbles of q[8..11] with the
         * top two bits of q[0..7] */
        const uint32_t wb = __builtin_amdgcn_perm(r.hd.z, r.hd.y, sel_b);
        const uint32_t wa = __builtin_amdgcn_perm(r.hd.w, r.hd.w, sel_a);
        uint32_t hi = (wa & 0x00000f0fu) | ((wa >> 4) & 0x0f0f0000u);
        hi |= (wb >> 2) & 0x30303030u;
        const uint32_t sm = ((wb & 0x3f3f3f3fu) & lo_mask) | (hi & ~lo_mask);
        const float dl = d * (float)(sm & 0xffu), dh = d * (float)((sm >> 8) & 0xffu);
        const float ml = dmin * (float)((sm >> 16) & 0xffu), mh = dmin * (float)(sm >> 24);
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        uint32_t cl[4], ch[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            cl[w] = q[w] & 0x0f0f0f0fu;
            ch[w] = (q[w] >> 4) & 0x0f0f0f0fu;
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            uint32_t l0 = 0u, l1 = 0u, h0 = 0u, h1 = 0u;
            int l2 = 0, h2 = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                l0 = __builtin_amdgcn_udot4(cl[w], word(b, w), l0, false);
                l1 = __builtin_amdgcn_udot4(cl[w], word(b, 4 + w), l1, false);
                l2 = __builtin_amdgcn_sdot4((int)cl[w], (int)word(b, 8 + w), l2, false);
                h0 = __builtin_amdgcn_udot4(ch[w], word(b, 16 + w), h0, false);
                h1 = __builtin_amdgcn_udot4(ch[w], word(b, 20 + w), h1, false);
                h2 = __builtin_amdgcn_sdot4((int)ch[w], (int)word(b, 24 + w), h2, false);
            }
            const float pwl = __uint_as_float(word(b, 12)), sxl = __uint_as_float(word(b, 13));
            const float pwh = __uint_as_float(word(b, 28)), sxh = __uint_as_float(word(b, 29));
            float v = (float)digit_sum((int)l0, (int)l1, l2) * (dl * pwl);
            v = fmaf(-ml, sxl, v);
            v = fmaf((float)digit_sum((int)h0, (int)h1, h2), dh * pwh, v);
            v = fmaf(-mh, sxh, v);
            acc[b] = v;
        }
    }
};

/* ---------------- Q6_K: 210 B blocks of 256 ---------------- */
/* Fields of 8 bytes at byte offset o (o even) are read as one 12-byte
 * dwordx3 window at o - (o & 3) and funnel-shifted; the sub-scales of the
 * second half (the last field of a block, ending at 208) use the window
 * [o - 4, o + 8) when o is 4-aligned, so no window passes the block's last
 * byte. A window may start 2 bytes before its block (inside the previous
 * block of the same buffer). */
template <int B>
struct LaneQ6K {
    static constexpr uint32_t kBlockBytes = 210u;
    /* raw 12-byte windows; aligned in dot() so that issuing the next group's
     * loads never waits for this group's data */
    struct Raw {
        kq_u32x3 wa, wb, wh, ws;
        uint32_t d, sh;
    };
    uint32_t off, n, t, k0;
    float xq[4][B][8], xs[4][B];

    /* l = lane index within the row: block l/8, half n, l-range 8t..8t+7 */
    __device__ __forceinline__ void setup(uint32_t l) {
        const uint32_t bb = l >> 3, s = l & 7u;
        n = s >> 2;
        t = s & 3u;
        off = kBlockBytes * bb;
        k0 = 256u * bb + 128u * n + 8u * t;
    }
    /* quarter q holds outputs k0 + 32q + 0..7 */
    /* natural column of chunk c of lane l */
    __device__ static __forceinline__ uint32_t xk(uint32_t l, int c) {
        const uint32_t k = 256u * (l >> 3) + 128u * ((l & 7u) >> 2) + 8u * (l & 3u);
        return k + 32u * (uint32_t)(c >> 1) + 4u * ((uint32_t)c & 1u);
    }
    __device__ __forceinline__ bool load_x(const float *x, uint32_t stride) {
        return load_x(XGlobal{x, stride});
    }
    template <class X>
    __device__ __forceinline__ bool load_x(const X &src) {
        bool bad = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            bad |= load_x8<B>(src, k0 + 32u * q, q, xq[q]);
            sum8<B>(xq[q], xs[q]);
        }
        return bad;
    }
    /* byte offset of the 12-byte window holding the 8 bytes at o */
    __device__ static __forceinline__ uint32_t window(uint32_t o, bool last) {
        const uint32_t sh = o & 3u;
        return (last && sh == 0u) ? o - 4u : o - sh;
    }
    __device__ static __forceinline__ uint2 align8(kq_u32x3 w, uint32_t sh, bool back) {
        uint2 r;
        r.x = back ? w.y : kq_align2(w.y, w.x, sh);
        r.y = back ? w.z : kq_align2(w.z, w.y, sh);
        return r;
    }
    template <int A>
    __device__ __forceinline__ Raw load(KqBufA<A> b, uint32_t row_off) const {
        const uint32_t p = row_off + off;
        Raw r;
        r.sh = p & 3u; /* every field of a block shares the block's alignment */
        r.wa = kq_ld96(b, window(p + 64u * n + 8u * t, false), 0u);
        r.wb = kq_ld96(b, window(p + 64u * n + 32u + 8u * t, false), 0u);
        r.wh = kq_ld96(b, window(p + 128u + 32u * n + 8u * t, false), 0u);
        r.ws = kq_ld96(b, window(p + 192u + 8u * n, n == 1u), 0u);
        r.d = kq_ld16(b, p + 208u, 0u);
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        r.wa = r.wb = r.wh = r.ws = kq_u32x3{0u, 0u, 0u};
        r.d = 0u;
        r.sh = 0u;
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float *acc, bool &malformed) const {
        const float d = kq_f16_to_f32_hw(r.d);
        malformed |= !kq_isfinite(d);
        const uint2 qa = align8(r.wa, r.sh, false), qb = align8(r.wb, r.sh, false);
        const uint2 qh = align8(r.wh, r.sh, false);
        const uint2 sc = align8(r.ws, r.sh, n == 1u && r.sh == 0u);
        /* quarter q uses sc[8n + (t>>1) + 2q]: byte (t>>1) or (t>>1)+2 of the
         * first or second dword of sc[8n .. 8n+7] */
        const uint32_t sh = (t >> 1) * 8u;
        const uint32_t sv[4] = {sc.x >> sh, sc.x >> (sh + 16u), sc.y >> sh,
                                sc.y >> (sh + 16u)};
        float dq[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) dq[q] = d * (float)(int8_t)(sv[q] & 0xffu);
        float part[4][B];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int b = 0; b < B; ++b) part[q][b] = 0.0f;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const uint32_t A = half ? qa.y : qa.x;
            const uint32_t Bq = half ? qb.y : qb.x;
            const uint32_t H = half ? qh.y : qh.x;
            const uint32_t c0 = (A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
            const uint32_t c1 = (Bq & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
            const uint32_t c2 = ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u);
            const uint32_t c3 = ((Bq >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
#pragma unroll
            for (int b = 0; b < B; ++b) {
                part[0][b] = dot4_u8(c0, &xq[0][b][4 * half], part[0][b]);
                part[1][b] = dot4_u8(c1, &xq[1][b][4 * half], part[1][b]);
                part[2][b] = dot4_u8(c2, &xq[2][b][4 * half], part[2][b]);
                part[3][b] = dot4_u8(c3, &xq[3][b][4 * half], part[3][b]);
            }
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float v = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) v = fmaf(dq[q], fmaf(-32.0f, xs[q][b], part[q][b]), v);
            acc[b] = v;
        }
    }
};

/* ---------------- Q8_0: 34 B blocks of 32 ---------------- */
/* A block at byte offset bo (even) is read as two 16-byte windows from
 * bo - (bo & 3) plus two 16-bit loads of its last four code bytes: every
 * read lies inside the block or the 2 bytes before it. */
template <int B>
struct LaneQ8 {
    static constexpr uint32_t kBlockBytes = 34u;
    /* raw windows; aligned in dot() (see LaneQ6K) */
    struct Raw {
        uint4 w0, w1;
        uint32_t t0, t1, sh;
    };
    uint32_t off, k0;
    float xv[4][B][8], xsum[B];

    __device__ __forceinline__ void setup(uint32_t l) {
        off = kBlockBytes * l;
        k0 = 32u * l;
    }
    /* natural column of chunk c of lane l */
    __device__ static __forceinline__ uint32_t xk(uint32_t l, int c) {
        return 32u * l + 4u * (uint32_t)c;
    }
    __device__ __forceinline__ bool load_x(const float *x, uint32_t stride) {
        return load_x(XGlobal{x, stride});
    }
    template <class X>
    __device__ __forceinline__ bool load_x(const X &src) {
        bool bad = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) bad |= load_x8<B>(src, k0 + 8u * q, q, xv[q]);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float a = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < 8; ++i) a += xv[q][b][i];
            xsum[b] = a;
        }
        return bad;
    }
    template <int A>
    __device__ __forceinline__ Raw load(KqBufA<A> b, uint32_t row_off) const {
        const uint32_t bo = row_off + off;
        Raw r;
        r.sh = bo & 3u;
        r.w0 = kq_ld128(b, bo - r.sh, 0u);
        r.w1 = kq_ld128(b, bo - r.sh + 16u, 0u);
        r.t0 = kq_ld16(b, bo + 30u, 0u);
        r.t1 = kq_ld16(b, bo + 32u, 0u);
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        /* codes decode to the +128 bias only: a zero scale gives 0 */
        r.w0 = make_uint4(0u, 0x80808080u, 0x80808080u, 0x80808080u);
        r.w1 = make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
        r.t0 = r.t1 = 0x8080u;
        r.sh = 0u;
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float *acc, bool &malformed) const {
        const uint32_t w[8] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w};
        const float d = kq_f16_to_f32_hw(r.sh ? (w[0] >> 16) : w[0]);
        malformed |= !kq_isfinite(d);
        /* code dword k = bytes bo+2+4k .. bo+5+4k of the block at bo */
        uint32_t u[8];
#pragma unroll
        for (int k = 0; k < 7; ++k) u[k] = kq_xor_80(r.sh ? w[k + 1] : kq_align2(w[k + 1], w[k], 2u));
        u[7] = kq_xor_80(r.t0 | (r.t1 << 16));
#pragma unroll
        for (int b = 0; b < B; ++b) {
            /* int8 code + 128 as an unsigned byte; the bias comes off with
             * the activation sum */
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) s = dot4_u8(u[j], &xv[j >> 1][b][4 * (j & 1)], s);
            acc[b] = d * fmaf(-128.0f, xsum[b], s);
        }
    }
};

/* Q6_K digit lane: LaneQ6K's loads; groups of 8 columns, one per quarter
 * of a lane. The codes carry +32, taken off in integers with the sum of X
 * (the record's sum), so a code of 32 contributes exactly zero however
 * large its activation: sum (c - 32) X = sum c X - 32 sum X, with
 * |sum c X| <= 8 * 63 * 2^22 < 2^31. Record of a group: plane p word w at
 * 2p + w, pw at 6, sum X at 7, in slots 2q and 2q + 1 for quarter q. */
template <int B>
struct LaneQ6KI : DigitSlots<B, 8, false, true> {
    static constexpr uint32_t kBlockBytes = 210u;
    static constexpr uint32_t kGroupCols = 8u;
    using Base = LaneQ6K<B>;
    using Raw = typename Base::Raw;
    using DigitSlots<B, 8, false, true>::word;
    uint32_t off, n, t;

    /* quarter q of lane 8bb + 4n + t holds columns 256bb + 128n + 8t + 32q
     * + 0..7 */
    __device__ static __forceinline__ void home(uint32_t g, uint32_t &lane, uint32_t &slot) {
        const uint32_t r = g % 32u;
        lane = 8u * (g / 32u) + 4u * (r / 16u) + r % 4u;
        slot = 2u * ((r % 16u) / 4u);
    }
    __device__ __forceinline__ void setup(uint32_t l) {
        const uint32_t s = l & 7u;
        n = s >> 2;
        t = s & 3u;
        off = kBlockBytes * (l >> 3);
    }
    template <int A>
    __device__ __forceinline__ Raw load(KqBufA<A> b, uint32_t row_off) const {
        const uint32_t p = row_off + off;
        Raw r;
        r.sh = p & 3u;
        r.wa = kq_ld96(b, Base::window(p + 64u * n + 8u * t, false), 0u);
        r.wb = kq_ld96(b, Base::window(p + 64u * n + 32u + 8u * t, false), 0u);
        r.wh = kq_ld96(b, Base::window(p + 128u + 32u * n + 8u * t, false), 0u);
        r.ws = kq_ld96(b, Base::window(p + 192u + 8u * n, n == 1u), 0u);
        r.d = kq_ld16(b, p + 208u, 0u);
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        r.wa = r.wb = r.wh = r.ws = kq_u32x3{0u, 0u, 0u};
        r.d = 0u;
        r.sh = 0u;
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float *acc, bool &malformed) const {
        const float d = kq_f16_to_f32_hw(r.d);
        malformed |= !kq_isfinite(d);
        const uint2 qa = Base::align8(r.wa, r.sh, false), qb = Base::align8(r.wb, r.sh, false);
        const uint2 qh = Base::align8(r.wh, r.sh, false);
        const uint2 sc = Base::align8(r.ws, r.sh, n == 1u && r.sh == 0u);
        const uint32_t sh = (t >> 1) * 8u;
        const uint32_t sv[4] = {sc.x >> sh, sc.x >> (sh + 16u), sc.y >> sh,
                                sc.y >> (sh + 16u)};
        /* codes of quarter q, columns 4h .. 4h + 3 */
        uint32_t c[4][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t A = h ? qa.y : qa.x, Bq = h ? qb.y : qb.x, H = h ? qh.y : qh.x;
            c[0][h] = (A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
            c[1][h] = (Bq & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
            c[2][h] = ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u);
            c[3][h] = ((Bq >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float v = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t s0 = 0u, s1 = 0u;
                int s2 = 0;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    s0 = __builtin_amdgcn_udot4(c[q][h], word(b, 8 * q + h), s0, false);
                    s1 = __builtin_amdgcn_udot4(c[q][h], word(b, 8 * q + 2 + h), s1, false);
                    s2 = __builtin_amdgcn_sdot4((int)c[q][h], (int)word(b, 8 * q + 4 + h), s2,
                                                false);
                }
                const float pw = __uint_as_float(word(b, 8 * q + 6));
                const uint32_t sxi = word(b, 8 * q + 7);
                const float dq = d * (float)(int8_t)(sv[q] & 0xffu);
                const int sq = (int)((uint32_t)digit_sum((int)s0, (int)s1, s2) - 32u * sxi);
                v = fmaf(dq, (float)sq * pw, v);
            }
            acc[b] = v;
        }
    }
};

/* Q8_0 digit lane: LaneQ8's loads; one group of 32 columns per lane (its
 * block). The int8 codes meet the planes as they are; the three plane sums
 * (each within 32 * 127 * 128) are joined in fp32. Record: plane p word w
 * at 8p + w, pw at 24 (slots 0..6). */
template <int B>
struct LaneQ8I : DigitSlots<B, 7, true, false, 0x40u> {
    static constexpr uint32_t kBlockBytes = 34u;
    static constexpr uint32_t kGroupCols = 32u;
    using Raw = typename LaneQ8<B>::Raw;
    using DigitSlots<B, 7, true, false, 0x40u>::word;
    uint32_t off;

    __device__ static __forceinline__ void home(uint32_t g, uint32_t &lane, uint32_t &slot) {
        lane = g;
        slot = 0u;
    }
    __device__ __forceinline__ void setup(uint32_t l) { off = kBlockBytes * l; }
    template <int A>
    __device__ __forceinline__ Raw load(KqBufA<A> b, uint32_t row_off) const {
        const uint32_t bo = row_off + off;
        Raw r;
        r.sh = bo & 3u;
        r.w0 = kq_ld128(b, bo - r.sh, 0u);
        r.w1 = kq_ld128(b, bo - r.sh + 16u, 0u);
        r.t0 = kq_ld16(b, bo + 30u, 0u);
        r.t1 = kq_ld16(b, bo + 32u, 0u);
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        r.w0 = r.w1 = make_uint4(0u, 0u, 0u, 0u);
        r.t0 = r.t1 = 0u;
        r.sh = 0u;
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float *acc, bool &malformed) const {
        const uint32_t w[8] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w};
        const float d = kq_f16_to_f32_hw(r.sh ? (w[0] >> 16) : w[0]);
        malformed |= !kq_isfinite(d);
        /* code dword k = bytes bo+2+4k .. bo+5+4k of the block at bo */
        uint32_t u[8];
#pragma unroll
        for (int k = 0; k < 7; ++k) u[k] = r.sh ? w[k + 1] : kq_align2(w[k + 1], w[k], 2u);
        u[7] = r.t0 | (r.t1 << 16);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                s0 = __builtin_amdgcn_sdot4((int)u[j], (int)word(b, j), s0, false);
                s1 = __builtin_amdgcn_sdot4((int)u[j], (int)word(b, 8 + j), s1, false);
                s2 = __builtin_amdgcn_sdot4((int)u[j], (int)word(b, 16 + j), s2, false);
            }
            const float lo = (float)(s0 + s1 * 256); /* |.| < 2^28: one rounding */
            const float sum = fmaf((float)s2, 65536.0f, lo);
            acc[b] = sum * (d * __uint_as_float(word(b, 24)));
        }
    }
};

/* ---------------- Q5_K: 176 B blocks of 256 ---------------- */
/* The Q4_K layout with a fifth code bit: d, dmin, 12 scale bytes @0,
 * qh[32] @16, qs[128] @48 (src/kq_numeric.c:223-277). Code i of sub-block
 * pair g is the nibble of qs[32g + i] plus 16 when bit 2g (low nibble) or
 * 2g+1 (high nibble) of qh[i] is set; the lane mapping is LaneQ4K's, and a
 * lane's 16 qs bytes pair with qh bytes 16h .. 16h+15. */
template <int B>
struct LaneQ5K {
    static constexpr uint32_t kBlockBytes = 176u;
    struct Raw {
        uint4 hd, qh, qs;
    };
    uint32_t off, qoff, hoff;
    uint32_t gq, k0;
    float xl[B][16], xh[B][16], sxl[B], sxh[B];

    __device__ __forceinline__ void setup(uint32_t l) {
        const uint32_t bb = l >> 3, c = l & 7u, h = c & 1u;
        gq = c >> 1;
        off = kBlockBytes * bb;
        qoff = 48u + 32u * gq + 16u * h;
        hoff = 16u + 16u * h;
        k0 = 256u * bb + 64u * gq + 16u * h;
    }
    /* natural column of chunk c of lane l */
    __device__ static __forceinline__ uint32_t xk(uint32_t l, int c) {
        const uint32_t k = 256u * (l >> 3) + 64u * ((l & 7u) >> 1) + 16u * (l & 1u);
        return k + (c >= 4 ? 32u : 0u) + 8u * ((uint32_t)(c >> 1) & 1u) + 4u * ((uint32_t)c & 1u);
    }
    __device__ __forceinline__ bool load_x(const float *x, uint32_t stride) {
        return load_x(XGlobal{x, stride});
    }
    template <class X>
    __device__ __forceinline__ bool load_x(const X &src) {
        float t0[B][8], t1[B][8], s0[B], s1[B];
        bool bad = load_x8<B>(src, k0, 0, t0);
        bad |= load_x8<B>(src, k0 + 8u, 1, t1);
        sum8<B>(t0, s0);
        sum8<B>(t1, s1);
#pragma unroll
        for (int b = 0; b < B; ++b) {
#pragma unroll
            for (int i = 0; i < 8; ++i) { xl[b][i] = t0[b][i]; xl[b][8 + i] = t1[b][i]; }
            sxl[b] = s0[b] + s1[b];
        }
        bad |= load_x8<B>(src, k0 + 32u, 2, t0);
        bad |= load_x8<B>(src, k0 + 40u, 3, t1);
        sum8<B>(t0, s0);
        sum8<B>(t1, s1);
#pragma unroll
        for (int b = 0; b < B; ++b) {
#pragma unroll
            for (int i = 0; i < 8; ++i) { xh[b][i] = t0[b][i]; xh[b][8 + i] = t1[b][i]; }
            sxh[b] = s0[b] + s1[b];
        }
        return bad;
    }
    template <int A>
    __device__ __forceinline__ Raw load(KqBufA<A> b, uint32_t row_off) const {
        Raw r;
        r.hd = kq_ld128(b, row_off + off, 0u);
        r.qh = kq_ld128(b, row_off + off + hoff, 0u);
        r.qs = kq_ld128(b, row_off + off + qoff, 0u);
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        r.hd = r.qh = r.qs = make_uint4(0, 0, 0, 0);
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float *acc, bool &malformed) const {
        const float d = kq_f16_to_f32_hw(r.hd.x);
        const float dmin = kq_f16_to_f32_hw(r.hd.x >> 16);
        malformed |= !kq_isfinite(d) || !kq_isfinite(dmin);
        uint32_t s0, m0, s1, m1;
        kq_k_scale_pair(gq, r.hd.y, r.hd.z, r.hd.w, &s0, &m0, &s1, &m1);
        const float dl = d * (float)s0, ml = dmin * (float)m0;
        const float dh = d * (float)s1, mh = dmin * (float)m1;
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        const uint32_t h[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        const uint32_t bl = 2u * gq;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            lo[w] = kq_and_0f(q[w]) | (((h[w] >> bl) & 0x01010101u) << 4);
            hi[w] = kq_and_0f(q[w] >> 4) | (((h[w] >> (bl + 1u)) & 0x01010101u) << 4);
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float sl = 0.0f, sh = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                sl = dot4_u8(lo[w], &xl[b][4 * w], sl);
                sh = dot4_u8(hi[w], &xh[b][4 * w], sh);
            }
            float v = dl * sl;
            v = fmaf(-ml, sxl[b], v);
            v = fmaf(dh, sh, v);
            v = fmaf(-mh, sxh[b], v);
            acc[b] = v;
        }
    }
};

/* bit j of the low 4 bits of n into bit 8j (bits 0, 8, 16, 24) */
__device__ __forceinline__ uint32_t spread4(uint32_t n) {
    return kq_mul_u24(n & 15u, 0x00204081u) & 0x01010101u;
}

/* ---------------- Q5_1: 24 B blocks of 32 ---------------- */
/* f16 d @0, f16 m @2, qh (u32) @4, qs[16] @8 (src/kq_numeric.c:190-209):
 * code i = nibble | (bit i of qh) << 4, the low nibbles of qs[0..15] being
 * codes 0..15 and the high nibbles codes 16..31; weight = code * d + m. One
 * lane per block; blocks lie at multiples of 8 bytes. */
template <int B>
struct LaneQ51 {
    static constexpr uint32_t kBlockBytes = 24u;
    struct Raw {
        kq_u32x2 hdr;
        uint4 qs;
    };
    uint32_t off, k0;
    float xv[4][B][8], xsum[B];

    __device__ __forceinline__ void setup(uint32_t l) {
        off = kBlockBytes * l;
        k0 = 32u * l;
    }
    /* natural column of chunk c of lane l */
    __device__ static __forceinline__ uint32_t xk(uint32_t l, int c) {
        return 32u * l + 4u * (uint32_t)c;
    }
    __device__ __forceinline__ bool load_x(const float *x, uint32_t stride) {
        return load_x(XGlobal{x, stride});
    }
    template <class X>
    __device__ __forceinline__ bool load_x(const X &src) {
        bool bad = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) bad |= load_x8<B>(src, k0 + 8u * q, q, xv[q]);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float a = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < 8; ++i) a += xv[q][b][i];
            xsum[b] = a;
        }
        return bad;
    }
    template <int A>
    __device__ __forceinline__ Raw load(KqBufA<A> b, uint32_t row_off) const {
        Raw r;
        r.hdr = kq_ld64(b, row_off + off, 0u);
        r.qs = kq_ld128(b, row_off + off + 8u, 0u);
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        r.hdr = kq_u32x2{0u, 0u};
        r.qs = make_uint4(0, 0, 0, 0);
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float *acc, bool &malformed) const {
        const float d = kq_f16_to_f32_hw(r.hdr.x);
        const float m = kq_f16_to_f32_hw(r.hdr.x >> 16);
        malformed |= !kq_isfinite(d) || !kq_isfinite(m);
        const uint32_t qh = r.hdr.y;
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            lo[w] = kq_and_0f(q[w]) | (spread4(qh >> (4 * w)) << 4);
            hi[w] = kq_and_0f(q[w] >> 4) | (spread4(qh >> (16 + 4 * w)) << 4);
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                s = dot4_u8(lo[w], &xv[w >> 1][b][4 * (w & 1)], s);
                s = dot4_u8(hi[w], &xv[2 + (w >> 1)][b][4 * (w & 1)], s);
            }
            acc[b] = fmaf(d, s, m * xsum[b]);
        }
    }
};

/* ---------------- IQ4_NL: 18 B blocks of 32 ---------------- */
/* f16 d @0, qs[16] @2 (src/kq_numeric.c:278-292): weight = d * T[nibble],
 * T the 16-entry non-linear table; low nibbles of qs[0..15] are weights
 * 0..15, high nibbles 16..31. The lane looks codes up in T + 128 (unsigned
 * bytes) with v_perm_b32 and takes the bias off with the activation sum.
 * The block at bo (even) is read as a 16-byte window from bo - (bo & 3)
 * plus two 16-bit loads of its bytes 14..17: no read passes the block's
 * last byte, so the last block of a buffer stays inside it. */
constexpr uint32_t kIq4T0 = 0x3f2d1801u; /* T + 128 for codes 0..3 */
constexpr uint32_t kIq4T1 = 0x766a5d4fu; /* 4..7 */
constexpr uint32_t kIq4T2 = 0xa6998d81u; /* 8..11 */
constexpr uint32_t kIq4T3 = 0xf1d9c5b5u; /* 12..15 */

/* four table bytes for the four nibbles (0..15) held in the bytes of n */
__device__ __forceinline__ uint32_t iq4_lookup(uint32_t n, uint32_t t0, uint32_t t1,
                                               uint32_t t2, uint32_t t3) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t a = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t b = __builtin_amdgcn_perm(t3, t2, sel);
    const uint32_t msk = ((n >> 3) & 0x01010101u) * 0xffu;
    return (a & ~msk) | (b & msk);
}

template <int B>
struct LaneIQ4NL {
    static constexpr uint32_t kBlockBytes = 18u;
    struct Raw {
        uint4 w;
        uint32_t t0, t1, sh;
    };
    uint32_t off, k0;
    float xv[4][B][8], xsum[B];

    __device__ __forceinline__ void setup(uint32_t l) {
        off = kBlockBytes * l;
        k0 = 32u * l;
    }
    /* natural column of chunk c of lane l */
    __device__ static __forceinline__ uint32_t xk(uint32_t l, int c) {
        return 32u * l + 4u * (uint32_t)c;
    }
    __device__ __forceinline__ bool load_x(const float *x, uint32_t stride) {
        return load_x(XGlobal{x, stride});
    }
    template <class X>
    __device__ __forceinline__ bool load_x(const X &src) {
        bool bad = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) bad |= load_x8<B>(src, k0 + 8u * q, q, xv[q]);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float a = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < 8; ++i) a += xv[q][b][i];
            xsum[b] = a;
        }
        return bad;
    }
    template <int A>
    __device__ __forceinline__ Raw load(KqBufA<A> b, uint32_t row_off) const {
        const uint32_t bo = row_off + off;
        Raw r;
        r.sh = bo & 3u;
        r.w = kq_ld128(b, bo - r.sh, 0u);
        r.t0 = kq_ld16(b, bo + 14u, 0u);
        r.t1 = kq_ld16(b, bo + 16u, 0u);
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        r.w = make_uint4(0, 0, 0, 0);
        r.t0 = r.t1 = 0u;
        r.sh = 0u;
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float *acc, bool &malformed) const {
        const uint32_t w[4] = {r.w.x, r.w.y, r.w.z, r.w.w};
        const float d = kq_f16_to_f32_hw(r.sh ? (w[0] >> 16) : w[0]);
        malformed |= !kq_isfinite(d);
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            /* qs bytes 4k .. 4k+3, i.e. block bytes 2+4k .. 5+4k; the last
             * dword is block bytes 14..17 */
            const uint32_t q = k == 3 ? (r.t0 | (r.t1 << 16))
                               : r.sh ? w[k + 1] : kq_align2(w[k + 1], w[k], 2u);
            lo[k] = iq4_lookup(q & 0x0f0f0f0fu, kIq4T0, kIq4T1, kIq4T2, kIq4T3);
            hi[k] = iq4_lookup((q >> 4) & 0x0f0f0f0fu, kIq4T0, kIq4T1, kIq4T2, kIq4T3);
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                s = dot4_u8(lo[k], &xv[k >> 1][b][4 * (k & 1)], s);
                s = dot4_u8(hi[k], &xv[2 + (k >> 1)][b][4 * (k & 1)], s);
            }
            acc[b] = d * fmaf(-128.0f, xsum[b], s);
        }
    }
};

template <uint32_t TYPE, int B>
struct LaneFor;
template <int B>
struct LaneFor<12u, B> {
    using T = LaneQ4K<B>;
};
template <int B>
struct LaneFor<14u, B> {
    using T = LaneQ6K<B>;
};
template <int B>
struct LaneFor<8u, B> {
    using T = LaneQ8<B>;
};
template <int B>
struct LaneFor<13u, B> {
    using T = LaneQ5K<B>;
};
template <int B>
struct LaneFor<7u, B> {
    using T = LaneQ51<B>;
};
template <int B>
struct LaneFor<20u, B> {
    using T = LaneIQ4NL<B>;
};

/* 32-weight blocks (Q8_0, Q5_1, IQ4_NL): one lane per block; 256-weight
 * K-quant blocks: eight lanes per block */
template <uint32_t TYPE>
__host__ __device__ constexpr bool small_block() {
    return TYPE == 8u || TYPE == 7u || TYPE == 20u;
}

/* lanes per row for a format and column count */
template <uint32_t TYPE>
__host__ __device__ constexpr uint32_t lanes_per_row(uint32_t cols) {
    return small_block<TYPE>() ? cols / 32u : (cols / 256u) * 8u;
}

template <uint32_t TYPE>
__host__ __device__ constexpr uint32_t row_bytes(uint32_t cols) {
    return small_block<TYPE>() ? (cols / 32u) * LaneFor<TYPE, 1>::T::kBlockBytes
                               : (cols / 256u) * LaneFor<TYPE, 1>::T::kBlockBytes;
}

/*
 * Row-group engine. A wave covers RPW = 64/LPR rows side by side and RT
 * such passes per group (GROUP = RPW*RT rows). load_group issues every load
 * of a group; groups entirely below `rows` take the unguarded path.
 */
template <uint32_t TYPE, uint32_t COLS, int B, int RT, class LaneT = typename LaneFor<TYPE, B>::T>
struct Rows {
    using Lane = LaneT;
    using Raw = typename Lane::Raw;
    static constexpr uint32_t LPR = lanes_per_row<TYPE>(COLS);
    static_assert(LPR >= 1 && LPR <= 64 && 64 % LPR == 0, "row must fit a wave");
    static constexpr uint32_t RPW = 64u / LPR;
    static constexpr uint32_t GROUP = RPW * RT;
    static constexpr uint32_t RB = row_bytes<TYPE>(COLS);
    static constexpr uint32_t kCols = COLS;
    static constexpr int NV = RT * B; /* partial sums per lane */
    /* the butterfly halves the count at every level: pad to a power of two */
    static constexpr int N = NV <= 1 ? 1 : NV <= 2 ? 2 : NV <= 4 ? 4 : NV <= 8 ? 8
                             : NV <= 16 ? 16 : 32;
    static constexpr int KEEP = N > (int)LPR ? N / (int)LPR : 1; /* after reduction */

    /* stride: bytes from one row to the next (RB, or more when the rows
     * are column segments of longer rows) */
    template <int A>
    __device__ static __forceinline__ void load_group(const Lane &ln, KqBufA<A> W, uint32_t g,
                                                      uint32_t rows, uint32_t sub,
                                                      Raw (&raw)[RT], uint32_t stride = RB) {
        const uint32_t row0 = g * GROUP + sub;
        if ((g + 1u) * GROUP <= rows) {
#pragma unroll
            for (int r = 0; r < RT; ++r) raw[r] = ln.load(W, (row0 + (uint32_t)r * RPW) * stride);
        } else {
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const uint32_t row = row0 + (uint32_t)r * RPW;
                raw[r] = row < rows ? ln.load(W, row * stride) : ln.zero();
            }
        }
    }

    /* the same loads without a branch: rows past the matrix read from
     * `oob` (at least 64 bytes past the buffer's end, so every window of the
     * row lies outside it), which the hardware returns as zeros, the value
     * of zero() */
    template <int A>
    __device__ static __forceinline__ void load_group_oob(const Lane &ln, KqBufA<A> W, uint32_t g,
                                                          uint32_t rows, uint32_t sub,
                                                          Raw (&raw)[RT], uint32_t stride,
                                                          uint32_t oob) {
        const uint32_t row0 = g * GROUP + sub;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const uint32_t row = row0 + (uint32_t)r * RPW;
            raw[r] = ln.load(W, row < rows ? row * stride : oob);
        }
    }

    /* partial dots of a group, reduced over each row's LPR lanes; on return
     * lane l (within its row group) holds value index idx(l, j) in v[j] */
    __device__ static __forceinline__ void dot_group(const Lane &ln, const Raw (&raw)[RT],
                                                     uint32_t l, float (&v)[N],
                                                     bool &malformed) {
#pragma unroll
        for (int r = 0; r < RT; ++r) ln.dot(raw[r], &v[r * B], malformed);
#pragma unroll
        for (int i = NV; i < N; ++i) v[i] = 0.0f;
        kq_group_reduce<(int)LPR, N>(v, l);
    }

    /* value index held in v[j] by lane l, or -1 (duplicate holder, padding) */
    __device__ static __forceinline__ int value_index(uint32_t l, int j) {
        int idx;
        if constexpr (N <= (int)LPR) {
            constexpr uint32_t span = LPR / (uint32_t)N;
            idx = (l % span == 0u && j == 0) ? (int)(l / span) : -1;
        } else {
            idx = (int)l * KEEP + j;
        }
        return idx < NV ? idx : -1;
    }
};

/* Activation staging for kernels whose waves share one set of activations
 * (COLS columns of B batch columns at x + b * stride). The NT threads of a
 * workgroup copy them once into the LDS image read through XLds; issue()
 * only requests the loads, so the caller can request its weights before
 * anything waits, and commit() checks the values and writes the image
 * (then an LDS barrier). */
template <class R, int B, int NT>
struct XStage {
    static constexpr uint32_t LPR = R::LPR;
    static constexpr uint32_t NP = (uint32_t)B * 8u * LPR; /* float4 words */
    static constexpr int NX = (int)((NP + (uint32_t)NT - 1u) / (uint32_t)NT);
    kq_u32x4 v[NX];

    /* valid: the columns that exist (a row's last chunk may be shorter
     * than kCols); the others stage as zeros */
    __device__ __forceinline__ void issue(const float *x, uint32_t stride, uint32_t tid,
                                          uint32_t valid = R::kCols) {
        const uint32_t bytes = ((uint32_t)(B - 1) * stride + valid) * 4u;
        const KqBuf xb = kq_buf(x, bytes);
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const uint32_t p = tid + (uint32_t)i * (uint32_t)NT;
            const uint32_t b = p / (8u * LPR), c = (p / LPR) & 7u, l = p % LPR;
            const uint32_t k = R::Lane::xk(l, (int)c);
            const uint32_t off = p < NP && k < valid ? (b * stride + k) * 4u : bytes;
            v[i] = __builtin_amdgcn_raw_buffer_load_b128(xb.r, (int)off, 0, 0);
        }
    }
    __device__ __forceinline__ bool commit(float4 *xs, uint32_t tid) const {
        bool bad = false;
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const uint32_t p = tid + (uint32_t)i * (uint32_t)NT;
            if (NP % (uint32_t)NT == 0u || p < NP) {
                const float4 f = make_float4(__uint_as_float(v[i].x), __uint_as_float(v[i].y),
                                             __uint_as_float(v[i].z), __uint_as_float(v[i].w));
                bad |= !kq_isfinite(f.x) || !kq_isfinite(f.y) || !kq_isfinite(f.z) ||
                       !kq_isfinite(f.w);
                xs[p] = f;
            }
        }
        return bad;
    }
    template <class L>
    __device__ __forceinline__ void load(L &ln, const float4 *xs, uint32_t l) const {
        ln.load_x(XLds{xs, l, LPR});
    }
};

/* Activation staging for the digit lanes: the same loads as XStage, then
 * per group of G consecutive columns (G = Lane::kGroupCols, G/4 threads of
 * one float4 each) the largest magnitude m, k = min(22 - e, 149) for
 * m = f * 2^e with f in [0.5, 1) (so |x| * 2^k < 2^22), X = rint(x * 2^k),
 * its byte digits and the fp32 column sum (the int32 sum of X for lanes
 * with kIntSum). Unsigned digits are X's low three
 * bytes (the third one signed: bits 23..31 of X all equal its sign);
 * balanced digits are the low three bytes of (X + 0x8080) ^ 0x8080: D0 = X
 * mod 256 taken in [-128, 127], D1 the same of (X - D0) / 256, D2 of
 * (X - D0 - 256 D1) / 65536. A group's
 * record (plane words, then 2^-k and the sum; the lane type fixes the
 * order) goes to the one lane that reads it (Lane::home), at
 * [b][slot][lane] in 16-byte slots, so that consecutive lanes read
 * consecutive words. The image has the size of XStage's. */
template <class R, int B, int NT>
struct XStageI {
    using L = typename R::Lane;
    static constexpr uint32_t GS = L::kGroupCols;
    static constexpr uint32_t TPG = GS / 4u;             /* threads per group */
    static constexpr uint32_t NG = R::kCols / GS;        /* groups per batch column */
    static constexpr uint32_t LPR = R::LPR;
    static constexpr uint32_t NQ = (uint32_t)B * R::kCols / 4u; /* float4 items */
    static constexpr uint32_t NP = NQ;                  /* float4 words of the image */
    static constexpr int NX = (int)((NQ + (uint32_t)NT - 1u) / (uint32_t)NT);
    static_assert(TPG == 2u || TPG == 4u || TPG == 8u, "group of 8, 16 or 32 columns");
    static_assert(NT % 64 == 0 && R::kCols % GS == 0u, "a group's threads share a wave");
    static_assert(NP == (uint32_t)B * 8u * LPR, "the image holds 8 slots per lane");
    kq_u32x4 v[NX];

    __device__ __forceinline__ void issue(const float *x, uint32_t stride, uint32_t tid,
                                          uint32_t valid = R::kCols) {
        const uint32_t bytes = ((uint32_t)(B - 1) * stride + valid) * 4u;
        const KqBuf xb = kq_buf(x, bytes);
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const uint32_t p = tid + (uint32_t)i * (uint32_t)NT;
            const uint32_t b = p / (R::kCols / 4u), k = (p % (R::kCols / 4u)) * 4u;
            const uint32_t off = p < NQ && k < valid ? (b * stride + k) * 4u : bytes;
            v[i] = __builtin_amdgcn_raw_buffer_load_b128(xb.r, (int)off, 0, 0);
        }
    }
    __device__ __forceinline__ bool commit(float4 *xs, uint32_t tid) const {
        uint32_t *img = reinterpret_cast<uint32_t *>(xs);
        bool bad = false;
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const uint32_t p = tid + (uint32_t)i * (uint32_t)NT;
            /* uniform over a group's threads: NQ and NT are multiples of TPG */
            if (NQ % (uint32_t)NT == 0u || p < NQ) {
                const float f[4] = {__uint_as_float(v[i].x), __uint_as_float(v[i].y),
                                    __uint_as_float(v[i].z), __uint_as_float(v[i].w)};
                float m = 0.0f, sum = (f[0] + f[1]) + (f[2] + f[3]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    bad |= !kq_isfinite(f[j]);
                    m = fmaxf(m, fabsf(f[j]));
                }
                m = fmaxf(m, kq_dpp_pair<1>(m));
                sum += kq_dpp_pair<1>(sum);
                if constexpr (TPG >= 4u) {
                    m = fmaxf(m, kq_dpp_pair<2>(m));
                    sum += kq_dpp_pair<2>(sum);
                }
                if constexpr (TPG >= 8u) { /* quads are uniform: the mirror swaps them */
                    m = fmaxf(m, kq_dpp_pair<7>(m));
                    sum += kq_dpp_pair<7>(sum);
                }
                const int e = __builtin_amdgcn_frexp_expf(m);
                const int k = min(22 - e, 149);
                uint32_t X[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) X[j] = (uint32_t)(int)rintf(ldexpf(f[j], k));
                if constexpr (L::kIntSum) {
                    uint32_t is = (X[0] + X[1]) + (X[2] + X[3]);
                    is += kq_dpp_pair<1>(is);
                    if constexpr (TPG >= 4u) is += kq_dpp_pair<2>(is);
                    if constexpr (TPG >= 8u) is += kq_dpp_pair<7>(is);
                    sum = __uint_as_float(is);
                }
                if constexpr (L::kBalanced)
#pragma unroll
                    for (int j = 0; j < 4; ++j) X[j] = (X[j] + 0x8080u) ^ 0x8080u;
                const uint32_t p01 = __builtin_amdgcn_perm(X[1], X[0], 0x05010400u);
                const uint32_t p23 = __builtin_amdgcn_perm(X[3], X[2], 0x05010400u);
                const uint32_t w0 = __builtin_amdgcn_perm(p23, p01, 0x05040100u);
                const uint32_t w1 = __builtin_amdgcn_perm(p23, p01, 0x07060302u);
                const uint32_t w2 = __builtin_amdgcn_perm(X[1], X[0], 0x0c0c0602u) |
                                    __builtin_amdgcn_perm(X[3], X[2], 0x06020c0cu);
                const uint32_t gb = p / TPG, qd = p % TPG, b = gb / NG;
                uint32_t lane, slot;
                L::home(gb % NG, lane, slot);
                /* record dword i -> slot + i / 4, component i % 4 */
                auto put = [&](uint32_t i, uint32_t val) {
                    img[((b * 8u + slot + i / 4u) * LPR + lane) * 4u + i % 4u] = val;
                };
                put(qd, w0);
                put(TPG + qd, w1);
                put(2u * TPG + qd, w2);
                if (qd == 0u) {
                    put(3u * TPG, __float_as_uint(ldexpf(1.0f, -k)));
                    put(3u * TPG + 1u, __float_as_uint(sum));
                }
            }
        }
        return bad;
    }
    template <class Ln>
    __device__ __forceinline__ void load(Ln &ln, const float4 *xs, uint32_t l) const {
        ln.load_digits(reinterpret_cast<const uint4 *>(xs), l, LPR);
    }
};

/* the lane a matvec uses for a format: digit lanes for Q4_K, Q6_K, Q8_0 */
template <uint32_t TYPE, int B>
struct MatvecLane {
    using T = typename LaneFor<TYPE, B>::T;
};
template <int B>
struct MatvecLane<12u, B> {
    using T = LaneQ4KI<B>;
};
template <int B>
struct MatvecLane<14u, B> {
    using T = LaneQ6KI<B>;
};
template <int B>
struct MatvecLane<8u, B> {
    using T = LaneQ8I<B>;
};

/* the staging a lane reads: XStageI for lanes with kDigits, else XStage */
template <class L, class = void>
struct DigitLane {
    static constexpr bool value = false;
};
template <class L>
struct DigitLane<L, std::void_t<decltype(L::kDigits)>> {
    static constexpr bool value = L::kDigits;
};
template <class R, int B, int NT>
using StageFor = std::conditional_t<DigitLane<typename R::Lane>::value, XStageI<R, B, NT>,
                                    XStage<R, B, NT>>;

}  // namespace kq

#endif
