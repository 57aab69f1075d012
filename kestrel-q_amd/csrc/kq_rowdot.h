/*
 * kq_rowdot.h — per-lane pieces of a dequant-fused row dot, shared by the
 * matvec, LM-head and MoE expert kernels.
 *
 * A row of C columns is split over C/32 lanes; each lane owns 32 weights
 * and holds the matching activations for batch columns 0..B-1 in registers
 * (load_x), streams its slice of every row it visits (load) and returns
 * its partial dot (dot). The decode of each format follows
 * src/kq_numeric.c:176-295 (Q8_0, Q4_K) and the GGML Q6_K layout; the
 * per-sub-block scale is applied once to a sum of code*x products, and the
 * block offset (Q4_K dmin*m, Q6_K -32, Q8_0 +128 bias) is taken off with a
 * precomputed activation sum.
 */
#ifndef KQ_ROWDOT_H
#define KQ_ROWDOT_H

#include "kq_device.h"

namespace kq {

template <int B>
__device__ __forceinline__ bool load_x8(const float *x, uint32_t stride, uint32_t k,
                                        float (&dst)[B][8]) {
    bool bad = false;
#pragma unroll
    for (int b = 0; b < B; ++b) {
        const float4 *p = (const float4 *)(x + (size_t)b * stride + k);
        float4 u = p[0], v = p[1];
        dst[b][0] = u.x; dst[b][1] = u.y; dst[b][2] = u.z; dst[b][3] = u.w;
        dst[b][4] = v.x; dst[b][5] = v.y; dst[b][6] = v.z; dst[b][7] = v.w;
#pragma unroll
        for (int i = 0; i < 8; ++i) bad |= !kq_isfinite(dst[b][i]);
    }
    return bad;
}

/* 4 packed byte codes of w dotted with 4 activations, fp32 fused. */
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
    static constexpr uint32_t kLanesPerBlock = 8u;
    struct Raw {
        uint4 hd, qs;
    };
    uint32_t off;  /* byte offset of this lane's block within the row */
    uint32_t qoff; /* offset of its 16 qs bytes within the block */
    uint32_t gq;
    float xl[B][16], xh[B][16], sxl[B], sxh[B];

    /* l = lane index within the row (0 .. 8*blocks-1) */
    __device__ __forceinline__ bool init(uint32_t l, const float *x, uint32_t stride) {
        const uint32_t bb = l >> 3, c = l & 7u, h = c & 1u;
        gq = c >> 1;
        off = kBlockBytes * bb;
        qoff = 16u + 32u * gq + 16u * h;
        const uint32_t k0 = 256u * bb + 64u * gq + 16u * h;
        return load_x(x, stride, k0);
    }
    __device__ __forceinline__ bool load_x(const float *x, uint32_t stride, uint32_t k0) {
        float t0[B][8], t1[B][8], s0[B], s1[B];
        bool bad = load_x8<B>(x, stride, k0, t0);
        bad |= load_x8<B>(x, stride, k0 + 8u, t1);
        sum8<B>(t0, s0);
        sum8<B>(t1, s1);
#pragma unroll
        for (int b = 0; b < B; ++b) {
#pragma unroll
            for (int i = 0; i < 8; ++i) { xl[b][i] = t0[b][i]; xl[b][8 + i] = t1[b][i]; }
            sxl[b] = s0[b] + s1[b];
        }
        bad |= load_x8<B>(x, stride, k0 + 32u, t0);
        bad |= load_x8<B>(x, stride, k0 + 40u, t1);
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
    __device__ __forceinline__ Raw load(const uint8_t *row, const uint8_t *) const {
        Raw r;
        r.hd = *(const uint4 *)(row + off);
        r.qs = *(const uint4 *)(row + off + qoff);
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        r.hd = make_uint4(0, 0, 0, 0);
        r.qs = make_uint4(0, 0, 0, 0);
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float (&acc)[B], bool &malformed) const {
        const float d = kq_f16_to_f32(r.hd.x & 0xffffu);
        const float dmin = kq_f16_to_f32(r.hd.x >> 16);
        malformed |= !kq_isfinite(d) || !kq_isfinite(dmin);
        uint32_t s0, m0, s1, m1;
        kq_k_scale(2u * gq, r.hd.y, r.hd.z, r.hd.w, &s0, &m0);
        kq_k_scale(2u * gq + 1u, r.hd.y, r.hd.z, r.hd.w, &s1, &m1);
        const float dl = d * (float)s0, ml = dmin * (float)m0;
        const float dh = d * (float)s1, mh = dmin * (float)m1;
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float lo = 0.0f, hi = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                lo = dot4_u8(q[w] & 0x0f0f0f0fu, &xl[b][4 * w], lo);
                hi = dot4_u8((q[w] >> 4) & 0x0f0f0f0fu, &xh[b][4 * w], hi);
            }
            float v = dl * lo;
            v = fmaf(-ml, sxl[b], v);
            v = fmaf(dh, hi, v);
            v = fmaf(-mh, sxh[b], v);
            acc[b] = v;
        }
    }
};

/* ---------------- Q6_K: 210 B blocks of 256 ---------------- */
template <int B>
struct LaneQ6K {
    static constexpr uint32_t kBlockBytes = 210u;
    static constexpr uint32_t kLanesPerBlock = 8u;
    struct Raw {
        uint2 qa, qb, qh, sc;
        uint32_t d;
    };
    uint32_t off, n, t;
    float xq[4][B][8], xs[4][B];

    __device__ __forceinline__ bool init(uint32_t l, const float *x, uint32_t stride) {
        const uint32_t bb = l >> 3, s = l & 7u;
        n = s >> 2;
        t = s & 3u;
        off = kBlockBytes * bb;
        return load_x(x, stride, 256u * bb + 128u * n + 8u * t);
    }
    /* quarter q holds outputs k0 + 32q + 0..7 */
    __device__ __forceinline__ bool load_x(const float *x, uint32_t stride, uint32_t k0) {
        bool bad = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            bad |= load_x8<B>(x, stride, k0 + 32u * q, xq[q]);
            sum8<B>(xq[q], xs[q]);
        }
        return bad;
    }
    __device__ __forceinline__ Raw load(const uint8_t *row, const uint8_t *end) const {
        const uint8_t *p = row + off;
        Raw r;
        r.qa = kq_load8_u2a(p + 64u * n + 8u * t, end);
        r.qb = kq_load8_u2a(p + 64u * n + 32u + 8u * t, end);
        r.qh = kq_load8_u2a(p + 128u + 32u * n + 8u * t, end);
        r.sc = kq_load8_u2a(p + 192u + 8u * n, end);
        r.d = *(const uint16_t *)(p + 208u);
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        r.qa = r.qb = r.qh = r.sc = make_uint2(0, 0);
        r.d = 0u;
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float (&acc)[B], bool &malformed) const {
        const float d = kq_f16_to_f32(r.d);
        malformed |= !kq_isfinite(d);
        /* quarter q uses sc[8n + (t>>1) + 2q] */
        const uint32_t sh = (t >> 1) * 8u;
        const uint32_t sv[4] = {r.sc.x >> sh, r.sc.x >> (sh + 16u), r.sc.y >> sh,
                                r.sc.y >> (sh + 16u)};
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
            const uint32_t A = half ? r.qa.y : r.qa.x;
            const uint32_t Bq = half ? r.qb.y : r.qb.x;
            const uint32_t H = half ? r.qh.y : r.qh.x;
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
template <int B>
struct LaneQ8 {
    static constexpr uint32_t kBlockBytes = 34u;
    static constexpr uint32_t kLanesPerBlock = 1u;
    struct Raw {
        uint32_t d;
        uint32_t c[8];
    };
    uint32_t off;
    float xv[4][B][8], xsum[B];

    __device__ __forceinline__ bool init(uint32_t l, const float *x, uint32_t stride) {
        off = kBlockBytes * l;
        return load_x(x, stride, 32u * l);
    }
    __device__ __forceinline__ bool load_x(const float *x, uint32_t stride, uint32_t k0) {
        bool bad = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) bad |= load_x8<B>(x, stride, k0 + 8u * q, xv[q]);
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
    __device__ __forceinline__ Raw load(const uint8_t *row, const uint8_t *end) const {
        const uint8_t *p = row + off;
        Raw r;
        r.d = *(const uint16_t *)p;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint2 u = kq_load8_u2a(p + 2u + 8u * j, end);
            r.c[2 * j] = u.x;
            r.c[2 * j + 1] = u.y;
        }
        return r;
    }
    __device__ __forceinline__ Raw zero() const {
        Raw r;
        r.d = 0u;
#pragma unroll
        for (int j = 0; j < 8; ++j) r.c[j] = 0x80808080u;
        return r;
    }
    __device__ __forceinline__ void dot(const Raw &r, float (&acc)[B], bool &malformed) const {
        const float d = kq_f16_to_f32(r.d);
        malformed |= !kq_isfinite(d);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            /* int8 code + 128 as an unsigned byte; the bias comes off with
             * the activation sum */
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                s = dot4_u8(r.c[j] ^ 0x80808080u, &xv[j >> 1][b][4 * (j & 1)], s);
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

/* lanes per row for a format and column count */
template <uint32_t TYPE>
__host__ __device__ constexpr uint32_t lanes_per_row(uint32_t cols) {
    return TYPE == 8u ? cols / 32u : (cols / 256u) * 8u;
}

template <uint32_t TYPE>
__host__ __device__ constexpr uint32_t row_bytes(uint32_t cols) {
    return TYPE == 8u ? (cols / 32u) * 34u : (cols / 256u) * (TYPE == 12u ? 144u : 210u);
}

}  // namespace kq

#endif
