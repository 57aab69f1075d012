/*
 * kq_grouped.hip — the multi-token (prefill) MoE layer as grouped expert
 * GEMMs on MFMA: a stable token->expert permutation, one gate/up + SwiGLU
 * pass and one down pass per expert over all of its tokens, and the ordered
 * combine with the sigmoid-gated shared expert.
 *
 * The reference runs the layer token by token (kq_moe_execute_common,
 * src/kq_moe_qwen38.c:666-865): for each token, route, then for every
 * selected expert in ascending id g = Wg x, u = Wu x, a = swiglu(g, u),
 * o = Wd a, routed_sum += o * w (:722-765), and out = routed_sum +
 * sigmoid(wsg . x) * shared(x) (:771-828). With T tokens every expert's
 * weights would stream once per token that selects it. Here each expert's
 * weights stream once for all of its tokens:
 *
 *   permute  offsets[e], and the (token, slot) pairs of expert e at
 *            positions offsets[e].. in ascending token order (a stable
 *            counting sort; bit-exact by construction)
 *   gate/up  act[pos] = swiglu(Wg_e x_t, Wu_e x_t) for every position of e
 *   down     o[pos] = Wd_e act[pos]
 *   combine  out[t] = sum over t's slots in ascending expert id of
 *            o[pos] * w, then + sigmoid(shared logit) * o_shared[t]
 *
 * GEMM numerics. Weight codes are small integers, exact in fp16, so the
 * quantized weights enter the MFMA exactly:
 *   Q4_K  the 6-bit sub-block scale s is folded into the code (s * q <=
 *         945, exact) with one packed fp16 FMA that also removes the
 *         1024 exponent bias of the byte->fp16 conversion; the super-block
 *         scale d multiplies the fp32 accumulator once per 256 columns and
 *         the dmin * m term is a second small MFMA against per-sub-block
 *         activation sums;
 *   Q6_K  the code q - 32 is exact; each 16-column sub-block is one
 *         16x16x16 MFMA step whose fp32 result is scaled by d * sc.
 * Activations are split per token into fp16 hi + lo (x = hi + lo to ~22
 * bits) after an exact power-of-two scaling that puts the row's largest
 * magnitude in [2^14, 2^15), so neither part overflows and small rows keep
 * their precision; every MFMA accumulates in fp32. Outputs are compared
 * with the CPU by tolerance (per element, 1e-4 absolute or 1e-3 relative).
 *
 * MFMA operands: A = activations (16 tokens x K), B = weights (K x 16
 * rows); lane l holds token / row l % 16 and a k-group l / 16, and the
 * result D[token][row] leaves lane l with row l % 16 of tokens
 * 4 (l / 16) .. + 3. Which hidden columns a k-slot of a step holds is free
 * as long as A and B agree; it is chosen per format so that each lane's
 * weight bytes are contiguous and share one scale.
 */
#include "kq_launch.h"
#include "kq_device.h"
#include "kq_dma.h"

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kTile = 16;          /* tokens per M-chunk, rows per N-tile */
constexpr uint32_t kMagic = 0x64646464u; /* fp16 0x64XX = 1024 + XX */

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u(h2 v) { return __builtin_bit_cast(uint32_t, v); }

/* bytes b0, b1 (sel 0x04010400) or b2, b3 (sel 0x04030402) of m as fp16
 * 1024 + byte */
__device__ __forceinline__ h2 bytes_lo(uint32_t m) {
    return as_h2(__builtin_amdgcn_perm(kMagic, m, 0x04010400u));
}
__device__ __forceinline__ h2 bytes_hi(uint32_t m) {
    return as_h2(__builtin_amdgcn_perm(kMagic, m, 0x04030402u));
}

__device__ __forceinline__ h2 fma2(h2 a, h2 b, h2 c) { return __builtin_elementwise_fma(a, b, c); }

__device__ __forceinline__ float f16f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu));
}

__device__ __forceinline__ float wave_max_abs(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, KQ_WAVE));
    return v;
}

/* ------------------------------------------------------------------ */
/* formats */

template <uint32_t FMT>
struct Fmt;

/* Q4_K: 144 B per 256 columns (d, dmin, 12 B of 6-bit scales/mins, 128 B
 * of nibbles; src/kq_numeric.c:223-277). Lane k-group g reads nibble group
 * g (qs bytes 32g..32g+31: sub-blocks 2g in the low nibbles, 2g+1 in the
 * high) of its row; step s (0..7) of a block covers hidden columns
 * 64g + 8s .. +7, low nibbles for s < 4, high nibbles for s >= 4. */
template <>
struct Fmt<KQ_LAUNCH_Q4_K> {
    static constexpr uint32_t kUnit = 256u;       /* columns per pass iteration */
    static constexpr uint32_t kUnitBytes = 144u;
    static constexpr bool kSums = true;           /* 32-column activation sums */
    static constexpr bool kK32 = true; /* 16x16x32 steps, b128 activation reads */
    struct Raw {
        uint4 hd, qa, qb;
    };
    __device__ static __forceinline__ Raw load(KqBuf w, uint32_t boff, uint32_t g) {
        Raw r;
        r.hd = kq_ld128(w, boff, 0u);
        r.qa = kq_ld128(w, boff + 16u + 32u * g, 0u);
        r.qb = kq_ld128(w, boff + 32u + 32u * g, 0u);
        return r;
    }
};

/* Q6_K: 210 B per 256 columns (ql[128], qh[64], int8 sc[16], f16 d; GGML
 * layout). Sub-block s = 8n + 2q + h (half n, quarter q, 16-column half
 * h) is one 16x16x16 step; lane k-group g holds its columns 4g .. 4g+3,
 * i.e. hidden 128n + 32q + 16h + 4g .. +3, whose codes come from the ql
 * dwords at 64n + 16h + 4g (q = 0, 2) and 64n + 32 + 16h + 4g (q = 1, 3)
 * and the qh dword at 128 + 32n + 16h + 4g. A block at an offset of 2 mod
 * 4 is read through aligned windows re-aligned with a byte funnel shift;
 * no window leaves the block. */
template <>
struct Fmt<KQ_LAUNCH_Q6_K> {
    static constexpr uint32_t kBytes = 210u;
    static constexpr uint32_t kUnit = 256u;
    static constexpr uint32_t kUnitBytes = 210u;
    static constexpr bool kSums = false;
    static constexpr bool kK32 = false;
    struct Raw {
        kq_u32x2 w[4][3]; /* [n * 2 + h][ql A, ql B, qh] */
        uint4 sc;         /* window over sc[16] */
        uint32_t sc_tail, d, sh;
    };
    __device__ static __forceinline__ Raw load(KqBuf w, uint32_t boff, uint32_t g) {
        Raw r;
        r.sh = boff & 3u;
        const uint32_t base = boff - r.sh;
#pragma unroll
        for (uint32_t nh = 0; nh < 4u; ++nh) {
            const uint32_t n = nh >> 1, h = nh & 1u;
            const uint32_t oa = 64u * n + 16u * h + 4u * g;
            r.w[nh][0] = kq_ld64(w, base + oa, 0u);
            r.w[nh][1] = kq_ld64(w, base + oa + 32u, 0u);
            r.w[nh][2] = kq_ld64(w, base + 128u + 32u * n + 16u * h + 4u * g, 0u);
        }
        /* sc[16] at 192: [192, 208) when aligned, else [190, 210); the
         * tail word is loaded on every path (a branch here would split the
         * wave) and only used for an unaligned block */
        r.sc = kq_ld128(w, base + 192u, 0u);
        r.sc_tail = kq_ld32(w, base + 208u, 0u);
        r.d = kq_ld16(w, boff + 208u, 0u);
        return r;
    }
};

/* Q8_0: 34 B per 32 columns (f16 d, 32 int8 codes; src/kq_numeric.c:
 * 176-196). An iteration takes two blocks (64 columns); each block is one
 * 16x16x32 step, lane k-group g holding its columns 8g .. 8g + 7, i.e. code
 * bytes 2 + 8g .. 9 + 8g. The first block's codes start at 2 mod 4, so they
 * come from a 12-byte window re-aligned by two bytes; each scale is half of
 * an aligned dword. Rows are whole units of 68 B, so a unit starts 4-byte
 * aligned. */
template <>
struct Fmt<KQ_LAUNCH_Q8_0> {
    static constexpr uint32_t kUnit = 64u;
    static constexpr uint32_t kUnitBytes = 68u;
    static constexpr bool kSums = false;
    static constexpr bool kK32 = true;
    struct Raw {
        kq_u32x3 c[2]; /* code windows of the two blocks */
        uint32_t d[2]; /* dwords holding the scales */
    };
    __device__ static __forceinline__ Raw load(KqBuf w, uint32_t uoff, uint32_t g) {
        Raw r;
#pragma unroll
        for (uint32_t bb = 0; bb < 2u; ++bb) {
            const uint32_t a = uoff + 34u * bb + 2u + 8u * g; /* codes */
            r.c[bb] = kq_ld96(w, a & ~3u, 0u);
            r.d[bb] = kq_ld32(w, (uoff + 34u * bb) & ~3u, 0u);
        }
        return r;
    }
};

/* Q5_1: 24 B per 32 columns (f16 d, f16 m, 32 high bits qh, 16 bytes of
 * nibbles: low nibble of byte i = element i, high = element i + 16, bit i
 * of qh = bit 4 of element i; src/kq_numeric.c:197-222). Four blocks per
 * iteration (96 B); lane k-group g holds elements 8g .. 8g + 7: nibbles of
 * bytes 8(g & 1) .. +7 (low for g < 2, high otherwise) and qh byte g. */
template <>
struct Fmt<KQ_LAUNCH_Q5_1> {
    static constexpr uint32_t kUnit = 128u;
    static constexpr uint32_t kUnitBytes = 96u;
    static constexpr bool kSums = true;
    static constexpr bool kK32 = true;
    struct Raw {
        kq_u32x2 q[4];
        uint32_t dm[4], qh[4];
    };
    __device__ static __forceinline__ Raw load(KqBuf w, uint32_t uoff, uint32_t g) {
        Raw r;
#pragma unroll
        for (uint32_t bb = 0; bb < 4u; ++bb) {
            const uint32_t o = uoff + 24u * bb;
            r.dm[bb] = kq_ld32(w, o, 0u);
            r.qh[bb] = kq_ld32(w, o + 4u, 0u);
            r.q[bb] = kq_ld64(w, o + 8u + 8u * (g & 1u), 0u);
        }
        return r;
    }
};

/* ------------------------------------------------------------------ */
/* LDS image of one M-chunk of activations */

template <uint32_t FMT, uint32_t KDIM>
struct Stage {
    /* row pitch in fp16: b128 reads (K32 steps) want a 16-byte skew per
     * row, b64 reads an 8-byte one, so that 8 / 16 lanes on consecutive
     * rows hit distinct banks */
    static constexpr uint32_t kPitch = KDIM + (Fmt<FMT>::kK32 ? 8u : 4u);
    static constexpr uint32_t kSub = KDIM / 32u; /* Q4_K sub-blocks per row */
    static constexpr uint32_t kSxPitch = kSub + 8u;
    static constexpr bool kSums = Fmt<FMT>::kSums;
    __align__(16) _Float16 xh[kTile * kPitch];
    __align__(16) _Float16 xl[kTile * kPitch];
    __align__(16) _Float16 sxh[kSums ? kTile * kSxPitch : 4];
    __align__(16) _Float16 sxl[kSums ? kTile * kSxPitch : 4];
    int sig[kTile];
};

/* Stage columns col0 .. col0 + KSL - 1 of rows src_row[i] (or zeros where
 * negative) of X [*, KDIM]: scale by 2^sig (the row's largest magnitude,
 * over all KDIM columns, into [2^14, 2^15), so every slice of a row gets
 * the same scale), split into fp16 hi + lo and, for formats with a min
 * term, form the 32-column sums of the scaled row times 2^-5 (so they fit
 * fp16), also split. One wave per row; lane l holds the float4 column
 * groups l, l + 64, ..., so that both the global reads and the LDS writes
 * of a wave are contiguous (no bank conflicts). Returns true if a
 * non-finite input was seen. col0 and KSL are multiples of 32. */
template <uint32_t FMT, uint32_t KDIM, uint32_t KSL>
__device__ bool stage_slice(Stage<FMT, KSL> &st, const float *__restrict__ X, uint32_t col0,
                            const int *src_row, uint32_t wave, uint32_t nwaves, uint32_t lane) {
    using S = Stage<FMT, KSL>;
    constexpr uint32_t NQ = (KDIM + 255u) / 256u;   /* float4 groups per lane, whole row */
    constexpr uint32_t NQS = (KSL + 255u) / 256u + (KSL % 256u != 0u ? 1u : 0u); /* a slice */
    bool bad = false;
    for (uint32_t i = wave; i < kTile; i += nwaves) {
        const int src = src_row[i];
        const float4 *p = (const float4 *)(X + (size_t)(src < 0 ? 0 : src) * KDIM) + lane;
        int sig;
        bool any_nf = false;
        if (col0 == 0u) {
            /* the scale, from the whole row (later slices of this chunk reuse
             * it, so every slice gets the same one) */
            float m = 0.0f;
            bool nf = false;
#pragma unroll 8
            for (uint32_t q = 0; q < NQ; ++q) {
                const bool in = src >= 0 && 256u * q + 4u * lane < KDIM;
                const float4 v = in ? p[64u * q] : make_float4(0.f, 0.f, 0.f, 0.f);
                nf |= !kq_isfinite(v.x) || !kq_isfinite(v.y) || !kq_isfinite(v.z) ||
                      !kq_isfinite(v.w);
                m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
            bad |= nf;
            m = wave_max_abs(m);
            any_nf = __ballot(nf) != 0ull;
            /* m = f * 2^e, f in [0.5, 1): m * 2^(15 - e) lies in [2^14, 2^15) */
            sig = 0;
            if (!any_nf && m > 0.0f) sig = 15 - __builtin_amdgcn_frexp_expf(m);
            if (any_nf) sig = 0x7fffffff; /* a row staged as zeros */
        } else {
            sig = st.sig[i];
            any_nf = sig == 0x7fffffff;
        }
        const uint32_t q0 = col0 / 256u;
        float4 v[NQS];
#pragma unroll
        for (uint32_t qq = 0; qq < NQS; ++qq) {
            const uint32_t col = 256u * (q0 + qq) + 4u * lane;
            const bool in = src >= 0 && col < KDIM;
            v[qq] = in ? p[64u * (q0 + qq)] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (uint32_t qq = 0; qq < NQS; ++qq) {
            const uint32_t col = 256u * (q0 + qq) + 4u * lane;
            const bool mine = col >= col0 && col < col0 + KSL;
            const float a[4] = {v[qq].x, v[qq].y, v[qq].z, v[qq].w};
            _Float16 hi[4], lo[4];
            float part = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float xs = any_nf ? 0.0f : ldexpf(a[c], sig);
                hi[c] = (_Float16)xs;
                lo[c] = (_Float16)(xs - (float)hi[c]);
                part += xs;
            }
            if (mine) {
                *(h4 *)(st.xh + i * S::kPitch + (col - col0)) = h4{hi[0], hi[1], hi[2], hi[3]};
                *(h4 *)(st.xl + i * S::kPitch + (col - col0)) = h4{lo[0], lo[1], lo[2], lo[3]};
            }
            if constexpr (S::kSums) {
                /* 32-column sums: 8 consecutive lanes hold one */
                part += __shfl_xor(part, 1, KQ_WAVE);
                part += __shfl_xor(part, 2, KQ_WAVE);
                part += __shfl_xor(part, 4, KQ_WAVE);
                if (mine && (lane & 7u) == 0u) {
                    const float s = part * 0.03125f;
                    const _Float16 sh = (_Float16)s;
                    const _Float16 sl = (_Float16)(s - (float)sh);
                    const uint32_t jsb = (col - col0) / 32u;
                    st.sxh[i * S::kSxPitch + jsb] = sh;
                    st.sxl[i * S::kSxPitch + jsb] = sl;
                }
            }
        }
        if (lane == 0u) st.sig[i] = sig;
    }
    return bad;
}

template <uint32_t FMT, uint32_t KDIM>
__device__ bool stage_rows(Stage<FMT, KDIM> &st, const float *__restrict__ X,
                           const int *src_row, uint32_t wave, uint32_t nwaves, uint32_t lane) {
    return stage_slice<FMT, KDIM, KDIM>(st, X, 0u, src_row, wave, nwaves, lane);
}

/* ------------------------------------------------------------------ */
/* one 16-row N-tile of NMAT matrices (gate and up share the activation
 * fragments of every step) against the staged 16-token chunk; acc[m] gets
 * block b of matrix m */

template <uint32_t FMT, uint32_t KDIM, int NMAT>
struct Tile;

template <uint32_t KDIM, int NMAT>
struct Tile<KQ_LAUNCH_Q4_K, KDIM, NMAT> {
    using F = Fmt<KQ_LAUNCH_Q4_K>;
    using S = Stage<KQ_LAUNCH_Q4_K, KDIM>;
    using Raw = F::Raw;

    __device__ static __forceinline__ void block(const Raw (&r)[NMAT], const S &st, uint32_t b,
                                                 uint32_t i, uint32_t g, f4 (&acc)[NMAT],
                                                 bool &malformed) {
        float d[NMAT], dm[NMAT];
        h2 S0[NMAT], C0[NMAT], S1[NMAT], C1[NMAT];
        h4 bm[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            d[m] = f16f(r[m].hd.x);
            const float dmin = f16f(r[m].hd.x >> 16);
            malformed |= !kq_isfinite(d[m]) || !kq_isfinite(dmin);
            dm[m] = dmin * 32.0f; /* the activation sums carry 2^-5 */
            /* scales of sub-blocks 2g and 2g+1 (src/kq_numeric.c:161-174) */
            const uint32_t u = r[m].hd.y >> (16u * (g & 1u)); /* q[2(g&1)], q[2(g&1)+1] */
            const uint32_t w = r[m].hd.w >> (16u * (g & 1u)); /* q[8+2(g&1)], q[9+2(g&1)] */
            uint32_t s0, s1;
            if (g < 2u) {
                s0 = u & 63u;
                s1 = (u >> 8) & 63u;
            } else {
                s0 = (w & 15u) | ((u >> 2) & 0x30u);
                s1 = ((w >> 8) & 15u) | ((u >> 10) & 0x30u);
            }
            const _Float16 fs0 = (_Float16)(float)s0, fs1 = (_Float16)(float)s1;
            S0[m] = h2{fs0, fs0};
            C0[m] = S0[m] * h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
            S1[m] = h2{fs1, fs1} * h2{(_Float16)0.0625f, (_Float16)0.0625f};
            C1[m] = h2{fs1, fs1} * h2{(_Float16)-64.0f, (_Float16)-64.0f};
            /* mins m_4g .. m_4g+3 for g < 2 (the min-term weights); 0 for g >= 2 */
            const uint32_t mq =
                g == 0u ? (r[m].hd.z & 0x3f3f3f3fu)
                        : (((r[m].hd.w >> 4) & 0x0f0f0f0fu) | ((r[m].hd.z >> 2) & 0x30303030u));
            const h2 one = h2{(_Float16)1.0f, (_Float16)1.0f};
            const h2 neg = h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
            h2 mlo = fma2(bytes_lo(mq), one, neg), mhi = fma2(bytes_hi(mq), one, neg);
            if (g >= 2u) {
                mlo = h2{(_Float16)0.0f, (_Float16)0.0f};
                mhi = mlo;
            }
            bm[m] = h4{mlo.x, mlo.y, mhi.x, mhi.y};
        }
        f4 q[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) q[m] = f4{0.f, 0.f, 0.f, 0.f};
        const _Float16 *xh = st.xh + i * S::kPitch + 256u * b + 64u * g;
        const _Float16 *xl = st.xl + i * S::kPitch + 256u * b + 64u * g;
#pragma unroll
        for (uint32_t s = 0; s < 8u; ++s) {
            const h8 ah = *(const h8 *)(xh + 8u * s);
            const h8 al = *(const h8 *)(xl + 8u * s);
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                const uint4 &qd = (s & 2u) ? r[m].qb : r[m].qa;
                const uint32_t raw0 = (s & 1u) ? qd.z : qd.x, raw1 = (s & 1u) ? qd.w : qd.y;
                const uint32_t m0 = s < 4u ? kq_and_0f(raw0) : kq_and_f0(raw0);
                const uint32_t m1 = s < 4u ? kq_and_0f(raw1) : kq_and_f0(raw1);
                const h2 Sc = s < 4u ? S0[m] : S1[m], Cc = s < 4u ? C0[m] : C1[m];
                const h2 w0 = fma2(bytes_lo(m0), Sc, Cc), w1 = fma2(bytes_hi(m0), Sc, Cc);
                const h2 w2 = fma2(bytes_lo(m1), Sc, Cc), w3 = fma2(bytes_hi(m1), Sc, Cc);
                const h8 bw = h8{w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
                q[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bw, q[m], 0, 0, 0);
                q[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bw, q[m], 0, 0, 0);
            }
            /* keep each step's fragments short-lived: without this the
             * scheduler hoists every step's LDS reads and runs out of VGPRs */
            __builtin_amdgcn_sched_barrier(0);
        }
        /* min term: sum_j m_j * (32-column sums * 2^-5) */
        const uint32_t so = i * S::kSxPitch + 8u * b + 4u * (g & 1u);
        const h4 sh4 = *(const h4 *)(st.sxh + so);
        const h4 sl4 = *(const h4 *)(st.sxl + so);
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            f4 mm = {0.f, 0.f, 0.f, 0.f};
            mm = __builtin_amdgcn_mfma_f32_16x16x16f16(sh4, bm[m], mm, 0, 0, 0);
            mm = __builtin_amdgcn_mfma_f32_16x16x16f16(sl4, bm[m], mm, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[m][t] = fmaf(d[m], q[m][t], fmaf(-dm[m], mm[t], acc[m][t]));
        }
    }
};

template <uint32_t KDIM, int NMAT>
struct Tile<KQ_LAUNCH_Q6_K, KDIM, NMAT> {
    using F = Fmt<KQ_LAUNCH_Q6_K>;
    using S = Stage<KQ_LAUNCH_Q6_K, KDIM>;
    using Raw = F::Raw;

    __device__ static __forceinline__ void block(const Raw (&r)[NMAT], const S &st, uint32_t b,
                                                 uint32_t i, uint32_t g, f4 (&acc)[NMAT],
                                                 bool &malformed) {
        float d[NMAT];
        uint32_t sc[NMAT][4];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            d[m] = f16f(r[m].d);
            malformed |= !kq_isfinite(d[m]);
            const uint32_t sh = r[m].sh ? 2u : 0u;
            sc[m][0] = kq_align2(r[m].sc.y, r[m].sc.x, sh);
            sc[m][1] = kq_align2(r[m].sc.z, r[m].sc.y, sh);
            sc[m][2] = kq_align2(r[m].sc.w, r[m].sc.z, sh);
            sc[m][3] = kq_align2(r[m].sc_tail, r[m].sc.w, sh);
            if (!r[m].sh) {
                sc[m][0] = r[m].sc.x;
                sc[m][1] = r[m].sc.y;
                sc[m][2] = r[m].sc.z;
                sc[m][3] = r[m].sc.w;
            }
        }
        const h2 bias = h2{(_Float16)-1056.0f, (_Float16)-1056.0f}; /* 1024 + 32 */
        const _Float16 *xh = st.xh + i * S::kPitch + 256u * b + 4u * g;
        const _Float16 *xl = st.xl + i * S::kPitch + 256u * b + 4u * g;
#pragma unroll
        for (uint32_t nh = 0; nh < 4u; ++nh) {
            const uint32_t n = nh >> 1, h = nh & 1u;
            uint32_t c[NMAT][4];
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                const uint32_t A = kq_align2(r[m].w[nh][0].y, r[m].w[nh][0].x, r[m].sh);
                const uint32_t B = kq_align2(r[m].w[nh][1].y, r[m].w[nh][1].x, r[m].sh);
                const uint32_t H = kq_align2(r[m].w[nh][2].y, r[m].w[nh][2].x, r[m].sh);
                c[m][0] = (A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
                c[m][1] = (B & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
                c[m][2] = ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u);
                c[m][3] = ((B >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
            }
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q) {
                const uint32_t s = 8u * n + 2u * q + h;
                const uint32_t ko = 128u * n + 32u * q + 16u * h;
                const h4 ah = *(const h4 *)(xh + ko);
                const h4 al = *(const h4 *)(xl + ko);
#pragma unroll
                for (int m = 0; m < NMAT; ++m) {
                    const h2 w0 = bytes_lo(c[m][q]) + bias, w1 = bytes_hi(c[m][q]) + bias;
                    const h4 bw = h4{w0.x, w0.y, w1.x, w1.y};
                    f4 t = {0.f, 0.f, 0.f, 0.f};
                    t = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bw, t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bw, t, 0, 0, 0);
                    const int8_t scv = (int8_t)((sc[m][s >> 2] >> (8u * (s & 3u))) & 0xffu);
                    const float ds = d[m] * (float)scv;
#pragma unroll
                    for (int k = 0; k < 4; ++k) acc[m][k] = fmaf(ds, t[k], acc[m][k]);
                }
            }
            /* as in the Q4_K tile: bound how far fragment reads are hoisted */
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

template <uint32_t KSL, int NMAT>
struct Tile<KQ_LAUNCH_Q8_0, KSL, NMAT> {
    using F = Fmt<KQ_LAUNCH_Q8_0>;
    using S = Stage<KQ_LAUNCH_Q8_0, KSL>;
    using Raw = F::Raw;

    /* iteration b: blocks 2b, 2b + 1 of the slice, one step each; the
     * int8 codes enter as fp16 through the offset-binary byte (q + 128) */
    __device__ static __forceinline__ void block(const Raw (&r)[NMAT], const S &st, uint32_t b,
                                                 uint32_t i, uint32_t g, f4 (&acc)[NMAT],
                                                 bool &malformed) {
        const _Float16 *xh = st.xh + i * S::kPitch + 64u * b + 8u * g;
        const _Float16 *xl = st.xl + i * S::kPitch + 64u * b + 8u * g;
        const h2 bias = h2{(_Float16)-1152.0f, (_Float16)-1152.0f}; /* 1024 + 128 */
#pragma unroll
        for (uint32_t bb = 0; bb < 2u; ++bb) {
            const h8 ah = *(const h8 *)(xh + 32u * bb);
            const h8 al = *(const h8 *)(xl + 32u * bb);
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                const kq_u32x3 wv = r[m].c[bb];
                /* codes start 2 bytes into the window of even blocks */
                uint32_t c0 = (bb & 1u) ? wv.x : kq_align2(wv.y, wv.x, 2u);
                uint32_t c1 = (bb & 1u) ? wv.y : kq_align2(wv.z, wv.y, 2u);
                c0 ^= 0x80808080u;
                c1 ^= 0x80808080u;
                const h2 w0 = bytes_lo(c0) + bias, w1 = bytes_hi(c0) + bias;
                const h2 w2 = bytes_lo(c1) + bias, w3 = bytes_hi(c1) + bias;
                const h8 bw = h8{w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
                f4 t = {0.f, 0.f, 0.f, 0.f};
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bw, t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bw, t, 0, 0, 0);
                const float d = f16f((bb & 1u) ? r[m].d[bb] >> 16 : r[m].d[bb]);
                malformed |= !kq_isfinite(d);
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[m][k] = fmaf(d, t[k], acc[m][k]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

template <uint32_t KSL, int NMAT>
struct Tile<KQ_LAUNCH_Q5_1, KSL, NMAT> {
    using F = Fmt<KQ_LAUNCH_Q5_1>;
    using S = Stage<KQ_LAUNCH_Q5_1, KSL>;
    using Raw = F::Raw;

    /* bit k of x (k < 4) to bit 8k + 4: the fifth bit of four codes */
    __device__ static __forceinline__ uint32_t spread4(uint32_t x) {
        return (kq_mul_u24(x, 0x00204081u) & 0x01010101u) << 4;
    }

    /* iteration b: blocks 4b .. 4b + 3 of the slice; codes 0..31 are
     * exact in fp16, d scales the step and m the block's activation sum */
    __device__ static __forceinline__ void block(const Raw (&r)[NMAT], const S &st, uint32_t b,
                                                 uint32_t i, uint32_t g, f4 (&acc)[NMAT],
                                                 bool &malformed) {
        const _Float16 *xh = st.xh + i * S::kPitch + 128u * b + 8u * g;
        const _Float16 *xl = st.xl + i * S::kPitch + 128u * b + 8u * g;
        const h2 bias = h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
#pragma unroll
        for (uint32_t bb = 0; bb < 4u; ++bb) {
            const h8 ah = *(const h8 *)(xh + 32u * bb);
            const h8 al = *(const h8 *)(xl + 32u * bb);
            /* this lane's four tokens' sums of the block (times 2^-5) */
            float sx[4];
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q) {
                const uint32_t so = (4u * g + q) * S::kSxPitch + 4u * b + bb;
                sx[q] = (float)st.sxh[so] + (float)st.sxl[so];
            }
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                const kq_u32x2 qv = r[m].q[bb];
                const uint32_t shn = g >= 2u ? 4u : 0u;
                const uint32_t hb = (r[m].qh[bb] >> (8u * g)) & 0xffu;
                const uint32_t c0 = ((qv.x >> shn) & 0x0f0f0f0fu) | spread4(hb & 15u);
                const uint32_t c1 = ((qv.y >> shn) & 0x0f0f0f0fu) | spread4(hb >> 4);
                const h2 w0 = bytes_lo(c0) + bias, w1 = bytes_hi(c0) + bias;
                const h2 w2 = bytes_lo(c1) + bias, w3 = bytes_hi(c1) + bias;
                const h8 bw = h8{w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
                f4 t = {0.f, 0.f, 0.f, 0.f};
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bw, t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bw, t, 0, 0, 0);
                const float d = f16f(r[m].dm[bb]), mn = f16f(r[m].dm[bb] >> 16);
                malformed |= !kq_isfinite(d) || !kq_isfinite(mn);
                const float m32 = mn * 32.0f; /* the sums carry 2^-5 */
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[m][k] = fmaf(d, t[k], fmaf(m32, sx[k], acc[m][k]));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

/* ------------------------------------------------------------------ */
/* grouped expert pass */

/* Who a workgroup serves: a routed expert (its tokens at positions
 * offsets[e] .. offsets[e+1]) or a range of 16-token chunks of the shared
 * expert (every token, positions T*K + t). */
struct Work {
    uint32_t first;  /* first position (routed) or first token (shared) */
    uint32_t count;  /* tokens */
    bool shared;
};

__device__ __forceinline__ Work work_of(uint32_t y, const uint32_t *offsets, uint32_t experts,
                                        uint32_t tokens, uint32_t shared_chunks) {
    Work w;
    if (y < experts) {
        w.first = offsets[y];
        w.count = offsets[y + 1u] - w.first;
        w.shared = false;
    } else {
        const uint32_t t0 = (y - experts) * shared_chunks * kTile;
        w.first = t0;
        w.count = t0 < tokens ? min(tokens - t0, shared_chunks * kTile) : 0u;
        w.shared = true;
    }
    return w;
}

/*
 * NMAT = 2: gate and up (rows = routed/shared intermediate, KDIM = hidden),
 *   input rows are the hidden states of the tokens, output act[pos][row] =
 *   swiglu(g, u).
 * NMAT = 1: down (rows = hidden, KDIM = intermediate), input rows are
 *   act[pos], output o[pos][row].
 * grid: x = slabs of NW * TPW * 16 rows, y = routed experts then shared
 * chunks. Positions: routed pairs 0 .. T*K-1 (permuted order), shared token
 * t at T*K + t.
 *
 * Each wave walks TPW 16-row tiles, all blocks of a tile in order, with the
 * next block's weights (across tile boundaries) in flight while one block is
 * multiplied. Every prefetch and every result store is issued on every
 * path -- ones past the data use offsets outside their buffer, which the
 * hardware drops -- so the memory counters the compiler waits on are the
 * same on every path and a wait never drains the prefetch.
 */
template <uint32_t GFMT, uint32_t KDIM, int NMAT, int NW, int TPW, int PD, int KS>
__global__ __launch_bounds__(NW * 64) void grouped_pass(
    const uint8_t *__restrict__ W0, const uint8_t *__restrict__ W1,
    const uint8_t *__restrict__ SW0, const uint8_t *__restrict__ SW1,
    const float *__restrict__ X, const uint32_t *__restrict__ offsets,
    const uint32_t *__restrict__ perm_tok, uint32_t experts, uint32_t tokens, uint32_t top_k,
    uint32_t rows, uint32_t shared_chunks, uint32_t ybase, float *__restrict__ out,
    uint32_t *status) {
    /* KS slices of KSL columns: the activation image of one slice is staged
     * at a time (a 2560-column image would not fit the LDS); the
     * accumulators carry over (one tile per wave then) */
    constexpr uint32_t KSL = KDIM / (uint32_t)KS;
    static_assert(KS == 1 || TPW == 1, "sliced passes run one tile per wave");
    using F = Fmt<GFMT>;
    using S = Stage<GFMT, KSL>;
    using T = Tile<GFMT, KSL, NMAT>;
    using Raw = typename F::Raw;
    constexpr uint32_t NB = KDIM / F::kUnit;       /* units of a row */
    constexpr uint32_t NBS = NB / (uint32_t)KS;    /* units of a slice */
    static_assert(NBS * (uint32_t)KS == NB && NB * F::kUnit == KDIM, "whole units per slice");
    constexpr uint32_t RB = NB * F::kUnitBytes;
    __shared__ S st;
    __shared__ int src_row[kTile];

    const uint32_t e = blockIdx.y + ybase;
    const Work wk = work_of(e, offsets, experts, tokens, shared_chunks);
    if (wk.count == 0u) return;
    /* the wave index is uniform across the wave; saying so keeps the weight
     * buffer descriptors in scalar registers (no per-lane waterfall) */
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t tk = tokens * top_k;
    /* tile t of this wave starts at row tile_row(t); tiles past the matrix
     * load nothing and store nothing */
    auto tile_row = [&](uint32_t t) { return ((blockIdx.x * TPW + t) * NW + wave) * kTile; };

    const uint32_t wbytes = rows * RB;
    KqBuf wb[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
        const uint8_t *base = wk.shared ? (m == 0 ? SW0 : SW1)
                                        : (m == 0 ? W0 : W1) + (size_t)e * rows * RB;
        wb[m] = kq_buf(base, wbytes);
    }
    /* byte offset of unit u of tile t for this lane's row, or the buffer
     * size (every field read from there is dropped) */
    auto boff = [&](uint32_t t, uint32_t u) {
        const uint32_t r0 = tile_row(t);
        return (t < (uint32_t)TPW && r0 < rows) ? (r0 + j) * RB + u * F::kUnitBytes : wbytes;
    };
    auto load = [&](Raw (&r)[NMAT], uint32_t off) {
#pragma unroll
        for (int m = 0; m < NMAT; ++m) r[m] = F::load(wb[m], off, g);
    };
    /* results go through a buffer over this workgroup's output rows */
    const uint32_t pos0 = wk.shared ? tk + wk.first : wk.first;
    const uint32_t obytes = wk.count * rows * 4u;
    const KqBuf ob = kq_buf(out + (size_t)pos0 * rows, obytes);

    /* the wave's iterations are (slice, tile, unit of the slice) in order;
     * iteration `it` reads ring slot it % R, which iteration it - PD filled */
    constexpr uint32_t PER = (uint32_t)TPW * NBS; /* iterations per slice */
    constexpr uint32_t NIT = (uint32_t)KS * PER;
    constexpr uint32_t R = (uint32_t)PD + 1u;
    auto it_off = [&](uint32_t it) {
        if (it >= NIT) return wbytes;
        const uint32_t ks = it / PER, rem = it % PER;
        return boff(rem / NBS, ks * NBS + rem % NBS);
    };

    bool bad = false, badin = false, malformed = false;
    auto stage = [&](uint32_t ks) {
        /* a non-finite hidden state is the caller's input; a non-finite
         * intermediate activation is a numeric failure of the layer */
        const bool nf = stage_slice<GFMT, KDIM, KSL>(st, X, ks * KSL, src_row, wave, NW, lane);
        if (NMAT == 2)
            badin |= nf;
        else
            bad |= nf;
    };
    for (uint32_t c0 = 0; c0 < wk.count; c0 += kTile) {
        /* the first PD units' weights are requested before the staging */
        Raw ring[R][NMAT];
#pragma unroll
        for (uint32_t it = 0; it < (uint32_t)PD; ++it) load(ring[it], it_off(it));
        __syncthreads(); /* the previous chunk's readers are done */
        if (threadIdx.x < kTile) {
            const uint32_t i = threadIdx.x;
            int src = -1;
            if (c0 + i < wk.count) {
                const uint32_t p = wk.first + c0 + i;
                if (NMAT == 2)
                    src = (int)(wk.shared ? p : perm_tok[p]);
                else
                    src = (int)(wk.shared ? tk + p : p);
            }
            src_row[i] = src;
        }
        __syncthreads();
        stage(0u);
        __syncthreads();

        f4 acc[NMAT];
        static_assert(NIT % R == 0u, "the ring must divide the iterations");
#pragma unroll 1
        for (uint32_t it0 = 0; it0 < NIT; it0 += R) {
#pragma unroll
            for (uint32_t r = 0; r < R; ++r) {
                const uint32_t it = it0 + r;
                const uint32_t ks = it / PER, rem = it % PER;
                const uint32_t t = rem / NBS, b = rem % NBS;
                if (KS > 1 && ks > 0u && rem == 0u) {
                    /* the next slice of the activations */
                    __syncthreads();
                    stage(ks);
                    __syncthreads();
                }
                if (b == 0u && ks == 0u) {
#pragma unroll
                    for (int m = 0; m < NMAT; ++m) acc[m] = f4{0.f, 0.f, 0.f, 0.f};
                }
                load(ring[(r + PD) % R], it_off(it + PD));
                T::block(ring[r], st, b, j, g, acc, malformed);
                __builtin_amdgcn_sched_barrier(0);
                if (b + 1u < NBS || ks + 1u < (uint32_t)KS) continue;
                /* D[token][row]: this lane holds row `row` of tokens 4g .. 4g+3 */
                const uint32_t row = tile_row(t) + j;
#pragma unroll
                for (uint32_t q = 0; q < 4u; ++q) {
                    const uint32_t i = 4u * g + q;
                    const bool valid = c0 + i < wk.count && row < rows;
                    const int sg = st.sig[i];
                    float v;
                    if constexpr (NMAT == 2) {
                        const float gv = ldexpf(acc[0][q], -sg), uv = ldexpf(acc[1][q], -sg);
                        v = kq_swiglu(gv, uv);
                        bad |= valid && (!kq_isfinite(gv) || !kq_isfinite(uv));
                    } else {
                        v = ldexpf(acc[0][q], -sg);
                    }
                    bad |= valid && !kq_isfinite(v);
                    const uint32_t off = valid ? ((c0 + i) * rows + row) * 4u : obytes;
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ob.r, (int)off, 0,
                                                          0);
                }
            }
        }
    }
    if (badin) kq_flag(status, KQ_DEV_INPUT);
    if (malformed) kq_flag(status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
}

/* ------------------------------------------------------------------ */
/* permutation: stable counting sort of (token, slot) pairs by expert id */

constexpr uint32_t kPermChunk = 256; /* tokens per rank pass */

/* The Q4_K gate/up pass's work list (kq_grouped_gu.hip, gu_items): one
 * item per kItemRows-token chunk of an expert, routed experts in id order,
 * then the shared expert's chunks; [0] the count, items from [4] on as
 * (expert | kItemShared, first | count << 24). */
constexpr uint32_t kItemRows = 16;
constexpr uint32_t kItemShared = 0x80000000u;

__global__ __launch_bounds__(1024) void moe_permute(const uint32_t *__restrict__ ids,
                                                    uint32_t tokens, uint32_t top_k,
                                                    uint32_t experts, uint32_t *__restrict__ offsets,
                                                    uint32_t *__restrict__ perm_tok,
                                                    uint32_t *__restrict__ pos,
                                                    uint32_t *__restrict__ pair_slot,
                                                    uint32_t *status, uint32_t *items,
                                                    uint32_t with_shared, uint32_t *zero,
                                                    uint32_t nzero) {
    __shared__ uint32_t cnt[1024];
    __shared__ uint32_t base[1024];
    __shared__ uint32_t bits[1024][kPermChunk / 32u];
    __shared__ uint32_t wsum[16];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t pairs = tokens * top_k;
    cnt[tid] = 0u;
    /* words a later pass accumulates into (atomic maxima) start at zero */
    for (uint32_t i = tid; i < nzero; i += 1024u) zero[i] = 0u;
    __syncthreads();
    bool bad = false;
    for (uint32_t p = tid; p < pairs; p += 1024u) {
        uint32_t e = ids[p];
        if (e >= experts) {
            bad = true;
            e = 0u;
        }
        atomicAdd(&cnt[e], 1u);
    }
    __syncthreads();
    /* exclusive scan of cnt[0 .. 1023] (entries past the experts are 0) */
    {
        const uint32_t v = cnt[tid];
        uint32_t incl = v;
#pragma unroll
        for (uint32_t o = 1; o < 64u; o <<= 1) {
            const uint32_t n = __shfl_up(incl, o, KQ_WAVE);
            if (lane >= o) incl += n;
        }
        if (lane == 63u) wsum[wave] = incl;
        __syncthreads();
        uint32_t before = 0u;
        for (uint32_t w = 0; w < wave; ++w) before += wsum[w];
        const uint32_t ex = before + incl - v;
        base[tid] = ex;
        if (tid < experts) offsets[tid] = ex;
        if (tid == experts) offsets[tid] = ex; /* = pairs */
    }
    __syncthreads();
    if (items != nullptr) {
        /* the gate/up work list from the same counts: exclusive scan of
         * the chunks per expert */
        __shared__ uint32_t csum[16];
        const uint32_t c = tid < experts ? cnt[tid] : 0u;
        const uint32_t nc = (c + kItemRows - 1u) / kItemRows;
        uint32_t incl = nc;
#pragma unroll
        for (uint32_t o = 1; o < 64u; o <<= 1) {
            const uint32_t n = __shfl_up(incl, o, KQ_WAVE);
            if (lane >= o) incl += n;
        }
        if (lane == 63u) csum[wave] = incl;
        __syncthreads();
        uint32_t ib = incl - nc, total = 0u;
        for (uint32_t w = 0; w < 16u; ++w) {
            ib += w < wave ? csum[w] : 0u;
            total += csum[w];
        }
        uint32_t *list = items + 4;
        const uint32_t o0 = base[tid];
        for (uint32_t k = 0; k < nc; ++k) {
            list[2u * (ib + k)] = tid;
            list[2u * (ib + k) + 1u] = (o0 + kItemRows * k) | (min(c - kItemRows * k, kItemRows) << 24);
        }
        const uint32_t nsh = with_shared ? (tokens + kItemRows - 1u) / kItemRows : 0u;
        for (uint32_t k = tid; k < nsh; k += 1024u) {
            list[2u * (total + k)] = kItemShared | k;
            list[2u * (total + k) + 1u] = (kItemRows * k) | (min(tokens - kItemRows * k, kItemRows) << 24);
        }
        if (tid == 0u) items[0] = total + nsh;
    }
    for (uint32_t t0 = 0; t0 < tokens; t0 += kPermChunk) {
        const uint32_t nt = min(kPermChunk, tokens - t0);
        for (uint32_t w = tid; w < 1024u * (kPermChunk / 32u); w += 1024u)
            (&bits[0][0])[w] = 0u;
        __syncthreads();
        const uint32_t np = nt * top_k;
        for (uint32_t p = tid; p < np; p += 1024u) {
            const uint32_t lt = p / top_k;
            uint32_t e = ids[(size_t)t0 * top_k + p];
            e = e < experts ? e : 0u;
            atomicOr(&bits[e][lt >> 5], 1u << (lt & 31u));
        }
        __syncthreads();
        for (uint32_t p = tid; p < np; p += 1024u) {
            const uint32_t lt = p / top_k;
            uint32_t e = ids[(size_t)t0 * top_k + p];
            e = e < experts ? e : 0u;
            uint32_t r = __popc(bits[e][lt >> 5] & ((1u << (lt & 31u)) - 1u));
            for (uint32_t w = 0; w < (lt >> 5); ++w) r += __popc(bits[e][w]);
            const uint32_t q = base[e] + r;
            pos[(size_t)t0 * top_k + p] = q;
            perm_tok[q] = t0 + lt;
            if (pair_slot != nullptr) pair_slot[q] = p - lt * top_k;
        }
        __syncthreads();
        {
            uint32_t c = 0u;
#pragma unroll
            for (uint32_t w = 0; w < kPermChunk / 32u; ++w) c += __popc(bits[tid][w]);
            base[tid] += c;
        }
        __syncthreads();
    }
    if (bad) kq_flag(status, KQ_DEV_RANGE);
}

/* ------------------------------------------------------------------ */
/* combine, in the reference's order (src/kq_moe_qwen38.c:722-765, :826) */

/* One thread per four consecutive outputs of a token: the slots' rows are
 * requested together (up to kCombineRun of them before the first add),
 * then summed in the reference's order with separately rounded products. */
constexpr uint32_t kCombineRun = 16;

__global__ __launch_bounds__(256) void moe_combine(
    const float *__restrict__ o, const uint32_t *__restrict__ pos,
    const uint32_t *__restrict__ order, const float *__restrict__ weights,
    const float *__restrict__ shared_scale, uint32_t tokens, uint32_t top_k, uint32_t hidden,
    float *__restrict__ out, uint32_t *status) {
    const uint32_t t = blockIdx.y;
    const uint32_t q = blockIdx.x * 256u + threadIdx.x; /* float4 of the row */
    const uint32_t hq = hidden / 4u;
    if (q >= hq) return;
    const uint32_t tk = tokens * top_k;
    const float4 *o4 = (const float4 *)o;
    bool bad = false;
    float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
    auto add = [&](const float4 v, const float w) {
        bad |= !kq_isfinite(v.x) || !kq_isfinite(v.y) || !kq_isfinite(v.z) || !kq_isfinite(v.w);
        float p;
        p = v.x * w; sum.x = sum.x + p;
        p = v.y * w; sum.y = sum.y + p;
        p = v.z * w; sum.z = sum.z + p;
        p = v.w * w; sum.w = sum.w + p;
    };
    for (uint32_t j0 = 0; j0 < top_k; j0 += kCombineRun) {
        float4 v[kCombineRun];
        float wv[kCombineRun];
#pragma unroll
        for (uint32_t i = 0; i < kCombineRun; ++i) {
            if (j0 + i < top_k) {
                const uint32_t sl = order[(size_t)t * top_k + j0 + i];
                const uint32_t p = pos[(size_t)t * top_k + sl];
                wv[i] = weights[(size_t)t * top_k + sl];
                v[i] = o4[(size_t)p * hq + q];
            }
        }
#pragma unroll
        for (uint32_t i = 0; i < kCombineRun; ++i)
            if (j0 + i < top_k) add(v[i], wv[i]);
    }
    const float4 so = o4[(size_t)(tk + t) * hq + q];
    const float sc = shared_scale[t];
    float4 r;
    auto fin = [&](float sv, float sm, float &dst) {
        const float gated = sv * sc;
        const float val = sm + gated;
        bad |= !kq_isfinite(sv) || !kq_isfinite(sm) || !kq_isfinite(gated) || !kq_isfinite(val);
        dst = val;
    };
    fin(so.x, sum.x, r.x);
    fin(so.y, sum.y, r.y);
    fin(so.z, sum.z, r.z);
    fin(so.w, sum.w, r.w);
    ((float4 *)out)[(size_t)t * hq + q] = r;
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
}

/* ------------------------------------------------------------------ */
/* launchers */

constexpr uint32_t kSharedChunks = 2; /* 16-token chunks per shared-expert workgroup */

/* Launch shape per pass: NW waves per workgroup, TPW 16-row tiles per
 * wave, PD blocks of weights in flight ahead of the one being multiplied.
 * The registers of a SIMD bound waves x (PD + 1) x block registers; the
 * gate/up image (136 KiB at 2048 columns) allows one workgroup per CU. */
#ifndef KQ_GU_NW
#define KQ_GU_NW 16
#define KQ_GU_TPW 1
#define KQ_GU_PD 1
#endif
#ifndef KQ_DN_NW
#define KQ_DN_NW 8
#define KQ_DN_TPW 4
#define KQ_DN_PD 1
#endif
#ifndef KQ_GU_KSL
#define KQ_GU_KSL 2048 /* widest activation slice staged at once */
#endif

/* slices of a row: the fewest whole-unit slices of at most KQ_GU_KSL
 * columns */
template <uint32_t GFMT, uint32_t KDIM>
constexpr int gu_slices() {
    for (int ks = 1; ks <= 16; ++ks) {
        const uint32_t w = KDIM / (uint32_t)ks;
        if (w * (uint32_t)ks == KDIM && w % Fmt<GFMT>::kUnit == 0u && w <= (uint32_t)KQ_GU_KSL)
            return ks;
    }
    return 0;
}
template <uint32_t GFMT, uint32_t KDIM, int NMAT>
struct Shape {
    /* rows longer than KQ_GU_KSL columns are staged in slices, one tile
     * per wave */
    static constexpr bool kSliced = KDIM > (uint32_t)KQ_GU_KSL;
    static constexpr int NW = NMAT == 2 ? (KDIM >= 1024u ? KQ_GU_NW : 8)
                                        : (kSliced ? KQ_GU_NW : KQ_DN_NW);
    static constexpr int TPW = NMAT == 2 ? (KDIM >= 1024u ? KQ_GU_TPW : 2)
                                         : (kSliced ? 1 : KQ_DN_TPW);
    static constexpr int KS = gu_slices<GFMT, KDIM>();
    static_assert(KS >= 1, "no slicing of this row length");
    static_assert(KS == 1 || TPW == 1, "sliced passes run one tile per wave");
    /* the ring (PD + 1 slots) is a power of two that divides the wave's
     * KS * TPW * KDIM / unit iterations */
    static constexpr int NIT = TPW * (int)(KDIM / Fmt<GFMT>::kUnit);
    static constexpr int WANT = (NMAT == 2 ? KQ_GU_PD : KQ_DN_PD) + 1;
    static constexpr int RING = WANT >= 8 && NIT % 8 == 0 ? 8
                                : WANT >= 4 && NIT % 4 == 0 ? 4
                                : WANT >= 2 && NIT % 2 == 0 ? 2 : 1;
    static constexpr int PD = RING > 1 ? RING - 1 : 0;
};

/* the Q6_K down pass with its weights streamed through LDS (below) */
template <uint32_t KDIM>
hipError_t launch_down_q6k(const uint8_t *W0, const uint8_t *SW0, const float *X,
                           const uint32_t *offsets, uint32_t experts, uint32_t tokens,
                           uint32_t top_k, uint32_t rows, uint32_t y0, uint32_t ny,
                           uint32_t chunks, float *out, uint32_t *status, hipStream_t s);

/* Workgroup rows y0 .. y0 + ny - 1 of the pass: experts 0 .. E-1, then the
 * shared expert's chunk groups. */
template <uint32_t GFMT, uint32_t KDIM, int NMAT>
hipError_t launch_pass(const uint8_t *W0, const uint8_t *W1, const uint8_t *SW0,
                       const uint8_t *SW1, const float *X, const uint32_t *offsets,
                       const uint32_t *perm_tok, uint32_t experts, uint32_t tokens,
                       uint32_t top_k, uint32_t rows, uint32_t y0, uint32_t ny, uint32_t chunks,
                       float *out, uint32_t *status, hipStream_t s) {
    if (ny == 0u) return hipSuccess;
    /* (an intermediate of 2048 leaves no LDS beside its activation image
     * for the weight slots) */
    if constexpr (GFMT == KQ_LAUNCH_Q6_K && NMAT == 1 && KDIM <= 1024u)
        return launch_down_q6k<KDIM>(W0, SW0, X, offsets, experts, tokens, top_k, rows, y0, ny,
                                     chunks, out, status, s);
    constexpr int NW = Shape<GFMT, KDIM, NMAT>::NW;
    constexpr int TPW = Shape<GFMT, KDIM, NMAT>::TPW;
    constexpr int PD = Shape<GFMT, KDIM, NMAT>::PD;
    constexpr int KS = Shape<GFMT, KDIM, NMAT>::KS;
    if (y0 >= experts && ny > 0u) {
        /* the shared expert alone (its format differs from the routed
         * one): a few rows for every token, so 64-row slabs and one
         * 16-token chunk per workgroup, which spreads it over the device */
        constexpr int NWS = 4;
        /* the ring (a power of two) must divide the TPW = 1 iterations */
        constexpr int NIT1 = (int)(KDIM / Fmt<GFMT>::kUnit);
        constexpr int R1 = (PD + 1) >= 8 && NIT1 % 8 == 0   ? 8
                           : (PD + 1) >= 4 && NIT1 % 4 == 0 ? 4
                           : (PD + 1) >= 2 && NIT1 % 2 == 0 ? 2
                                                            : 1;
        constexpr int PD1 = R1 - 1;
        const uint32_t nys = (tokens + kTile - 1u) / kTile;
        const dim3 grid((rows + NWS * kTile - 1u) / (NWS * kTile), nys);
        hipLaunchKernelGGL((grouped_pass<GFMT, KDIM, NMAT, NWS, 1, PD1, KS>), grid,
                           dim3(NWS * 64), 0, s, W0, W1, SW0, SW1, X, offsets, perm_tok, experts,
                           tokens, top_k, rows, 1u, y0, out, status);
        return hipGetLastError();
    }
    const uint32_t slab = (uint32_t)(NW * TPW) * kTile;
    const dim3 grid((rows + slab - 1u) / slab, ny);
    hipLaunchKernelGGL((grouped_pass<GFMT, KDIM, NMAT, NW, TPW, PD, KS>), grid, dim3(NW * 64), 0,
                       s, W0, W1, SW0, SW1, X, offsets, perm_tok, experts, tokens, top_k, rows,
                       chunks, y0, out, status);
    return hipGetLastError();
}

/* the row lengths each format's pass is built for: whole units, and the
 * activation image of a slice within the LDS */
template <uint32_t GFMT, int NMAT>
constexpr bool pass_dim(uint32_t k) {
    if (k % Fmt<GFMT>::kUnit != 0u) return false;
    if (NMAT == 2) return k == 256u || k == 512u || k == 1024u || k == 2048u || k == 2560u;
    return k == 256u || k == 320u || k == 512u || k == 640u || k == 1024u || k == 2048u ||
           k == 10240u;
}

template <uint32_t GFMT, int NMAT>
hipError_t pass_cols(uint32_t kdim, const uint8_t *W0, const uint8_t *W1, const uint8_t *SW0,
                     const uint8_t *SW1, const float *X, const uint32_t *offsets,
                     const uint32_t *perm_tok, uint32_t experts, uint32_t tokens, uint32_t top_k,
                     uint32_t rows, uint32_t y0, uint32_t ny, uint32_t chunks, float *out,
                     uint32_t *status, hipStream_t s) {
#define KQ_PASS(K)                                                                               \
    if constexpr (pass_dim<GFMT, NMAT>(K))                                                       \
        return launch_pass<GFMT, K, NMAT>(W0, W1, SW0, SW1, X, offsets, perm_tok, experts,       \
                                          tokens, top_k, rows, y0, ny, chunks, out, status, s);  \
    return hipErrorInvalidValue
    switch (kdim) {
    case 256: { KQ_PASS(256u); }
    case 320: { KQ_PASS(320u); }
    case 512: { KQ_PASS(512u); }
    case 640: { KQ_PASS(640u); }
    case 1024: { KQ_PASS(1024u); }
    case 2048: { KQ_PASS(2048u); }
    case 2560: { KQ_PASS(2560u); }
    case 10240: { KQ_PASS(10240u); }
    default: return hipErrorInvalidValue;
    }
#undef KQ_PASS
}

/* pass_dim for a run-time format */
bool pass_dim_rt(uint32_t type, int nmat, uint32_t k) {
    switch (type) {
    case KQ_LAUNCH_Q4_K: return nmat == 2 ? pass_dim<KQ_LAUNCH_Q4_K, 2>(k) : pass_dim<KQ_LAUNCH_Q4_K, 1>(k);
    case KQ_LAUNCH_Q6_K: return nmat == 1 && pass_dim<KQ_LAUNCH_Q6_K, 1>(k);
    case KQ_LAUNCH_Q8_0: return nmat == 2 ? pass_dim<KQ_LAUNCH_Q8_0, 2>(k) : pass_dim<KQ_LAUNCH_Q8_0, 1>(k);
    case KQ_LAUNCH_Q5_1: return nmat == 1 && pass_dim<KQ_LAUNCH_Q5_1, 1>(k);
    default: return false;
    }
}

/* one pass of a role whose routed and shared matrices may differ in
 * format: one launch when they agree, else the routed workgroups and the
 * shared ones as two launches */
template <int NMAT>
hipError_t pass_any(uint32_t type, uint32_t kdim, const uint8_t *W0, const uint8_t *W1,
                    const uint8_t *SW0, const uint8_t *SW1, const float *X,
                    const uint32_t *offsets, const uint32_t *perm_tok, uint32_t experts,
                    uint32_t tokens, uint32_t top_k, uint32_t rows, uint32_t y0, uint32_t ny,
                    float *out, uint32_t *status, hipStream_t s) {
#define KQ_ANY(F)                                                                              \
    pass_cols<F, NMAT>(kdim, W0, W1, SW0, SW1, X, offsets, perm_tok, experts, tokens, top_k, \
                       rows, y0, ny, kSharedChunks, out, status, s)
    switch (type) {
    case KQ_LAUNCH_Q4_K: return KQ_ANY(KQ_LAUNCH_Q4_K);
    case KQ_LAUNCH_Q8_0: return KQ_ANY(KQ_LAUNCH_Q8_0);
    case KQ_LAUNCH_Q6_K:
        if constexpr (NMAT == 1) return KQ_ANY(KQ_LAUNCH_Q6_K);
        return hipErrorInvalidValue;
    case KQ_LAUNCH_Q5_1:
        if constexpr (NMAT == 1) return KQ_ANY(KQ_LAUNCH_Q5_1);
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
#undef KQ_ANY
}

/* ------------------------------------------------------------------ */
/* Batched Q6_K matvec on MFMA: y[b] = W x[b] for 2 .. 4 activation columns
 *
 * The row engine keeps every lane's activations in registers, 32 per batch
 * column; at 4 columns that leaves no room for the weights in flight. Here
 * the columns ride on the token dimension of 16x16x32 matrix steps: they are
 * staged once per workgroup as fp16 hi + lo after an exact power-of-two
 * scaling (an LDS image of kMvCols rows). The four columns' hi and lo parts
 * fill 8 token rows, so one step carries two 16-column sub-blocks of the
 * block: token rows 0..7 hold the first sub-block's activations on k 0..15
 * (zeros on k 16..31) and rows 8..15 the second's on k 16..31. Each product
 * row then belongs to one sub-block, and lane l keeps row l % 16 of a
 * 16-row tile for the four token rows 4 (l / 16) .. + 3: its sub-block's
 * scale applies to all four.
 *
 * Weights: the MFMA operand wants scattered 4-byte pieces of a block per
 * lane, which as global loads would touch 16 rows per instruction. So each
 * wave streams one block of its tile's 16 rows at a time (16 windows of 224
 * bytes from the block's aligned start) with four LDS-DMA loads straight
 * into a ring of NS private LDS slots, NS - 1 blocks ahead of the one it
 * multiplies, and reads the operand pieces from there. Eight waves with a
 * four-slot ring fill the LDS beside the activation image at 2,048 columns;
 * on the 151936 x 2048 LM head at 4 columns this was faster than 4, 6, 10,
 * 12 or 16 waves with the rings that fit them (92.7, 84.2, 77.6, 81.3 and
 * 82.1 us against 70.9-75.6 us). The per-row fp32 sums are compared with
 * the CPU by tolerance; the argmax partials (largest value, lowest row on
 * ties) are exact over them. */

constexpr uint32_t kMvCols = 4;      /* staged activation columns */
constexpr int kMvWaves = 8;          /* waves per workgroup */
constexpr uint32_t kMvMaxK = 4096u;
constexpr uint32_t kMvWin = 224u;    /* bytes of a row's block window (>= 210 + 2) */
constexpr uint32_t kMvPitch = 240u;  /* slot row pitch: lanes (j, g) hit distinct banks */
constexpr uint32_t kMvSlot = kTile * kMvPitch;
constexpr uint32_t kMvUnits = kTile * (kMvWin / 16u); /* 16-byte loads per block: 224 */
constexpr int kMvLoads = (int)((kMvUnits + 63u) / 64u); /* per lane: 4 */
constexpr uint32_t kMvUnitsPerRow = kMvPitch / 16u; /* 15: 14 window units + 1 gap */
constexpr int kMvDma = (int)((kMvSlot / 16u + 63u) / 64u); /* DMA loads per block: 4 */
constexpr uint32_t kMvZero = 256u; /* fp16 zeros: k 8 g + 128 n + 32 q .. + 7 < 256 */
constexpr uint32_t kMvLdsMax = 160u * 1024u;
constexpr uint32_t kMvMaxSlots = 4u; /* block slots per wave, at most */

__device__ __forceinline__ void mv_argmax_merge(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

/* x image pitch in fp16 (a 32-byte skew per column keeps the 16 operand
 * reads of a step on distinct banks) */
__host__ __device__ __forceinline__ uint32_t mv_xpitch(uint32_t nb) { return nb * 256u + 16u; }

__host__ __device__ __forceinline__ uint32_t mv_lds_bytes(uint32_t nb, uint32_t ns) {
    return 2u * kMvCols * mv_xpitch(nb) * 2u + kMvCols * 4u + kMvZero * 2u +
           (uint32_t)kMvWaves * ns * kMvSlot;
}

/* NS block slots per wave: block it is multiplied from slot it % NS while
 * blocks it + 1 .. it + NS - 1 are in flight */
template <uint32_t NS>
__global__ __launch_bounds__(kMvWaves * 64) void matvec_mfma_q6k(
    const uint8_t *__restrict__ W, uint32_t rows, uint32_t nb, const float *__restrict__ x,
    uint32_t batch, float *__restrict__ y, uint32_t *status, float *part_v, uint32_t *part_i,
    uint32_t part_stride) {
    using F = Fmt<KQ_LAUNCH_Q6_K>;
    extern __shared__ __align__(16) _Float16 mv_lds[];
    const uint32_t K = nb * 256u, pitch = mv_xpitch(nb);
    _Float16 *xh = mv_lds, *xl = mv_lds + kMvCols * pitch;
    int *sig = (int *)(xl + kMvCols * pitch);
    /* the zero operand of the token rows off their sub-block (16 bytes past
     * a 32-byte boundary of the x image, so its broadcast reads sit on the
     * banks the live rows leave free) */
    _Float16 *xz = (_Float16 *)(sig + kMvCols);
    uint8_t *slots = (uint8_t *)(xz + kMvZero);

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t gw = blockIdx.x * (uint32_t)kMvWaves + wave;
    const uint32_t nwaves = gridDim.x * (uint32_t)kMvWaves;
    const uint32_t rb = nb * F::kBytes;
    const uint32_t wbytes = rows * rb;
    const kq_i4v wr = dma_rsrc(W, wbytes);
    const uint32_t ntiles = (rows + kTile - 1u) / kTile;
    uint8_t *myslot = slots + wave * NS * kMvSlot;
    const uint32_t myslot_lds = lds_addr(myslot);

    /* Work item it = block it % nb of tile gw + nwaves * (it / nb), walked
     * with counters (t, b) and the tile's byte offset tb = 16 t rb (no
     * division or 32-bit multiply per item; tb is used only while
     * t < ntiles, where it stays below wbytes). */
    struct Pos {
        uint32_t t, b, tb;
    };
    const uint32_t tstep = nwaves * kTile * rb;
    auto advance = [&](Pos &q) {
        if (++q.b == nb) {
            q.b = 0u;
            q.t += nwaves;
            q.tb += tstep;
        }
    };
    /* A block's DMA: load i, lane l writes slot bytes [16 p, 16 p + 16) with
     * p = 64 i + l, which is unit p % 15 of row p / 15 (row pitch 240: 14
     * units of the row's window -- the block's start rounded down to 4
     * bytes -- and a gap). Gap units and rows past the matrix read the
     * matrix's first bytes instead (whatever lands there is never a result:
     * gap bytes are not read, and rows past the matrix are not stored); the
     * last load runs on the 48 lanes that reach the slot's 3,840 bytes. */
    uint32_t ld_r[kMvDma], ld_rb[kMvDma], ld_u[kMvDma];
#pragma unroll
    for (int i = 0; i < kMvDma; ++i) {
        const uint32_t p = (uint32_t)i * 64u + lane;
        const uint32_t r = p / kMvUnitsPerRow, u = p - kMvUnitsPerRow * r;
        ld_r[i] = (r < kTile && u * 16u < kMvWin) ? r : 0xffffu;
        ld_u[i] = 16u * u;
        ld_rb[i] = r * rb;
    }
    auto dma_item = [&](const Pos &q, uint32_t slot) {
        const uint32_t dst = myslot_lds + slot * kMvSlot;
#pragma unroll
        for (int i = 0; i < kMvDma; ++i) {
            const uint32_t row = q.t * kTile + ld_r[i];
            const uint32_t o = q.tb + ld_rb[i] + q.b * F::kBytes;
            const uint32_t off =
                (ld_r[i] < kTile && q.t < ntiles && row < rows) ? (o & ~3u) + ld_u[i] : ld_u[i];
            if ((uint32_t)i * 64u + 64u <= kMvSlot / 16u) {
                dma16(wr, off, dst + 1024u * (uint32_t)i);
            } else if ((uint32_t)i * 64u + lane < kMvSlot / 16u) {
                dma16(wr, off, dst + 1024u * (uint32_t)i);
            }
        }
    };

    /* the first block is requested before the staging, the next NS - 1
     * after it (the staging's own loads wait for every load issued before
     * theirs) */
    const uint32_t nitems = ntiles > gw ? ((ntiles - gw + nwaves - 1u) / nwaves) * nb : 0u;
    Pos ld = {gw, 0u, gw * kTile * rb}, pr = ld;
    if (nitems > 0u) {
        dma_item(ld, 0u);
        advance(ld);
    }

    /* stage column i (one wave each): scale by 2^sig[i], split into hi + lo */
    bool bad = false;
    for (uint32_t i = wave; i < kMvCols; i += (uint32_t)kMvWaves) {
        const bool real = i < batch;
        float m = 0.0f;
        bool nf = false;
        for (uint32_t c = 4u * lane; c < K; c += 256u) {
            const float4 v = real ? *(const float4 *)(x + (size_t)i * K + c)
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
            nf |= !kq_isfinite(v.x) || !kq_isfinite(v.y) || !kq_isfinite(v.z) || !kq_isfinite(v.w);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        bad |= nf;
        m = wave_max_abs(m);
        const bool any_nf = __ballot(nf) != 0ull;
        int e = 0;
        if (!any_nf && m > 0.0f) e = 15 - __builtin_amdgcn_frexp_expf(m);
        for (uint32_t c = 4u * lane; c < K; c += 256u) {
            const float4 v = real ? *(const float4 *)(x + (size_t)i * K + c)
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
            const float a[4] = {v.x, v.y, v.z, v.w};
            _Float16 hi[4], lo[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float xs = any_nf ? 0.0f : ldexpf(a[q], e);
                hi[q] = (_Float16)xs;
                lo[q] = (_Float16)(xs - (float)hi[q]);
            }
            *(h4 *)(xh + i * pitch + c) = h4{hi[0], hi[1], hi[2], hi[3]};
            *(h4 *)(xl + i * pitch + c) = h4{lo[0], lo[1], lo[2], lo[3]};
        }
        if (lane == 0u) sig[i] = e;
    }
    if (threadIdx.x < kMvZero / 8u) *(h8 *)(xz + 8u * threadIdx.x) = h8{};
#pragma unroll
    for (uint32_t sl = 1u; sl < NS; ++sl) {
        if (sl < nitems) {
            dma_item(ld, sl);
            advance(ld);
        }
    }
    kq_lds_barrier();
    int unscale[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) unscale[k] = -sig[k];

    bool malformed = false, nonfinite = false;
    float best_v[4];
    uint32_t best_i[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        best_v[k] = -__builtin_inff();
        best_i[k] = 0xffffffffu;
    }
    /* Lane l supplies token row j = l % 16 of the A operand on k 8 (l / 16)
     * .. + 7: rows 0..3 are the hi parts of columns 0..3, rows 4..7 their lo
     * parts, rows 8..15 repeat them for the step's second sub-block. Lanes
     * whose k range belongs to the other sub-block read zeros. Product rows
     * 4 (l / 16) .. + 3 in lane l are then: l / 16 = 0 hi and 1 lo of the
     * first sub-block, 2 hi and 3 lo of the second. */
    const bool live = (j >> 3) == (g >> 1);
    const _Float16 *xa = live ? ((j & 4u) ? xl : xh) + (j & 3u) * pitch + 8u * g : xz + 8u * g;
    const uint32_t xstep = live ? 256u : 0u;
    const uint32_t hsh = 8u * (g >> 1); /* this lane's scale byte within a pair */
    const h2 bias = h2{(_Float16)-1056.0f, (_Float16)-1056.0f}; /* 1024 + 32 */
    f4 acc = {0.f, 0.f, 0.f, 0.f};

    /* item from its slot: 8 two-sub-block steps into acc; at the tile's last
     * block lanes 0..15 write row t*16 + j of columns 0 .. batch-1. Every LDS
     * read of the item is issued before its first product. */
    const uint32_t jrb = j * rb;
    auto process = [&](const Pos &q, const uint8_t *sp, auto &&refill) {
        const uint32_t bb = q.b;
        const uint32_t row = q.t * kTile + j;
        const uint32_t sh = (q.tb + jrb + bb * F::kBytes) & 3u;
        const uint8_t *p = sp + j * kMvPitch;
        auto w32 = [&](uint32_t o) { return *(const uint32_t *)(p + o); };
        /* columns 128 n + 32 q + 8 g .. + 7 of step (n, q): ql bytes 64 n +
         * 8 g (q = 0, 2) and + 32 (q = 1, 3), qh bytes 128 + 32 n + 8 g; the
         * scales at 192 and d at 208 (the window starts up to 3 bytes early) */
        uint32_t wa[2][3], wbv[2][3], wq[2][3], ws[6];
#pragma unroll
        for (uint32_t n = 0; n < 2u; ++n) {
            const uint32_t oa = 64u * n + 8u * g, oq = 128u + 32u * n + 8u * g;
#pragma unroll
            for (uint32_t e = 0; e < 3u; ++e) {
                wa[n][e] = w32(oa + 4u * e);
                wbv[n][e] = w32(oa + 32u + 4u * e);
                wq[n][e] = w32(oq + 4u * e);
            }
        }
#pragma unroll
        for (uint32_t e = 0; e < 6u; ++e) ws[e] = w32(192u + 4u * e);
        const _Float16 *pa = xa + xstep * bb;
        h8 av[2][4];
#pragma unroll
        for (uint32_t n = 0; n < 2u; ++n)
#pragma unroll
            for (uint32_t qq = 0; qq < 4u; ++qq) av[n][qq] = *(const h8 *)(pa + 128u * n + 32u * qq);
        /* every read of the slot has landed: its next block can be requested
         * before the products */
        wait_lgkm0();
        refill();
        __builtin_amdgcn_sched_barrier(0);

        const float d = f16f(kq_align2(ws[5], ws[4], sh)); /* block bytes 208, 209 */
        malformed |= row < rows && !kq_isfinite(d);
        uint32_t sc[4];
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) sc[e] = kq_align2(ws[e + 1u], ws[e], sh) >> hsh;
#pragma unroll
        for (uint32_t n = 0; n < 2u; ++n) {
            const uint32_t A[2] = {kq_align2(wa[n][1], wa[n][0], sh),
                                   kq_align2(wa[n][2], wa[n][1], sh)};
            const uint32_t B[2] = {kq_align2(wbv[n][1], wbv[n][0], sh),
                                   kq_align2(wbv[n][2], wbv[n][1], sh)};
            const uint32_t H[2] = {kq_align2(wq[n][1], wq[n][0], sh),
                                   kq_align2(wq[n][2], wq[n][1], sh)};
            uint32_t c[4][2];
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                c[0][w] = (A[w] & 0x0f0f0f0fu) | ((H[w] << 4) & 0x30303030u);
                c[1][w] = (B[w] & 0x0f0f0f0fu) | ((H[w] << 2) & 0x30303030u);
                c[2][w] = ((A[w] >> 4) & 0x0f0f0f0fu) | (H[w] & 0x30303030u);
                c[3][w] = ((B[w] >> 4) & 0x0f0f0f0fu) | ((H[w] >> 2) & 0x30303030u);
            }
            /* the four steps are independent products: all are issued
             * before any result is scaled, so the matrix core's latency
             * overlaps the next products and the scaling */
            f4 tm[4];
#pragma unroll
            for (uint32_t qq = 0; qq < 4u; ++qq) {
                const h2 w0 = bytes_lo(c[qq][0]) + bias, w1 = bytes_hi(c[qq][0]) + bias;
                const h2 w2 = bytes_lo(c[qq][1]) + bias, w3 = bytes_hi(c[qq][1]) + bias;
                const h8 bw = h8{w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
                tm[qq] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[n][qq], bw,
                                                                f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            }
#pragma unroll
            for (uint32_t qq = 0; qq < 4u; ++qq) {
                /* sub-block 8 n + 2 qq + (g >> 1): byte (2 qq) & 3 of word
                 * 2 n + qq / 2, pre-shifted by this lane's half */
                const int8_t scv = (int8_t)((sc[2u * n + (qq >> 1)] >> (16u * (qq & 1u))) & 0xffu);
                const float ds = d * (float)scv;
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[k] = fmaf(ds, tm[qq][k], acc[k]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (bb + 1u == nb) {
            /* column k of row j = the four lanes j + 16 G: hi and lo of both
             * sub-block halves */
            f4 o;
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = acc[k] + __shfl_down(acc[k], 32, KQ_WAVE);
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] += __shfl_down(o[k], 16, KQ_WAVE);
            if (g == 0u && row < rows) {
#pragma unroll
                for (uint32_t k = 0; k < 4u; ++k) {
                    if (k < batch) {
                        const float v = ldexpf(o[k], unscale[k]);
                        nonfinite |= !kq_isfinite(v);
                        y[(size_t)k * rows + row] = v;
                        mv_argmax_merge(best_v[k], best_i[k], v, row);
                    }
                }
            }
            acc = f4{0.f, 0.f, 0.f, 0.f};
        }
    };
    /* Before block it: every DMA issued after its own has not necessarily
     * landed, and there are min(NS - 1, nitems - 1 - it) of them (kMvDma
     * loads each; the y stores between are not loads). Once its reads are
     * in registers, its slot takes block it + NS. */
    uint32_t slot = 0u;
    for (uint32_t it = 0u; it < nitems; ++it) {
        const uint32_t after = nitems - 1u - it;
        wait_after<(uint32_t)kMvDma, NS - 1u>(after);
        process(pr, myslot + slot * kMvSlot, [&]() {
            if (it + NS < nitems) {
                dma_item(ld, slot);
                advance(ld);
            }
        });
        advance(pr);
        slot = slot + 1u == NS ? 0u : slot + 1u;
    }
    if (bad) kq_flag(status, KQ_DEV_INPUT);
    if (malformed) kq_flag(status, KQ_DEV_MALFORMED);
    if (nonfinite) kq_flag(status, KQ_DEV_NUMERIC);
    if (part_v != nullptr) {
#pragma unroll
        for (uint32_t k = 0; k < 4u; ++k) {
            float bv = best_v[k];
            uint32_t bi = best_i[k];
            /* lanes 16..63 hold no real column: only lanes 0..15 merge */
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o, KQ_WAVE);
                const uint32_t oi = __shfl_xor(bi, o, KQ_WAVE);
                mv_argmax_merge(bv, bi, ov, oi);
            }
            if (lane == 0u && k < batch) {
                part_v[(size_t)k * part_stride + gw] = bv;
                part_i[(size_t)k * part_stride + gw] = bi;
                for (uint32_t sl = gw + nwaves; sl < part_stride; sl += nwaves) {
                    part_v[(size_t)k * part_stride + sl] = -__builtin_inff();
                    part_i[(size_t)k * part_stride + sl] = 0xffffffffu;
                }
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* The same product at 2,048 columns on whole tiles shared by a workgroup
 *
 * matvec_mfma_q6k gives every wave its own ring of block slots and its own
 * tiles, so the weights in flight grow with the waves and two waves per
 * SIMD fill the LDS. Here a workgroup of eight waves owns a contiguous run
 * of 16-row tiles; a tile (16 rows x 1,680 contiguous bytes) is copied into
 * a two-slot LDS ring by 1 KiB LDS-DMA instructions spread over the waves,
 * one tile ahead of the one being multiplied, and wave b multiplies Q6_K
 * block b of every row of it. Its activation operand (the block's 256
 * columns of the four columns, hi and lo, laid out as above) is 32
 * registers held for the whole run, so nothing but the tile is read from
 * LDS and two workgroups share a CU (four waves per SIMD). Each wave sums
 * its product rows across lanes and leaves 16 rows x 4 columns in LDS;
 * after the next barrier wave 0 adds the eight blocks in order, unscales,
 * stores and keeps the argmax partials: one per workgroup and column. */

constexpr uint32_t kLtWaves = 8u;                      /* one per 256-column block */
constexpr uint32_t kLtRow = 8u * 210u;                 /* row bytes at 2,048 columns */
constexpr uint32_t kLtTile = kTile * kLtRow;           /* 26,880 */
constexpr uint32_t kLtIns = (kLtTile + 1023u) / 1024u; /* DMA instructions per tile: 27 */
constexpr uint32_t kLtSlot = kLtIns * 1024u;
constexpr uint32_t kLtIpw = (kLtIns + kLtWaves - 1u) / kLtWaves; /* per wave, at most 4 */

__global__ __launch_bounds__(kLtWaves * 64) __attribute__((amdgpu_waves_per_eu(4, 4)))
void lm_q6k_tiles(const uint8_t *__restrict__ W, uint32_t rows, const float *__restrict__ x,
                  uint32_t batch, float *__restrict__ y, uint32_t *status, float *part_v,
                  uint32_t *part_i, uint32_t part_stride) {
    constexpr uint32_t K = 2048u;
    __shared__ __align__(16) uint8_t ring[2][kLtSlot];
    __shared__ __align__(16) float part[2][kLtWaves][64];
    __shared__ float smax[kLtWaves][kMvCols];
    __shared__ uint32_t snf[kLtWaves][kMvCols];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t b = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); /* block of the row */
    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t ntiles = (rows + kTile - 1u) / kTile;
    const uint32_t lo = (uint32_t)((uint64_t)ntiles * blockIdx.x / gridDim.x);
    const uint32_t hi = (uint32_t)((uint64_t)ntiles * (blockIdx.x + 1u) / gridDim.x);
    const kq_i4v wr = dma_rsrc(W, rows * kLtRow);

    /* instruction n = b + 8 q of a tile: lane l copies tile bytes
     * [16 (64 n + l), + 16) to the same place in the slot; units past the
     * tile re-read its first bytes (never used) */
    uint32_t rel[kLtIpw];
#pragma unroll
    for (uint32_t q = 0; q < kLtIpw; ++q) {
        const uint32_t u = (b + kLtWaves * q) * 64u + lane;
        rel[q] = u * 16u < kLtTile ? u * 16u : 0u;
    }
    auto issue = [&](uint32_t t, uint32_t s) {
        const uint32_t toff = t * kLtTile, dst = lds_addr(&ring[s][0]);
#pragma unroll
        for (uint32_t q = 0; q < kLtIpw; ++q) {
            const uint32_t n = b + kLtWaves * q; /* wave-uniform */
            if (n < kLtIns) dma16(wr, toff + rel[q], dst + 1024u * n);
        }
    };
    if (lo < hi) issue(lo, 0u);

    /* column k's power of two from its largest magnitude: wave b scans its
     * block's 256 columns of the four (16 per lane), the workgroup merges */
    bool bad = false;
    {
        const uint32_t k = lane >> 4, c0 = 256u * b + 16u * (lane & 15u);
        float m = 0.0f;
        uint32_t nf = 0u;
        if (k < batch) {
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i) {
                const float4 v = *(const float4 *)(x + (size_t)k * K + c0 + 4u * i);
                nf |= (!kq_isfinite(v.x) || !kq_isfinite(v.y) || !kq_isfinite(v.z) ||
                       !kq_isfinite(v.w)) ? 1u : 0u;
                m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) {
            m = fmaxf(m, __shfl_xor(m, o, KQ_WAVE));
            nf |= __shfl_xor(nf, o, KQ_WAVE);
        }
        bad = nf != 0u;
        if ((lane & 15u) == 0u) {
            smax[b][k] = m;
            snf[b][k] = nf;
        }
    }
    __syncthreads();
    int sig[kMvCols];
    bool zero[kMvCols];
#pragma unroll
    for (uint32_t k = 0; k < kMvCols; ++k) {
        float m = 0.0f;
        uint32_t nf = 0u;
#pragma unroll
        for (uint32_t w = 0; w < kLtWaves; ++w) {
            m = fmaxf(m, smax[w][k]);
            nf |= snf[w][k];
        }
        zero[k] = nf != 0u;
        sig[k] = (nf == 0u && m > 0.0f) ? 15 - __builtin_amdgcn_frexp_expf(m) : 0;
    }

    /* lane (j, g): token row j of the A operand on k 8 g .. + 7 of step
     * (n, qq) = columns 256 b + 128 n + 32 qq + 8 g ..; rows 0..3 the hi
     * parts of columns 0..3, 4..7 their lo parts, 8..15 the same for the
     * step's second sub-block; lanes off their sub-block hold zeros */
    h8 av[2][4];
    {
        const uint32_t c = j & 3u;
        const bool live = (j >> 3) == (g >> 1) && c < batch && !zero[c];
        const bool want_lo = (j & 4u) != 0u;
        int e = sig[0];
#pragma unroll
        for (uint32_t k = 1; k < kMvCols; ++k) e = c == k ? sig[k] : e;
        const float *xp = x + (size_t)(live ? c : 0u) * K + 256u * b + 8u * g;
#pragma unroll
        for (uint32_t n = 0; n < 2u; ++n)
#pragma unroll
            for (uint32_t qq = 0; qq < 4u; ++qq) {
                float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                if (live) {
                    const float4 p0 = *(const float4 *)(xp + 128u * n + 32u * qq);
                    const float4 p1 = *(const float4 *)(xp + 128u * n + 32u * qq + 4u);
                    v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w;
                    v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
                }
                h8 h;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float xs = ldexpf(v[i], e);
                    const _Float16 hv = (_Float16)xs;
                    h[i] = want_lo ? (_Float16)(xs - (float)hv) : hv;
                }
                av[n][qq] = h;
            }
    }

    const uint32_t hsh = 8u * (g >> 1); /* this lane's scale byte within a pair */
    const h2 bias = h2{(_Float16)-1056.0f, (_Float16)-1056.0f}; /* 1024 + 32 */
    /* row j's block b in a slot: from its 4-byte aligned start, sh bytes in */
    const uint32_t boff = j * kLtRow + 210u * b;
    const uint32_t sh = boff & 3u, wbase = boff & ~3u;
    bool malformed = false, nonfinite = false;
    float best_v = -__builtin_inff();
    uint32_t best_i = 0xffffffffu;
    const uint32_t rk = lane >> 4, rr = lane & 15u; /* wave 0's output: column, row */

    for (uint32_t tau = lo; tau < hi + 1u; ++tau) {
        wait_vm<0>();
        kq_lds_barrier();
        if (tau + 1u < hi) issue(tau + 1u, (tau + 1u - lo) & 1u);
        if (tau > lo && b == 0u) {
            /* tile tau - 1: the eight blocks' sums in order */
            const uint32_t pb = (tau - 1u - lo) & 1u;
            float s = 0.0f;
#pragma unroll
            for (uint32_t w = 0; w < kLtWaves; ++w) s += part[pb][w][lane];
            const uint32_t row = (tau - 1u) * kTile + rr;
            if (row < rows && rk < batch) {
                const float v = ldexpf(s, -sig[rk]);
                nonfinite |= !kq_isfinite(v);
                y[(size_t)rk * rows + row] = v;
                mv_argmax_merge(best_v, best_i, v, row);
            }
        }
        if (tau == hi) break;

        const uint8_t *p = &ring[(tau - lo) & 1u][wbase];
        auto w32 = [&](uint32_t o) { return *(const uint32_t *)(p + o); };
        uint32_t wa[2][3], wbv[2][3], wq[2][3], ws[6];
#pragma unroll
        for (uint32_t n = 0; n < 2u; ++n) {
            const uint32_t oa = 64u * n + 8u * g, oq = 128u + 32u * n + 8u * g;
#pragma unroll
            for (uint32_t e = 0; e < 3u; ++e) {
                wa[n][e] = w32(oa + 4u * e);
                wbv[n][e] = w32(oa + 32u + 4u * e);
                wq[n][e] = w32(oq + 4u * e);
            }
        }
#pragma unroll
        for (uint32_t e = 0; e < 6u; ++e) ws[e] = w32(192u + 4u * e);
        const uint32_t row = tau * kTile + j;
        const float d = f16f(kq_align2(ws[5], ws[4], sh)); /* block bytes 208, 209 */
        malformed |= row < rows && !kq_isfinite(d);
        uint32_t sc[4];
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) sc[e] = kq_align2(ws[e + 1u], ws[e], sh) >> hsh;
        f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t n = 0; n < 2u; ++n) {
            const uint32_t A[2] = {kq_align2(wa[n][1], wa[n][0], sh),
                                   kq_align2(wa[n][2], wa[n][1], sh)};
            const uint32_t B[2] = {kq_align2(wbv[n][1], wbv[n][0], sh),
                                   kq_align2(wbv[n][2], wbv[n][1], sh)};
            const uint32_t H[2] = {kq_align2(wq[n][1], wq[n][0], sh),
                                   kq_align2(wq[n][2], wq[n][1], sh)};
            uint32_t c[4][2];
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                c[0][w] = (A[w] & 0x0f0f0f0fu) | ((H[w] << 4) & 0x30303030u);
                c[1][w] = (B[w] & 0x0f0f0f0fu) | ((H[w] << 2) & 0x30303030u);
                c[2][w] = ((A[w] >> 4) & 0x0f0f0f0fu) | (H[w] & 0x30303030u);
                c[3][w] = ((B[w] >> 4) & 0x0f0f0f0fu) | ((H[w] >> 2) & 0x30303030u);
            }
            f4 tm[4];
#pragma unroll
            for (uint32_t qq = 0; qq < 4u; ++qq) {
                const h2 w0 = bytes_lo(c[qq][0]) + bias, w1 = bytes_hi(c[qq][0]) + bias;
                const h2 w2 = bytes_lo(c[qq][1]) + bias, w3 = bytes_hi(c[qq][1]) + bias;
                const h8 bw = h8{w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
                tm[qq] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[n][qq], bw,
                                                                f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            }
#pragma unroll
            for (uint32_t qq = 0; qq < 4u; ++qq) {
                const int8_t scv = (int8_t)((sc[2u * n + (qq >> 1)] >> (16u * (qq & 1u))) & 0xffu);
                const float ds = d * (float)scv;
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[k] = fmaf(ds, tm[qq][k], acc[k]);
            }
        }
        /* column k of row j = the four lanes j + 16 G: hi and lo of both
         * sub-block halves */
        f4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = acc[k] + __shfl_down(acc[k], 32, KQ_WAVE);
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] += __shfl_down(o[k], 16, KQ_WAVE);
        if (g == 0u) {
#pragma unroll
            for (uint32_t k = 0; k < 4u; ++k) part[(tau - lo) & 1u][b][16u * k + j] = o[k];
        }
    }
    /* no LDS-DMA load may outlive the workgroup */
    wait_vm<0>();
    if (bad) kq_flag(status, KQ_DEV_INPUT);
    if (malformed) kq_flag(status, KQ_DEV_MALFORMED);
    if (nonfinite) kq_flag(status, KQ_DEV_NUMERIC);
    if (part_v != nullptr && b == 0u) {
        /* wave 0's lanes 16 k .. 16 k + 15 hold column k's candidates */
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) {
            const float ov = __shfl_xor(best_v, o, KQ_WAVE);
            const uint32_t oi = __shfl_xor(best_i, o, KQ_WAVE);
            mv_argmax_merge(best_v, best_i, ov, oi);
        }
        if (rr == 0u && rk < batch) {
            part_v[(size_t)rk * part_stride + blockIdx.x] = best_v;
            part_i[(size_t)rk * part_stride + blockIdx.x] = best_i;
            for (uint32_t sl = blockIdx.x + gridDim.x; sl < part_stride; sl += gridDim.x) {
                part_v[(size_t)rk * part_stride + sl] = -__builtin_inff();
                part_i[(size_t)rk * part_stride + sl] = 0xffffffffu;
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* grouped Q6_K down pass with its weights streamed through LDS
 *
 * The same work split, staging and Tile<Q6_K> steps as grouped_pass, but
 * the block operand pieces (twelve scattered 4-byte windows per lane) are
 * not fetched from global memory: each wave loads one 16-row block of its
 * tile contiguously (as matvec_mfma_q6k does) into a private LDS slot, two
 * blocks ahead of the one it multiplies, and the Raw pieces are read from
 * there. Offsets past the matrix read as zeros and stores past the
 * workgroup's outputs are dropped, so no path branches around a load. */
template <uint32_t KDIM, int NW, int TPW>
__global__ __launch_bounds__(NW * 64) void grouped_down_q6k(
    const uint8_t *__restrict__ W0, const uint8_t *__restrict__ SW0,
    const float *__restrict__ X, const uint32_t *__restrict__ offsets, uint32_t experts,
    uint32_t tokens, uint32_t top_k, uint32_t rows, uint32_t shared_chunks, uint32_t ybase,
    float *__restrict__ out, uint32_t *status) {
    using F = Fmt<KQ_LAUNCH_Q6_K>;
    using S = Stage<KQ_LAUNCH_Q6_K, KDIM>;
    using T = Tile<KQ_LAUNCH_Q6_K, KDIM, 1>;
    using Raw = F::Raw;
    constexpr uint32_t NB = KDIM / 256u;
    constexpr uint32_t RB = NB * F::kBytes;
    constexpr uint32_t NIT = (uint32_t)TPW * NB;
    static_assert(NIT % 2u == 0u, "items run in pairs");
    __shared__ S st;
    __shared__ int src_row[kTile];
    __shared__ __align__(16) uint8_t slots[NW][2][kMvSlot];

    const uint32_t e = blockIdx.y + ybase;
    const Work wk = work_of(e, offsets, experts, tokens, shared_chunks);
    if (wk.count == 0u) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t tk = tokens * top_k;
    auto tile_row = [&](uint32_t t) { return ((blockIdx.x * TPW + t) * NW + wave) * kTile; };
    const uint32_t wbytes = rows * RB;
    const KqBuf wb = kq_buf(wk.shared ? SW0 : W0 + (size_t)e * rows * RB, wbytes);
    const uint32_t pos0 = wk.shared ? tk + wk.first : wk.first;
    const uint32_t obytes = wk.count * rows * 4u;
    const KqBuf ob = kq_buf(out + (size_t)pos0 * rows, obytes);
    uint8_t *myslot = &slots[wave][0][0];

    /* item it = block it % NB of tile it / NB; unit e = i * 64 + lane of
     * its 224 loads covers bytes [16u, 16u + 16) of row e / 14's window
     * (the block start rounded down to 4 bytes) */
    typedef kq_u32x4 Ld[kMvLoads];
    auto load_item = [&](uint32_t it, Ld &v) {
        const uint32_t t = it / NB, b = it % NB;
#pragma unroll
        for (int i = 0; i < kMvLoads; ++i) {
            const uint32_t u0 = (uint32_t)i * 64u + lane;
            const uint32_t r = u0 / 14u, u = u0 - 14u * r;
            const uint32_t row = tile_row(t) + r;
            const uint32_t o = row * RB + b * F::kBytes;
            const uint32_t off = (u0 < kMvUnits && t < (uint32_t)TPW && row < rows)
                                     ? (o & ~3u) + 16u * u
                                     : wbytes + 256u;
            v[i] = __builtin_amdgcn_raw_buffer_load_b128(wb.r, (int)off, 0, 0);
        }
    };
    auto store_item = [&](uint32_t slot, const Ld &v) {
#pragma unroll
        for (int i = 0; i < kMvLoads; ++i) {
            const uint32_t u0 = (uint32_t)i * 64u + lane;
            const uint32_t r = u0 / 14u, u = u0 - 14u * r;
            if (u0 < kMvUnits)
                *(kq_u32x4 *)(myslot + slot * kMvSlot + r * kMvPitch + 16u * u) = v[i];
        }
    };
    /* the pieces Fmt<Q6_K>::load would read, from this lane's row in slot */
    auto lds_raw = [&](uint32_t slot, uint32_t t, uint32_t b) {
        const uint32_t o = (tile_row(t) + j) * RB + b * F::kBytes;
        const uint8_t *p = myslot + slot * kMvSlot + j * kMvPitch;
        auto w32 = [&](uint32_t off) { return *(const uint32_t *)(p + off); };
        Raw r;
        r.sh = o & 3u;
#pragma unroll
        for (uint32_t nh = 0; nh < 4u; ++nh) {
            const uint32_t n = nh >> 1, h = nh & 1u;
            const uint32_t oa = 64u * n + 16u * h + 4u * g;
            const uint32_t oq = 128u + 32u * n + 16u * h + 4u * g;
            r.w[nh][0] = kq_u32x2{w32(oa), w32(oa + 4u)};
            r.w[nh][1] = kq_u32x2{w32(oa + 32u), w32(oa + 36u)};
            r.w[nh][2] = kq_u32x2{w32(oq), w32(oq + 4u)};
        }
        r.sc = make_uint4(w32(192u), w32(196u), w32(200u), w32(204u));
        r.sc_tail = w32(208u);
        r.d = *(const uint16_t *)(p + r.sh + 208u);
        return r;
    };

    bool bad = false, malformed = false;
    for (uint32_t c0 = 0; c0 < wk.count; c0 += kTile) {
        Ld va, vb;
        load_item(0u, va);
        load_item(1u, vb);
        __syncthreads(); /* the previous chunk's readers are done */
        if (threadIdx.x < kTile) {
            const uint32_t i = threadIdx.x;
            int src = -1;
            if (c0 + i < wk.count) {
                const uint32_t p = wk.first + c0 + i;
                src = (int)(wk.shared ? tk + p : p);
            }
            src_row[i] = src;
        }
        __syncthreads();
        /* a non-finite intermediate activation is a numeric failure */
        bad |= stage_rows<KQ_LAUNCH_Q6_K, KDIM>(st, X, src_row, wave, NW, lane);
        __syncthreads();
        store_item(0u, va);
        load_item(2u, va);

        f4 acc[1];
        auto process = [&](uint32_t it, uint32_t slot) {
            const uint32_t t = it / NB, b = it % NB;
            if (b == 0u) acc[0] = f4{0.f, 0.f, 0.f, 0.f};
            const Raw rr[1] = {lds_raw(slot, t, b)};
            T::block(rr, st, b, j, g, acc, malformed);
            __builtin_amdgcn_sched_barrier(0);
            if (b + 1u < NB) return;
            /* D[token][row]: this lane holds row `row` of tokens 4g .. 4g+3 */
            const uint32_t row = tile_row(t) + j;
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q) {
                const uint32_t i = 4u * g + q;
                const bool valid = c0 + i < wk.count && row < rows;
                const float v = ldexpf(acc[0][q], -st.sig[i]);
                bad |= valid && !kq_isfinite(v);
                const uint32_t off = valid ? ((c0 + i) * rows + row) * 4u : obytes;
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ob.r, (int)off, 0, 0);
            }
        };
#pragma unroll 1
        for (uint32_t it = 0; it < NIT; it += 2u) {
            process(it, 0u);
            store_item(1u, vb);
            load_item(it + 3u, vb);
            process(it + 1u, 1u);
            store_item(0u, va);
            load_item(it + 4u, va);
        }
    }
    if (malformed) kq_flag(status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
}

template <uint32_t KDIM>
hipError_t launch_down_q6k(const uint8_t *W0, const uint8_t *SW0, const float *X,
                           const uint32_t *offsets, uint32_t experts, uint32_t tokens,
                           uint32_t top_k, uint32_t rows, uint32_t y0, uint32_t ny,
                           uint32_t chunks, float *out, uint32_t *status, hipStream_t s) {
    constexpr int NW = Shape<KQ_LAUNCH_Q6_K, KDIM, 1>::NW;
    constexpr int TPW = Shape<KQ_LAUNCH_Q6_K, KDIM, 1>::TPW;
    const uint32_t slab = (uint32_t)(NW * TPW) * kTile;
    const dim3 grid((rows + slab - 1u) / slab, ny);
    hipLaunchKernelGGL((grouped_down_q6k<KDIM, NW, TPW>), grid, dim3(NW * 64), 0, s, W0, SW0, X,
                       offsets, experts, tokens, top_k, rows, chunks, y0, out, status);
    return hipGetLastError();
}

}  // namespace

extern "C" int kq_launch_moe_grouped_supported(const kq_launch_moe_dims *d,
                                               const kq_launch_moe_weights *w) {
    /* gate/up in Q4_K (the 6-bit scales fold into exact fp16 weights) or
     * Q8_0, or Q5_K through the LDS pass (a Q5_K shared expert only with
     * Q5_K routed experts, in the same pass); down in Q4_K, Q6_K, Q5_1 or
     * Q8_0; routed and shared each of their own format, at the row lengths
     * each pass is built for */
    const bool q5 = w->gate_type == KQ_LAUNCH_Q5_K &&
                    kq_launch_gu_lds_supported(KQ_LAUNCH_Q5_K, d->hidden);
    return w->up_type == w->gate_type && w->shared_up_type == w->shared_gate_type &&
           (pass_dim_rt(w->gate_type, 2, d->hidden) || q5) &&
           (pass_dim_rt(w->shared_gate_type, 2, d->hidden) ||
            (q5 && w->shared_gate_type == KQ_LAUNCH_Q5_K)) &&
           pass_dim_rt(w->down_type, 1, d->inter) &&
           pass_dim_rt(w->shared_down_type, 1, d->inter) && d->inter == d->shared_inter &&
           d->experts <= 1023u;
}

extern "C" hipError_t kq_launch_moe_permute(const uint32_t *ids, uint32_t tokens, uint32_t top_k,
                                            uint32_t experts, uint32_t *offsets,
                                            uint32_t *pair_token, uint32_t *pos,
                                            uint32_t *pair_slot, uint32_t *status,
                                            hipStream_t s) {
    hipLaunchKernelGGL(moe_permute, dim3(1), dim3(1024), 0, s, ids, tokens, top_k, experts,
                       offsets, pair_token, pos, pair_slot, status, nullptr, 0u, nullptr, 0u);
    return hipGetLastError();
}

static bool gu_lds_routed(const kq_launch_moe_dims *d, const kq_launch_moe_weights *w) {
    return kq_launch_gu_lds_supported(w->gate_type, d->hidden) != 0;
}

extern "C" void *kq_launch_moe_grouped_stage(const kq_launch_moe_dims *d,
                                             const kq_launch_moe_weights *w,
                                             const kq_launch_moe_ws *ws) {
    return gu_lds_routed(d, w) ? (void *)ws->outp : nullptr;
}

extern "C" hipError_t kq_launch_moe_grouped(const kq_launch_moe_dims *d,
                                            const kq_launch_moe_weights *w, const float *hidden,
                                            uint32_t tokens, const kq_launch_moe_ws *ws,
                                            int staged, float *out, uint32_t *status,
                                            hipStream_t s) {
    /* Q4_K and Q5_K gate/up rows stream through LDS (kq_grouped_gu.hip) from
     * activations split once per token into the start of outp, which only
     * the down pass writes later; the work list the permutation builds for
     * it (gitems) also drives the Q6_K down pass (kq_grouped_dn.hip) */
    const bool lds_routed = gu_lds_routed(d, w);
    const bool lds_shared = lds_routed && w->shared_gate_type == w->gate_type;
    /* the mixed-tile gate/up pass (hidden 2048) records each position's
     * largest activation, and the Q6_K pair down pass (intermediate 512)
     * then splits its own operand: no dn_stage. The maxima live in dstage,
     * which only dn_stage and the dense shared expert use otherwise. */
    const bool fused_split = lds_shared && d->hidden == 2048u && d->inter == 512u &&
                             w->down_type == KQ_LAUNCH_Q6_K &&
                             w->shared_down_type == KQ_LAUNCH_Q6_K;
    uint32_t *posmax = fused_split ? (uint32_t *)ws->dstage : nullptr;
    hipLaunchKernelGGL(moe_permute, dim3(1), dim3(1024), 0, s, ws->ids, tokens, d->top_k,
                       d->experts, ws->offsets, ws->perm_tok, ws->pos, nullptr, status,
                       lds_routed ? (uint32_t *)ws->gitems : nullptr, lds_shared ? 1u : 0u,
                       posmax, posmax != nullptr ? tokens * (d->top_k + 1u) : 0u);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint8_t *g = (const uint8_t *)w->gate, *u = (const uint8_t *)w->up;
    const uint8_t *sg = (const uint8_t *)w->shared_gate, *su = (const uint8_t *)w->shared_up;
    const uint32_t E = d->experts;
    const uint32_t sh_wgs = (tokens + kSharedChunks * kTile - 1u) / (kSharedChunks * kTile);
    /* gate/up + SwiGLU, then down: the routed experts' workgroups and the
     * shared expert's in one launch when their formats agree */
    if (lds_routed && !staged) {
        e = kq_launch_gu_stage(hidden, tokens, d->hidden, ws->outp, status, s);
        if (e != hipSuccess) return e;
    }
    if (lds_routed) {
        e = kq_launch_gu_lds(w->gate_type, d->hidden, g, u, sg, su, ws->outp, ws->offsets,
                             ws->perm_tok, E, tokens, d->top_k, d->inter, lds_shared ? 1 : 0, 1,
                             ws->gitems, ws->act, posmax, status, s);
        if (e == hipSuccess && !lds_shared && w->shared_gate_type == KQ_LAUNCH_Q8_0 &&
            kq_launch_dense_q8_supported(d->inter, d->hidden, tokens)) {
            /* a Q8_0 shared expert sees every token: the dense product on
             * the same per-token split (kq_stage.h: xh [T][H], xl [T][H],
             * the 32-column sums [T][H/128][8] fp16, sig [T]), its rows
             * after the routed pairs' */
            const uint8_t *st = (const uint8_t *)ws->outp;
            const size_t th = (size_t)tokens * d->hidden;
            const int *sig =
                (const int *)(st + th * 4u + (size_t)tokens * (d->hidden / 128u) * 16u);
            float *sact = ws->act + (size_t)tokens * d->top_k * d->inter;
            /* the columns in up to four runs (more workgroups for the few
             * rows), their gate/up partials in dstage (free until the down
             * pass), summed in order with the SwiGLU */
            const uint32_t sp = kq_launch_dense_q8_splits(d->hidden, 4u);
            const uint64_t need = (uint64_t)sp * tokens * 2u * d->inter * 4u;
            const uint32_t ai = d->inter > d->shared_inter ? d->inter : d->shared_inter;
            if (sp > 1u && need <= kq_launch_dn_stage_bytes(tokens * (d->top_k + 1u), ai)) {
                e = kq_launch_dense_q8(sg, su, d->inter, d->hidden, st, st + th * 2u, sig, tokens,
                                       4u, (float *)ws->dstage, status, s);
                if (e == hipSuccess)
                    e = kq_launch_dense_swiglu((const float *)ws->dstage, sp, tokens, d->inter,
                                               sact, status, s);
            } else {
                e = kq_launch_dense_q8(sg, su, d->inter, d->hidden, st, st + th * 2u, sig, tokens,
                                       1u, sact, status, s);
            }
        } else if (e == hipSuccess && !lds_shared) {
            e = pass_any<2>(w->shared_gate_type, d->hidden, g, u, sg, su, hidden, ws->offsets,
                            ws->perm_tok, E, tokens, d->top_k, d->inter, E, sh_wgs, ws->act,
                            status, s);
        }
    } else if (w->shared_gate_type == w->gate_type) {
        e = pass_any<2>(w->gate_type, d->hidden, g, u, sg, su, hidden, ws->offsets, ws->perm_tok,
                        E, tokens, d->top_k, d->inter, 0u, E + sh_wgs, ws->act, status, s);
    } else {
        e = pass_any<2>(w->gate_type, d->hidden, g, u, sg, su, hidden, ws->offsets, ws->perm_tok,
                        E, tokens, d->top_k, d->inter, 0u, E, ws->act, status, s);
        if (e == hipSuccess)
            e = pass_any<2>(w->shared_gate_type, d->hidden, g, u, sg, su, hidden, ws->offsets,
                            ws->perm_tok, E, tokens, d->top_k, d->inter, E, sh_wgs, ws->act,
                            status, s);
    }
    if (e != hipSuccess) return e;
    const uint8_t *dn = (const uint8_t *)w->down, *sd = (const uint8_t *)w->shared_down;
    if (lds_shared && w->down_type == KQ_LAUNCH_Q6_K && w->shared_down_type == KQ_LAUNCH_Q6_K &&
        kq_launch_dn_lds_supported(d->inter)) {
        /* over the gate/up pass's item list (routed and shared chunks) */
        e = kq_launch_dn_lds(d->inter, d->hidden, dn, sd, ws->act, tokens, d->top_k, ws->gitems,
                             ws->dstage, posmax, ws->outp, status, s);
    } else if (lds_routed && kq_launch_dn_small_supported(w->down_type, d->inter) &&
               (!lds_shared || w->shared_down_type == w->down_type)) {
        /* Q5_1 or Q8_0 rows through the same per-wave LDS-DMA pipeline,
         * over the item list (the shared expert's chunks are in it when its
         * gate/up ran in the LDS gate/up pass; otherwise it runs below) */
        e = kq_launch_dn_small(w->down_type, d->inter, d->hidden, dn, sd, ws->act, tokens,
                               d->top_k, ws->gitems, ws->dstage, ws->outp, status, s);
        const size_t tk = (size_t)tokens * d->top_k;
        if (e == hipSuccess && !lds_shared && w->shared_down_type == KQ_LAUNCH_Q8_0 &&
            kq_launch_dense_q8_supported(d->hidden, d->inter, tokens)) {
            /* the dstage split above holds every position in natural order,
             * the shared expert's rows last */
            uint8_t *xs = (uint8_t *)ws->dstage;
            const size_t npos = tk + tokens, xb = npos * d->inter * 2u;
            e = kq_launch_dense_q8(sd, nullptr, d->hidden, d->inter, xs + tk * d->inter * 2u,
                                   xs + xb + tk * d->inter * 2u, (const int *)(xs + 2u * xb) + tk,
                                   tokens, 1u, ws->outp + tk * d->hidden, status, s);
        } else if (e == hipSuccess && !lds_shared) {
            e = pass_any<1>(w->shared_down_type, d->inter, dn, nullptr, sd, nullptr, ws->act,
                            ws->offsets, ws->perm_tok, E, tokens, d->top_k, d->hidden, E, sh_wgs,
                            ws->outp, status, s);
        }
    } else if (w->shared_down_type == w->down_type) {
        e = pass_any<1>(w->down_type, d->inter, dn, nullptr, sd, nullptr, ws->act, ws->offsets,
                        ws->perm_tok, E, tokens, d->top_k, d->hidden, 0u, E + sh_wgs, ws->outp,
                        status, s);
    } else {
        e = pass_any<1>(w->down_type, d->inter, dn, nullptr, sd, nullptr, ws->act, ws->offsets,
                        ws->perm_tok, E, tokens, d->top_k, d->hidden, 0u, E, ws->outp, status, s);
        const size_t tk = (size_t)tokens * d->top_k;
        if (e == hipSuccess && w->shared_down_type == KQ_LAUNCH_Q8_0 &&
            kq_launch_dense_q8_supported(d->hidden, d->inter, tokens)) {
            /* a Q8_0 shared expert's down on the dense product: its T
             * activation rows (after the routed pairs') split into dstage,
             * which only the LDS down pass uses */
            uint8_t *xs = (uint8_t *)ws->dstage;
            const size_t ti = (size_t)tokens * d->inter;
            e = kq_launch_dense_split(ws->act + tk * d->inter, tokens, d->inter, xs, xs + ti * 2u,
                                      (int *)(xs + ti * 4u), 0, status, s);
            if (e == hipSuccess)
                e = kq_launch_dense_q8(sd, nullptr, d->hidden, d->inter, xs, xs + ti * 2u,
                                       (const int *)(xs + ti * 4u), tokens, 1u,
                                       ws->outp + tk * d->hidden, status, s);
        } else if (e == hipSuccess) {
            e = pass_any<1>(w->shared_down_type, d->inter, dn, nullptr, sd, nullptr, ws->act,
                            ws->offsets, ws->perm_tok, E, tokens, d->top_k, d->hidden, E, sh_wgs,
                            ws->outp, status, s);
        }
    }
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(moe_combine, dim3((d->hidden / 4u + 255u) / 256u, tokens), dim3(256), 0, s,
                       ws->outp, ws->pos, ws->order, ws->weights, ws->shared_scale, tokens,
                       d->top_k, d->hidden, out, status);
    return hipGetLastError();
}

/* y[t] = W x[t] for every token: a Q8_0 matrix against many activation
 * rows on MFMA, as the grouped pass runs a shared matrix (16-token chunks,
 * one per workgroup), so the weights stream once per chunk instead of once
 * per four tokens */
extern "C" int kq_launch_gemm_q8_0_supported(uint32_t rows, uint32_t cols) {
    return rows != 0u && pass_dim<KQ_LAUNCH_Q8_0, 1>(cols);
}

extern "C" hipError_t kq_launch_gemm_q8_0(const void *W, uint32_t rows, uint32_t cols,
                                          const float *x, uint32_t tokens, float *y,
                                          uint32_t *status, hipStream_t s) {
    if (!kq_launch_gemm_q8_0_supported(rows, cols) || tokens == 0u) return hipErrorInvalidValue;
    const uint32_t ny = (tokens + kTile - 1u) / kTile;
    return pass_cols<KQ_LAUNCH_Q8_0, 1>(cols, nullptr, nullptr, (const uint8_t *)W, nullptr, x,
                                        nullptr, nullptr, 0u, tokens, 0u, rows, 0u, ny, 1u, y,
                                        status, s);
}

/* batched Q6_K matvec on MFMA: rows of 256 .. 4096 columns (whole blocks),
 * 2 .. 4 activation columns, at least 65,536 rows (enough 16-row tiles to
 * fill the device) */
extern "C" int kq_launch_matvec_mfma_supported(uint32_t type, uint32_t rows, uint32_t cols,
                                               uint32_t batch) {
    /* block offsets, and the out-of-range offset past the last row, stay
     * within 32 bits */
    const uint64_t bytes = (uint64_t)rows * (cols / 256u) * 210u;
    return type == KQ_LAUNCH_Q6_K && batch >= 2u && batch <= kMvCols && cols % 256u == 0u &&
           cols >= 256u && cols <= kMvMaxK && rows >= 65536u && bytes <= 0xfffff000ull;
}

/* block slots per wave: as many (2 .. kMvMaxSlots) as fit beside the
 * activation image */
static uint32_t mv_ns(uint32_t nb) {
    uint32_t ns = kMvMaxSlots;
    while (ns > 2u && mv_lds_bytes(nb, ns) > kMvLdsMax) --ns;
    return ns;
}
/* f(std::integral_constant<uint32_t, ns>) for ns in 2 .. kMvMaxSlots */
template <uint32_t NS = 2u, typename Fn>
static void kq_mv_ns_dispatch(uint32_t ns, Fn &&f) {
    if constexpr (NS <= kMvMaxSlots) {
        if (ns == NS) f(std::integral_constant<uint32_t, NS>{});
        else kq_mv_ns_dispatch<NS + 1u>(ns, f);
    }
}
template <uint32_t NS>
static hipError_t mv_occupancy(int *n, uint32_t nb) {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(n, matvec_mfma_q6k<NS>, kMvWaves * 64,
                                                         mv_lds_bytes(nb, NS));
}

/* a resident grid (workgroups that fit at once), capped by the tile count */
static uint32_t mv_blocks(uint32_t rows, uint32_t nb) {
    static uint32_t per_cu_cache[kMvMaxK / 256u + 1u];
    uint32_t &per = per_cu_cache[nb];
    if (per == 0u) {
        int dev = 0, cus = 0, n = 0;
        const uint32_t ns = mv_ns(nb);
        hipError_t oe = hipErrorInvalidValue;
        kq_mv_ns_dispatch(ns, [&](auto c) { oe = mv_occupancy<decltype(c)::value>(&n, nb); });
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus < 1)
            cus = 256;
        if (oe != hipSuccess || n < 1) n = 1;
        per = (uint32_t)(n * cus);
    }
    const uint32_t tiles = (rows + kTile - 1u) / kTile;
    uint32_t blocks = (tiles + (uint32_t)kMvWaves - 1u) / (uint32_t)kMvWaves;
    if (blocks > per) blocks = per;
    return blocks < 1u ? 1u : blocks;
}

/* lm_q6k_tiles (2,048 columns): two workgroups per CU */
static uint32_t lt_blocks() {
    static uint32_t blocks = 0u;
    if (blocks == 0u) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus < 1)
            cus = 256;
        blocks = 2u * (uint32_t)cus;
    }
    return blocks;
}

/* argmax partials per column: one per wave (matvec_mfma_q6k) or per
 * workgroup (lm_q6k_tiles) */
extern "C" uint32_t kq_launch_matvec_mfma_waves(uint32_t rows, uint32_t cols) {
    if (cols == 2048u) return lt_blocks();
    return mv_blocks(rows, cols / 256u) * (uint32_t)kMvWaves;
}

extern "C" hipError_t kq_launch_matvec_mfma(const void *W, uint32_t rows, uint32_t cols,
                                            const float *x, uint32_t batch, float *y,
                                            uint32_t *status, float *part_v, uint32_t *part_i,
                                            uint32_t part_stride, hipStream_t stream) {
    const uint32_t nb = cols / 256u;
    if (nb == 8u) {
        hipLaunchKernelGGL(lm_q6k_tiles, dim3(lt_blocks()), dim3(kLtWaves * 64), 0, stream,
                           (const uint8_t *)W, rows, x, batch, y, status, part_v, part_i,
                           part_stride);
        return hipGetLastError();
    }
    const uint32_t ns = mv_ns(nb);
    const dim3 grid(mv_blocks(rows, nb)), block(kMvWaves * 64);
#define KQ_MV(NS)                                                                              \
    hipLaunchKernelGGL(matvec_mfma_q6k<NS>, grid, block, mv_lds_bytes(nb, NS), stream,         \
                       (const uint8_t *)W, rows, nb, x, batch, y, status, part_v, part_i,      \
                       part_stride)
    kq_mv_ns_dispatch(ns, [&](auto c) { KQ_MV(decltype(c)::value); });
#undef KQ_MV
    return hipGetLastError();
}
