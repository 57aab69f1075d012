/*
 * kq_dense.hip — one Q8_0 matrix against many activation rows on MFMA:
 * y[t] = W x[t] for every token t, or swiglu(Wg x[t], Wu x[t]) for a
 * gate/up pair. These are the projections that see every token: the gated
 * residual's rank projections (src/kq_layer_qwen38.c:40-180, Q8_0 hc_*_down
 * and hc_*_up) and a shared expert of its own type
 * (src/kq_moe_qwen38.c:771-820). The reference forms them one token at a
 * time through kq_weight_provider_linear_f32 (src/kq_weight_provider.c:
 * 378-509).
 *
 * Activations are split once per row (dense_split, or the Q4_K gate/up
 * pass's split, kq_stage.h): scaled by an exact power of two (largest
 * magnitude into [2^14, 2^15)) and cut into fp16 hi + lo. Each wave of
 * dense_q8 owns 16 tokens by NT 16-row tiles and walks the columns in units
 * of two Q8_0 blocks, reading both operands straight from global memory
 * (the 4 waves of a workgroup read the same 16 activation rows, which L1
 * then serves) with the next units' loads in flight (a ring of R stages
 * in registers). Per block and tile:
 * the int8 codes enter fp16 exactly through the offset-binary byte, one
 * 16x16x32 MFMA step each for hi and lo, the fp32 result scaled by d.
 *
 * A split launch (grid z > 1) gives workgroup z an equal run of the units
 * and stores its unscaled-back partial products in slice z of the output
 * ([splits][tokens][rows]); the caller sums the slices in order.
 */
#include "kq_device.h"
#include "kq_launch.h"

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kTile = 16;
constexpr uint32_t kWaves = 4;
constexpr int kBadRow = 0x7fffffff;
constexpr uint32_t kMagic = 0x64646464u; /* fp16 0x64XX = 1024 + XX */

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ h2 bytes_lo(uint32_t m) {
    return as_h2(__builtin_amdgcn_perm(kMagic, m, 0x04010400u));
}
__device__ __forceinline__ h2 bytes_hi(uint32_t m) {
    return as_h2(__builtin_amdgcn_perm(kMagic, m, 0x04030402u));
}
__device__ __forceinline__ float f16f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu));
}

/* Row t of X [tokens][k] (k a multiple of 4): sig[t] and the scaled row as
 * fp16 hi + lo in xh, xl [tokens][k]; a row with a non-finite value is
 * staged as zeros with sig = kBadRow. One workgroup of 256 per row. */
__global__ __launch_bounds__(256) void dense_split(const float *__restrict__ X, uint32_t k,
                                                   _Float16 *__restrict__ xh,
                                                   _Float16 *__restrict__ xl,
                                                   int *__restrict__ sig_out, uint32_t flag,
                                                   uint32_t *status) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    __shared__ float s_max[4];
    __shared__ uint32_t s_bad[4];
    const uint32_t t = blockIdx.x, lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    const float4 *row = (const float4 *)(X + (size_t)t * k);
    const uint32_t ng = k / 4u;
    float m = 0.0f;
    bool nf = false;
    for (uint32_t i = threadIdx.x; i < ng; i += 256u) {
        const float4 v = row[i];
        nf |= !kq_isfinite(v.x) || !kq_isfinite(v.y) || !kq_isfinite(v.z) || !kq_isfinite(v.w);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const bool wbad = __ballot(nf) != 0ull;
    if (lane == 0u) {
        s_max[w] = m;
        s_bad[w] = wbad ? 1u : 0u;
    }
    __syncthreads();
    m = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    const bool bad = (s_bad[0] | s_bad[1] | s_bad[2] | s_bad[3]) != 0u;
    int sig = 0;
    if (!bad && m > 0.0f) sig = 15 - __builtin_amdgcn_frexp_expf(m);
    if (bad) sig = kBadRow;
    for (uint32_t i = threadIdx.x; i < ng; i += 256u) {
        const float4 v = row[i];
        const float a[4] = {v.x, v.y, v.z, v.w};
        _Float16 hi[4], lo[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float xs = bad ? 0.0f : ldexpf(a[c], sig);
            hi[c] = (_Float16)xs;
            lo[c] = (_Float16)(xs - (float)hi[c]);
        }
        *(h4 *)(xh + (size_t)t * k + 4u * i) = h4{hi[0], hi[1], hi[2], hi[3]};
        *(h4 *)(xl + (size_t)t * k + 4u * i) = h4{lo[0], lo[1], lo[2], lo[3]};
    }
    if (threadIdx.x == 0u) {
        sig_out[t] = sig;
        if (bad) kq_flag(status, flag);
    }
}

struct DenseArgs {
    const uint8_t *w0, *w1;        /* Q8_0 [rows][k]; w1 the up matrix (NMAT = 2) */
    const _Float16 *xh, *xl;       /* split activations [tokens][k] */
    const int *sig;                /* [tokens] */
    uint32_t rows, k, tokens;
    uint32_t units_per_split;      /* 64-column units per workgroup z */
    float *out;                    /* [splits][tokens][rows] (row stride `rows`) */
    uint32_t *status;
};

/* the codes and scales of one 64-column unit (two blocks) of a row: code
 * bytes 2 + 8g .. 9 + 8g of each block from a 12-byte aligned window, the
 * scale as half of an aligned dword */
struct Unit {
    kq_u32x3 c[2];
    uint32_t d[2];
};

__device__ __forceinline__ Unit load_unit(KqBuf w, uint32_t uoff, uint32_t g) {
    Unit r;
#pragma unroll
    for (uint32_t bb = 0; bb < 2u; ++bb) {
        const uint32_t a = uoff + 34u * bb + 2u + 8u * g;
        r.c[bb] = kq_ld96(w, a & ~3u, 0u);
        r.d[bb] = kq_ld32(w, (uoff + 34u * bb) & ~3u, 0u);
    }
    return r;
}

/* NT tiles of 16 rows per wave and matrix; waves of a workgroup take
 * consecutive tile groups; grid: x = row groups, y = 16-token chunks,
 * z = column splits */
template <int NMAT, int NT, int R>
__global__ __launch_bounds__(kWaves * 64) void dense_q8(DenseArgs a) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t rb = a.k / 32u * 34u; /* row bytes */
    const uint32_t nunits = a.k / 64u;
    const uint32_t u0 = blockIdx.z * a.units_per_split;
    const uint32_t u1 = min(nunits, u0 + a.units_per_split);
    const uint32_t t0 = blockIdx.y * kTile;
    const uint32_t r0 = (blockIdx.x * kWaves + wave) * (uint32_t)NT * kTile;
    const KqBuf bw[2] = {kq_buf(a.w0, a.rows * rb), kq_buf(NMAT == 2 ? a.w1 : a.w0, a.rows * rb)};
    /* this lane's activation row (token t0 + j; past the tokens: zeros) */
    const uint32_t xbytes = a.tokens * a.k * 2u;
    const KqBuf bh = kq_buf(a.xh, xbytes), bl = kq_buf(a.xl, xbytes);
    const uint32_t xo = t0 + j < a.tokens ? ((t0 + j) * a.k + 8u * g) * 2u : xbytes;
    /* this lane's row of tile i (past the rows: zeros, never stored) */
    uint32_t wo[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const uint32_t row = r0 + (uint32_t)i * kTile + j;
        wo[i] = row < a.rows ? row * rb : a.rows * rb;
    }

    f4 acc[NMAT][NT];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int i = 0; i < NT; ++i) acc[m][i] = f4{0.f, 0.f, 0.f, 0.f};

    struct Stage {
        uint4 xh[2], xl[2];
        Unit w[NMAT][NT];
    };
    auto fetch = [&](Stage &s, uint32_t u) {
        /* past the run: offsets beyond the buffers read zeros */
        const bool in = u < u1;
        const uint32_t xa = in ? xo + u * 128u : xbytes;
#pragma unroll
        for (uint32_t bb = 0; bb < 2u; ++bb) {
            s.xh[bb] = kq_ld128(bh, xa + 64u * bb, 0u);
            s.xl[bb] = kq_ld128(bl, xa + 64u * bb, 0u);
        }
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int i = 0; i < NT; ++i)
                s.w[m][i] = load_unit(bw[m], in ? wo[i] + u * 68u : a.rows * rb, g);
    };
    bool malformed = false;
    const h2 bias = h2{(_Float16)-1152.0f, (_Float16)-1152.0f}; /* 1024 + 128 */
    auto compute = [&](const Stage &s) {
#pragma unroll
        for (uint32_t bb = 0; bb < 2u; ++bb) {
            const h8 ah = __builtin_bit_cast(h8, s.xh[bb]);
            const h8 al = __builtin_bit_cast(h8, s.xl[bb]);
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    const kq_u32x3 wv = s.w[m][i].c[bb];
                    /* codes start 2 bytes into the window of even blocks */
                    uint32_t c0 = bb ? wv.x : kq_align2(wv.y, wv.x, 2u);
                    uint32_t c1 = bb ? wv.y : kq_align2(wv.z, wv.y, 2u);
                    c0 ^= 0x80808080u;
                    c1 ^= 0x80808080u;
                    const h2 q0 = bytes_lo(c0) + bias, q1 = bytes_hi(c0) + bias;
                    const h2 q2 = bytes_lo(c1) + bias, q3 = bytes_hi(c1) + bias;
                    const h8 bv = h8{q0.x, q0.y, q1.x, q1.y, q2.x, q2.y, q3.x, q3.y};
                    f4 t = {0.f, 0.f, 0.f, 0.f};
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bv, t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bv, t, 0, 0, 0);
                    const float d = f16f(bb ? s.w[m][i].d[bb] >> 16 : s.w[m][i].d[bb]);
                    malformed |= !kq_isfinite(d);
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[m][i][q] = fmaf(d, t[q], acc[m][i][q]);
                }
        }
    };

    /* a ring of R stages: the next R - 1 units' loads are in flight while
     * one is multiplied */
    Stage st[R];
#pragma unroll
    for (int p = 0; p < R - 1; ++p) fetch(st[p], u0 + (uint32_t)p);
    for (uint32_t u = u0; u < u1; u += (uint32_t)R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (u + (uint32_t)r >= u1) break;
            fetch(st[(r + R - 1) % R], u + (uint32_t)(r + R - 1));
            compute(st[r]);
        }
    }

    /* D[token][row]: this lane holds row r0 + 16 i + j of tokens
     * t0 + 4 g .. + 3 */
    bool bad = false;
    /* a split gate/up pair stores its gate and up partials ([z][tokens]
     * [2 rows]) for dense_swiglu; one matrix stores [z][tokens][rows] */
    const bool parts2 = NMAT == 2 && gridDim.z > 1u;
    const uint32_t ostride = parts2 ? 2u * a.rows : a.rows;
    float *out = a.out + (size_t)blockIdx.z * a.tokens * ostride;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t t = t0 + 4u * g + (uint32_t)q;
        if (t >= a.tokens) continue;
        const int sg = a.sig[t];
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const uint32_t row = r0 + (uint32_t)i * kTile + j;
            if (row >= a.rows) continue;
            float v;
            if constexpr (NMAT == 2) {
                const float gv = ldexpf(acc[0][i][q], -sg), uv = ldexpf(acc[1][i][q], -sg);
                if (parts2) {
                    out[(size_t)t * ostride + row] = gv;
                    out[(size_t)t * ostride + a.rows + row] = uv;
                    continue;
                }
                v = kq_swiglu(gv, uv);
                bad |= !kq_isfinite(gv) || !kq_isfinite(uv);
            } else {
                v = ldexpf(acc[0][i][q], -sg);
            }
            bad |= !kq_isfinite(v);
            out[(size_t)t * ostride + row] = v;
        }
    }
    if (malformed) kq_flag(a.status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(a.status, KQ_DEV_NUMERIC);
}

/* act[t][r] = swiglu(sum of the gate partials, sum of the up partials),
 * the splits summed in order (parts [splits][tokens][2 rows]) */
__global__ __launch_bounds__(256) void dense_swiglu(const float *__restrict__ parts,
                                                    uint32_t splits, uint32_t tokens,
                                                    uint32_t rows, float *__restrict__ out,
                                                    uint32_t *status) {
    const uint32_t n = tokens * rows;
    bool bad = false;
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u) {
        const uint32_t t = i / rows, r = i - t * rows;
        const size_t o = (size_t)t * 2u * rows + r, zs = (size_t)tokens * 2u * rows;
        float gv = parts[o], uv = parts[o + rows];
        for (uint32_t z = 1; z < splits; ++z) {
            gv = gv + parts[z * zs + o];
            uv = uv + parts[z * zs + o + rows];
        }
        const float v = kq_swiglu(gv, uv);
        bad |= !kq_isfinite(gv) || !kq_isfinite(uv) || !kq_isfinite(v);
        out[i] = v;
    }
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
}

}  // namespace

extern "C" hipError_t kq_launch_dense_swiglu(const float *parts, uint32_t splits,
                                             uint32_t tokens, uint32_t rows, float *out,
                                             uint32_t *status, hipStream_t s) {
    const uint32_t n = tokens * rows;
    uint32_t g = (n + 255u) / 256u;
    if (g > 4096u) g = 4096u;
    hipLaunchKernelGGL(dense_swiglu, dim3(g), dim3(256), 0, s, parts, splits, tokens, rows, out,
                       status);
    return hipGetLastError();
}

extern "C" int kq_launch_dense_q8_supported(uint32_t rows, uint32_t k, uint32_t tokens) {
    return rows != 0u && tokens != 0u && k % 64u == 0u && k != 0u &&
           (uint64_t)rows * (k / 32u) * 34u < (UINT64_C(1) << 31) &&
           (uint64_t)tokens * k * 2u < (UINT64_C(1) << 31);
}

/* the column splits a launch asked for `splits` actually makes (each an
 * equal run of 64-column units, none empty) */
extern "C" uint32_t kq_launch_dense_q8_splits(uint32_t k, uint32_t splits) {
    const uint32_t nunits = k / 64u;
    if (nunits == 0u || splits == 0u) return 1u;
    const uint32_t per = (nunits + splits - 1u) / splits;
    return (nunits + per - 1u) / per;
}

extern "C" hipError_t kq_launch_dense_split(const float *x, uint32_t tokens, uint32_t k,
                                            void *xh, void *xl, int *sig, int input,
                                            uint32_t *status, hipStream_t s) {
    if (k % 4u != 0u || tokens == 0u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dense_split, dim3(tokens), dim3(256), 0, s, x, k, (_Float16 *)xh,
                       (_Float16 *)xl, sig, input ? KQ_DEV_INPUT : KQ_DEV_NUMERIC, status);
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_dense_q8(const void *w0, const void *w1, uint32_t rows,
                                         uint32_t k, const void *xh, const void *xl,
                                         const int *sig, uint32_t tokens, uint32_t splits,
                                         float *out, uint32_t *status, hipStream_t s) {
    if (!kq_launch_dense_q8_supported(rows, k, tokens) || splits == 0u)
        return hipErrorInvalidValue;
    DenseArgs a;
    a.w0 = (const uint8_t *)w0;
    a.w1 = (const uint8_t *)w1;
    a.xh = (const _Float16 *)xh;
    a.xl = (const _Float16 *)xl;
    a.sig = sig;
    a.rows = rows;
    a.k = k;
    a.tokens = tokens;
    const uint32_t nunits = k / 64u;
    a.units_per_split = (nunits + splits - 1u) / splits;
    a.out = out;
    a.status = status;
    const uint32_t z = (nunits + a.units_per_split - 1u) / a.units_per_split;
    /* two 16-row tiles per wave; a gate/up pair (twice the tiles, fewer
     * workgroups) keeps three units in flight, one matrix one */
    const uint32_t per_wg = kWaves * 2u * kTile;
    const dim3 grid((rows + per_wg - 1u) / per_wg, (tokens + kTile - 1u) / kTile, z);
    if (w1 != nullptr)
        hipLaunchKernelGGL((dense_q8<2, 2, 4>), grid, dim3(kWaves * 64), 0, s, a);
    else
        hipLaunchKernelGGL((dense_q8<1, 2, 2>), grid, dim3(kWaves * 64), 0, s, a);
    return hipGetLastError();
}
