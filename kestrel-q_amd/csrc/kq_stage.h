/*
 * kq_stage.h — the per-token activation split read by the Q4_K prefill
 * gate/up pass (kq_grouped_gu.hip). It is formed by gu_stage or, when the
 * route runs first, by the route finish's workgroup of the same token
 * (kq_moe.hip), which reads that row anyway.
 *
 * Layout of the staged rows (one region):
 *   xh[t][K], xl[t][K]   fp16, the scaled row split hi + lo
 *   sx[t][K/128][8]      fp16: sums of sub-blocks 4q .. 4q + 3 (hi), then
 *                        the same four (lo); the sums carry 2^-5
 *   sig[t]               the row's power-of-two scale, or kBadRow
 */
#ifndef KQ_STAGE_H
#define KQ_STAGE_H

#include "kq_device.h"

namespace kq {

constexpr int kBadRow = 0x7fffffff;

struct StagedX {
    _Float16 *xh, *xl, *sx;
    int *sig;
};

__device__ __forceinline__ StagedX staged_at(void *base, uint32_t tokens, uint32_t k) {
    StagedX s;
    uint8_t *p = (uint8_t *)base;
    s.xh = (_Float16 *)p;
    p += (size_t)tokens * k * 2u;
    s.xl = (_Float16 *)p;
    p += (size_t)tokens * k * 2u;
    s.sx = (_Float16 *)p;
    p += (size_t)tokens * (k / 128u) * 16u;
    s.sig = (int *)p;
    return s;
}

/* Token t's row of X [tokens][k] (k a multiple of 256) scaled by 2^sig,
 * its largest magnitude in [2^14, 2^15), split hi + lo, with its 32-column
 * sums. The whole workgroup takes part (blockDim.x a multiple of 64, at
 * most 1024): each pass gives every wave all or none of its lanes. */
__device__ __forceinline__ void stage_row(const float *__restrict__ X, uint32_t t, uint32_t tokens,
                                          uint32_t k, void *staged, uint32_t *status) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    __shared__ float s_max[16];
    __shared__ uint32_t s_bad[16];
    const StagedX sx = staged_at(staged, tokens, k);
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const float4 *row = (const float4 *)(X + (size_t)t * k);
    const uint32_t ng = k / 4u; /* float4 groups, a multiple of 64 */
    float m = 0.0f;
    bool nf = false;
    for (uint32_t i = threadIdx.x; i < ng; i += blockDim.x) {
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
    m = 0.0f;
    uint32_t anybad = 0u;
    for (uint32_t q = 0; q < nw; ++q) {
        m = fmaxf(m, s_max[q]);
        anybad |= s_bad[q];
    }
    const bool bad = anybad != 0u;
    int sig = 0;
    if (!bad && m > 0.0f) sig = 15 - __builtin_amdgcn_frexp_expf(m);
    if (bad) sig = kBadRow;
    for (uint32_t i = threadIdx.x; i < ng; i += blockDim.x) {
        const float4 v = row[i];
        const float a[4] = {v.x, v.y, v.z, v.w};
        _Float16 hi[4], lo[4];
        float part = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float xs = bad ? 0.0f : ldexpf(a[c], sig);
            hi[c] = (_Float16)xs;
            lo[c] = (_Float16)(xs - (float)hi[c]);
            part += xs;
        }
        *(h4 *)(sx.xh + (size_t)t * k + 4u * i) = h4{hi[0], hi[1], hi[2], hi[3]};
        *(h4 *)(sx.xl + (size_t)t * k + 4u * i) = h4{lo[0], lo[1], lo[2], lo[3]};
        /* 32-column sums: groups 8j .. 8j + 7 are eight consecutive lanes */
        part += __shfl_xor(part, 1, 64);
        part += __shfl_xor(part, 2, 64);
        part += __shfl_xor(part, 4, 64);
        if ((i & 7u) == 0u) {
            const uint32_t sb = i / 8u;
            const float s = part * 0.03125f;
            const _Float16 sh = (_Float16)s;
            const _Float16 sl = (_Float16)(s - (float)sh);
            _Float16 *e = sx.sx + ((size_t)t * (k / 128u) + sb / 4u) * 8u;
            e[sb % 4u] = sh;
            e[4u + sb % 4u] = sl;
        }
    }
    if (threadIdx.x == 0u) {
        sx.sig[t] = sig;
        if (bad) kq_flag(status, KQ_DEV_INPUT);
    }
}

}  // namespace kq

#endif
