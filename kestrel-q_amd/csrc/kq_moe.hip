/*
 * kq_moe.hip — MoE layer on gfx950: exact router, softmax and
 * partial-selection top-k, grouped expert gate/up + SwiGLU, grouped down,
 * and the ordered combine with the sigmoid-gated shared expert.
 *
 * Restates kq_moe_execute_common (src/kq_moe_qwen38.c:604-867):
 *   route   logits[e] = sequential fp32 dot(router[e], x)    (:276-376)
 *           softmax (max, expf(l-max), left-to-right sum, divide)
 *           partial-selection top-k, then w = p / sum_topk(p)  (:211-274)
 *   expert  g = Wg x, u = Wu x, a = swiglu(g, u), o = Wd a     (:378-434)
 *   combine routed_sum += o * w in ascending expert id         (:722-765)
 *           out = routed_sum + sigmoid(wsg . x) * shared(x)    (:771-828)
 *
 * Router exactness. Expert ids must equal the CPU's bit for bit, so every
 * logit is the CPU's left-to-right binary32 sum: one lane per expert runs the
 * H-step chain. The router matrix (plus the shared gate vector as row E) is
 * first transposed to [H/4][E_pad][4] so that step q of all lanes of a wave
 * reads 1 KiB contiguous; for a single token the transpose also forms the
 * products w*x (each a rounded binary32 product, as the CPU forms them), so
 * the chain is one add per step.
 *
 * Top-k. The CPU's partial selection (seed ids 0..k-1; a later id replaces
 * the worst -- lowest value, lowest id among equals -- only when strictly
 * greater) selects exactly this set, which one workgroup computes in
 * parallel: with v* the k-th largest probability (with multiplicity),
 * G = {p > v*} and T = {p == v*}, let t0 be the index at which the running
 * count of {p >= v*} reaches k; the kept ties are T ∩ [0, t0] minus its
 * |G ∩ (t0, E)| lowest ids. (Derivation and brute-force check in the
 * oracle tests.) Final order: descending p, ascending id.
 */
#include "kq_launch.h"
#include "kq_rowdot.h"

namespace {

constexpr int kThreads = 256;

uint32_t pad64(uint32_t n) { return (n + 63u) & ~63u; }

/* ------------------------- router transpose ------------------------- */
/* Tile: 64 rows (experts) x 64 columns. Rows >= experts+1 are zero; row
 * `experts` is the shared gate vector. With PRODUCTS the tile is multiplied
 * by x (one token). Output [H/4][Ep][4]. */
template <bool PRODUCTS>
__global__ __launch_bounds__(kThreads) void router_transpose(
    const float *__restrict__ router, const float *__restrict__ shared_gate_weight,
    const float *__restrict__ x, uint32_t experts, uint32_t hidden, uint32_t ep,
    float *__restrict__ out, uint32_t *status) {
    __shared__ float4 tile[64][17];
    const uint32_t e0 = blockIdx.x * 64u, q0 = blockIdx.y * 16u;
    const uint32_t tid = threadIdx.x;
    bool bad = false;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t idx = tid + kThreads * k; /* 0..1023 */
        const uint32_t er = idx >> 4, qc = idx & 15u;
        const uint32_t e = e0 + er, q = q0 + qc;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (q * 4u < hidden) {
            if (e < experts)
                v = *(const float4 *)(router + (size_t)e * hidden + 4u * q);
            else if (e == experts)
                v = *(const float4 *)(shared_gate_weight + 4u * q);
            bad |= !kq_isfinite(v.x) || !kq_isfinite(v.y) || !kq_isfinite(v.z) ||
                   !kq_isfinite(v.w);
            if (PRODUCTS) {
                const float4 xv = *(const float4 *)(x + 4u * q);
                v.x = v.x * xv.x;
                v.y = v.y * xv.y;
                v.z = v.z * xv.z;
                v.w = v.w * xv.w;
            }
        }
        tile[er][qc] = v;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t idx = tid + kThreads * k;
        const uint32_t qc = idx >> 6, er = idx & 63u;
        const uint32_t q = q0 + qc;
        if (q * 4u < hidden) *(float4 *)(out + ((size_t)q * ep + e0 + er) * 4u) = tile[er][qc];
    }
    if (bad) kq_flag(status, KQ_DEV_INPUT);
}

/* ------------------------- router chain ------------------------- */
/* One lane per expert (and lane `experts` for the shared gate logit): the
 * CPU's left-to-right binary32 accumulation over H terms. One wave per
 * workgroup so the 64-lane chains spread over CUs. */
template <bool PRODUCTS>
__global__ __launch_bounds__(64) void router_chain(const float *__restrict__ src,
                                                   const float *__restrict__ hidden_states,
                                                   uint32_t experts, uint32_t hidden,
                                                   uint32_t ep, float *__restrict__ logits,
                                                   float *__restrict__ shared_logit) {
    const uint32_t e = blockIdx.x * 64u + threadIdx.x;
    const uint32_t t = blockIdx.y;
    const float *x = hidden_states + (size_t)t * hidden;
    const float4 *s = (const float4 *)src + e;
    const uint32_t nq = hidden / 4u;
    float acc = 0.0f;
    uint32_t q = 0;
    for (; q + 8u <= nq; q += 8u) {
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = s[(size_t)(q + j) * ep];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (PRODUCTS) {
                acc = acc + v[j].x;
                acc = acc + v[j].y;
                acc = acc + v[j].z;
                acc = acc + v[j].w;
            } else {
                const float4 xv = *(const float4 *)(x + 4u * (q + j));
                float p;
                p = v[j].x * xv.x; acc = acc + p;
                p = v[j].y * xv.y; acc = acc + p;
                p = v[j].z * xv.z; acc = acc + p;
                p = v[j].w * xv.w; acc = acc + p;
            }
        }
    }
    for (; q < nq; ++q) {
        const float4 v = s[(size_t)q * ep];
        if (PRODUCTS) {
            acc = acc + v.x;
            acc = acc + v.y;
            acc = acc + v.z;
            acc = acc + v.w;
        } else {
            const float4 xv = *(const float4 *)(x + 4u * q);
            float p;
            p = v.x * xv.x; acc = acc + p;
            p = v.y * xv.y; acc = acc + p;
            p = v.z * xv.z; acc = acc + p;
            p = v.w * xv.w; acc = acc + p;
        }
    }
    if (e < experts)
        logits[(size_t)t * experts + e] = acc;
    else if (e == experts)
        shared_logit[t] = acc;
}

/* ------------------------- route finish ------------------------- */
__device__ __forceinline__ float block_max(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, KQ_WAVE));
    const uint32_t w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63u) == 0u) red[w] = v;
    __syncthreads();
    float m = red[0];
    for (uint32_t i = 1; i < nw; ++i) m = fmaxf(m, red[i]);
    return m;
}

__device__ __forceinline__ uint32_t block_count(bool pred, uint32_t *cnt) {
    const uint64_t m = __ballot(pred);
    const uint32_t w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63u) == 0u) cnt[w] = (uint32_t)__popcll(m);
    __syncthreads();
    uint32_t c = 0;
    for (uint32_t i = 0; i < nw; ++i) c += cnt[i];
    return c;
}

/* exclusive prefix count of pred over thread index (all threads) */
__device__ __forceinline__ uint32_t block_prefix(bool pred, uint32_t *cnt) {
    const uint64_t m = __ballot(pred);
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0u) cnt[w] = (uint32_t)__popcll(m);
    __syncthreads();
    uint32_t before = 0;
    for (uint32_t i = 0; i < w; ++i) before += cnt[i];
    const uint64_t below = lane ? (m & (~0ull >> (64u - lane))) : 0ull;
    return before + (uint32_t)__popcll(below);
}

/* One workgroup per token; thread e owns expert e (blockDim = Ep <= 1024). */
__global__ __launch_bounds__(1024) void route_finish(
    const float *__restrict__ logits_all, const float *__restrict__ shared_logit,
    uint32_t experts, uint32_t top_k, float *__restrict__ probs_all, uint32_t *__restrict__ ids_all,
    float *__restrict__ weights_all, uint32_t *__restrict__ order_all,
    float *__restrict__ shared_scale, uint32_t *status) {
    __shared__ float ev[1024];
    __shared__ float red[16];
    __shared__ uint32_t cnt[16];
    __shared__ uint32_t sel_id[64];
    __shared__ float sel_p[64];
    __shared__ float s_sum;
    __shared__ uint32_t s_t0;
    const uint32_t t = blockIdx.x, e = threadIdx.x;
    const bool live = e < experts;
    const float *logits = logits_all + (size_t)t * experts;
    float l = live ? logits[e] : -__builtin_inff();
    const bool bad_in = live && !kq_isfinite(l);
    if (block_count(bad_in, cnt) != 0u) {
        /* fail closed, but leave in-range ids for the expert kernels */
        if (e < top_k) {
            ids_all[(size_t)t * top_k + e] = e;
            weights_all[(size_t)t * top_k + e] = 0.0f;
            order_all[(size_t)t * top_k + e] = e;
        }
        if (e == 0) {
            shared_scale[t] = 0.0f;
            kq_flag(status, KQ_DEV_NUMERIC);
        }
        return;
    }
    /* softmax: exact max, expf(l - max), left-to-right sum, divide */
    const float m = block_max(l, red);
    const float ex = live ? kq_expf(l - m) : 0.0f;
    ev[e] = ex;
    __syncthreads();
    if (e == 0) {
        float s = 0.0f;
        for (uint32_t i = 0; i < experts; ++i) s = s + ev[i];
        s_sum = s;
        shared_scale[t] = kq_sigmoid(shared_logit[t]);
        if (!kq_isfinite(s) || !(s > 0.0f)) kq_flag(status, KQ_DEV_NUMERIC);
    }
    __syncthreads();
    const float p = live ? ex / s_sum : -__builtin_inff();
    if (live) probs_all[(size_t)t * experts + e] = p;

    /* v* = k-th largest probability counting multiplicity */
    float vstar = 0.0f;
    {
        float cur = p;
        uint32_t taken = 0;
        for (uint32_t round = 0; round < top_k; ++round) {
            const float mx = block_max(cur, red);
            const uint32_t c = block_count(live && p == mx, cnt);
            taken += c;
            if (taken >= top_k) {
                vstar = mx;
                break;
            }
            if (p == mx) cur = -__builtin_inff();
        }
    }
    const bool in_g = live && p > vstar;
    const bool in_t = live && p == vstar;
    /* t0: index where the running count of {p >= v*} reaches k */
    if (e == 0) s_t0 = experts - 1u;
    const uint32_t ge_before = block_prefix(in_g || in_t, cnt);
    if ((in_g || in_t) && ge_before + 1u == top_k) s_t0 = e;
    __syncthreads();
    const uint32_t t0 = s_t0;
    const uint32_t g_after = block_count(in_g && e > t0, cnt);
    const uint32_t tie_rank = block_prefix(in_t && e <= t0, cnt);
    const bool keep = in_g || (in_t && e <= t0 && tie_rank >= g_after);
    const uint32_t slot = block_prefix(keep, cnt);
    /* the selection has exactly k members by construction; a defect would
     * otherwise index past sel_id, so it fails closed with in-range ids */
    const uint32_t kept = block_count(keep, cnt);
    if (kept == top_k) {
        if (keep) {
            sel_id[slot] = e;
            sel_p[slot] = p;
        }
    } else {
        if (e < top_k) {
            sel_id[e] = e;
            sel_p[e] = 0.0f;
        }
        if (e == 0) kq_flag(status, KQ_DEV_NUMERIC);
    }
    __syncthreads();
    if (e < top_k) {
        /* position in descending-p, ascending-id order; position in
         * ascending-id order (the combine order) is the compaction slot */
        const float my_p = sel_p[e];
        const uint32_t my_id = sel_id[e];
        uint32_t pos = 0;
        for (uint32_t j = 0; j < top_k; ++j) {
            const float pj = sel_p[j];
            const uint32_t ij = sel_id[j];
            pos += (pj > my_p || (pj == my_p && ij < my_id)) ? 1u : 0u;
        }
        ids_all[(size_t)t * top_k + pos] = my_id;
        weights_all[(size_t)t * top_k + pos] = my_p;
        order_all[(size_t)t * top_k + e] = pos;
    }
    __syncthreads();
    if (e == 0) {
        /* w = p / (left-to-right sum in top-k order) */
        float *w = weights_all + (size_t)t * top_k;
        float s = 0.0f;
        for (uint32_t j = 0; j < top_k; ++j) s += w[j];
        bool ok = kq_isfinite(s) && s > 0.0f;
        for (uint32_t j = 0; j < top_k; ++j) {
            w[j] /= s;
            ok = ok && kq_isfinite(w[j]);
        }
        if (!ok) kq_flag(status, KQ_DEV_NUMERIC);
    }
}

/* ---------------------- expert gate/up + SwiGLU ---------------------- */
/* grid: x = row groups, y = slot (0..K-1 routed by top-k position, K = the
 * shared expert), z = token. act[t][slot][row] = swiglu(g, u). Each wave
 * requests its gate and up rows before the activations (kq_rowdot.h). */
template <uint32_t TYPE, uint32_t COLS, int RT>
__global__ __launch_bounds__(kThreads) void expert_gateup(
    const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up,
    const uint8_t *__restrict__ sgate, const uint8_t *__restrict__ sup,
    const float *__restrict__ hidden_states, const uint32_t *__restrict__ ids,
    uint32_t top_k, uint32_t inter, uint32_t shared_inter, uint32_t act_stride,
    float *__restrict__ act, uint32_t *status) {
    using R = kq::Rows<TYPE, COLS, 1, RT>;
    using Raw = typename R::Raw;
    const uint32_t slot = blockIdx.y, t = blockIdx.z;
    const bool shared = slot == top_k;
    const uint32_t rows = shared ? shared_inter : inter;
    const uint8_t *G, *U;
    if (shared) {
        G = sgate;
        U = sup;
    } else {
        const uint32_t e = ids[(size_t)t * top_k + slot];
        G = gate + (size_t)e * inter * R::RB;
        U = up + (size_t)e * inter * R::RB;
    }
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = (blockIdx.x * kThreads + threadIdx.x) >> 6;
    const uint32_t nwaves = (gridDim.x * kThreads) >> 6;
    const uint32_t sub = lane / R::LPR, l = lane % R::LPR;
    const uint32_t ngroups = (rows + R::GROUP - 1u) / R::GROUP;
    typename R::Lane ln;
    ln.setup(l);
    Raw rg[RT], ru[RT];
    uint32_t g = wave;
    const KqBuf gb = kq_buf(G, rows * R::RB), ub = kq_buf(U, rows * R::RB);
    if (g < ngroups) {
        R::load_group(ln, gb, g, rows, sub, rg);
        R::load_group(ln, ub, g, rows, sub, ru);
    }
    if (ln.load_x(hidden_states + (size_t)t * COLS, COLS)) kq_flag(status, KQ_DEV_INPUT);
    bool bad = false, malformed = false;
    float *out = act + ((size_t)t * (top_k + 1u) + slot) * act_stride;
    for (; g < ngroups; g += nwaves) {
        if (g != wave) {
            R::load_group(ln, gb, g, rows, sub, rg);
            R::load_group(ln, ub, g, rows, sub, ru);
        }
        float vg[R::N], vu[R::N];
        R::dot_group(ln, rg, l, vg, malformed);
        R::dot_group(ln, ru, l, vu, malformed);
#pragma unroll
        for (int j = 0; j < R::KEEP; ++j) {
            const int idx = R::value_index(l, j);
            if (idx >= 0) {
                const uint32_t row = g * R::GROUP + (uint32_t)idx * R::RPW + sub;
                if (row < rows) {
                    const float a = kq_swiglu(vg[j], vu[j]);
                    bad |= !kq_isfinite(vg[j]) || !kq_isfinite(vu[j]) || !kq_isfinite(a);
                    out[row] = a;
                }
            }
        }
    }
    if (malformed) kq_flag(status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
}

/* ------------------------------ down ------------------------------ */
/* grid: x = row groups over hidden, y = slot, z = token.
 * expert_out[t][slot][f] = Wd[f] . act[t][slot]. */
template <uint32_t TYPE, uint32_t COLS, int RT>
__global__ __launch_bounds__(kThreads) void expert_down(
    const uint8_t *__restrict__ down, const uint8_t *__restrict__ sdown,
    const float *__restrict__ act, const uint32_t *__restrict__ ids, uint32_t top_k,
    uint32_t hidden, uint32_t act_stride, float *__restrict__ expert_out, uint32_t *status) {
    using R = kq::Rows<TYPE, COLS, 1, RT>;
    using Raw = typename R::Raw;
    const uint32_t slot = blockIdx.y, t = blockIdx.z;
    const bool shared = slot == top_k;
    const uint8_t *D =
        shared ? sdown : down + (size_t)ids[(size_t)t * top_k + slot] * hidden * R::RB;
    const KqBuf db = kq_buf(D, hidden * R::RB);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = (blockIdx.x * kThreads + threadIdx.x) >> 6;
    const uint32_t nwaves = (gridDim.x * kThreads) >> 6;
    const uint32_t sub = lane / R::LPR, l = lane % R::LPR;
    const uint32_t ngroups = (hidden + R::GROUP - 1u) / R::GROUP;
    typename R::Lane ln;
    ln.setup(l);
    Raw rd[RT];
    uint32_t g = wave;
    if (g < ngroups) R::load_group(ln, db, g, hidden, sub, rd);
    if (ln.load_x(act + ((size_t)t * (top_k + 1u) + slot) * act_stride, COLS))
        kq_flag(status, KQ_DEV_NUMERIC);
    bool bad = false, malformed = false;
    float *out = expert_out + ((size_t)t * (top_k + 1u) + slot) * hidden;
    for (; g < ngroups; g += nwaves) {
        if (g != wave) R::load_group(ln, db, g, hidden, sub, rd);
        float v[R::N];
        R::dot_group(ln, rd, l, v, malformed);
#pragma unroll
        for (int j = 0; j < R::KEEP; ++j) {
            const int idx = R::value_index(l, j);
            if (idx >= 0) {
                const uint32_t row = g * R::GROUP + (uint32_t)idx * R::RPW + sub;
                if (row < hidden) {
                    bad |= !kq_isfinite(v[j]);
                    out[row] = v[j];
                }
            }
        }
    }
    if (malformed) kq_flag(status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
}

/* ------------------------------ combine ------------------------------ */
/* routed_sum = 0; for experts in ascending id: routed_sum += o * w;
 * out = routed_sum + o_shared * sigmoid(shared logit). */
__global__ __launch_bounds__(kThreads) void moe_combine(
    const float *__restrict__ expert_out, const float *__restrict__ weights,
    const uint32_t *__restrict__ order, const float *__restrict__ shared_scale, uint32_t top_k,
    uint32_t hidden, float *__restrict__ out, uint32_t *status) {
    const uint32_t t = blockIdx.y;
    const uint32_t f = blockIdx.x * kThreads + threadIdx.x;
    if (f >= hidden) return;
    const float *eo = expert_out + (size_t)t * (top_k + 1u) * hidden;
    const float *w = weights + (size_t)t * top_k;
    const uint32_t *ord = order + (size_t)t * top_k;
    float sum = 0.0f;
    bool bad = false;
    for (uint32_t j = 0; j < top_k; ++j) {
        const uint32_t s = ord[j];
        const float weighted = eo[(size_t)s * hidden + f] * w[s];
        sum = sum + weighted;
        bad |= !kq_isfinite(sum);
    }
    const float gated = eo[(size_t)top_k * hidden + f] * shared_scale[t];
    const float v = sum + gated;
    bad |= !kq_isfinite(gated) || !kq_isfinite(v);
    out[(size_t)t * hidden + f] = v;
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
}

template <uint32_t TYPE, uint32_t COLS>
hipError_t launch_gateup(const kq_launch_moe_dims *d, const kq_launch_moe_weights *w,
                         const float *hidden, uint32_t tokens, const kq_launch_moe_ws *ws,
                         uint32_t act_stride, uint32_t *status, hipStream_t s) {
    constexpr int RT = 2;
    const uint32_t rows = d->inter > d->shared_inter ? d->inter : d->shared_inter;
    const uint32_t rows_per_wave = kq::Rows<TYPE, COLS, 1, RT>::GROUP;
    const uint32_t waves = (rows + rows_per_wave - 1u) / rows_per_wave;
    const uint32_t blocks = (waves + 3u) / 4u;
    hipLaunchKernelGGL((expert_gateup<TYPE, COLS, RT>), dim3(blocks, d->top_k + 1u, tokens),
                       dim3(kThreads), 0, s, (const uint8_t *)w->gate, (const uint8_t *)w->up,
                       (const uint8_t *)w->shared_gate, (const uint8_t *)w->shared_up, hidden,
                       ws->ids, d->top_k, d->inter, d->shared_inter, act_stride, ws->act,
                       status);
    return hipGetLastError();
}

template <uint32_t TYPE, uint32_t COLS>
hipError_t launch_down(const kq_launch_moe_dims *d, const kq_launch_moe_weights *w,
                       uint32_t tokens, const kq_launch_moe_ws *ws, uint32_t act_stride,
                       uint32_t *status, hipStream_t s) {
    constexpr int RT = 2;
    const uint32_t rows_per_wave = kq::Rows<TYPE, COLS, 1, RT>::GROUP;
    const uint32_t waves = (d->hidden + rows_per_wave - 1u) / rows_per_wave;
    const uint32_t blocks = (waves + 3u) / 4u;
    hipLaunchKernelGGL((expert_down<TYPE, COLS, RT>), dim3(blocks, d->top_k + 1u, tokens),
                       dim3(kThreads), 0, s, (const uint8_t *)w->down,
                       (const uint8_t *)w->shared_down, ws->act, ws->ids, d->top_k, d->hidden,
                       act_stride, ws->expert_out, status);
    return hipGetLastError();
}

template <uint32_t TYPE>
hipError_t gateup_cols(const kq_launch_moe_dims *d, const kq_launch_moe_weights *w,
                       const float *hidden, uint32_t tokens, const kq_launch_moe_ws *ws,
                       uint32_t act_stride, uint32_t *status, hipStream_t s) {
    switch (d->hidden) {
    case 256: return launch_gateup<TYPE, 256u>(d, w, hidden, tokens, ws, act_stride, status, s);
    case 512: return launch_gateup<TYPE, 512u>(d, w, hidden, tokens, ws, act_stride, status, s);
    case 1024: return launch_gateup<TYPE, 1024u>(d, w, hidden, tokens, ws, act_stride, status, s);
    case 2048: return launch_gateup<TYPE, 2048u>(d, w, hidden, tokens, ws, act_stride, status, s);
    default: return hipErrorInvalidValue;
    }
}

template <uint32_t TYPE>
hipError_t down_cols(const kq_launch_moe_dims *d, const kq_launch_moe_weights *w,
                     uint32_t tokens, const kq_launch_moe_ws *ws, uint32_t act_stride,
                     uint32_t *status, hipStream_t s) {
    switch (d->inter) {
    case 256: return launch_down<TYPE, 256u>(d, w, tokens, ws, act_stride, status, s);
    case 512: return launch_down<TYPE, 512u>(d, w, tokens, ws, act_stride, status, s);
    case 1024: return launch_down<TYPE, 1024u>(d, w, tokens, ws, act_stride, status, s);
    case 2048: return launch_down<TYPE, 2048u>(d, w, tokens, ws, act_stride, status, s);
    default: return hipErrorInvalidValue;
    }
}

bool quant_type(uint32_t t) {
    return t == KQ_LAUNCH_Q4_K || t == KQ_LAUNCH_Q6_K || t == KQ_LAUNCH_Q8_0;
}

bool cols_ok(uint32_t c) { return c == 256u || c == 512u || c == 1024u || c == 2048u; }

}  // namespace

extern "C" uint32_t kq_launch_moe_experts_padded(uint32_t experts) { return pad64(experts + 1u); }

static uint64_t align256(uint64_t v) { return (v + 255u) & ~(uint64_t)255u; }

extern "C" uint64_t kq_launch_moe_ws_bytes(const kq_launch_moe_dims *d, uint32_t tokens) {
    const uint64_t ep = pad64(d->experts + 1u);
    const uint64_t ai = d->inter > d->shared_inter ? d->inter : d->shared_inter;
    uint64_t b = 0;
    b += align256((uint64_t)d->hidden * ep * 4u);                   /* router_t */
    b += align256((uint64_t)tokens * d->experts * 4u) * 2u;         /* logits, probs */
    b += align256((uint64_t)tokens * d->top_k * 4u) * 3u;           /* ids, weights, order */
    b += align256((uint64_t)tokens * 4u) * 2u;                      /* shared logit, scale */
    b += align256((uint64_t)tokens * (d->top_k + 1u) * ai * 4u);    /* act */
    b += align256((uint64_t)tokens * (d->top_k + 1u) * d->hidden * 4u); /* expert_out */
    return b;
}

extern "C" void kq_launch_moe_ws_carve(const kq_launch_moe_dims *d, uint32_t tokens, void *base,
                                       kq_launch_moe_ws *ws) {
    const uint64_t ep = pad64(d->experts + 1u);
    const uint64_t ai = d->inter > d->shared_inter ? d->inter : d->shared_inter;
    uint8_t *p = (uint8_t *)base;
    ws->router_t = (float *)p; p += align256((uint64_t)d->hidden * ep * 4u);
    ws->logits = (float *)p; p += align256((uint64_t)tokens * d->experts * 4u);
    ws->probs = (float *)p; p += align256((uint64_t)tokens * d->experts * 4u);
    ws->ids = (uint32_t *)p; p += align256((uint64_t)tokens * d->top_k * 4u);
    ws->weights = (float *)p; p += align256((uint64_t)tokens * d->top_k * 4u);
    ws->order = (uint32_t *)p; p += align256((uint64_t)tokens * d->top_k * 4u);
    ws->shared_logit = (float *)p; p += align256((uint64_t)tokens * 4u);
    ws->shared_scale = (float *)p; p += align256((uint64_t)tokens * 4u);
    ws->act = (float *)p; p += align256((uint64_t)tokens * (d->top_k + 1u) * ai * 4u);
    ws->expert_out = (float *)p;
}

extern "C" int kq_launch_moe_supported(const kq_launch_moe_dims *d,
                                       const kq_launch_moe_weights *w) {
    if (d->hidden % 4u != 0u || d->experts + 1u > 1024u || d->top_k < 1u ||
        d->top_k > d->experts || d->top_k > 64u)
        return 0;
    if (w == nullptr) return 1;
    if (!quant_type(w->gate_type) || w->up_type != w->gate_type ||
        w->shared_gate_type != w->gate_type || w->shared_up_type != w->gate_type)
        return 0;
    if (!quant_type(w->down_type) || w->shared_down_type != w->down_type) return 0;
    if (!cols_ok(d->hidden) || !cols_ok(d->inter) || d->inter != d->shared_inter) return 0;
    return 1;
}

extern "C" hipError_t kq_launch_moe_route(const kq_launch_moe_dims *d, const float *router,
                                          const float *shared_gate_weight, const float *hidden,
                                          uint32_t tokens, const kq_launch_moe_ws *ws,
                                          uint32_t *status, hipStream_t s) {
    const uint32_t ep = pad64(d->experts + 1u);
    const dim3 tgrid(ep / 64u, (d->hidden / 4u + 15u) / 16u);
    const bool products = tokens == 1u;
    if (products)
        hipLaunchKernelGGL((router_transpose<true>), tgrid, dim3(kThreads), 0, s, router,
                           shared_gate_weight, hidden, d->experts, d->hidden, ep, ws->router_t,
                           status);
    else
        hipLaunchKernelGGL((router_transpose<false>), tgrid, dim3(kThreads), 0, s, router,
                           shared_gate_weight, hidden, d->experts, d->hidden, ep, ws->router_t,
                           status);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (products)
        hipLaunchKernelGGL((router_chain<true>), dim3(ep / 64u, tokens), dim3(64), 0, s,
                           ws->router_t, hidden, d->experts, d->hidden, ep, ws->logits,
                           ws->shared_logit);
    else
        hipLaunchKernelGGL((router_chain<false>), dim3(ep / 64u, tokens), dim3(64), 0, s,
                           ws->router_t, hidden, d->experts, d->hidden, ep, ws->logits,
                           ws->shared_logit);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(route_finish, dim3(tokens), dim3(ep), 0, s, ws->logits, ws->shared_logit,
                       d->experts, d->top_k, ws->probs, ws->ids, ws->weights, ws->order,
                       ws->shared_scale, status);
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_moe_experts(const kq_launch_moe_dims *d,
                                            const kq_launch_moe_weights *w, const float *hidden,
                                            uint32_t tokens, const kq_launch_moe_ws *ws,
                                            float *out, uint32_t *status, hipStream_t s) {
    const uint32_t act_stride = d->inter > d->shared_inter ? d->inter : d->shared_inter;
    hipError_t e;
    switch (w->gate_type) {
    case KQ_LAUNCH_Q4_K:
        e = gateup_cols<KQ_LAUNCH_Q4_K>(d, w, hidden, tokens, ws, act_stride, status, s);
        break;
    case KQ_LAUNCH_Q6_K:
        e = gateup_cols<KQ_LAUNCH_Q6_K>(d, w, hidden, tokens, ws, act_stride, status, s);
        break;
    case KQ_LAUNCH_Q8_0:
        e = gateup_cols<KQ_LAUNCH_Q8_0>(d, w, hidden, tokens, ws, act_stride, status, s);
        break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    switch (w->down_type) {
    case KQ_LAUNCH_Q4_K: e = down_cols<KQ_LAUNCH_Q4_K>(d, w, tokens, ws, act_stride, status, s); break;
    case KQ_LAUNCH_Q6_K: e = down_cols<KQ_LAUNCH_Q6_K>(d, w, tokens, ws, act_stride, status, s); break;
    case KQ_LAUNCH_Q8_0: e = down_cols<KQ_LAUNCH_Q8_0>(d, w, tokens, ws, act_stride, status, s); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(moe_combine, dim3((d->hidden + kThreads - 1u) / kThreads, tokens),
                       dim3(kThreads), 0, s, ws->expert_out, ws->weights, ws->order,
                       ws->shared_scale, d->top_k, d->hidden, out, status);
    return hipGetLastError();
}
