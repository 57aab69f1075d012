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
#include <type_traits>

#include "kq_launch.h"
#include "kq_rowdot.h"
#include "kq_stage.h"

namespace {

constexpr int kThreads = 256;

uint32_t pad64(uint32_t n) { return (n + 63u) & ~63u; }

/* ------------------------- router, one token ------------------------- */
/* One workgroup per 8 logit rows: expert rows, then the shared gate vector
 * as row `experts`; rows past it load nothing and are discarded. Every
 * thread issues all of its loads at once (HBM latency exceeds the chain
 * time of a segment), then the four waves form the rounded binary32
 * products w*x (as the CPU forms them) segment by segment and stage them in
 * LDS as [q][row] float4, q = column / 4, with one float4 of padding per q
 * so that every eight consecutive q of a store hit distinct banks. Lanes
 * 0..7 of wave 0 run the left-to-right chains from LDS, one segment of 512
 * columns behind the staging; a barrier per segment publishes it. The chain
 * is 4 adds per q: a 2048-column router is 2048 dependent adds. */
constexpr uint32_t kRtRows = 8;
constexpr uint32_t kRtSegQ = 128;
constexpr uint32_t kRtPitch = kRtRows + 1u;
constexpr uint32_t kRtPerSeg = kRtRows * kRtSegQ / kThreads; /* float4 per thread */

__device__ __forceinline__ void add4(float &acc, const float4 v) {
    acc = acc + v.x;
    acc = acc + v.y;
    acc = acc + v.z;
    acc = acc + v.w;
}

/* acc += b[0], b[pitch], ... for n float4 in order; full runs of 128 are
 * software-pipelined so the next eight reads are in flight during the adds */
__device__ __forceinline__ void chain_lds(const float4 *b, uint32_t pitch, uint32_t n,
                                          float &acc) {
    if (n == kRtSegQ) {
        float4 va[8], vb[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) va[j] = b[j * pitch];
#pragma unroll
        for (uint32_t q = 0; q < kRtSegQ; q += 16u) {
#pragma unroll
            for (int j = 0; j < 8; ++j) vb[j] = b[(q + 8u + j) * pitch];
#pragma unroll
            for (int j = 0; j < 8; ++j) add4(acc, va[j]);
            if (q + 16u < kRtSegQ) {
#pragma unroll
                for (int j = 0; j < 8; ++j) va[j] = b[(q + 16u + j) * pitch];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) add4(acc, vb[j]);
        }
    } else {
        for (uint32_t q = 0; q < n; ++q) add4(acc, b[q * pitch]);
    }
}

__device__ __forceinline__ float4 as_f4(const uint4 u) {
    return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                       __uint_as_float(u.w));
}

/* The chains of logit rows row0 .. row0 + 7 (the experts, then the shared
 * gate vector as row E), computed by the workgroup's first kThreads
 * threads; any further threads only take part in the barriers. */
template <uint32_t HIDDEN>
__device__ __forceinline__ void router_decode_rows(
    const float *__restrict__ router, const float *__restrict__ shared_gate_weight,
    const float *__restrict__ x, uint32_t experts, float *__restrict__ logits,
    float *__restrict__ shared_logit, uint32_t *status, uint32_t row0) {
    constexpr uint32_t NQ = HIDDEN / 4u;
    constexpr uint32_t NSEG = (NQ + kRtSegQ - 1u) / kRtSegQ;
    __shared__ float4 buf[NSEG * kRtSegQ * kRtPitch];
    const uint32_t tid = threadIdx.x;
    const bool active = tid < (uint32_t)kThreads; /* whole waves */
    /* thread covers column group ql of rows rsub + 2k (k < 4); rsub is
     * uniform across a wave, so each row's buffer descriptor is scalar.
     * Rows past the shared gate row get an empty buffer and columns past
     * the row's end lie outside it: the buffer loads return zeros. */
    const uint32_t ql = tid % kRtSegQ;
    const uint32_t rsub = __builtin_amdgcn_readfirstlane(tid / kRtSegQ);
    /* at most four segments' loads are held in registers; segment sg + 4
     * is requested once segment sg has been staged */
    constexpr uint32_t NR = NSEG < 4u ? NSEG : 4u;
    uint4 v[NR][kRtPerSeg], xr[NR];
    KqBuf rb[kRtPerSeg];
    const KqBuf xb = kq_buf(x, HIDDEN * 4u);
    auto issue = [&](uint32_t sg) {
        const uint32_t off = (sg * kRtSegQ + ql) * 16u, r = sg % NR;
        xr[r] = kq_ld128(xb, off, 0);
#pragma unroll
        for (uint32_t k = 0; k < kRtPerSeg; ++k) v[r][k] = kq_ld128(rb[k], off, 0);
    };
    if (active) {
#pragma unroll
        for (uint32_t k = 0; k < kRtPerSeg; ++k) {
            const uint32_t e = row0 + rsub + 2u * k;
            rb[k] = kq_buf(e < experts ? router + (size_t)e * HIDDEN : shared_gate_weight,
                           e <= experts ? HIDDEN * 4u : 0u);
        }
#pragma unroll
        for (uint32_t sg = 0; sg < NR; ++sg) issue(sg);
    }
    bool bad = false;
    auto stage = [&](uint32_t sg) {
        if (!active) return;
        float4 *b = buf + (sg * kRtSegQ + ql) * kRtPitch + rsub;
        const float4 xq = as_f4(xr[sg % NR]);
#pragma unroll
        for (uint32_t k = 0; k < kRtPerSeg; ++k) {
            const float4 w = as_f4(v[sg % NR][k]);
            bad |= !kq_isfinite(w.x) || !kq_isfinite(w.y) || !kq_isfinite(w.z) ||
                   !kq_isfinite(w.w);
            float4 p;
            p.x = w.x * xq.x;
            p.y = w.y * xq.y;
            p.z = w.z * xq.z;
            p.w = w.w * xq.w;
            b[2u * k] = p;
        }
    };
    /* after the barrier that follows stage(sg), segment sg's registers are
     * free: request segment sg + NR there (the barrier keeps the loads
     * from being hoisted into the registers still in use) */
    auto refill = [&](uint32_t sg) {
        if (active && sg + NR < NSEG) issue(sg + NR);
    };
    stage(0);
    __syncthreads();
    refill(0);
    float acc = 0.0f;
#pragma unroll
    for (uint32_t sg = 0; sg < NSEG; ++sg) {
        if (tid < kRtRows) {
            constexpr uint32_t kLast = NQ - (NSEG - 1u) * kRtSegQ;
            chain_lds(buf + sg * kRtSegQ * kRtPitch + tid, kRtPitch,
                      sg + 1u < NSEG ? kRtSegQ : kLast, acc);
        }
        if (sg + 1u < NSEG) {
            stage(sg + 1u);
            __syncthreads();
            refill(sg + 1u);
        }
    }
    if (tid < kRtRows) {
        const uint32_t e = row0 + tid;
        if (e < experts)
            logits[e] = acc;
        else if (e == experts)
            *shared_logit = acc;
    }
    if (bad) kq_flag(status, KQ_DEV_INPUT);
}

template <uint32_t HIDDEN>
__global__ __launch_bounds__(kThreads) void router_decode(
    const float *__restrict__ router, const float *__restrict__ shared_gate_weight,
    const float *__restrict__ x, uint32_t experts, float *__restrict__ logits,
    float *__restrict__ shared_logit, uint32_t *status) {
    router_decode_rows<HIDDEN>(router, shared_gate_weight, x, experts, logits, shared_logit,
                               status, blockIdx.x * kRtRows);
}

/* ---------------------- router, several tokens ---------------------- */
/* The router matrix (plus the shared gate vector as row E) is transposed to
 * [H/4][E_pad][4] (64x64 LDS tiles; rows past E are zero) so that step q of
 * a wave's 64 chains reads 1 KiB contiguous. */
__global__ __launch_bounds__(kThreads) void router_transpose(
    const float *__restrict__ router, const float *__restrict__ shared_gate_weight,
    uint32_t experts, uint32_t hidden, uint32_t ep, float *__restrict__ out, uint32_t *status) {
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

/* One lane per (token, expert): p = w * x rounded, acc = acc + p, in column
 * order. One wave per workgroup so the chains spread over CUs. */
__global__ __launch_bounds__(64) void router_chain(const float *__restrict__ wt,
                                                   const float *__restrict__ hidden_states,
                                                   uint32_t experts, uint32_t hidden,
                                                   uint32_t ep, float *__restrict__ logits,
                                                   float *__restrict__ shared_logit) {
    const uint32_t e = blockIdx.x * 64u + threadIdx.x;
    const uint32_t t = blockIdx.y;
    const float4 *x = (const float4 *)(hidden_states + (size_t)t * hidden);
    const float4 *s = (const float4 *)wt + e;
    const uint32_t nq = hidden / 4u;
    float acc = 0.0f;
    auto step = [&](const float4 w, const float4 xv) {
        float p;
        p = w.x * xv.x; acc = acc + p;
        p = w.y * xv.y; acc = acc + p;
        p = w.z * xv.z; acc = acc + p;
        p = w.w * xv.w; acc = acc + p;
    };
    uint32_t q = 0;
    for (; q + 8u <= nq; q += 8u) {
        float4 v[8], xv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[j] = s[(size_t)(q + j) * ep];
            xv[j] = x[q + j];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) step(v[j], xv[j]);
    }
    for (; q < nq; ++q) step(s[(size_t)q * ep], x[q]);
    if (e < experts)
        logits[(size_t)t * experts + e] = acc;
    else if (e == experts)
        shared_logit[t] = acc;
}

/* Many tokens, the router read where it lies (no transposed copy): lane e
 * of a wave runs the chain of expert e0 + e for one token; the kSxWaves
 * waves of a workgroup take consecutive tokens and share one copy of their
 * 64 router rows, which the workgroup moves into LDS 64 columns at a time,
 * transposed to [q][expert] (one float4 of padding per q line), double
 * buffered: one barrier per 64 columns. A token's activations are the same
 * in every lane, so they come through scalar loads into SGPRs and each term
 * is two VALU instructions, p = w * x rounded, then acc = acc + p, in
 * column order. One token per wave keeps four waves on every SIMD to cover
 * the loads' latency (two tokens per wave halve the LDS reads per term but
 * leave two waves per SIMD, and ran 30% slower at 512 x 512). Rows past the
 * experts read as zeros and are not stored; the shared gate vector is not a
 * row here (its logit only feeds the sigmoid gate, compared by tolerance). */
constexpr uint32_t kSxTW = 1;
constexpr uint32_t kSxWaves = 8;
constexpr uint32_t kSxCols = 64;

__global__ __launch_bounds__(64 * kSxWaves) void router_chain_sx(
    const float *__restrict__ router, const float *__restrict__ hidden_states, uint32_t tokens,
    uint32_t experts, uint32_t hidden, float *__restrict__ logits, uint32_t *status) {
    constexpr uint32_t NQ = kSxCols / 4u;  /* float4 per row per chunk */
    constexpr uint32_t PITCH = 65u;        /* float4 per q line */
    constexpr uint32_t LOADS = 64u * NQ / (64u * kSxWaves); /* float4 per thread per chunk */
    __shared__ float4 tile[2][NQ * PITCH];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t e0 = blockIdx.y * 64u;
    const uint32_t tb = (blockIdx.x * kSxWaves + wave) * kSxTW;
    /* loader: float4 q = tid % NQ of rows tid / NQ + (64 * kSxWaves / NQ) * k */
    const uint32_t lq = tid % NQ, lr = tid / NQ;
    constexpr uint32_t RSTEP = 64u * kSxWaves / NQ;
    const float *xr[kSxTW];
#pragma unroll
    for (uint32_t b = 0; b < kSxTW; ++b) {
        const uint32_t t = tb + b < tokens ? tb + b : tokens - 1u;
        xr[b] = hidden_states + (size_t)__builtin_amdgcn_readfirstlane(t) * hidden;
    }
    float4 ld[LOADS];
    bool bad = false;
    auto gload = [&](uint32_t c) {
#pragma unroll
        for (uint32_t k = 0; k < LOADS; ++k) {
            const uint32_t e = e0 + lr + RSTEP * k;
            ld[k] = e < experts
                        ? *(const float4 *)(router + (size_t)e * hidden + c * kSxCols + 4u * lq)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto lstore = [&](uint32_t buf) {
#pragma unroll
        for (uint32_t k = 0; k < LOADS; ++k) {
            const float4 v = ld[k];
            bad |= !kq_isfinite(v.x) || !kq_isfinite(v.y) || !kq_isfinite(v.z) ||
                   !kq_isfinite(v.w);
            tile[buf][lq * PITCH + lr + RSTEP * k] = v;
        }
    };
    float acc[kSxTW];
#pragma unroll
    for (uint32_t b = 0; b < kSxTW; ++b) acc[b] = 0.0f;
    const uint32_t nc = hidden / kSxCols;
    gload(0u);
    lstore(0u);
    __syncthreads();
    if (nc > 1u) gload(1u);
    for (uint32_t c = 0; c < nc; ++c) {
        const float4 *tl = tile[c & 1u] + lane;
        /* the chunk's 64 columns of the token in SGPRs, one wait per chunk */
#pragma unroll
        for (uint32_t q = 0; q < NQ; ++q) {
            const float4 w = tl[q * PITCH];
#pragma unroll
            for (uint32_t b = 0; b < kSxTW; ++b) {
                const float4 xv = *(const float4 *)(xr[b] + c * kSxCols + 4u * q);
                float p;
                p = w.x * xv.x; acc[b] = acc[b] + p;
                p = w.y * xv.y; acc[b] = acc[b] + p;
                p = w.z * xv.z; acc[b] = acc[b] + p;
                p = w.w * xv.w; acc[b] = acc[b] + p;
            }
        }
        /* the other buffer was last read before the previous barrier */
        if (c + 1u < nc) lstore((c + 1u) & 1u);
        __syncthreads();
        if (c + 2u < nc) gload(c + 2u);
    }
    const uint32_t e = e0 + lane;
#pragma unroll
    for (uint32_t b = 0; b < kSxTW; ++b) {
        if (tb + b < tokens && e < experts) logits[(size_t)(tb + b) * experts + e] = acc[b];
    }
    if (bad) kq_flag(status, KQ_DEV_INPUT);
}

/* Maximum over the 64 lanes of a wave, returned in every lane: DPP within
 * 16-lane rows, then permlane swaps across rows. All lanes must be active. */
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, kq_dpp_pair<1>(v));
    v = fmaxf(v, kq_dpp_pair<2>(v));
    v = fmaxf(v, kq_dpp_pair<7>(v));
    v = fmaxf(v, kq_dpp_pair<15>(v));
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

/* ---------------- certified routing for one token ---------------- */
/*
 * Expert ids must be the CPU's, whose logits are left-to-right binary32
 * sums (2048 dependent adds per logit). For one token the execute path first
 * tries to certify the selection without those chains:
 *
 * Bounds: for each logit row the rounded products p_i = w_i * x_i are
 *   formed exactly as the CPU does and fp64 prefix sums give their partial
 *   sums S_i. The CPU's sum l satisfies
 *   |l - S_n| <= u / (1 - u) * sum_{i>=2} |l_i| (recursive summation, l_i the
 *   CPU's own partial sums, u = 2^-24), and sum |l_i| <= sum |S_i| /
 *   (1 - n u / (1 - u)); with n <= 2048 the bound below takes
 *   1.001 * u * sum |S_i|, which covers both factors and the fp64 rounding.
 *   Any non-finite product, or partial sums near the binary32 range, make
 *   the bound infinite.
 * Certification: with a_e = S_n and bounds b_e, the top-k by a_e is the
 *   CPU's selection in the CPU's order if every adjacent pair in it, and
 *   its last member against every unselected expert, is separated by more
 *   than the two bounds plus a margin, and the higher member's probability
 *   is a normal binary32 number: the margin keeps the rounded
 *   probabilities fl(fl(exp(fl(l - max))) / s) strictly ordered too, so no
 *   tie (and no tie-break) can occur. It then writes the ids, the weights
 *   p / sum(p) from the fp64 values (compared by tolerance like the layer
 *   output), the ascending-id slot order and the shared gate, and sets the
 *   flag that makes the exact router and route finish return at once;
 *   otherwise they run and overwrite everything.
 */
/* Rows of route_bounds: one logit row per workgroup of four waves, each
 * wave a quarter of the columns (E + 1 workgroups spread over the CUs). */
constexpr uint32_t kSelRows = 1;
constexpr uint32_t kSelParts = 4;

constexpr uint32_t kMaxTopK = 64;
constexpr uint32_t kCertCand = 128; /* candidates one wave ranks, two per lane */

/* hi - bhi exceeds lo + blo by more than the bounds and 16 units in the
 * last place of the probability terms involved (m: the largest a), and the
 * higher one's probability exp(hi - max) / sum is a normal binary32 number
 * (sum <= 1024 terms of at most 1): a lower probability may round to a
 * subnormal or to zero, but not up to it. Two probabilities that both
 * underflow tie on the CPU, which then orders them by id. */
__device__ __forceinline__ bool certify_sep(double hi, double bhi, double lo, double blo,
                                            double m) {
    const double margin = 0x1p-20 * (4.0 + fabs(hi - m) + fabs(lo - m));
    return (hi - bhi) - m > -75.0 && (hi - bhi) - (lo + blo) > margin;
}

__device__ __forceinline__ float rdl_f32(float v, uint32_t lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)lane));
}

/* set bits of m below this lane */
__device__ __forceinline__ uint32_t bits_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

/*
 * One workgroup of 16 waves (1024 threads), one thread per expert, after
 * the bounds kernel. The top-k by a (larger
 * first, lower id among equals) is found without sorting all experts, with
 * keys f = (float)a (rounding is monotone):
 *   1. each full wave (64 experts; the one partial wave when E < 64) finds
 *      its per-th largest key, per = ceil(need / such waves),
 *      need = min(k + 1, E) (per > 64 finds -inf);
 *   2. t = the least of those keys: every such wave has at least `per` keys
 *      >= t, so at least `need` experts do;
 *   3. each wave appends its experts with f >= t to one list (an LDS
 *      counter hands out the places) and keeps the largest a + b among its
 *      other experts;
 *   4. wave 0 ranks the candidates by a itself. More than 64 candidates
 *      leaves the selection uncertified.
 * Only wave 0 runs after the second barrier, and a lone wave pays each
 * instruction's latency, so that part is short and free of table reads.
 * The weights and the shared gate use the hardware exponential: they are
 * compared by tolerance, like the layer output.
 */
struct CertCand {
    double a;
    uint32_t id, pad;
};

__device__ __forceinline__ float fast_expf(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    v += kq_dpp_pair<1>(v);
    v += kq_dpp_pair<2>(v);
    v += kq_dpp_pair<7>(v);
    v += kq_dpp_pair<15>(v);
    v = kq_fold16(v, v);
    return kq_fold32(v, v);
}

/*
 * Bounds of all logit rows (the shared gate vector as row E).
 * Wave w of a workgroup takes quarter w % 4 of row kSelRows * blockIdx.x +
 * w / 4;
 * its lanes hold C consecutive columns each, so the wave's partial sums are
 * the lane's own running sum plus a wave scan, and the row's are those plus
 * the totals of the quarters before it.
 */
template <uint32_t HIDDEN>
__device__ __forceinline__ void bounds_rows(
    const float *__restrict__ router, const float *__restrict__ shared_gate_weight,
    const float *__restrict__ x, uint32_t experts, double *__restrict__ bound) {
    constexpr uint32_t PART = HIDDEN / kSelParts;
    constexpr uint32_t C = PART / 64u; /* 1 .. 8 */
    __shared__ double p_tot[16], p_abs[16];
    __shared__ uint32_t p_bad[16];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t part = w % kSelParts;
    const uint32_t row = blockIdx.x * kSelRows + w / kSelParts;
    const bool have = row <= experts; /* uniform over the wave */
    float pr[C];
    double incl = 0.0;
    if (have) {
        const float *wr = (row < experts ? router + (size_t)row * HIDDEN : shared_gate_weight) +
                          part * PART + lane * C;
        const float *xr = x + part * PART + lane * C;
        float wv[C], xv[C];
        if constexpr (C % 4u == 0u) {
#pragma unroll
            for (uint32_t q = 0; q < C / 4u; ++q) {
                const float4 a = ((const float4 *)wr)[q], b = ((const float4 *)xr)[q];
                wv[4u * q] = a.x, wv[4u * q + 1u] = a.y, wv[4u * q + 2u] = a.z, wv[4u * q + 3u] = a.w;
                xv[4u * q] = b.x, xv[4u * q + 1u] = b.y, xv[4u * q + 2u] = b.z, xv[4u * q + 3u] = b.w;
            }
        } else {
#pragma unroll
            for (uint32_t i = 0; i < C; ++i) {
                wv[i] = wr[i];
                xv[i] = xr[i];
            }
        }
        bool bad = false;
        double run = 0.0;
#pragma unroll
        for (uint32_t i = 0; i < C; ++i) {
            pr[i] = wv[i] * xv[i];
            bad |= !kq_isfinite(pr[i]); /* also NaN or infinite w or x */
            run += (double)pr[i];
        }
        incl = kq_wave_scan_f64(run);
        const bool any_bad = __ballot(bad) != 0ull;
        if (lane == 63u) {
            p_tot[w] = incl;
            p_bad[w] = any_bad ? 1u : 0u;
        }
    }
    __syncthreads();
    if (have) {
        /* S_i of this lane's columns: earlier quarters, earlier lanes, then
         * the lane's own products */
        double s = kq_wave_shr1_f64(incl);
        for (uint32_t q = 0; q < part; ++q) s += p_tot[w - part + q];
        double s4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (uint32_t i = 0; i < C; ++i) {
            s += (double)pr[i];
            s4[i & 3u] += fabs(s);
        }
        const double sabs = kq_wave_sum_f64((s4[0] + s4[1]) + (s4[2] + s4[3]));
        if (lane == 0u) p_abs[w] = sabs;
    }
    __syncthreads();
    /* thread 0 writes the workgroup's rows */
    if (threadIdx.x == 0u) {
        for (uint32_t r = 0; r < kSelRows; ++r) {
            const uint32_t rr = blockIdx.x * kSelRows + r;
            if (rr > experts) break;
            double tot = 0.0, sab = 0.0;
            uint32_t bad = 0;
#pragma unroll
            for (uint32_t q = 0; q < kSelParts; ++q) {
                tot += p_tot[r * kSelParts + q];
                sab += p_abs[r * kSelParts + q];
                bad |= p_bad[r * kSelParts + q];
            }
            bound[2u * rr] = tot;
            /* partial sums near the binary32 range could overflow in the
             * CPU's chain: only the exact path reports that */
            bound[2u * rr + 1u] =
                bad || !(sab < 0x1p126) ? __builtin_inf() : 1.001 * 0x1p-24 * sab;
        }
    }
}

/* ------------------------- route finish ------------------------- */
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
    const uint32_t lane = threadIdx.x & 63u;
    return (uint32_t)__popcll(lane ? (m & (~0ull >> (64u - lane))) : 0ull);
}

__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

/* Maximum over the wave of int keys, in every lane (DPP within rows,
 * permlane swaps across rows; all lanes active). */
template <int CTRL>
__device__ __forceinline__ int dpp_imax(int v) {
    return max(v, __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ int wave_imax(int v) {
    v = dpp_imax<0xB1>(v);  /* lane ^ 1 */
    v = dpp_imax<0x4E>(v);  /* lane ^ 2 */
    v = dpp_imax<0x141>(v); /* mirror within 8 */
    v = dpp_imax<0x140>(v); /* mirror within 16 */
    auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    v = max((int)r[0], (int)r[1]);
    r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    return max((int)r[0], (int)r[1]);
}

template <int S>
__device__ __forceinline__ int tree_imax(const int *c) {
    if constexpr (S == 1) {
        return c[0];
    } else {
        return max(tree_imax<S / 2>(c), tree_imax<S / 2>(c + S / 2));
    }
}

/* k-th largest (with multiplicity) of v[0..n-1], n <= 64 * S, in every lane
 * of the calling wave. The values are +0 or positive (softmax numerators),
 * so their bit patterns order as int32, and -inf (negative as int32) marks
 * an empty slot. Each round takes the maximum of what remains, counts its
 * copies and removes them all. */
template <int S>
__device__ __forceinline__ float kth_largest(const float *v, uint32_t n, uint32_t k) {
    const uint32_t lane = threadIdx.x & 63u;
    constexpr int kEmpty = (int)0xff800000u;
    int c[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const uint32_t i = lane + 64u * s;
        c[s] = i < n ? __float_as_int(v[i]) : kEmpty;
    }
    uint32_t taken = 0;
    int m = kEmpty;
    for (uint32_t r = 0; r < k; ++r) {
        m = wave_imax(tree_imax<S>(c));
        uint32_t cnt = 0;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const bool hit = c[s] == m;
            cnt += (uint32_t)__popcll(__ballot(hit));
            c[s] = hit ? kEmpty : c[s];
        }
        taken += cnt;
        if (taken >= k || cnt == 0u) break;
    }
    return __int_as_float(m);
}

/* Ballot masks of up to 16 waves: count of set bits in waves before `w`
 * and in all waves. Entries of absent waves hold 0. */
__device__ __forceinline__ void mask_counts(const uint64_t *msk, uint32_t w, uint32_t &before,
                                            uint32_t &total) {
    before = 0u;
    total = 0u;
#pragma unroll
    for (uint32_t i = 0; i < 16u; ++i) {
        const uint32_t c = (uint32_t)__popcll(msk[i]);
        before += i < w ? c : 0u;
        total += c;
    }
}

/* One workgroup per token; thread e owns expert e. The last wave (an extra
 * all-padding wave when the block has room) runs the softmax's
 * left-to-right sum on lane 0 while wave 0 finds the k-th largest ex.
 *
 * Selection runs on ex = expf(l - max): p = fl(ex / s) is non-decreasing in
 * ex for the one divisor s, so the k-th largest p (with multiplicity) is
 * v* = fl(ex* / s) for the k-th largest ex*. With G = {p > v*}, T = {p ==
 * v*} and c(e) = |(G u T) n [0, e]|, the CPU's partial selection keeps G
 * and the members e of T with c(e) <= k, less the |G n {c > k}| lowest ids
 * among them (c(e) <= k is e <= t0 for members, t0 being the member at
 * which the running count reaches k). */
__device__ __forceinline__ void route_finish_body(
    uint32_t t, const float *__restrict__ logits_all, const float *__restrict__ shared_logit,
    uint32_t experts, uint32_t top_k, float *__restrict__ probs_all, uint32_t *__restrict__ ids_all,
    float *__restrict__ weights_all, uint32_t *__restrict__ order_all,
    float *__restrict__ shared_scale, uint32_t *status) {
    __shared__ __align__(16) float ev[1024];
    __shared__ __align__(16) float wmx[16];
    __shared__ __align__(16) uint32_t wbad[16];
    __shared__ __align__(16) uint64_t msk[4][16];
    __shared__ __align__(16) uint32_t sel_id[64];
    __shared__ __align__(16) float sel_p[64];
    __shared__ __align__(16) float sorted_p[64];
    __shared__ float s_sum, s_exk;
    const uint32_t e = threadIdx.x;
    const uint32_t lane = e & 63u, w = e >> 6, nw = blockDim.x >> 6;
    const uint32_t sum_wave = nw - 1u;
    const bool live = e < experts;
    const float l = live ? logits_all[(size_t)t * experts + e] : -__builtin_inff();
    const float sl = e == 0u ? shared_logit[t] : 0.0f;
    const bool bad_in = live && !kq_isfinite(l);
    if (e < 16u && e >= nw) {
        wmx[e] = -__builtin_inff();
        wbad[e] = 0u;
        for (int r = 0; r < 4; ++r) msk[r][e] = 0ull;
    }
    if (e < 64u) sorted_p[e] = 0.0f;

    /* max of the logits and the count of non-finite ones, one barrier */
    {
        const float wm = wave_max(l);
        const uint64_t bm = __ballot(bad_in);
        if (lane == 0u) {
            wmx[w] = wm;
            wbad[w] = (uint32_t)__popcll(bm);
        }
    }
    __syncthreads();
    float m = -__builtin_inff();
    uint32_t nbad = 0;
#pragma unroll
    for (uint32_t i = 0; i < 16u; ++i) {
        m = fmaxf(m, wmx[i]);
        nbad += wbad[i];
    }
    if (nbad != 0u) {
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

    const float ex = live ? kq_expf(l - m) : 0.0f;
    ev[e] = ex;
    __syncthreads();
    /* Softmax sum, left to right. Entries past the experts hold +0, which
     * leaves a non-negative running sum unchanged, so the sum runs over
     * whole float4 in pipelined runs. Global stores wait until after the
     * last barrier (a barrier waits for the wave's outstanding stores). */
    if (w == sum_wave && lane == 0u) {
        float sum = 0.0f;
        const uint32_t nv = (experts + 3u) / 4u;
        for (uint32_t i = 0; i < nv; i += kRtSegQ) {
            const uint32_t left = nv - i;
            chain_lds((const float4 *)ev + i, 1u, left < kRtSegQ ? left : kRtSegQ, sum);
        }
        s_sum = sum;
    }
    if (w == 0u) {
        float exk;
        if (experts <= 64u)
            exk = kth_largest<1>(ev, experts, top_k);
        else if (experts <= 128u)
            exk = kth_largest<2>(ev, experts, top_k);
        else if (experts <= 256u)
            exk = kth_largest<4>(ev, experts, top_k);
        else if (experts <= 512u)
            exk = kth_largest<8>(ev, experts, top_k);
        else
            exk = kth_largest<16>(ev, experts, top_k);
        if (lane == 0u) s_exk = exk;
    }
    __syncthreads();
    const float s = s_sum;
    const float p = live ? ex / s : -__builtin_inff();
    const float vstar = s_exk / s;
    const bool in_g = live && p > vstar;
    const bool in_t = live && p == vstar;
    {
        const uint64_t gm = __ballot(in_g);
        const uint64_t tm = __ballot(in_t);
        if (lane == 0u) {
            msk[0][w] = gm;
            msk[1][w] = tm;
        }
    }
    __syncthreads();
    /* c(e) = members of G u T up to e; the tie candidates are the members
     * of T with c(e) <= k, and the last k - |G| of them are kept */
    uint32_t g_before, g_total, t_before, t_total;
    mask_counts(msk[0], w, g_before, g_total);
    mask_counts(msk[1], w, t_before, t_total);
    const uint32_t g_pre = g_before + lanes_below(msk[0][w]);
    const uint32_t t_pre = t_before + lanes_below(msk[1][w]);
    const bool tie_cand = in_t && g_pre + t_pre + 1u <= top_k;
    {
        const uint64_t cm = __ballot(tie_cand);
        if (lane == 0u) msk[2][w] = cm;
    }
    __syncthreads();
    uint32_t c_before, cands;
    mask_counts(msk[2], w, c_before, cands);
    const uint32_t c_pre = c_before + lanes_below(msk[2][w]); /* tie candidates below e */
    const uint32_t need = top_k > g_total ? top_k - g_total : 0u;
    const uint32_t drop = cands > need ? cands - need : 0u;    /* lowest candidates dropped */
    const bool keep = in_g || (tie_cand && c_pre >= drop);
    /* ascending-id slot: G members below e plus kept candidates below e */
    const uint32_t slot = g_pre + (c_pre > drop ? c_pre - drop : 0u);
    const uint32_t kept = g_total + (cands < need ? cands : need);
    /* the selection has exactly k members by construction; a defect would
     * otherwise index past sel_id, so it fails closed with in-range ids */
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
    /* position in descending-p, ascending-id order; the position in
     * ascending-id order (the combine order) is the compaction slot */
    uint32_t pos = 0, my_id = 0;
    float my_p = 0.0f;
    if (e < top_k) {
        my_p = sel_p[e];
        my_id = sel_id[e];
        for (uint32_t j0 = 0; j0 < top_k; j0 += 4u) {
            const float4 pj = *(const float4 *)(sel_p + j0);
            const uint4 ij = *(const uint4 *)(sel_id + j0);
            const float pv[4] = {pj.x, pj.y, pj.z, pj.w};
            const uint32_t iv[4] = {ij.x, ij.y, ij.z, ij.w};
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q)
                pos += (j0 + q < top_k && (pv[q] > my_p || (pv[q] == my_p && iv[q] < my_id)))
                           ? 1u : 0u;
        }
        sorted_p[pos] = my_p;
    }
    __syncthreads();
    /* w = p / (left-to-right sum in top-k order); entries past k hold +0 */
    float ws = 0.0f;
    if (e < top_k) chain_lds((const float4 *)sorted_p, 1u, (top_k + 3u) / 4u, ws);
    if (e < top_k) {
        const float wgt = my_p / ws;
        ids_all[(size_t)t * top_k + pos] = my_id;
        weights_all[(size_t)t * top_k + pos] = wgt;
        order_all[(size_t)t * top_k + e] = pos;
        if (!kq_isfinite(wgt) || !kq_isfinite(ws) || !(ws > 0.0f)) kq_flag(status, KQ_DEV_NUMERIC);
    }
    if (live) probs_all[(size_t)t * experts + e] = p;
    if (e == 0u) {
        shared_scale[t] = kq_sigmoid(sl);
        if (!kq_isfinite(s) || !(s > 0.0f)) kq_flag(status, KQ_DEV_NUMERIC);
    }
}

/* One workgroup per token. With sgw given, the token's shared gate logit
 * is first formed here as sgw . x in any order (it only feeds the sigmoid
 * gate, compared by tolerance); thread 0 stores it and reads it back in
 * the body. With stage given, the workgroup also splits the token's row
 * for the Q4_K prefill gate/up pass (kq_stage.h). */
__global__ __launch_bounds__(1024) void route_finish(
    const float *__restrict__ logits_all, float *__restrict__ shared_logit,
    uint32_t experts, uint32_t top_k, float *__restrict__ probs_all, uint32_t *__restrict__ ids_all,
    float *__restrict__ weights_all, uint32_t *__restrict__ order_all,
    float *__restrict__ shared_scale, uint32_t *status, const float *__restrict__ sgw,
    const float *__restrict__ hidden_states, uint32_t hidden, void *stage) {
    if (stage != nullptr) kq::stage_row(hidden_states, blockIdx.x, gridDim.x, hidden, stage, status);
    if (sgw != nullptr) {
        __shared__ float part[16];
        const uint32_t e = threadIdx.x, lane = e & 63u, nw = blockDim.x >> 6;
        const float4 *xq = (const float4 *)(hidden_states + (size_t)blockIdx.x * hidden);
        const float4 *gq = (const float4 *)sgw;
        float acc = 0.0f;
        bool bad = false;
        for (uint32_t q = e; q < hidden / 4u; q += blockDim.x) {
            const float4 gv = gq[q], xv = xq[q];
            bad |= !kq_isfinite(gv.x) || !kq_isfinite(gv.y) || !kq_isfinite(gv.z) ||
                   !kq_isfinite(gv.w);
            acc = fmaf(gv.x, xv.x, acc);
            acc = fmaf(gv.y, xv.y, acc);
            acc = fmaf(gv.z, xv.z, acc);
            acc = fmaf(gv.w, xv.w, acc);
        }
        acc = wave_sum_f32(acc);
        if (lane == 0u) part[e >> 6] = acc;
        __syncthreads();
        if (e == 0u) {
            float sum = 0.0f;
            for (uint32_t i = 0; i < nw; ++i) sum += part[i];
            shared_logit[blockIdx.x] = sum;
        }
        if (bad) kq_flag(status, KQ_DEV_INPUT);
    }
    route_finish_body(blockIdx.x, logits_all, shared_logit, experts, top_k, probs_all, ids_all,
                      weights_all, order_all, shared_scale, status);
}

/*
 * The one-token route in two launches: route_bounds forms the bounds of
 * every logit row, four rows per workgroup; route_select (one workgroup)
 * selects:
 *
 *   1. certified: the top-k by the fp64 sums a when the bounds separate
 *      every adjacent selected pair and the last selected from the rest;
 *   2. refined: otherwise, with L the least a - b of the top-k by a (each
 *      of those k experts has an exact logit >= L, so the k-th largest
 *      exact logit is >= L), every expert not separated from L by its
 *      bound is a contender; the exact left-to-right chains of the
 *      contenders (at most 64) replace their bounds, and the selection is
 *      certified again on them (an expert left out has logit <= a + b,
 *      which is separated from L, hence from the k-th exact logit);
 *   3. exact: otherwise (ties, or non-finite products), the chains of all
 *      rows, then the route finish, as the several-token path does.
 *
 * The certified flag reads 1, 2 or 0 after the call for the three cases.
 */
struct RouteArgs {
    const float *router, *sgw, *x;
    uint32_t experts, top_k;
    double *bound;           /* [E + 1][2] */
    float *logits, *shared_logit, *probs;
    uint32_t *ids, *ids_out; /* ids_out: the caller's copy (may be null) */
    float *weights;
    uint32_t *order;
    float *shared_scale;
    uint32_t *status, *certified;
};

constexpr uint32_t kExQ = 16;    /* float4 of a row per stage of exact_rows */
constexpr uint32_t kExDepth = 4; /* stages each thread has in flight */

/* Exact chains of up to 64 logit rows (ids in rows[], `experts` meaning the
 * shared gate vector) by a workgroup of 1024 threads: stage s takes columns
 * 64s .. 64s + 63 of every row, each thread one float4 of one row; the
 * rounded products w*x (as the CPU forms them) go to LDS, and lane r of
 * wave 0 adds row r's 64 products to its chain, left to right, while the
 * other threads form the next stage. out[r] gets row r's logit. */
template <uint32_t HIDDEN>
__device__ __forceinline__ void exact_rows(const float *__restrict__ router,
                                           const float *__restrict__ sgw,
                                           const float *__restrict__ x, uint32_t experts,
                                           const uint32_t *rows, uint32_t n, float *out,
                                           uint32_t *status) {
    constexpr uint32_t NS = HIDDEN / 64u;
    __shared__ float4 tile[2][64][kExQ + 1u];
    const uint32_t t = threadIdx.x, r = t / kExQ, q = t % kExQ;
    const bool have = r < n;
    const uint32_t e = have ? rows[r] : 0u;
    const float4 *src = (const float4 *)(e < experts ? router + (size_t)e * HIDDEN : sgw);
    const float4 *xs = (const float4 *)x;
    float4 wv[kExDepth], xv[kExDepth];
#pragma unroll
    for (uint32_t d = 0; d < kExDepth; ++d) {
        if (have && d < NS) {
            wv[d] = src[d * kExQ + q];
            xv[d] = xs[d * kExQ + q];
        }
    }
    bool bad = false;
    float acc = 0.0f;
    static_assert(NS % kExDepth == 0u, "stages come in whole rounds of the prefetch depth");
    for (uint32_t s0 = 0; s0 < NS; s0 += kExDepth) {
#pragma unroll
        for (uint32_t d = 0; d < kExDepth; ++d) {
            const uint32_t s = s0 + d;
            if (have) {
                const float4 w = wv[d], xq = xv[d];
                bad |= !kq_isfinite(w.x) || !kq_isfinite(w.y) || !kq_isfinite(w.z) ||
                       !kq_isfinite(w.w);
                float4 p;
                p.x = w.x * xq.x;
                p.y = w.y * xq.y;
                p.z = w.z * xq.z;
                p.w = w.w * xq.w;
                tile[s & 1u][r][q] = p;
                if (s + kExDepth < NS) {
                    wv[d] = src[(s + kExDepth) * kExQ + q];
                    xv[d] = xs[(s + kExDepth) * kExQ + q];
                }
            }
            __syncthreads();
            if (t < n) {
#pragma unroll 4
                for (uint32_t j = 0; j < kExQ; ++j) add4(acc, tile[s & 1u][t][j]);
            }
        }
    }
    if (t < n) out[t] = acc;
    if (bad) kq_flag(status, KQ_DEV_INPUT);
    __syncthreads();
}

/* Exact chains of every logit row (experts rows, then the shared gate
 * vector as row `experts`; experts + 1 <= 1024) by a workgroup of 1024
 * threads, each row's chain on its own lane: stage s forms the rounded
 * products w * x (as the CPU forms them) of columns C s .. C s + C - 1 of
 * every row into LDS (a float4 of up to K rows per thread, the next
 * stage's loads in flight; the activations from an LDS copy), and thread r
 * adds its row's C products to its chain, left to right, one barrier per
 * stage. C = 16 while two stages of rows fit kAllFloats, else 8. The
 * chains of the rows run side by side, so the route costs one row's chain
 * (HIDDEN dependent adds) plus the staging, instead of one per 64 rows.
 * logits[r] (r < experts) and *shared_logit get the results. */
constexpr uint32_t kAllFloats = 2u * 1024u * 9u; /* LDS floats of the stages */

template <uint32_t HIDDEN, uint32_t C>
__device__ __forceinline__ void exact_all_rows_c(const float *__restrict__ router,
                                                 const float *__restrict__ sgw,
                                                 const float *__restrict__ x, uint32_t experts,
                                                 float *stage, const float *xs, float *logits,
                                                 float *shared_logit, uint32_t *status) {
    static_assert(HIDDEN % C == 0u && C % 8u == 0u, "whole stages of float4 pairs");
    constexpr uint32_t NS = HIDDEN / C, P = C + 1u; /* odd pitch: conflict-free chain reads */
    constexpr uint32_t Q = C / 4u;                  /* float4 per row and stage */
    /* thread t stages float4 q = t % Q of rows t / Q + k (1024 / Q), k < K:
     * rows <= 542 at C = 16, <= 1024 at C = 8 */
    constexpr uint32_t RPP = 1024u / Q;
    constexpr uint32_t MAXR = C == 16u ? 542u : 1024u;
    constexpr uint32_t K = (MAXR + RPP - 1u) / RPP;
    const uint32_t t = threadIdx.x, rows = experts + 1u;
    const uint32_t half = (uint32_t)kAllFloats / 2u;
    const uint32_t q = t % Q, r0 = t / Q;
    bool bad = false;
    float4 wv[K];
    auto load = [&](uint32_t s) {
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            const uint32_t r = r0 + k * RPP;
            if (r < rows) {
                const float *row = r < experts ? router + (size_t)r * HIDDEN : sgw;
                wv[k] = *(const float4 *)(row + C * s + 4u * q);
            }
        }
    };
    float acc = 0.0f;
    load(0u);
    for (uint32_t s = 0; s < NS; ++s) {
        float *buf = stage + (s & 1u) * half;
        const float4 xv = *(const float4 *)(xs + C * s + 4u * q);
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            const uint32_t r = r0 + k * RPP;
            if (r < rows) {
                const float4 w = wv[k];
                bad |= !kq_isfinite(w.x) || !kq_isfinite(w.y) || !kq_isfinite(w.z) ||
                       !kq_isfinite(w.w);
                float *d = buf + r * P + 4u * q;
                d[0] = w.x * xv.x;
                d[1] = w.y * xv.y;
                d[2] = w.z * xv.z;
                d[3] = w.w * xv.w;
            }
        }
        if (s + 1u < NS) load(s + 1u);
        __syncthreads();
        if (t < rows) {
            const float *src = buf + t * P;
#pragma unroll
            for (uint32_t j = 0; j < C; ++j) acc = acc + src[j];
        }
    }
    if (t < experts)
        logits[t] = acc;
    else if (t == experts)
        *shared_logit = acc;
    if (bad) kq_flag(status, KQ_DEV_INPUT);
    __syncthreads();
}

template <uint32_t HIDDEN>
__device__ __forceinline__ void exact_all_rows(const float *__restrict__ router,
                                               const float *__restrict__ sgw,
                                               const float *__restrict__ x, uint32_t experts,
                                               float *logits, float *shared_logit,
                                               uint32_t *status) {
    __shared__ float stage[kAllFloats];
    __shared__ __align__(16) float xs[HIDDEN];
    for (uint32_t i = threadIdx.x; i < HIDDEN / 4u; i += blockDim.x)
        reinterpret_cast<float4 *>(xs)[i] = reinterpret_cast<const float4 *>(x)[i];
    __syncthreads();
    if (2u * (experts + 1u) * 17u <= kAllFloats)
        exact_all_rows_c<HIDDEN, 16u>(router, sgw, x, experts, stage, xs, logits, shared_logit,
                                      status);
    else
        exact_all_rows_c<HIDDEN, 8u>(router, sgw, x, experts, stage, xs, logits, shared_logit,
                                     status);
}

/* Ranks (descending value, ascending id) of two entries (m0, i0), (m1, i1)
 * among the first `count` entries of v/id, in eight-entry runs of LDS
 * broadcast reads. Entries past count read as (-inf, max id). */
__device__ __forceinline__ void rank2(const double *v, const uint32_t *id, uint32_t count,
                                      double m0, uint32_t i0, double m1, uint32_t i1,
                                      uint32_t &r0, uint32_t &r1) {
    r0 = 0u;
    r1 = 0u;
    for (uint32_t j0 = 0; j0 < count; j0 += 8u) {
        double o[8];
        uint32_t oi[8];
#pragma unroll
        for (uint32_t q = 0; q < 8u; ++q) {
            const bool in = j0 + q < count;
            o[q] = in ? v[j0 + q] : -__builtin_inf();
            oi[q] = in ? id[j0 + q] : 0xffffffffu;
        }
#pragma unroll
        for (uint32_t q = 0; q < 8u; ++q) {
            r0 += (uint32_t)(o[q] > m0) | ((uint32_t)(o[q] == m0) & (uint32_t)(oi[q] < i0));
            r1 += (uint32_t)(o[q] > m1) | ((uint32_t)(o[q] == m1) & (uint32_t)(oi[q] < i1));
        }
    }
}

/* Writes the selection: sorted ids/values in srt_v/srt_id (descending), the
 * weights p / sum of the selected p with p = exp(v - v_0) (the softmax
 * denominator cancels; the hardware exponential, compared by tolerance
 * like the layer output), and the ascending-id rank of each slot. Wave 0. */
__device__ __forceinline__ void write_selection(const RouteArgs &a, const double *srt_v,
                                                const uint32_t *srt_id) {
    const uint32_t lane = threadIdx.x & 63u, k = a.top_k;
    const double m = srt_v[0];
    const uint32_t my_id = lane < k ? srt_id[lane] : 0xffffffffu;
    const float ex = lane < k ? fast_expf((float)(srt_v[lane < k ? lane : 0] - m)) : 0.0f;
    const float psel = wave_sum_f32(ex);
    /* the slot's place in ascending id order, from the other lanes' ids
     * (register reads, not an LDS round trip per slot) */
    uint32_t rk = 0;
    for (uint32_t j = 0; j < k; ++j)
        rk += (uint32_t)((uint32_t)__builtin_amdgcn_readlane((int)my_id, (int)j) < my_id);
    if (lane < k) {
        a.ids[lane] = my_id;
        if (a.ids_out) a.ids_out[lane] = my_id;
        a.weights[lane] = ex / psel;
        a.order[rk] = lane;
    }
}

/* Adjacent selected pairs, and the last selected against `rest` (the
 * largest upper value outside the selection, -inf if none), separated. */
__device__ __forceinline__ bool separated(const double *srt_v, const double *srt_b, uint32_t k,
                                          double rest) {
    const uint32_t lane = threadIdx.x & 63u;
    const double m = srt_v[0];
    const uint32_t l1 = lane + 1u < k ? lane + 1u : 0u;
    const bool pair_ok =
        lane + 1u >= k || certify_sep(srt_v[lane < k ? lane : 0], srt_b[lane < k ? lane : 0],
                                      srt_v[l1], srt_b[l1], m);
    bool ok = __ballot(!pair_ok) == 0ull;
    if (ok && rest > -__builtin_inf())
        ok = certify_sep(srt_v[k - 1u], srt_b[k - 1u], rest, 0.0, m);
    return ok;
}

template <uint32_t HIDDEN>
__device__ __forceinline__ void select_one(const RouteArgs &a) {
    __shared__ double cv[kCertCand], cb[kCertCand], sv[kCertCand], sb[kCertCand];
    __shared__ uint32_t cid[kCertCand], sid[kCertCand];
    __shared__ __align__(16) float w_key[16];
    __shared__ __align__(16) double w_rest[16];
    __shared__ __align__(16) uint32_t w_bad[16];
    __shared__ uint32_t s_count, s_cn, s_state;
    __shared__ double s_lw, s_m;
    __shared__ float ex_l[64];
    const uint32_t experts = a.experts, top_k = a.top_k;
    const uint32_t e = threadIdx.x, lane = e & 63u;
    const uint32_t w = __builtin_amdgcn_readfirstlane(e >> 6);
    const double ninf = -__builtin_inf();
    const bool live = e < experts;
    if (w == 15u && lane == 0u) {
        /* the shared gate from the fp64 sum; the exact route overwrites it */
        const double sh_a = a.bound[2u * experts];
        *a.shared_scale = 1.0f / (1.0f + fast_expf(-(float)sh_a));
    }
    const double sh_b = a.bound[2u * experts + 1u];
    const double ar = live ? a.bound[2u * e] : ninf;
    const double b = live ? a.bound[2u * e + 1u] : 0.0;
    const double av = ar == ar ? ar : ninf; /* a NaN total has an infinite bound */
    const float key = (float)av;
    const uint32_t need = top_k + 1u < experts ? top_k + 1u : experts;
    const uint32_t ns = experts >= 64u ? experts / 64u : 1u;
    const uint32_t per = (need + ns - 1u) / ns;
    if (e == 0u) {
        s_count = 0u;
        s_cn = 0u;
    }
    /* candidates: each full wave's per-th largest key, t the least of them;
     * every expert with key >= t is listed, the others' a + b maximised */
    {
        float m = __builtin_inff();
        if (w < ns) {
            float v = key;
            for (uint32_t r = 0; r < per; ++r) {
                m = wave_max(v);
                const uint64_t hit = __ballot(v == m);
                if (lane == (uint32_t)__builtin_ctzll(hit)) v = -__builtin_inff();
            }
        }
        if (lane == 0u) w_key[w] = m;
    }
    __syncthreads();
    float t = w_key[0];
#pragma unroll
    for (uint32_t k = 1; k < 16u; ++k) t = fminf(t, w_key[k]);
    {
        const bool c = live && key >= t;
        const uint64_t cbm = __ballot(c);
        uint32_t at = 0;
        if (lane == 0u) at = atomicAdd(&s_count, (uint32_t)__popcll(cbm));
        at = __builtin_amdgcn_readfirstlane(at) + bits_below(cbm);
        if (c && at < kCertCand) {
            cv[at] = av;
            cb[at] = b;
            cid[at] = e;
        }
        const double rest_w = kq_wave_max_f64(live && !c ? av + b : ninf);
        const bool bad_w = __ballot(live && !(b < __builtin_inf())) != 0ull;
        if (lane == 0u) {
            w_rest[w] = rest_w;
            w_bad[w] = bad_w ? 1u : 0u;
        }
    }
    __syncthreads();
    const uint32_t total = s_count;
    if (total <= kCertCand) {
        /* every thread: candidate c = e / 8 against candidates e % 8,
         * e % 8 + 8, ... (descending a, ascending id); the eight partial
         * counts of lanes 8c .. 8c + 7 summed give its rank, and lane 8c
         * places it. A lone wave ranking all of them paid an LDS round
         * trip per eight candidates. */
        const uint32_t c = e >> 3, sl = e & 7u;
        uint32_t r = 0u;
        double mc = 0.0;
        uint32_t ic = 0u;
        if (c < total) {
            mc = cv[c];
            ic = cid[c];
            for (uint32_t j = sl; j < total; j += 8u) {
                const double o = cv[j];
                const uint32_t oi = cid[j];
                r += (uint32_t)(o > mc) | ((uint32_t)(o == mc) & (uint32_t)(oi < ic));
            }
        }
        r += __shfl_xor(r, 1, 64);
        r += __shfl_xor(r, 2, 64);
        r += __shfl_xor(r, 4, 64);
        if (c < total && sl == 0u) {
            sv[r] = mc;
            sb[r] = cb[c];
            sid[r] = ic;
        }
    }
    __syncthreads();
    if (w == 0u) {
        double rest = w_rest[0];
        uint32_t anybad = w_bad[0];
#pragma unroll
        for (uint32_t k = 1; k < 16u; ++k) {
            rest = fmax(rest, w_rest[k]);
            anybad |= w_bad[k];
        }
        uint32_t state = 3u;
        if (anybad == 0u && total <= kCertCand && sh_b < __builtin_inf()) {
            /* the candidates ranked k and after join the rest */
            const uint32_t j1 = lane + 64u;
            const double o0 = lane >= top_k && lane < total ? sv[lane] + sb[lane] : ninf;
            const double o1 = j1 >= top_k && j1 < total ? sv[j1] + sb[j1] : ninf;
            rest = fmax(rest, kq_wave_max_f64(fmax(o0, o1)));
            if (separated(sv, sb, top_k, rest)) {
                write_selection(a, sv, sid);
                state = 1u;
            } else {
                /* L: the least a - b of the top-k by a */
                const double lo = lane < top_k ? sv[lane] - sb[lane] : __builtin_inf();
                const double lw = -kq_wave_max_f64(-lo);
                if (lane == 0u) {
                    s_lw = lw;
                    s_m = sv[0];
                }
                state = 0u;
            }
        }
        if (lane == 0u) s_state = state;
    }
    __syncthreads();
    uint32_t state = s_state;
    if (state == 0u) {
        /* contenders: not separated from L by their bounds */
        const bool inc = live && !certify_sep(s_lw, 0.0, av, b, s_m);
        const uint64_t im = __ballot(inc);
        uint32_t at = 0;
        if (lane == 0u && im) at = atomicAdd(&s_cn, (uint32_t)__popcll(im));
        at = __builtin_amdgcn_readfirstlane(at) + bits_below(im);
        if (inc && at < 64u) cid[at] = e;
        __syncthreads();
        const uint32_t n = s_cn;
        if (n > 64u || n < top_k) {
            state = 3u;
        } else {
            exact_rows<HIDDEN>(a.router, a.sgw, a.x, experts, cid, n, ex_l, a.status);
            if (w == 0u) {
                const bool have = lane < n;
                const double mine = have ? (double)ex_l[lane] : ninf;
                const uint32_t my_id = have ? cid[lane] : 0xffffffffu;
                for (uint32_t j = lane; j < n; j += 64u) cv[j] = (double)ex_l[j];
                uint32_t rank, unused;
                rank2(cv, cid, n, mine, my_id, ninf, 0xffffffffu, rank, unused);
                rank = have ? rank : lane;
                sv[rank] = mine;
                sb[rank] = 0.0;
                sid[rank] = my_id;
                const bool fin = __ballot(have && !kq_isfinite(ex_l[lane])) == 0ull;
                const double rest = n > top_k ? sv[top_k] : ninf;
                uint32_t st = 3u;
                if (fin && separated(sv, sb, top_k, rest)) {
                    write_selection(a, sv, sid);
                    st = 2u;
                }
                if (lane == 0u) s_state = st;
            }
            __syncthreads();
            state = s_state;
        }
    }
    if (state == 3u) {
        /* every row's chain, all rows side by side, then the route finish */
        exact_all_rows<HIDDEN>(a.router, a.sgw, a.x, experts, a.logits, a.shared_logit,
                               a.status);
        route_finish_body(0u, a.logits, a.shared_logit, experts, top_k, a.probs, a.ids,
                          a.weights, a.order, a.shared_scale, a.status);
        __syncthreads();
        if (a.ids_out && e < top_k) a.ids_out[e] = a.ids[e];
    }
    if (e == 0u) *a.certified = state == 1u ? 1u : (state == 2u ? 2u : 0u);
}

template <uint32_t HIDDEN>
__global__ __launch_bounds__(64 * kSelRows * kSelParts) void route_bounds(RouteArgs a) {
    bounds_rows<HIDDEN>(a.router, a.sgw, a.x, a.experts, a.bound);
}

/* one workgroup: the bounds are another launch's stores, so they are read
 * here without any fence (a cross-workgroup hand-off inside one launch
 * would need an agent-scope release per workgroup, a write-back of its L2) */
template <uint32_t HIDDEN>
__global__ __launch_bounds__(1024) void route_select(RouteArgs a) {
    select_one<HIDDEN>(a);
}

/* ---------------------- expert gate/up + SwiGLU ---------------------- */
/* Rows longer than one wave covers (or of a width the row engine has no
 * instance for) are cut into column segments, widest first, one launch
 * each: the first segment writes its partial gate/up dots to `part`, later
 * ones add theirs, and the last applies SwiGLU. A shared expert whose type
 * differs from the routed one runs as its own launch of the same kernel.
 *
 * Arguments common to every segment launch of one call. */
struct GateupArgs {
    const uint8_t *gate, *up, *sgate, *sup; /* routed stacks, shared matrices */
    const float *x;                         /* hidden states [tokens][hidden] */
    const uint32_t *ids;
    uint32_t top_k, inter, shared_inter, hidden;
    uint32_t rstride, srstride; /* full row bytes, routed and shared */
    uint32_t act_stride;
    float *act;   /* [tokens][top_k + 1][act_stride] */
    float *part;  /* [tokens][top_k + 1][2][act_stride] partial dots */
    uint32_t *status;
};

enum : uint32_t { kSegFirst = 1u, kSegLast = 2u };

/* Gate/up + SwiGLU rows of one slot (matrices G and U: `rows` rows of
 * `stride` bytes, columns [col0, col0 + COLS)) for one token, by wave
 * `wave` of the `nwaves` working on the slot, in workgroups of NT threads.
 * The caller has requested the token's activations into `stage` (issue());
 * here every wave requests its first gate and up rows without a branch,
 * then the activations are checked and written to the workgroup's LDS
 * image behind an LDS-only barrier while the weights are in flight, and
 * the check is flagged at the end. */
template <uint32_t TYPE, uint32_t COLS, int RT, int NT>
struct GateupEngine {
    using R = kq::Rows<TYPE, COLS, 1, RT, typename kq::MatvecLane<TYPE, 1>::T>;
    using Raw = typename R::Raw;
    using XS = kq::StageFor<R, 1, NT>;
    static constexpr uint32_t kImage = XS::NP; /* float4 words of the LDS image */

    __device__ static __forceinline__ void run(const GateupArgs &a, const XS &stage, float4 *xs,
                                               uint32_t slot, uint32_t t, const uint8_t *G,
                                               const uint8_t *U, uint32_t rows, uint32_t stride,
                                               uint32_t wave, uint32_t nwaves, uint32_t col0,
                                               uint32_t seg) {
        const uint32_t boff = kq::row_bytes<TYPE>(col0);
        const uint32_t lane = threadIdx.x & 63u;
        const uint32_t sub = lane / R::LPR, l = lane % R::LPR;
        const uint32_t ngroups = (rows + R::GROUP - 1u) / R::GROUP;
        typename R::Lane ln;
        ln.setup(l);
        Raw rg[RT], ru[RT];
        uint32_t g = wave;
        const uint32_t wbytes = rows * stride - boff;
        const KqBuf gb = kq_buf(G + boff, wbytes), ub = kq_buf(U + boff, wbytes);
        R::load_group_oob(ln, gb, g, rows, sub, rg, stride, wbytes + 64u);
        R::load_group_oob(ln, ub, g, rows, sub, ru, stride, wbytes + 64u);
        const bool xbad = stage.commit(xs, threadIdx.x);
        kq_lds_barrier();
        stage.load(ln, xs, l);
        bool bad = false, malformed = false;
        const size_t at = (size_t)t * (a.top_k + 1u) + slot;
        float *out = a.act + at * a.act_stride;
        float *pg = a.part + at * 2u * a.act_stride, *pu = pg + a.act_stride;
        for (; g < ngroups; g += nwaves) {
            if (g != wave) {
                R::load_group(ln, gb, g, rows, sub, rg, stride);
                R::load_group(ln, ub, g, rows, sub, ru, stride);
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
                        float gv = vg[j], uv = vu[j];
                        if (!(seg & kSegFirst)) {
                            gv = pg[row] + gv;
                            uv = pu[row] + uv;
                        }
                        if (seg & kSegLast) {
                            const float r = kq_swiglu(gv, uv);
                            bad |= !kq_isfinite(gv) || !kq_isfinite(uv) || !kq_isfinite(r);
                            out[row] = r;
                        } else {
                            pg[row] = gv;
                            pu[row] = uv;
                        }
                    }
                }
            }
        }
        if (xbad) kq_flag(a.status, KQ_DEV_INPUT);
        if (malformed) kq_flag(a.status, KQ_DEV_MALFORMED);
        if (bad) kq_flag(a.status, KQ_DEV_NUMERIC);
    }
};

/* grid: x = row groups, y = slot - slot0 (slots 0..K-1 routed by top-k
 * position, K the shared expert), z = token. This launch covers columns
 * [col0, col0 + COLS) of every row. The activations are requested before
 * the routed expert's id is read. */
template <uint32_t TYPE, uint32_t COLS, int RT>
__global__ __launch_bounds__(kThreads) void expert_gateup(GateupArgs a, uint32_t slot0,
                                                          uint32_t col0, uint32_t seg) {
    using E = GateupEngine<TYPE, COLS, RT, kThreads>;
    __shared__ __align__(16) float4 xs[E::kImage];
    const uint32_t slot = blockIdx.y + slot0, t = blockIdx.z;
    typename E::XS stage;
    stage.issue(a.x + (size_t)t * a.hidden + col0, COLS, threadIdx.x);
    const bool shared = slot == a.top_k;
    const uint32_t rows = shared ? a.shared_inter : a.inter;
    const uint32_t stride = shared ? a.srstride : a.rstride;
    const uint8_t *G, *U;
    if (shared) {
        G = a.sgate;
        U = a.sup;
    } else {
        const uint32_t e = a.ids[(size_t)t * a.top_k + slot];
        G = a.gate + (size_t)e * a.inter * stride;
        U = a.up + (size_t)e * a.inter * stride;
    }
    const uint32_t wave =
        __builtin_amdgcn_readfirstlane((blockIdx.x * kThreads + threadIdx.x) >> 6);
    const uint32_t nwaves = (gridDim.x * kThreads) >> 6;
    E::run(a, stage, xs, slot, t, G, U, rows, stride, wave, nwaves, col0, seg);
}

/* -------------------------- down + combine -------------------------- */
/* grid: x = groups of R::GROUP output rows, y = token; the launch covers
 * slots [slot0, slot1) (0..K-1 routed by top-k position, K the shared
 * expert), one wave per slot and further slots in steps of the wave count,
 * and columns [col0, col0 + COLS) of the rows. Each wave reduces its slot's
 * rows Wd[f] . act[t][slot] into LDS. Segments other than the last, and a
 * launch that only computes the shared expert, store the sums in
 * part[t][slot][row] (later segments add to them); the last segment of the
 * routed launch forms the combine in the CPU's order:
 *   routed_sum = 0; for slots in ascending expert id: routed_sum += o * w;
 *   out = routed_sum + o_shared * sigmoid(shared logit),
 * taking o_shared from part[t][K] when another launch computed it. */
constexpr uint32_t kMaxSlots = 65;

constexpr uint32_t kDownWaves = 12;

struct DownArgs {
    const uint8_t *down, *sdown;
    const float *act;
    const uint32_t *ids, *order;
    const float *weights, *shared_scale;
    uint32_t top_k, hidden, rstride, srstride, act_stride;
    float *part; /* [tokens][top_k + 1][hidden] */
    float *out;
    uint32_t *status;
};

enum : uint32_t { kSegCombine = 4u };

template <uint32_t TYPE, uint32_t COLS, int RT>
__global__ __launch_bounds__(64 * kDownWaves) void expert_down_combine(
    DownArgs a, uint32_t slot0, uint32_t slot1, uint32_t col0, uint32_t seg) {
    using R = kq::Rows<TYPE, COLS, 1, RT>;
    using Raw = typename R::Raw;
    __shared__ float res[kMaxSlots][R::GROUP];
    __shared__ uint32_t ord_s[64];
    __shared__ float w_s[64];
    const uint32_t g = blockIdx.x, t = blockIdx.y;
    const uint32_t lane = threadIdx.x & 63u, nwv = blockDim.x >> 6;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t sub = lane / R::LPR, l = lane % R::LPR;
    const uint32_t top_k = a.top_k, nslots = top_k + 1u, hidden = a.hidden;
    const uint32_t boff = kq::row_bytes<TYPE>(col0);
    const bool combine = (seg & kSegCombine) != 0u;
    if (combine && threadIdx.x < top_k) {
        const uint32_t s = a.order[(size_t)t * top_k + threadIdx.x];
        ord_s[threadIdx.x] = s;
        w_s[threadIdx.x] = a.weights[(size_t)t * top_k + s];
    }
    typename R::Lane ln;
    ln.setup(l);
    auto matrix = [&](uint32_t slot) {
        if (slot == top_k) return kq_buf(a.sdown + boff, hidden * a.srstride - boff);
        const uint8_t *D = a.down + (size_t)a.ids[(size_t)t * top_k + slot] * hidden * a.rstride;
        return kq_buf(D + boff, hidden * a.rstride - boff);
    };
    auto stride_of = [&](uint32_t slot) { return slot == top_k ? a.srstride : a.rstride; };
    auto act_of = [&](uint32_t slot) {
        return a.act + ((size_t)t * nslots + slot) * a.act_stride + col0;
    };
    bool bad = false, malformed = false;
    Raw ra[RT], rb[RT];
    uint32_t slot = slot0 + wv;
    if (slot < slot1) R::load_group(ln, matrix(slot), g, hidden, sub, ra, stride_of(slot));
    auto reduce = [&](const Raw (&raw)[RT], uint32_t sl) {
        float v[R::N];
        R::dot_group(ln, raw, l, v, malformed);
#pragma unroll
        for (int j = 0; j < R::KEEP; ++j) {
            const int idx = R::value_index(l, j);
            if (idx >= 0) res[sl][(uint32_t)idx * R::RPW + sub] = v[j];
        }
    };
    /* ping-pong over this wave's slots: the next slot's rows are requested
     * before this slot's activations */
    while (slot < slot1) {
        uint32_t next = slot + nwv;
        if (next < slot1) R::load_group(ln, matrix(next), g, hidden, sub, rb, stride_of(next));
        bad |= ln.load_x(act_of(slot), COLS);
        reduce(ra, slot);
        slot = next;
        if (slot >= slot1) break;
        next = slot + nwv;
        if (next < slot1) R::load_group(ln, matrix(next), g, hidden, sub, ra, stride_of(next));
        bad |= ln.load_x(act_of(slot), COLS);
        reduce(rb, slot);
        slot = next;
    }
    __syncthreads();
    /* one thread per output row of the group (a group may have more rows
     * than the launch has threads) */
    for (uint32_t i = threadIdx.x; i < R::GROUP; i += blockDim.x) {
        const uint32_t row = g * R::GROUP + i;
        if (row >= hidden) break;
        float *prow = a.part + (size_t)t * nslots * hidden + row;
        if (!(seg & kSegFirst)) {
            for (uint32_t s = slot0; s < slot1; ++s)
                res[s][i] = prow[(size_t)s * hidden] + res[s][i];
        }
        if (!combine) {
            for (uint32_t s = slot0; s < slot1; ++s) prow[(size_t)s * hidden] = res[s][i];
            continue;
        }
        float sum = 0.0f;
        for (uint32_t j = 0; j < top_k; ++j) {
            const uint32_t s = ord_s[j];
            const float o = res[s][i];
            bad |= !kq_isfinite(o);
            const float weighted = o * w_s[j];
            sum = sum + weighted;
        }
        const float so = slot1 > top_k ? res[top_k][i] : prow[(size_t)top_k * hidden];
        const float gated = so * a.shared_scale[t];
        const float v = sum + gated;
        bad |= !kq_isfinite(so) || !kq_isfinite(sum) || !kq_isfinite(gated) || !kq_isfinite(v);
        a.out[(size_t)t * hidden + row] = v;
    }
    if (malformed) kq_flag(a.status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(a.status, KQ_DEV_NUMERIC);
}

/* ------------------- one launch per role: fused segments ------------------- */
/* Rows of up to two column segments (C0 columns, then C1 from column C0;
 * C1 = 0 for one) and a shared expert of its own format in one launch per
 * role: each segment's engine forms its partial dots of the workgroup's
 * rows into LDS, the segments' sums are added there (first segment, then
 * second, as the segment launches add them), and the workgroup finishes
 * the rows. kFuseRows rows per workgroup; a segment's engine takes row
 * groups of at most that many rows. */
constexpr uint32_t kFuseRows = 16;

/* passes of RT rows: two while that keeps four groups per workgroup */
template <uint32_t T, uint32_t C>
constexpr int fuse_rt() {
    return (kFuseRows / (64u / kq::lanes_per_row<T>(C))) >= 8u ? 2 : 1;
}

/* one segment's dots of rows row0 .. row0 + kFuseRows - 1 of matrices M[m]
 * (NM of them) against x (the segment's own columns), into dst[m][row -
 * row0] (added when !first) */
template <uint32_t T, uint32_t C, int NM>
__device__ __forceinline__ void fuse_segment(const uint8_t *const (&M)[NM], uint32_t stride,
                                             uint32_t col0, uint32_t rows, uint32_t row0,
                                             const float *x, float (*dst)[kFuseRows],
                                             bool first, uint32_t wave, uint32_t nwaves,
                                             bool &badx, bool &malformed) {
    constexpr int RT = fuse_rt<T, C>();
    using R = kq::Rows<T, C, 1, RT>;
    using Raw = typename R::Raw;
    static_assert(R::GROUP <= kFuseRows && kFuseRows % R::GROUP == 0u, "groups tile the rows");
    constexpr uint32_t NG = kFuseRows / R::GROUP;
    if (wave >= NG) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t sub = lane / R::LPR, l = lane % R::LPR;
    typename R::Lane ln;
    ln.setup(l);
    const uint32_t boff = kq::row_bytes<T>(col0);
    const uint32_t wbytes = rows * stride - boff;
    KqBuf wb[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) wb[m] = kq_buf(M[m] + boff, wbytes);
    const uint32_t gbase = row0 / R::GROUP;
    Raw ra[NM][RT], rb[NM][RT];
#pragma unroll
    for (int m = 0; m < NM; ++m) R::load_group(ln, wb[m], gbase + wave, rows, sub, ra[m], stride);
    badx |= ln.load_x(kq::XGlobal{x, 0u});
    auto finish = [&](const Raw (&raw)[NM][RT], uint32_t gi) {
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            float v[R::N];
            R::dot_group(ln, raw[m], l, v, malformed);
#pragma unroll
            for (int j = 0; j < R::KEEP; ++j) {
                const int idx = R::value_index(l, j);
                if (idx >= 0) {
                    const uint32_t r = gi * R::GROUP + (uint32_t)idx * R::RPW + sub;
                    dst[m][r] = first ? v[j] : dst[m][r] + v[j];
                }
            }
        }
    };
    /* ping-pong over this wave's groups */
    uint32_t gi = wave;
    while (gi < NG) {
        uint32_t gn = gi + nwaves;
        if (gn < NG) {
#pragma unroll
            for (int m = 0; m < NM; ++m) R::load_group(ln, wb[m], gbase + gn, rows, sub, rb[m], stride);
        }
        finish(ra, gi);
        gi = gn;
        if (gi >= NG) break;
        gn = gi + nwaves;
        if (gn < NG) {
#pragma unroll
            for (int m = 0; m < NM; ++m) R::load_group(ln, wb[m], gbase + gn, rows, sub, ra[m], stride);
        }
        finish(rb, gi);
        gi = gn;
    }
}

/* grid: x = groups of kFuseRows rows, y = slot (0..K-1 routed by top-k
 * position, K the shared expert), z = token; 4 waves */
template <uint32_t TR, uint32_t TS, uint32_t C0, uint32_t C1>
__global__ __launch_bounds__(kThreads) void expert_gateup_fused(GateupArgs a) {
    __shared__ float part[2][kFuseRows];
    const uint32_t slot = blockIdx.y, t = blockIdx.z;
    const bool shared = slot == a.top_k;
    const uint32_t rows = shared ? a.shared_inter : a.inter;
    const uint32_t row0 = blockIdx.x * kFuseRows;
    if (row0 >= rows) return;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nwaves = kThreads / 64u;
    const float *x = a.x + (size_t)t * a.hidden;
    bool badx = false, malformed = false, bad = false;
    auto run = [&](auto tag) {
        constexpr uint32_t T = decltype(tag)::value;
        const uint32_t stride = shared ? a.srstride : a.rstride;
        const uint8_t *G, *U;
        if (shared) {
            G = a.sgate;
            U = a.sup;
        } else {
            const uint32_t e = a.ids[(size_t)t * a.top_k + slot];
            G = a.gate + (size_t)e * a.inter * stride;
            U = a.up + (size_t)e * a.inter * stride;
        }
        const uint8_t *const M[2] = {G, U};
        fuse_segment<T, C0, 2>(M, stride, 0u, rows, row0, x, part, true, wave, nwaves, badx,
                               malformed);
        if constexpr (C1 != 0u) {
            __syncthreads();
            fuse_segment<T, C1, 2>(M, stride, C0, rows, row0, x + C0, part, false, wave, nwaves,
                                   badx, malformed);
        }
    };
    if (shared)
        run(std::integral_constant<uint32_t, TS>{});
    else
        run(std::integral_constant<uint32_t, TR>{});
    __syncthreads();
    if (threadIdx.x < kFuseRows && row0 + threadIdx.x < rows) {
        const float gv = part[0][threadIdx.x], uv = part[1][threadIdx.x];
        const float r = kq_swiglu(gv, uv);
        bad |= !kq_isfinite(gv) || !kq_isfinite(uv) || !kq_isfinite(r);
        a.act[((size_t)t * (a.top_k + 1u) + slot) * a.act_stride + row0 + threadIdx.x] = r;
    }
    if (badx) kq_flag(a.status, KQ_DEV_INPUT);
    if (malformed) kq_flag(a.status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(a.status, KQ_DEV_NUMERIC);
}

/* down and the ordered combine: grid x = groups of kFuseRows output rows,
 * y = token; one wave per slot (K + 1 <= 16), each forming its slot's rows
 * into LDS over both segments */
template <uint32_t TR, uint32_t TS, uint32_t C0, uint32_t C1>
__global__ __launch_bounds__(1024) void expert_down_fused(DownArgs a) {
    __shared__ float res[16][kFuseRows];
    __shared__ uint32_t ord_s[16];
    __shared__ float w_s[16];
    const uint32_t t = blockIdx.y, row0 = blockIdx.x * kFuseRows;
    const uint32_t top_k = a.top_k, nslots = top_k + 1u, hidden = a.hidden;
    const uint32_t slot = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (threadIdx.x < top_k) {
        const uint32_t s = a.order[(size_t)t * top_k + threadIdx.x];
        ord_s[threadIdx.x] = s;
        w_s[threadIdx.x] = a.weights[(size_t)t * top_k + s];
    }
    bool badx = false, malformed = false, bad = false;
    if (slot < nslots) {
        const bool shared = slot == top_k;
        const float *act = a.act + ((size_t)t * nslots + slot) * a.act_stride;
        float(*dst)[kFuseRows] = &res[slot];
        auto run = [&](auto tag) {
            constexpr uint32_t T = decltype(tag)::value;
            const uint32_t stride = shared ? a.srstride : a.rstride;
            const uint8_t *D =
                shared ? a.sdown
                       : a.down + (size_t)a.ids[(size_t)t * top_k + slot] * hidden * stride;
            const uint8_t *const M[1] = {D};
            /* one wave per slot: it owns every row of its slot, so its two
             * segments need no barrier between them */
            fuse_segment<T, C0, 1>(M, stride, 0u, hidden, row0, act, dst, true, 0u, 1u, badx,
                                   malformed);
            if constexpr (C1 != 0u)
                fuse_segment<T, C1, 1>(M, stride, C0, hidden, row0, act + C0, dst, false, 0u, 1u,
                                       badx, malformed);
        };
        if (shared)
            run(std::integral_constant<uint32_t, TS>{});
        else
            run(std::integral_constant<uint32_t, TR>{});
    }
    __syncthreads();
    if (threadIdx.x < kFuseRows && row0 + threadIdx.x < hidden) {
        const uint32_t i = threadIdx.x;
        float sum = 0.0f;
        for (uint32_t j = 0; j < top_k; ++j) {
            const float o = res[ord_s[j]][i];
            bad |= !kq_isfinite(o);
            const float weighted = o * w_s[j];
            sum = sum + weighted;
        }
        const float so = res[top_k][i];
        const float gated = so * a.shared_scale[t];
        const float v = sum + gated;
        bad |= !kq_isfinite(so) || !kq_isfinite(sum) || !kq_isfinite(gated) || !kq_isfinite(v);
        a.out[(size_t)t * hidden + row0 + i] = v;
    }
    /* a non-finite activation is the layer's own intermediate */
    if (badx || bad) kq_flag(a.status, KQ_DEV_NUMERIC);
    if (malformed) kq_flag(a.status, KQ_DEV_MALFORMED);
}

template <uint32_t TYPE, uint32_t COLS>
hipError_t launch_gateup(const GateupArgs &a, uint32_t tokens, uint32_t slot0, uint32_t nslot,
                         uint32_t col0, uint32_t seg, hipStream_t s) {
    constexpr int RT = 2;
    const uint32_t both = a.inter > a.shared_inter ? a.inter : a.shared_inter;
    const uint32_t rows = slot0 == a.top_k ? a.shared_inter
                          : slot0 + nslot > a.top_k ? both : a.inter;
    const uint32_t rows_per_wave = kq::Rows<TYPE, COLS, 1, RT>::GROUP;
    const uint32_t waves = (rows + rows_per_wave - 1u) / rows_per_wave;
    const uint32_t blocks = (waves + 3u) / 4u;
    hipLaunchKernelGGL((expert_gateup<TYPE, COLS, RT>), dim3(blocks, nslot, tokens),
                       dim3(kThreads), 0, s, a, slot0, col0, seg);
    return hipGetLastError();
}

template <uint32_t TYPE, uint32_t COLS>
hipError_t launch_down(const DownArgs &a, uint32_t tokens, uint32_t slot0, uint32_t slot1,
                       uint32_t col0, uint32_t seg, hipStream_t s) {
    constexpr int RT = 2;
    const uint32_t group = kq::Rows<TYPE, COLS, 1, RT>::GROUP;
    const uint32_t blocks = (a.hidden + group - 1u) / group;
    uint32_t waves = slot1 - slot0;
    if (waves > kDownWaves) waves = kDownWaves;
    hipLaunchKernelGGL((expert_down_combine<TYPE, COLS, RT>), dim3(blocks, tokens),
                       dim3(64u * waves), 0, s, a, slot0, slot1, col0, seg);
    return hipGetLastError();
}

/* Column segment widths with an engine instance, widest first; the 32-weight
 * formats also take 128, 64 and 32. */
constexpr uint32_t kSegWidths[] = {2048u, 1024u, 512u, 256u, 128u, 64u, 32u};

bool small_type(uint32_t t) {
    return t == KQ_LAUNCH_Q8_0 || t == KQ_LAUNCH_Q5_1 || t == KQ_LAUNCH_IQ4_NL;
}

/* Cuts cols into segment widths usable by every type given (0 = none);
 * returns the count, or 0 when cols cannot be cut so. */
uint32_t segments(uint32_t cols, uint32_t t0, uint32_t t1, uint32_t (&w)[16]) {
    const uint32_t min = small_type(t0) && small_type(t1) ? 32u : 256u;
    uint32_t n = 0, left = cols;
    for (uint32_t k = 0; k < sizeof(kSegWidths) / sizeof(kSegWidths[0]) && left; ++k) {
        if (kSegWidths[k] < min) break;
        while (left >= kSegWidths[k] && n < 16u) {
            w[n++] = kSegWidths[k];
            left -= kSegWidths[k];
        }
    }
    return left == 0u && cols != 0u ? n : 0u;
}

template <uint32_t TYPE>
hipError_t gateup_width(uint32_t width, const GateupArgs &a, uint32_t tokens, uint32_t slot0,
                        uint32_t nslot, uint32_t col0, uint32_t seg, hipStream_t s) {
    switch (width) {
    case 2048: return launch_gateup<TYPE, 2048u>(a, tokens, slot0, nslot, col0, seg, s);
    case 1024: return launch_gateup<TYPE, 1024u>(a, tokens, slot0, nslot, col0, seg, s);
    case 512: return launch_gateup<TYPE, 512u>(a, tokens, slot0, nslot, col0, seg, s);
    case 256: return launch_gateup<TYPE, 256u>(a, tokens, slot0, nslot, col0, seg, s);
    default: break;
    }
    if constexpr (kq::small_block<TYPE>()) {
        switch (width) {
        case 128: return launch_gateup<TYPE, 128u>(a, tokens, slot0, nslot, col0, seg, s);
        case 64: return launch_gateup<TYPE, 64u>(a, tokens, slot0, nslot, col0, seg, s);
        case 32: return launch_gateup<TYPE, 32u>(a, tokens, slot0, nslot, col0, seg, s);
        default: break;
        }
    }
    return hipErrorInvalidValue;
}

template <uint32_t TYPE>
hipError_t down_width(uint32_t width, const DownArgs &a, uint32_t tokens, uint32_t slot0,
                      uint32_t slot1, uint32_t col0, uint32_t seg, hipStream_t s) {
    switch (width) {
    case 2048: return launch_down<TYPE, 2048u>(a, tokens, slot0, slot1, col0, seg, s);
    case 1024: return launch_down<TYPE, 1024u>(a, tokens, slot0, slot1, col0, seg, s);
    case 512: return launch_down<TYPE, 512u>(a, tokens, slot0, slot1, col0, seg, s);
    case 256: return launch_down<TYPE, 256u>(a, tokens, slot0, slot1, col0, seg, s);
    default: break;
    }
    if constexpr (kq::small_block<TYPE>()) {
        switch (width) {
        case 128: return launch_down<TYPE, 128u>(a, tokens, slot0, slot1, col0, seg, s);
        case 64: return launch_down<TYPE, 64u>(a, tokens, slot0, slot1, col0, seg, s);
        case 32: return launch_down<TYPE, 32u>(a, tokens, slot0, slot1, col0, seg, s);
        default: break;
        }
    }
    return hipErrorInvalidValue;
}

/* The fused launches built: the reference model's layers (hidden 2560 =
 * 2048 + 512 columns of Q4_K gate/up, or Q5_K in its layer 2; intermediate
 * 640 = 512 + 128 columns of Q5_1 down, or Q8_0 in its layers 2, 4, 30, 46
 * and 47; a Q8_0 shared expert throughout) and the same with routed and
 * shared of one format. Returns false (nothing launched) for other formats
 * and widths. */
template <uint32_t TR>
bool gateup_fused_tr(uint32_t ts, const dim3 &grid, const GateupArgs &a, hipStream_t s) {
    if (ts == KQ_LAUNCH_Q8_0)
        hipLaunchKernelGGL((expert_gateup_fused<TR, KQ_LAUNCH_Q8_0, 2048u, 512u>), grid,
                           dim3(kThreads), 0, s, a);
    else if (ts == TR)
        hipLaunchKernelGGL((expert_gateup_fused<TR, TR, 2048u, 512u>), grid, dim3(kThreads), 0, s,
                           a);
    else
        return false;
    return true;
}

bool gateup_fused(uint32_t tr, uint32_t ts, uint32_t ng, const uint32_t (&gw)[16],
                  const GateupArgs &a, uint32_t tokens, hipError_t &e, hipStream_t s) {
    if (ng != 2u || gw[0] != 2048u || gw[1] != 512u) return false;
    const uint32_t rows = a.inter > a.shared_inter ? a.inter : a.shared_inter;
    const dim3 grid((rows + kFuseRows - 1u) / kFuseRows, a.top_k + 1u, tokens);
    bool launched = false;
    if (tr == KQ_LAUNCH_Q4_K)
        launched = gateup_fused_tr<KQ_LAUNCH_Q4_K>(ts, grid, a, s);
    else if (tr == KQ_LAUNCH_Q5_K)
        launched = gateup_fused_tr<KQ_LAUNCH_Q5_K>(ts, grid, a, s);
    if (!launched) return false;
    e = hipGetLastError();
    return true;
}

template <uint32_t TR>
bool down_fused_tr(uint32_t ts, const dim3 &grid, const dim3 &block, const DownArgs &a,
                   hipStream_t s) {
    if (ts == KQ_LAUNCH_Q8_0)
        hipLaunchKernelGGL((expert_down_fused<TR, KQ_LAUNCH_Q8_0, 512u, 128u>), grid, block, 0,
                           s, a);
    else if (ts == TR)
        hipLaunchKernelGGL((expert_down_fused<TR, TR, 512u, 128u>), grid, block, 0, s, a);
    else
        return false;
    return true;
}

bool down_fused(uint32_t tr, uint32_t ts, uint32_t nd, const uint32_t (&dw)[16],
                const DownArgs &a, uint32_t tokens, hipError_t &e, hipStream_t s) {
    if (nd != 2u || dw[0] != 512u || dw[1] != 128u || a.top_k + 1u > 16u) return false;
    const dim3 grid((a.hidden + kFuseRows - 1u) / kFuseRows, tokens);
    const dim3 block(64u * (a.top_k + 1u));
    bool launched = false;
    if (tr == KQ_LAUNCH_Q5_1)
        launched = down_fused_tr<KQ_LAUNCH_Q5_1>(ts, grid, block, a, s);
    else if (tr == KQ_LAUNCH_Q8_0)
        launched = down_fused_tr<KQ_LAUNCH_Q8_0>(ts, grid, block, a, s);
    if (!launched) return false;
    e = hipGetLastError();
    return true;
}

#define KQ_TYPE_SWITCH(TYPE_ID, CALL)                                   \
    switch (TYPE_ID) {                                                  \
    case KQ_LAUNCH_Q4_K: { constexpr uint32_t T_ = KQ_LAUNCH_Q4_K; return CALL; }     \
    case KQ_LAUNCH_Q6_K: { constexpr uint32_t T_ = KQ_LAUNCH_Q6_K; return CALL; }     \
    case KQ_LAUNCH_Q8_0: { constexpr uint32_t T_ = KQ_LAUNCH_Q8_0; return CALL; }     \
    case KQ_LAUNCH_Q5_K: { constexpr uint32_t T_ = KQ_LAUNCH_Q5_K; return CALL; }     \
    case KQ_LAUNCH_Q5_1: { constexpr uint32_t T_ = KQ_LAUNCH_Q5_1; return CALL; }     \
    case KQ_LAUNCH_IQ4_NL: { constexpr uint32_t T_ = KQ_LAUNCH_IQ4_NL; return CALL; } \
    default: return hipErrorInvalidValue;                               \
    }

hipError_t gateup_launch(uint32_t type, uint32_t width, const GateupArgs &a, uint32_t tokens,
                         uint32_t slot0, uint32_t nslot, uint32_t col0, uint32_t seg,
                         hipStream_t s) {
    KQ_TYPE_SWITCH(type, gateup_width<T_>(width, a, tokens, slot0, nslot, col0, seg, s))
}

hipError_t down_launch(uint32_t type, uint32_t width, const DownArgs &a, uint32_t tokens,
                       uint32_t slot0, uint32_t slot1, uint32_t col0, uint32_t seg,
                       hipStream_t s) {
    KQ_TYPE_SWITCH(type, down_width<T_>(width, a, tokens, slot0, slot1, col0, seg, s))
}

#undef KQ_TYPE_SWITCH

uint32_t row_bytes_of(uint32_t type, uint32_t cols) {
    switch (type) {
    case KQ_LAUNCH_Q4_K: return cols / 256u * 144u;
    case KQ_LAUNCH_Q5_K: return cols / 256u * 176u;
    case KQ_LAUNCH_Q6_K: return cols / 256u * 210u;
    case KQ_LAUNCH_Q8_0: return cols / 32u * 34u;
    case KQ_LAUNCH_Q5_1: return cols / 32u * 24u;
    case KQ_LAUNCH_IQ4_NL: return cols / 32u * 18u;
    default: return 0u;
    }
}

bool quant_type(uint32_t t) {
    return t == KQ_LAUNCH_Q4_K || t == KQ_LAUNCH_Q5_K || t == KQ_LAUNCH_Q6_K ||
           t == KQ_LAUNCH_Q8_0 || t == KQ_LAUNCH_Q5_1 || t == KQ_LAUNCH_IQ4_NL;
}


}  // namespace

extern "C" uint32_t kq_launch_moe_experts_padded(uint32_t experts) { return pad64(experts + 1u); }

static uint64_t align256(uint64_t v) { return (v + 255u) & ~(uint64_t)255u; }

/* outp holds, per token and slot, the grouped path's down outputs or the
 * per-token path's partial sums of column segments: hidden floats for
 * down, 2 x intermediate for gate/up */
static uint64_t outp_row(const kq_launch_moe_dims *d) {
    const uint64_t ai = d->inter > d->shared_inter ? d->inter : d->shared_inter;
    return d->hidden > 2u * ai ? d->hidden : 2u * ai;
}

/* outp also holds the grouped gate/up pass's split activations before the
 * down pass writes it */
static uint64_t outp_bytes(const kq_launch_moe_dims *d, uint32_t tokens) {
    const uint64_t o = align256((uint64_t)tokens * (d->top_k + 1u) * outp_row(d) * 4u);
    const uint64_t g = align256(kq_launch_gu_stage_bytes(tokens, d->hidden));
    return o > g ? o : g;
}

extern "C" uint64_t kq_launch_moe_ws_bytes(const kq_launch_moe_dims *d, uint32_t tokens) {
    const uint64_t ep = pad64(d->experts + 1u);
    const uint64_t ai = d->inter > d->shared_inter ? d->inter : d->shared_inter;
    uint64_t b = 0;
    b += align256((uint64_t)d->hidden * ep * 4u);                   /* router_t */
    b += align256((uint64_t)tokens * d->experts * 4u) * 2u;         /* logits, probs */
    b += align256((uint64_t)tokens * d->top_k * 4u) * 3u;           /* ids, weights, order */
    b += align256((uint64_t)tokens * 4u) * 2u;                      /* shared logit, scale */
    b += align256((uint64_t)tokens * (d->top_k + 1u) * ai * 4u);    /* act */
    b += align256((uint64_t)(d->experts + 1u) * 4u);                 /* offsets */
    b += align256((uint64_t)tokens * d->top_k * 4u) * 2u;           /* perm_tok, pos */
    b += outp_bytes(d, tokens);                                      /* outp */
    b += align256((uint64_t)(d->experts + 1u) * 16u);                /* bound */
    b += align256(kq_launch_dn_stage_bytes(tokens * (d->top_k + 1u), ai)); /* dstage */
    b += align256(kq_launch_gu_items_bytes(d->experts, tokens, d->top_k));  /* gitems */
    b += 256u;                          /* certified flag (the last slot) */
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
    ws->offsets = (uint32_t *)p; p += align256((uint64_t)(d->experts + 1u) * 4u);
    ws->perm_tok = (uint32_t *)p; p += align256((uint64_t)tokens * d->top_k * 4u);
    ws->pos = (uint32_t *)p; p += align256((uint64_t)tokens * d->top_k * 4u);
    ws->outp = (float *)p; p += outp_bytes(d, tokens);
    ws->bound = (double *)p; p += align256((uint64_t)(d->experts + 1u) * 16u);
    ws->dstage = p; p += align256(kq_launch_dn_stage_bytes(tokens * (d->top_k + 1u), ai));
    ws->gitems = p; p += align256(kq_launch_gu_items_bytes(d->experts, tokens, d->top_k));
    ws->certified = (uint32_t *)p;
}

extern "C" int kq_launch_moe_supported(const kq_launch_moe_dims *d,
                                       const kq_launch_moe_weights *w) {
    uint32_t seg[16];
    if (d->hidden % 4u != 0u || d->experts + 1u > 1024u || d->top_k < 1u ||
        d->top_k > d->experts || d->top_k > 64u)
        return 0;
    if (w == nullptr) return 1;
    if (d->inter != d->shared_inter || d->hidden > 65536u || d->inter > 65536u) return 0;
    /* gate and up share a type (routed, and shared); each role's rows are
     * whole blocks cut into segments that both of its types can run */
    if (!quant_type(w->gate_type) || w->up_type != w->gate_type ||
        !quant_type(w->shared_gate_type) || w->shared_up_type != w->shared_gate_type)
        return 0;
    if (!quant_type(w->down_type) || !quant_type(w->shared_down_type)) return 0;
    return segments(d->hidden, w->gate_type, w->shared_gate_type, seg) != 0u &&
           segments(d->inter, w->down_type, w->shared_down_type, seg) != 0u;
}

extern "C" hipError_t kq_launch_moe_route(const kq_launch_moe_dims *d, const float *router,
                                          const float *shared_gate_weight, const float *hidden,
                                          uint32_t tokens, const kq_launch_moe_ws *ws,
                                          uint32_t *status, int certify, uint32_t *ids_out,
                                          void *stage, hipStream_t s) {
    const uint32_t ep = pad64(d->experts + 1u);
    const uint32_t groups = (d->experts + 1u + kRtRows - 1u) / kRtRows;
    bool fused = tokens == 1u;
    uint32_t fin = 64u * ((d->experts + 63u) / 64u + 1u);
    if (fin > 1024u) fin = 1024u;
    /* one token, ids only needed exactly: the bounds, then the selection
     * (certified, refined or exact) in one workgroup */
    if (fused && certify && d->top_k <= kMaxTopK) {
        RouteArgs a;
        a.router = router;
        a.sgw = shared_gate_weight;
        a.x = hidden;
        a.experts = d->experts;
        a.top_k = d->top_k;
        a.bound = ws->bound;
        a.logits = ws->logits;
        a.shared_logit = ws->shared_logit;
        a.probs = ws->probs;
        a.ids = ws->ids;
        a.ids_out = ids_out;
        a.weights = ws->weights;
        a.order = ws->order;
        a.shared_scale = ws->shared_scale;
        a.status = status;
        a.certified = ws->certified;
        const uint32_t bgroups = (d->experts + kSelRows) / kSelRows; /* E + 1 rows */
        bool have = true;
#define KQ_ROUTE_ONE(H)                                                                  \
    hipLaunchKernelGGL(route_bounds<H>, dim3(bgroups), dim3(64u * kSelRows * kSelParts), 0, s, \
                       a);                                                               \
    hipLaunchKernelGGL(route_select<H>, dim3(1), dim3(1024), 0, s, a)
        switch (d->hidden) {
        case 256: KQ_ROUTE_ONE(256u); break;
        case 512: KQ_ROUTE_ONE(512u); break;
        case 1024: KQ_ROUTE_ONE(1024u); break;
        case 2048: KQ_ROUTE_ONE(2048u); break;
        case 2560: KQ_ROUTE_ONE(2560u); break;
        default: have = false;
        }
#undef KQ_ROUTE_ONE
        if (have) return hipGetLastError();
    }
#define KQ_ROUTER_DECODE(H)                                                                   \
    hipLaunchKernelGGL(router_decode<H>, dim3(groups), dim3(kThreads), 0, s, router,          \
                       shared_gate_weight, hidden, d->experts, ws->logits, ws->shared_logit, \
                       status)
    if (fused) {
        switch (d->hidden) {
        case 256: KQ_ROUTER_DECODE(256u); break;
        case 512: KQ_ROUTER_DECODE(512u); break;
        case 1024: KQ_ROUTER_DECODE(1024u); break;
        case 2048: KQ_ROUTER_DECODE(2048u); break;
        case 2560: KQ_ROUTER_DECODE(2560u); break;
        default: fused = false;
        }
    }
#undef KQ_ROUTER_DECODE
    /* several tokens: the chains read the router in place and the route
     * finish forms the shared gate's logit */
    const bool in_place = !fused && d->hidden % kSxCols == 0u;
    if (in_place) {
        const uint32_t per_wg = kSxTW * kSxWaves;
        hipLaunchKernelGGL(router_chain_sx,
                           dim3((tokens + per_wg - 1u) / per_wg, (d->experts + 63u) / 64u),
                           dim3(64u * kSxWaves), 0, s, router, hidden, tokens, d->experts,
                           d->hidden, ws->logits, status);
    } else if (!fused) {
        /* a hidden size the chunked chains do not cover */
        const dim3 tgrid(ep / 64u, (d->hidden / 4u + 15u) / 16u);
        hipLaunchKernelGGL(router_transpose, tgrid, dim3(kThreads), 0, s, router,
                           shared_gate_weight, d->experts, d->hidden, ep, ws->router_t, status);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(router_chain, dim3(ep / 64u, tokens), dim3(64), 0, s, ws->router_t,
                           hidden, d->experts, d->hidden, ep, ws->logits, ws->shared_logit);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(route_finish, dim3(tokens), dim3(fin), 0, s, ws->logits, ws->shared_logit,
                       d->experts, d->top_k, ws->probs, ws->ids, ws->weights, ws->order,
                       ws->shared_scale, status, in_place ? shared_gate_weight : nullptr, hidden,
                       d->hidden, stage);
    e = hipGetLastError();
    /* the one-token selection writes the caller's ids itself; here they
     * are copied (several tokens, or a hidden size without an instance) */
    if (e == hipSuccess && ids_out != nullptr)
        e = hipMemcpyAsync(ids_out, ws->ids, (size_t)tokens * d->top_k * 4u,
                           hipMemcpyDeviceToDevice, s);
    return e;
}

extern "C" hipError_t kq_launch_moe_route_finish(const float *logits, const float *shared_logit,
                                                 uint32_t experts, uint32_t top_k,
                                                 uint32_t tokens, float *probs, uint32_t *ids,
                                                 float *weights, uint32_t *order,
                                                 float *shared_scale, uint32_t *status,
                                                 hipStream_t s) {
    const uint32_t fin = 64u * ((experts + 63u) / 64u + 1u);
    if (fin > 1024u || top_k == 0u || top_k > experts || top_k > kMaxTopK)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(route_finish, dim3(tokens), dim3(fin), 0, s, logits,
                       const_cast<float *>(shared_logit), experts, top_k, probs, ids, weights,
                       order, shared_scale, status, nullptr, nullptr, 0u, nullptr);
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_moe_experts(const kq_launch_moe_dims *d,
                                            const kq_launch_moe_weights *w, const float *hidden,
                                            uint32_t tokens, const kq_launch_moe_ws *ws,
                                            float *out, uint32_t *status, hipStream_t s) {
    const uint32_t K = d->top_k;
    uint32_t gw[16], dw[16];
    const uint32_t ng = segments(d->hidden, w->gate_type, w->shared_gate_type, gw);
    const uint32_t nd = segments(d->inter, w->down_type, w->shared_down_type, dw);
    if (ng == 0u || nd == 0u) return hipErrorInvalidValue;
    GateupArgs ga;
    ga.gate = (const uint8_t *)w->gate;
    ga.up = (const uint8_t *)w->up;
    ga.sgate = (const uint8_t *)w->shared_gate;
    ga.sup = (const uint8_t *)w->shared_up;
    ga.x = hidden;
    ga.ids = ws->ids;
    ga.top_k = K;
    ga.inter = d->inter;
    ga.shared_inter = d->shared_inter;
    ga.hidden = d->hidden;
    ga.rstride = row_bytes_of(w->gate_type, d->hidden);
    ga.srstride = row_bytes_of(w->shared_gate_type, d->hidden);
    ga.act_stride = d->inter > d->shared_inter ? d->inter : d->shared_inter;
    ga.act = ws->act;
    ga.part = ws->outp;
    ga.status = status;
    /* the shared expert rides in the routed launch when its type matches */
    const bool gsame = w->shared_gate_type == w->gate_type;
    hipError_t e = hipSuccess;
    const bool gf = gateup_fused(w->gate_type, w->shared_gate_type, ng, gw, ga, tokens, e, s);
    for (uint32_t k = 0, col = 0; !gf && k < ng && e == hipSuccess; col += gw[k], ++k) {
        const uint32_t seg = (k == 0u ? kSegFirst : 0u) | (k + 1u == ng ? kSegLast : 0u);
        e = gateup_launch(w->gate_type, gw[k], ga, tokens, 0u, gsame ? K + 1u : K, col, seg, s);
        if (e == hipSuccess && !gsame)
            e = gateup_launch(w->shared_gate_type, gw[k], ga, tokens, K, 1u, col, seg, s);
    }
    if (e != hipSuccess) return e;
    DownArgs da;
    da.down = (const uint8_t *)w->down;
    da.sdown = (const uint8_t *)w->shared_down;
    da.act = ws->act;
    da.ids = ws->ids;
    da.order = ws->order;
    da.weights = ws->weights;
    da.shared_scale = ws->shared_scale;
    da.top_k = K;
    da.hidden = d->hidden;
    da.rstride = row_bytes_of(w->down_type, d->inter);
    da.srstride = row_bytes_of(w->shared_down_type, d->inter);
    da.act_stride = ga.act_stride;
    da.part = ws->outp;
    da.out = out;
    da.status = status;
    const bool dsame = w->shared_down_type == w->down_type;
    if (down_fused(w->down_type, w->shared_down_type, nd, dw, da, tokens, e, s)) return e;
    /* a shared expert of its own type is finished (into part[t][K]) before
     * the routed launches that combine it */
    if (!dsame) {
        for (uint32_t k = 0, col = 0; k < nd && e == hipSuccess; col += dw[k], ++k) {
            const uint32_t seg = (k == 0u ? kSegFirst : 0u) | (k + 1u == nd ? kSegLast : 0u);
            e = down_launch(w->shared_down_type, dw[k], da, tokens, K, K + 1u, col, seg, s);
        }
    }
    for (uint32_t k = 0, col = 0; k < nd && e == hipSuccess; col += dw[k], ++k) {
        const uint32_t seg = (k == 0u ? kSegFirst : 0u) | (k + 1u == nd ? kSegLast | kSegCombine : 0u);
        e = down_launch(w->down_type, dw[k], da, tokens, 0u, dsame ? K + 1u : K, col, seg, s);
    }
    return e;
}
