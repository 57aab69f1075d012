/*
 * kq_moe_f32.hip — the MoE operator on F32 expert weights, in the
 * reference's arithmetic order: kq_moe_execute_f32
 * (src/kq_moe_qwen38.c:604-880) with kq_moe_project / kq_f32_dot
 * (src/kq_moe_qwen38.c:198-209, src/kq_numeric.c:591-625), kq_f32_swiglu,
 * kq_f32_scale, kq_f32_add and the ascending-expert accumulation
 * (src/kq_moe_qwen38.c:722-765, :771-826).
 *
 * Every dot is one thread's left-to-right binary32 chain of separately
 * rounded products (the file is compiled with -ffp-contract=off), so each
 * checkpoint is bit-identical to the reference's. Threads own output rows;
 * slot k < top_k of a token is its k-th selected expert (top-k order), slot
 * top_k the shared expert. Every intermediate stays in the caller's scratch
 * (the trace the host hands to checkpoint observers):
 *   gate, up, activated [T][K+1][I'] (I' = max(routed, shared) intermediate),
 *   expert output, weighted output [T][K+1][H] (slot K: shared output and
 *   gated shared output), routed sum [T][H].
 * Any non-finite weight, input or result sets the NUMERIC bit of the status
 * word (the reference validates every weight and result the same way).
 */
#include "kq_device.h"
#include "kq_launch.h"

namespace {

constexpr int kF32Threads = 256;

/* left-to-right binary32 dot of n values, products rounded first */
__device__ __forceinline__ float chain_dot(const float *__restrict__ w, const float *__restrict__ x,
                                           uint32_t n) {
    float acc = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        const float p = w[i] * x[i];
        acc = acc + p;
    }
    return acc;
}

__global__ __launch_bounds__(kF32Threads) void f32_scan(const float *__restrict__ p, uint64_t n,
                                                        uint32_t *status) {
    bool bad = false;
    const uint64_t stride = (uint64_t)gridDim.x * kF32Threads;
    for (uint64_t i = (uint64_t)blockIdx.x * kF32Threads + threadIdx.x; i < n; i += stride)
        bad |= !kq_isfinite(p[i]);
    if (__ballot(bad) != 0ull && (threadIdx.x & 63u) == 0u) kq_flag(status, KQ_DEV_NUMERIC);
}

/* router logits (rows 0..E-1) and the shared gate logit (row E) */
__global__ __launch_bounds__(kF32Threads) void f32_route_logits(
    const float *__restrict__ router, const float *__restrict__ sgw, const float *__restrict__ x,
    uint32_t hidden, uint32_t experts, float *__restrict__ logits,
    float *__restrict__ shared_logit, uint32_t *status) {
    const uint32_t r = blockIdx.x * kF32Threads + threadIdx.x, t = blockIdx.y;
    if (r > experts) return;
    const float *w = r < experts ? router + (size_t)r * hidden : sgw;
    const float l = chain_dot(w, x + (size_t)t * hidden, hidden);
    if (!kq_isfinite(l)) kq_flag(status, KQ_DEV_NUMERIC);
    if (r < experts)
        logits[(size_t)t * experts + r] = l;
    else
        shared_logit[t] = l;
}

struct F32Args {
    const float *gate, *up, *down;    /* routed stacks [E][I][H], [E][I][H], [E][H][I] */
    const float *sgate, *sup, *sdown; /* shared [S][H], [S][H], [H][S] */
    const float *x;                   /* [T][H] */
    const uint32_t *ids;              /* [T][K] top-k order */
    const uint32_t *order;            /* [T][K] top-k position of the j-th smallest id */
    const float *weights;             /* [T][K] */
    const float *shared_scale;        /* [T] */
    float *gate_o, *up_o, *act;       /* [T][K+1][Ip] */
    float *out_o, *wout;              /* [T][K+1][H] */
    float *routed_sum, *y;            /* [T][H] */
    uint32_t hidden, inter, shared_inter, top_k, ip;
    uint32_t *status;
};

/* gate and up rows of slot blockIdx.y of token blockIdx.z, then SwiGLU */
__global__ __launch_bounds__(kF32Threads) void f32_gateup(F32Args a) {
    const uint32_t r = blockIdx.x * kF32Threads + threadIdx.x;
    const uint32_t k = blockIdx.y, t = blockIdx.z, H = a.hidden;
    const bool shared = k == a.top_k;
    const uint32_t rows = shared ? a.shared_inter : a.inter;
    if (r >= rows) return;
    const float *g, *u;
    if (shared) {
        g = a.sgate + (size_t)r * H;
        u = a.sup + (size_t)r * H;
    } else {
        const size_t e = a.ids[(size_t)t * a.top_k + k];
        g = a.gate + (e * a.inter + r) * H;
        u = a.up + (e * a.inter + r) * H;
    }
    const float *x = a.x + (size_t)t * H;
    const float gv = chain_dot(g, x, H), uv = chain_dot(u, x, H);
    const float av = kq_swiglu(gv, uv);
    if (!kq_isfinite(gv) || !kq_isfinite(uv) || !kq_isfinite(av)) kq_flag(a.status, KQ_DEV_NUMERIC);
    const size_t o = ((size_t)t * (a.top_k + 1u) + k) * a.ip + r;
    a.gate_o[o] = gv;
    a.up_o[o] = uv;
    a.act[o] = av;
}

/* down rows of slot blockIdx.y: expert output and its weighted copy (the
 * shared expert: its output and the gated output) */
__global__ __launch_bounds__(kF32Threads) void f32_down(F32Args a) {
    const uint32_t h = blockIdx.x * kF32Threads + threadIdx.x;
    const uint32_t k = blockIdx.y, t = blockIdx.z, H = a.hidden;
    if (h >= H) return;
    const bool shared = k == a.top_k;
    const uint32_t cols = shared ? a.shared_inter : a.inter;
    const float *w;
    float s;
    if (shared) {
        w = a.sdown + (size_t)h * cols;
        s = a.shared_scale[t];
    } else {
        const size_t e = a.ids[(size_t)t * a.top_k + k];
        w = a.down + (e * H + h) * cols;
        s = a.weights[(size_t)t * a.top_k + k];
    }
    const size_t slot = (size_t)t * (a.top_k + 1u) + k;
    const float o = chain_dot(w, a.act + slot * a.ip, cols);
    const float ws = o * s;
    if (!kq_isfinite(o) || !kq_isfinite(ws)) kq_flag(a.status, KQ_DEV_NUMERIC);
    a.out_o[slot * H + h] = o;
    a.wout[slot * H + h] = ws;
}

/* routed sum in ascending expert id, then + gated shared output */
__global__ __launch_bounds__(kF32Threads) void f32_combine(F32Args a) {
    const uint32_t h = blockIdx.x * kF32Threads + threadIdx.x, t = blockIdx.y, H = a.hidden;
    if (h >= H) return;
    const size_t base = (size_t)t * (a.top_k + 1u);
    float sum = 0.0f;
    bool bad = false;
    for (uint32_t j = 0; j < a.top_k; ++j) {
        const uint32_t k = a.order[(size_t)t * a.top_k + j];
        sum = sum + a.wout[(base + k) * H + h];
        bad |= !kq_isfinite(sum);
    }
    const float y = sum + a.wout[(base + a.top_k) * H + h];
    if (bad || !kq_isfinite(y)) kq_flag(a.status, KQ_DEV_NUMERIC);
    a.routed_sum[(size_t)t * H + h] = sum;
    a.y[(size_t)t * H + h] = y;
}

/* one routed expert (src/kq_moe_qwen38.c:436-459): gate and up rows, then
 * SwiGLU, one thread per row */
__global__ __launch_bounds__(kF32Threads) void f32_member_gateup(
    const float *__restrict__ gw, const float *__restrict__ uw, const float *__restrict__ x,
    uint32_t hidden, uint32_t inter, float *__restrict__ gate, float *__restrict__ up,
    float *__restrict__ act, uint32_t *status) {
    const uint32_t r = blockIdx.x * kF32Threads + threadIdx.x;
    if (r >= inter) return;
    const float gv = chain_dot(gw + (size_t)r * hidden, x, hidden);
    const float uv = chain_dot(uw + (size_t)r * hidden, x, hidden);
    const float av = kq_swiglu(gv, uv);
    if (!kq_isfinite(gv) || !kq_isfinite(uv) || !kq_isfinite(av)) kq_flag(status, KQ_DEV_NUMERIC);
    gate[r] = gv;
    up[r] = uv;
    act[r] = av;
}

/* its down rows over the activated vector */
__global__ __launch_bounds__(kF32Threads) void f32_member_down(
    const float *__restrict__ dw, const float *__restrict__ act, uint32_t hidden, uint32_t inter,
    float *__restrict__ out, uint32_t *status) {
    const uint32_t h = blockIdx.x * kF32Threads + threadIdx.x;
    if (h >= hidden) return;
    const float o = chain_dot(dw + (size_t)h * inter, act, inter);
    if (!kq_isfinite(o)) kq_flag(status, KQ_DEV_NUMERIC);
    out[h] = o;
}

uint32_t blocks_for(uint64_t n) { return (uint32_t)((n + kF32Threads - 1u) / kF32Threads); }

}  // namespace

extern "C" hipError_t kq_launch_routed_expert_f32(const float *gate_w, const float *up_w,
                                                  const float *down_w, const float *x,
                                                  uint32_t hidden, uint32_t inter, float *gate,
                                                  float *up, float *act, float *out,
                                                  uint32_t *status, hipStream_t s) {
    hipLaunchKernelGGL(f32_member_gateup, dim3(blocks_for(inter)), dim3(kF32Threads), 0, s,
                       gate_w, up_w, x, hidden, inter, gate, up, act, status);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(f32_member_down, dim3(blocks_for(hidden)), dim3(kF32Threads), 0, s,
                       down_w, act, hidden, inter, out, status);
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_f32_scan(const float *p, uint64_t n, uint32_t *status,
                                         hipStream_t s) {
    if (n == 0u) return hipSuccess;
    uint64_t b = (n + kF32Threads - 1u) / kF32Threads;
    if (b > 4096u) b = 4096u;
    hipLaunchKernelGGL(f32_scan, dim3((uint32_t)b), dim3(kF32Threads), 0, s, p, n, status);
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_moe_f32(const kq_launch_moe_dims *d,
                                        const kq_launch_moe_f32_weights *w, const float *hidden,
                                        uint32_t tokens, const kq_launch_moe_f32_ws *ws,
                                        float *out, uint32_t *status, hipStream_t s) {
    const uint32_t E = d->experts, K = d->top_k, H = d->hidden;
    hipLaunchKernelGGL(f32_route_logits, dim3(blocks_for(E + 1u), tokens), dim3(kF32Threads), 0,
                       s, w->router, w->shared_gate_weight, hidden, H, E, ws->logits,
                       ws->shared_logit, status);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess)
        e = kq_launch_moe_route_finish(ws->logits, ws->shared_logit, E, K, tokens, ws->probs,
                                       ws->ids, ws->weights, ws->order, ws->shared_scale, status,
                                       s);
    if (e != hipSuccess) return e;
    F32Args a;
    a.gate = w->gate;
    a.up = w->up;
    a.down = w->down;
    a.sgate = w->shared_gate;
    a.sup = w->shared_up;
    a.sdown = w->shared_down;
    a.x = hidden;
    a.ids = ws->ids;
    a.order = ws->order;
    a.weights = ws->weights;
    a.shared_scale = ws->shared_scale;
    a.gate_o = ws->gate;
    a.up_o = ws->up;
    a.act = ws->act;
    a.out_o = ws->out;
    a.wout = ws->weighted;
    a.routed_sum = ws->routed_sum;
    a.y = out;
    a.hidden = H;
    a.inter = d->inter;
    a.shared_inter = d->shared_inter;
    a.top_k = K;
    a.ip = d->inter > d->shared_inter ? d->inter : d->shared_inter;
    a.status = status;
    hipLaunchKernelGGL(f32_gateup, dim3(blocks_for(a.ip), K + 1u, tokens), dim3(kF32Threads), 0,
                       s, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(f32_down, dim3(blocks_for(H), K + 1u, tokens), dim3(kF32Threads), 0, s, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(f32_combine, dim3(blocks_for(H), tokens), dim3(kF32Threads), 0, s, a);
    return hipGetLastError();
}
