/*
 * kq_gr.hip — the gated residual around a layer block (hyper-connection
 * read and write) on gfx950.
 *
 * Restates kq_layer_gr_read_common and kq_layer_gr_write_f32
 * (src/kq_layer_qwen38.c:40-208), which src/kq_layer.c:779-813 calls
 * around the MoE. A token's state is B residual branches of H values
 * (width W = B * H):
 *
 *   read   normalized[b]  = rms_norm(branches[b], norm[b])
 *          rank           = silu(down . normalized / B)           (rank r)
 *          read_gate      = sigmoid(up . rank)                    (W)
 *          mixed[i]       = sum_b read_gate[b,i] * normalized[b,i] / B
 *          write_gate[b]  = 2 * sigmoid(inject[b] . normalized / B)
 *   write  out[b,i]       = branches[b,i] + block_output[i] * write_gate[b]
 *
 * The two projections run on the quantized matvec (the model's hc_*_down /
 * hc_*_up are Q8_0) or, for F32 weights, on matvec_f32w below. The RMS
 * norm's sum of squares and the inject dots are workgroup reductions (fp32,
 * compared with the CPU's left-to-right sums by tolerance); the per-element
 * steps keep the reference's order of separately rounded operations (this
 * file builds with -ffp-contract=off), and the write is exact.
 */
#include "kq_device.h"
#include "kq_launch.h"

namespace {

constexpr int kThreads = 256;
constexpr int kNormThreads = 256; /* a branch of H values, float4 per thread where H % 4 == 0 */

/* sum over the workgroup (NT threads), returned to every thread */
template <int NT>
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, KQ_WAVE);
    const uint32_t wave = threadIdx.x >> 6;
    __syncthreads(); /* earlier readers of red are done */
    if ((threadIdx.x & 63u) == 0u) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) s += red[w];
    return s;
}

/* grid (B, T): one workgroup per branch of a token (src/kq_numeric.c:722-775) */
__global__ __launch_bounds__(kNormThreads) void gr_norm(const float *__restrict__ x,
                                                    const float *__restrict__ norm, uint32_t B,
                                                    uint32_t H, float eps,
                                                    float *__restrict__ out, uint32_t *status) {
    __shared__ float red[kNormThreads / 64];
    const uint32_t b = blockIdx.x, t = blockIdx.y;
    const size_t base = ((size_t)t * B + b) * H;
    const float *w = norm + (size_t)b * H;
    bool badin = false, bad = false;
    float s = 0.0f;
    /* (the state is 16-byte aligned; the norm weights may be only 4) */
    const bool v4 = H % 4u == 0u && ((uintptr_t)w & 15u) == 0u;
    if (v4) {
        const float4 *x4 = (const float4 *)(x + base), *w4 = (const float4 *)w;
        for (uint32_t i = threadIdx.x; i < H / 4u; i += kNormThreads) {
            const float4 v = x4[i], wv = w4[i];
            badin |= !kq_isfinite(v.x) || !kq_isfinite(v.y) || !kq_isfinite(v.z) ||
                     !kq_isfinite(v.w) || !kq_isfinite(wv.x) || !kq_isfinite(wv.y) ||
                     !kq_isfinite(wv.z) || !kq_isfinite(wv.w);
            float sq;
            sq = v.x * v.x; s += sq;
            sq = v.y * v.y; s += sq;
            sq = v.z * v.z; s += sq;
            sq = v.w * v.w; s += sq;
        }
    } else {
        for (uint32_t i = threadIdx.x; i < H; i += kNormThreads) {
            const float v = x[base + i];
            badin |= !kq_isfinite(v) || !kq_isfinite(w[i]);
            const float sq = v * v;
            s += sq;
        }
    }
    s = block_sum<kNormThreads>(s, red);
    const float mean = s / (float)H;
    const float inv = 1.0f / sqrtf(mean + eps);
    bad |= !kq_isfinite(inv);
    auto one = [&](float xv, float wv) {
        const float nv = xv * inv;
        const float wt = 1.0f + wv;
        const float r = nv * wt;
        bad |= !kq_isfinite(r);
        return r;
    };
    if (v4) {
        const float4 *x4 = (const float4 *)(x + base), *w4 = (const float4 *)w;
        float4 *o4 = (float4 *)(out + base);
        for (uint32_t i = threadIdx.x; i < H / 4u; i += kNormThreads) {
            const float4 v = x4[i], wv = w4[i];
            o4[i] = make_float4(one(v.x, wv.x), one(v.y, wv.y), one(v.z, wv.z), one(v.w, wv.w));
        }
    } else {
        for (uint32_t i = threadIdx.x; i < H; i += kNormThreads) out[base + i] = one(x[base + i], w[i]);
    }
    if (badin) kq_flag(status, KQ_DEV_INPUT);
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
}

/* rank[i] = silu(raw[i] / B) over T * r values: raw in place, or (parts)
 * the sum of nparts slices of a split projection, in slice order */
__global__ __launch_bounds__(kThreads) void gr_rank(float *__restrict__ v, uint32_t n, uint32_t B,
                                                    const float *__restrict__ parts,
                                                    uint32_t nparts, uint32_t *status) {
    bool bad = false;
    for (uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads) {
        float raw;
        if (parts != nullptr) {
            raw = parts[i];
            for (uint32_t k = 1; k < nparts; ++k) raw = raw + parts[(size_t)k * n + i];
        } else {
            raw = v[i];
        }
        const float a = raw / (float)B;
        const float s = kq_sigmoid(a);
        const float r = a * s;
        bad |= !kq_isfinite(r);
        v[i] = r;
    }
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
}

/* grid (G + B, T), G = ceil(H / kThreads): workgroups below G mix kThreads
 * values of the token's state each (read gates, branch mix); workgroup G + b
 * forms write gate b from the inject dot over the whole width */
__global__ __launch_bounds__(kThreads) void gr_mix(const float *__restrict__ read_raw,
                                                   const float *__restrict__ normalized,
                                                   const float *__restrict__ inject, uint32_t B,
                                                   uint32_t H, float *__restrict__ mixed,
                                                   float *__restrict__ write_gate,
                                                   uint32_t *status) {
    __shared__ float red[kThreads / 64];
    const uint32_t t = blockIdx.y;
    const uint32_t W = B * H;
    const uint32_t G = (H + kThreads - 1) / kThreads;
    const float *rr = read_raw + (size_t)t * W;
    const float *nm = normalized + (size_t)t * W;
    bool bad = false;
    if (blockIdx.x < G) {
        const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
        if (i < H) {
            float sum = 0.0f;
#pragma unroll 4
            for (uint32_t b = 0; b < B; ++b) {
                const float g = kq_sigmoid(rr[(size_t)b * H + i]);
                const float p = g * nm[(size_t)b * H + i];
                sum += p;
            }
            const float m = sum / (float)B;
            bad = !kq_isfinite(m);
            mixed[(size_t)t * H + i] = m;
        }
    } else {
        const uint32_t b = blockIdx.x - G;
        const float *inj = inject + (size_t)b * W;
        float s = 0.0f;
#pragma unroll 8
        for (uint32_t i = threadIdx.x; i < W; i += kThreads) {
            const float p = inj[i] * nm[i];
            s += p;
        }
        s = block_sum<kThreads>(s, red);
        if (threadIdx.x == 0u) {
            const float g = s / (float)B;
            const float r = 2.0f * kq_sigmoid(g);
            bad = !kq_isfinite(r);
            write_gate[(size_t)t * B + b] = r;
        }
    }
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
}

/* out[t][b][i] = x[t][b][i] + block_output[t][i] * write_gate[t][b]; out
 * may be x (every element reads only its own position of x) */
__global__ __launch_bounds__(kThreads) void gr_write(const float *x, const float *block_output,
                                                     const float *write_gate, uint32_t T,
                                                     uint32_t B, uint32_t H, float *out,
                                                     uint32_t *status) {
    const size_t n = (size_t)T * B * H;
    bool bad = false;
    for (size_t k = (size_t)blockIdx.x * kThreads + threadIdx.x; k < n;
         k += (size_t)gridDim.x * kThreads) {
        const size_t i = k % H, tb = k / H, t = tb / B;
        const float p = block_output[t * H + i] * write_gate[tb];
        const float r = x[k] + p;
        bad |= !kq_isfinite(r);
        out[k] = r;
    }
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
}

/* y[b][r] = W[r] . x[b] for F32 weights [rows][cols] (cols % 4 == 0),
 * batch <= 8: one row per wave, float4 loads, a wave reduction per
 * activation column */
template <int NB>
__global__ __launch_bounds__(kThreads) void matvec_f32w(const float *__restrict__ Wt,
                                                        uint32_t rows, uint32_t cols,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, uint32_t *status) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = __builtin_amdgcn_readfirstlane((blockIdx.x * kThreads + threadIdx.x) >> 6);
    if (row >= rows) return;
    const float4 *w4 = (const float4 *)(Wt + (size_t)row * cols);
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
    bool bad = false;
    for (uint32_t q = lane; q < cols / 4u; q += 64u) {
        const float4 w = w4[q];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float4 v = ((const float4 *)(x + (size_t)b * cols))[q];
            bad |= !kq_isfinite(v.x) || !kq_isfinite(v.y) || !kq_isfinite(v.z) ||
                   !kq_isfinite(v.w);
            acc[b] = fmaf(w.x, v.x, acc[b]);
            acc[b] = fmaf(w.y, v.y, acc[b]);
            acc[b] = fmaf(w.z, v.z, acc[b]);
            acc[b] = fmaf(w.w, v.w, acc[b]);
        }
    }
    bool nonfinite = false;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        float s = acc[b];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, KQ_WAVE);
        nonfinite |= !kq_isfinite(s);
        if (lane == 0u) y[(size_t)b * rows + row] = s;
    }
    if (bad) kq_flag(status, KQ_DEV_INPUT);
    if (nonfinite) kq_flag(status, KQ_DEV_NUMERIC);
}

/* y[b][r] = W[r] . x[b] for Q8_0 rows wider than the row engine's widest
 * segment (2048 columns), batch <= 4, in one launch: one row per wave, lane
 * j takes blocks j, j + 64, ... (34 bytes: an f16 scale and 32 int8 codes,
 * read as 17 halfwords), each block's d * sum(q * x) added to the lane's
 * sum, then a wave reduction */
template <int NB>
__global__ __launch_bounds__(kThreads) void matvec_q8w(const uint8_t *__restrict__ Wq,
                                                       uint32_t rows, uint32_t nblk,
                                                       const float *__restrict__ x,
                                                       float *__restrict__ y, uint32_t *status) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = __builtin_amdgcn_readfirstlane((blockIdx.x * kThreads + threadIdx.x) >> 6);
    if (row >= rows) return;
    const uint32_t cols = nblk * 32u;
    const uint16_t *wr = (const uint16_t *)(Wq + (size_t)row * nblk * 34u);
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
    bool badx = false, bads = false;
    for (uint32_t k = lane; k < nblk; k += 64u) {
        const uint16_t *h = wr + (size_t)k * 17u;
        uint32_t q[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) q[j] = h[1 + j];
        const float d = kq_f16_to_f32(h[0]);
        bads |= !kq_isfinite(d);
        float part[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) part[b] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float q0 = (float)(int8_t)(q[2 * j] & 0xffu);
            const float q1 = (float)(int8_t)(q[2 * j] >> 8);
            const float q2 = (float)(int8_t)(q[2 * j + 1] & 0xffu);
            const float q3 = (float)(int8_t)(q[2 * j + 1] >> 8);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float4 v = *(const float4 *)(x + (size_t)b * cols + (size_t)k * 32u + 4u * j);
                badx |= !kq_isfinite(v.x) || !kq_isfinite(v.y) || !kq_isfinite(v.z) ||
                        !kq_isfinite(v.w);
                part[b] = fmaf(q0, v.x, part[b]);
                part[b] = fmaf(q1, v.y, part[b]);
                part[b] = fmaf(q2, v.z, part[b]);
                part[b] = fmaf(q3, v.w, part[b]);
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = fmaf(d, part[b], acc[b]);
    }
    bool nonfinite = false;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        float s = acc[b];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, KQ_WAVE);
        nonfinite |= !kq_isfinite(s);
        if (lane == 0u) y[(size_t)b * rows + row] = s;
    }
    if (badx) kq_flag(status, KQ_DEV_INPUT);
    if (bads) kq_flag(status, KQ_DEV_MALFORMED);
    if (nonfinite) kq_flag(status, KQ_DEV_NUMERIC);
}

uint32_t grid_for(size_t n) {
    size_t b = (n + kThreads - 1) / kThreads;
    if (b > 4096u) b = 4096u;
    return b < 1u ? 1u : (uint32_t)b;
}

}  // namespace

extern "C" hipError_t kq_launch_gr_norm(const float *x, const float *norm, uint32_t tokens,
                                        uint32_t branches, uint32_t hidden, float eps,
                                        float *normalized, uint32_t *status, hipStream_t s) {
    hipLaunchKernelGGL(gr_norm, dim3(branches, tokens), dim3(kNormThreads), 0, s, x, norm, branches,
                       hidden, eps, normalized, status);
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_gr_rank(float *rank, uint32_t n, uint32_t branches,
                                        const float *parts, uint32_t nparts, uint32_t *status,
                                        hipStream_t s) {
    hipLaunchKernelGGL(gr_rank, dim3(grid_for(n)), dim3(kThreads), 0, s, rank, n, branches,
                       parts, nparts, status);
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_gr_mix(const float *read_raw, const float *normalized,
                                       const float *inject, uint32_t tokens, uint32_t branches,
                                       uint32_t hidden, float *mixed, float *write_gate,
                                       uint32_t *status, hipStream_t s) {
    const uint32_t groups = (hidden + kThreads - 1) / kThreads + branches;
    hipLaunchKernelGGL(gr_mix, dim3(groups, tokens), dim3(kThreads), 0, s, read_raw, normalized, inject,
                       branches, hidden, mixed, write_gate, status);
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_gr_write(const float *x, const float *block_output,
                                         const float *write_gate, uint32_t tokens,
                                         uint32_t branches, uint32_t hidden, float *out,
                                         uint32_t *status, hipStream_t s) {
    hipLaunchKernelGGL(gr_write, dim3(grid_for((size_t)tokens * branches * hidden)),
                       dim3(kThreads), 0, s, x, block_output, write_gate, tokens, branches,
                       hidden, out, status);
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_matvec_f32w(const float *W, uint32_t rows, uint32_t cols,
                                            const float *x, uint32_t batch, float *y,
                                            uint32_t *status, hipStream_t s) {
    const dim3 grid((rows + kThreads / 64 - 1) / (kThreads / 64));
    for (uint32_t done = 0; done < batch;) {
        const uint32_t nb = batch - done >= 4u ? 4u : batch - done;
        const float *xb = x + (size_t)done * cols;
        float *yb = y + (size_t)done * rows;
        switch (nb) {
        case 1: hipLaunchKernelGGL(matvec_f32w<1>, grid, dim3(kThreads), 0, s, W, rows, cols, xb, yb, status); break;
        case 2: hipLaunchKernelGGL(matvec_f32w<2>, grid, dim3(kThreads), 0, s, W, rows, cols, xb, yb, status); break;
        case 3: hipLaunchKernelGGL(matvec_f32w<3>, grid, dim3(kThreads), 0, s, W, rows, cols, xb, yb, status); break;
        default: hipLaunchKernelGGL(matvec_f32w<4>, grid, dim3(kThreads), 0, s, W, rows, cols, xb, yb, status); break;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        done += nb;
    }
    return hipSuccess;
}

extern "C" hipError_t kq_launch_matvec_q8w(const void *W, uint32_t rows, uint32_t cols,
                                           const float *x, uint32_t batch, float *y,
                                           uint32_t *status, hipStream_t s) {
    if (cols % 32u != 0u) return hipErrorInvalidValue;
    const uint8_t *wq = (const uint8_t *)W;
    const uint32_t nblk = cols / 32u;
    const dim3 grid((rows + kThreads / 64 - 1) / (kThreads / 64));
    for (uint32_t done = 0; done < batch;) {
        const uint32_t nb = batch - done >= 4u ? 4u : batch - done;
        const float *xb = x + (size_t)done * cols;
        float *yb = y + (size_t)done * rows;
        switch (nb) {
        case 1: hipLaunchKernelGGL(matvec_q8w<1>, grid, dim3(kThreads), 0, s, wq, rows, nblk, xb, yb, status); break;
        case 2: hipLaunchKernelGGL(matvec_q8w<2>, grid, dim3(kThreads), 0, s, wq, rows, nblk, xb, yb, status); break;
        case 3: hipLaunchKernelGGL(matvec_q8w<3>, grid, dim3(kThreads), 0, s, wq, rows, nblk, xb, yb, status); break;
        default: hipLaunchKernelGGL(matvec_q8w<4>, grid, dim3(kThreads), 0, s, wq, rows, nblk, xb, yb, status); break;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        done += nb;
    }
    return hipSuccess;
}
