/*
 * kq_dequant.hip — GGUF block dequantization to fp32 on gfx950.
 *
 * Restates kq_decode_one_block / kq_dequantize_blocks_f32
 * (src/kq_numeric.c:176-359) for F32, BF16, Q5_1, Q8_0, Q4_K, Q5_K and
 * IQ4_NL, and the GGML Q6_K layout (absent from the reference). Results are bit-identical to the CPU decode:
 * every scale product and subtraction is a separately rounded binary32
 * operation in the reference's order (this file builds with
 * -ffp-contract=off), and the f16 scales convert exactly.
 *
 * HBM layout and traffic: the packed blocks are streamed once and the fp32
 * output (4 B per weight) is written once with 16-byte stores; the output is
 * 3.8-7.1x the input, so the kernel is write-bandwidth bound. Each lane
 * produces 4 consecutive outputs; a 64-lane wave covers one 256-weight
 * K-quant block or eight Q8_0 blocks per step (1 KiB of contiguous output).
 */
#include "kq_device.h"
#include "kq_launch.h"

namespace {

constexpr int kThreads = 256;
constexpr uint64_t kMaxBlocks = 256 * 16;

__device__ __forceinline__ void store4(float *out, float a, float b, float c, float d) {
    *(float4 *)out = make_float4(a, b, c, d);
}

/* Q4_K: 144 B -> 256 floats. Lane l writes outputs 4l..4l+3: group g = l/16;
 * the first 8 lanes of a group take low nibbles (sub-block 2g), the next 8
 * take high nibbles (sub-block 2g+1) of qs[32g .. 32g+31]. */
__global__ __launch_bounds__(kThreads) void dequant_q4k(const uint8_t *__restrict__ packed,
                                                        uint64_t blocks, float *__restrict__ out,
                                                        uint32_t *status) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t wave = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
    const uint64_t nwaves = ((uint64_t)gridDim.x * kThreads) >> 6;
    const uint32_t g = lane >> 4, j = (lane & 15u) * 4u;
    const bool high = j >= 32u;
    const uint32_t sub = 2u * g + (high ? 1u : 0u);
    const uint32_t qoff = 16u + 32u * g + (high ? j - 32u : j);
    bool bad = false;
    for (uint64_t blk = wave; blk < blocks; blk += nwaves) {
        const uint8_t *p = packed + blk * 144u;
        const uint4 hd = *(const uint4 *)p;
        const uint32_t q = *(const uint32_t *)(p + qoff);
        const float d = kq_f16_to_f32(hd.x & 0xffffu);
        const float dmin = kq_f16_to_f32(hd.x >> 16);
        bad |= !kq_isfinite(d) || !kq_isfinite(dmin);
        uint32_t sc, mn;
        kq_k_scale(sub, hd.y, hd.z, hd.w, &sc, &mn);
        const float ds = d * (float)sc;
        const float dm = dmin * (float)mn;
        const uint32_t c = high ? (q >> 4) & 0x0f0f0f0fu : q & 0x0f0f0f0fu;
        store4(out + blk * 256u + 4u * lane,
               ds * (float)(c & 0xffu) - dm, ds * (float)((c >> 8) & 0xffu) - dm,
               ds * (float)((c >> 16) & 0xffu) - dm, ds * (float)(c >> 24) - dm);
    }
    if (bad) kq_flag(status, KQ_DEV_MALFORMED);
}

/* Q8_0: 34 B -> 32 floats. A wave step covers 8 blocks; lane l handles block
 * l/8, codes 4*(l%8) .. +3: y = (float)int8 * d. */
__global__ __launch_bounds__(kThreads) void dequant_q8_0(const uint8_t *__restrict__ packed,
                                                         uint64_t blocks, float *__restrict__ out,
                                                         uint32_t *status) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t wave = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
    const uint64_t nwaves = ((uint64_t)gridDim.x * kThreads) >> 6;
    const uint8_t *end = packed + blocks * 34u;
    bool bad = false;
    for (uint64_t step = wave; step * 8u < blocks; step += nwaves) {
        const uint64_t blk = step * 8u + (lane >> 3);
        if (blk < blocks) {
            const uint8_t *p = packed + blk * 34u;
            const float d = kq_f16_to_f32(*(const uint16_t *)p);
            bad |= !kq_isfinite(d);
            const uint32_t c = kq_load4_u2a_end(p + 2u + 4u * (lane & 7u), end);
            store4(out + blk * 32u + 4u * (lane & 7u),
                   (float)(int8_t)(c & 0xffu) * d, (float)(int8_t)((c >> 8) & 0xffu) * d,
                   (float)(int8_t)((c >> 16) & 0xffu) * d, (float)(int8_t)(c >> 24) * d);
        }
    }
    if (bad) kq_flag(status, KQ_DEV_MALFORMED);
}

/* Q6_K: 210 B -> 256 floats (GGML block_q6_K: ql[128] @0, qh[64] @128,
 * int8 sc[16] @192, f16 d @208). Lane l writes outputs o = 4l..4l+3 of half
 * n = l/32, quarter = (l/8)%4, position 4*(l%8) within the quarter:
 * q = (nibble of ql) | (2 bits of qh) << 4, y = (d * sc[o/16]) * (q - 32). */
__global__ __launch_bounds__(kThreads) void dequant_q6k(const uint8_t *__restrict__ packed,
                                                        uint64_t blocks, float *__restrict__ out,
                                                        uint32_t *status) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t wave = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
    const uint64_t nwaves = ((uint64_t)gridDim.x * kThreads) >> 6;
    const uint32_t n = lane >> 5, quarter = (lane >> 3) & 3u, l0 = 4u * (lane & 7u);
    const uint32_t ql_off = 64u * n + l0 + ((quarter & 1u) ? 32u : 0u);
    const uint32_t nib_shift = quarter >= 2u ? 4u : 0u;
    const uint32_t qh_off = 128u + 32u * n + l0;
    const uint32_t sc_off = 192u + (lane >> 2);
    bool bad = false;
    for (uint64_t blk = wave; blk < blocks; blk += nwaves) {
        const uint8_t *p = packed + blk * 210u;
        const float d = kq_f16_to_f32(*(const uint16_t *)(p + 208u));
        bad |= !kq_isfinite(d);
        const uint32_t ql = kq_load4_u2a(p + ql_off);
        const uint32_t qh = kq_load4_u2a(p + qh_off);
        const float ds = d * (float)(int8_t)p[sc_off];
        const uint32_t c = ((ql >> nib_shift) & 0x0f0f0f0fu) |
                           (((qh >> (2u * quarter)) & 0x03030303u) << 4);
        store4(out + blk * 256u + 4u * lane,
               ds * (float)((int)(c & 0xffu) - 32), ds * (float)((int)((c >> 8) & 0xffu) - 32),
               ds * (float)((int)((c >> 16) & 0xffu) - 32), ds * (float)((int)(c >> 24) - 32));
    }
    if (bad) kq_flag(status, KQ_DEV_MALFORMED);
}

/* Q5_K: 176 B -> 256 floats (d, dmin, scales @0, qh[32] @16, qs[128] @48;
 * src/kq_numeric.c:223-277). Lane l writes outputs 4l..4l+3 as in dequant_q4k,
 * the code gaining 16 from bit 2g (low nibbles) or 2g+1 (high nibbles) of
 * qh[i], i the position within the 32-weight sub-block. */
__global__ __launch_bounds__(kThreads) void dequant_q5k(const uint8_t *__restrict__ packed,
                                                        uint64_t blocks, float *__restrict__ out,
                                                        uint32_t *status) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t wave = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
    const uint64_t nwaves = ((uint64_t)gridDim.x * kThreads) >> 6;
    const uint32_t g = lane >> 4, j = (lane & 15u) * 4u;
    const bool high = j >= 32u;
    const uint32_t i = high ? j - 32u : j;
    const uint32_t sub = 2u * g + (high ? 1u : 0u);
    const uint32_t qoff = 48u + 32u * g + i, hoff = 16u + i;
    bool bad = false;
    for (uint64_t blk = wave; blk < blocks; blk += nwaves) {
        const uint8_t *p = packed + blk * 176u;
        const uint4 hd = *(const uint4 *)p;
        const uint32_t q = *(const uint32_t *)(p + qoff);
        const uint32_t h = *(const uint32_t *)(p + hoff);
        const float d = kq_f16_to_f32(hd.x & 0xffffu);
        const float dmin = kq_f16_to_f32(hd.x >> 16);
        bad |= !kq_isfinite(d) || !kq_isfinite(dmin);
        uint32_t sc, mn;
        kq_k_scale(sub, hd.y, hd.z, hd.w, &sc, &mn);
        const float ds = d * (float)sc;
        const float dm = dmin * (float)mn;
        const uint32_t c = ((high ? q >> 4 : q) & 0x0f0f0f0fu) |
                           (((h >> sub) & 0x01010101u) << 4);
        store4(out + blk * 256u + 4u * lane,
               ds * (float)(c & 0xffu) - dm, ds * (float)((c >> 8) & 0xffu) - dm,
               ds * (float)((c >> 16) & 0xffu) - dm, ds * (float)(c >> 24) - dm);
    }
    if (bad) kq_flag(status, KQ_DEV_MALFORMED);
}

/* bit j of the low 4 bits of n into bit 8j */
__device__ __forceinline__ uint32_t spread4(uint32_t n) {
    return ((n & 15u) * 0x00204081u) & 0x01010101u;
}

/* Q5_1: 24 B -> 32 floats (f16 d, f16 m, qh u32, qs[16]; src/kq_numeric.c:
 * 190-209). A wave step covers 8 blocks; lane l handles block l/8: j = l%8
 * below 4 takes the low nibbles of qs[4j..4j+3] (outputs 4j..), from 4 the
 * high nibbles of qs[4(j-4)..] (outputs 16 + 4(j-4)..); the code's bit 4 is
 * bit (output index) of qh. y = code * d + m. */
__global__ __launch_bounds__(kThreads) void dequant_q5_1(const uint8_t *__restrict__ packed,
                                                         uint64_t blocks, float *__restrict__ out,
                                                         uint32_t *status) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t wave = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
    const uint64_t nwaves = ((uint64_t)gridDim.x * kThreads) >> 6;
    const uint32_t j = lane & 7u, k = j & 3u;
    const bool high = j >= 4u;
    const uint32_t o = (high ? 16u : 0u) + 4u * k; /* first output of the lane */
    bool bad = false;
    for (uint64_t step = wave; step * 8u < blocks; step += nwaves) {
        const uint64_t blk = step * 8u + (lane >> 3);
        if (blk < blocks) {
            const uint8_t *p = packed + blk * 24u;
            const uint32_t dm = *(const uint32_t *)p;
            const uint32_t qh = *(const uint32_t *)(p + 4u);
            const uint32_t q = *(const uint32_t *)(p + 8u + 4u * k);
            const float d = kq_f16_to_f32(dm & 0xffffu);
            const float m = kq_f16_to_f32(dm >> 16);
            bad |= !kq_isfinite(d) || !kq_isfinite(m);
            const uint32_t c = ((high ? q >> 4 : q) & 0x0f0f0f0fu) | (spread4(qh >> o) << 4);
            store4(out + blk * 32u + o, (float)(c & 0xffu) * d + m,
                   (float)((c >> 8) & 0xffu) * d + m, (float)((c >> 16) & 0xffu) * d + m,
                   (float)(c >> 24) * d + m);
        }
    }
    if (bad) kq_flag(status, KQ_DEV_MALFORMED);
}

/* IQ4_NL: 18 B -> 32 floats (f16 d, qs[16]; src/kq_numeric.c:278-292):
 * y = d * T[nibble]. Lanes as in dequant_q5_1; the table bytes come from
 * v_perm_b32 over T (as int8) packed in four dwords. */
constexpr uint32_t kIq4S0 = 0xbfad9881u; /* T[0..3] as int8 bytes */
constexpr uint32_t kIq4S1 = 0xf6eaddcfu; /* T[4..7] */
constexpr uint32_t kIq4S2 = 0x26190d01u; /* T[8..11] */
constexpr uint32_t kIq4S3 = 0x71594535u; /* T[12..15] */

__global__ __launch_bounds__(kThreads) void dequant_iq4nl(const uint8_t *__restrict__ packed,
                                                          uint64_t blocks, float *__restrict__ out,
                                                          uint32_t *status) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t wave = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
    const uint64_t nwaves = ((uint64_t)gridDim.x * kThreads) >> 6;
    const uint32_t j = lane & 7u, k = j & 3u;
    const bool high = j >= 4u;
    const uint32_t o = (high ? 16u : 0u) + 4u * k;
    const uint8_t *end = packed + blocks * 18u;
    bool bad = false;
    for (uint64_t step = wave; step * 8u < blocks; step += nwaves) {
        const uint64_t blk = step * 8u + (lane >> 3);
        if (blk < blocks) {
            const uint8_t *p = packed + blk * 18u;
            const float d = kq_f16_to_f32(*(const uint16_t *)p);
            bad |= !kq_isfinite(d);
            const uint32_t q = kq_load4_u2a_end(p + 2u + 4u * k, end);
            const uint32_t n = (high ? q >> 4 : q) & 0x0f0f0f0fu;
            const uint32_t sel = n & 0x07070707u;
            const uint32_t a = __builtin_amdgcn_perm(kIq4S1, kIq4S0, sel);
            const uint32_t b = __builtin_amdgcn_perm(kIq4S3, kIq4S2, sel);
            const uint32_t msk = ((n >> 3) & 0x01010101u) * 0xffu;
            const uint32_t t = (a & ~msk) | (b & msk);
            store4(out + blk * 32u + o, d * (float)(int8_t)(t & 0xffu),
                   d * (float)(int8_t)((t >> 8) & 0xffu), d * (float)(int8_t)((t >> 16) & 0xffu),
                   d * (float)(int8_t)(t >> 24));
        }
    }
    if (bad) kq_flag(status, KQ_DEV_MALFORMED);
}

/* F32 (bit copy) and BF16 (bits << 16): one element per block
 * (src/kq_numeric.c:182-189). */
__global__ __launch_bounds__(kThreads) void dequant_f32(const uint32_t *__restrict__ in,
                                                        uint64_t n, float *__restrict__ out) {
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * kThreads)
        out[i] = __uint_as_float(in[i]);
}

__global__ __launch_bounds__(kThreads) void dequant_bf16(const uint16_t *__restrict__ in,
                                                         uint64_t n, float *__restrict__ out) {
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * kThreads)
        out[i] = __uint_as_float((uint32_t)in[i] << 16);
}

__global__ __launch_bounds__(kThreads) void expf_kernel(const float *__restrict__ in, uint64_t n,
                                                        float *__restrict__ out) {
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * kThreads)
        out[i] = kq_expf(in[i]);
}

int grid_for(uint64_t waves) {
    uint64_t b = (waves + (kThreads / 64) - 1) / (kThreads / 64);
    if (b > kMaxBlocks) b = kMaxBlocks;
    return b < 1 ? 1 : (int)b;
}

}  // namespace

extern "C" hipError_t kq_launch_dequant(uint32_t type, const void *packed, uint64_t blocks,
                                        float *out, uint32_t *status, hipStream_t stream) {
    const uint8_t *p = (const uint8_t *)packed;
    switch (type) {
    case KQ_LAUNCH_Q4_K:
        hipLaunchKernelGGL(dequant_q4k, dim3(grid_for(blocks)), dim3(kThreads), 0, stream, p,
                           blocks, out, status);
        break;
    case KQ_LAUNCH_Q8_0:
        hipLaunchKernelGGL(dequant_q8_0, dim3(grid_for((blocks + 7) / 8)), dim3(kThreads), 0,
                           stream, p, blocks, out, status);
        break;
    case KQ_LAUNCH_Q6_K:
        hipLaunchKernelGGL(dequant_q6k, dim3(grid_for(blocks)), dim3(kThreads), 0, stream, p,
                           blocks, out, status);
        break;
    case KQ_LAUNCH_Q5_K:
        hipLaunchKernelGGL(dequant_q5k, dim3(grid_for(blocks)), dim3(kThreads), 0, stream, p,
                           blocks, out, status);
        break;
    case KQ_LAUNCH_Q5_1:
        hipLaunchKernelGGL(dequant_q5_1, dim3(grid_for((blocks + 7) / 8)), dim3(kThreads), 0,
                           stream, p, blocks, out, status);
        break;
    case KQ_LAUNCH_IQ4_NL:
        hipLaunchKernelGGL(dequant_iq4nl, dim3(grid_for((blocks + 7) / 8)), dim3(kThreads), 0,
                           stream, p, blocks, out, status);
        break;
    case KQ_LAUNCH_F32:
        hipLaunchKernelGGL(dequant_f32, dim3(grid_for((blocks + 255) / 256 * 4)), dim3(kThreads),
                           0, stream, (const uint32_t *)packed, blocks, out);
        break;
    case KQ_LAUNCH_BF16:
        hipLaunchKernelGGL(dequant_bf16, dim3(grid_for((blocks + 255) / 256 * 4)), dim3(kThreads),
                           0, stream, (const uint16_t *)packed, blocks, out);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_expf(const float *in, uint64_t n, float *out,
                                     hipStream_t stream) {
    uint64_t blocks = (n + kThreads - 1) / kThreads;
    if (blocks > 65536u) blocks = 65536u;
    if (blocks < 1u) blocks = 1u;
    hipLaunchKernelGGL(expf_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, in, n, out);
    return hipGetLastError();
}
