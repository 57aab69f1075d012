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

/* 4 floats at byte offset o of the output buffer; stores at or past its
 * end are dropped by the hardware */
__device__ __forceinline__ void store4(KqBuf ob, uint32_t o, float a, float b, float c, float d) {
    kq_u32x4 v = {__float_as_uint(a), __float_as_uint(b), __float_as_uint(c), __float_as_uint(d)};
    __builtin_amdgcn_raw_buffer_store_b128(v, ob.r, (int)o, 0, 0);
}

/*
 * Block decoders. A wave step is one K-quant block (64 lanes x 4 outputs)
 * or eight 32-weight blocks (8 lanes each). load() only requests the
 * step's bytes (raw buffer loads, no branch: a step past the end reads
 * whatever lies at or past the last block and is never emitted), emit()
 * decodes and stores. Each decoder's arithmetic is the reference's
 * (src/kq_numeric.c:176-295), separately rounded in its order.
 */

/* Q4_K: 144 B -> 256 floats. Lane l writes outputs 4l..4l+3: group g = l/16;
 * the first 8 lanes of a group take low nibbles (sub-block 2g), the next 8
 * take high nibbles (sub-block 2g+1) of qs[32g .. 32g+31]. */
struct DeqQ4K {
    static constexpr uint32_t kBytes = 144u, kPerStep = 1u, kOut = 256u;
    struct Raw {
        uint4 hd;
        uint32_t q;
    };
    uint32_t lane, sub, qoff;
    bool high;
    __device__ void setup(uint32_t l) {
        lane = l;
        const uint32_t g = l >> 4, j = (l & 15u) * 4u;
        high = j >= 32u;
        sub = 2u * g + (high ? 1u : 0u);
        qoff = 16u + 32u * g + (high ? j - 32u : j);
    }
    __device__ Raw load(KqBuf b, uint32_t s) const {
        const uint32_t o = s * kBytes;
        Raw r;
        r.hd = kq_ld128(b, o, 0u);
        r.q = kq_ld32(b, o + qoff, 0u);
        return r;
    }
    __device__ void emit(const Raw &r, uint32_t s, bool valid, KqBuf out, bool &bad) const {
        const float d = kq_f16_to_f32(r.hd.x & 0xffffu);
        const float dmin = kq_f16_to_f32(r.hd.x >> 16);
        bad |= valid && (!kq_isfinite(d) || !kq_isfinite(dmin));
        uint32_t sc, mn;
        kq_k_scale(sub, r.hd.y, r.hd.z, r.hd.w, &sc, &mn);
        const float ds = d * (float)sc;
        const float dm = dmin * (float)mn;
        const uint32_t c = high ? (r.q >> 4) & 0x0f0f0f0fu : r.q & 0x0f0f0f0fu;
        store4(out, (s * 256u + 4u * lane) * 4u,
               ds * (float)(c & 0xffu) - dm, ds * (float)((c >> 8) & 0xffu) - dm,
               ds * (float)((c >> 16) & 0xffu) - dm, ds * (float)(c >> 24) - dm);
    }
};

/* Q5_K: 176 B -> 256 floats (d, dmin, scales @0, qh[32] @16, qs[128] @48;
 * src/kq_numeric.c:223-277). Lanes as in Q4_K, the code gaining 16 from bit
 * 2g (low nibbles) or 2g+1 (high nibbles) of qh[i], i the position within
 * the 32-weight sub-block. */
struct DeqQ5K {
    static constexpr uint32_t kBytes = 176u, kPerStep = 1u, kOut = 256u;
    struct Raw {
        uint4 hd;
        uint32_t q, h;
    };
    uint32_t lane, sub, qoff, hoff;
    bool high;
    __device__ void setup(uint32_t l) {
        lane = l;
        const uint32_t g = l >> 4, j = (l & 15u) * 4u;
        high = j >= 32u;
        const uint32_t i = high ? j - 32u : j;
        sub = 2u * g + (high ? 1u : 0u);
        qoff = 48u + 32u * g + i;
        hoff = 16u + i;
    }
    __device__ Raw load(KqBuf b, uint32_t s) const {
        const uint32_t o = s * kBytes;
        Raw r;
        r.hd = kq_ld128(b, o, 0u);
        r.q = kq_ld32(b, o + qoff, 0u);
        r.h = kq_ld32(b, o + hoff, 0u);
        return r;
    }
    __device__ void emit(const Raw &r, uint32_t s, bool valid, KqBuf out, bool &bad) const {
        const float d = kq_f16_to_f32(r.hd.x & 0xffffu);
        const float dmin = kq_f16_to_f32(r.hd.x >> 16);
        bad |= valid && (!kq_isfinite(d) || !kq_isfinite(dmin));
        uint32_t sc, mn;
        kq_k_scale(sub, r.hd.y, r.hd.z, r.hd.w, &sc, &mn);
        const float ds = d * (float)sc;
        const float dm = dmin * (float)mn;
        const uint32_t c = ((high ? r.q >> 4 : r.q) & 0x0f0f0f0fu) |
                           (((r.h >> sub) & 0x01010101u) << 4);
        store4(out, (s * 256u + 4u * lane) * 4u,
               ds * (float)(c & 0xffu) - dm, ds * (float)((c >> 8) & 0xffu) - dm,
               ds * (float)((c >> 16) & 0xffu) - dm, ds * (float)(c >> 24) - dm);
    }
};

/* Q6_K: 210 B -> 256 floats (GGML block_q6_K: ql[128] @0, qh[64] @128,
 * int8 sc[16] @192, f16 d @208). Lane l writes outputs o = 4l..4l+3 of half
 * n = l/32, quarter = (l/8)%4, position 4*(l%8) within the quarter:
 * q = (nibble of ql) | (2 bits of qh) << 4, y = (d * sc[o/16]) * (q - 32).
 * A block starting 2 mod 4 is read through aligned 8-byte windows. */
struct DeqQ6K {
    static constexpr uint32_t kBytes = 210u, kPerStep = 1u, kOut = 256u;
    struct Raw {
        kq_u32x2 ql, qh;
        uint32_t sc, d, sh;
    };
    uint32_t lane, ql_off, qh_off, sc_off, nib_shift, quarter;
    __device__ void setup(uint32_t l) {
        lane = l;
        const uint32_t n = l >> 5, l0 = 4u * (l & 7u);
        quarter = (l >> 3) & 3u;
        ql_off = 64u * n + l0 + ((quarter & 1u) ? 32u : 0u);
        nib_shift = quarter >= 2u ? 4u : 0u;
        qh_off = 128u + 32u * n + l0;
        sc_off = 192u + (l >> 2);
    }
    __device__ Raw load(KqBuf b, uint32_t s) const {
        const uint32_t o = s * kBytes;
        Raw r;
        r.sh = o & 3u;
        r.ql = kq_ld64(b, o + ql_off - r.sh, 0u);
        r.qh = kq_ld64(b, o + qh_off - r.sh, 0u);
        r.sc = kq_ld32(b, (o + sc_off) & ~3u, 0u) >> (8u * ((o + sc_off) & 3u));
        r.d = kq_ld16(b, o + 208u, 0u);
        return r;
    }
    __device__ void emit(const Raw &r, uint32_t s, bool valid, KqBuf out, bool &bad) const {
        const float d = kq_f16_to_f32(r.d);
        bad |= valid && !kq_isfinite(d);
        const uint32_t ql = kq_align2(r.ql.y, r.ql.x, r.sh);
        const uint32_t qh = kq_align2(r.qh.y, r.qh.x, r.sh);
        const float ds = d * (float)(int8_t)(r.sc & 0xffu);
        const uint32_t c = ((ql >> nib_shift) & 0x0f0f0f0fu) |
                           (((qh >> (2u * quarter)) & 0x03030303u) << 4);
        store4(out, (s * 256u + 4u * lane) * 4u,
               ds * (float)((int)(c & 0xffu) - 32), ds * (float)((int)((c >> 8) & 0xffu) - 32),
               ds * (float)((int)((c >> 16) & 0xffu) - 32), ds * (float)((int)(c >> 24) - 32));
    }
};

/* Q8_0: 34 B -> 32 floats. A step covers 8 blocks; lane l handles block
 * l/8, codes 4*(l%8) .. +3 (an aligned 8-byte window): y = (float)int8 * d. */
struct DeqQ8 {
    static constexpr uint32_t kBytes = 34u, kPerStep = 8u, kOut = 32u;
    struct Raw {
        kq_u32x2 w;
        uint32_t d, sh;
    };
    uint32_t lane, k;
    __device__ void setup(uint32_t l) {
        lane = l;
        k = l & 7u;
    }
    __device__ Raw load(KqBuf b, uint32_t s) const {
        const uint32_t o = (8u * s + (lane >> 3)) * kBytes;
        const uint32_t c = o + 2u + 4u * k;
        Raw r;
        r.sh = c & 3u;
        r.w = kq_ld64(b, c - r.sh, 0u);
        r.d = kq_ld16(b, o, 0u);
        return r;
    }
    __device__ void emit(const Raw &r, uint32_t s, bool valid, KqBuf out, bool &bad) const {
        const uint32_t blk = 8u * s + (lane >> 3);
        const float d = kq_f16_to_f32(r.d);
        bad |= valid && !kq_isfinite(d);
        const uint32_t c = kq_align2(r.w.y, r.w.x, r.sh);
        store4(out, (blk * 32u + 4u * k) * 4u,
               (float)(int8_t)(c & 0xffu) * d, (float)(int8_t)((c >> 8) & 0xffu) * d,
               (float)(int8_t)((c >> 16) & 0xffu) * d, (float)(int8_t)(c >> 24) * d);
    }
};

/* bit j of the low 4 bits of n into bit 8j */
__device__ __forceinline__ uint32_t spread4(uint32_t n) {
    return ((n & 15u) * 0x00204081u) & 0x01010101u;
}

/* Q5_1: 24 B -> 32 floats (f16 d, f16 m, qh u32, qs[16]; src/kq_numeric.c:
 * 190-209). y[i] = (q_i | bit i of qh << 4) * d + m (low nibbles i < 16,
 * high nibbles i >= 16). A step covers 8 blocks; lane l handles block
 * l/8, outputs o .. o+3 with o = 16*(j/4) + 4*(j%4), j = l%8. */
struct DeqQ51 {
    static constexpr uint32_t kBytes = 24u, kPerStep = 8u, kOut = 32u;
    struct Raw {
        uint32_t dm, qh, q;
    };
    uint32_t lane, k, o;
    bool high;
    __device__ void setup(uint32_t l) {
        lane = l;
        const uint32_t j = l & 7u;
        k = j & 3u;
        high = j >= 4u;
        o = (high ? 16u : 0u) + 4u * k;
    }
    __device__ Raw load(KqBuf b, uint32_t s) const {
        const uint32_t p = (8u * s + (lane >> 3)) * kBytes;
        Raw r;
        r.dm = kq_ld32(b, p, 0u);
        r.qh = kq_ld32(b, p + 4u, 0u);
        r.q = kq_ld32(b, p + 8u + 4u * k, 0u);
        return r;
    }
    __device__ void emit(const Raw &r, uint32_t s, bool valid, KqBuf out, bool &bad) const {
        const uint32_t blk = 8u * s + (lane >> 3);
        const float d = kq_f16_to_f32(r.dm & 0xffffu);
        const float m = kq_f16_to_f32(r.dm >> 16);
        bad |= valid && (!kq_isfinite(d) || !kq_isfinite(m));
        const uint32_t c = ((high ? r.q >> 4 : r.q) & 0x0f0f0f0fu) | (spread4(r.qh >> o) << 4);
        store4(out, (blk * 32u + o) * 4u, (float)(c & 0xffu) * d + m,
               (float)((c >> 8) & 0xffu) * d + m, (float)((c >> 16) & 0xffu) * d + m,
               (float)(c >> 24) * d + m);
    }
};

/* IQ4_NL: 18 B -> 32 floats (f16 d, qs[16]; src/kq_numeric.c:278-292):
 * y[i] = d * T[nibble], T the fixed 16-entry non-linear table (kvalues of
 * the IQ4_NL format), low nibbles i < 16, high nibbles i >= 16. The table
 * lookup is two byte permutes over the table packed as int8, selected by
 * the nibble's top bit. */
constexpr uint32_t kIq4S0 = 0xbfad9881u; /* T[0..3] as int8 bytes */
constexpr uint32_t kIq4S1 = 0xf6eaddcfu; /* T[4..7] */
constexpr uint32_t kIq4S2 = 0x26190d01u; /* T[8..11] */
constexpr uint32_t kIq4S3 = 0x71594535u; /* T[12..15] */

struct DeqIQ4NL {
    static constexpr uint32_t kBytes = 18u, kPerStep = 8u, kOut = 32u;
    struct Raw {
        kq_u32x2 w;
        uint32_t d, sh;
    };
    uint32_t lane, k, o;
    bool high;
    __device__ void setup(uint32_t l) {
        lane = l;
        const uint32_t j = l & 7u;
        k = j & 3u;
        high = j >= 4u;
        o = (high ? 16u : 0u) + 4u * k;
    }
    __device__ Raw load(KqBuf b, uint32_t s) const {
        const uint32_t p = (8u * s + (lane >> 3)) * kBytes;
        const uint32_t c = p + 2u + 4u * k;
        Raw r;
        r.sh = c & 3u;
        r.w = kq_ld64(b, c - r.sh, 0u);
        r.d = kq_ld16(b, p, 0u);
        return r;
    }
    __device__ void emit(const Raw &r, uint32_t s, bool valid, KqBuf out, bool &bad) const {
        const uint32_t blk = 8u * s + (lane >> 3);
        const float d = kq_f16_to_f32(r.d);
        bad |= valid && !kq_isfinite(d);
        const uint32_t q = kq_align2(r.w.y, r.w.x, r.sh);
        const uint32_t n = (high ? q >> 4 : q) & 0x0f0f0f0fu;
        const uint32_t sel = n & 0x07070707u;
        const uint32_t a = __builtin_amdgcn_perm(kIq4S1, kIq4S0, sel);
        const uint32_t b = __builtin_amdgcn_perm(kIq4S3, kIq4S2, sel);
        const uint32_t msk = ((n >> 3) & 0x01010101u) * 0xffu;
        const uint32_t t = (a & ~msk) | (b & msk);
        store4(out, (blk * 32u + o) * 4u, d * (float)(int8_t)(t & 0xffu),
               d * (float)(int8_t)((t >> 8) & 0xffu), d * (float)(int8_t)((t >> 16) & 0xffu),
               d * (float)(int8_t)(t >> 24));
    }
};

/* Each wave takes kUnroll consecutive steps at a time and requests all of
 * their bytes before decoding the first, so every wave keeps kUnroll steps
 * of loads in flight. The buffer's byte count is rounded up to a dword so
 * that no dword of the last block straddles it. */
constexpr uint32_t kUnroll = 4u;

template <class D>
__global__ __launch_bounds__(kThreads) void dequant_blocks(const uint8_t *__restrict__ packed,
                                                           uint32_t blocks,
                                                           float *__restrict__ out,
                                                           uint32_t *status) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane((blockIdx.x * kThreads + threadIdx.x) >> 6);
    const uint32_t nwaves = (gridDim.x * kThreads) >> 6;
    const uint32_t steps = (blocks + D::kPerStep - 1u) / D::kPerStep;
    const KqBuf b = kq_buf(packed, (blocks * D::kBytes + 3u) & ~3u);
    /* outputs of blocks past the end fall outside this buffer */
    const KqBuf ob = kq_buf(out, blocks * D::kOut * 4u);
    D dec;
    dec.setup(lane);
    bool bad = false;
    for (uint32_t s0 = wave * kUnroll; s0 < steps; s0 += nwaves * kUnroll) {
        typename D::Raw r[kUnroll];
#pragma unroll
        for (uint32_t u = 0; u < kUnroll; ++u) r[u] = dec.load(b, s0 + u);
#pragma unroll
        for (uint32_t u = 0; u < kUnroll; ++u) {
            const uint32_t s = s0 + u;
            const bool valid = D::kPerStep == 1u ? s < steps : 8u * s + (lane >> 3) < blocks;
            dec.emit(r[u], s, valid, ob, bad);
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

/* One launch per chunk of at most 1 GiB of packed bytes and 2 GiB of
 * output (a multiple of 8 blocks, so every chunk starts 16-byte aligned
 * relative to the input): offsets inside a launch stay 32-bit. */
template <class D>
hipError_t launch_blocks(const uint8_t *p, uint64_t blocks, float *out, uint32_t *status,
                         hipStream_t stream) {
    constexpr uint64_t kIn = (1ull << 30) / D::kBytes, kOutMax = (1ull << 31) / (D::kOut * 4u);
    constexpr uint64_t kChunk = (kIn < kOutMax ? kIn : kOutMax) & ~7ull;
    constexpr uint64_t kOut = D::kOut;
    for (uint64_t done = 0; done < blocks; done += kChunk) {
        const uint64_t n = blocks - done < kChunk ? blocks - done : kChunk;
        const uint64_t steps = (n + D::kPerStep - 1u) / D::kPerStep;
        hipLaunchKernelGGL(dequant_blocks<D>, dim3(grid_for((steps + kUnroll - 1u) / kUnroll)),
                           dim3(kThreads), 0, stream, p + done * D::kBytes, (uint32_t)n,
                           out + done * kOut, status);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

extern "C" hipError_t kq_launch_dequant(uint32_t type, const void *packed, uint64_t blocks,
                                        float *out, uint32_t *status, hipStream_t stream) {
    const uint8_t *p = (const uint8_t *)packed;
    switch (type) {
    case KQ_LAUNCH_Q4_K: return launch_blocks<DeqQ4K>(p, blocks, out, status, stream);
    case KQ_LAUNCH_Q8_0: return launch_blocks<DeqQ8>(p, blocks, out, status, stream);
    case KQ_LAUNCH_Q6_K: return launch_blocks<DeqQ6K>(p, blocks, out, status, stream);
    case KQ_LAUNCH_Q5_K: return launch_blocks<DeqQ5K>(p, blocks, out, status, stream);
    case KQ_LAUNCH_Q5_1: return launch_blocks<DeqQ51>(p, blocks, out, status, stream);
    case KQ_LAUNCH_IQ4_NL: return launch_blocks<DeqIQ4NL>(p, blocks, out, status, stream);
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
