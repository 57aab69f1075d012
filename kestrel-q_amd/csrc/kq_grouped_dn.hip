/*
 * kq_grouped_dn.hip — the prefill down pass of Q6_K experts: one
 * independent weight pipeline per wave at intermediate 256 (dn_q6k), one
 * per pair of waves at intermediate 512 (dn_q6k_pair, below), and the Q5_1
 * and Q8_0 down passes (dn_small_pair).
 *
 * The reference forms o = Wd a for every (token, selected expert) pair one
 * token at a time (src/kq_moe_qwen38.c:722-765 via
 * kq_weight_provider_linear_f32, src/kq_weight_provider.c:378-509). Here
 * every expert's down rows stream once for all of its tokens:
 *
 *   - The work is the gate/up pass's item list (one item per 16-token chunk
 *     of an expert, kq_grouped_gu.hip), each of ceil(hidden / 16) tiles of
 *     16 down rows. Every wave of the grid walks its own contiguous range
 *     of that tile sequence: no barrier, no shared state between waves.
 *   - A tile's 16 rows of intermediate / 256 Q6_K blocks are one contiguous
 *     byte range; the wave copies it into a private LDS slot with 16-byte
 *     LDS-DMA loads (1 KiB per instruction) while it multiplies the tile
 *     before, and reads the operand pieces from there.
 *   - The activation operand (16 positions x intermediate, hi + lo) lives
 *     in the wave's registers for a whole item: rows of the intermediate
 *     activations are split once per position by dn_stage, in the order
 *     the lanes read them.
 *
 * Arithmetic per 16-column Q6_K sub-block (the grouped pass's): exact codes
 * q - 32 in fp16, one 16x16x16 MFMA step each for the hi and lo parts of
 * the activations, the fp32 result scaled by d * sc.
 *
 * The LDS-DMA loads are issued from inline assembly and waited for with
 * s_waitcnt vmcnt(n), counting only this wave's loads issued after the
 * ones it needs (loads complete in order).
 */
#include "kq_launch.h"
#include "kq_device.h"
#include "kq_dma.h"

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef kq_i4v i4v;

constexpr uint32_t kT = 16;
constexpr uint32_t kShared = 0x80000000u; /* item flag: the shared expert */
constexpr int kBadRow = 0x7fffffff;

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ h2 byte_pair_lo(uint32_t m) {
    return as_h2(__builtin_amdgcn_perm(0x64646464u, m, 0x04010400u));
}
__device__ __forceinline__ h2 byte_pair_hi(uint32_t m) {
    return as_h2(__builtin_amdgcn_perm(0x64646464u, m, 0x04030402u));
}
__device__ __forceinline__ float half_bits(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
}

__device__ __forceinline__ uint32_t sload(const uint32_t *p) {
    const uint64_t a = (uint64_t)(uintptr_t)p;
    /* (readfirstlane returns int: zero-extend each half, never sign-extend) */
    const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a) |
                       ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32);
    uint32_t v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(u) : "memory");
    return v;
}

/* ------------------------------------------------------------------ */
/* per-position activation split, in lane order */

/* Staged rows: xh[p][K], xl[p][K] (fp16) and sig[p]. Column c = 256b +
 * 128n + 32q + 16h + 4g + e sits at index ((((g KB + b) 2 + n) 2 + h) 4 + q)
 * 4 + e of its row, so MFMA lane k-group g reads one contiguous run. */
struct DnStaged {
    _Float16 *xh, *xl;
    int *sig;
};
__device__ __forceinline__ DnStaged dn_staged_at(void *base, uint32_t npos, uint32_t k) {
    DnStaged s;
    uint8_t *p = (uint8_t *)base;
    s.xh = (_Float16 *)p;
    p += (size_t)npos * k * 2u;
    s.xl = (_Float16 *)p;
    p += (size_t)npos * k * 2u;
    s.sig = (int *)p;
    return s;
}
__device__ __forceinline__ uint32_t dn_index(uint32_t c, uint32_t kb) {
    const uint32_t e = c & 3u, g = (c >> 2) & 3u, h = (c >> 4) & 1u, q = (c >> 5) & 3u,
                   n = (c >> 7) & 1u, b = c >> 8;
    return ((((g * kb + b) * 2u + n) * 2u + h) * 4u + q) * 4u + e;
}

/* grid: one wave per position; k a multiple of 256 */
__global__ __launch_bounds__(64) void dn_stage(const float *__restrict__ X, uint32_t npos,
                                               uint32_t k, void *staged, uint32_t *status) {
    const DnStaged sx = dn_staged_at(staged, npos, k);
    const uint32_t p = blockIdx.x, lane = threadIdx.x;
    const float4 *row = (const float4 *)(X + (size_t)p * k);
    const uint32_t ng = k / 4u;
    float m = 0.0f;
    bool nf = false;
    for (uint32_t i = lane; i < ng; i += 64u) {
        const float4 v = row[i];
        nf |= !kq_isfinite(v.x) || !kq_isfinite(v.y) || !kq_isfinite(v.z) || !kq_isfinite(v.w);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const bool bad = __ballot(nf) != 0ull;
    /* largest magnitude into [2^14, 2^15) */
    int sig = 0;
    if (!bad && m > 0.0f) sig = 15 - __builtin_amdgcn_frexp_expf(m);
    if (bad) sig = kBadRow;
    for (uint32_t i = lane; i < ng; i += 64u) {
        const float4 v = row[i];
        const float a[4] = {v.x, v.y, v.z, v.w};
        _Float16 hi[4], lo[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float xs = bad ? 0.0f : ldexpf(a[c], sig);
            hi[c] = (_Float16)xs;
            lo[c] = (_Float16)(xs - (float)hi[c]);
        }
        const size_t o = (size_t)p * k + dn_index(4u * i, k / 256u);
        *(h4 *)(sx.xh + o) = h4{hi[0], hi[1], hi[2], hi[3]};
        *(h4 *)(sx.xl + o) = h4{lo[0], lo[1], lo[2], lo[3]};
    }
    if (lane == 0u) {
        sx.sig[p] = sig;
        /* a non-finite intermediate activation is a numeric failure */
        if (bad) kq_flag(status, KQ_DEV_NUMERIC);
    }
}

/* ------------------------------------------------------------------ */
/* the pass */

template <uint32_t KB>
struct DnShape {
    static constexpr uint32_t RB = 210u * KB;                /* row bytes */
    static constexpr uint32_t TB = kT * RB;                  /* tile bytes */
    static constexpr uint32_t IPT = (TB + 1023u) / 1024u;    /* loads per tile */
    static constexpr uint32_t SLOT = IPT * 1024u;
    /* one wave per SIMD: the activation operand alone takes 64 KB registers
     * per block, so each wave gets the whole register file, and the LDS
     * holds RING - 1 tiles in flight per wave */
    static constexpr uint32_t W = 4u;                        /* waves per workgroup */
    static constexpr uint32_t RING = KB == 1u ? 8u : 5u;     /* slots per wave */
    static constexpr uint32_t PD = RING - 1u;
    static_assert(W * RING * SLOT <= 160u * 1024u, "LDS");
};

struct DnArgs {
    const uint8_t *down, *sdown;  /* routed stack, shared matrix */
    const void *staged;           /* dn_stage output, positions 0 .. T*K + T - 1 */
    const float *act;             /* fused split: the activations [T*K + T][inter] */
    const uint32_t *posmax;       /* and each position's largest |act| (float bits) */
    const uint32_t *items, *n_items;
    uint32_t tokens, top_k, hidden, npos;
    float *out; /* [T*K + T][hidden] */
    uint32_t *status;
};

template <uint32_t KB>
__global__ __launch_bounds__(DnShape<KB>::W * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void dn_q6k(DnArgs a) {
    using S = DnShape<KB>;
    constexpr uint32_t KD = 256u * KB;
    __shared__ __align__(16) uint8_t slots[S::W][S::RING][S::SLOT];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t gw = blockIdx.x * S::W + w, nw = gridDim.x * S::W;
    const uint32_t nt = (a.hidden + kT - 1u) / kT; /* tiles per item */
    const uint64_t total = (uint64_t)(*a.n_items) * nt;
    const uint32_t lo = (uint32_t)(total * gw / nw), hi = (uint32_t)(total * (gw + 1u) / nw);
    if (lo >= hi) return;

    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t wbytes = a.hidden * S::RB;
    const uint32_t base_lds = lds_addr(&slots[w][0][0]);
    const uint8_t *myslots = &slots[w][0][0];

    /* the next tile to request */
    uint32_t iss_it = lo / nt, iss_tile = lo - (lo / nt) * nt, iss_slot = 0u;
    bool iss_new = true;
    i4v rw = {0, 0, 0, 0};
    auto issue = [&]() {
        if (iss_new) {
            iss_new = false;
            const uint32_t ex = sload(a.items + 2u * iss_it);
            rw = dma_rsrc((ex & kShared) ? a.sdown : a.down + (size_t)ex * wbytes, wbytes);
        }
        const uint32_t toff = iss_tile * S::TB;
#pragma unroll
        for (uint32_t q = 0; q < S::IPT; ++q) {
            /* bytes past the tile re-read its start (their slot bytes are
             * never read) */
            const uint32_t c = 64u * q + lane;
            dma16(rw, toff + (16u * c < S::TB ? 16u * c : 0u),
                  base_lds + iss_slot * S::SLOT + q * 1024u);
        }
        iss_slot = iss_slot + 1u == S::RING ? 0u : iss_slot + 1u;
        if (++iss_tile == nt) {
            iss_tile = 0u;
            ++iss_it;
            iss_new = true;
        }
    };

    const DnStaged sx = dn_staged_at(const_cast<void *>(a.staged), a.npos, KD);
    const KqBuf bxh = kq_buf(sx.xh, a.npos * KD * 2u), bxl = kq_buf(sx.xl, a.npos * KD * 2u);
    const KqBuf bsg = kq_buf(sx.sig, a.npos * 4u);
    const uint32_t tk = a.tokens * a.top_k;
    bool bad = false, malformed = false;

#pragma unroll
    for (uint32_t t = 0; t < S::PD; ++t)
        if (lo + t < hi) issue();

    /* the item being multiplied: activation operand of lane (j, g) (token
     * row j, k-group g), the scales of the four positions this lane's
     * results belong to */
    uint4 axh[KB][8], axl[KB][8]; /* 16-byte loads: h4 steps 2v and 2v + 1 */
    int sg[4];
    uint32_t cur = 0u, pos0 = 0u, count = 0u;
    auto enter = [&](uint32_t it) {
        cur = it;
        const uint32_t ex = sload(a.items + 2u * it), fc = sload(a.items + 2u * it + 1u);
        const uint32_t first = fc & 0xffffffu;
        count = fc >> 24;
        pos0 = (ex & kShared) ? tk + first : first;
        /* rows past the chunk read at 2^31, past the buffer */
        const uint32_t xo = j < count ? ((pos0 + j) * KD + g * (KD / 4u)) * 2u : 0x80000000u;
#pragma unroll
        for (uint32_t b = 0; b < KB; ++b)
#pragma unroll
            for (uint32_t v = 0; v < 8u; ++v) {
                axh[b][v] = kq_ld128(bxh, xo + (b * 8u + v) * 16u, 0u);
                axl[b][v] = kq_ld128(bxl, xo + (b * 8u + v) * 16u, 0u);
            }
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) {
            const uint32_t i = 4u * g + q;
            sg[q] = (int)kq_ld32(bsg, i < count ? (pos0 + i) * 4u : 0x80000000u, 0u);
        }
        wait_vm_all();
    };
    uint32_t ctile = lo - (lo / nt) * nt, cslot = 0u;
    enter(lo / nt);

    const h2 bias = h2{(_Float16)-1056.0f, (_Float16)-1056.0f}; /* 1024 + 32 */
    for (uint32_t tau = lo; tau < hi; ++tau) {
        if (ctile == nt) {
            ctile = 0u;
            enter(cur + 1u);
        }
        if (tau + S::PD < hi) issue();
        /* tile tau's loads have landed; those of the (at most PD) tiles
         * issued after it may still be in flight */
        const uint32_t after = hi - 1u - tau < S::PD ? hi - 1u - tau : S::PD;
        wait_after<S::IPT, S::PD>(after);
        const uint8_t *tile = myslots + cslot * S::SLOT;
        cslot = cslot + 1u == S::RING ? 0u : cslot + 1u;
        const uint32_t row0 = ctile * kT;
        ++ctile;

        f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t b = 0; b < KB; ++b) {
            /* block b of row j: 4-byte aligned windows, re-aligned by sh */
            const uint32_t o = j * S::RB + b * 210u;
            const uint32_t sh = o & 3u;
            const uint32_t *p = (const uint32_t *)(tile + (o - sh));
            auto win = [&](uint32_t off) { return kq_align2(p[off / 4u + 1u], p[off / 4u], sh); };
            const float d = half_bits(sh ? (p[52] >> 16) : p[52]);
            malformed |= !kq_isfinite(d);
            uint32_t sc[4];
#pragma unroll
            for (uint32_t k = 0; k < 4u; ++k) sc[k] = win(192u + 4u * k);
#pragma unroll
            for (uint32_t nh = 0; nh < 4u; ++nh) {
                const uint32_t n = nh >> 1, h = nh & 1u;
                const uint32_t oa = 64u * n + 16u * h + 4u * g;
                const uint32_t A = win(oa), B = win(oa + 32u);
                const uint32_t H = win(128u + 32u * n + 16u * h + 4u * g);
                uint32_t c[4];
                c[0] = (A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
                c[1] = (B & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
                c[2] = ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u);
                c[3] = ((B >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
#pragma unroll
                for (uint32_t q = 0; q < 4u; ++q) {
                    const uint32_t s = 8u * n + 2u * q + h; /* sub-block */
                    const h2 w0 = byte_pair_lo(c[q]) + bias, w1 = byte_pair_hi(c[q]) + bias;
                    const h4 bw = h4{w0.x, w0.y, w1.x, w1.y};
                    /* columns 128n + 32q + 16h + 4g .. +3 of block b */
                    const uint32_t ai = (n * 2u + h) * 4u + q;
                    const uint4 &xh = axh[b][ai >> 1], &xl = axl[b][ai >> 1];
                    const h4 ah = __builtin_bit_cast(h4, (ai & 1u) ? make_uint2(xh.z, xh.w) : make_uint2(xh.x, xh.y));
                    const h4 al = __builtin_bit_cast(h4, (ai & 1u) ? make_uint2(xl.z, xl.w) : make_uint2(xl.x, xl.y));
                    f4 t = {0.f, 0.f, 0.f, 0.f};
                    t = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bw, t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bw, t, 0, 0, 0);
                    const int8_t scv = (int8_t)((sc[s >> 2] >> (8u * (s & 3u))) & 0xffu);
                    const float ds = d * (float)scv;
#pragma unroll
                    for (int k = 0; k < 4; ++k) acc[k] = fmaf(ds, t[k], acc[k]);
                }
            }
        }
        /* D[token][row]: this lane holds row row0 + j of tokens 4g .. 4g+3 */
        const uint32_t row = row0 + j;
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) {
            const uint32_t i = 4u * g + q;
            const bool valid = i < count && row < a.hidden;
            const float v = ldexpf(acc[q], -sg[q]);
            bad |= valid && !kq_isfinite(v);
            if (valid) a.out[(size_t)(pos0 + i) * a.hidden + row] = v;
        }
    }
    /* no LDS-DMA load may outlive the wave */
    wait_vm<0>();
    if (malformed) kq_flag(a.status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(a.status, KQ_DEV_NUMERIC);
}

/* ------------------------------------------------------------------ */
/* intermediate 512: the two blocks of a row on a pair of waves */

/* With both blocks' activation operand (128 registers) in one wave, the
 * MFMA results spill into accumulation registers and one wave per SIMD
 * pays every latency itself. Here wave h of a pair multiplies block h of
 * each tile: its operand is 64 registers, and eight one-pair workgroups per
 * CU put four waves on each SIMD (measured on the 512-expert T = 512
 * layer: 161.6 us with one wave per SIMD, 134.5 with two and a ring of
 * five tiles, 125.5 with three and three, 123.3 with four and two).
 *   - A workgroup of W waves (W / 2 pairs) owns a contiguous range of the
 *     (item, 16-row tile) sequence; pair p takes tiles lo + p, lo + p +
 *     W / 2, ..., one per round.
 *   - A tile (16 rows x 420 bytes, one contiguous range) goes into a ring
 *     slot of its pair by 16-byte LDS-DMA loads, 1 KiB per instruction:
 *     wave 0 of the pair issues instructions 0-3, wave 1 instructions 4-6
 *     and one that lands in a scratch area. PD tiles stay in flight while
 *     one is multiplied.
 *   - Round k: each wave waits for its own loads of tile k, then one
 *     barrier makes both halves visible and frees the slot of round k - 1,
 *     which then takes the request for tile k + PD. The block-1 wave leaves
 *     its partial sums in an exchange slot of the round's parity; the
 *     block-0 wave adds them after the next barrier, scales and stores. */
struct DnPair {
    static constexpr uint32_t W = 2u;        /* waves per workgroup: one pair */
    static constexpr uint32_t NP = W / 2u;   /* pairs */
    static constexpr uint32_t TB = kT * 420u;               /* tile bytes */
    static constexpr uint32_t IPT = (TB + 1023u) / 1024u;   /* instructions per tile: 7 */
    static constexpr uint32_t IPW = (IPT + 1u) / 2u;        /* per wave: 4 */
    static constexpr uint32_t SLOT = IPT * 1024u;
    static constexpr uint32_t RING = 2u;     /* slots per pair */
    static constexpr uint32_t PD = RING - 1u;
    static_assert(NP * RING * SLOT + 1024u + 2u * NP * 64u * 16u <= 20u * 1024u,
                  "eight workgroups per CU");
};

template <bool FUSED>
__global__ __launch_bounds__(DnPair::W * 64) __attribute__((amdgpu_waves_per_eu(4, 4)))
void dn_q6k_pair(DnArgs a) {
    using S = DnPair;
    constexpr uint32_t KD = 512u, RB = 420u;
    __shared__ __align__(16) uint8_t slots[S::NP][S::RING][S::SLOT];
    __shared__ __align__(16) uint8_t trash[1024];
    __shared__ __align__(16) f4 xch[2][S::NP][64];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t p = w % S::NP, h = w / S::NP; /* pair, block */
    const uint32_t nt = (a.hidden + kT - 1u) / kT; /* tiles per item (>= 16) */
    const uint64_t total = (uint64_t)(*a.n_items) * nt;
    const uint32_t lo = (uint32_t)(total * blockIdx.x / gridDim.x);
    const uint32_t hi = (uint32_t)(total * (blockIdx.x + 1u) / gridDim.x);
    if (lo >= hi) return; /* the whole workgroup */
    const uint32_t rounds = (hi - lo + S::NP - 1u) / S::NP;
    const uint32_t first = lo + p;

    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t wbytes = a.hidden * RB;
    const uint8_t *pslots = &slots[p][0][0];
    const uint32_t pair_lds = lds_addr(pslots);

    /* this wave's instructions of a tile: n = h * IPW + q; past IPT, a
     * re-read of the tile's start into the scratch area */
    uint32_t rel[S::IPW];
#pragma unroll
    for (uint32_t q = 0; q < S::IPW; ++q) {
        const uint32_t c = 64u * (h * S::IPW + q) + lane;
        /* bytes past the tile re-read its start (their slot bytes are
         * never read) */
        rel[q] = 16u * c < S::TB ? 16u * c : 0u;
    }

    /* the next tile to request (stride NP), as item and tile within it */
    uint32_t iss_it = first / nt, iss_in = first - (first / nt) * nt, iss_slot = 0u;
    bool iss_new = true;
    i4v rw = {0, 0, 0, 0};
    auto issue = [&]() {
        if (iss_new) {
            iss_new = false;
            const uint32_t ex = sload(a.items + 2u * iss_it);
            rw = dma_rsrc((ex & kShared) ? a.sdown : a.down + (size_t)ex * wbytes, wbytes);
        }
        const uint32_t toff = iss_in * S::TB;
#pragma unroll
        for (uint32_t q = 0; q < S::IPW; ++q) {
            const uint32_t n = h * S::IPW + q; /* wave-uniform */
            dma16(rw, toff + rel[q],
                  n < S::IPT ? pair_lds + iss_slot * S::SLOT + n * 1024u : lds_addr(trash));
        }
        iss_slot = iss_slot + 1u == S::RING ? 0u : iss_slot + 1u;
        iss_in += S::NP;
        if (iss_in >= nt) {
            iss_in -= nt;
            ++iss_it;
            iss_new = true;
        }
    };

    const DnStaged sx = dn_staged_at(const_cast<void *>(a.staged), a.npos, KD);
    const KqBuf bxh = kq_buf(sx.xh, a.npos * KD * 2u), bxl = kq_buf(sx.xl, a.npos * KD * 2u);
    const KqBuf bsg = kq_buf(sx.sig, a.npos * 4u);
    const uint32_t tk = a.tokens * a.top_k;
    bool bad = false, malformed = false;

#pragma unroll
    for (uint32_t t = 0; t < S::PD; ++t)
        if (first + t * S::NP < hi) issue();

    /* the item being multiplied: block h of the activation operand of lane
     * (j, g), the scales of the four positions of this lane's results */
    uint4 axh[8], axl[8];
    int sg[4];
    uint32_t cur = 0xffffffffu, pos0 = 0u, count = 0u;
    auto enter = [&](uint32_t it) {
        cur = it;
        const uint32_t ex = sload(a.items + 2u * it), fc = sload(a.items + 2u * it + 1u);
        const uint32_t f0 = fc & 0xffffffu;
        count = fc >> 24;
        pos0 = (ex & kShared) ? tk + f0 : f0;
        if constexpr (FUSED) {
            /* the operand split here from the fp32 activations, scaled by
             * each position's largest magnitude exactly as dn_stage does:
             * sub-block s of block h holds columns 256h + 16s .. + 15, of
             * which lane group g takes 4g .. 4g + 3; operand entry ai =
             * (2n + hh) 4 + q is sub-block 8n + 2q + hh */
            const KqBuf bact = kq_buf(a.act, a.npos * KD * 4u);
            const KqBuf bpm = kq_buf(a.posmax, a.npos * 4u);
            const uint32_t fo = j < count ? ((pos0 + j) * KD + 256u * h + 4u * g) * 4u
                                          : 0x80000000u;
            uint4 raw[16];
#pragma unroll
            for (uint32_t ai = 0; ai < 16u; ++ai) {
                const uint32_t sb = 8u * (ai >> 3) + 2u * (ai & 3u) + ((ai >> 2) & 1u);
                raw[ai] = kq_ld128(bact, fo + 64u * sb, 0u);
            }
            const uint32_t mj = kq_ld32(bpm, j < count ? (pos0 + j) * 4u : 0x80000000u, 0u);
            uint32_t mq[4];
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q) {
                const uint32_t i = 4u * g + q;
                mq[q] = kq_ld32(bpm, i < count ? (pos0 + i) * 4u : 0x80000000u, 0u);
            }
            wait_vm_all();
            auto sig_of = [](uint32_t bits) {
                const float m = __builtin_bit_cast(float, bits);
                return m > 0.0f && kq_isfinite(m) ? 15 - __builtin_amdgcn_frexp_expf(m) : 0;
            };
            const int sj = sig_of(mj);
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q) sg[q] = sig_of(mq[q]);
#pragma unroll
            for (uint32_t ai = 0; ai < 16u; ++ai) {
                const float v[4] = {__builtin_bit_cast(float, raw[ai].x),
                                    __builtin_bit_cast(float, raw[ai].y),
                                    __builtin_bit_cast(float, raw[ai].z),
                                    __builtin_bit_cast(float, raw[ai].w)};
                _Float16 hi[4], lo[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float xs = ldexpf(v[c], sj);
                    hi[c] = (_Float16)xs;
                    lo[c] = (_Float16)(xs - (float)hi[c]);
                }
                const uint2 hv = __builtin_bit_cast(uint2, h4{hi[0], hi[1], hi[2], hi[3]});
                const uint2 lv = __builtin_bit_cast(uint2, h4{lo[0], lo[1], lo[2], lo[3]});
                if (ai & 1u) {
                    axh[ai >> 1].z = hv.x, axh[ai >> 1].w = hv.y;
                    axl[ai >> 1].z = lv.x, axl[ai >> 1].w = lv.y;
                } else {
                    axh[ai >> 1].x = hv.x, axh[ai >> 1].y = hv.y;
                    axl[ai >> 1].x = lv.x, axl[ai >> 1].y = lv.y;
                }
            }
        } else {
            /* rows past the chunk read at 2^31, past the buffer */
            const uint32_t xo = j < count ? ((pos0 + j) * KD + g * (KD / 4u) + h * 64u) * 2u
                                          : 0x80000000u;
#pragma unroll
            for (uint32_t v = 0; v < 8u; ++v) {
                axh[v] = kq_ld128(bxh, xo + v * 16u, 0u);
                axl[v] = kq_ld128(bxl, xo + v * 16u, 0u);
            }
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q) {
                const uint32_t i = 4u * g + q;
                sg[q] = (int)kq_ld32(bsg, i < count ? (pos0 + i) * 4u : 0x80000000u, 0u);
            }
            wait_vm_all();
        }
    };

    /* block 0's sums of the previous round plus block 1's: D[token][row],
     * this lane holds row row0 + j of tokens 4g .. 4g + 3 */
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    uint32_t prow0 = 0u, ppos0 = 0u, pcount = 0u;
    int psg[4] = {0, 0, 0, 0};
    auto finish = [&](uint32_t k) {
        const f4 o = xch[k & 1u][p][lane];
        const uint32_t row = prow0 + j;
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) {
            const uint32_t i = 4u * g + q;
            const bool valid = i < pcount && row < a.hidden;
            const float v = ldexpf(acc[q] + o[q], -psg[q]);
            bad |= valid && !kq_isfinite(v);
            if (valid) a.out[(size_t)(ppos0 + i) * a.hidden + row] = v;
        }
    };

    const h2 bias = h2{(_Float16)-1056.0f, (_Float16)-1056.0f}; /* 1024 + 32 */
    uint32_t c_it = first / nt, c_in = first - (first / nt) * nt, cslot = 0u;
    uint32_t tau = first;
    bool prev = false;
    for (uint32_t k = 0; k < rounds; ++k, tau += S::NP) {
        const bool live = tau < hi; /* uniform over the pair */
        if (live) {
            if (c_it != cur) enter(c_it);
            /* this wave's loads of tile tau have landed; those of the later
             * tiles requested so far (at most PD - 1) may be in flight */
            const uint32_t later = (hi - 1u - tau) / S::NP;
            wait_after<S::IPW, S::PD - 1u>(later < S::PD - 1u ? later : S::PD - 1u);
        }
        /* both halves of tile tau are in LDS, the slot of the previous
         * round is free, the previous round's exchange slot is written */
        kq_lds_barrier();
        if (live && tau + S::NP * S::PD < hi) issue();
        if (prev && h == 0u) finish(k - 1u);
        prev = live;
        if (live) {
            const uint8_t *tile = pslots + cslot * S::SLOT;
            cslot = cslot + 1u == S::RING ? 0u : cslot + 1u;
            prow0 = c_in * kT;
            ppos0 = pos0;
            pcount = count;
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q) psg[q] = sg[q];
            c_in += S::NP;
            if (c_in >= nt) {
                c_in -= nt;
                ++c_it;
            }
            /* block h of row j: 4-byte aligned windows, re-aligned by sh */
            const uint32_t o = j * RB + h * 210u;
            const uint32_t sh = o & 3u;
            const uint32_t *pw = (const uint32_t *)(tile + (o - sh));
            auto win = [&](uint32_t off) { return kq_align2(pw[off / 4u + 1u], pw[off / 4u], sh); };
            const float d = half_bits(sh ? (pw[52] >> 16) : pw[52]);
            malformed |= !kq_isfinite(d);
            uint32_t sc[4];
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q) sc[q] = win(192u + 4u * q);
            acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (uint32_t nh = 0; nh < 4u; ++nh) {
                const uint32_t n = nh >> 1, hh = nh & 1u;
                const uint32_t oa = 64u * n + 16u * hh + 4u * g;
                const uint32_t A = win(oa), B = win(oa + 32u);
                const uint32_t H = win(128u + 32u * n + 16u * hh + 4u * g);
                uint32_t c[4];
                c[0] = (A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
                c[1] = (B & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
                c[2] = ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u);
                c[3] = ((B >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
#pragma unroll
                for (uint32_t q = 0; q < 4u; ++q) {
                    const uint32_t s = 8u * n + 2u * q + hh; /* sub-block */
                    const h2 w0 = byte_pair_lo(c[q]) + bias, w1 = byte_pair_hi(c[q]) + bias;
                    const h4 bw = h4{w0.x, w0.y, w1.x, w1.y};
                    /* columns 128n + 32q + 16hh + 4g .. +3 of block h */
                    const uint32_t ai = (n * 2u + hh) * 4u + q;
                    const uint4 &xh = axh[ai >> 1], &xl = axl[ai >> 1];
                    const h4 ah = __builtin_bit_cast(h4, (ai & 1u) ? make_uint2(xh.z, xh.w) : make_uint2(xh.x, xh.y));
                    const h4 al = __builtin_bit_cast(h4, (ai & 1u) ? make_uint2(xl.z, xl.w) : make_uint2(xl.x, xl.y));
                    f4 t = {0.f, 0.f, 0.f, 0.f};
                    t = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bw, t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bw, t, 0, 0, 0);
                    const int8_t scv = (int8_t)((sc[s >> 2] >> (8u * (s & 3u))) & 0xffu);
                    const float ds = d * (float)scv;
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[e] = fmaf(ds, t[e], acc[e]);
                }
            }
            if (h == 1u) xch[k & 1u][p][lane] = acc;
        }
    }
    kq_lds_barrier();
    if (prev && h == 0u) finish(rounds - 1u);
    /* no LDS-DMA load may outlive the wave */
    wait_vm<0>();
    if (malformed) kq_flag(a.status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(a.status, KQ_DEV_NUMERIC);
}

/* ------------------------------------------------------------------ */
/* rows of 32-weight blocks: Q5_1 (the reference
 * model's routed down: 24 B per block, f16 d, f16 m, 32 high bits, 16
 * bytes of nibbles; src/kq_numeric.c:197-222, every block 4-byte aligned)
 * and Q8_0 (its layers 2, 4, 30, 46 and 47: 34 B per block, f16 d and 32
 * int8 codes; src/kq_numeric.c:208-221, blocks alternately at 0 and 2 mod
 * 4 in a row). The activations are split in natural column order
 * (dense_split), so lane (j, g) reads columns 32b + 8g .. + 7 of block b
 * as one 16-byte run. Per block and tile: the codes enter fp16 exactly,
 * one 16x16x32 step each for hi and lo scaled by d; for Q5_1 the min term
 * m * sum(x) is one small step per 16 blocks of the mins against the
 * token's block sums (formed once per item from the activation
 * registers), added unscaled. */
template <uint32_t FMT, uint32_t KD>
struct DnSmallShape {
    static_assert(FMT == KQ_LAUNCH_Q5_1 || FMT == KQ_LAUNCH_Q8_0, "format");
    static constexpr bool Q51 = FMT == KQ_LAUNCH_Q5_1;
    static constexpr uint32_t BB = Q51 ? 24u : 34u;          /* block bytes */
    static constexpr uint32_t NBK = KD / 32u;                /* blocks per row */
    static constexpr uint32_t RB = BB * NBK;                 /* row bytes */
    static_assert(RB % 4u == 0u, "rows start 4-byte aligned in the slot");
    static constexpr uint32_t TB = kT * RB;                  /* tile bytes */
};

/* bits 0..3 of x (x < 16) to bit 4 of bytes 0..3 */
__device__ __forceinline__ uint32_t spread4(uint32_t x) {
    return (kq_mul_u24(x, 0x00204081u) & 0x01010101u) << 4;
}

/* The Q5_1 / Q8_0 down pass on pairs of waves, as dn_q6k_pair: wave h of a
 * pair multiplies blocks h NH .. h NH + NH - 1 of every row (NH = blocks per
 * row / 2), so its activation operand is half a row (80 registers at
 * intermediate 640) and two or three waves share a SIMD; the pair's tiles go
 * through a two-slot ring it shares, and the block-1 wave's partial sums
 * (min term included) reach the block-0 wave through LDS once per tile. */
template <uint32_t FMT, uint32_t KD>
struct DnSmallPair {
    using B = DnSmallShape<FMT, KD>;
    static constexpr uint32_t NH = B::NBK / 2u;             /* blocks per wave */
    static_assert(B::NBK % 4u == 0u, "an even number of blocks per wave");
    static constexpr uint32_t IPT = (B::TB + 1023u) / 1024u; /* instructions per tile */
    static constexpr uint32_t IPW = (IPT + 1u) / 2u;         /* per wave */
    static constexpr uint32_t SLOT = IPT * 1024u;
    static constexpr uint32_t RING = 2u;
    static constexpr uint32_t PD = RING - 1u;
    static constexpr uint32_t LDS = RING * SLOT + 1024u + 2u * 64u * 16u;
    /* waves per SIMD: three for Q8_0 (six one-pair workgroups per CU),
     * two for Q5_1, whose decode and min term need more than the 168
     * registers of three at intermediate 640 */
    static constexpr uint32_t WPE = B::Q51 ? 2u : 3u;
    static constexpr uint32_t WGS = 2u * WPE;
    static_assert(WGS * LDS <= 160u * 1024u, "LDS");
};

template <uint32_t FMT, uint32_t KD>
__global__ __launch_bounds__(128)
__attribute__((amdgpu_waves_per_eu(DnSmallPair<FMT, KD>::WPE, DnSmallPair<FMT, KD>::WPE)))
void dn_small_pair(DnArgs a) {
    using S = DnSmallPair<FMT, KD>;
    using B = typename S::B;
    constexpr uint32_t NH = S::NH;
    __shared__ __align__(16) uint8_t slots[S::RING][S::SLOT];
    __shared__ __align__(16) uint8_t trash[1024];
    __shared__ __align__(16) f4 xch[2][64];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t h = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); /* block half */
    const uint32_t nt = (a.hidden + kT - 1u) / kT; /* tiles per item */
    const uint64_t total = (uint64_t)(*a.n_items) * nt;
    const uint32_t lo = (uint32_t)(total * blockIdx.x / gridDim.x);
    const uint32_t hi = (uint32_t)(total * (blockIdx.x + 1u) / gridDim.x);
    if (lo >= hi) return; /* the whole workgroup */

    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t wbytes = a.hidden * B::RB;
    const uint32_t pair_lds = lds_addr(&slots[0][0]);

    /* this wave's instructions of a tile: n = h * IPW + q; past IPT, a
     * re-read of the tile's start into the scratch area */
    uint32_t rel[S::IPW];
#pragma unroll
    for (uint32_t q = 0; q < S::IPW; ++q) {
        const uint32_t c = 64u * (h * S::IPW + q) + lane;
        rel[q] = 16u * c < B::TB ? 16u * c : 0u;
    }

    uint32_t iss_it = lo / nt, iss_in = lo - (lo / nt) * nt, iss_slot = 0u;
    bool iss_new = true;
    i4v rw = {0, 0, 0, 0};
    auto issue = [&]() {
        if (iss_new) {
            iss_new = false;
            const uint32_t ex = sload(a.items + 2u * iss_it);
            rw = dma_rsrc((ex & kShared) ? a.sdown : a.down + (size_t)ex * wbytes, wbytes);
        }
        const uint32_t toff = iss_in * B::TB;
#pragma unroll
        for (uint32_t q = 0; q < S::IPW; ++q) {
            const uint32_t n = h * S::IPW + q; /* wave-uniform */
            dma16(rw, toff + rel[q],
                  n < S::IPT ? pair_lds + iss_slot * S::SLOT + n * 1024u : lds_addr(trash));
        }
        iss_slot = iss_slot + 1u == S::RING ? 0u : iss_slot + 1u;
        if (++iss_in == nt) {
            iss_in = 0u;
            ++iss_it;
            iss_new = true;
        }
    };

    /* dense_split layout: xh [npos][KD], xl [npos][KD], sig [npos] */
    const uint8_t *st = (const uint8_t *)a.staged;
    const uint32_t xbytes = a.npos * KD * 2u;
    const KqBuf bxh = kq_buf(st, xbytes), bxl = kq_buf(st + xbytes, xbytes);
    const KqBuf bsg = kq_buf(st + 2u * (size_t)xbytes, a.npos * 4u);
    const uint32_t tk = a.tokens * a.top_k;
    bool bad = false, malformed = false;

#pragma unroll
    for (uint32_t t = 0; t < S::PD; ++t)
        if (lo + t < hi) issue();

    uint4 axh[NH], axl[NH];
    constexpr uint32_t NMS = (NH + 15u) / 16u; /* 16-block steps of the min term */
    h4 sxh[NMS], sxl[NMS];
    int sg[4];
    uint32_t cur = 0xffffffffu, pos0 = 0u, count = 0u;
    auto enter = [&](uint32_t it) {
        cur = it;
        const uint32_t ex = sload(a.items + 2u * it), fc = sload(a.items + 2u * it + 1u);
        const uint32_t first = fc & 0xffffffu;
        count = fc >> 24;
        pos0 = (ex & kShared) ? tk + first : first;
        /* rows past the chunk read at 2^31, past the buffer */
        const uint32_t xo =
            j < count ? ((pos0 + j) * KD + 8u * g + 32u * NH * h) * 2u : 0x80000000u;
#pragma unroll
        for (uint32_t b = 0; b < NH; ++b) {
            axh[b] = kq_ld128(bxh, xo + 64u * b, 0u);
            axl[b] = kq_ld128(bxl, xo + 64u * b, 0u);
        }
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) {
            const uint32_t i = 4u * g + q;
            sg[q] = (int)kq_ld32(bsg, i < count ? (pos0 + i) * 4u : 0x80000000u, 0u);
        }
        wait_vm_all();
        if constexpr (!B::Q51) return;
        /* the min term's operand: each of this wave's blocks' column sum
         * of token row j (the four lanes of row j hold 8 columns each),
         * times 2^-5 so it fits fp16, split hi + lo; lane (j, g) keeps
         * blocks 4g .. 4g+3 and 16 + 4g .. (the blocks past NH are zero) */
        float bs[NMS * 16u];
#pragma unroll
        for (uint32_t b = 0; b < NMS * 16u; ++b) bs[b] = 0.0f;
#pragma unroll
        for (uint32_t b = 0; b < NH; ++b) {
            const h8 hh = __builtin_bit_cast(h8, axh[b]), ll = __builtin_bit_cast(h8, axl[b]);
            float p = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) p += (float)hh[e] + (float)ll[e];
            p += __shfl_xor(p, 16, 64);
            p += __shfl_xor(p, 32, 64);
            bs[b] = p * 0.03125f;
        }
#pragma unroll
        for (uint32_t st4 = 0; st4 < NMS; ++st4) {
            _Float16 hv[4], lv[4];
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) {
                float v = 0.0f;
#pragma unroll
                for (uint32_t gg = 0; gg < 4u; ++gg)
                    if (gg == g) v = bs[16u * st4 + 4u * gg + e];
                hv[e] = (_Float16)v;
                lv[e] = (_Float16)(v - (float)hv[e]);
            }
            sxh[st4] = h4{hv[0], hv[1], hv[2], hv[3]};
            sxl[st4] = h4{lv[0], lv[1], lv[2], lv[3]};
        }
    };

    /* the previous round's block-0 sums and where they go */
    f4 part = {0.f, 0.f, 0.f, 0.f};
    uint32_t prow0 = 0u, ppos0 = 0u, pcount = 0u;
    int psg[4] = {0, 0, 0, 0};
    auto finish = [&](uint32_t k) {
        const f4 o = xch[k & 1u][lane];
        const uint32_t r = prow0 + j;
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) {
            const uint32_t i = 4u * g + q;
            const bool valid = i < pcount && r < a.hidden;
            const float v = ldexpf(part[q] + o[q], -psg[q]);
            bad |= valid && !kq_isfinite(v);
            if (valid) a.out[(size_t)(ppos0 + i) * a.hidden + r] = v;
        }
    };

    /* fp16 1024 + code: Q5_1 codes are unsigned, Q8_0 ones offset by 128 */
    const h2 bias = B::Q51 ? h2{(_Float16)-1024.0f, (_Float16)-1024.0f}
                           : h2{(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t shn = g >= 2u ? 4u : 0u;
    uint32_t c_it = lo / nt, c_in = lo - (lo / nt) * nt, cslot = 0u;
    const uint32_t rounds = hi - lo;
    for (uint32_t k = 0; k < rounds; ++k) {
        const uint32_t tau = lo + k;
        if (c_it != cur) enter(c_it);
        {
            /* this wave's loads of tile tau have landed; the later tile
             * requested so far (at most PD - 1 = 0) may be in flight */
            wait_vm<0>();
        }
        /* both halves of tile tau are in LDS, the slot of the previous
         * round is free, the previous round's exchange slot is written */
        kq_lds_barrier();
        if (tau + S::PD < hi) issue();
        if (k > 0u && h == 0u) finish(k - 1u);
        const uint8_t *tile = &slots[cslot][0];
        cslot = cslot + 1u == S::RING ? 0u : cslot + 1u;
        prow0 = c_in * kT;
        ppos0 = pos0;
        pcount = count;
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) psg[q] = sg[q];
        if (++c_in == nt) {
            c_in = 0u;
            ++c_it;
        }
        /* this wave's blocks of row j (h NH B::BB is a multiple of 4) */
        const uint32_t *row = (const uint32_t *)(tile + j * B::RB + h * NH * B::BB);
        f4 acc = {0.f, 0.f, 0.f, 0.f}, macc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t b = 0; b < NH; ++b) {
            uint32_t c0, c1;
            float d;
            if constexpr (B::Q51) {
                const uint32_t *blk = row + 6u * b;
                const uint32_t dm = blk[0];
                const uint32_t hb = (blk[1] >> (8u * g)) & 0xffu;
                const uint2 qv = *(const uint2 *)(blk + 2u + 2u * (g & 1u));
                c0 = ((qv.x >> shn) & 0x0f0f0f0fu) | spread4(hb & 15u);
                c1 = ((qv.y >> shn) & 0x0f0f0f0fu) | spread4(hb >> 4);
                d = half_bits(dm);
                const float mn = half_bits(dm >> 16);
                malformed |= !kq_isfinite(d) || !kq_isfinite(mn);
            } else {
                /* block b at byte 34 b of the half row (NH is even, so
                 * it has the parity of the block in the whole row): d in
                 * the low half of dword 17 b / 2 (b even) or the high half
                 * of dword (34 b - 2) / 4 (b odd); lane g's eight codes at
                 * byte 34 b + 2 + 8 g, 2 mod 4 (b even) or 0 mod 4 (b
                 * odd). The codes, offset by 128, become fp16 1024 + c +
                 * 128. */
                if (b % 2u == 0u) {
                    const uint32_t *blk = row + 17u * (b / 2u);
                    d = half_bits(blk[0]);
                    const uint32_t q0 = blk[2u * g], q1 = blk[2u * g + 1u],
                                   q2 = blk[2u * g + 2u];
                    c0 = kq_align2(q1, q0, 2u) ^ 0x80808080u;
                    c1 = kq_align2(q2, q1, 2u) ^ 0x80808080u;
                } else {
                    const uint32_t *blk = row + (34u * b - 2u) / 4u;
                    d = half_bits(blk[0] >> 16);
                    c0 = blk[1u + 2u * g] ^ 0x80808080u;
                    c1 = blk[2u + 2u * g] ^ 0x80808080u;
                }
                malformed |= !kq_isfinite(d);
            }
            const h2 w0 = byte_pair_lo(c0) + bias, w1 = byte_pair_hi(c0) + bias;
            const h2 w2 = byte_pair_lo(c1) + bias, w3 = byte_pair_hi(c1) + bias;
            const h8 bw = h8{w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
            const h8 ah = __builtin_bit_cast(h8, axh[b]), al = __builtin_bit_cast(h8, axl[b]);
            f4 t = {0.f, 0.f, 0.f, 0.f};
            t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bw, t, 0, 0, 0);
            t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bw, t, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = fmaf(d, t[e], acc[e]);
        }
#pragma unroll
        for (uint32_t st4 = 0; st4 < (B::Q51 ? NMS : 0u); ++st4) {
            _Float16 mv[4];
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) {
                const uint32_t b = 16u * st4 + 4u * g + e;
                mv[e] = b < NH ? __builtin_bit_cast(_Float16, (uint16_t)(row[6u * b] >> 16))
                               : (_Float16)0.0f;
            }
            const h4 mb = h4{mv[0], mv[1], mv[2], mv[3]};
            macc = __builtin_amdgcn_mfma_f32_16x16x16f16(sxh[st4], mb, macc, 0, 0, 0);
            macc = __builtin_amdgcn_mfma_f32_16x16x16f16(sxl[st4], mb, macc, 0, 0, 0);
        }
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) part[q] = fmaf(32.0f, macc[q], acc[q]);
        if (h == 1u) xch[k & 1u][lane] = part;
    }
    kq_lds_barrier();
    if (h == 0u) finish(rounds - 1u);
    /* no LDS-DMA load may outlive the wave */
    wait_vm<0>();
    if (malformed) kq_flag(a.status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(a.status, KQ_DEV_NUMERIC);
}

template <uint32_t KB>
hipError_t launch_dn(const DnArgs &a, hipStream_t s, bool fused) {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus < 1)
            cus = 256;
    }
    if constexpr (KB == 2u) {
        /* eight workgroups per CU: four waves per SIMD */
        if (fused)
            hipLaunchKernelGGL(dn_q6k_pair<true>, dim3(8u * (uint32_t)cus), dim3(DnPair::W * 64), 0,
                               s, a);
        else
            hipLaunchKernelGGL(dn_q6k_pair<false>, dim3(8u * (uint32_t)cus), dim3(DnPair::W * 64),
                               0, s, a);
    } else {
        /* one workgroup per CU (the slots' LDS) */
        hipLaunchKernelGGL((dn_q6k<KB>), dim3((uint32_t)cus), dim3(DnShape<KB>::W * 64), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace

extern "C" int kq_launch_dn_lds_supported(uint32_t inter) { return inter == 256u || inter == 512u; }

extern "C" int kq_launch_dn_small_supported(uint32_t type, uint32_t inter) {
    return (type == KQ_LAUNCH_Q5_1 || type == KQ_LAUNCH_Q8_0) && (inter == 640u || inter == 512u);
}

/* Q5_1 or Q8_0 down over the item list the permutation built: the
 * activation rows split in natural order (dense_split) into staged, then
 * dn_small_pair */
extern "C" hipError_t kq_launch_dn_small(uint32_t type, uint32_t inter, uint32_t hidden,
                                         const void *down, const void *shared_down,
                                         const float *act, uint32_t tokens, uint32_t top_k,
                                         const void *items, void *staged, float *out,
                                         uint32_t *status, hipStream_t s) {
    if (!kq_launch_dn_small_supported(type, inter)) return hipErrorInvalidValue;
    const uint32_t npos = tokens * top_k + tokens;
    uint8_t *st = (uint8_t *)staged;
    const size_t xb = (size_t)npos * inter * 2u;
    hipError_t e = kq_launch_dense_split(act, npos, inter, st, st + xb, (int *)(st + 2u * xb), 0,
                                         status, s);
    if (e != hipSuccess) return e;
    DnArgs a;
    a.down = (const uint8_t *)down;
    a.sdown = (const uint8_t *)shared_down;
    a.staged = staged;
    a.act = nullptr;
    a.posmax = nullptr;
    a.n_items = (const uint32_t *)items;
    a.items = (const uint32_t *)items + 4;
    a.tokens = tokens;
    a.top_k = top_k;
    a.hidden = hidden;
    a.npos = npos;
    a.out = out;
    a.status = status;
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus < 1)
            cus = 256;
    }
#define KQ_DN_SMALL(F, K)                                                                   \
    hipLaunchKernelGGL((dn_small_pair<F, K>), dim3(DnSmallPair<F, K>::WGS * (uint32_t)cus),  \
                       dim3(128), 0, s, a)
    if (type == KQ_LAUNCH_Q5_1) {
        if (inter == 640u)
            KQ_DN_SMALL(KQ_LAUNCH_Q5_1, 640u);
        else
            KQ_DN_SMALL(KQ_LAUNCH_Q5_1, 512u);
    } else {
        if (inter == 640u)
            KQ_DN_SMALL(KQ_LAUNCH_Q8_0, 640u);
        else
            KQ_DN_SMALL(KQ_LAUNCH_Q8_0, 512u);
    }
#undef KQ_DN_SMALL
    return hipGetLastError();
}

extern "C" uint64_t kq_launch_dn_stage_bytes(uint32_t npos, uint32_t inter) {
    return (uint64_t)npos * inter * 4u + (uint64_t)npos * 4u;
}

/* down over the item list the gate/up pass built (items, as written by
 * kq_launch_gu_lds): the per-position split of act, then the pass; with
 * posmax (each position's largest |act|, recorded by the mixed-tile gate/up
 * pass; intermediate 512 only) the pass splits its operand itself */
extern "C" hipError_t kq_launch_dn_lds(uint32_t inter, uint32_t hidden, const void *down,
                                       const void *shared_down, const float *act,
                                       uint32_t tokens, uint32_t top_k, const void *items,
                                       void *staged, const uint32_t *posmax, float *out,
                                       uint32_t *status, hipStream_t s) {
    if (!kq_launch_dn_lds_supported(inter) || (posmax != nullptr && inter != 512u))
        return hipErrorInvalidValue;
    const uint32_t npos = tokens * top_k + tokens;
    if (posmax == nullptr) {
        hipLaunchKernelGGL(dn_stage, dim3(npos), dim3(64), 0, s, act, npos, inter, staged,
                           status);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    DnArgs a;
    a.down = (const uint8_t *)down;
    a.sdown = (const uint8_t *)shared_down;
    a.staged = staged;
    a.act = act;
    a.posmax = posmax;
    a.n_items = (const uint32_t *)items;
    a.items = (const uint32_t *)items + 4;
    a.tokens = tokens;
    a.top_k = top_k;
    a.hidden = hidden;
    a.npos = npos;
    a.out = out;
    a.status = status;
    return inter == 256u ? launch_dn<1>(a, s, false) : launch_dn<2>(a, s, posmax != nullptr);
}
