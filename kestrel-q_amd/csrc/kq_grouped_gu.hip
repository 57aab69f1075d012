/*
 * kq_grouped_gu.hip — the prefill gate/up + SwiGLU pass of Q4_K and Q5_K
 * experts with the weights streamed into LDS by direct (LDS-DMA) buffer
 * loads.
 *
 * The reference computes g = Wg x, u = Wu x and a = swiglu(g, u) for every
 * (token, selected expert) pair one token at a time
 * (src/kq_moe_qwen38.c:722-765 via kq_weight_provider_linear_f32,
 * src/kq_weight_provider.c:378-509). Here every expert's rows stream once for
 * all of its tokens (the grouped path of kq_grouped.hip), and this pass is
 * shaped around how the weights are read:
 *
 *   - The work is a list of items, one per 16-token chunk of an expert
 *     (gu_items), each of ceil(rows / 16) tiles of 16 gate rows and the
 *     same 16 up rows. One workgroup per CU walks a contiguous range of
 *     that tile sequence, so every CU streams the same number of tiles and
 *     the weight pipeline runs on across item boundaries.
 *   - The NB waves of a workgroup split the hidden dimension: wave b
 *     multiplies 256-column block b of every tile. The activation operand
 *     of a wave is therefore the same for every tile of an item, and lives
 *     in registers (no activation image in LDS); it is reloaded when the
 *     item changes.
 *   - The 16 gate rows and 16 up rows of a tile are two contiguous byte
 *     ranges. The workgroup copies them into an LDS ring with 16-byte
 *     LDS-DMA loads, 1 KiB per wave instruction over consecutive bytes, and
 *     keeps RING - 1 tiles in flight ahead of the one being multiplied.
 *     Rows sit in LDS at an odd pitch of 16-byte chunks, so the 16 rows a
 *     block's operand reads touch distinct banks.
 *   - Each wave leaves its block's 16 x 16 partial dots (gate and up) in
 *     LDS; after the tile's barrier they are summed in block order,
 *     unscaled, passed through SwiGLU and stored.
 *
 * Activations come pre-split from gu_stage: per token, the row scaled by
 * 2^sig (largest magnitude in [2^14, 2^15)), as fp16 hi + lo, and the
 * 32-column sums of the scaled row times 2^-5 (also hi + lo) for the
 * min term. The arithmetic per block is the grouped pass's: the 6-bit
 * sub-block scale folds into exact fp16 weights, d scales the fp32 MFMA
 * result, dmin * m is a small MFMA against the sums.
 *
 * Q5_K (176-byte blocks: d, dmin, the same 12 scale bytes, 32 bytes qh of
 * fifth bits, 128 bytes qs of low nibbles; src/kq_numeric.c) differs from
 * Q4_K (144 bytes: d, dmin, scales, qs) only in the code: byte l of the
 * 32-byte qs run of sub-block pair p holds weights 64 p + l (low nibble)
 * and 64 p + 32 + l (high nibble), whose fifth bits are bits 2 p and
 * 2 p + 1 of qh[l] (src/kq_numeric.c:223-270). The five-bit code q <= 31
 * times the scale s <= 63 is at most 1953, still exact in fp16.
 *
 * The LDS-DMA loads are issued from inline assembly, so the compiler's
 * memory-counter bookkeeping never waits on them; the pass waits for them
 * itself with s_waitcnt vmcnt(n), counting only the loads issued after the
 * ones it needs (loads complete in order). Every wave issues the same
 * number of loads per tile, and waits for all of its loads before it ends.
 */
#include "kq_launch.h"
#include "kq_stage.h"
#include "kq_device.h"
#include "kq_dma.h"

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef kq_i4v i4v;

constexpr uint32_t kT = 16; /* tokens per chunk, rows per tile */

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
/* bytes b0, b1 / b2, b3 of m as fp16 0x64XX = 1024 + XX */
__device__ __forceinline__ h2 byte_pair_lo(uint32_t m) {
    return as_h2(__builtin_amdgcn_perm(0x64646464u, m, 0x04010400u));
}
__device__ __forceinline__ h2 byte_pair_hi(uint32_t m) {
    return as_h2(__builtin_amdgcn_perm(0x64646464u, m, 0x04030402u));
}
__device__ __forceinline__ h2 fma2(h2 a, h2 b, h2 c) { return __builtin_elementwise_fma(a, b, c); }
__device__ __forceinline__ float half_bits(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
}

/* ------------------------------------------------------------------ */
/* per-token activation split */

/* grid: one workgroup of 256 threads per token; k a multiple of 256 */
__global__ __launch_bounds__(256) void gu_stage(const float *__restrict__ X, uint32_t tokens,
                                                uint32_t k, void *staged, uint32_t *status) {
    kq::stage_row(X, blockIdx.x, tokens, k, staged, status);
}

/* ------------------------------------------------------------------ */
/* the pass */

/* LDS shape for rows of NB blocks of format FMT (Q4_K or Q5_K), WPB waves
 * per block (2: one matrix per wave; 1: gate and up in one wave) */
template <uint32_t FMT, uint32_t NB, uint32_t WPB>
struct GuShape {
    static_assert(FMT == KQ_LAUNCH_Q4_K || FMT == KQ_LAUNCH_Q5_K, "format");
    static constexpr bool Q5 = FMT == KQ_LAUNCH_Q5_K;
    static constexpr uint32_t BB = Q5 ? 176u : 144u;         /* block bytes */
    static constexpr uint32_t CB = BB / 16u;                /* 16-byte chunks per block */
    static constexpr uint32_t QS = Q5 ? 48u : 16u;          /* offset of qs in a block */
    static constexpr uint32_t W = NB * WPB;                 /* waves */
    static constexpr uint32_t RB = BB * NB;                 /* row bytes */
    static constexpr uint32_t CH = RB / 16u;                /* 16-byte chunks per row */
    static constexpr uint32_t PITCH = (CH & 1u) ? CH : CH + 1u; /* odd: conflict-free rows */
    static constexpr uint32_t SLOTS = kT * PITCH;           /* chunk slots per matrix tile */
    static constexpr uint32_t IM = (SLOTS + 63u) / 64u;     /* instructions per matrix tile */
    static constexpr uint32_t LPW = (2u * IM + W - 1u) / W; /* loads per wave per tile */
    static constexpr uint32_t ENTRY = 2u * IM * 1024u;      /* bytes per ring entry */
    static constexpr uint32_t PART = NB * 2u * 4u * 64u;     /* floats per partial buffer */
    static constexpr uint32_t FIXED = 1024u + 2u * PART * 4u;
    /* three tiles in the ring where they fit, else two */
    static constexpr uint32_t RING = 3u * ENTRY + FIXED <= 160u * 1024u ? 3u : 2u;
    static constexpr uint32_t PD = RING - 1u;                /* tiles in flight ahead */
    static constexpr uint32_t LDS = RING * ENTRY + FIXED;
    static_assert(LDS <= 160u * 1024u, "LDS");
    static_assert(W <= 16u, "workgroup size");
};

struct GuArgs {
    const uint8_t *gate, *up, *sgate, *sup; /* routed stacks, shared matrices */
    const void *staged;                     /* gu_stage output */
    const uint32_t *perm_tok;
    const uint32_t *items;   /* [n][2]: expert (bit 31: shared), first | count << 24 */
    const uint32_t *n_items;
    uint32_t tokens, top_k, rows;
    float *act; /* [T*K + T][rows] */
    uint32_t *posmax; /* [T*K + T] or null: each position's largest |act| (float bits) */
    uint32_t *status;
};

constexpr uint32_t kShared = 0x80000000u;

/* The work list: one item per 16-token chunk of an expert (routed experts
 * in id order, then the shared expert when it runs here), each first |
 * count << 24 with first the chunk's first permuted position (routed) or
 * token (shared). One workgroup of 1024 threads; experts <= 1023. */
__global__ __launch_bounds__(1024) void gu_items(const uint32_t *__restrict__ offsets,
                                                 uint32_t experts, uint32_t tokens,
                                                 uint32_t with_shared, uint32_t *items,
                                                 uint32_t *n_items) {
    __shared__ uint32_t wsum[16];
    const uint32_t e = threadIdx.x, lane = e & 63u, w = e >> 6;
    const uint32_t o0 = e < experts ? offsets[e] : 0u;
    const uint32_t cnt = e < experts ? offsets[e + 1u] - o0 : 0u;
    const uint32_t nc = (cnt + kT - 1u) / kT;
    /* exclusive scan of the chunk counts: wave scan, then the wave totals */
    uint32_t incl = nc;
    for (uint32_t o = 1; o < 64u; o <<= 1) {
        const uint32_t v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
    }
    if (lane == 63u) wsum[w] = incl;
    __syncthreads();
    uint32_t base = incl - nc;
    for (uint32_t q = 0; q < w; ++q) base += wsum[q];
    uint32_t total = 0;
    for (uint32_t q = 0; q < 16u; ++q) total += wsum[q];
    for (uint32_t c = 0; c < nc; ++c) {
        items[2u * (base + c)] = e;
        items[2u * (base + c) + 1u] = (o0 + kT * c) | (min(cnt - kT * c, kT) << 24);
    }
    const uint32_t nsh = with_shared ? (tokens + kT - 1u) / kT : 0u;
    for (uint32_t c = e; c < nsh; c += 1024u) {
        items[2u * (total + c)] = kShared | c;
        items[2u * (total + c) + 1u] = (kT * c) | (min(tokens - kT * c, kT) << 24);
    }
    if (e == 0u) *n_items = total + nsh;
}

/* a wave-uniform dword through the scalar cache (written by an earlier
 * launch); a scalar load counts in lgkmcnt, so it never waits on the
 * LDS-DMA loads in flight */
__device__ __forceinline__ uint32_t sload(const uint32_t *p) {
    const uint64_t a = (uint64_t)(uintptr_t)p;
    /* (readfirstlane returns int: zero-extend each half, never sign-extend) */
    const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a) |
                       ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32);
    uint32_t v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(u) : "memory");
    return v;
}

/* s_waitcnt vmcnt(0) the compiler knows about (gfx9 encoding: expcnt and
 * lgkmcnt left at their maxima) */

/* A persistent grid: workgroup w owns tiles [w N / G, (w + 1) N / G) of the
 * N = items x tiles-per-item sequence, so every workgroup streams the same
 * number of tiles, and its ring keeps running across item boundaries; only
 * the activation operand is reloaded when the item changes. */
template <uint32_t FMT, uint32_t NB, uint32_t WPB>
__global__ __launch_bounds__(NB * WPB * 64) void gu_kq(GuArgs a) {
    using S = GuShape<FMT, NB, WPB>;
    constexpr uint32_t KD = 256u * NB;
    __shared__ __align__(16) uint8_t ring[S::RING * S::ENTRY];
    __shared__ __align__(16) uint8_t trash[1024]; /* landing place of the padding loads */
    __shared__ __align__(16) float part[2][S::PART];
    __shared__ int s_sig[2][kT];   /* by item parity */

    const uint32_t nt = (a.rows + kT - 1u) / kT; /* tiles per item */
    const uint64_t total = (uint64_t)(*a.n_items) * nt;
    const uint32_t lo = (uint32_t)(total * blockIdx.x / gridDim.x);
    const uint32_t hi = (uint32_t)(total * (blockIdx.x + 1u) / gridDim.x);
    if (lo >= hi) return;

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t b = w % NB;   /* this wave's block */
    const uint32_t mw = w / NB;  /* its matrix when WPB == 2 */
    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t wbytes = a.rows * S::RB;

    /* this wave's LPW instructions of a tile (instruction n = w * LPW + q:
     * gate rows for n < IM, up rows for n < 2 IM, padding after): the
     * lane's byte offset relative to the tile's first row */
    uint32_t rel[S::LPW];
#pragma unroll
    for (uint32_t q = 0; q < S::LPW; ++q) {
        const uint32_t n = w * S::LPW + q;
        const uint32_t s = (n < S::IM ? n : n - S::IM) * 64u + lane;
        const uint32_t jj = s / S::PITCH, c = s % S::PITCH;
        /* a pad slot (c == CH) holds the next row's first chunk; slots past
         * the tile and the padding instructions re-read the tile's start */
        rel[q] = (n < 2u * S::IM && s < S::SLOTS) ? 16u * (jj * S::CH + c) : 0u;
    }
    /* the next tile to request: item, tile within it, ring slot (counters,
     * no division in the loop) */
    uint32_t iss_it = lo / nt, iss_tile = lo - (lo / nt) * nt, iss_slot = 0u;
    bool iss_new = true;
    i4v rg = {0, 0, 0, 0}, ru = {0, 0, 0, 0};
    auto issue = [&]() {
        if (iss_new) {
            iss_new = false;
            const uint32_t ex = sload(a.items + 2u * iss_it);
            const uint8_t *gb = (ex & kShared) ? a.sgate : a.gate + (size_t)ex * wbytes;
            const uint8_t *ub = (ex & kShared) ? a.sup : a.up + (size_t)ex * wbytes;
            rg = dma_rsrc(gb, wbytes);
            ru = dma_rsrc(ub, wbytes);
        }
        const uint32_t toff = iss_tile * kT * S::RB;
        const uint32_t slot = lds_addr(ring) + iss_slot * S::ENTRY;
#pragma unroll
        for (uint32_t q = 0; q < S::LPW; ++q) {
            const uint32_t n = w * S::LPW + q; /* wave-uniform */
            const bool up = n >= S::IM && n < 2u * S::IM;
            dma16(up ? ru : rg, toff + rel[q], n < 2u * S::IM ? slot + n * 1024u : lds_addr(trash));
        }
        iss_slot = iss_slot + 1u == S::RING ? 0u : iss_slot + 1u;
        if (++iss_tile == nt) {
            iss_tile = 0u;
            ++iss_it;
            iss_new = true;
        }
    };

    const kq::StagedX sx = kq::staged_at(const_cast<void *>(a.staged), a.tokens, KD);
    const KqBuf bxh = kq_buf(sx.xh, a.tokens * KD * 2u), bxl = kq_buf(sx.xl, a.tokens * KD * 2u);
    const KqBuf bsx = kq_buf(sx.sx, a.tokens * (KD / 128u) * 16u);
    const uint32_t tk = a.tokens * a.top_k;
    float *out = a.act;
    bool bad = false, malformed = false;

    /* the first PD tiles are requested before anything else */
#pragma unroll
    for (uint32_t t = 0; t < S::PD; ++t)
        if (lo + t < hi) issue();

    /* the item being multiplied: its activation operand, the positions its
     * results go to, and the parity of its s_sig slot */
    h8 ah[8], al[8];
    h4 sh4, sl4;
    uint32_t cur = 0xffffffffu, pos0 = 0u, count = 0u, par = 1u;
    /* the tile being multiplied: its index within item cur, its ring slot;
     * the tile reduced next */
    uint32_t ctile = lo - (lo / nt) * nt, cslot = 0u, rtile = 0u;
    auto enter = [&](uint32_t it) {
        cur = it;
        par ^= 1u;
        const uint32_t ex = sload(a.items + 2u * it), fc = sload(a.items + 2u * it + 1u);
        const uint32_t first = fc & 0xffffffu;
        count = fc >> 24;
        const bool sh = (ex & kShared) != 0u;
        pos0 = sh ? tk + first : first;
        /* lane j's token (MFMA row j), its scale into s_sig */
        uint32_t tok = 0xffffffffu;
        if (j < count) tok = sh ? first + j : a.perm_tok[first + j];
        const int sg = tok < a.tokens ? sx.sig[tok] : 0;
        /* the activation operand of block b: hi and lo of the eight steps
         * (columns 256b + 64g + 8s .. + 7), and the sub-block sums; an
         * absent token reads at 2^31, past the buffer for every step */
        const uint32_t xo = tok < a.tokens ? (tok * KD + 256u * b + 64u * g) * 2u : 0x80000000u;
#pragma unroll
        for (uint32_t s = 0; s < 8u; ++s) {
            ah[s] = __builtin_bit_cast(h8, kq_ld128(bxh, xo + 16u * s, 0u));
            al[s] = __builtin_bit_cast(h8, kq_ld128(bxl, xo + 16u * s, 0u));
        }
        const uint32_t so =
            tok < a.tokens ? ((tok * (KD / 128u)) + 2u * b + (g & 1u)) * 16u : 0x80000000u;
        const uint4 sums = kq_ld128(bsx, so, 0u);
        sh4 = __builtin_bit_cast(h4, make_uint2(sums.x, sums.y));
        sl4 = __builtin_bit_cast(h4, make_uint2(sums.z, sums.w));
        if (threadIdx.x < kT) s_sig[par][threadIdx.x] = sg;
        /* everything this wave loaded so far has landed: the compiler
         * then adds no wait of its own at the first use */
        wait_vm_all();
    };
    enter(lo / nt);

    for (uint32_t tau = lo;; ++tau) {
        /* this wave's loads of tile tau have landed (the next tile's may
         * still be in flight), then every wave's have */
        if (tau + S::PD - 1u < hi && S::PD >= 2u)
            wait_vm<(int)S::LPW * (S::PD >= 2u ? (int)S::PD - 1 : 0)>();
        else
            wait_vm<0>();
        kq_lds_barrier();
        if (tau > lo) {
            /* tile tau - 1 (of item cur): sum the blocks' partials in
             * order, SwiGLU */
            const float *pp = part[(tau - 1u) & 1u];
            const uint32_t row0 = rtile * kT;
            for (uint32_t t4 = threadIdx.x; t4 < 256u; t4 += S::W * 64u) {
                const uint32_t L = t4 & 63u, q = t4 >> 6;
                float gs = 0.0f, us = 0.0f;
#pragma unroll
                for (uint32_t bb = 0; bb < NB; ++bb) {
                    gs += pp[((bb * 2u + 0u) * 4u + q) * 64u + L];
                    us += pp[((bb * 2u + 1u) * 4u + q) * 64u + L];
                }
                const uint32_t i = 4u * (L >> 4) + q, row = row0 + (L & 15u);
                const bool valid = i < count && row < a.rows;
                const int sg = s_sig[par][i];
                const float gv = ldexpf(gs, -sg), uv = ldexpf(us, -sg);
                /* silu(g) u with the hardware exponential: the activations
                 * are compared by tolerance like every accumulated output */
                const float v = gv * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gv * 1.44269504088896341f)) * uv;
                bad |= valid && (!kq_isfinite(gv) || !kq_isfinite(uv) || !kq_isfinite(v));
                if (valid) out[(size_t)(pos0 + i) * a.rows + row] = v;
            }
        }
        if (tau == hi) break;
        if (ctile == nt) {
            ctile = 0u;
            enter(cur + 1u);
        }
        if (tau + S::PD < hi) issue();

        /* block b of tile tau: matrix mw (WPB == 2) or both, their MFMA
         * chains interleaved step by step */
        constexpr int NM = WPB == 2u ? 1 : 2;
        const uint8_t *ent = ring + cslot * S::ENTRY;
        rtile = ctile++;
        cslot = cslot + 1u == S::RING ? 0u : cslot + 1u;
            uint4 hd[NM], qa[NM], qb[NM], ha[NM], hb[NM];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const uint32_t mat = WPB == 2u ? mw : (uint32_t)m;
                const uint8_t *rowp =
                    ent + mat * S::IM * 1024u + (j * S::PITCH + S::CB * b) * 16u;
                hd[m] = *(const uint4 *)rowp;
                qa[m] = *(const uint4 *)(rowp + S::QS + 32u * g);
                qb[m] = *(const uint4 *)(rowp + S::QS + 16u + 32u * g);
                if constexpr (S::Q5) {
                    /* qh[0..15], qh[16..31]: the fifth bits of every qs byte */
                    ha[m] = *(const uint4 *)(rowp + 16u);
                    hb[m] = *(const uint4 *)(rowp + 32u);
                }
            }
            float d[NM], dm[NM];
            h2 S0[NM], C0[NM], S1[NM], C1[NM];
            h4 bm[NM];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                d[m] = half_bits(hd[m].x);
                const float dmin = half_bits(hd[m].x >> 16);
                malformed |= !kq_isfinite(d[m]) || !kq_isfinite(dmin);
                dm[m] = dmin * 32.0f; /* the sums carry 2^-5 */
                /* scales of sub-blocks 2g and 2g + 1 (src/kq_numeric.c:161-174),
                 * bitwise selects (a ?: on g becomes a divergent branch) */
                uint32_t s0, s1, m0u, m1u;
                kq_k_scale_pair(g, hd[m].y, hd[m].z, hd[m].w, &s0, &m0u, &s1, &m1u);
                const _Float16 fs0 = (_Float16)(float)s0, fs1 = (_Float16)(float)s1;
                S0[m] = h2{fs0, fs0};
                C0[m] = S0[m] * h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
                if constexpr (S::Q5) {
                    /* both halves as whole five-bit codes: (1024 + q) s - 1024 s */
                    S1[m] = h2{fs1, fs1};
                    C1[m] = S1[m] * h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
                } else {
                    /* high nibbles as 16 q: (1024 + 16 q) s / 16 - 64 s */
                    S1[m] = h2{fs1, fs1} * h2{(_Float16)0.0625f, (_Float16)0.0625f};
                    C1[m] = h2{fs1, fs1} * h2{(_Float16)-64.0f, (_Float16)-64.0f};
                }
                /* mins m_4g .. m_4g+3 for g < 2; zero for g >= 2 */
                const uint32_t k0 = 0u - (uint32_t)(g == 0u), k01 = 0u - (uint32_t)(g < 2u);
                const uint32_t mq = ((hd[m].z & 0x3f3f3f3fu) & k0) |
                                    ((((hd[m].w >> 4) & 0x0f0f0f0fu) | ((hd[m].z >> 2) & 0x30303030u)) & ~k0);
                const h2 one = h2{(_Float16)1.0f, (_Float16)1.0f};
                const h2 neg = h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
                const uint32_t mlo = __builtin_bit_cast(uint32_t, fma2(byte_pair_lo(mq), one, neg)) & k01;
                const uint32_t mhi = __builtin_bit_cast(uint32_t, fma2(byte_pair_hi(mq), one, neg)) & k01;
                bm[m] = __builtin_bit_cast(h4, make_uint2(mlo, mhi));
            }
            f4 qacc[NM];
#pragma unroll
            for (int m = 0; m < NM; ++m) qacc[m] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (uint32_t s = 0; s < 8u; ++s) {
#pragma unroll
                for (int m = 0; m < NM; ++m) {
                    const uint4 &qd = (s & 2u) ? qb[m] : qa[m];
                    const uint32_t raw0 = (s & 1u) ? qd.z : qd.x, raw1 = (s & 1u) ? qd.w : qd.y;
                    uint32_t m0, m1;
                    if constexpr (S::Q5) {
                        /* nibble | fifth bit << 4 per byte: the bit of qh[l]
                         * for sub-block 2 g (low nibbles) or 2 g + 1 (high),
                         * moved to bit 4 */
                        const uint4 &hq = (s & 2u) ? hb[m] : ha[m];
                        const uint32_t h0 = (s & 1u) ? hq.z : hq.x, h1 = (s & 1u) ? hq.w : hq.y;
                        const uint32_t sh = s < 4u ? 2u * g : 2u * g + 1u;
                        const uint32_t n0 = s < 4u ? raw0 : raw0 >> 4;
                        const uint32_t n1 = s < 4u ? raw1 : raw1 >> 4;
                        m0 = (n0 & 0x0f0f0f0fu) | (((h0 >> sh) & 0x01010101u) << 4);
                        m1 = (n1 & 0x0f0f0f0fu) | (((h1 >> sh) & 0x01010101u) << 4);
                    } else {
                        m0 = s < 4u ? kq_and_0f(raw0) : kq_and_f0(raw0);
                        m1 = s < 4u ? kq_and_0f(raw1) : kq_and_f0(raw1);
                    }
                    const h2 Sc = s < 4u ? S0[m] : S1[m], Cc = s < 4u ? C0[m] : C1[m];
                    const h2 w0 = fma2(byte_pair_lo(m0), Sc, Cc), w1 = fma2(byte_pair_hi(m0), Sc, Cc);
                    const h2 w2 = fma2(byte_pair_lo(m1), Sc, Cc), w3 = fma2(byte_pair_hi(m1), Sc, Cc);
                    const h8 bw = h8{w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
                    qacc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[s], bw, qacc[m], 0, 0, 0);
                    qacc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[s], bw, qacc[m], 0, 0, 0);
                }
            }
            float *pw = part[tau & 1u];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                f4 mm = {0.f, 0.f, 0.f, 0.f};
                mm = __builtin_amdgcn_mfma_f32_16x16x16f16(sh4, bm[m], mm, 0, 0, 0);
                mm = __builtin_amdgcn_mfma_f32_16x16x16f16(sl4, bm[m], mm, 0, 0, 0);
                const uint32_t mat = WPB == 2u ? mw : (uint32_t)m;
#pragma unroll
                for (uint32_t q = 0; q < 4u; ++q)
                    pw[((b * 2u + mat) * 4u + q) * 64u + lane] = fmaf(d[m], qacc[m][q], -dm[m] * mm[q]);
            }
    }
    /* no LDS-DMA load may outlive the workgroup */
    wait_vm<0>();
    if (malformed) kq_flag(a.status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(a.status, KQ_DEV_NUMERIC);
}

/* ------------------------------------------------------------------ */
/* the pass on mixed tiles: 8 gate rows and the same 8 up rows per tile */

/* With 16 gate and 16 up rows per tile a workgroup's ring and partial sums
 * need one CU's LDS, so the CU runs one workgroup whose waves meet at a
 * barrier every tile. Here one 16-row MFMA operand holds rows r0 .. r0 + 7
 * of gate (operand rows 0-7) and the same rows of up (8-15): a tile is half
 * the bytes, two workgroups share a CU, and their barriers are independent.
 * The arithmetic per block and row is gu_kq's; the SwiGLU pairs result
 * column j (gate) with column j + 8 (up). */
template <uint32_t FMT, uint32_t NB>
struct GuMixShape {
    static_assert(FMT == KQ_LAUNCH_Q4_K || FMT == KQ_LAUNCH_Q5_K, "format");
    static constexpr bool Q5 = FMT == KQ_LAUNCH_Q5_K;
    static constexpr uint32_t MR = 8u;                      /* rows per matrix and tile */
    static constexpr uint32_t BB = Q5 ? 176u : 144u;        /* block bytes */
    static constexpr uint32_t CB = BB / 16u;
    static constexpr uint32_t QS = Q5 ? 48u : 16u;
    static constexpr uint32_t W = NB;                       /* waves: one per block */
    static constexpr uint32_t RB = BB * NB;                 /* row bytes */
    static constexpr uint32_t CH = RB / 16u;
    static constexpr uint32_t PITCH = (CH & 1u) ? CH : CH + 1u; /* odd: conflict-free rows */
    static constexpr uint32_t SLOTS = MR * PITCH;           /* chunk slots per matrix half */
    static constexpr uint32_t IM = (SLOTS + 63u) / 64u;     /* instructions per half */
    static constexpr uint32_t LPW = (2u * IM + W - 1u) / W; /* loads per wave per tile */
    static constexpr uint32_t ENTRY = 2u * IM * 1024u;
    static constexpr uint32_t PART = NB * 4u * 64u;         /* floats per partial buffer */
    static constexpr uint32_t FIXED = 1024u + 2u * PART * 4u + 2u * kT * 4u;
    static constexpr uint32_t BUDGET = 80u * 1024u;         /* two workgroups per CU */
    static constexpr uint32_t RING = 3u * ENTRY + FIXED <= BUDGET ? 3u : 2u;
    static constexpr uint32_t PD = RING - 1u;
    static_assert(RING * ENTRY + FIXED <= BUDGET, "LDS");
    static_assert(W <= 16u, "workgroup size");
};

template <uint32_t FMT, uint32_t NB>
__global__ __launch_bounds__(NB * 64) void gu_mix(GuArgs a) {
    using S = GuMixShape<FMT, NB>;
    constexpr uint32_t KD = 256u * NB;
    __shared__ __align__(16) uint8_t ring[S::RING * S::ENTRY];
    __shared__ __align__(16) uint8_t trash[1024]; /* landing place of the padding loads */
    __shared__ __align__(16) float part[2][S::PART];
    __shared__ int s_sig[2][kT]; /* by item parity */

    const uint32_t nt = (a.rows + S::MR - 1u) / S::MR; /* tiles per item */
    const uint64_t total = (uint64_t)(*a.n_items) * nt;
    const uint32_t lo = (uint32_t)(total * blockIdx.x / gridDim.x);
    const uint32_t hi = (uint32_t)(total * (blockIdx.x + 1u) / gridDim.x);
    if (lo >= hi) return;

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t b = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); /* this wave's block */
    const uint32_t j = lane & 15u, g = lane >> 4;
    const uint32_t wbytes = a.rows * S::RB;

    /* this wave's LPW instructions of a tile (instruction n = b * LPW + q:
     * gate rows for n < IM, up rows for n < 2 IM, padding after): the
     * lane's byte offset relative to the tile's first row */
    uint32_t rel[S::LPW];
#pragma unroll
    for (uint32_t q = 0; q < S::LPW; ++q) {
        const uint32_t n = b * S::LPW + q;
        const uint32_t s = (n < S::IM ? n : n - S::IM) * 64u + lane;
        const uint32_t jj = s / S::PITCH, c = s % S::PITCH;
        /* a pad slot (c == CH) holds the next row's first chunk; slots past
         * the tile and the padding instructions re-read the tile's start */
        rel[q] = (n < 2u * S::IM && s < S::SLOTS) ? 16u * (jj * S::CH + c) : 0u;
    }
    uint32_t iss_it = lo / nt, iss_tile = lo - (lo / nt) * nt, iss_slot = 0u;
    bool iss_new = true;
    i4v rg = {0, 0, 0, 0}, ru = {0, 0, 0, 0};
    auto issue = [&]() {
        if (iss_new) {
            iss_new = false;
            const uint32_t ex = sload(a.items + 2u * iss_it);
            const uint8_t *gb = (ex & kShared) ? a.sgate : a.gate + (size_t)ex * wbytes;
            const uint8_t *ub = (ex & kShared) ? a.sup : a.up + (size_t)ex * wbytes;
            rg = dma_rsrc(gb, wbytes);
            ru = dma_rsrc(ub, wbytes);
        }
        const uint32_t toff = iss_tile * S::MR * S::RB;
        const uint32_t slot = lds_addr(ring) + iss_slot * S::ENTRY;
#pragma unroll
        for (uint32_t q = 0; q < S::LPW; ++q) {
            const uint32_t n = b * S::LPW + q; /* wave-uniform */
            const bool up = n >= S::IM && n < 2u * S::IM;
            dma16(up ? ru : rg, toff + rel[q], n < 2u * S::IM ? slot + n * 1024u : lds_addr(trash));
        }
        iss_slot = iss_slot + 1u == S::RING ? 0u : iss_slot + 1u;
        if (++iss_tile == nt) {
            iss_tile = 0u;
            ++iss_it;
            iss_new = true;
        }
    };

    const kq::StagedX sx = kq::staged_at(const_cast<void *>(a.staged), a.tokens, KD);
    const KqBuf bxh = kq_buf(sx.xh, a.tokens * KD * 2u), bxl = kq_buf(sx.xl, a.tokens * KD * 2u);
    const KqBuf bsx = kq_buf(sx.sx, a.tokens * (KD / 128u) * 16u);
    const uint32_t tk = a.tokens * a.top_k;
    float *out = a.act;
    bool bad = false, malformed = false;

#pragma unroll
    for (uint32_t t = 0; t < S::PD; ++t)
        if (lo + t < hi) issue();

    h8 ah[8], al[8];
    h4 sh4, sl4;
    uint32_t cur = 0xffffffffu, pos0 = 0u, count = 0u, par = 1u;
    uint32_t ctile = lo - (lo / nt) * nt, cslot = 0u, rtile = 0u;
    auto enter = [&](uint32_t it) {
        cur = it;
        par ^= 1u;
        const uint32_t ex = sload(a.items + 2u * it), fc = sload(a.items + 2u * it + 1u);
        const uint32_t first = fc & 0xffffffu;
        count = fc >> 24;
        const bool sh = (ex & kShared) != 0u;
        pos0 = sh ? tk + first : first;
        uint32_t tok = 0xffffffffu;
        if (j < count) tok = sh ? first + j : a.perm_tok[first + j];
        const int sg = tok < a.tokens ? sx.sig[tok] : 0;
        const uint32_t xo = tok < a.tokens ? (tok * KD + 256u * b + 64u * g) * 2u : 0x80000000u;
#pragma unroll
        for (uint32_t s = 0; s < 8u; ++s) {
            ah[s] = __builtin_bit_cast(h8, kq_ld128(bxh, xo + 16u * s, 0u));
            al[s] = __builtin_bit_cast(h8, kq_ld128(bxl, xo + 16u * s, 0u));
        }
        const uint32_t so =
            tok < a.tokens ? ((tok * (KD / 128u)) + 2u * b + (g & 1u)) * 16u : 0x80000000u;
        const uint4 sums = kq_ld128(bsx, so, 0u);
        sh4 = __builtin_bit_cast(h4, make_uint2(sums.x, sums.y));
        sl4 = __builtin_bit_cast(h4, make_uint2(sums.z, sums.w));
        if (threadIdx.x < kT) s_sig[par][threadIdx.x] = sg;
        wait_vm_all();
    };
    enter(lo / nt);

    /* lane (j, g)'s operand row: gate (j < 8) or up row r0 + (j & 7) */
    const uint32_t half = j >> 3, jr = j & 7u;
    for (uint32_t tau = lo;; ++tau) {
        if (tau + S::PD - 1u < hi && S::PD >= 2u)
            wait_vm<(int)S::LPW * (S::PD >= 2u ? (int)S::PD - 1 : 0)>();
        else
            wait_vm<0>();
        kq_lds_barrier();
        if (tau > lo) {
            /* tile tau - 1 (of item cur): sum the blocks' partials in
             * order, SwiGLU: result (token 4g + q, gate row r) sits in
             * column r of the lanes of k-group g, the up row in column
             * r + 8 */
            const float *pp = part[(tau - 1u) & 1u];
            const uint32_t row0 = rtile * S::MR;
            for (uint32_t t4 = threadIdx.x; t4 < kT * S::MR; t4 += S::W * 64u) {
                const uint32_t r = t4 & 7u, i = t4 >> 3, q = i & 3u, lg = (i >> 2) * 16u + r;
                float gs = 0.0f, us = 0.0f;
#pragma unroll
                for (uint32_t bb = 0; bb < NB; ++bb) {
                    gs += pp[(bb * 4u + q) * 64u + lg];
                    us += pp[(bb * 4u + q) * 64u + lg + 8u];
                }
                const uint32_t row = row0 + r;
                const bool valid = i < count && row < a.rows;
                const int sg = s_sig[par][i];
                const float gv = ldexpf(gs, -sg), uv = ldexpf(us, -sg);
                /* silu(g) u with the hardware exponential: the activations
                 * are compared by tolerance like every accumulated output */
                const float v = gv * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gv * 1.44269504088896341f)) * uv;
                bad |= valid && (!kq_isfinite(gv) || !kq_isfinite(uv) || !kq_isfinite(v));
                if (valid) out[(size_t)(pos0 + i) * a.rows + row] = v;
                if (a.posmax != nullptr) {
                    /* the position's largest magnitude over the tile's 8
                     * rows (lanes 8i .. 8i + 7), then over all tiles: float
                     * bits of non-negative values order as integers */
                    float mv = valid && kq_isfinite(v) ? fabsf(v) : 0.0f;
                    mv = fmaxf(mv, __shfl_xor(mv, 1, 64));
                    mv = fmaxf(mv, __shfl_xor(mv, 2, 64));
                    mv = fmaxf(mv, __shfl_xor(mv, 4, 64));
                    if (r == 0u && i < count && mv > 0.0f)
                        atomicMax(a.posmax + pos0 + i, __builtin_bit_cast(uint32_t, mv));
                }
            }
        }
        if (tau == hi) break;
        if (ctile == nt) {
            ctile = 0u;
            enter(cur + 1u);
        }
        if (tau + S::PD < hi) issue();

        const uint8_t *ent = ring + cslot * S::ENTRY;
        rtile = ctile++;
        cslot = cslot + 1u == S::RING ? 0u : cslot + 1u;
        const uint8_t *rowp = ent + half * S::IM * 1024u + (jr * S::PITCH + S::CB * b) * 16u;
        const uint4 hd = *(const uint4 *)rowp;
        const uint4 qa = *(const uint4 *)(rowp + S::QS + 32u * g);
        const uint4 qb = *(const uint4 *)(rowp + S::QS + 16u + 32u * g);
        uint4 ha = {0u, 0u, 0u, 0u}, hb = {0u, 0u, 0u, 0u};
        if constexpr (S::Q5) {
            ha = *(const uint4 *)(rowp + 16u);
            hb = *(const uint4 *)(rowp + 32u);
        }
        const float d = half_bits(hd.x);
        const float dmin = half_bits(hd.x >> 16);
        malformed |= !kq_isfinite(d) || !kq_isfinite(dmin);
        const float dm = dmin * 32.0f; /* the sums carry 2^-5 */
        /* scales of sub-blocks 2g and 2g + 1 (src/kq_numeric.c:161-174),
         * bitwise selects (a ?: on g becomes a divergent branch) */
        uint32_t s0, s1, m0u, m1u;
        kq_k_scale_pair(g, hd.y, hd.z, hd.w, &s0, &m0u, &s1, &m1u);
        const _Float16 fs0 = (_Float16)(float)s0, fs1 = (_Float16)(float)s1;
        const h2 S0 = h2{fs0, fs0};
        const h2 C0 = S0 * h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
        h2 S1, C1;
        if constexpr (S::Q5) {
            S1 = h2{fs1, fs1};
            C1 = S1 * h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
        } else {
            S1 = h2{fs1, fs1} * h2{(_Float16)0.0625f, (_Float16)0.0625f};
            C1 = h2{fs1, fs1} * h2{(_Float16)-64.0f, (_Float16)-64.0f};
        }
        /* mins m_4g .. m_4g+3 for g < 2; zero for g >= 2 */
        const uint32_t k0 = 0u - (uint32_t)(g == 0u), k01 = 0u - (uint32_t)(g < 2u);
        const uint32_t mq = ((hd.z & 0x3f3f3f3fu) & k0) |
                            ((((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u)) & ~k0);
        const h2 one = h2{(_Float16)1.0f, (_Float16)1.0f};
        const h2 neg = h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
        const uint32_t mlo = __builtin_bit_cast(uint32_t, fma2(byte_pair_lo(mq), one, neg)) & k01;
        const uint32_t mhi = __builtin_bit_cast(uint32_t, fma2(byte_pair_hi(mq), one, neg)) & k01;
        const h4 bm = __builtin_bit_cast(h4, make_uint2(mlo, mhi));
        f4 qacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t s = 0; s < 8u; ++s) {
            const uint4 &qd = (s & 2u) ? qb : qa;
            const uint32_t raw0 = (s & 1u) ? qd.z : qd.x, raw1 = (s & 1u) ? qd.w : qd.y;
            uint32_t m0, m1;
            if constexpr (S::Q5) {
                const uint4 &hq = (s & 2u) ? hb : ha;
                const uint32_t h0 = (s & 1u) ? hq.z : hq.x, h1 = (s & 1u) ? hq.w : hq.y;
                const uint32_t sh = s < 4u ? 2u * g : 2u * g + 1u;
                const uint32_t n0 = s < 4u ? raw0 : raw0 >> 4;
                const uint32_t n1 = s < 4u ? raw1 : raw1 >> 4;
                m0 = (n0 & 0x0f0f0f0fu) | (((h0 >> sh) & 0x01010101u) << 4);
                m1 = (n1 & 0x0f0f0f0fu) | (((h1 >> sh) & 0x01010101u) << 4);
            } else {
                m0 = s < 4u ? kq_and_0f(raw0) : kq_and_f0(raw0);
                m1 = s < 4u ? kq_and_0f(raw1) : kq_and_f0(raw1);
            }
            const h2 Sc = s < 4u ? S0 : S1, Cc = s < 4u ? C0 : C1;
            const h2 w0 = fma2(byte_pair_lo(m0), Sc, Cc), w1 = fma2(byte_pair_hi(m0), Sc, Cc);
            const h2 w2 = fma2(byte_pair_lo(m1), Sc, Cc), w3 = fma2(byte_pair_hi(m1), Sc, Cc);
            const h8 bw = h8{w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
            qacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[s], bw, qacc, 0, 0, 0);
            qacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[s], bw, qacc, 0, 0, 0);
        }
        f4 mm = {0.f, 0.f, 0.f, 0.f};
        mm = __builtin_amdgcn_mfma_f32_16x16x16f16(sh4, bm, mm, 0, 0, 0);
        mm = __builtin_amdgcn_mfma_f32_16x16x16f16(sl4, bm, mm, 0, 0, 0);
        float *pw = part[tau & 1u];
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) pw[(b * 4u + q) * 64u + lane] = fmaf(d, qacc[q], -dm * mm[q]);
    }
    wait_vm<0>();
    if (malformed) kq_flag(a.status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(a.status, KQ_DEV_NUMERIC);
}

/* waves per block: one (gate and up in one wave) */
template <uint32_t NB>
constexpr uint32_t gu_wpb() {
    return 1u;
}

template <uint32_t FMT, uint32_t NB>
hipError_t launch_gu(const GuArgs &a, hipStream_t s) {
    constexpr uint32_t WPB = gu_wpb<NB>();
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus < 1)
            cus = 256;
    }
    if constexpr (NB == 8u) {
        /* mixed tiles: two workgroups of eight waves per CU */
        hipLaunchKernelGGL((gu_mix<FMT, NB>), dim3(2u * (uint32_t)cus), dim3(NB * 64), 0, s, a);
    } else {
        /* one workgroup per CU: the LDS ring holds one */
        hipLaunchKernelGGL((gu_kq<FMT, NB, WPB>), dim3((uint32_t)cus), dim3(NB * WPB * 64), 0, s,
                           a);
    }
    return hipGetLastError();
}

}  // namespace

extern "C" int kq_launch_gu_lds_supported(uint32_t type, uint32_t hidden) {
    return (type == KQ_LAUNCH_Q4_K || type == KQ_LAUNCH_Q5_K) &&
           (hidden == 256u || hidden == 512u || hidden == 1024u || hidden == 2048u ||
            hidden == 2560u);
}

extern "C" uint64_t kq_launch_gu_stage_bytes(uint32_t tokens, uint32_t hidden) {
    return (uint64_t)tokens * hidden * 4u + (uint64_t)tokens * (hidden / 128u) * 16u +
           (uint64_t)tokens * 4u;
}

extern "C" hipError_t kq_launch_gu_stage(const float *hidden_states, uint32_t tokens,
                                         uint32_t hidden, void *staged, uint32_t *status,
                                         hipStream_t s) {
    hipLaunchKernelGGL(gu_stage, dim3(tokens), dim3(256), 0, s, hidden_states, tokens, hidden,
                       staged, status);
    return hipGetLastError();
}

extern "C" uint64_t kq_launch_gu_items_bytes(uint32_t experts, uint32_t tokens,
                                             uint32_t top_k) {
    const uint64_t n = experts + ((uint64_t)tokens * top_k + kT - 1u) / kT +
                       (tokens + kT - 1u) / kT + 1u;
    return n * 8u + 16u;
}

/* the routed experts' chunks (and the shared expert's when with_shared)
 * of a permutation (offsets) as the pass's work list, then the pass over
 * it; items holds kq_launch_gu_items_bytes */
extern "C" hipError_t kq_launch_gu_lds(uint32_t type, uint32_t hidden, const void *gate,
                                       const void *up,
                                       const void *shared_gate, const void *shared_up,
                                       const void *staged, const uint32_t *offsets,
                                       const uint32_t *perm_tok, uint32_t experts,
                                       uint32_t tokens, uint32_t top_k, uint32_t rows,
                                       int with_shared, int items_ready, void *items,
                                       float *act, uint32_t *posmax, uint32_t *status,
                                       hipStream_t s) {
    if (experts > 1023u || !kq_launch_gu_lds_supported(type, hidden)) return hipErrorInvalidValue;
    uint32_t *n_items = (uint32_t *)items;
    uint32_t *list = n_items + 4;
    if (!items_ready) {
        hipLaunchKernelGGL(gu_items, dim3(1), dim3(1024), 0, s, offsets, experts, tokens,
                           with_shared ? 1u : 0u, list, n_items);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    GuArgs a;
    a.gate = (const uint8_t *)gate;
    a.up = (const uint8_t *)up;
    a.sgate = (const uint8_t *)shared_gate;
    a.sup = (const uint8_t *)shared_up;
    a.staged = staged;
    a.perm_tok = perm_tok;
    a.items = list;
    a.n_items = n_items;
    a.tokens = tokens;
    a.top_k = top_k;
    a.rows = rows;
    a.act = act;
    /* the positions' maxima come from the mixed-tile pass only */
    if (posmax != nullptr && hidden != 2048u) return hipErrorInvalidValue;
    a.posmax = posmax;
    a.status = status;
#define KQ_GU_HIDDEN(F)                               \
    switch (hidden) {                                 \
    case 256: return launch_gu<F, 1>(a, s);           \
    case 512: return launch_gu<F, 2>(a, s);           \
    case 1024: return launch_gu<F, 4>(a, s);          \
    case 2048: return launch_gu<F, 8>(a, s);          \
    case 2560: return launch_gu<F, 10>(a, s);         \
    default: return hipErrorInvalidValue;             \
    }
    if (type == KQ_LAUNCH_Q5_K) {
        KQ_GU_HIDDEN(KQ_LAUNCH_Q5_K)
    }
    KQ_GU_HIDDEN(KQ_LAUNCH_Q4_K)
#undef KQ_GU_HIDDEN
}
