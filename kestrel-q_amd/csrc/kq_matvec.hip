/*
 * kq_matvec.hip — dequant-fused matrix-vector products y = W x for GGUF
 * Q4_K, Q5_K, Q6_K, Q8_0, Q5_1 and IQ4_NL rows (batch 1..4, fp32 activations and outputs) and
 * greedy argmax over the results.
 *
 * Restates the row loop of kq_weight_provider_linear_f32
 * (src/kq_weight_provider.c:464-475) around kq_quantized_row_dot_f32
 * (src/kq_numeric.c:420-503), and kq_model_exec_greedy_argmax_f32
 * (src/kq_model_exec.c:566-584). Weights decode exactly as the reference
 * decodes them; the row sum is a wave-parallel fp32 reduction compared by
 * tolerance. The argmax is exact (first maximum, lowest row on ties).
 *
 * Each 64-lane wavefront keeps its lanes' activations in registers for the
 * whole launch and walks groups of RT row passes (kq_rowdot.h): the
 * activation loads are issued first, then the first group's weight loads,
 * and each following group's loads are in flight while the current group is
 * reduced.
 * Row sums finish with a transposed butterfly (permlane swaps and DPP), so a
 * group of RT*B partial sums costs a few cross-lane operations. For the
 * fused LM head every wave also keeps a running (max, row) per batch column
 * and writes one partial; a one-block kernel merges the partials.
 */
#include <mutex>

#include "kq_launch.h"
#include "kq_rowdot.h"

/* Argmax partials of the allocation-free LM head
 * (kq_hip_lm_head_greedy_f32_noalloc): kNoallocParts values, then as many
 * row ids. Each device holds its own copy for the life of the process and
 * every call on that device shares it. Host code reaches it only through
 * the address hipGetSymbolAddress returns for the device
 * (kq_launch_noalloc_scratch_init); the name itself is not a device
 * address on the host. */
constexpr uint32_t kNoallocParts = 1u << 17;
static __device__ __align__(256) uint8_t scratch[kNoallocParts * 8u];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

}  // namespace

extern "C" uint32_t kq_launch_noalloc_parts(void) { return kNoallocParts; }

/* Looks up this device's copy of `scratch` once per device; `device` must
 * be the current device. */
extern "C" hipError_t kq_launch_noalloc_scratch_init(int device, void **out) {
    if (device < 0 || device >= kMaxDevices || out == nullptr) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device] == nullptr) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

namespace {

constexpr int kThreads = 256;

/* larger value wins, equal values keep the lower row */
__device__ __forceinline__ void argmax_merge(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__device__ __forceinline__ void wave_argmax(float &bv, uint32_t &bi) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(bv, o, KQ_WAVE);
        uint32_t oi = __shfl_xor(bi, o, KQ_WAVE);
        argmax_merge(bv, bi, ov, oi);
    }
}

/* One column segment of COLS columns: row r's segment starts at
 * W + r * row_bytes, batch column b's activations at x + b * x_stride. With
 * y_prev (which may be y itself) the segment's sums are added to the
 * previous segments' ones, in segment order. */
template <uint32_t TYPE, uint32_t COLS, int B, int RT, int NT>
__global__ __launch_bounds__(NT) void matvec_kernel(
    const uint8_t *__restrict__ W, uint32_t rows, uint32_t row_bytes,
    const float *__restrict__ x, uint32_t x_stride, float *y, const float *y_prev,
    uint32_t *status, float *part_v, uint32_t *part_i, uint32_t part_stride) {
    using R = kq::Rows<TYPE, COLS, B, RT, typename kq::MatvecLane<TYPE, B>::T>;
    using Raw = typename R::Raw;
    const uint32_t lane = threadIdx.x & 63u;
    /* uniform across the wave: the group loop and the full-group test stay
     * scalar branches */
    const uint32_t wave =
        __builtin_amdgcn_readfirstlane((blockIdx.x * NT + threadIdx.x) >> 6);
    const uint32_t nwaves = (gridDim.x * NT) >> 6;
    const uint32_t sub = lane / R::LPR, l = lane % R::LPR;
    const uint32_t ngroups = (rows + R::GROUP - 1u) / R::GROUP;

    typename R::Lane ln;
    ln.setup(l);
    const uint32_t wbytes = (rows - 1u) * row_bytes + R::RB;
    /* one group per wave (small matrices): non-temporal weight loads */
    const auto wb = kq_buf<(RT == 1 ? kKqNt : 0)>(W, wbytes);
    Raw ra[RT], rb[RT];
    uint32_t g = wave;
    /* The workgroup requests its activations (once, into LDS), then every
     * wave its first group's weights, without a branch; the activation
     * loads complete first, are checked and written to LDS behind an
     * LDS-only barrier while the weights are still in flight. The check is
     * flagged at the end. */
    using XS = kq::StageFor<R, B, NT>;
    __shared__ __align__(16) float4 xs[XS::NP];
    XS stage;
    stage.issue(x, x_stride, threadIdx.x);
    R::load_group_oob(ln, wb, g, rows, sub, ra, row_bytes, wbytes + 64u);
    const bool xbad = stage.commit(xs, threadIdx.x);
    kq_lds_barrier();
    stage.load(ln, xs, l);

    bool bad = false, malformed = false;
    float best_v[B];
    uint32_t best_i[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        best_v[b] = -__builtin_inff();
        best_i[b] = 0xffffffffu;
    }
    auto finish = [&](const Raw (&raw)[RT], uint32_t gg) {
        float v[R::N];
        R::dot_group(ln, raw, l, v, malformed);
#pragma unroll
        for (int j = 0; j < R::KEEP; ++j) {
            const int idx = R::value_index(l, j);
            if (idx >= 0) {
                const uint32_t r = (uint32_t)idx / B, b = (uint32_t)idx % B;
                const uint32_t row = gg * R::GROUP + r * R::RPW + sub;
                if (row < rows) {
                    float s = v[j];
                    if (y_prev != nullptr) s = y_prev[(size_t)b * rows + row] + s;
                    y[(size_t)b * rows + row] = s;
                    bad |= !kq_isfinite(s);
                    argmax_merge(best_v[b], best_i[b], s, row);
                }
            }
        }
    };
    /* ping-pong: the next group's loads are in flight while one is reduced.
     * They are issued without a branch (rows past the matrix read zeros
     * from beyond the buffer), so every path has the same loads
     * outstanding and the waits before a group's use count only its own:
     * a conditional prefetch makes the compiler wait for all loads. The
     * scheduling barrier keeps the loads ahead of the reduction. */
    const uint32_t oob = wbytes + 64u;
    while (g < ngroups) {
        uint32_t gn = g + nwaves;
        R::load_group_oob(ln, wb, gn, rows, sub, rb, row_bytes, oob);
        __builtin_amdgcn_sched_barrier(0);
        finish(ra, g);
        g = gn;
        if (g >= ngroups) break;
        gn = g + nwaves;
        R::load_group_oob(ln, wb, gn, rows, sub, ra, row_bytes, oob);
        __builtin_amdgcn_sched_barrier(0);
        finish(rb, g);
        g = gn;
    }
    if (xbad) kq_flag(status, KQ_DEV_INPUT);
    if (malformed) kq_flag(status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
    if (part_v != nullptr) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float bv = best_v[b];
            uint32_t bi = best_i[b];
            wave_argmax(bv, bi);
            if (lane == 0) {
                part_v[(size_t)b * part_stride + wave] = bv;
                part_i[(size_t)b * part_stride + wave] = bi;
                /* slots past this launch's waves (another launch of the same
                 * call may have more) hold the neutral entry */
                for (uint32_t sl = wave + nwaves; sl < part_stride; sl += nwaves) {
                    part_v[(size_t)b * part_stride + sl] = -__builtin_inff();
                    part_i[(size_t)b * part_stride + sl] = 0xffffffffu;
                }
            }
        }
    }
}

/* Rows wider than one engine width in one launch. A row of `cols` columns
 * is NCH chunks of 2048 (the last one `tail` columns, a whole number of
 * blocks). The workgroup stages every chunk's activations once (one LDS
 * image per chunk); each wave keeps its lanes' partial dots of RT rows in
 * registers while it walks the chunks, the next chunk's weights in flight
 * while one is dotted, and reduces across the lanes once per row group.
 * In the last chunk the lanes past `tail` read outside the buffer (zeros,
 * whose scale is zero) against zero activations. The per-lane sums
 * accumulate chunk by chunk, so the fp32 order differs from the
 * per-segment launches (compared by tolerance like every row sum). */
constexpr uint32_t kWideCols = 2048u;

template <uint32_t TYPE, int B, int RT, int NT, uint32_t NCH>
__global__ __launch_bounds__(NT) void matvec_wide(
    const uint8_t *__restrict__ W, uint32_t rows, uint32_t row_bytes, uint32_t tail,
    const float *__restrict__ x, uint32_t x_stride, float *y, uint32_t *status, float *part_v,
    uint32_t *part_i, uint32_t part_stride) {
    using R = kq::Rows<TYPE, kWideCols, B, RT, typename kq::MatvecLane<TYPE, B>::T>;
    using Raw = typename R::Raw;
    static_assert(R::LPR == 64u && R::RPW == 1u, "a 2048-column chunk takes the whole wave");
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave =
        __builtin_amdgcn_readfirstlane((blockIdx.x * NT + threadIdx.x) >> 6);
    const uint32_t nwaves = (gridDim.x * NT) >> 6;
    const uint32_t ngroups = (rows + R::GROUP - 1u) / R::GROUP;
    const uint32_t wbytes = (rows - 1u) * row_bytes + (NCH - 1u) * R::RB +
                            kq::row_bytes<TYPE>(tail);
    const uint32_t oob = wbytes + 64u;
    const auto wb = kq_buf<(RT == 1 ? kKqNt : 0)>(W, wbytes);
    /* lanes of the last chunk that hold columns */
    const bool tail_lane = lane < tail / 32u;

    typename R::Lane ln;
    ln.setup(lane);
    using XS = kq::StageFor<R, B, NT>;
    __shared__ __align__(16) float4 xs[NCH][XS::NP];
    /* chunk c of row group g: its RT rows, lanes past the tail outside */
    auto load = [&](uint32_t g, uint32_t c, Raw (&raw)[RT]) {
        const bool live = c + 1u < NCH || tail_lane;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const uint32_t row = g * R::GROUP + (uint32_t)r;
            raw[r] = ln.load(wb, live && row < rows ? row * row_bytes + c * R::RB : oob);
        }
    };
    Raw ra[RT], rb[RT];
    uint32_t g = wave;
    load(g, 0u, ra);
    /* every chunk's activations requested before any is written to LDS */
    XS stage[NCH];
#pragma unroll
    for (uint32_t c = 0; c < NCH; ++c)
        stage[c].issue(x + c * kWideCols, x_stride, threadIdx.x,
                       c + 1u < NCH ? kWideCols : tail);
    bool xbad = false;
#pragma unroll
    for (uint32_t c = 0; c < NCH; ++c) xbad |= stage[c].commit(xs[c], threadIdx.x);
    kq_lds_barrier();

    bool bad = false, malformed = false;
    float best_v[B];
    uint32_t best_i[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        best_v[b] = -__builtin_inff();
        best_i[b] = 0xffffffffu;
    }
    while (g < ngroups) {
        float acc[R::N];
#pragma unroll
        for (int i = 0; i < R::N; ++i) acc[i] = 0.0f;
        /* chunk c from ra (even) or rb (odd); chunk c + 1, or the next
         * group's chunk 0, in flight meanwhile */
#pragma unroll
        for (uint32_t c = 0; c < NCH; ++c) {
            Raw(&cur)[RT] = (c & 1u) ? rb : ra;
            Raw(&nxt)[RT] = (c & 1u) ? ra : rb;
            if (c + 1u < NCH)
                load(g, c + 1u, nxt);
            else
                load(g + nwaves, 0u, nxt);
            __builtin_amdgcn_sched_barrier(0);
            stage[c].load(ln, xs[c], lane);
            float v[R::NV];
#pragma unroll
            for (int r = 0; r < RT; ++r) ln.dot(cur[r], &v[r * B], malformed);
#pragma unroll
            for (int i = 0; i < R::NV; ++i) acc[i] += v[i];
        }
        /* the next group's chunk 0 is in the register set chunk NCH used
         * for its successor: move it to ra when NCH is odd (a wait for
         * those loads; odd chunk counts are the narrow-row shapes, one
         * group per wave) */
        if constexpr (NCH % 2u == 1u) {
#pragma unroll
            for (int r = 0; r < RT; ++r) ra[r] = rb[r];
        }
        kq_group_reduce<64, R::N>(acc, lane);
#pragma unroll
        for (int j = 0; j < R::KEEP; ++j) {
            const int idx = R::value_index(lane, j);
            if (idx >= 0) {
                const uint32_t r = (uint32_t)idx / B, b = (uint32_t)idx % B;
                const uint32_t row = g * R::GROUP + r;
                if (row < rows) {
                    const float s = acc[j];
                    y[(size_t)b * rows + row] = s;
                    bad |= !kq_isfinite(s);
                    argmax_merge(best_v[b], best_i[b], s, row);
                }
            }
        }
        g += nwaves;
    }
    if (xbad) kq_flag(status, KQ_DEV_INPUT);
    if (malformed) kq_flag(status, KQ_DEV_MALFORMED);
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
    if (part_v != nullptr) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float bv = best_v[b];
            uint32_t bi = best_i[b];
            wave_argmax(bv, bi);
            if (lane == 0) {
                part_v[(size_t)b * part_stride + wave] = bv;
                part_i[(size_t)b * part_stride + wave] = bi;
                for (uint32_t sl = wave + nwaves; sl < part_stride; sl += nwaves) {
                    part_v[(size_t)b * part_stride + sl] = -__builtin_inff();
                    part_i[(size_t)b * part_stride + sl] = 0xffffffffu;
                }
            }
        }
    }
}

/* ---- argmax over rows of logits (two stages) ---- */
__global__ __launch_bounds__(kThreads) void argmax_partial(const float *__restrict__ logits,
                                                           uint32_t count, float *part_v,
                                                           uint32_t *part_i, uint32_t *status) {
    const uint32_t b = blockIdx.y;
    const float *v = logits + (size_t)b * count;
    const uint32_t wave = (blockIdx.x * kThreads + threadIdx.x) >> 6;
    const uint32_t nwaves = (gridDim.x * kThreads) >> 6;
    float bv = -__builtin_inff();
    uint32_t bi = 0xffffffffu;
    bool bad = false;
    for (uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < count; i += gridDim.x * kThreads) {
        const float f = v[i];
        bad |= !kq_isfinite(f);
        argmax_merge(bv, bi, f, i);
    }
    if (bad) kq_flag(status, KQ_DEV_NUMERIC);
    wave_argmax(bv, bi);
    if ((threadIdx.x & 63u) == 0u) {
        part_v[(size_t)b * nwaves + wave] = bv;
        part_i[(size_t)b * nwaves + wave] = bi;
    }
}

__global__ __launch_bounds__(kThreads) void argmax_final(const float *part_v,
                                                         const uint32_t *part_i,
                                                         uint32_t nparts, uint32_t *ids) {
    __shared__ float sv[kThreads / 64];
    __shared__ uint32_t si[kThreads / 64];
    const uint32_t b = blockIdx.x;
    float bv = -__builtin_inff();
    uint32_t bi = 0xffffffffu;
    for (uint32_t i = threadIdx.x; i < nparts; i += kThreads)
        argmax_merge(bv, bi, part_v[(size_t)b * nparts + i], part_i[(size_t)b * nparts + i]);
    wave_argmax(bv, bi);
    if ((threadIdx.x & 63u) == 0u) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / 64; ++w) argmax_merge(bv, bi, sv[w], si[w]);
        ids[b] = bi;
    }
}

/* Row groups per wave: one group of RT passes per wave when that fills the
 * GPU (small matrices: latency bound, every wave issues its loads at once),
 * otherwise a grid of resident waves that stride over groups with the next
 * group's loads in flight while the current one is reduced. */
constexpr uint32_t kResidentWaves = 256u * 4u * 4u;

uint32_t lanes_for(uint32_t cols) { return cols / 32u; }

uint32_t group_rows(uint32_t cols, uint32_t rt) {
    const uint32_t lanes = lanes_for(cols);
    return (lanes >= 64u ? 1u : 64u / lanes) * rt;
}

/* RT = 1 (one group per wave) for matrices whose RT = 4 grid would leave
 * the GPU under-filled */
uint32_t pick_rt(uint32_t rows, uint32_t cols) {
    const uint32_t groups4 = (rows + group_rows(cols, 4) - 1u) / group_rows(cols, 4);
    return groups4 >= kResidentWaves ? 4u : 1u;
}

/* Threads per workgroup: 512 for one group per wave (the activation image
 * is built once per 8 waves), 256 for the resident grid of RT = 4. */
constexpr int kThreadsRt1 = 512;
constexpr int kThreadsRt4 = 256;

/* Between the two, for one activation column: two rows per wave on a grid
 * of two 256-thread workgroups per CU, each wave striding over row pairs
 * with the next pair's loads in flight. It serves matrices too small for
 * the RT = 4 grid whose rows carry the most bytes per 2048 columns (Q8_0
 * 2,176, Q6_K 1,680: one row per wave leaves too few bytes in flight), in
 * one chunk or several. Measured against one row per wave: Q8_0 4096 x
 * 2048 5.17 -> 4.23 us, Q6_K 4.85 -> 4.55 us, the 10240 x 2560, 6144 x
 * 2560 and 2560 x 6144 Q8_0 projections 13.4 -> 8.5, 8.8 -> 6.6 and
 * 10.4 -> 7.1 us. Q5_1 (1,536 bytes) and Q4_K (1,152) are slower this way
 * (4096 x 2048: 3.61 -> 4.08 and 3.39 -> 3.8 us) and keep one row per
 * wave. */
constexpr int kThreadsRt2 = 256;
constexpr uint32_t kRt2MinChunkBytes = 1680u;
constexpr uint32_t kRt2BlocksPerCu = 2u;

uint32_t rt2_blocks(uint32_t rows) {
    static uint32_t cus = 0u;
    if (cus == 0u) {
        int dev = 0, n = 0;
        cus = hipGetDevice(&dev) == hipSuccess &&
                      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) ==
                          hipSuccess &&
                      n > 0
                  ? (uint32_t)n
                  : 256u;
    }
    const uint32_t per_block = (uint32_t)kThreadsRt2 / 64u * 2u; /* rows */
    uint32_t blocks = (rows + per_block - 1u) / per_block;
    if (blocks > kRt2BlocksPerCu * cus) blocks = kRt2BlocksPerCu * cus;
    return blocks < 1u ? 1u : blocks;
}


/* workgroups of `kernel` (kThreadsRt4 threads) that fit on the device at once */
template <class K>
uint32_t resident_blocks(K kernel) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < 1)
        cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreadsRt4, 0) != hipSuccess ||
        per_cu < 1)
        per_cu = 1;
    return (uint32_t)(per_cu * cus);
}

/* Where a launch's column segment lies: bytes from row to row, the
 * activations' batch stride and, after the first segment, the sums to add
 * to (y itself). */
struct Seg {
    uint32_t row_bytes, x_stride;
    const float *y_prev;
};

/* Launches one segment, or (waves != nullptr) only reports the number of
 * waves it would launch: one group per wave for RT = 1; for RT = 4 as many
 * workgroups as are resident at once, striding over the groups. */
template <uint32_t TYPE, uint32_t COLS, int B>
hipError_t launch_one(const uint8_t *W, uint32_t rows, Seg sg, const float *x, float *y,
                      uint32_t *st, float *pv, uint32_t *pi, uint32_t ps, hipStream_t s,
                      uint32_t *waves) {
    const uint32_t rt = pick_rt(rows, COLS);
    if constexpr (COLS == 2048u && B == 1 && kq::row_bytes<TYPE>(2048u) >= kRt2MinChunkBytes) {
        if (rt == 1u) {
            const uint32_t blocks = rt2_blocks(rows);
            if (waves != nullptr) {
                *waves = blocks * ((uint32_t)kThreadsRt2 / 64u);
                return hipSuccess;
            }
            hipLaunchKernelGGL((matvec_kernel<TYPE, COLS, B, 2, kThreadsRt2>), dim3(blocks),
                               dim3(kThreadsRt2), 0, s, W, rows, sg.row_bytes, x, sg.x_stride, y,
                               sg.y_prev, st, pv, pi, ps);
            return hipGetLastError();
        }
    }
    const uint32_t threads = rt == 4u ? (uint32_t)kThreadsRt4 : (uint32_t)kThreadsRt1;
    const uint32_t waves_per_block = threads / 64u;
    const uint32_t groups = (rows + group_rows(COLS, rt) - 1u) / group_rows(COLS, rt);
    uint32_t blocks = (groups + waves_per_block - 1u) / waves_per_block;
    if (rt == 4u) {
        static const uint32_t resident =
            resident_blocks(matvec_kernel<TYPE, COLS, B, 4, kThreadsRt4>);
        if (blocks > resident) blocks = resident;
    }
    if (blocks < 1u) blocks = 1u;
    if (waves != nullptr) {
        *waves = blocks * waves_per_block;
        return hipSuccess;
    }
    if (rt == 4u)
        hipLaunchKernelGGL((matvec_kernel<TYPE, COLS, B, 4, kThreadsRt4>), dim3(blocks),
                           dim3(threads), 0, s, W, rows, sg.row_bytes, x, sg.x_stride, y,
                           sg.y_prev, st, pv, pi, ps);
    else
        hipLaunchKernelGGL((matvec_kernel<TYPE, COLS, B, 1, kThreadsRt1>), dim3(blocks),
                           dim3(threads), 0, s, W, rows, sg.row_bytes, x, sg.x_stride, y,
                           sg.y_prev, st, pv, pi, ps);
    return hipGetLastError();
}

template <uint32_t TYPE, int B>
hipError_t launch_cols(uint32_t cols, const uint8_t *W, uint32_t rows, Seg sg, const float *x,
                       float *y, uint32_t *st, float *pv, uint32_t *pi, uint32_t ps,
                       hipStream_t s, uint32_t *wv) {
    switch (cols) {
    case 32:
    case 64:
    case 128:
        /* short segments exist only for 32-element blocks */
        if constexpr (kq::small_block<TYPE>()) {
            if (cols == 32) return launch_one<TYPE, 32u, B>(W, rows, sg, x, y, st, pv, pi, ps, s, wv);
            if (cols == 64) return launch_one<TYPE, 64u, B>(W, rows, sg, x, y, st, pv, pi, ps, s, wv);
            return launch_one<TYPE, 128u, B>(W, rows, sg, x, y, st, pv, pi, ps, s, wv);
        }
        break;
    case 256: return launch_one<TYPE, 256u, B>(W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    case 512: return launch_one<TYPE, 512u, B>(W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    case 1024: return launch_one<TYPE, 1024u, B>(W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    case 2048: return launch_one<TYPE, 2048u, B>(W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    default: break;
    }
    return hipErrorInvalidValue;
}

template <int B>
hipError_t launch_b(uint32_t type, uint32_t cols, const uint8_t *W, uint32_t rows, Seg sg,
                    const float *x, float *y, uint32_t *st, float *pv, uint32_t *pi,
                    uint32_t ps, hipStream_t s, uint32_t *wv) {
    switch (type) {
    case KQ_LAUNCH_Q4_K:
        return launch_cols<KQ_LAUNCH_Q4_K, B>(cols, W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    case KQ_LAUNCH_Q6_K:
        return launch_cols<KQ_LAUNCH_Q6_K, B>(cols, W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    case KQ_LAUNCH_Q8_0:
        return launch_cols<KQ_LAUNCH_Q8_0, B>(cols, W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    case KQ_LAUNCH_Q5_K:
        return launch_cols<KQ_LAUNCH_Q5_K, B>(cols, W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    case KQ_LAUNCH_Q5_1:
        return launch_cols<KQ_LAUNCH_Q5_1, B>(cols, W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    case KQ_LAUNCH_IQ4_NL:
        return launch_cols<KQ_LAUNCH_IQ4_NL, B>(cols, W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    default: return hipErrorInvalidValue;
    }
}

/* One launch of matvec_wide over all rows (or, with waves set, only its
 * wave count): like launch_one, a resident striding grid for RT = 4;
 * below that size two rows per wave on the RT = 2 grid for the formats
 * above at one activation column, one row group per wave otherwise. */
template <uint32_t TYPE, int B, uint32_t NCH>
hipError_t launch_wide_n(const uint8_t *W, uint32_t rows, uint32_t row_bytes, uint32_t tail,
                         const float *x, uint32_t x_stride, float *y, uint32_t *st, float *pv,
                         uint32_t *pi, uint32_t ps, hipStream_t s, uint32_t *waves) {
    const uint32_t rt = pick_rt(rows, kWideCols);
    if constexpr (B == 1 && kq::row_bytes<TYPE>(kWideCols) >= kRt2MinChunkBytes) {
        if (rt == 1u) {
            const uint32_t blocks = rt2_blocks(rows);
            if (waves != nullptr) {
                *waves = blocks * ((uint32_t)kThreadsRt2 / 64u);
                return hipSuccess;
            }
            hipLaunchKernelGGL((matvec_wide<TYPE, B, 2, kThreadsRt2, NCH>), dim3(blocks),
                               dim3(kThreadsRt2), 0, s, W, rows, row_bytes, tail, x, x_stride, y,
                               st, pv, pi, ps);
            return hipGetLastError();
        }
    }
    const uint32_t threads = rt == 4u ? (uint32_t)kThreadsRt4 : (uint32_t)kThreadsRt1;
    const uint32_t waves_per_block = threads / 64u;
    const uint32_t groups = (rows + rt - 1u) / rt;
    uint32_t blocks = (groups + waves_per_block - 1u) / waves_per_block;
    if (rt == 4u) {
        static const uint32_t resident =
            resident_blocks(matvec_wide<TYPE, B, 4, kThreadsRt4, NCH>);
        if (blocks > resident) blocks = resident;
    }
    if (blocks < 1u) blocks = 1u;
    if (waves != nullptr) {
        *waves = blocks * waves_per_block;
        return hipSuccess;
    }
    if (rt == 4u)
        hipLaunchKernelGGL((matvec_wide<TYPE, B, 4, kThreadsRt4, NCH>), dim3(blocks),
                           dim3(threads), 0, s, W, rows, row_bytes, tail, x, x_stride, y, st, pv,
                           pi, ps);
    else
        hipLaunchKernelGGL((matvec_wide<TYPE, B, 1, kThreadsRt1, NCH>), dim3(blocks),
                           dim3(threads), 0, s, W, rows, row_bytes, tail, x, x_stride, y, st, pv,
                           pi, ps);
    return hipGetLastError();
}

/* chunk counts with an instance: 2 .. 5 at one batch column, 2 .. 3 at two,
 * 2 at three (the LDS holds one activation image per chunk and column) */
constexpr bool wide_shape(uint32_t nch, uint32_t batch) {
    return batch == 1u ? (nch >= 2u && nch <= 5u)
                       : batch == 2u ? (nch == 2u || nch == 3u) : batch == 3u && nch == 2u;
}

template <uint32_t TYPE>
hipError_t launch_wide_t(uint32_t nch, uint32_t batch, const uint8_t *W, uint32_t rows,
                         uint32_t row_bytes, uint32_t tail, const float *x, uint32_t x_stride,
                         float *y, uint32_t *st, float *pv, uint32_t *pi, uint32_t ps,
                         hipStream_t s, uint32_t *wv) {
#define KQ_WIDE(BB, N)                                                                        \
    if (batch == BB && nch == N)                                                              \
    return launch_wide_n<TYPE, BB, N>(W, rows, row_bytes, tail, x, x_stride, y, st, pv, pi, ps, \
                                      s, wv)
    KQ_WIDE(1, 2u);
    KQ_WIDE(1, 3u);
    KQ_WIDE(1, 4u);
    KQ_WIDE(1, 5u);
    KQ_WIDE(2, 2u);
    KQ_WIDE(2, 3u);
    KQ_WIDE(3, 2u);
#undef KQ_WIDE
    return hipErrorInvalidValue;
}

hipError_t launch_wide(uint32_t type, uint32_t nch, uint32_t batch, const uint8_t *W,
                       uint32_t rows, uint32_t row_bytes, uint32_t tail, const float *x,
                       uint32_t x_stride, float *y, uint32_t *st, float *pv, uint32_t *pi,
                       uint32_t ps, hipStream_t s, uint32_t *wv) {
    switch (type) {
#define KQ_WIDE_T(T)                                                                          \
    case T:                                                                                   \
        return launch_wide_t<T>(nch, batch, W, rows, row_bytes, tail, x, x_stride, y, st, pv, \
                                pi, ps, s, wv)
        KQ_WIDE_T(KQ_LAUNCH_Q4_K);
        KQ_WIDE_T(KQ_LAUNCH_Q6_K);
        KQ_WIDE_T(KQ_LAUNCH_Q8_0);
        KQ_WIDE_T(KQ_LAUNCH_Q5_K);
        KQ_WIDE_T(KQ_LAUNCH_Q5_1);
        KQ_WIDE_T(KQ_LAUNCH_IQ4_NL);
#undef KQ_WIDE_T
    default: return hipErrorInvalidValue;
    }
}

/* block elements and bytes of the product formats (0 for others) */
void block_geometry(uint32_t type, uint32_t &be, uint32_t &bb) {
    switch (type) {
    case KQ_LAUNCH_Q4_K: be = 256u; bb = 144u; return;
    case KQ_LAUNCH_Q5_K: be = 256u; bb = 176u; return;
    case KQ_LAUNCH_Q6_K: be = 256u; bb = 210u; return;
    case KQ_LAUNCH_Q8_0: be = 32u; bb = 34u; return;
    case KQ_LAUNCH_Q5_1: be = 32u; bb = 24u; return;
    case KQ_LAUNCH_IQ4_NL: be = 32u; bb = 18u; return;
    default: be = 0u; bb = 0u; return;
    }
}

/* the widest segment (2048 .. 256, and 128 .. 32 for 32-element blocks)
 * that fits in `left` columns */
uint32_t segment_cols(uint32_t be, uint32_t left) {
    for (uint32_t c = 2048u; c >= be && c >= 32u; c >>= 1)
        if (c <= left) return c;
    return 0u;
}

hipError_t launch_batch(uint32_t type, uint32_t cols, const uint8_t *W, uint32_t rows, Seg sg,
                        const float *x, uint32_t batch, float *y, uint32_t *st, float *pv,
                        uint32_t *pi, uint32_t ps, hipStream_t s, uint32_t *wv) {
    switch (batch) {
    case 1: return launch_b<1>(type, cols, W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    case 2: return launch_b<2>(type, cols, W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    case 3: return launch_b<3>(type, cols, W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    case 4: return launch_b<4>(type, cols, W, rows, sg, x, y, st, pv, pi, ps, s, wv);
    default: return hipErrorInvalidValue;
    }
}

/* A row of any whole number of blocks is cut into segments of supported
 * widths, widest first; each segment is one launch over all rows, and the
 * ones after the first add to y. Only the last segment's launch writes the
 * argmax partials (over the finished sums); with wv set, only that
 * launch's wave count is reported and nothing is launched. */
hipError_t dispatch(uint32_t type, const void *W, uint32_t rows, uint32_t cols, const float *x,
                    uint32_t batch, float *y, uint32_t *status, float *pv, uint32_t *pi,
                    uint32_t ps, hipStream_t stream, uint32_t *wv) {
    uint32_t be, bb;
    block_geometry(type, be, bb);
    if (be == 0u || cols == 0u || cols % be != 0u) return hipErrorInvalidValue;
    const uint8_t *w = (const uint8_t *)W;
    const uint32_t row_bytes = cols / be * bb;
    /* rows wider than one engine width: one launch when a chunk count has
     * an instance */
    const uint32_t nch = (cols + kWideCols - 1u) / kWideCols;
    if (cols > kWideCols && wide_shape(nch, batch))
        return launch_wide(type, nch, batch, w, rows, row_bytes, cols - (nch - 1u) * kWideCols, x,
                           cols, y, status, pv, pi, ps, stream, wv);
    uint32_t off = 0u;
    while (off < cols) {
        const uint32_t seg = segment_cols(be, cols - off);
        if (seg == 0u) return hipErrorInvalidValue;
        const bool last = off + seg == cols;
        if (wv == nullptr || last) {
            const Seg sg{row_bytes, cols, off == 0u ? nullptr : y};
            const hipError_t e = launch_batch(
                type, seg, w == nullptr ? nullptr : w + off / be * bb, rows, sg,
                x == nullptr ? nullptr : x + off, batch, y, status, last ? pv : nullptr,
                last ? pi : nullptr, ps, stream, last ? wv : nullptr);
            if (e != hipSuccess) return e;
        }
        off += seg;
    }
    return hipSuccess;
}

}  // namespace

/* at most 32 segment launches per product */
constexpr uint32_t kMaxCols = 65536u;

extern "C" int kq_launch_matvec_supported(uint32_t type, uint32_t cols, uint32_t batch) {
    if (batch < 1u || batch > 4u) return 0;
    uint32_t be, bb;
    block_geometry(type, be, bb);
    return be != 0u && cols != 0u && cols % be == 0u && cols <= kMaxCols;
}

extern "C" uint32_t kq_launch_matvec_waves(uint32_t type, uint32_t rows, uint32_t cols,
                                           uint32_t batch) {
    if (kq_launch_matvec_mfma_supported(type, rows, cols, batch))
        return kq_launch_matvec_mfma_waves(rows, cols);
    uint32_t waves = 0u;
    if (dispatch(type, nullptr, rows, cols, nullptr, batch, nullptr, nullptr, nullptr, nullptr,
                 0u, nullptr, &waves) != hipSuccess)
        return 0u;
    return waves;
}

extern "C" hipError_t kq_launch_matvec(uint32_t type, const void *W, uint32_t rows,
                                       uint32_t cols, const float *x, uint32_t batch, float *y,
                                       uint32_t *status, float *part_v, uint32_t *part_i,
                                       uint32_t part_stride, hipStream_t stream) {
    if (kq_launch_matvec_mfma_supported(type, rows, cols, batch))
        return kq_launch_matvec_mfma(W, rows, cols, x, batch, y, status, part_v, part_i,
                                     part_stride, stream);
    return dispatch(type, W, rows, cols, x, batch, y, status, part_v, part_i, part_stride, stream,
                    nullptr);
}

extern "C" uint32_t kq_launch_argmax_parts(uint32_t count) {
    uint32_t blocks = (count + kThreads * 8u - 1u) / (kThreads * 8u);
    if (blocks > 1024u) blocks = 1024u;
    if (blocks < 1u) blocks = 1u;
    return blocks * (kThreads / 64u);
}

extern "C" hipError_t kq_launch_argmax(const float *logits, uint32_t count, uint32_t batch,
                                       float *part_v, uint32_t *part_i, uint32_t *ids,
                                       uint32_t *status, hipStream_t stream) {
    const uint32_t parts = kq_launch_argmax_parts(count);
    hipLaunchKernelGGL(argmax_partial, dim3(parts / (kThreads / 64u), batch), dim3(kThreads), 0,
                       stream, logits, count, part_v, part_i, status);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_final, dim3(batch), dim3(kThreads), 0, stream, part_v, part_i,
                       parts, ids);
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_argmax_from_parts(const float *part_v, const uint32_t *part_i,
                                                  uint32_t nparts, uint32_t batch, uint32_t *ids,
                                                  hipStream_t stream) {
    hipLaunchKernelGGL(argmax_final, dim3(batch), dim3(kThreads), 0, stream, part_v, part_i,
                       nparts, ids);
    return hipGetLastError();
}
