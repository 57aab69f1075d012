/*
 * kq_sample.hip — the token sampler on the device: temperature, top-k,
 * top-p and the categorical draw of src/kq_sampling.c:576-772, with the
 * same ids, the same RNG word and the same float bits.
 *
 * The reference's sums are sequential binary32 (binary64 for the draw) in a
 * fixed order, so they are replayed here in that order, on one wave: the
 * lanes load and exponentiate 64 terms at once, then the wave adds them one
 * after another through v_readlane (every lane holds the same running sum).
 * Everything that does not depend on the order runs wide:
 *
 *   sample_prep   (grid over the vocabulary) scores = logits / temperature,
 *                 the finiteness flag per workgroup, order-preserving u32
 *                 keys (-0 folded onto +0, which compares equal), ids, and
 *                 the by-id probability array cleared;
 *   sort          rocPRIM's radix sort of (key, id) pairs: LSD radix sort is
 *                 stable, so equal scores stay in ascending id order, the
 *                 reference's (score, id) order (src/kq_sampling.c:276-331);
 *   sample_tail   one workgroup: the top-k threshold by binary search in the
 *                 sorted keys, the softmax mass in ascending-score order, the
 *                 top-p walk from the low end, the kept ids' mass again in id
 *                 order (an LDS sort of the kept ids when they fit, else a
 *                 walk over the by-id array), the normalisation, and the
 *                 categorical walk in binary64.
 *
 * Adding +0 to a running sum of non-negative terms leaves it unchanged, so
 * walks over the by-id array may add the zeros of dropped ids: the result
 * is the reference's sum over the kept ids only.
 */
#include <rocprim/device/device_radix_sort.hpp>

#include "kq_device.h"
#include "kq_launch.h"

namespace {

constexpr int kPrepThreads = 256;
constexpr int kTailThreads = 1024;
constexpr uint32_t kKeptCap = 4096; /* kept ids sorted in LDS up to this many */
constexpr int kRun = 8;             /* 64-term chunks a serial walk loads at once */

__device__ __forceinline__ uint32_t order_key(float v) {
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(kPrepThreads) void sample_prep(
    const float *__restrict__ logits, uint32_t count, float temperature, float *__restrict__ scores,
    uint32_t *__restrict__ keys, uint32_t *__restrict__ ids, float *__restrict__ probs,
    uint32_t *__restrict__ bad_per_block, uint32_t *__restrict__ max_per_block) {
    __shared__ uint32_t any;
    __shared__ uint32_t wmax[kPrepThreads / 64];
    if (threadIdx.x == 0) any = 0u;
    __syncthreads();
    const uint32_t i = blockIdx.x * kPrepThreads + threadIdx.x;
    uint32_t key = 0u; /* below every key of a finite score */
    if (i < count) {
        float v = logits[i];
        bool bad = !kq_isfinite(v);
        if (temperature != 1.0f) {
            v = v / temperature;
            bad = bad || !kq_isfinite(v);
        }
        scores[i] = v;
        key = order_key(v);
        keys[i] = key;
        ids[i] = i;
        probs[i] = 0.0f;
        if (bad) any = 1u; /* benign race: every writer stores 1 */
    }
    for (int off = 32; off > 0; off >>= 1) key = max(key, (uint32_t)__shfl_xor((int)key, off));
    if (threadIdx.x % 64u == 0u) wmax[threadIdx.x / 64u] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        bad_per_block[blockIdx.x] = any;
        uint32_t m = wmax[0];
        for (uint32_t w = 1; w < kPrepThreads / 64u; ++w) m = max(m, wmax[w]);
        max_per_block[blockIdx.x] = m;
    }
}

/* the sampler's device result record (host mirror in kq_launch.h) */
using Out = kq_launch_sample_out;

__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

__device__ __forceinline__ double lane_d(double v, int l) {
    const int64_t b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const int hi = __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)b >> 32), l);
    return __longlong_as_double((int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}

/* s + v[lane 0] + v[lane 1] + ... + v[lane 63], each sum rounded */
__device__ __forceinline__ float chain_f(float s, float v) {
#pragma unroll
    for (int l = 0; l < 64; ++l) s = s + lane_f(v, l);
    return s;
}

__device__ __forceinline__ double chain_d(double s, double v) {
#pragma unroll
    for (int l = 0; l < 64; ++l) s = s + lane_d(v, l);
    return s;
}

/* kRun chunks of 64 consecutive values from p[i0..], zero past n */
__device__ __forceinline__ void load_run(const float *p, uint32_t i0, uint32_t n,
                                         float (&w)[kRun]) {
    const uint32_t lane = threadIdx.x % 64u;
#pragma unroll
    for (int u = 0; u < kRun; ++u) {
        const uint32_t i = i0 + 64u * (uint32_t)u + lane;
        w[u] = i < n ? p[i] : 0.0f;
    }
}

/* s + p[0] + p[1] + ... + p[n - 1] (zeros past n), each sum rounded, on one
 * wave whose lanes all hold the running sum. The terms go through LDS 64 x
 * kRun at a time (stage: 2 x 64 x kRun floats) and come back as broadcast
 * reads (every lane the same address), so each term is one dependent add
 * with no lane extraction; the next run's global loads are in flight
 * meanwhile. LDS operations of one wave complete in order, so the wave
 * reads back what its lanes wrote without a barrier. */
__device__ __forceinline__ float serial_sum(const float *p, uint32_t n, float *stage, float s) {
    const uint32_t lane = threadIdx.x % 64u;
    const uint32_t runs = (n + 64u * kRun - 1u) / (64u * kRun);
    float w[kRun], nx[kRun];
    load_run(p, 0u, n, w);
    for (uint32_t r = 0u; r < runs; ++r) {
        load_run(p, (r + 1u) * 64u * kRun, n, nx);
        float *buf = stage + (r & 1u) * 64u * kRun;
#pragma unroll
        for (int u = 0; u < kRun; ++u) buf[64u * (uint32_t)u + lane] = w[u];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const float4 *b4 = reinterpret_cast<const float4 *>(buf);
#pragma unroll
        for (uint32_t j = 0; j < 16u * kRun; ++j) {
            const float4 t = b4[j];
            s = s + t.x;
            s = s + t.y;
            s = s + t.z;
            s = s + t.w;
        }
#pragma unroll
        for (int u = 0; u < kRun; ++u) w[u] = nx[u];
    }
    return s;
}

/* inclusive prefix sums of one int64 per lane across the wave */
__device__ __forceinline__ int64_t wave_scan_i64(int64_t v) {
    const uint32_t lane = threadIdx.x % 64u;
#pragma unroll
    for (uint32_t o = 1u; o < 64u; o <<= 1) {
        const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)v, o, 64);
        const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)((uint64_t)v >> 32), o, 64);
        if (lane >= o) v += (int64_t)(((uint64_t)hi << 32) | lo);
    }
    return v;
}

/* the categorical draw (src/kq_sampling.c:400-447) on one wave: uniform =
 * word / 2^32, threshold = uniform * total, the first kept id whose
 * binary64 running sum exceeds the threshold (walk), else the last kept id
 * while the threshold is below the total; lane 0 writes the record */
template <class Walk>
__device__ __forceinline__ void draw(Out *o, double total, uint32_t last, float last_p,
                                     uint32_t word, Walk walk, uint32_t top_k_retained,
                                     uint32_t retained, float maxp, float norm_sum,
                                     uint32_t canonical) {
    const uint32_t lane = threadIdx.x % 64u;
    if (!__builtin_isfinite(total) || !(total > 0.0) || last == 0xffffffffu) {
        if (lane == 0) o->status = KQ_SAMPLE_NUMERIC_IN_DRAW;
        return;
    }
    const double uniform = (double)word / 4294967296.0;
    const double thr = uniform * total;
    uint32_t sel = 0xffffffffu;
    float selp = 0.0f;
    walk(thr, sel, selp);
    if (sel == 0xffffffffu && thr < total) {
        sel = last;
        selp = last_p;
    }
    if (lane != 0) return;
    if (sel == 0xffffffffu) {
        o->status = KQ_SAMPLE_NUMERIC_IN_DRAW;
        return;
    }
    o->selected = sel;
    o->top_k_retained = top_k_retained;
    o->retained = retained;
    o->selected_probability = selp;
    o->maximum_probability = maxp;
    o->normalized_sum = norm_sum;
    o->uniform = uniform;
    o->status = sel >= canonical ? KQ_SAMPLE_INVALID_TOKEN : KQ_SAMPLE_OK;
}

struct TailArgs {
    const float *scores;  /* by id */
    uint32_t *skeys;       /* ascending */
    uint32_t *sids;
    const uint32_t *keys;  /* by id (the fast path's source) */
    const uint32_t *max_per_block;
    uint32_t fast;         /* 1: build the sorted top from the block maxima;
                              2: every id kept, no sorted order */
    float *probs; /* by id, cleared by sample_prep */
    const uint32_t *bad_per_block;
    uint32_t prep_blocks;
    uint32_t count;
    uint32_t canonical;
    uint32_t top_k;
    float top_p;
    uint32_t word;
    Out *out;
    uint32_t sequential; /* the sequential walk even where a shortcut is certified */
};

/* ascending bitonic sort of one 64-bit value per lane across a wave (no
 * barrier: exchanges through ds_bpermute) */
__device__ __forceinline__ uint64_t wave_sort64(uint64_t v) {
    const uint32_t lane = threadIdx.x % 64u;
#pragma unroll
    for (uint32_t size = 2u; size <= 64u; size <<= 1u) {
#pragma unroll
        for (uint32_t stride = size / 2u; stride > 0u; stride >>= 1u) {
            const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, (int)stride);
            const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), (int)stride);
            const uint64_t o = ((uint64_t)hi << 32) | lo;
            const bool up = (lane & size) == 0u, lower = (lane & stride) == 0u;
            const uint64_t mn = o < v ? o : v, mx = o < v ? v : o;
            v = lower == up ? mn : mx;
        }
    }
    return v;
}

constexpr uint32_t kFastMaxK = 64;      /* top-k the fast path takes */
constexpr uint32_t kFastBlocks = 128;   /* blocks it gathers at most */

/* The k-th largest of up to 1024 block maxima by an MSB-first radix select
 * over 8-bit digits (an LDS histogram per digit), then the gather and sort
 * of the keys >= it. Returns their count, 0 when they do not fit. vals and
 * cand are LDS arrays of kKeptCap entries. Every thread of the workgroup
 * calls it. */
__device__ uint32_t fast_top(const TailArgs &a, uint32_t v, uint32_t *ids_lds, uint32_t *keys_lds) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_sel[2];
    __shared__ uint32_t blk[kFastBlocks];
    __shared__ uint32_t s_nb, s_nc;
    const uint32_t tid = threadIdx.x, lane = tid % 64u, wave = tid / 64u;
    const uint32_t nb = a.prep_blocks;
    uint32_t prefix = 0u, mask = 0u, krem = a.top_k;
    for (int pass = 0; pass < 4; ++pass) {
        const uint32_t shift = 24u - 8u * (uint32_t)pass;
        if (tid < 256u) hist[tid] = 0u;
        __syncthreads();
        if (tid < nb && (v & mask) == prefix) atomicAdd(&hist[(v >> shift) & 255u], 1u);
        __syncthreads();
        if (wave == 0u) {
            /* lane l holds digits 255 - 4l .. 252 - 4l (largest first) */
            uint32_t c[4], tot = 0u;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                c[q] = hist[255u - 4u * lane - (uint32_t)q];
                tot += c[q];
            }
            uint32_t incl = tot;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t y = (uint32_t)__shfl_up((int)incl, off);
                if (lane >= (uint32_t)off) incl += y;
            }
            uint32_t before = incl - tot;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (before < krem && krem <= before + c[q]) {
                    s_sel[0] = 255u - 4u * lane - (uint32_t)q;
                    s_sel[1] = krem - before;
                }
                before += c[q];
            }
        }
        __syncthreads();
        prefix |= s_sel[0] << shift;
        mask |= 255u << shift;
        krem = s_sel[1];
        __syncthreads();
    }
    const uint32_t t0 = prefix;
    /* the blocks that can hold a key >= t0 */
    if (tid == 0u) {
        s_nb = 0u;
        s_nc = 0u;
    }
    __syncthreads();
    if (tid < nb && v >= t0) {
        const uint32_t at = atomicAdd(&s_nb, 1u);
        if (at < kFastBlocks) blk[at] = tid;
    }
    __syncthreads();
    const uint32_t nbl = s_nb;
    if (nbl > kFastBlocks) return 0u;
    /* their keys >= t0, kGather loads in flight per thread */
    constexpr uint32_t kGather = 8u;
    for (uint32_t j0 = 0u; j0 < nbl * kPrepThreads; j0 += kGather * kTailThreads) {
        uint32_t key[kGather], kid[kGather];
#pragma unroll
        for (uint32_t u = 0; u < kGather; ++u) {
            const uint32_t j = j0 + u * kTailThreads + tid;
            kid[u] = j < nbl * kPrepThreads
                         ? blk[j / kPrepThreads] * kPrepThreads + j % kPrepThreads
                         : a.count;
            key[u] = kid[u] < a.count ? a.keys[kid[u]] : 0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < kGather; ++u) {
            if (kid[u] < a.count && key[u] >= t0) {
                const uint32_t at = atomicAdd(&s_nc, 1u);
                if (at < kKeptCap) {
                    keys_lds[at] = key[u];
                    ids_lds[at] = kid[u];
                }
            }
        }
    }
    __syncthreads();
    const uint32_t nc = s_nc;
    if (nc > kKeptCap) return 0u;
    /* sort by (key, id) ascending: bitonic on the 64-bit pair; up to 64
     * entries within wave 0 */
    if (nc <= 64u) {
        if (wave == 0u) {
            uint64_t x = lane < nc ? ((uint64_t)keys_lds[lane] << 32) | ids_lds[lane] : ~0ull;
            x = wave_sort64(x);
            if (lane < nc) {
                keys_lds[lane] = (uint32_t)(x >> 32);
                ids_lds[lane] = (uint32_t)x;
            }
        }
        __syncthreads();
        return nc;
    }
    uint32_t m2 = 1u;
    while (m2 < nc) m2 <<= 1u;
    for (uint32_t i = nc + tid; i < m2; i += kTailThreads) {
        keys_lds[i] = 0xffffffffu;
        ids_lds[i] = 0xffffffffu;
    }
    __syncthreads();
    for (uint32_t size = 2u; size <= m2; size <<= 1u) {
        for (uint32_t stride = size / 2u; stride > 0u; stride >>= 1u) {
            for (uint32_t i = tid; i < m2 / 2u; i += kTailThreads) {
                const uint32_t lo = 2u * i - (i & (stride - 1u));
                const uint32_t hi = lo + stride;
                const bool up = (lo & size) == 0u;
                const uint64_t x = ((uint64_t)keys_lds[lo] << 32) | ids_lds[lo];
                const uint64_t y = ((uint64_t)keys_lds[hi] << 32) | ids_lds[hi];
                if ((x > y) == up) {
                    keys_lds[lo] = (uint32_t)(y >> 32);
                    ids_lds[lo] = (uint32_t)y;
                    keys_lds[hi] = (uint32_t)(x >> 32);
                    ids_lds[hi] = (uint32_t)x;
                }
            }
            __syncthreads();
        }
    }
    /* keys_lds[0 .. nc) / ids_lds[0 .. nc) are the last nc positions of
     * the sorted order */
    return nc;
}

__device__ __forceinline__ void fail(Out *o, uint32_t code) {
    if (threadIdx.x == 0) o->status = code;
}

/* the score of an order key (order_key's inverse; -0 comes back as +0,
 * which gives every weight expf(score - maximum) the same value) */
__device__ __forceinline__ float key_score(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__global__ __launch_bounds__(kTailThreads) void sample_tail(TailArgs a) {
    __shared__ uint32_t s_ids[kKeptCap];
    __shared__ __align__(16) float s_w[kKeptCap];
    /* the fast path's top of the sorted order: positions base .. n - 1 */
    __shared__ uint32_t f_keys[kKeptCap], f_ids[kKeptCap];
    __shared__ uint32_t s_flag;
    __shared__ float s_max_p[kTailThreads / 64];
    __shared__ uint32_t s_u[4];
    __shared__ float s_f[4]; /* [2]: the by-id mass of the wide path */
    __shared__ __align__(16) float s_stage[2 * 64 * kRun];
    __shared__ int64_t s_qsum[kTailThreads / 64];
    __shared__ double s_dsum[kTailThreads / 64];
    __shared__ uint32_t s_ok[kTailThreads / 64], s_last[kTailThreads / 64];
    const uint32_t tid = threadIdx.x, lane = tid % 64u, wave = tid / 64u;
    const uint32_t n = a.count;
    Out *o = a.out;

    if (tid == 0) s_flag = 0u;
    __syncthreads();
    /* the fast path's block maximum is requested with the flags */
    const uint32_t vmax = a.fast == 1u && tid < a.prep_blocks ? a.max_per_block[tid] : 0u;
    for (uint32_t b = tid; b < a.prep_blocks; b += kTailThreads)
        if (a.bad_per_block[b]) s_flag = 1u;
    __syncthreads();
    if (s_flag) return fail(o, KQ_SAMPLE_NUMERIC_BEFORE_DRAW);

    /* The fast path (1 <= k <= 64, at most 1024 prep blocks): t0 = the k-th
     * largest block maximum; at least k keys reach it, so the k-th largest
     * key does, and every key >= t0 sits in a block whose maximum is >= t0.
     * Those blocks' keys >= t0 are gathered and sorted here by (key, id):
     * they are the top of the whole sorted order, its positions lo0 .. n-1,
     * and stay in LDS (a score is its key's inverse). Too many blocks or
     * keys: status FULL_SORT, and the caller sorts everything. */
    uint32_t lo0 = 0u;
    const bool lds_top = a.fast == 1u;
    if (lds_top) {
        const uint32_t got = fast_top(a, vmax, f_ids, f_keys);
        if (got == 0u) return fail(o, KQ_SAMPLE_FULL_SORT);
        lo0 = n - got;
    }
    /* sorted position j (j >= lo0 on the fast path) */
    auto key_at = [&](uint32_t j) { return lds_top ? f_keys[j - lo0] : a.skeys[j]; };
    auto id_at = [&](uint32_t j) { return lds_top ? f_ids[j - lo0] : a.sids[j]; };
    auto score_at = [&](uint32_t j) {
        return lds_top ? key_score(f_keys[j - lo0]) : a.scores[a.sids[j]];
    };

    /* top-k: the first sorted position whose key reaches the k-th largest
     * key (src/kq_sampling.c:660-667) */
    uint32_t top_start = lo0;
    if (a.top_k != 0u && a.fast != 2u) {
        const uint32_t t = key_at(n - a.top_k);
        uint32_t lo = lo0, hi = n - a.top_k; /* first index in [lo, hi] with key >= t */
        while (lo < hi) {
            const uint32_t mid = lo + (hi - lo) / 2u;
            if (key_at(mid) < t) lo = mid + 1u;
            else hi = mid;
        }
        top_start = lo;
    }
    /* the largest score: the sorted order's last, or, with nothing to cut
     * (fast == 2, no sort), the largest block maximum's score (keys of -0
     * and +0 agree, and either gives the same weights) */
    float maximum;
    if (a.fast == 2u) {
        if (wave == 0u) {
            uint32_t m = 0u;
            for (uint32_t b = lane; b < a.prep_blocks; b += 64u) m = max(m, a.max_per_block[b]);
            for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off));
            if (lane == 0) s_u[2] = m;
        }
        __syncthreads();
        const uint32_t m = s_u[2];
        maximum = __uint_as_float((m & 0x80000000u) ? (m & 0x7fffffffu) : ~m);
    } else {
        maximum = score_at(n - 1u);
    }

    /* wave 0: the softmax mass over [top_start, n) in ascending order, then
     * the top-p walk (src/kq_sampling.c:673-697). The mass only feeds the
     * top-p walk and a validity check that cannot fail (the largest weight
     * is expf(0) = 1, the others lie in [0, 1]), so without top-p neither
     * runs. Terms are gathered kRun at a time per lane, so one load latency
     * serves 64 * kRun serial adds. */
    if (wave == 0u) {
        float sum = 0.0f;
        bool bad = false;
        uint32_t keep = top_start;
        if (a.top_p < 1.0f) {
            auto weights = [&](uint32_t j0, float (&w)[kRun]) {
                float sc[kRun];
#pragma unroll
                for (int u = 0; u < kRun; ++u) {
                    const uint32_t j = j0 + 64u * (uint32_t)u + lane;
                    sc[u] = j < n ? score_at(j) : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < kRun; ++u) {
                    const uint32_t j = j0 + 64u * (uint32_t)u + lane;
                    w[u] = j < n ? kq_expf(sc[u] - maximum) : 0.0f;
                    bad = bad || !kq_isfinite(w[u]);
                }
            };
            for (uint32_t j0 = top_start; j0 < n; j0 += 64u * kRun) {
                float w[kRun];
                weights(j0, w);
                /* chunks past n add zeros: skipped */
#pragma unroll
                for (int u = 0; u < kRun; ++u)
                    if (j0 + 64u * (uint32_t)u < n) sum = chain_f(sum, w[u]);
            }
            bad = __ballot(bad) != 0u;
            if (!bad && kq_isfinite(sum) && sum > 0.0f) {
                const float cutoff = 1.0f - a.top_p;
                float c = 0.0f;
                bool found = false;
                for (uint32_t j0 = top_start; j0 < n && !found; j0 += 64u * kRun) {
                    float w[kRun];
                    weights(j0, w);
#pragma unroll
                    for (int u = 0; u < kRun; ++u) {
                        const float p = w[u] / sum;
                        const uint32_t b0 = j0 + 64u * (uint32_t)u;
                        if (b0 >= n || found) break; /* uniform over the wave */
#pragma unroll
                        for (int l = 0; l < 64; ++l) {
                            c = c + lane_f(p, l);
                            const uint32_t at = b0 + (uint32_t)l;
                            if (!found && at < n && (at == n - 1u || c > cutoff)) {
                                found = true;
                                keep = at;
                            }
                        }
                    }
                }
            }
        } else {
            sum = 1.0f;
        }
        if (lane == 0) {
            s_u[0] = bad || !kq_isfinite(sum) || !(sum > 0.0f) ? 1u : 0u;
            s_u[1] = keep;
        }
    }
    __syncthreads();
    if (s_u[0]) return fail(o, KQ_SAMPLE_NUMERIC_BEFORE_DRAW);
    const uint32_t keep = s_u[1];
    const uint32_t kept = n - keep;

    float norm_sum = 0.0f, sum2 = 0.0f;
    if (kept <= kKeptCap) {
        /* the kept ids, sorted by id in LDS (bitonic; ids are distinct; up
         * to 64 within wave 0) */
        uint32_t m2 = 1u;
        while (m2 < kept) m2 <<= 1u;
        if (kept <= 64u) {
            if (wave == 0u) {
                uint64_t x = ~0ull;
                if (lane < kept)
                    x = ((uint64_t)id_at(keep + lane) << 32) |
                        __float_as_uint(kq_expf(score_at(keep + lane) - maximum));
                x = wave_sort64(x);
                s_ids[lane] = lane < kept ? (uint32_t)(x >> 32) : 0xffffffffu;
                s_w[lane] = lane < kept ? __uint_as_float((uint32_t)x) : 0.0f;
            }
            m2 = 0u; /* sorted */
        }
        for (uint32_t i = tid; i < m2; i += kTailThreads) {
            if (i < kept) {
                s_ids[i] = id_at(keep + i);
                s_w[i] = kq_expf(score_at(keep + i) - maximum);
            } else {
                s_ids[i] = 0xffffffffu;
                s_w[i] = 0.0f;
            }
        }
        __syncthreads();
        for (uint32_t size = 2u; size <= m2; size <<= 1u) {
            for (uint32_t stride = size / 2u; stride > 0u; stride >>= 1u) {
                for (uint32_t i = tid; i < m2 / 2u; i += kTailThreads) {
                    const uint32_t lo = 2u * i - (i & (stride - 1u));
                    const uint32_t hi = lo + stride;
                    const bool up = (lo & size) == 0u;
                    const uint32_t x = s_ids[lo], y = s_ids[hi];
                    if ((x > y) == up) {
                        const float wx = s_w[lo];
                        s_ids[lo] = y;
                        s_ids[hi] = x;
                        s_w[lo] = s_w[hi];
                        s_w[hi] = wx;
                    }
                }
                __syncthreads();
            }
        }
        /* the mass again in id order, the normalisation, and the draw
         * (src/kq_sampling.c:701-760, :400-447) */
        if (wave == 0u) {
            bool bad = false;
            float maxp = 0.0f;
            for (uint32_t i0 = 0u; i0 < kept; i0 += 64u) {
                const uint32_t i = i0 + lane;
                sum2 = chain_f(sum2, i < kept ? s_w[i] : 0.0f);
            }
            if (kq_isfinite(sum2) && sum2 > 0.0f) {
                for (uint32_t i0 = 0u; i0 < kept; i0 += 64u) {
                    const uint32_t i = i0 + lane;
                    float p = 0.0f;
                    if (i < kept && s_w[i] > 0.0f) {
                        p = s_w[i] / sum2;
                        bad = bad || !kq_isfinite(p);
                        a.probs[s_ids[i]] = p;
                    }
                    if (i < kept) s_w[i] = p;
                    norm_sum = chain_f(norm_sum, p);
                    maxp = fmaxf(maxp, p);
                }
                for (int off = 32; off > 0; off >>= 1) maxp = fmaxf(maxp, __shfl_xor(maxp, off));
                bad = __ballot(bad) != 0u;
            } else {
                bad = true;
            }
            if (!bad && (!kq_isfinite(norm_sum) || !(norm_sum > 0.0f))) bad = true;
            if (bad) {
                if (lane == 0) o->status = KQ_SAMPLE_NUMERIC_BEFORE_DRAW;
            } else {
                double total = 0.0;
                uint32_t last = 0xffffffffu;
                float last_p = 0.0f;
                for (uint32_t i0 = 0u; i0 < kept; i0 += 64u) {
                    const uint32_t i = i0 + lane;
                    const float p = i < kept ? s_w[i] : 0.0f;
                    total = chain_d(total, (double)p);
                    const uint64_t has = __ballot(p > 0.0f);
                    if (has) {
                        const int hl = 63 - __builtin_clzll(has);
                        last = s_ids[i0 + (uint32_t)hl];
                        last_p = lane_f(p, hl);
                    }
                }
                draw(o, total, last, last_p, a.word, [&](double thr, uint32_t &sel, float &selp) {
                    double cum = 0.0;
                    for (uint32_t i0 = 0u; i0 < kept && sel == 0xffffffffu; i0 += 64u) {
                        const uint32_t i = i0 + lane;
                        const float p = i < kept ? s_w[i] : 0.0f;
                        const double pd = (double)p;
#pragma unroll
                        for (int l = 0; l < 64; ++l) {
                            cum = cum + lane_d(pd, l);
                            const float pl = lane_f(p, l);
                            if (sel == 0xffffffffu && pl > 0.0f && thr < cum) {
                                sel = s_ids[i0 + (uint32_t)l];
                                selp = pl;
                            }
                        }
                    }
                }, n - top_start, kept, maxp, norm_sum, a.canonical);
            }
        }
        return;
    }

    /* many kept ids: weights scattered into the by-id array (every id's when
     * nothing is cut, without the sort), then walks over the whole
     * vocabulary in id order */
    if (a.fast == 2u) {
        for (uint32_t i = tid; i < n; i += kTailThreads) a.probs[i] = kq_expf(a.scores[i] - maximum);
    } else {
        for (uint32_t j = keep + tid; j < n; j += kTailThreads) {
            const uint32_t id = a.sids[j];
            a.probs[id] = kq_expf(a.scores[id] - maximum);
        }
    }
    __syncthreads();
    const uint32_t runs = (n + 64u * kRun - 1u) / (64u * kRun);
    if (wave == 0u) {
        sum2 = serial_sum(a.probs, n, s_stage, sum2);
        if (lane == 0) s_f[2] = sum2;
    }
    __syncthreads();
    sum2 = s_f[2];
    if (!kq_isfinite(sum2) || !(sum2 > 0.0f)) return fail(o, KQ_SAMPLE_NUMERIC_BEFORE_DRAW);
    /* The normalisation, by contiguous segments of whole 64-id chunks, one
     * per wave. Each wave also forms what decides whether the draw's
     * binary64 running sum is exact: when every p is a multiple of 2^-52
     * and their total is at most 2, every running sum is a multiple of
     * 2^-52 below 2, which binary64 holds exactly, so the sequential sums
     * equal the exact prefix sums q = p * 2^52 summed as integers (in any
     * order). Beside it: the segment's integer total and its last id with
     * p > 0. */
    const uint32_t nchunk = (n + 63u) / 64u;
    const uint32_t per_wave = (nchunk + kTailThreads / 64u - 1u) / (kTailThreads / 64u);
    const uint32_t seg0 = wave * per_wave * 64u, seg1 = min(n, (wave + 1u) * per_wave * 64u);
    {
        float maxp = 0.0f;
        bool bad = false, exact = true;
        int64_t qs = 0;
        double ds = 0.0;
        uint32_t lastw = 0xffffffffu;
        for (uint32_t i0 = seg0; i0 < seg1; i0 += 64u) {
            const uint32_t i = i0 + lane;
            float p = 0.0f;
            if (i < seg1) {
                const float w = a.probs[i];
                if (w > 0.0f) {
                    p = w / sum2;
                    bad = bad || !kq_isfinite(p);
                    a.probs[i] = p;
                    maxp = fmaxf(maxp, p);
                }
            }
            const double q = (double)p * 0x1p52;
            exact = exact && q == __builtin_trunc(q);
            qs += (int64_t)q;
            ds += (double)p;
            const uint64_t has = __ballot(p > 0.0f);
            if (has) lastw = i0 + 63u - (uint32_t)__builtin_clzll(has);
        }
        for (int off = 32; off > 0; off >>= 1) maxp = fmaxf(maxp, __shfl_xor(maxp, off));
        for (int off = 32; off > 0; off >>= 1) {
            const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)qs, off);
            const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)((uint64_t)qs >> 32), off);
            qs += (int64_t)(((uint64_t)hi << 32) | lo);
        }
        for (int off = 32; off > 0; off >>= 1) ds += __shfl_xor(ds, off);
        bad = __ballot(bad) != 0u;
        exact = __ballot(!exact) == 0u;
        if (lane == 0) {
            s_max_p[wave] = bad ? -1.0f : maxp;
            s_qsum[wave] = qs;
            s_dsum[wave] = ds;
            s_ok[wave] = exact ? 1u : 0u;
            s_last[wave] = lastw;
        }
    }
    __syncthreads();
    if (wave != 0u) return;
    float maxp = lane < kTailThreads / 64u ? s_max_p[lane] : 0.0f;
    const bool bad = __ballot(maxp < 0.0f) != 0u;
    for (int off = 32; off > 0; off >>= 1) maxp = fmaxf(maxp, __shfl_xor(maxp, off));
    int64_t qtotal = 0;
    bool exact = true;
    uint32_t last = 0xffffffffu;
    for (uint32_t wv = 0; wv < kTailThreads / 64u; ++wv) {
        qtotal += s_qsum[wv];
        exact = exact && s_ok[wv] != 0u;
        if (s_last[wv] != 0xffffffffu) last = s_last[wv];
    }
    exact = exact && qtotal <= ((int64_t)1 << 53) && !a.sequential;
    if (exact) {
        /* the float mass of the normalised values, in id order, and the
         * draw from the exact prefix sums */
        norm_sum = serial_sum(a.probs, n, s_stage, norm_sum);
        if (bad || !kq_isfinite(norm_sum) || !(norm_sum > 0.0f)) {
            if (lane == 0) o->status = KQ_SAMPLE_NUMERIC_BEFORE_DRAW;
            return;
        }
        const double total = (double)qtotal * 0x1p-52;
        const float last_p = last != 0xffffffffu ? a.probs[last] : 0.0f;
        draw(o, total, last, last_p, a.word, [&](double thr, uint32_t &sel, float &selp) {
            /* the first id whose prefix sum passes thr (it has p > 0: the
             * prefix sums never decrease): the segment, then its chunk */
            const double t52 = thr * 0x1p52;
            int64_t base = 0;
            uint32_t wv = 0;
            for (; wv < kTailThreads / 64u; ++wv) {
                if ((double)(base + s_qsum[wv]) > t52) break;
                base += s_qsum[wv];
            }
            if (wv == kTailThreads / 64u) return;
            const uint32_t b0 = wv * per_wave * 64u, b1 = min(n, (wv + 1u) * per_wave * 64u);
            for (uint32_t i0 = b0; i0 < b1; i0 += 64u) {
                const uint32_t i = i0 + lane;
                const float p = i < b1 ? a.probs[i] : 0.0f;
                const int64_t run = base + wave_scan_i64((int64_t)((double)p * 0x1p52));
                const uint64_t hit = __ballot(i < b1 && (double)run > t52);
                if (hit) {
                    const int hl = __builtin_ctzll(hit);
                    sel = i0 + (uint32_t)hl;
                    selp = lane_f(p, hl);
                    return;
                }
                const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)run, 63);
                const uint32_t hi =
                    (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)run >> 32), 63);
                base = (int64_t)(((uint64_t)hi << 32) | lo);
            }
        }, n - top_start, kept, maxp, norm_sum, a.canonical);
        return;
    }
    /* Otherwise the sequential binary64 sums carry rounding, but for
     * non-negative terms every running sum of the walk (and the total its
     * threshold comes from) is within n u total of the exact prefix sum
     * (u = 2^-53, recursive summation), and prefix sums formed here in any
     * order are within the same bound. So when the threshold from these sums
     * lies farther than M = (8 n + 8) u total from the sums just before and
     * at the first id whose sum passes it, the walk selects that id too:
     * the sums before it stay at or below its threshold, the one at it
     * above. Any closer call takes the sequential walk below. */
    if (!bad && !a.sequential) {
        double dtotal = 0.0;
        for (uint32_t wv = 0; wv < kTailThreads / 64u; ++wv) dtotal += s_dsum[wv];
        const double uniform = (double)a.word / 4294967296.0;
        const double thr = uniform * dtotal;
        const double margin = (8.0 * (double)n + 8.0) * 0x1p-53 * dtotal;
        uint32_t cand = 0xffffffffu;
        float cand_p = 0.0f;
        bool sure = false;
        if (kq_isfinite(dtotal) && dtotal > 0.0 && last != 0xffffffffu) {
            double base = 0.0;
            uint32_t wv = 0;
            for (; wv < kTailThreads / 64u; ++wv) {
                if (base + s_dsum[wv] > thr) break;
                base += s_dsum[wv];
            }
            if (wv < kTailThreads / 64u) {
                const uint32_t b0 = wv * per_wave * 64u, b1 = min(n, (wv + 1u) * per_wave * 64u);
                for (uint32_t i0 = b0; i0 < b1; i0 += 64u) {
                    const uint32_t i = i0 + lane;
                    const float p = i < b1 ? a.probs[i] : 0.0f;
                    double run = (double)p;
#pragma unroll
                    for (uint32_t o = 1u; o < 64u; o <<= 1) {
                        const double v = __shfl_up(run, o, 64);
                        if (lane >= o) run += v;
                    }
                    run += base;
                    const uint64_t hit = __ballot(i < b1 && run > thr);
                    if (hit) {
                        const int hl = __builtin_ctzll(hit);
                        const double at = lane_d(run, hl);
                        const double before = hl > 0 ? lane_d(run, hl - 1) : base;
                        cand = i0 + (uint32_t)hl;
                        cand_p = lane_f(p, hl);
                        sure = at - thr > margin && thr - before > margin;
                        break;
                    }
                    base = lane_d(run, 63);
                }
            }
        }
        if (sure) {
            norm_sum = serial_sum(a.probs, n, s_stage, norm_sum);
            if (!kq_isfinite(norm_sum) || !(norm_sum > 0.0f)) {
                if (lane == 0) o->status = KQ_SAMPLE_NUMERIC_BEFORE_DRAW;
                return;
            }
            const float last_p = a.probs[last];
            draw(o, dtotal, last, last_p, a.word, [&](double, uint32_t &sel, float &selp) {
                sel = cand;
                selp = cand_p;
            }, n - top_start, kept, maxp, norm_sum, a.canonical);
            return;
        }
    }
    /* otherwise one pass for the float mass of the normalised values and
     * the binary64 total the draw uses, both in id order; the total's
     * running value at the end of every group of `every` runs is kept in
     * LDS, so the draw walks only the group where the running sum first
     * passes its threshold, starting from the value the full walk would
     * hold there */
    double *s_cp = reinterpret_cast<double *>(s_w); /* kKeptCap / 2 entries */
    const uint32_t every = (runs + kKeptCap / 2u - 1u) / (kKeptCap / 2u);
    double total = 0.0;
    float last_p = 0.0f;
    last = 0xffffffffu;
    {
        float w[kRun], nx[kRun];
        load_run(a.probs, 0u, n, w);
        for (uint32_t r = 0u; r < runs; ++r) {
            load_run(a.probs, (r + 1u) * 64u * kRun, n, nx);
#pragma unroll
            for (int u = 0; u < kRun; ++u) {
#pragma unroll
                for (int l = 0; l < 64; ++l) {
                    const float pl = lane_f(w[u], l);
                    norm_sum = norm_sum + pl;
                    total = total + (double)pl;
                }
                const uint64_t has = __ballot(w[u] > 0.0f);
                if (has) {
                    const int hl = 63 - __builtin_clzll(has);
                    last = (r * kRun + (uint32_t)u) * 64u + (uint32_t)hl;
                    last_p = lane_f(w[u], hl);
                }
                w[u] = nx[u];
            }
            if ((r + 1u) % every == 0u || r + 1u == runs)
                if (lane == 0) s_cp[r / every] = total;
        }
    }
    if (bad || !kq_isfinite(norm_sum) || !(norm_sum > 0.0f)) {
        if (lane == 0) o->status = KQ_SAMPLE_NUMERIC_BEFORE_DRAW;
        return;
    }
    const uint32_t groups = (runs + every - 1u) / every;
    draw(o, total, last, last_p, a.word, [&](double thr, uint32_t &sel, float &selp) {
        /* the first group whose end value passes the threshold; running
         * sums never decrease, so no earlier id can pass it */
        uint32_t g = groups;
        for (uint32_t g0 = 0u; g0 < groups && g == groups; g0 += 64u) {
            const uint32_t gi = g0 + lane;
            const uint64_t hit = __ballot(gi < groups && thr < s_cp[gi]);
            if (hit) g = g0 + (uint32_t)__builtin_ctzll(hit);
        }
        if (g == groups) return;
        double cum = g == 0u ? 0.0 : s_cp[g - 1u];
        const uint32_t end = min(n, (g + 1u) * every * 64u * kRun);
        for (uint32_t i0 = g * every * 64u * kRun; i0 < end && sel == 0xffffffffu; i0 += 64u) {
            const uint32_t i = i0 + lane;
            const float p = i < n ? a.probs[i] : 0.0f;
#pragma unroll
            for (int l = 0; l < 64; ++l) {
                const float pl = lane_f(p, l);
                cum = cum + (double)pl;
                if (sel == 0xffffffffu && pl > 0.0f && thr < cum) {
                    sel = i0 + (uint32_t)l;
                    selp = pl;
                }
            }
        }
    }, n - top_start, kept, maxp, norm_sum, a.canonical);
}

}  // namespace

extern "C" hipError_t kq_launch_sample_sort_bytes(uint32_t count, size_t *bytes) {
    size_t b = 0;
    hipError_t e = rocprim::radix_sort_pairs((void *)nullptr, b, (const uint32_t *)nullptr,
                                             (uint32_t *)nullptr, (const uint32_t *)nullptr,
                                             (uint32_t *)nullptr, count, 0u, 32u, (hipStream_t)0);
    *bytes = b;
    return e;
}

extern "C" int kq_launch_sample_fast(uint32_t count, uint32_t top_k, float top_p) {
    const uint32_t blocks = (count + kPrepThreads - 1u) / kPrepThreads;
    if (top_k >= 1u && top_k <= kFastMaxK && top_k <= blocks && blocks <= 1024u) return 1;
    if ((top_k == 0u || top_k == count) && !(top_p < 1.0f) && count > kKeptCap) return 2;
    return 0;
}

/* full != 0: sort every key (rocPRIM) after the prep; else the fast path,
 * whose tail reports KQ_SAMPLE_FULL_SORT when its top does not fit (then
 * kq_launch_sample_full runs the sort and the tail again on the same prep) */
static hipError_t launch_tail(const kq_launch_sample_args *p, uint32_t fast, hipStream_t s) {
    TailArgs a;
    a.scores = p->scores;
    a.skeys = p->sorted_keys;
    a.sids = p->sorted_ids;
    a.keys = p->keys;
    a.max_per_block = p->max_per_block;
    a.fast = fast;
    a.probs = p->probs;
    a.bad_per_block = p->bad_per_block;
    a.prep_blocks = (p->count + kPrepThreads - 1u) / kPrepThreads;
    a.count = p->count;
    a.canonical = p->canonical;
    a.top_k = p->top_k;
    a.top_p = p->top_p;
    a.word = p->word;
    a.out = p->out;
    a.sequential = p->sequential_draw;
    hipLaunchKernelGGL(sample_tail, dim3(1), dim3(kTailThreads), 0, s, a);
    return hipGetLastError();
}

extern "C" hipError_t kq_launch_sample(const kq_launch_sample_args *p, hipStream_t s) {
    const uint32_t n = p->count;
    if (n == 0u || p->top_k > n) return hipErrorInvalidValue;
    const uint32_t blocks = (n + kPrepThreads - 1u) / kPrepThreads;
    hipLaunchKernelGGL(sample_prep, dim3(blocks), dim3(kPrepThreads), 0, s, p->logits, n,
                       p->temperature, p->scores, p->keys, p->ids, p->probs, p->bad_per_block,
                       p->max_per_block);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int fast = kq_launch_sample_fast(n, p->top_k, p->top_p);
    if (fast) return launch_tail(p, (uint32_t)fast, s);
    return kq_launch_sample_full(p, s);
}

extern "C" hipError_t kq_launch_sample_full(const kq_launch_sample_args *p, hipStream_t s) {
    size_t tmp = p->sort_bytes;
    hipError_t e = rocprim::radix_sort_pairs(p->sort_temp, tmp, p->keys, p->sorted_keys, p->ids,
                                             p->sorted_ids, p->count, 0u, 32u, s);
    if (e != hipSuccess) return e;
    return launch_tail(p, 0u, s);
}
