/*
 * kq_layout.hip — canonical-order copies of the GDN tensors whose GGUF
 * rows or columns are stored in another order.
 *
 * The reference reorders at every call: its provider dots canonical row r
 * with physical row physical_row_for(r), and for GDN_OUT scatters the
 * activation into physical column order first
 * (src/kq_weight_provider.c:205-248, :438-475). Here the weights are
 * gathered once, on the device, into canonical order (whole rows, or whole
 * 128-column units of packed blocks); the ordinary matvec then computes the
 * same products with no per-call gather.
 *
 * The physical index of canonical index c in a region of 48 units of width
 * w (16 key heads x 3 value repeats): group = c / (3w), repeat = c % (3w) / w,
 * feature = c % w, physical = (repeat * 16 + group) * w + feature. A region
 * may follow an identity prefix (the q/k rows of attn_qkv and the conv).
 */
#include "kq_device.h"
#include "kq_launch.h"

namespace {

constexpr int kLayoutThreads = 256;

__device__ __forceinline__ uint64_t grouped_to_tiled(uint64_t c, uint64_t w) {
    const uint64_t group = c / (3u * w), within = c % (3u * w);
    return (within / w * 16u + group) * w + within % w;
}

/* one workgroup per destination unit: unit j of the canonical copy takes
 * physical unit map(j), unit_bytes / 2 halfwords each */
__global__ __launch_bounds__(kLayoutThreads) void gather_units(
    const uint16_t *__restrict__ src, uint16_t *__restrict__ dst, uint64_t units,
    uint32_t unit_half, uint32_t mode, uint64_t prefix, uint32_t width, uint32_t per_row) {
    const uint64_t j = blockIdx.x;
    if (j >= units) return;
    uint64_t from;
    if (mode == 0u) { /* rows: identity prefix, then the permuted region */
        from = j < prefix ? j : prefix + grouped_to_tiled(j - prefix, width);
    } else { /* 128-column units within each row: unit u of a row */
        const uint64_t row = j / per_row, u = j % per_row;
        from = row * per_row + (u % 3u) * 16u + u / 3u;
    }
    const uint16_t *s = src + from * unit_half;
    uint16_t *d = dst + j * unit_half;
    for (uint32_t i = threadIdx.x; i < unit_half; i += kLayoutThreads) d[i] = s[i];
}

}  // namespace

extern "C" hipError_t kq_launch_gdn_gather(const void *physical, void *canonical, uint64_t units,
                                           uint32_t unit_bytes, int columns, uint64_t prefix,
                                           uint32_t width, uint32_t units_per_row,
                                           hipStream_t s) {
    if (units == 0u || units > 0x7fffffffu || unit_bytes == 0u || unit_bytes % 2u != 0u)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gather_units, dim3((uint32_t)units), dim3(kLayoutThreads), 0, s,
                       (const uint16_t *)physical, (uint16_t *)canonical, units, unit_bytes / 2u,
                       columns ? 1u : 0u, prefix, width, units_per_row);
    return hipGetLastError();
}
