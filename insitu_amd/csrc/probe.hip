// Measurement probes: what one launch can read from HBM, and what an empty
// launch costs. They are the GPU analogue of the reference's DDR bandwidth
// probe (rtl/ddr_probe.sv, results/step1_ddr_sweep_run2_medians.log): the
// ceiling the attend's scan is judged against. No value of the attention path
// comes from here.
#include "insitu_internal.h"

using namespace insitu;

namespace {

// Read nbytes (a multiple of 64) with 16-byte loads, four independent loads in
// flight per thread. layout 0: grid-stride (consecutive threads, consecutive
// 16-byte words); layout 1: each workgroup reads one contiguous span, as an
// attend workgroup reads its chunk. The XOR of everything is written only if
// it equals a value it almost surely does not, so the loads stay live and
// nothing else is written.
__global__ void __launch_bounds__(256) probe_read_kernel(const uint4 *__restrict__ src, int64_t n16,
                                                         int32_t layout, uint32_t *sink) {
    uint32_t x = 0;
    int64_t lo, hi, step;
    if (layout == 0) {
        lo = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
        hi = n16;
        step = (int64_t)gridDim.x * blockDim.x;
    } else {
        const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
        const int64_t b0 = (int64_t)blockIdx.x * per;
        lo = b0 + threadIdx.x;
        hi = b0 + per < n16 ? b0 + per : n16;
        step = blockDim.x;
    }
    int64_t i = lo;
    for (; i + 3 * step < hi; i += 4 * step) {
        const uint4 a = src[i], b = src[i + step], c = src[i + 2 * step], d = src[i + 3 * step];
        x ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < hi; i += step) {
        const uint4 a = src[i];
        x ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (x == 0x9E3779B9u) sink[blockIdx.x & 255] = x;
}

__global__ void __launch_bounds__(256) probe_empty_kernel(uint32_t *sink) {
    if (threadIdx.x == 1024) sink[0] = 1;   // never true: blockDim is at most 256
}

}  // namespace

extern "C" {

int insitu_probe_read(insitu_ctx *c, const void *src_dev, int64_t nbytes, int32_t n_wg, int32_t layout,
                      uint32_t *sink_dev) {
    if (!c || !src_dev || !sink_dev) return set_last_error(INSITU_EINVAL, "null argument");
    if (nbytes <= 0 || nbytes % 64) return set_last_error(INSITU_EBADLEN, "nbytes must be a positive multiple of 64");
    if (n_wg < 1 || n_wg > (1 << 20) || (layout != 0 && layout != 1))
        return set_last_error(INSITU_EINVAL, "n_wg in 1 .. 2^20, layout 0 or 1");
    if (hipSetDevice(ctx_device(c)) != hipSuccess) return set_last_error(INSITU_EHIP, "hipSetDevice");
    LaunchEv ev;
    int rc = timing_events(c, &ev);
    if (rc) return rc;
    hipExtLaunchKernelGGL(probe_read_kernel, dim3((unsigned)n_wg), dim3(256), 0, ctx_stream(c), ev.start,
                          ev.stop, 0, (const uint4 *)src_dev, nbytes / 16, layout, sink_dev);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? INSITU_OK : set_last_error(INSITU_EHIP, hipGetErrorString(e));
}

int insitu_probe_empty(insitu_ctx *c, int32_t n_wg, uint32_t *sink_dev) {
    if (!c || !sink_dev) return set_last_error(INSITU_EINVAL, "null argument");
    if (n_wg < 1 || n_wg > (1 << 20)) return set_last_error(INSITU_EINVAL, "n_wg in 1 .. 2^20");
    if (hipSetDevice(ctx_device(c)) != hipSuccess) return set_last_error(INSITU_EHIP, "hipSetDevice");
    LaunchEv ev;
    int rc = timing_events(c, &ev);
    if (rc) return rc;
    hipExtLaunchKernelGGL(probe_empty_kernel, dim3((unsigned)n_wg), dim3(256), 0, ctx_stream(c), ev.start,
                          ev.stop, 0, sink_dev);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? INSITU_OK : set_last_error(INSITU_EHIP, hipGetErrorString(e));
}

}  // extern "C"
