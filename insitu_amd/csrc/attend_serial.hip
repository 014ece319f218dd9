// The serial attend kernel: one wave per (sequence, query head), running
// serial_head (attend_online / attend_two_pass token by token). It is the
// INSITU_SERIAL mode and the path for formats the chunked kernel does not
// instantiate.
#include "serial_head.h"

namespace insitu {

constexpr int SERIAL_RS = 272;   // >= the widest row (8b/8b at d=128: 260 B)

template <int CPL>
__global__ void __launch_bounds__(64) attend_serial_kernel(Geom g, const Tables *__restrict__ tabs,
                                                           const int32_t *__restrict__ q,
                                                           int32_t *out,
                                                           const int64_t *__restrict__ len,
                                                           int two_pass, DevStats *st) {
    __shared__ int64_t kc[256], vc[256];
    __shared__ __align__(16) SerialLds<SERIAL_RS> L;
    const int lane = threadIdx.x;
    const int b = blockIdx.x / g.n_q;
    const int qh = blockIdx.x % g.n_q;
    const int kvh = qh / g.G;
    for (int i = lane; i < (1 << g.kb); i += 64) kc[i] = tabs->kc[i];
    for (int i = lane; i < (1 << g.vb); i += 64) vc[i] = tabs->vc[i];
    const int32_t *qrow = q + ((int64_t)b * g.n_q + qh) * g.d;
    for (int c = lane; c < g.d; c += 64) {
        int64_t qv = qrow[c];
        if (qv >= Q_ROT_LIMIT || qv <= -Q_ROT_LIMIT) atomicAdd(&st->range_errors, 1ull);
    }
    __syncthreads();
    serial_head<CPL, SERIAL_RS>(g, tabs, kc, vc, qrow, b, kvh, len[b], two_pass, true, L,
                                out + ((int64_t)b * g.n_q + qh) * g.d, st);
}

hipError_t launch_attend_serial(hipStream_t s, const Geom &g, const Tables *t, const int32_t *q,
                                int32_t *out, const int64_t *len, int two_pass, LaunchEv ev,
                                DevStats *st) {
    const int64_t blocks = (int64_t)g.batch * g.n_q;
    if (blocks <= 0) return hipSuccess;
    if (g.d <= 64)
        hipExtLaunchKernelGGL(attend_serial_kernel<1>, dim3((unsigned)blocks), dim3(64), 0, s,
                              ev.start, ev.stop, 0, g, t, q, out, len, two_pass, st);
    else
        hipExtLaunchKernelGGL(attend_serial_kernel<2>, dim3((unsigned)blocks), dim3(64), 0, s,
                              ev.start, ev.stop, 0, g, t, q, out, len, two_pass, st);
    return hipGetLastError();
}

}  // namespace insitu
