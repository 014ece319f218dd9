// The host half of the block on the GPU, either side of the seam.
//
// In front of the seam (kernel.py:198-249): the q/k/v projections
// (ops/project.py:21-52: fp16 weights and activations, fp32 accumulation),
// the attention scale on q, RoPE (ops/rope.py:144-198) and the one fp -> fixed
// cast (ops/convert.py:44-57), giving the Q8.16 wire rows the attend path
// takes. Behind it (kernel.py:348-356): the Q16 output back to float, and the
// output projection through W_o' (R^-1 folded in, ops/output.py:49-78).
//
// The projections are fp16 products with fp32 accumulation. A decode step (up
// to 4 tokens) runs them as one GEMV kernel of this file that streams the
// weights once and casts its inputs to fp16 itself; a prompt runs them as
// rocBLAS GEMMs behind a cast kernel. The seam epilogue's float steps follow
// numpy's float64 arithmetic operation by operation (no fused multiply-add), so
// that for the same fp32 projections the wire rows are the reference's integers
// exactly. Only the projections' summation order differs from a CPU BLAS.

#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <cmath>
#include <cstdint>
#include <type_traits>

#include "insitu_internal.h"

namespace insitu {

// x fp32 -> fp16, round to nearest even (numerics/fp.py:20-22).
__global__ void f32_to_f16_kernel(const float *__restrict__ x, _Float16 *__restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = (_Float16)x[i];
}

// Q(frac) int32 -> float64 (exact: the value over 2^frac) -> fp16, one rounding
// (kernel.py:354 to_float, then the projection's fp16 cast).
__global__ void fixed_to_f16_kernel(const int32_t *__restrict__ x, _Float16 *__restrict__ y, int64_t n,
                                    double scale) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = (_Float16)((double)x[i] * scale);
}

// y[r][c] += bias[c] in fp32 (ops/project.py:45-46).
__global__ void add_bias_kernel(float *__restrict__ y, const float *__restrict__ bias, int64_t rows,
                                int32_t cols) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < rows * cols) y[i] = y[i] + bias[i % cols];
}

// y (n, out_f) = fp16(x) (n, in_f) . W^T, W fp16 (out_f, in_f) row-major, for n <= GEMV_N
// tokens: the products are exact in fp32 (11 x 11 significant bits) and each is added with
// one rounding (fmaf). fp16(x) from fp32 (FIXED = false) or from Q(frac) int32 through
// float64 (FIXED = true, one rounding, kernel.py:354 to_float).
constexpr int GEMV_N = 4;

// fp16(x / 2^16) for int32 x, rounded to nearest even, in integer steps: |x| rounded to 11
// significant bits (half to even), then scaled, which is exact in fp32 and in fp16 (|x| / 2^16
// < 2^15, inside fp16's range; below 2^-14 the value has at most 2 bits, on fp16's subnormal
// grid). The same value as (_Float16)((double)x / 2^16), for ~20 instructions instead of a
// float64-to-fp16 conversion.
__device__ __forceinline__ float q16_to_f16f(int32_t x) {
    const uint32_t a = x < 0 ? 0u - (uint32_t)x : (uint32_t)x;
    const int msb = 31 - __builtin_clz(a | 1u);
    const int sh = msb > 10 ? msb - 10 : 0;
    uint32_t r = a >> sh;
    const uint32_t rem = a & ((1u << sh) - 1u), half = sh ? 1u << (sh - 1) : 1u;
    r += (sh && (rem > half || (rem == half && (r & 1u)))) ? 1u : 0u;
    const float m = __builtin_ldexpf((float)r, sh - 16);
    return (float)(_Float16)(x < 0 ? -m : m);
}

// The sum of a float over the wave's 64 lanes (in lane 0; a fixed order): within each
// row of 16 lanes by quad permutes and mirrors, then the four rows by readlane.
__device__ __forceinline__ float wave_sum_f32(float v) {
    auto dpp = [](float x, auto ctrl) __attribute__((always_inline)) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                      decltype(ctrl)::value, 0xF, 0xF, false));
    };
    v += dpp(v, std::integral_constant<int, 0xB1>{});     // quad_perm [1,0,3,2]
    v += dpp(v, std::integral_constant<int, 0x4E>{});     // quad_perm [2,3,0,1]
    v += dpp(v, std::integral_constant<int, 0x141>{});    // row_half_mirror
    v += dpp(v, std::integral_constant<int, 0x140>{});    // row_mirror
    auto rl = [](float x, int l) __attribute__((always_inline)) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
    };
    return (rl(v, 0) + rl(v, 16)) + (rl(v, 32) + rl(v, 48));
}
// The columns are split over the workgroup: a workgroup takes GV_RB rows, its 256 lanes 8
// consecutive columns each (2,048 columns a pass). Every lane issues its 16-byte weight loads
// of all GV_RB rows first, then reads its 8 columns of each token's x straight into
// registers, fp16-rounded: no staging of x and no barrier before the arithmetic, so that the
// whole matrix is in flight at once. Each row's partial sums reduce over the wave (DPP,
// readlane) and then over the 4 waves through LDS. GV_RB = 2 for fp32 x and 4 for Q16 x
// (whose conversion through float64 costs more per workgroup): 4.9-5.2 and 5.5 us for the
// 3,072 x 2,048 and 2,048 x 2,048 decode projections, against 6.9 and 6.1 us for one row
// per wave with x staged in LDS first, and 5.9-6.1 / 6.6-6.7 us for 8 rows a workgroup.
// The workgroup's rows row0 + r * rstride (r < GV_RB): each wave's partial sums of row r and
// token t into part[wave][r][t]; the workgroup has passed a barrier when it returns. The
// row's sum is then (part[0] + part[1]) + (part[2] + part[3]).
template <bool FIXED, int GV_RB>
__device__ __forceinline__ void gemv_partials(const uint16_t *__restrict__ w, int32_t out_f, int32_t in_f,
                                              const void *__restrict__ xin, int32_t n, double fscale, int row0,
                                              int rstride, float (*part)[GV_RB][GEMV_N]) {
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const bool q16 = FIXED && fscale == 1.0 / 65536.0;        // the seam's Q16 (uniform)
    float acc[GV_RB][GEMV_N];
#pragma unroll
    for (int r = 0; r < GV_RB; ++r)
#pragma unroll
        for (int t = 0; t < GEMV_N; ++t) acc[r][t] = 0.0f;
    for (int c0 = 0; c0 < in_f; c0 += 2048) {
        const int c = c0 + tid * 8;
        const bool on = c < in_f;                     // in_f is a multiple of 8
        uint4 wq[GV_RB];
#pragma unroll
        for (int r = 0; r < GV_RB; ++r) {
            const int row = row0 + r * rstride < out_f ? row0 + r * rstride : out_f - 1;   // clamped: in bounds
            wq[r] = on ? *(const uint4 *)(w + (int64_t)row * in_f + c) : make_uint4(0, 0, 0, 0);
        }
        float xs[GEMV_N][8];
#pragma unroll
        for (int t = 0; t < GEMV_N; ++t) {
#pragma unroll
            for (int e = 0; e < 8; ++e) xs[t][e] = 0.0f;
            if (t >= n) continue;                    // uniform: only the tokens there are converted
            uint4 a = make_uint4(0, 0, 0, 0), b = make_uint4(0, 0, 0, 0);
            if (on) {
                const uint4 *src = (const uint4 *)((const char *)xin + ((int64_t)t * in_f + c) * 4);
                a = src[0];
                b = src[1];
            }
            const uint32_t wd[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (FIXED)
                    xs[t][e] = q16 ? q16_to_f16f((int32_t)wd[e])
                                   : (float)(_Float16)((double)(int32_t)wd[e] * fscale);
                else
                    xs[t][e] = (float)(_Float16)__builtin_bit_cast(float, wd[e]);
            }
        }
#pragma unroll
        for (int r = 0; r < GV_RB; ++r) {
            _Float16 hw[8];
            __builtin_memcpy(hw, &wq[r], 16);
#pragma unroll
            for (int t = 0; t < GEMV_N; ++t) {
                if (t < n) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[r][t] = fmaf((float)hw[e], xs[t][e], acc[r][t]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < GV_RB; ++r) {
#pragma unroll
        for (int t = 0; t < GEMV_N; ++t) {
            if (t >= n) break;                       // uniform: only the tokens there are
            const float v = wave_sum_f32(acc[r][t]);
            if (lane == 0) part[wv][r][t] = v;
        }
    }
    __syncthreads();
}

template <bool FIXED, int GV_RB>
__global__ __launch_bounds__(256) void gemv_f16_rows_kernel(
    const uint16_t *__restrict__ w, int32_t out_f, int32_t in_f, const void *__restrict__ xin, int32_t n,
    double fscale, const float *__restrict__ bias, float *__restrict__ y) {
    __shared__ float part[4][GV_RB][GEMV_N];
    const int row0 = blockIdx.x * GV_RB, tid = threadIdx.x;
    gemv_partials<FIXED, GV_RB>(w, out_f, in_f, xin, n, fscale, row0, 1, part);
    if (tid < GV_RB * GEMV_N) {
        const int r = tid / GEMV_N, t = tid % GEMV_N, row = row0 + r;
        if (t < n && row < out_f) {
            const float v = (part[0][r][t] + part[1][r][t]) + (part[2][r][t] + part[3][r][t]);
            y[(int64_t)t * out_f + row] = bias ? v + bias[row] : v;
        }
    }
}

// numpy's rint (half to even), then the Q(24, 16) clamp (fixed.py:158-164).
__device__ __forceinline__ int64_t to_fixed_q16(double a, unsigned long long *sat) {
#pragma clang fp contract(off)
    const double r = rint(a * 65536.0);
    const double lo = -(double)(1 << 23), hi = (double)((1 << 23) - 1);
    if (r < lo || r > hi) {
        atomicAdd(sat, 1ull);
        return r < lo ? -(int64_t)(1 << 23) : (int64_t)((1 << 23) - 1);
    }
    return (int64_t)r;
}

// The seam epilogue for one token and one head (one wave, lane = channel pair):
// p = the fp32 projections (q, k, v concatenated), bias added in fp32; q times
// the attention scale in float64; then either to_fixed and fixed-point RoPE
// (cast_after_rope = 0, the board's order) or float RoPE and to_fixed (1).
// RoPE pairs channel j with j + d/2 (the half split, rope.py:144-174).
struct SeamArgs {
    const float *bias;
    int32_t n_q, n_kv, d;
    const int64_t *pos;
    int64_t pos0;
    const int64_t *cos_t, *sin_t;
    int64_t max_pos;
    int32_t frac;
    double attn_scale;
    int32_t cast_after_rope;
    int32_t *q, *k, *v;
    unsigned long long *sat, *range_err;
};

// The seam of one channel pair (j, j + d/2) of head h, token t, from its fp32 projections.
__device__ __forceinline__ void seam_pair(float lo32, float hi32, int64_t t, int h, int j, const SeamArgs &a) {
#pragma clang fp contract(off)
    const int n_q = a.n_q, n_kv = a.n_kv, d = a.d;
    const int half = d / 2;
    const int kind = h < n_q ? 0 : (h < n_q + n_kv ? 1 : 2);       // q, k, v
    const int hh = kind == 0 ? h : (kind == 1 ? h - n_q : h - n_q - n_kv);
    int32_t *dst = kind == 0 ? a.q + (t * n_q + hh) * d : (kind == 1 ? a.k + (t * n_kv + hh) * d
                                                                     : a.v + (t * n_kv + hh) * d);
    const int64_t ps = a.pos ? a.pos[t] : a.pos0 + t;
    const bool rope = kind != 2;
    if (rope && (ps < 0 || ps >= a.max_pos)) {
        if (j == 0) atomicAdd(a.range_err, 1ull);                  // once a row
        return;
    }
    if (a.bias) {
        lo32 = lo32 + a.bias[h * d + j];
        hi32 = hi32 + a.bias[h * d + j + half];
    }
    double lo = (double)lo32, hi = (double)hi32;
    if (kind == 0) {
        lo = lo * a.attn_scale;
        hi = hi * a.attn_scale;
    }
    if (!rope) {
        dst[j] = (int32_t)to_fixed_q16(lo, a.sat);
        dst[j + half] = (int32_t)to_fixed_q16(hi, a.sat);
        return;
    }
    const int64_t c = a.cos_t[ps * half + j], s = a.sin_t[ps * half + j];
    if (a.cast_after_rope) {
        const double cf = (double)c / (double)(1ll << a.frac), sf = (double)s / (double)(1ll << a.frac);
        const double e0 = lo * cf, e1 = hi * sf, e2 = lo * sf, e3 = hi * cf;
        dst[j] = (int32_t)to_fixed_q16(e0 - e1, a.sat);
        dst[j + half] = (int32_t)to_fixed_q16(e2 + e3, a.sat);
    } else {
        const int64_t li = to_fixed_q16(lo, a.sat), hi_ = to_fixed_q16(hi, a.sat);
        // Q(16 + frac), one floor shift at the end; not clamped (the RTL flags range)
        const int64_t ol = (li * c - hi_ * s) >> a.frac;
        const int64_t oh = (li * s + hi_ * c) >> a.frac;
        dst[j] = (int32_t)ol;
        dst[j + half] = (int32_t)oh;
    }
}

__global__ void seam_wire_kernel(const float *__restrict__ p, int64_t n, SeamArgs a) {
    const int heads = a.n_q + 2 * a.n_kv;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    if (wave >= n * heads) return;
    const int64_t t = wave / heads;
    const int h = (int)(wave % heads), half = a.d / 2;
    const float *row = p + t * heads * a.d + (int64_t)h * a.d;
    for (int j = threadIdx.x & 63; j < half; j += 64) seam_pair(row[j], row[j + half], t, h, j, a);
}

// The decode projection of q|k|v fused with the seam epilogue (kernel.py:198-249 for n <=
// GEMV_N tokens). RoPE pairs channel j of a head with j + d/2 and nothing else, so a
// workgroup that computes exactly those two rows (h d + j and h d + j + d/2) has all the
// seam needs: thread t of it adds the bias, scales, rotates and casts token t's pair, and
// writes p as well. No workgroup waits for another. (A ticket per head, the last of its
// workgroups running the head's seam, took 15.6 us against 4.9 + 4.2 for the two launches:
// each workgroup waited out its stores and its ticket.)
__global__ __launch_bounds__(256) void gemv_seam_kernel(const uint16_t *__restrict__ w, int32_t out_f, int32_t in_f,
                                                        const float *__restrict__ x, int32_t n, float *p, SeamArgs a) {
    __shared__ float part[4][2][GEMV_N];
    const int half = a.d / 2;
    const int h = blockIdx.x / half, j = blockIdx.x % half;
    const int row0 = h * a.d + j;
    gemv_partials<false, 2>(w, out_f, in_f, x, n, 0.0, row0, half, part);
    const int t = threadIdx.x;
    if (t < n) {
        const float lo = (part[0][0][t] + part[1][0][t]) + (part[2][0][t] + part[3][0][t]);
        const float hi = (part[0][1][t] + part[1][1][t]) + (part[2][1][t] + part[3][1][t]);
        p[(int64_t)t * out_f + row0] = lo;
        p[(int64_t)t * out_f + row0 + half] = hi;
        seam_pair(lo, hi, t, h, j, a);
    }
}

}  // namespace insitu

using namespace insitu;

namespace {

int fail(int code, const char *msg) { return set_last_error(code, msg); }

#define HIP_TRY(expr, what)                                                                 \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) return set_last_error(INSITU_EHIP, hipGetErrorString(e_));    \
    } while (0)

struct Blas {
    rocblas_handle h = nullptr;
    _Float16 *x16 = nullptr;
    size_t x16_n = 0;
    unsigned long long *counters = nullptr;     // saturated, range errors
};

Blas &blas_of(insitu_ctx *c);

int gemm_f16(insitu_ctx *c, const uint16_t *w, int32_t out_f, int32_t in_f, const _Float16 *x16,
             int64_t n, float *y) {
    Blas &b = blas_of(c);
    if (!b.h) return fail(INSITU_EHIP, "rocBLAS handle");
    const float one = 1.0f, zero = 0.0f;
    // column-major: Y (out x n) = W^T (out x in) X (in x n); W is (out, in) row-major
    const rocblas_status st = rocblas_gemm_ex(
        b.h, rocblas_operation_transpose, rocblas_operation_none, out_f, (rocblas_int)n, in_f, &one, w,
        rocblas_datatype_f16_r, in_f, x16, rocblas_datatype_f16_r, in_f, &zero, y, rocblas_datatype_f32_r,
        out_f, y, rocblas_datatype_f32_r, out_f, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    if (st != rocblas_status_success) return fail(INSITU_EHIP, "rocblas_gemm_ex failed");
    return INSITU_OK;
}

int ensure_x16(insitu_ctx *c, size_t n) {
    Blas &b = blas_of(c);
    if (b.x16_n >= n) return INSITU_OK;
    // the old staging may still feed a GEMM queued on the stream
    if (b.x16) {
        HIP_TRY(hipStreamSynchronize(ctx_stream(c)), "sync");
        hipFree(b.x16);
    }
    b.x16 = nullptr;
    b.x16_n = 0;
    HIP_TRY(hipMalloc(&b.x16, n * sizeof(_Float16)), "hipMalloc");
    b.x16_n = n;
    return INSITU_OK;
}

bool gemv_fits(int64_t n, int32_t in_f) {
    return n <= GEMV_N && in_f % 8 == 0;
}

template <bool FIXED>
int gemv(insitu_ctx *c, const uint16_t *w, int32_t out_f, int32_t in_f, const void *x, int64_t n, double fscale,
         const float *bias, float *y) {
    constexpr int RB = 2;
    hipLaunchKernelGGL((gemv_f16_rows_kernel<FIXED, RB>), dim3((unsigned)((out_f + RB - 1) / RB)), dim3(256), 0,
                       ctx_stream(c), w, out_f, in_f, x, (int32_t)n, fscale, bias, y);
    HIP_TRY(hipGetLastError(), "gemv");
    return INSITU_OK;
}

}  // namespace

// One rocBLAS handle, staging buffer and counter pair per context, made on first
// use on the context's device and stream, released by insitu_ctx_destroy.
namespace {
Blas &blas_of(insitu_ctx *c) {
    void *&p = ctx_blas(c);
    if (!p) p = new Blas();
    Blas &b = *(Blas *)p;
    if (!b.h) {
        if (rocblas_create_handle(&b.h) != rocblas_status_success) b.h = nullptr;
        if (b.h) rocblas_set_stream(b.h, ctx_stream(c));
        if (!b.counters && hipMalloc(&b.counters, 2 * sizeof(unsigned long long)) != hipSuccess)
            b.counters = nullptr;
    }
    return b;
}
}  // namespace

namespace {
// The seam's counts into counts_host (when given): {saturated, rows beyond the RoPE table}.
int seam_counts(insitu_ctx *c, unsigned long long *counts_host) {
    Blas &b = blas_of(c);
    if (counts_host) {
        HIP_TRY(hipMemcpyAsync(counts_host, b.counters, 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost,
                               ctx_stream(c)),
                "counts");
        HIP_TRY(hipStreamSynchronize(ctx_stream(c)), "sync");
        if (counts_host[1]) return fail(INSITU_ERANGE, "a position beyond the RoPE table (rope.py:163-167)");
    }
    return INSITU_OK;
}
}  // namespace

void insitu::blas_release(insitu_ctx *c) {
    Blas *b = (Blas *)ctx_blas(c);
    if (!b) return;
    if (b->h) rocblas_destroy_handle(b->h);
    if (b->x16) hipFree(b->x16);
    if (b->counters) hipFree(b->counters);
    delete b;
    ctx_blas(c) = nullptr;
}

extern "C" {

int insitu_project(insitu_ctx *c, const uint16_t *w, int32_t out_f, int32_t in_f, const float *x, int64_t n,
                   const float *bias, float *y) {
    if (!c || !w || (n && (!x || !y))) return fail(INSITU_EINVAL, "null argument");
    if (out_f <= 0 || in_f <= 0 || n < 0) return fail(INSITU_EBADLEN, "bad projection shape");
    if (n == 0) return INSITU_OK;
    HIP_TRY(hipSetDevice(ctx_device(c)), "hipSetDevice");
    if (gemv_fits(n, in_f)) return gemv<false>(c, w, out_f, in_f, x, n, 0.0, bias, y);
    int rc = ensure_x16(c, (size_t)n * in_f);
    if (rc) return rc;
    Blas &b = blas_of(c);
    const int64_t nx = n * in_f;
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)((nx + 255) / 256)), dim3(256), 0, ctx_stream(c), x,
                       b.x16, nx);
    HIP_TRY(hipGetLastError(), "fp16 cast");
    rc = gemm_f16(c, w, out_f, in_f, b.x16, n, y);
    if (rc) return rc;
    if (bias) {
        const int64_t ny = n * out_f;
        hipLaunchKernelGGL(add_bias_kernel, dim3((unsigned)((ny + 255) / 256)), dim3(256), 0, ctx_stream(c), y,
                           bias, n, out_f);
        HIP_TRY(hipGetLastError(), "bias");
    }
    return INSITU_OK;
}

int insitu_seam_wire(insitu_ctx *c, const float *p, const float *bias, int64_t n, int32_t n_q, int32_t n_kv,
                     int32_t d, const int64_t *pos, int64_t pos0, const int64_t *cos_t, const int64_t *sin_t, int64_t max_pos,
                     int32_t frac, double attn_scale, int32_t cast_after_rope, int32_t *q, int32_t *k,
                     int32_t *v, unsigned long long *counts_host) {
    if (!c || (n && (!p || !cos_t || !sin_t || !q || !k || !v))) return fail(INSITU_EINVAL, "null argument");
    if (n < 0 || n_q <= 0 || n_kv <= 0 || d <= 0 || d % 2 || frac < 0 || frac > 30 || max_pos <= 0)
        return fail(INSITU_EBADLEN, "bad seam shape");
    HIP_TRY(hipSetDevice(ctx_device(c)), "hipSetDevice");
    Blas &b = blas_of(c);
    if (!b.counters) return fail(INSITU_EHIP, "counters");
    if (counts_host) HIP_TRY(hipMemsetAsync(b.counters, 0, 2 * sizeof(unsigned long long), ctx_stream(c)), "memset");
    if (n) {
        const int64_t waves = n * (n_q + 2 * n_kv);
        const SeamArgs a{bias, n_q, n_kv, d, pos, pos0, cos_t, sin_t, max_pos, frac, attn_scale, cast_after_rope,
                         q, k, v, b.counters, b.counters + 1};
        hipLaunchKernelGGL(seam_wire_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, ctx_stream(c), p, n,
                           a);
        HIP_TRY(hipGetLastError(), "seam epilogue");
    }
    return seam_counts(c, counts_host);
}

int insitu_project_seam(insitu_ctx *c, const uint16_t *w, int32_t in_f, const float *x, int64_t n,
                        const float *bias, int32_t n_q, int32_t n_kv, int32_t d, const int64_t *pos, int64_t pos0,
                        const int64_t *cos_t, const int64_t *sin_t, int64_t max_pos, int32_t frac, double attn_scale,
                        int32_t cast_after_rope, float *p, int32_t *q, int32_t *k, int32_t *v,
                        unsigned long long *counts_host) {
    if (!c || !w || (n && (!x || !p || !cos_t || !sin_t || !q || !k || !v))) return fail(INSITU_EINVAL, "null argument");
    if (in_f <= 0 || n < 0 || n_q <= 0 || n_kv <= 0 || d <= 0 || d % 2 || frac < 0 || frac > 30 || max_pos <= 0)
        return fail(INSITU_EBADLEN, "bad projection or seam shape");
    const int32_t heads = n_q + 2 * n_kv;
    const int32_t out_f = heads * d;
    if (!gemv_fits(n, in_f)) {
        const int rc = insitu_project(c, w, out_f, in_f, x, n, nullptr, p);
        if (rc) return rc;
        return insitu_seam_wire(c, p, bias, n, n_q, n_kv, d, pos, pos0, cos_t, sin_t, max_pos, frac, attn_scale,
                                cast_after_rope, q, k, v, counts_host);
    }
    HIP_TRY(hipSetDevice(ctx_device(c)), "hipSetDevice");
    Blas &b = blas_of(c);
    if (!b.counters) return fail(INSITU_EHIP, "counters");
    if (counts_host) HIP_TRY(hipMemsetAsync(b.counters, 0, 2 * sizeof(unsigned long long), ctx_stream(c)), "memset");
    if (n) {
        const SeamArgs a{bias, n_q, n_kv, d, pos, pos0, cos_t, sin_t, max_pos, frac, attn_scale, cast_after_rope,
                         q, k, v, b.counters, b.counters + 1};
        hipLaunchKernelGGL(gemv_seam_kernel, dim3((unsigned)(out_f / 2)), dim3(256), 0, ctx_stream(c), w, out_f,
                           in_f, x, (int32_t)n, p, a);
        HIP_TRY(hipGetLastError(), "projection and seam");
    }
    return seam_counts(c, counts_host);
}

int insitu_output_projection(insitu_ctx *c, const int32_t *out, int64_t n, int32_t width, int32_t frac,
                             const uint16_t *wo, int32_t hidden, const float *bias, float *y) {
    if (!c || !wo || (n && (!out || !y))) return fail(INSITU_EINVAL, "null argument");
    if (n < 0 || width <= 0 || hidden <= 0 || frac < 0 || frac > 62) return fail(INSITU_EBADLEN, "bad shape");
    if (n == 0) return INSITU_OK;
    HIP_TRY(hipSetDevice(ctx_device(c)), "hipSetDevice");
    if (gemv_fits(n, width)) return gemv<true>(c, wo, hidden, width, out, n, std::ldexp(1.0, -frac), bias, y);
    int rc = ensure_x16(c, (size_t)n * width);
    if (rc) return rc;
    Blas &b = blas_of(c);
    const int64_t nx = n * width;
    hipLaunchKernelGGL(fixed_to_f16_kernel, dim3((unsigned)((nx + 255) / 256)), dim3(256), 0, ctx_stream(c), out,
                       b.x16, nx, std::ldexp(1.0, -frac));
    HIP_TRY(hipGetLastError(), "fixed to fp16");
    rc = gemm_f16(c, wo, hidden, width, b.x16, n, y);
    if (rc) return rc;
    if (bias) {
        const int64_t ny = n * hidden;
        hipLaunchKernelGGL(add_bias_kernel, dim3((unsigned)((ny + 255) / 256)), dim3(256), 0, ctx_stream(c), y,
                           bias, n, hidden);
        HIP_TRY(hipGetLastError(), "bias");
    }
    return INSITU_OK;
}

}  // extern "C"
