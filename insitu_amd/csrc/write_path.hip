// The write path: rotation, norm + threshold encode, row packing and the
// plane-layout append (the codec itself is row_codec.h); plus the small test
// hooks (qtab, exp LUT, finalize).
//
// append   cache/compressed.py:64-86 + quantize.py:237-252 + hw/ddr_layout.py:198-214
#include "insitu_internal.h"
#include "query.h"
#include "row_codec.h"

namespace insitu {

// ---------------------------------------------------------------------------
// rotation
// ---------------------------------------------------------------------------

template <int CPL>
__global__ void __launch_bounds__(64) rotate_kernel(const int32_t *__restrict__ x, int32_t *y,
                                                    int64_t n_vec, int d, int rounds, RotSigns sg,
                                                    unsigned long long *range_err) {
    const int64_t vec = blockIdx.x;
    if (vec >= n_vec) return;
    const int lane = threadIdx.x;
    int32_t r[CPL];
    rotate_vec<CPL>(x + vec * d, d, rounds, sg, r, range_err);
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
        int ch = lane + 64 * k;
        if (ch < d) y[vec * d + ch] = r[k];
    }
}


hipError_t launch_rotate(hipStream_t s, const int32_t *x, int32_t *y, int64_t n_vec, int d,
                         int rounds, const uint64_t (*signs)[2], unsigned long long *range_err) {
    if (n_vec <= 0) return hipSuccess;
    if (rounds > 2) return hipErrorInvalidValue;  // the kernel carries two sign diagonals
    const RotSigns sg = rot_signs(rounds, signs);
    dim3 grid((unsigned)n_vec), block(64);
    if (d <= 64)
        hipLaunchKernelGGL(rotate_kernel<1>, grid, block, 0, s, x, y, n_vec, d, rounds, sg, range_err);
    else
        hipLaunchKernelGGL(rotate_kernel<2>, grid, block, 0, s, x, y, n_vec, d, rounds, sg, range_err);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// norm + encode
// ---------------------------------------------------------------------------

template <int CPL>
__global__ void __launch_bounds__(64) encode_kernel(const int32_t *__restrict__ x, int64_t n_vec,
                                                    int d, int norm_frac,
                                                    const int64_t *__restrict__ bnd, int n_b,
                                                    int32_t *norm, uint8_t *codes) {
    __shared__ int64_t sb[256];
    const int lane = threadIdx.x;
    for (int i = lane; i < n_b; i += 64) sb[i] = bnd[i];
    __syncthreads();
    const int64_t vec = blockIdx.x;
    if (vec >= n_vec) return;
    int64_t v[CPL];
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
        int ch = lane + 64 * k;
        v[k] = ch < d ? (int64_t)x[vec * d + ch] : 0;
    }
    int64_t w = norm_wire<CPL>(v, d, norm_frac);
    if (lane == 0) norm[vec] = (int32_t)w;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
        int ch = lane + 64 * k;
        if (ch < d) codes[vec * d + ch] = (uint8_t)encode_one(v[k], w, sb, n_b, norm_frac);
    }
}

hipError_t launch_encode(hipStream_t s, const int32_t *x, int64_t n_vec, int d, int norm_frac,
                         const int64_t *bounds_dev, int n_bounds, int32_t *norm, uint8_t *codes) {
    if (n_vec <= 0) return hipSuccess;
    dim3 grid((unsigned)n_vec), block(64);
    if (d <= 64)
        hipLaunchKernelGGL(encode_kernel<1>, grid, block, 0, s, x, n_vec, d, norm_frac, bounds_dev,
                           n_bounds, norm, codes);
    else
        hipLaunchKernelGGL(encode_kernel<2>, grid, block, 0, s, x, n_vec, d, norm_frac, bounds_dev,
                           n_bounds, norm, codes);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// append: one wave per (sequence, token, kv head) -> one packed row
// ---------------------------------------------------------------------------

template <int CPL>
__global__ void __launch_bounds__(64) append_kernel(Geom g, const Tables *__restrict__ tabs,
                                                    const int32_t *__restrict__ k,
                                                    const int32_t *__restrict__ v, int n_tok,
                                                    int seq_lo, const int64_t *__restrict__ len_in,
                                                    int64_t *len_out, int seq_hi,
                                                    DevStats *st) {
    __shared__ uint8_t codes[2][MAX_D];
    __shared__ int64_t bnd[2][255];
    const int lane = threadIdx.x;
    const int h = blockIdx.x % g.n_kv;
    stage_bounds(tabs, g, bnd);
    const int t = (blockIdx.x / g.n_kv) % n_tok;
    const int b = seq_lo + blockIdx.x / (g.n_kv * n_tok);
    const int d = g.d;

    // The length bookkeeping rides on block 0: len_out = len_in + n_tok for the
    // sequences this call appends to, len_in elsewhere (double-buffered so no
    // block can observe a half-updated length).
    if (blockIdx.x == 0) {
        for (int i = lane; i < g.batch; i += 64)
            len_out[i] = len_in[i] + ((i >= seq_lo && i < seq_hi) ? n_tok : 0);
    }

    const int64_t pos = len_in[b] + t;
    if (pos >= g.capacity) {     // the host checks capacity first; this only guards memory
        if (lane == 0) atomicAdd(&st->fault, 1ull);
        return;
    }
    const int64_t src = (((int64_t)(b - seq_lo) * n_tok + t) * g.n_kv + h) * d;
    __syncthreads();
    int64_t nk, nv;
    {
        int64_t x[CPL];
#pragma unroll
        for (int q = 0; q < CPL; ++q) {
            int ch = lane + 64 * q;
            x[q] = ch < d ? (int64_t)k[src + ch] : 0;
        }
        nk = encode_field<CPL>(x, d, g.norm_frac, bnd[0], (1 << g.kb) - 1, codes[0]);
    }
    {
        int64_t x[CPL];
#pragma unroll
        for (int q = 0; q < CPL; ++q) {
            int ch = lane + 64 * q;
            x[q] = ch < d ? (int64_t)v[src + ch] : 0;
        }
        nv = encode_field<CPL>(x, d, g.norm_frac, bnd[1], (1 << g.vb) - 1, codes[1]);
    }
    __syncthreads();
    pack_store_row(g, codes, nk, nv, b, h, pos);
}

// ---------------------------------------------------------------------------
// the fused decode step's writes (kernel.py:271-284): rotate k, v and q,
// encode and append every (sequence, KV head)'s row, stage the query rows
// ---------------------------------------------------------------------------

// One workgroup per (sequence b, KV head h) and 2 + G waves: wave 0 takes the
// key, wave 1 the value, waves 2 .. 2 + G - 1 the group's query heads. The
// rotated queries go to qr (int32); with qd, also to the chunked attend's fp64
// staging (query.h), which needs G == GF.
template <int CPL>
__global__ void __launch_bounds__((2 + MAX_G) * 64) step_write_kernel(
        Geom g, const Tables *__restrict__ tabs, const int32_t *__restrict__ qw,
        const int32_t *__restrict__ kw, const int32_t *__restrict__ vw, int rounds, RotSigns sg,
        int32_t *qr, double *qd, int32_t *qok, const int64_t *__restrict__ len_in, int64_t *len_out,
        DevStats *st) {
    __shared__ uint8_t codes[2][MAX_D];
    __shared__ int64_t bnd[2][255];
    __shared__ int64_t norms[2];
    __shared__ int ok_s;
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int chain = blockIdx.x;
    const int b = chain / g.n_kv, h = chain % g.n_kv;
    const int d = g.d;

    if (blockIdx.x == 0 && wv == 0) {
        for (int i = lane; i < g.batch; i += 64) len_out[i] = len_in[i] + 1;
    }
    if (threadIdx.x == 0) ok_s = 1;
    stage_bounds(tabs, g, bnd);
    const int64_t pos = len_in[b];
    const bool room = pos < g.capacity;   // the host checks capacity first; this only guards memory
    __syncthreads();
    if (wv < 2) {
        const int32_t *src = (wv == 0 ? kw : vw) + ((int64_t)b * g.n_kv + h) * d;
        int32_t r[CPL];
        rotate_vec<CPL>(src, d, rounds, sg, r, &st->range_errors);
        int64_t x[CPL];
#pragma unroll
        for (int k = 0; k < CPL; ++k) x[k] = r[k];
        const int64_t n = wv == 0
            ? encode_field<CPL>(x, d, g.norm_frac, bnd[0], (1 << g.kb) - 1, codes[0])
            : encode_field<CPL>(x, d, g.norm_frac, bnd[1], (1 << g.vb) - 1, codes[1]);
        if (lane == 0) norms[wv] = n;
    } else if (wv < 2 + g.G) {
        const int qh = h * g.G + (wv - 2);
        const int64_t row = ((int64_t)b * g.n_q + qh) * d;
        int32_t r[CPL];
        rotate_vec<CPL>(qw + row, d, rounds, sg, r, &st->range_errors);
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
            const int ch = lane + 64 * k;
            if (ch < d) qr[row + ch] = r[k];
        }
        if (qd) {
            const bool ok = stage_query_head<CPL>(r, d, wv - 2, qd + (int64_t)chain * d * GF,
                                                  tabs->kc_absmax, &st->range_errors);
            if (lane == 0 && !ok) atomicAnd(&ok_s, 0);
        }
    }
    __syncthreads();
    if (wv == 0) {
        if (room)
            pack_store_row(g, codes, norms[0], norms[1], b, h, pos);
        else if (lane == 0)
            atomicAdd(&st->fault, 1ull);
    }
    if (qd && threadIdx.x == 0) qok[chain] = ok_s;
}

hipError_t launch_step_write(hipStream_t s, const Geom &g, const Tables *t, const int32_t *qw,
                             const int32_t *kw, const int32_t *vw, int rounds,
                             const uint64_t (*signs)[2], int32_t *qr, double *qd, int32_t *qok,
                             const int64_t *len_in, int64_t *len_out, DevStats *st) {
    const int64_t blocks = (int64_t)g.batch * g.n_kv;
    if (blocks <= 0) return hipSuccess;
    if (rounds > 2 || g.G > MAX_G || (qd && g.G != GF) || blocks > 0x7fffffff)
        return hipErrorInvalidValue;
    const RotSigns sg = rot_signs(rounds, signs);
    dim3 grid((unsigned)blocks), block((unsigned)((2 + g.G) * 64));
    if (g.d <= 64)
        hipLaunchKernelGGL(step_write_kernel<1>, grid, block, 0, s, g, t, qw, kw, vw, rounds, sg, qr,
                           qd, qok, len_in, len_out, st);
    else
        hipLaunchKernelGGL(step_write_kernel<2>, grid, block, 0, s, g, t, qw, kw, vw, rounds, sg, qr,
                           qd, qok, len_in, len_out, st);
    return hipGetLastError();
}

hipError_t launch_append(hipStream_t s, const Geom &g, const Tables *t, const int32_t *k,
                         const int32_t *v, int n_tok, int seq_lo, int seq_hi, const int64_t *len_in,
                         int64_t *len_out, DevStats *st) {
    const int64_t blocks = (int64_t)(seq_hi - seq_lo) * n_tok * g.n_kv;
    if (blocks <= 0) return hipSuccess;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    dim3 grid((unsigned)blocks), block(64);
    if (g.d <= 64)
        hipLaunchKernelGGL(append_kernel<1>, grid, block, 0, s, g, t, k, v, n_tok, seq_lo, len_in,
                           len_out, seq_hi, st);
    else
        hipLaunchKernelGGL(append_kernel<2>, grid, block, 0, s, g, t, k, v, n_tok, seq_lo, len_in,
                           len_out, seq_hi, st);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// test hooks
// ---------------------------------------------------------------------------

__global__ void qtab_kernel(const int32_t *__restrict__ q, int n_heads, int d,
                            const int64_t *__restrict__ c, int n_c, int64_t *table) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)n_heads * d * n_c;
    if (i >= total) return;
    const int ci = (int)(i % n_c);
    const int64_t hc = i / n_c;
    table[i] = (int64_t)q[hc] * c[ci];
}

hipError_t launch_qtab(hipStream_t s, const int32_t *q, int n_heads, int d, const int64_t *c_dev,
                       int n_c, int64_t *table) {
    const int64_t total = (int64_t)n_heads * d * n_c;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(qtab_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, q,
                       n_heads, d, c_dev, n_c, table);
    return hipGetLastError();
}

__global__ void exp_lut_kernel(const Tables *__restrict__ t, const int64_t *__restrict__ delta,
                               int64_t n, int32_t *p) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t dl = delta[i];
    p[i] = dl < 0 ? -1 : exp_lut(dl, t->exp_table, t->delta_max);
}

hipError_t launch_exp_lut(hipStream_t s, const Tables *t, const int64_t *delta, int64_t n,
                          int32_t *p) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(exp_lut_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, t,
                       delta, n, p);
    return hipGetLastError();
}

__global__ void finalize_kernel(const int64_t *__restrict__ acc, const int64_t *__restrict__ l,
                                int rows, int d, int64_t *out, int64_t *recip, int32_t *shift) {
    const int r = blockIdx.x;
    if (r >= rows) return;
    Recip rc = reciprocal(l[r]);
    if (threadIdx.x == 0) {
        if (recip) recip[r] = rc.r;
        if (shift) shift[r] = rc.shift;
    }
    for (int j = threadIdx.x; j < d; j += blockDim.x)
        out[(int64_t)r * d + j] = wmul(acc[(int64_t)r * d + j], rc.r) >> rc.shift;
}

hipError_t launch_finalize(hipStream_t s, const int64_t *acc, const int64_t *l, int rows, int d,
                           int64_t *out, int64_t *recip, int32_t *shift) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(finalize_kernel, dim3(rows), dim3(64), 0, s, acc, l, rows, d, out, recip,
                       shift);
    return hipGetLastError();
}

}  // namespace insitu
