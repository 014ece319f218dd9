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
// append: every wave packs rows in turn, lane = channel
// ---------------------------------------------------------------------------

// The code of x under the boundaries bnd[0 .. n_b), #{i : (x << s) > norm * bnd[i]}
// (quantize.py:183-196). With the boundaries non-decreasing and norm >= 0 the compare is
// true for a prefix of i, so the count is found by bisection: log2(n_b + 1) compares.
__device__ __forceinline__ int encode_bisect(int64_t x, int64_t norm, const int64_t *bnd, int bits,
                                             int norm_frac) {
    const int64_t xs = x << (CENT_FRAC + norm_frac - QK_FRAC);
    const int n_b = (1 << bits) - 1;
    int c = 0;
    for (int step = 1 << (bits - 1); step > 0; step >>= 1) {
        const int i = c + step - 1;
        if (i < n_b && xs > norm * bnd[i]) c += step;
    }
    return c;
}

// One wave: the norm and codes of a field in registers (lane = channel): the codes into
// c (registers) and codes[0 .. d) (LDS, for the widths the register packer does not take).
template <int CPL>
__device__ __forceinline__ int64_t encode_field_fast(const int64_t (&x)[CPL], int d, int norm_frac,
                                                     const int64_t *__restrict__ bnd, int bits, bool bisect,
                                                     int (&c)[CPL], uint8_t *codes, bool to_lds) {
    const int lane = threadIdx.x & 63;
    const int64_t n = norm_wire<CPL>(x, d, norm_frac);
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
        const int ch = lane + 64 * q;
        c[q] = bisect ? encode_bisect(x[q], n, bnd, bits, norm_frac)
                      : encode_one(x[q], n, bnd, (1 << bits) - 1, norm_frac);
        if (to_lds && ch < d) codes[ch] = (uint8_t)c[q];
    }
    return n;
}

// Rows in (sequence, KV head, token) order, token fastest, so that the waves of a
// workgroup write neighbouring rows of each plane. Each wave takes rows wave, wave + W,
// ... (W waves in the grid) and loads its next row's k and v while it encodes the current
// one. ROT: the rows are wire values and are rotated first (the decode step's rotation,
// rotate.py:170-197), so that a prompt's k/v go from the wire to the cache in one pass.
constexpr int APPEND_WAVES = 4;

template <int CPL, bool ROT>
__global__ void __launch_bounds__(64 * APPEND_WAVES) append_kernel(
        Geom g, const Tables *__restrict__ tabs, const int32_t *__restrict__ k, const int32_t *__restrict__ v,
        int n_tok, int seq_lo, const int64_t *__restrict__ len_in, int64_t *len_out, int seq_hi, int rounds,
        RotSigns sg, DevStats *st) {
    __shared__ uint8_t codes[APPEND_WAVES][2][MAX_D];
    __shared__ int64_t bnd[2][255];
    // wv is uniform in the wave: the row indices below are then scalar
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    stage_bounds(tabs, g, bnd);
    // The length bookkeeping rides on workgroup 0: len_out = len_in + n_tok for the
    // sequences this call appends to, len_in elsewhere (double-buffered so no
    // workgroup can observe a half-updated length).
    if (blockIdx.x == 0) {
        for (int i = threadIdx.x; i < g.batch; i += blockDim.x)
            len_out[i] = len_in[i] + ((i >= seq_lo && i < seq_hi) ? n_tok : 0);
    }
    const bool bisect = tabs->bnd_sorted != 0;
    const bool regpack = (32 % g.kb) == 0 && (32 % g.vb) == 0;   // widths 1, 2, 4, 8
    // where this lane's stores go, relative to a row's (sequence, KV head) and token
    const RegPackLocs<CPL> locs = reg_pack_locs<CPL>(g);
    const WordLoc myloc = word_loc(g, lane < g.row_bytes / 4 ? lane : 0);
    __syncthreads();
    const int d = g.d;
    // Wave w takes the contiguous rows [w R, (w + 1) R) of the (sequence, KV head, token)
    // order: its first row's indices by division, then token by token.
    const int64_t rows = (int64_t)(seq_hi - seq_lo) * g.n_kv * n_tok;
    const int64_t nwaves = (int64_t)gridDim.x * APPEND_WAVES;
    const int64_t per = (rows + nwaves - 1) / nwaves;
    const int64_t r0 = ((int64_t)blockIdx.x * APPEND_WAVES + wv) * per;
    const int64_t r1 = r0 + per < rows ? r0 + per : rows;
    if (r0 >= r1) return;
    int t = (int)(r0 % n_tok);
    int h = (int)((r0 / n_tok) % g.n_kv);
    int bb = (int)(r0 / ((int64_t)n_tok * g.n_kv));          // sequence - seq_lo
    auto src_of = [&](int b_, int t_, int h_) { return (((int64_t)b_ * n_tok + t_) * g.n_kv + h_) * d; };
    int32_t kn[CPL], vn[CPL];
    load_vec<CPL>(k + src_of(bb, t, h), d, kn);
    load_vec<CPL>(v + src_of(bb, t, h), d, vn);
    int64_t base_len = len_in[seq_lo + bb];
    for (int64_t r = r0; r < r1; ++r) {
        int32_t kc[CPL], vc[CPL];
#pragma unroll
        for (int q = 0; q < CPL; ++q) {
            kc[q] = kn[q];
            vc[q] = vn[q];
        }
        const int b = seq_lo + bb;
        const int hh = h;
        const int64_t pos = base_len + t;
        // the next row's indices, and its k and v in flight while this one is encoded
        if (++t == n_tok) {
            t = 0;
            if (++h == g.n_kv) {
                h = 0;
                ++bb;
            }
        }
        if (r + 1 < r1) {
            load_vec<CPL>(k + src_of(bb, t, h), d, kn);
            load_vec<CPL>(v + src_of(bb, t, h), d, vn);
        }
        if (pos >= g.capacity) {     // the host checks capacity first; this only guards memory
            if (lane == 0) atomicAdd(&st->fault, 1ull);
        } else {
            if (ROT) {
                rotate_loaded<CPL>(kc, d, rounds, sg, kc, &st->range_errors);
                rotate_loaded<CPL>(vc, d, rounds, sg, vc, &st->range_errors);
            }
            int64_t xk[CPL], xv[CPL];
#pragma unroll
            for (int q = 0; q < CPL; ++q) {
                xk[q] = kc[q];
                xv[q] = vc[q];
            }
            int ck[CPL], cv[CPL];
            const int64_t nk = encode_field_fast<CPL>(xk, d, g.norm_frac, bnd[0], g.kb, bisect, ck, codes[wv][0], !regpack);
            const int64_t nv = encode_field_fast<CPL>(xv, d, g.norm_frac, bnd[1], g.vb, bisect, cv, codes[wv][1], !regpack);
            if (regpack) {
                pack_store_row_regs<CPL>(g, locs, ck, cv, nk, nv, b, hh, pos);
            } else {
                __builtin_amdgcn_wave_barrier();         // the wave's codes, written above, read below
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (lane < g.row_bytes / 4) *word_ptr(g, myloc, b, hh, pos) = pack_row_word(g, codes[wv], nk, nv, lane);
                __builtin_amdgcn_wave_barrier();         // the codes are read before the next row's
            }
        }
        if (seq_lo + bb != b && r + 1 < r1) base_len = len_in[seq_lo + bb];
    }
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
                         int64_t *len_out, DevStats *st, int rounds, const uint64_t (*signs)[2]) {
    const int64_t rows = (int64_t)(seq_hi - seq_lo) * n_tok * g.n_kv;
    if (rows <= 0) return hipSuccess;
    if (rounds < 0 || rounds > 2 || (rounds && !signs)) return hipErrorInvalidValue;
    const RotSigns sg = rounds ? rot_signs(rounds, signs) : RotSigns{};
    // about 8 rows a wave at the most, 4 waves a workgroup, up to 8 workgroups a CU
    int64_t blocks = (rows + 8 * APPEND_WAVES - 1) / (8 * APPEND_WAVES);
    if (blocks > 2048) blocks = 2048;
    if (blocks < 1) blocks = 1;
    dim3 grid((unsigned)blocks), block(64 * APPEND_WAVES);
    const bool rot = rounds > 0;
    if (g.d <= 64) {
        if (rot)
            hipLaunchKernelGGL((append_kernel<1, true>), grid, block, 0, s, g, t, k, v, n_tok, seq_lo, len_in,
                               len_out, seq_hi, rounds, sg, st);
        else
            hipLaunchKernelGGL((append_kernel<1, false>), grid, block, 0, s, g, t, k, v, n_tok, seq_lo, len_in,
                               len_out, seq_hi, rounds, sg, st);
    } else {
        if (rot)
            hipLaunchKernelGGL((append_kernel<2, true>), grid, block, 0, s, g, t, k, v, n_tok, seq_lo, len_in,
                               len_out, seq_hi, rounds, sg, st);
        else
            hipLaunchKernelGGL((append_kernel<2, false>), grid, block, 0, s, g, t, k, v, n_tok, seq_lo, len_in,
                               len_out, seq_hi, rounds, sg, st);
    }
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
