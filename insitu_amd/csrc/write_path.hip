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
// append, lane = row (d = 64, code widths 1, 2 or 4 bits)
// ---------------------------------------------------------------------------
//
// A wave takes 64 consecutive rows of the input's (sequence, token, KV head) order, which
// are 16 KB of contiguous k (and of v): loaded with whole-wave 16-byte loads, turned round
// through LDS (a row per 66 dwords, so that the row reads spread over the banks) and read
// back one row per lane. Each lane then rotates, measures and encodes its own row in
// registers: no cross-lane step at all. The arithmetic is fp64 on integers, exact while
// every value stays below 2^53:
//   - the rotation's values stay below 2^31 * 2^6 * 2^6 * 2^3 (two rounds);
//   - sum(x^2) is exact when the computed sum is below 2^53 (below that every square and
//     partial sum is an integer that a double holds; at or above it, the computed sum is at
//     least 2^53, since rounding to nearest never crosses a representable number); rows at
//     or above take the int64 path, wrapping as the lane-per-channel kernel does;
//   - isqrt by the correctly rounded fp64 sqrt, then corrected as quantize.py:42-60 does;
//   - the half-even requantize is rint of the scaled root (quantize.py:164-181);
//   - a threshold compare (x << e) > n * b_i is x > floor(n * b_i / 2^e) for integer x, in
//     int32 (|n * b_i / 2^e| < 2^31 when |b_i| < 2^24: the launcher checks).
// Rotated values outside int32 are counted as range errors and wrap to int32, as the
// lane-per-channel kernel's rotate_loaded does.
constexpr int AR_WAVES = 4;
constexpr int AR_STRIDE = 66;

// x * s_c / 8, s_c = -1 where bit c of the signs is set (sw: the 32-bit half of the sign
// word that holds bit c): the rotation's sign and its 1/sqrt(64) in one exact multiply. The
// FWHT of x / 8 is FWHT(x) / 8 exactly (its sums keep 3 fractional bits, far below 2^53),
// so floor of it is rotate.py's floor(FWHT(x) / 8).
__device__ __forceinline__ double ar_sign_scale(double x, uint32_t sw, int c) {
    return x * (((sw >> (c & 31)) & 1u) ? -0.125 : 0.125);
}

// The 64-point FWHT of the row (hadamard butterflies, fixed.py fwht), in place.
__device__ __forceinline__ void ar_fwht64(double (&x)[64]) {
#pragma unroll
    for (int H = 1; H < 64; H <<= 1) {
#pragma unroll
        for (int i = 0; i < 64; ++i) {
            if (i & H) continue;
            const double a = x[i], b = x[i + H];
            x[i] = a + b;
            x[i + H] = a - b;
        }
    }
}

// The int64 sum of squares of the row, wrapping, and the norm from it as norm_wire does.
__device__ __forceinline__ int32_t ar_norm_int64(const int32_t (&x)[64], int norm_frac) {
    uint64_t sq = 0;
#pragma unroll
    for (int c = 0; c < 64; ++c) {
        const int64_t xi = x[c];
        sq += (uint64_t)xi * (uint64_t)xi;
    }
    const int64_t mean = (int64_t)sq >> 6;
    int64_t w = rshift_even(isqrt64(mean), QK_FRAC - norm_frac);
    if (w > 32767) w = 32767;
    if (w < -32768) w = -32768;
    return (int32_t)w;
}

// The rotated row's values outside int32, recounted by the whole wave (lane = channel, the
// rotation of rotate_loaded) from the wire row in memory: the rows of the lanes in `need`
// (live lanes whose largest |value| reached 2^31, which is rare), one after another, so that
// the lane = row path keeps no unwrapped copy of its row. Returns this lane's count; adds
// each recounted row's count to range_err.
__device__ __forceinline__ unsigned long long ar_range_recount(uint64_t need, const int32_t *__restrict__ rows0,
                                                               int rounds,
                                                               const RotSigns &sg,
                                                               unsigned long long *range_err) {
    const int lane = threadIdx.x & 63;
    unsigned long long mine = 0;
    while (need) {
        const int j = __builtin_ctzll(need);
        need &= need - 1;
        int64_t x[1] = {rows0[(int64_t)j * 64 + lane]};
        for (int r = 0; r < rounds; ++r) {
            const uint64_t w = r == 0 ? sg.s0a : sg.s1a;
            if ((w >> lane) & 1) x[0] = -x[0];
            fwht_wave<1>(x, 64);
            x[0] = rot_scale(x[0], 64);
        }
        const unsigned long long cnt =
            (unsigned long long)__popcll(__ballot(x[0] < INT32_MIN || x[0] > INT32_MAX));
        if (lane == j) mine = cnt;
        if (lane == 0 && cnt && range_err) atomicAdd(range_err, cnt);
    }
    return mine;
}

// The rotation of a row in registers, lane = row (rotate.py:170-197, rounds 1 or 2): the
// sign and 1/8 in one exact multiply, the FWHT's butterflies, the floor, all in fp64 on
// integers; xr the rotated row as int32 (wrapped), S (when WANT_S) its sum of squares in fp64
// partial sums (exact below 2^53; +inf when values wrapped, so that the caller takes the
// int64 path). Values beyond int32 are counted into range_err for live lanes (recounted by the
// whole wave, lane = channel, from rows0: the fast path keeps no unwrapped copy of the row).
template <bool WANT_S>
__device__ __forceinline__ void ar_rotate_row(const int32_t (&xi)[64], int rounds, const RotSigns &sg, bool live,
                                             const int32_t *rows0, unsigned long long *range_err,
                                             int32_t (&xr)[64], double &S) {
    double x[64];
#pragma unroll
    for (int c = 0; c < 64; ++c) x[c] = (double)xi[c];
    // a round: the signs and 1/8, the FWHT, the floor (rotate.py:170-197); rounds is 1 or 2
    auto round = [&](uint64_t s) {
        // (a fresh copy of the word each round: the key and value fields share it, and
        // factors the compiler shared between them would stay live from one to the other)
        uint32_t slo = (uint32_t)s, shi = (uint32_t)(s >> 32);
        asm volatile("" : "+s"(slo), "+s"(shi));
        // in groups of 8 channels, so that the scalar factors are made where they are used
#pragma unroll
        for (int c = 0; c < 64; ++c) {
            x[c] = ar_sign_scale(x[c], c < 32 ? slo : shi, c);
            if ((c & 7) == 7) __builtin_amdgcn_sched_barrier(0);
        }
        ar_fwht64(x);
#pragma unroll
        for (int c = 0; c < 64; ++c) x[c] = floor(x[c]);
    };
    round(sg.s0a);
    if (rounds > 1) round(sg.s1a);
    double amax = 0.0, s4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int c = 0; c < 64; ++c) {
        amax = fmax(amax, fabs(x[c]));
        if (WANT_S) s4[c & 3] = fma(x[c], x[c], s4[c & 3]);
        // |x| < 2^51: the low dword of x + 1.5 * 2^52 is x mod 2^32, the int32 wrap
        xr[c] = (int32_t)(uint32_t)__double_as_longlong(x[c] + 6755399441055744.0);
    }
    S = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    // rare: values may have wrapped (live lanes only: the others' rows are not stored, and
    // a recount reads rows0 + 64 j only for j below the tile's row count)
    const uint64_t need = __ballot(live && amax >= 2147483648.0);
    if (need) {
        const unsigned long long cnt = ar_range_recount(need, rows0, rounds, sg, range_err);
        if (cnt) S = __builtin_inf();               // the squares are of the wrapped values
    }
}

// One field of a lane's row: xi (int32, the row as loaded) rotated when ROT, its norm
// returned and its codes packed into w (BITS-wide, LSB first, quantize.py:271-289). A lane
// that is not live (past the tile's rows) counts no range errors; rows0 is the tile's first
// row in memory (for the recount).
template <int BITS, bool ROT>
__device__ __forceinline__ int32_t ar_field(const int32_t (&xi)[64], int rounds, const RotSigns &sg,
                                            const int64_t *__restrict__ bnd, int norm_frac, bool live,
                                            const int32_t *rows0, unsigned long long *range_err,
                                            uint32_t (&w)[2 * BITS]) {
    // xr: the row as int32 (rotated and wrapped when ROT); S: sum(x^2) in fp64, in four
    // partial sums (exact below 2^53; +inf sends the row to the int64 path)
    int32_t xr[64];
    double S;
    if constexpr (ROT) {
        ar_rotate_row<true>(xi, rounds, sg, live, rows0, range_err, xr, S);
    } else {
        double s4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int c = 0; c < 64; ++c) {
            xr[c] = xi[c];
            const double xd = (double)xi[c];
            s4[c & 3] = fma(xd, xd, s4[c & 3]);
        }
        S = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    }
    int32_t n;
    if (S < 9007199254740992.0) {
        const double m = floor(S * (1.0 / 64.0));
        double r = floor(sqrt(m));
        if (r * r > m) r -= 1.0;
        if ((r + 1.0) * (r + 1.0) <= m) r += 1.0;
        const double wn = rint(r * __builtin_ldexp(1.0, norm_frac - QK_FRAC));
        n = (int32_t)(wn < 32767.0 ? wn : 32767.0);
    } else {
        n = ar_norm_int64(xr, norm_frac);
    }
    constexpr int NB = (1 << BITS) - 1, PER = 32 / BITS;
    const double sc = __builtin_ldexp(1.0, QK_FRAC - CENT_FRAC - norm_frac);
    const double nd = (double)n;
    int32_t th[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) th[i] = (int32_t)floor(nd * ((double)bnd[i] * sc));
#pragma unroll
    for (int j = 0; j < 2 * BITS; ++j) w[j] = 0;
#pragma unroll
    for (int c = 0; c < 64; ++c) {
        const int32_t xv = xr[c];
        uint32_t code;
        if constexpr (BITS == 4) {
            // #{i : xv > th[i]} by bisection over the sorted thresholds (a prefix of them is
            // below xv): each step halves the candidates, the next threshold chosen by select
            const bool c3 = xv > th[7];
            const bool c2 = xv > (c3 ? th[11] : th[3]);
            const bool c1 = xv > (c3 ? (c2 ? th[13] : th[9]) : (c2 ? th[5] : th[1]));
            const int32_t hi = c2 ? (c1 ? th[14] : th[12]) : (c1 ? th[10] : th[8]);
            const int32_t lo = c2 ? (c1 ? th[6] : th[4]) : (c1 ? th[2] : th[0]);
            const bool c0 = xv > (c3 ? hi : lo);
            code = (uint32_t)c3 * 8u + (uint32_t)c2 * 4u + (uint32_t)c1 * 2u + (uint32_t)c0;
        } else {
            code = 0;
#pragma unroll
            for (int i = 0; i < NB; ++i) code += xv > th[i] ? 1u : 0u;
        }
        w[c / PER] |= code << (BITS * (c % PER));
    }
    return n;
}

// insitu_rotate at d = 64 with one or two rounds, lane = row: a wave takes 64 consecutive
// vectors (16 KB), turned round through LDS as the append does, rotates one per lane
// (ar_rotate_row) and writes them back through LDS with whole-wave 16-byte stores.
__global__ void __launch_bounds__(64 * AR_WAVES) rotate_rows_kernel(const int32_t *__restrict__ x, int32_t *y,
                                                                   int n_vec, int rounds, RotSigns sg,
                                                                   unsigned long long *range_err) {
    __shared__ int32_t tile[AR_WAVES][64 * AR_STRIDE];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r0 = (blockIdx.x * AR_WAVES + wv) * 64;
    if (r0 >= n_vec) return;
    const int nr = n_vec - r0 < 64 ? n_vec - r0 : 64;
    const int sub = lane >> 4, q4 = (lane & 15) * 4;
    uint4 raw[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = 4 * i + sub < nr ? 4 * i + sub : nr - 1;
        raw[i] = *(const uint4 *)(x + ((int64_t)r0 + r) * 64 + q4);
    }
    int32_t *T = tile[wv];
    auto sync = [&]() {
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int32_t *p = T + (4 * i + sub) * AR_STRIDE + q4;
        *(uint2 *)p = make_uint2(raw[i].x, raw[i].y);
        *(uint2 *)(p + 2) = make_uint2(raw[i].z, raw[i].w);
    }
    sync();
    int32_t xi[64];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const uint2 u = *(const uint2 *)(T + lane * AR_STRIDE + 2 * j);
        xi[2 * j] = (int32_t)u.x;
        xi[2 * j + 1] = (int32_t)u.y;
    }
    sync();
    int32_t xr[64];
    double S;
    ar_rotate_row<false>(xi, rounds, sg, lane < nr, x + (int64_t)r0 * 64, range_err, xr, S);
#pragma unroll
    for (int j = 0; j < 32; ++j) *(uint2 *)(T + lane * AR_STRIDE + 2 * j) = make_uint2(xr[2 * j], xr[2 * j + 1]);
    sync();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = 4 * i + sub;
        if (r < nr) {
            const int32_t *p = T + r * AR_STRIDE + q4;
            const uint2 a = *(const uint2 *)p, b = *(const uint2 *)(p + 2);
            *(uint4 *)(y + ((int64_t)r0 + r) * 64 + q4) = make_uint4(a.x, a.y, b.x, b.y);
        }
    }
}

hipError_t launch_rotate(hipStream_t s, const int32_t *x, int32_t *y, int64_t n_vec, int d,
                         int rounds, const uint64_t (*signs)[2], unsigned long long *range_err) {
    if (n_vec <= 0) return hipSuccess;
    if (rounds > 2) return hipErrorInvalidValue;  // the kernel carries two sign diagonals
    const RotSigns sg = rot_signs(rounds, signs);
    // d = 64, one or two rounds, 16-byte aligned vectors, x and y apart: lane = row
    if (d == 64 && rounds >= 1 && n_vec < 0x7fffffff - 64 && !(((uintptr_t)x | (uintptr_t)y) & 15) &&
        (y + n_vec * 64 <= x || x + n_vec * 64 <= y)) {
        const int waves = (int)((n_vec + 63) / 64);
        hipLaunchKernelGGL(rotate_rows_kernel, dim3((unsigned)((waves + AR_WAVES - 1) / AR_WAVES)),
                           dim3(64 * AR_WAVES), 0, s, x, y, (int)n_vec, rounds, sg, range_err);
        return hipGetLastError();
    }
    dim3 grid((unsigned)n_vec), block(64);
    if (d <= 64)
        hipLaunchKernelGGL(rotate_kernel<1>, grid, block, 0, s, x, y, n_vec, d, rounds, sg, range_err);
    else
        hipLaunchKernelGGL(rotate_kernel<2>, grid, block, 0, s, x, y, n_vec, d, rounds, sg, range_err);
    return hipGetLastError();
}

template <int KB, int VB, bool ROT>
__global__ void __launch_bounds__(64 * AR_WAVES) append_rows_kernel(
        Geom g, const Tables *__restrict__ tabs, const int32_t *__restrict__ k, const int32_t *__restrict__ v,
        int n_tok, int seq_lo, const int64_t *__restrict__ len_in, int64_t *len_out, int seq_hi, int rounds,
        RotSigns sg, DevStats *st, int rows) {
    static_assert(32 % KB == 0 && 32 % VB == 0 && KB <= 4 && VB <= 4, "code widths of 1, 2 or 4 bits");
    constexpr int NW = 2 * KB + 2 * VB + 1;            // the row's dwords: key codes, value codes, norms
    __shared__ int32_t tile[AR_WAVES][64 * AR_STRIDE];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // the length bookkeeping rides on workgroup 0 (as in append_kernel)
    if (blockIdx.x == 0) {
        for (int i = threadIdx.x; i < g.batch; i += blockDim.x)
            len_out[i] = len_in[i] + ((i >= seq_lo && i < seq_hi) ? n_tok : 0);
    }
    const int r0 = (blockIdx.x * AR_WAVES + wv) * 64;
    if (r0 >= rows) return;
    const int nr = rows - r0 < 64 ? rows - r0 : 64;    // rows of this tile
    // load i, lane l: row 4 i + l / 16 of the tile, dwords 4 (l % 16) .. + 3 (rows past the
    // input's end read its last row, and are not stored)
    const int sub = lane >> 4, q4 = (lane & 15) * 4;
    uint4 rk[16], rv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = 4 * i + sub < nr ? 4 * i + sub : nr - 1;
        rk[i] = *(const uint4 *)(k + ((int64_t)r0 + r) * 64 + q4);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = 4 * i + sub < nr ? 4 * i + sub : nr - 1;
        rv[i] = *(const uint4 *)(v + ((int64_t)r0 + r) * 64 + q4);
    }
    // this lane's row: (sequence, token, KV head) and where it goes
    const int R = r0 + (lane < nr ? lane : nr - 1);
    const int hh = R % g.n_kv, tt = R / g.n_kv;
    const int t = tt % n_tok, b = seq_lo + tt / n_tok;
    const int64_t pos = len_in[b] + t;
    int32_t *T = tile[wv];
    auto to_lds = [&](const uint4 (&raw)[16]) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int32_t *p = T + (4 * i + sub) * AR_STRIDE + q4;
            *(uint2 *)p = make_uint2(raw[i].x, raw[i].y);
            *(uint2 *)(p + 2) = make_uint2(raw[i].z, raw[i].w);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // each field's row is read where its arithmetic starts (a read moved up would keep two
    // rows in registers at once)
    auto row_from_lds = [&](int32_t (&x)[64]) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const uint2 u = *(const uint2 *)(T + lane * AR_STRIDE + 2 * j);
            x[2 * j] = (int32_t)u.x;
            x[2 * j + 1] = (int32_t)u.y;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        __builtin_amdgcn_sched_barrier(0);
    };
    int32_t x[64];
    to_lds(rk);
    row_from_lds(x);
    to_lds(rv);                                          // the key rows have been read
    uint32_t word[NW];
    uint32_t kw[2 * KB], vw[2 * VB];
    // (lanes past the tile's rows hold its last row again: their recount reads that row)
    int32_t nk = ar_field<KB, ROT>(x, rounds, sg, tabs->kbnd, g.norm_frac, lane < nr, k + (int64_t)r0 * 64,
                                   &st->range_errors, kw);
    // the key field's codes are finished here (left to the compiler, their arithmetic sinks
    // to the stores and keeps the key row live through the value field)
#pragma unroll
    for (int j = 0; j < 2 * KB; ++j) asm volatile("" : "+v"(kw[j]));
    asm volatile("" : "+v"(nk));
    row_from_lds(x);
    const int32_t nv = ar_field<VB, ROT>(x, rounds, sg, tabs->vbnd, g.norm_frac, lane < nr, v + (int64_t)r0 * 64,
                                         &st->range_errors, vw);
#pragma unroll
    for (int j = 0; j < 2 * KB; ++j) word[j] = kw[j];
#pragma unroll
    for (int j = 0; j < 2 * VB; ++j) word[2 * KB + j] = vw[j];
    word[NW - 1] = (uint32_t)(nk & 0xFFFF) | ((uint32_t)(nv & 0xFFFF) << 16);
    // where each of the row's dwords goes (scalar; found here, after the arithmetic, so that
    // it holds no scalar registers through it)
    WordLoc loc[NW];
#pragma unroll
    for (int j = 0; j < NW; ++j) loc[j] = word_loc(g, j);
    if (lane < nr) {
        if (pos >= g.capacity) {         // the host checks capacity first; this only guards memory
            atomicAdd(&st->fault, 1ull);
        } else {
#pragma unroll
            for (int j = 0; j < NW; ++j) *word_ptr(g, loc[j], b, hh, pos) = word[j];
        }
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

// The lane = row kernel takes the append when: d = 64; key and value codes of 1, 2 or 4
// bits (instantiated here for 4/2 and 2/2); the boundaries non-decreasing (4-bit codes are
// found by bisection); every boundary below 2^24 in magnitude and the
// encoder's shift CENT_FRAC + norm_frac - QK_FRAC at least 0 (its int32 thresholds are then
// exact); k and v 16-byte aligned (whole-wave 16-byte loads); fewer than 2^31 rows.
bool append_rows_ok(const Geom &g, const Tables &th, const int32_t *k, const int32_t *v, int64_t rows) {
    if (g.d != 64 || rows >= (int64_t(1) << 31) - 64) return false;
    if (!((g.kb == 4 && g.vb == 2) || (g.kb == 2 && g.vb == 2))) return false;
    if (CENT_FRAC + g.norm_frac - QK_FRAC < 0 || g.norm_frac > QK_FRAC) return false;
    if (((uintptr_t)k | (uintptr_t)v) & 15) return false;
    if (!th.bnd_sorted) return false;
    const int64_t lim = int64_t(1) << 24;
    for (int i = 0; i + 1 < (1 << g.kb); ++i)
        if (th.kbnd[i] >= lim || th.kbnd[i] <= -lim) return false;
    for (int i = 0; i + 1 < (1 << g.vb); ++i)
        if (th.vbnd[i] >= lim || th.vbnd[i] <= -lim) return false;
    return true;
}

hipError_t launch_append(hipStream_t s, const Geom &g, const Tables *t, const int32_t *k,
                         const int32_t *v, int n_tok, int seq_lo, int seq_hi, const int64_t *len_in,
                         int64_t *len_out, DevStats *st, int rounds, const uint64_t (*signs)[2],
                         const Tables *host_tabs) {
    const int64_t rows = (int64_t)(seq_hi - seq_lo) * n_tok * g.n_kv;
    if (rows <= 0) return hipSuccess;
    if (rounds < 0 || rounds > 2 || (rounds && !signs)) return hipErrorInvalidValue;
    const RotSigns sg = rounds ? rot_signs(rounds, signs) : RotSigns{};
    if (host_tabs && append_rows_ok(g, *host_tabs, k, v, rows)) {
        const int waves = (int)((rows + 63) / 64);
        dim3 grid((unsigned)((waves + AR_WAVES - 1) / AR_WAVES)), block(64 * AR_WAVES);
        const int nr = (int)rows;
#define INSITU_AR(KB, VB, ROT)                                                                     \
    hipLaunchKernelGGL((append_rows_kernel<KB, VB, ROT>), grid, block, 0, s, g, t, k, v, n_tok, seq_lo, \
                       len_in, len_out, seq_hi, rounds, sg, st, nr)
        if (g.kb == 4) {
            if (rounds) INSITU_AR(4, 2, true); else INSITU_AR(4, 2, false);
        } else {
            if (rounds) INSITU_AR(2, 2, true); else INSITU_AR(2, 2, false);
        }
#undef INSITU_AR
        return hipGetLastError();
    }
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
