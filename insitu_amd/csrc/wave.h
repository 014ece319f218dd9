// Wave-wide (64-lane) reductions and scans built on DPP row operations and
// readlane, so that no step goes through the LDS permute unit (ds_bpermute)
// and its round-trip latency. CDNA waves are 64 lanes in four rows of 16.
//
// The reductions return a wave-uniform value; the scans are inclusive in lane
// order. All of them expect every lane of the wave to be active.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace insitu {

// DPP controls (GCN3/CDNA encoding).
constexpr int DPP_QUAD_1032 = 0xB1;     // quad_perm [1,0,3,2]: lane ^ 1
constexpr int DPP_QUAD_2301 = 0x4E;     // quad_perm [2,3,0,1]: lane ^ 2
constexpr int DPP_ROW_SHR1 = 0x111;
constexpr int DPP_ROW_SHR2 = 0x112;
constexpr int DPP_ROW_SHR4 = 0x114;
constexpr int DPP_ROW_SHR8 = 0x118;
constexpr int DPP_ROW_SHL4 = 0x104;          // lane i <- lane i + 4 within a row
constexpr int DPP_ROW_ROR8 = 0x128;          // lane i <- lane (i + 8) mod 16 within a row
constexpr int DPP_ROW_MIRROR = 0x140;        // lane i <-> 15 - i within a row
constexpr int DPP_ROW_HALF_MIRROR = 0x141;   // lane i <-> 7 - i within 8 lanes
constexpr int DPP_ROW_BCAST15 = 0x142;       // lane 15 of each row -> the next row
constexpr int DPP_ROW_BCAST31 = 0x143;       // lane 31 -> rows 2 and 3
constexpr int DPP_WAVE_SHR1 = 0x138;         // lane i <- lane i - 1 across the wave

// v from the lane selected by CTRL; lanes without a source (or outside ROWS)
// get `fill`.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp32(uint32_t fill, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)fill, (int)v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int64_t dpp64(int64_t fill, int64_t v) {
    const uint32_t lo = dpp32<CTRL, ROWS>((uint32_t)fill, (uint32_t)v);
    const uint32_t hi = dpp32<CTRL, ROWS>((uint32_t)((uint64_t)fill >> 32), (uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), lane);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// A value every lane holds the same copy of (read from LDS, say), made
// wave-uniform for the compiler so that it lives in SGPRs and drives scalar
// branches.
__device__ __forceinline__ int32_t uni32(int32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uni64(int64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

struct OpMax64 {
    __device__ static int64_t f(int64_t a, int64_t b) { return a > b ? a : b; }
};
struct OpAdd64 {
    __device__ static int64_t f(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
};

// Reduction of every lane's value, wave-uniform. Within each row the four DPP
// steps leave every lane with the row's result; readlane combines the rows.
template <class OP>
__device__ __forceinline__ int64_t wave_reduce64(int64_t v) {
    v = OP::f(v, dpp64<DPP_QUAD_1032>(v, v));
    v = OP::f(v, dpp64<DPP_QUAD_2301>(v, v));
    v = OP::f(v, dpp64<DPP_ROW_HALF_MIRROR>(v, v));
    v = OP::f(v, dpp64<DPP_ROW_MIRROR>(v, v));
    const int64_t r0 = readlane64(v, 0), r1 = readlane64(v, 16);
    const int64_t r2 = readlane64(v, 32), r3 = readlane64(v, 48);
    return OP::f(OP::f(r0, r1), OP::f(r2, r3));
}

__device__ __forceinline__ int64_t wave_max_i64(int64_t v) { return wave_reduce64<OpMax64>(v); }
__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) { return wave_reduce64<OpAdd64>(v); }

// Inclusive scan in lane order; `id` is the operation's identity.
template <class OP>
__device__ __forceinline__ int64_t wave_scan64(int64_t v, int64_t id) {
    v = OP::f(v, dpp64<DPP_ROW_SHR1>(id, v));
    v = OP::f(v, dpp64<DPP_ROW_SHR2>(id, v));
    v = OP::f(v, dpp64<DPP_ROW_SHR4>(id, v));
    v = OP::f(v, dpp64<DPP_ROW_SHR8>(id, v));
    v = OP::f(v, dpp64<DPP_ROW_BCAST15, 0xA>(id, v));
    v = OP::f(v, dpp64<DPP_ROW_BCAST31, 0xC>(id, v));
    return v;
}

// The value of the previous lane (lane 0 gets `id`).
__device__ __forceinline__ int64_t wave_shr1_64(int64_t v, int64_t id) {
    return dpp64<DPP_WAVE_SHR1>(id, v);
}

// The maximum of a signed 32-bit value over the wave, wave-uniform: DPP steps within each
// row of 16 lanes (32-bit ops, one instruction each), then readlane combines the rows.
__device__ __forceinline__ int32_t wave_max_i32(int32_t v) {
    auto mx = [](int32_t a, int32_t b) { return a > b ? a : b; };
    v = mx(v, (int32_t)dpp32<DPP_QUAD_1032>((uint32_t)v, (uint32_t)v));
    v = mx(v, (int32_t)dpp32<DPP_QUAD_2301>((uint32_t)v, (uint32_t)v));
    v = mx(v, (int32_t)dpp32<DPP_ROW_HALF_MIRROR>((uint32_t)v, (uint32_t)v));
    v = mx(v, (int32_t)dpp32<DPP_ROW_MIRROR>((uint32_t)v, (uint32_t)v));
    const int32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
    const int32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return mx(mx(r0, r1), mx(r2, r3));
}
// The maximum of a value in [-2^47, 2^47) over the wave, wave-uniform and exact, in 32-bit
// steps: the largest v >> 16 first, then the largest low 16 bits among the lanes that hold it.
__device__ __forceinline__ int64_t wave_max_s48(int64_t v) {
    const int32_t hi = (int32_t)(v >> 16);
    const int32_t mhi = wave_max_i32(hi);
    const int32_t lo = hi == mhi ? (int32_t)(v & 0xFFFF) : 0;
    return (int64_t)mhi * 65536 + wave_max_i32(lo);
}

// wave_max_s48 of N values at once, step by step: each DPP step and each readlane round issues
// N independent operations, so that one value's dependent chain does not stall the wave (a DPP
// read of a VGPR written by the previous VALU op needs wait states).
template <int N>
__device__ __forceinline__ void wave_max_s48_n(const int64_t (&v)[N], int64_t (&out)[N]) {
    auto mx = [](int32_t a, int32_t b) { return a > b ? a : b; };
    int32_t hi[N], m[N];
#pragma unroll
    for (int i = 0; i < N; ++i) m[i] = hi[i] = (int32_t)(v[i] >> 16);
    auto rowmax = [&](int32_t (&x)[N]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = mx(x[i], (int32_t)dpp32<DPP_QUAD_1032>((uint32_t)x[i], (uint32_t)x[i]));
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = mx(x[i], (int32_t)dpp32<DPP_QUAD_2301>((uint32_t)x[i], (uint32_t)x[i]));
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = mx(x[i], (int32_t)dpp32<DPP_ROW_HALF_MIRROR>((uint32_t)x[i], (uint32_t)x[i]));
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = mx(x[i], (int32_t)dpp32<DPP_ROW_MIRROR>((uint32_t)x[i], (uint32_t)x[i]));
    };
    rowmax(m);
    int32_t mhi[N], lo[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        mhi[i] = mx(mx(__builtin_amdgcn_readlane(m[i], 0), __builtin_amdgcn_readlane(m[i], 16)),
                    mx(__builtin_amdgcn_readlane(m[i], 32), __builtin_amdgcn_readlane(m[i], 48)));
        lo[i] = hi[i] == mhi[i] ? (int32_t)(v[i] & 0xFFFF) : 0;
    }
    rowmax(lo);
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int32_t mlo = mx(mx(__builtin_amdgcn_readlane(lo[i], 0), __builtin_amdgcn_readlane(lo[i], 16)),
                               mx(__builtin_amdgcn_readlane(lo[i], 32), __builtin_amdgcn_readlane(lo[i], 48)));
        out[i] = (int64_t)mhi[i] * 65536 + mlo;
    }
}

// The signed 32-bit maximum over the wave of 5 values at once, wave-uniform: fused v_max_i32_dpp
// steps, 4 within each row of 16 lanes and 2 that carry rows 0-1 into 1 and 3, then rows 0-2
// into 3 (row_bcast), so that lane 63 holds the maximum. One asm block, the 5 values' steps
// interleaved: a value's next DPP read comes 4 instructions after its write (2 wait states are
// needed), and s_nop 1 covers the writes before the block.
__device__ __forceinline__ void wave_max_i32_x5(int32_t (&x)[5]) {
#define INSITU_MAX5(CTRL)                                                              \
    "v_max_i32_dpp %0, %0, %0 " CTRL "\n\t"                                             \
    "v_max_i32_dpp %1, %1, %1 " CTRL "\n\t"                                             \
    "v_max_i32_dpp %2, %2, %2 " CTRL "\n\t"                                             \
    "v_max_i32_dpp %3, %3, %3 " CTRL "\n\t"                                             \
    "v_max_i32_dpp %4, %4, %4 " CTRL "\n\t"
    asm volatile("s_nop 1\n\t"
                 INSITU_MAX5("quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf")
                 INSITU_MAX5("quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf")
                 INSITU_MAX5("row_half_mirror row_mask:0xf bank_mask:0xf")
                 INSITU_MAX5("row_mirror row_mask:0xf bank_mask:0xf")
                 INSITU_MAX5("row_bcast:15 row_mask:0xa bank_mask:0xf")
                 INSITU_MAX5("row_bcast:31 row_mask:0xc bank_mask:0xf")
                 "s_nop 1"
                 : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]));
#undef INSITU_MAX5
#pragma unroll
    for (int i = 0; i < 5; ++i) x[i] = __builtin_amdgcn_readlane(x[i], 63);
}

// wave_max_s48 of 5 values at once with the fused steps above: the largest v >> 16, then the
// largest low 16 bits among the lanes that hold it.
__device__ __forceinline__ void wave_max_s48_x5(const int64_t (&v)[5], int64_t (&out)[5]) {
    int32_t hi[5], m[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) m[i] = hi[i] = (int32_t)(v[i] >> 16);
    wave_max_i32_x5(m);
    int32_t lo[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) lo[i] = hi[i] == m[i] ? (int32_t)(v[i] & 0xFFFF) : 0;
    wave_max_i32_x5(lo);
#pragma unroll
    for (int i = 0; i < 5; ++i) out[i] = (int64_t)m[i] * 65536 + lo[i];
}

// Sums over the wave of N unsigned 32-bit values at once (each below 2^26 / 64 lanes' worth,
// so that no sum wraps), wave-uniform, step by step like wave_max_s48_n.
template <int N>
__device__ __forceinline__ void wave_sum_u32_n(const uint32_t (&v)[N], uint32_t (&out)[N]) {
    uint32_t x[N];
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = v[i];
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += dpp32<DPP_QUAD_1032>(x[i], x[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += dpp32<DPP_QUAD_2301>(x[i], x[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += dpp32<DPP_ROW_HALF_MIRROR>(x[i], x[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += dpp32<DPP_ROW_MIRROR>(x[i], x[i]);
#pragma unroll
    for (int i = 0; i < N; ++i)
        out[i] = ((uint32_t)__builtin_amdgcn_readlane((int)x[i], 0) + (uint32_t)__builtin_amdgcn_readlane((int)x[i], 16)) +
                 ((uint32_t)__builtin_amdgcn_readlane((int)x[i], 32) + (uint32_t)__builtin_amdgcn_readlane((int)x[i], 48));
}

// 32-bit inclusive running maximum (signed) in lane order.
__device__ __forceinline__ int32_t wave_scan_max32(int32_t v) {
    auto mx = [](int32_t a, int32_t b) { return a > b ? a : b; };
    const uint32_t lo = 0x80000000u;
    v = mx(v, (int32_t)dpp32<DPP_ROW_SHR1>(lo, (uint32_t)v));
    v = mx(v, (int32_t)dpp32<DPP_ROW_SHR2>(lo, (uint32_t)v));
    v = mx(v, (int32_t)dpp32<DPP_ROW_SHR4>(lo, (uint32_t)v));
    v = mx(v, (int32_t)dpp32<DPP_ROW_SHR8>(lo, (uint32_t)v));
    v = mx(v, (int32_t)dpp32<DPP_ROW_BCAST15, 0xA>(lo, (uint32_t)v));
    v = mx(v, (int32_t)dpp32<DPP_ROW_BCAST31, 0xC>(lo, (uint32_t)v));
    return v;
}

// 32-bit inclusive prefix sum in lane order.
__device__ __forceinline__ uint32_t wave_scan_add32(uint32_t v) {
    v += dpp32<DPP_ROW_SHR1>(0u, v);
    v += dpp32<DPP_ROW_SHR2>(0u, v);
    v += dpp32<DPP_ROW_SHR4>(0u, v);
    v += dpp32<DPP_ROW_SHR8>(0u, v);
    v += dpp32<DPP_ROW_BCAST15, 0xA>(0u, v);
    v += dpp32<DPP_ROW_BCAST31, 0xC>(0u, v);
    return v;
}

}  // namespace insitu
