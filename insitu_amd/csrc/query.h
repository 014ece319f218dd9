// The query side of the chunked attend.
//
// Each KV group's GF rotated query rows are staged once per call as fp64, in
// the layout [chain][channel][head] (chain = sequence * n_kv + KV head), by the
// kernel that produces them: the rotation of the fused decode step, or the
// query-prep kernel in front of a standalone attend. Every workgroup of the
// chain then reads them through scalar loads and uses them as the scalar
// operand of its score FMAs, so the scoring loop reads only the key centroids
// from LDS. A per-chain flag records whether every score of the group stays
// an exact fp64 integer (attention.py:333-359 computes them in int64):
// |dot| <= ||q||_1 * max|c| < 2^51.
#pragma once

#include "insitu_internal.h"
#include "wave.h"

namespace insitu {

constexpr int GF = 4;                                // query heads per KV head on the chunked path
constexpr double DOT_LIMIT = 2251799813685248.0;     // 2^51

// One wave stages query head h of a group: lane c (and c + 64) holds channel
// c's rotated value. Writes the head's fp64 column of the block qdc (global
// staging or a workgroup's LDS copy), counts values beyond the +-2^27 the
// 24-bit seam can produce as range errors (unless range_err is null), and
// returns (wave-uniform) whether the head's scores stay exact.
template <int CPL>
__device__ __forceinline__ bool stage_query_head(const int32_t (&v)[CPL], int d, int h,
                                                 double *qdc, double kc_absmax,
                                                 unsigned long long *range_err) {
    const int lane = threadIdx.x & 63;
    int64_t l1 = 0, bad = 0;
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
        const int c = lane + 64 * k;
        if (c < d) {
            const int64_t x = v[k];
            qdc[c * GF + h] = (double)x;
            l1 += x < 0 ? -x : x;
            bad += (x >= Q_ROT_LIMIT || x <= -Q_ROT_LIMIT) ? 1 : 0;
        }
    }
    l1 = wave_sum_i64(l1);          // < 2^38: exact as a double below
    bad = wave_sum_i64(bad);
    if (range_err && lane == 0 && bad) atomicAdd(range_err, (unsigned long long)bad);
    return (double)l1 * kc_absmax < DOT_LIMIT;
}

}  // namespace insitu
