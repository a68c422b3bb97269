// Population-weighted KV4 block masses of one row (reference:
// csrc/ibcs.cu:495-538):
//   m_j = sum_s fmaf(n_s, exp2(l_sj - M_s) * (1/D_s), .) * (1 / sum_s n_s)
// from the fp16 pair-LSEs l [8, ld] of the row, the populations n_s and the
// per-centroid maxima M_s and normalisers D_s. Shared by the masses kernel
// (scores to global memory) and the fused masses + SIP kernel (scores into
// LDS), so both produce the same bits: the same operations in the same order,
// every product rounded before its sum (the library builds with
// -ffp-contract=off).
#pragma once

#include "common.hpp"

namespace ab {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

struct RowMasses {
    float weight[kCentroids], inv_den[kCentroids], mx[kCentroids];
    float inv_total;

    __device__ __forceinline__ void load(const float* __restrict__ pops, const float* __restrict__ lse_max,
                                         const float* __restrict__ lse_den, int64_t row) {
        float total = 0.0f;
#pragma unroll
        for (int s = 0; s < kCentroids; ++s) {
            weight[s] = pops[row * kCentroids + s];
            inv_den[s] = __fdiv_rn(1.0f, lse_den[row * kCentroids + s]);
            mx[s] = lse_max[row * kCentroids + s];
            total += weight[s];
        }
        inv_total = __fdiv_rn(1.0f, total);
    }

    // Masses of blocks j0 .. j0+7 from their pair-LSEs h[s] (centroid s).
    __device__ __forceinline__ void eight(const f16x8 (&h)[kCentroids], float (&out)[8]) const {
        float score[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) score[e] = 0.0f;
#pragma unroll
        for (int s = 0; s < kCentroids; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                score[e] =
                    __builtin_fmaf(weight[s], fast_exp2(static_cast<float>(h[s][e]) - mx[s]) * inv_den[s], score[e]);
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = score[e] * inv_total;
    }
};

}  // namespace ab
