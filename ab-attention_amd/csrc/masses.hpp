// Population-weighted KV4 block masses of one row (reference:
// csrc/ibcs.cu:495-538):
//   m_j = sum_s fmaf(c_s, exp2(l_sj - M_s), .) * (1 / sum_s n_s),
//   c_s = n_s * (1/D_s) (rounded once per row and centroid)
// from the fp16 pair-LSEs l [8, ld] of the row, the populations n_s and the
// per-centroid maxima M_s and normalisers D_s. The reference forms
// n_s * (exp2(l - M_s) / D_s) per element; folding n_s / D_s into one
// coefficient per row changes a mass by about one float ulp (within the
// tolerance against the CPU oracle) and saves a multiplication per element,
// and l - M_s is one v_fma_mix_f32 (exact conversion, one rounding): three
// instructions per (centroid, block) instead of five. Shared by the masses
// kernel (scores to global memory) and the fused masses + SIP kernel (scores
// into LDS), so both produce the same bits: the same operations in the same
// order (the library builds with -ffp-contract=off).
#pragma once

#include "common.hpp"

namespace ab {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// The constants of one row; every thread of a workgroup holds the same row,
// so they are wave-uniform (SGPRs).
struct RowMasses {
    float coef[kCentroids], mx[kCentroids];
    float inv_total;

    __device__ __forceinline__ void load(const float* __restrict__ pops, const float* __restrict__ lse_max,
                                         const float* __restrict__ lse_den, int64_t row) {
        float total = 0.0f;
#pragma unroll
        for (int s = 0; s < kCentroids; ++s) {
            const float weight = pops[row * kCentroids + s];
            coef[s] = weight * __fdiv_rn(1.0f, lse_den[row * kCentroids + s]);
            mx[s] = lse_max[row * kCentroids + s];
            total += weight;
        }
        inv_total = __fdiv_rn(1.0f, total);
    }

    // Masses of blocks j0 .. j0+7 from their pair-LSEs h[s] (centroid s).
    __device__ __forceinline__ void eight(const f16x8 (&h)[kCentroids], float (&out)[8]) const {
        float score[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) score[e] = 0.0f;
#pragma unroll
        for (int s = 0; s < kCentroids; ++s) {
            // The whole vector is bit-cast (never one element of it).
            const u32x4 pairs = __builtin_bit_cast(u32x4, h[s]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                score[2 * e] =
                    __builtin_fmaf(coef[s], fast_exp2(f16_minus_uniform<false>(pairs[e], mx[s])), score[2 * e]);
                score[2 * e + 1] =
                    __builtin_fmaf(coef[s], fast_exp2(f16_minus_uniform<true>(pairs[e], mx[s])), score[2 * e + 1]);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = score[e] * inv_total;
    }
};

}  // namespace ab
