// IBCS on gfx950: query clustering + key pooling, centroid/key pair-LSE with
// per-centroid normalisers, and population-weighted block masses.
//
// Dataflow (one head chunk, the caller's workspace holds every intermediate):
//   cluster_pool_kernel  Q,K -> scaled centroids [rows,8,128] bf16, populations
//                        [rows,8] f32, pooled keys [bh,fb,2,128] bf16
//   (lse.hip)            centroids x pooled keys (bf16 MFMA) -> fp16 pair-LSE
//                        [rows,8,ld] and (max, den) [rows,8]
//   masses_kernel        pair-LSE + normalisers + populations -> scores [rows,fb]
//
// Reference stages: csrc/ibcs.cu:106-238 (cluster), :244-266 (pool),
// :329-489 (LSE), :495-538 (scores). Exactness notes:
//   - cluster/pool follow the reference's fp32 operation order (lane-strided
//     fmaf chains, xor-butterfly sums, row-order centroid sums, IEEE division),
//     so they match the CPU oracle bit for bit;
//   - pair-LSE uses one exp2 and one log2 per (centroid, block):
//     exp2(a-mx) + exp2(b-mx) == 1 + exp2(min-mx) because exp2(0) == 1. The
//     reference's max(sum, 1e-20) floor never binds for finite inputs (sum >= 1);
//   - the normaliser D is accumulated tile by tile from the fp16-rounded values
//     (online max/rescale), matching the reference up to fp32 rounding order.
#include <cfloat>

#include "common.hpp"
#include "masses.hpp"

namespace ab {
namespace {

// ---------------------------------------------------------------------------
// Stage 1+2: clustering of one 128-query block and pooling of the same 128
// key tokens. One workgroup of 128 threads per (query block, head): thread i
// owns query i (its row kept in 128 VGPRs as f32); thread d owns dim d in the
// column sums, which read the block from LDS one 64-row half at a time
// (17 KB of LDS and 162 VGPRs: three waves per SIMD).

constexpr int kClusterThreads = 128;
constexpr int kHalfRows = 64;
constexpr int kRowWords = kHeadDim / 2 + 1;  // padded bf16 row: 65 dwords

// The reference's distance (csrc/ibcs.cu:143-155, :171-181) is 32 partial
// chains, chain l = fmaf over dims l, l+32, l+64, l+96, summed by the xor
// butterfly 16,8,4,2,1 (every lane of a butterfly ends with the pairwise
// tree). That tree is evaluated depth first here: its k-th leaf is chain
// bitrev5(k), and a leaf's value is added to the pending partial of each
// level its index completes, so one partial per level is live instead of
// 32. The additions are the tree's, so the bits are the same.
__host__ __device__ constexpr int leaf_chain(int k) {
    return ((k & 1) << 4) | ((k & 2) << 2) | (k & 4) | ((k & 8) >> 2) | ((k & 16) >> 4);
}
// Rows are held in leaf order, the four dims of a chain together: element
// [k][r] of a row is dim leaf_chain(k) + 32r. A query's row sits in 32 f32x4
// registers that way, and the centre row in LDS (one 16-byte read or write
// per chain).
__device__ __forceinline__ int center_pos(int d) { return 4 * leaf_chain(d & 31) + (d >> 5); }
__device__ __forceinline__ float row_dim(const f32x4 (&x)[32], int d) { return x[leaf_chain(d & 31)][d >> 5]; }

__device__ __forceinline__ float lane_distance(const f32x4 (&x)[32], const float* __restrict__ center) {
    float pending[6];
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const f32x4 c = *reinterpret_cast<const f32x4*>(center + 4 * k);
        float acc = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float delta = x[k][r] - c[r];
            acc = __builtin_fmaf(delta, delta, acc);
        }
        float v = acc;
        int level = 0;
#pragma unroll
        for (int b = 0; b < 5; ++b)
            if (((k >> b) & 1) && level == b) {
                v = pending[b] + v;
                level = b + 1;
            }
        pending[level] = v;
    }
    return pending[5];
}

// Block-wide argmax over the 128 threads' values: largest value, lowest
// thread index on ties (cub::ArgMax semantics, csrc/ibcs.cu:94-102), valid
// in every thread. Per wave: the maximum by an xor butterfly (exact, so every
// lane holds the same value), then the lowest lane holding it from a ballot;
// the two waves meet in LDS. One barrier: the caller places another barrier
// between this call and the next (the LDS slots are reused).
__device__ __forceinline__ int block_argmax(float value, float* s_val, int* s_idx) {
    float m = value;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    const uint64_t hit = __ballot(value == m);  // empty only if every value is NaN
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        s_val[wave] = m;
        s_idx[wave] = 64 * wave + (hit != 0u ? static_cast<int>(__builtin_ctzll(hit)) : 0);
    }
    __syncthreads();
    const float v0 = s_val[0], v1 = s_val[1];
    const int i0 = s_idx[0], i1 = s_idx[1];
    return v1 > v0 ? i1 : i0;  // equal values: wave 0 holds the lower index
}

// Byte selector of v_perm_b32 that moves the bf16 of dim `dim` of a packed
// pair into the high half of a float (low half zero): bytes 1,0 for an even
// dim, 3,2 for an odd one (0x0c selects a zero byte).
__device__ __forceinline__ uint32_t bf16_select(int dim) { return (dim & 1) ? 0x03020c0cu : 0x01000c0cu; }

// One dim of a staged row, with the selector precomputed: one v_perm_b32.
__device__ __forceinline__ float block_elem_sel(const uint32_t* block, int row, int word, uint32_t sel) {
    const uint32_t w = block[row * kRowWords + word];
    return __uint_as_float(__builtin_amdgcn_perm(w, w, sel));
}

__global__ __launch_bounds__(kClusterThreads) __attribute__((amdgpu_waves_per_eu(3, 3))) void cluster_pool_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    uint16_t* __restrict__ centroids, float* __restrict__ pops, uint16_t* __restrict__ pooled,
    int64_t n, int64_t qb, float qk_scale_log2, const int32_t* __restrict__ order) {
    __shared__ uint32_t half_block[kHalfRows * kRowWords];
    __shared__ __align__(16) float center_row[kHeadDim];
    __shared__ float s_val[2];
    __shared__ int s_idx[2];
    __shared__ uint64_t slot_mask[kClusterThreads / 64][kCentroids];

    const int tid = threadIdx.x, wave = tid >> 6;
    const int64_t blk = blockIdx.x, bh = blockIdx.y;
    const int64_t base = blk * kQueryBlock;
    const int valid = static_cast<int>(min<int64_t>(kQueryBlock, n - base));
    const int64_t row = bh * qb + blk;

    // Loads, all issued before any is used: the key pairs this thread pools
    // (16 bytes of pairs tid/16 + 8i, i < 8) and this thread's own query row
    // (256 bytes). Token t of the head is stored row t, or order[t] for a
    // permuted token layout (clamped into the head); rows past the sequence
    // end are clamped and their data discarded. Offsets are in 16-byte units
    // from the head's base (32-bit: a head has at most 131,072 tokens).
    const u32x4* qhead = reinterpret_cast<const u32x4*>(q + bh * n * kHeadDim);
    const u32x4* khead = reinterpret_cast<const u32x4*>(k + bh * n * kHeadDim);
    const int c16 = tid & 15, r0 = tid >> 4;
    const int pairs = valid / 2;
    const int nm1 = static_cast<int>(n - 1), b32 = static_cast<int>(base);
    auto stored = [&](int t) {  // t: token index inside the block
        const int tok = b32 + min(t, valid - 1);
        return order ? min(max(order[tok], 0), nm1) : tok;
    };
    u32x4 ka[8], kb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int p = r0 + 8 * i;
        ka[i] = khead[uint32_t(stored(2 * p)) * 16u + c16];
        kb[i] = khead[uint32_t(stored(2 * p + 1)) * 16u + c16];
    }
    f32x4 x[32];
    {
        const uint32_t qoff = uint32_t(stored(tid)) * 16u;
        u32x4 qv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) qv[j] = qhead[qoff + j];
        // Pool the keys: bf16(0.5 * (k_2r + k_2r+1)) (:244-266).
        u32x4* kdst = reinterpret_cast<u32x4*>(pooled + (bh * (n / 2) + base / 2) * kHeadDim);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int p = r0 + 8 * i;
            if (p < pairs) {
                u32x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float lo = 0.5f * (bf16_lo(ka[i][e]) + bf16_lo(kb[i][e]));
                    const float hi = 0.5f * (bf16_hi(ka[i][e]) + bf16_hi(kb[i][e]));
                    o[e] = pack_bf16(lo, hi);
                }
                kdst[p * 16 + c16] = o;
            }
        }
        // Queries past the sequence end are zero rows.
        const bool zero_row = tid >= valid;
#pragma unroll
        for (int j = 0; j < 16; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t w = zero_row ? 0u : qv[j][e];
                const int d = 8 * j + 2 * e;
                x[leaf_chain(d & 31)][d >> 5] = bf16_lo(w);
                x[leaf_chain((d + 1) & 31)][(d + 1) >> 5] = bf16_hi(w);
            }
    }

    // Thread tid owns dim tid in the column passes: its word of a packed row
    // and the selector of its half.
    const int my_word = tid >> 1;
    const uint32_t my_sel = bf16_select(tid);
    // The rows of half h (queries 64h .. 64h+63) into LDS, written by wave h
    // from its registers: v_perm_b32 takes the high halves of two floats,
    // which gives back the loaded bf16 pair bit for bit.
    auto stage_half = [&](int h) {
        if (wave == h) {
            uint32_t* dst = half_block + (tid & 63) * kRowWords;
#pragma unroll
            for (int w = 0; w < kHeadDim / 2; ++w)
                dst[w] = __builtin_amdgcn_perm(__float_as_uint(row_dim(x, 2 * w + 1)),
                                               __float_as_uint(row_dim(x, 2 * w)), 0x07060302u);
        }
        __syncthreads();
    };

    // Per-dim mean over valid queries in row order (csrc/ibcs.cu:130-140).
    {
        float sum = 0.0f;
        for (int h = 0; h < 2; ++h) {
            stage_half(h);
            const int end = min(valid - kHalfRows * h, kHalfRows);
            int i = 0;
            for (; i + 8 <= end; i += 8) {  // 8 reads in flight, adds in row order
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = block_elem_sel(half_block, i + e, my_word, my_sel);
#pragma unroll
                for (int e = 0; e < 8; ++e) sum += v[e];
            }
            for (; i < end; ++i) sum += block_elem_sel(half_block, i, my_word, my_sel);
            __syncthreads();
        }
        center_row[center_pos(tid)] = __fdiv_rn(sum, static_cast<float>(valid));
    }
    __syncthreads();

    // Farthest-first centres with nearest-centre assignment (:158-197).
    const bool live = tid < valid;
    float min_d = live ? lane_distance(x, center_row) : -INFINITY;
    int center = block_argmax(min_d, s_val, s_idx);
    min_d = INFINITY;
    int assign = 0;
    for (int slot = 0; slot < kCentroids; ++slot) {
        // The centre's own thread publishes its row (every thread has read
        // the previous centre row and the argmax slots before the argmax's
        // barrier).
        if (tid == center) {
#pragma unroll
            for (int kk = 0; kk < 32; ++kk) *reinterpret_cast<f32x4*>(center_row + 4 * kk) = x[kk];
        }
        __syncthreads();
        if (live) {
            const float dist = lane_distance(x, center_row);
            if (dist < min_d) {
                min_d = dist;
                assign = slot;
            }
        }
        if (slot + 1 < kCentroids) center = block_argmax(live ? min_d : -INFINITY, s_val, s_idx);
    }

    // Members of each slot: per wave, the ballot of the queries assigned to
    // it. Queries 64w + bit, walked wave by wave and bit by bit, come in
    // query order (the reference's member order).
#pragma unroll
    for (int s = 0; s < kCentroids; ++s) {
        const uint64_t m = __ballot(live && assign == s);
        if ((tid & 63) == 0) slot_mask[wave][s] = m;
    }
    __syncthreads();
    if (tid < kCentroids)
        pops[row * kCentroids + tid] =
            static_cast<float>(__popcll(slot_mask[0][tid]) + __popcll(slot_mask[1][tid]));

    // Centroid = bf16(member sum / count), then the LSE pre-scale
    // bf16(centroid * 128^-0.5 * log2 e) (csrc/ibcs.cu:213-237, :293-295).
    // Members are added in query order (half 0, then half 1), read from the
    // staged half that holds them, 8 loads in flight.
    // The member masks are made wave-uniform (SGPRs), so the walk over the
    // members (find first set bit, clear it) is scalar work.
    float msum[kCentroids];
#pragma unroll
    for (int s = 0; s < kCentroids; ++s) msum[s] = 0.0f;
    for (int h = 0; h < 2; ++h) {
        stage_half(h);
        for (int s = 0; s < kCentroids; ++s) {
            const uint64_t lds_m = slot_mask[h][s];
            const uint32_t m_lo = __builtin_amdgcn_readfirstlane(uint32_t(lds_m));
            const uint32_t m_hi = __builtin_amdgcn_readfirstlane(uint32_t(lds_m >> 32));
            uint64_t m = (uint64_t(m_hi) << 32) | m_lo;
            float sum = msum[s];
            for (int left = __popcll(m); left >= 8; left -= 8) {
                int idx[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    idx[e] = static_cast<int>(__builtin_ctzll(m));
                    m &= m - 1u;
                }
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = block_elem_sel(half_block, idx[e], my_word, my_sel);
#pragma unroll
                for (int e = 0; e < 8; ++e) sum += v[e];
            }
            for (; m != 0u; m &= m - 1u) sum += block_elem_sel(half_block, __builtin_ctzll(m), my_word, my_sel);
            msum[s] = sum;
        }
        __syncthreads();
    }
    uint16_t* dst = centroids + row * kCentroids * kHeadDim + tid;
#pragma unroll
    for (int s = 0; s < kCentroids; ++s) {
        const int cnt = __popcll(slot_mask[0][s]) + __popcll(slot_mask[1][s]);
        const uint32_t c = cnt > 0 ? f32_to_bf16(__fdiv_rn(msum[s], static_cast<float>(cnt))) : 0u;
        dst[s * kHeadDim] = static_cast<uint16_t>(f32_to_bf16(__uint_as_float(c << 16) * qk_scale_log2));
    }
}

// ---------------------------------------------------------------------------
// Stage 4: population-weighted masses, one workgroup per row:
//   m_j = sum_s fmaf(n_s / D_s, exp2(l_sj - M_s), .) * (1 / sum_s n_s)
// (RowMasses in masses.hpp).

constexpr int kMassThreads = 256;

__global__ __launch_bounds__(kMassThreads) void masses_kernel(
    const _Float16* __restrict__ lse, const float* __restrict__ pops,
    const float* __restrict__ lse_max, const float* __restrict__ lse_den,
    float* __restrict__ scores, int fb, int64_t ld) {
    const int64_t row = blockIdx.x;
    RowMasses rm;
    rm.load(pops, lse_max, lse_den, row);
    const _Float16* src = lse + row * kCentroids * ld;
    float* dst = scores + row * int64_t(fb);
    for (int j0 = threadIdx.x * 8; j0 < fb; j0 += kMassThreads * 8) {
        f16x8 h[kCentroids];
#pragma unroll
        for (int s = 0; s < kCentroids; ++s) h[s] = *reinterpret_cast<const f16x8*>(src + s * ld + j0);
        float score[8];
        rm.eight(h, score);
        // Two 16-byte stores (rows start at any multiple of 4 bytes, which
        // global stores accept); the ragged end of the row element by element.
        typedef float f32x4_u __attribute__((ext_vector_type(4), aligned(4)));
        if (j0 + 8 <= fb) {
            *reinterpret_cast<f32x4_u*>(dst + j0) = f32x4_u{score[0], score[1], score[2], score[3]};
            *reinterpret_cast<f32x4_u*>(dst + j0 + 4) = f32x4_u{score[4], score[5], score[6], score[7]};
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (j0 + e < fb) dst[j0 + e] = score[e];
        }
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Host launchers (validated by the C-ABI layer in api.hip).

int64_t lse_stride(int64_t fb) { return (fb + 63) / 64 * 64; }

int launch_cluster_pool(const void* q, const void* k, int64_t bh, int64_t n, void* centroids,
                        float* pops, void* pooled, float qk_scale_log2, const int32_t* order, hipStream_t stream) {
    // The kernel addresses a head with 32-bit offsets.
    if (n <= 0 || n > kMaxKvBlocks * kKvBlock) return set_error(1, "ibcs: %lld tokens per head", (long long)n);
    const int64_t qb = (n + kQueryBlock - 1) / kQueryBlock;
    dim3 grid(static_cast<unsigned>(qb), static_cast<unsigned>(bh));
    hipLaunchKernelGGL(cluster_pool_kernel, grid, dim3(kClusterThreads), 0, stream,
                       static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                       static_cast<uint16_t*>(centroids), pops, static_cast<uint16_t*>(pooled), n, qb,
                       qk_scale_log2, order);
    return check_launch("cluster_pool_kernel");
}

int launch_masses(const void* lse, const float* pops, const float* lse_max, const float* lse_den,
                  int64_t rows, int64_t fb, float* scores, hipStream_t stream) {
    hipLaunchKernelGGL(masses_kernel, dim3(static_cast<unsigned>(rows)), dim3(kMassThreads), 0, stream,
                       static_cast<const _Float16*>(lse), pops, lse_max, lse_den, scores,
                       static_cast<int>(fb), lse_stride(fb));
    return check_launch("masses_kernel");
}

}  // namespace ab
