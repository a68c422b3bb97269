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
// owns query i (kept in 128 VGPRs); thread d owns dim d for the column sums.

constexpr int kClusterThreads = 128;
constexpr int kRowWords = kHeadDim / 2 + 1;  // padded bf16 row: 65 dwords

// Squared distance with the reference association (csrc/ibcs.cu:143-155,
// :171-181): partial l chains fmaf over dims l, l+32, l+64, l+96; the 32
// partials are summed by the xor butterfly 16,8,4,2,1 (every lane of a
// butterfly ends with the pairwise tree below).
__device__ __forceinline__ float lane_distance(const float (&x)[kHeadDim],
                                               const float* __restrict__ center) {
    float p[32];
#pragma unroll
    for (int l = 0; l < 32; ++l) {
        float acc = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float delta = x[l + 32 * r] - center[l + 32 * r];
            acc = __builtin_fmaf(delta, delta, acc);
        }
        p[l] = acc;
    }
#pragma unroll
    for (int mask = 16; mask >= 1; mask >>= 1)
#pragma unroll
        for (int l = 0; l < mask; ++l) p[l] = p[l] + p[l + mask];
    return p[0];
}

// Block-wide argmax over 128 threads: largest value, lowest index on ties
// (cub::ArgMax semantics, csrc/ibcs.cu:94-102). Result valid in every thread.
__device__ __forceinline__ int block_argmax(float value, int index, float* s_val, int* s_idx) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(value, off);
        const int oi = __shfl_xor(index, off);
        if (ov > value || (ov == value && oi < index)) {
            value = ov;
            index = oi;
        }
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        s_val[wave] = value;
        s_idx[wave] = index;
    }
    __syncthreads();
    const float v0 = s_val[0], v1 = s_val[1];
    const int i0 = s_idx[0], i1 = s_idx[1];
    __syncthreads();
    return (v1 > v0 || (v1 == v0 && i1 < i0)) ? i1 : i0;
}

// Byte selector of v_perm_b32 that moves the bf16 of dim `dim` of a packed
// pair into the high half of a float (low half zero): bytes 1,0 for an even
// dim, 3,2 for an odd one (0x0c selects a zero byte).
__device__ __forceinline__ uint32_t bf16_select(int dim) { return (dim & 1) ? 0x03020c0cu : 0x01000c0cu; }

// block_elem for a per-lane dim, with the selector precomputed: one v_perm_b32
// instead of both conversions and a select.
__device__ __forceinline__ float block_elem_sel(const uint32_t* block, int row, int word, uint32_t sel) {
    const uint32_t w = block[row * kRowWords + word];
    return __uint_as_float(__builtin_amdgcn_perm(w, w, sel));
}

__global__ __launch_bounds__(kClusterThreads) void cluster_pool_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    uint16_t* __restrict__ centroids, float* __restrict__ pops, uint16_t* __restrict__ pooled,
    int64_t n, int64_t qb, float qk_scale_log2, const int32_t* __restrict__ order) {
    __shared__ uint32_t block[kQueryBlock * kRowWords];
    __shared__ float center_row[kHeadDim];
    __shared__ float s_val[2];
    __shared__ int s_idx[2];
    __shared__ uint64_t slot_mask[kClusterThreads / 64][kCentroids];

    const int tid = threadIdx.x;
    const int64_t blk = blockIdx.x, bh = blockIdx.y;
    const int64_t base = blk * kQueryBlock;
    const int valid = static_cast<int>(min<int64_t>(kQueryBlock, n - base));
    const int64_t row = bh * qb + blk;

    // Every global load of the workgroup is issued at once, before any is
    // used: thread tid loads 16 bytes of query rows tid/16 + 8i (i < 16) and
    // of the key pairs tid/16 + 8i (i < 8), so the block costs one memory
    // round trip instead of one per row group. Rows past the sequence end
    // read as zero (queries) or are skipped (keys).
    const u32x4* qhead = reinterpret_cast<const u32x4*>(q + bh * n * kHeadDim);
    const u32x4* khead = reinterpret_cast<const u32x4*>(k + bh * n * kHeadDim);
    const int c16 = tid & 15, r0 = tid >> 4;
    const int pairs = valid / 2;
    // Token t of the head is stored row t, or order[t] for a permuted token
    // layout (clamped into the head). Stored rows of query row r0 + 8i and of
    // key rows 2p + (i & 1), p = r0 + 8(i/2); rows past the sequence end are
    // clamped (their loads are discarded), and every order entry is loaded
    // before any data load.
    // Offsets in 16-byte units from the head's base (32-bit: a head has at
    // most 131,072 tokens, 2,097,152 units).
    const int nm1 = static_cast<int>(n - 1), b32 = static_cast<int>(base);
    uint32_t soff[16];
    if (order) {
        int32_t o[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) o[i] = order[b32 + min(r0 + 8 * i, valid - 1)];
#pragma unroll
        for (int i = 0; i < 16; ++i) soff[i] = uint32_t(min(max(o[i], 0), nm1)) * 16u + c16;
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) soff[i] = uint32_t(b32 + min(r0 + 8 * i, valid - 1)) * 16u + c16;
    }
    uint32_t koff[16];
    if (order) {
        int32_t o[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) o[i] = order[b32 + min(2 * (r0 + 8 * (i >> 1)) + (i & 1), valid - 1)];
#pragma unroll
        for (int i = 0; i < 16; ++i) koff[i] = uint32_t(min(max(o[i], 0), nm1)) * 16u + c16;
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) koff[i] = uint32_t(b32 + min(2 * (r0 + 8 * (i >> 1)) + (i & 1), valid - 1)) * 16u + c16;
    }
    u32x4 qv[16], ka[8], kb[8];
#pragma unroll
    for (int i = 0; i < 16; ++i) qv[i] = qhead[soff[i]];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        ka[i] = khead[koff[2 * i]];
        kb[i] = khead[koff[2 * i + 1]];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (r0 + 8 * i >= valid) qv[i] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        uint32_t* dst = block + (r0 + 8 * i) * kRowWords + c16 * 4;
        dst[0] = qv[i].x;
        dst[1] = qv[i].y;
        dst[2] = qv[i].z;
        dst[3] = qv[i].w;
    }
    // Pool the same tokens' keys: bf16(0.5 * (k_2r + k_2r+1)) (:244-266).
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
    __syncthreads();

    // Thread tid owns dim tid in the column passes: its word of a packed row
    // and the selector of its half.
    const int my_word = tid >> 1;
    const uint32_t my_sel = bf16_select(tid);
    // Per-dim mean over valid queries in row order (csrc/ibcs.cu:130-140).
    {
        float sum = 0.0f;
        int i = 0;
        for (; i + 8 <= valid; i += 8) {  // 8 reads in flight, adds in row order
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = block_elem_sel(block, i + e, my_word, my_sel);
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += v[e];
        }
        for (; i < valid; ++i) sum += block_elem_sel(block, i, my_word, my_sel);
        center_row[tid] = __fdiv_rn(sum, static_cast<float>(valid));
    }
    float x[kHeadDim];
#pragma unroll
    for (int w = 0; w < kHeadDim / 2; ++w) {
        const uint32_t v = block[tid * kRowWords + w];
        x[2 * w] = bf16_lo(v);
        x[2 * w + 1] = bf16_hi(v);
    }
    __syncthreads();

    // Farthest-first centres with nearest-centre assignment (:158-197).
    const bool live = tid < valid;
    float min_d = live ? lane_distance(x, center_row) : -INFINITY;
    int center = block_argmax(min_d, tid, s_val, s_idx);
    min_d = INFINITY;
    int assign = 0;
    for (int slot = 0; slot < kCentroids; ++slot) {
        center_row[tid] = block_elem_sel(block, center, my_word, my_sel);
        __syncthreads();
        if (live) {
            const float dist = lane_distance(x, center_row);
            if (dist < min_d) {
                min_d = dist;
                assign = slot;
            }
        }
        if (slot + 1 < kCentroids) center = block_argmax(live ? min_d : -INFINITY, tid, s_val, s_idx);
        __syncthreads();
    }

    // Members of each slot: per wave, the ballot of the queries assigned to
    // it. Queries 64w + bit, walked wave by wave and bit by bit, come in
    // query order (the reference's member order).
    {
        const int wave = tid >> 6;
#pragma unroll
        for (int s = 0; s < kCentroids; ++s) {
            const uint64_t m = __ballot(live && assign == s);
            if ((tid & 63) == 0) slot_mask[wave][s] = m;
        }
    }
    __syncthreads();
    if (tid < kCentroids)
        pops[row * kCentroids + tid] =
            static_cast<float>(__popcll(slot_mask[0][tid]) + __popcll(slot_mask[1][tid]));

    // Centroid = bf16(member sum / count), then the LSE pre-scale
    // bf16(centroid * 128^-0.5 * log2 e) (csrc/ibcs.cu:213-237, :293-295).
    // Members are read 8 at a time; the sum adds them in query order (the
    // unused tail of a group adds +0.0f, which leaves a sum that started at
    // +0.0f unchanged).
    {
        uint16_t* dst = centroids + row * kCentroids * kHeadDim + tid;
        for (int s = 0; s < kCentroids; ++s) {
            float sum = 0.0f;
            int cnt = 0;
#pragma unroll
            for (int w = 0; w < kClusterThreads / 64; ++w) {
                uint64_t m = slot_mask[w][s];
                cnt += __popcll(m);
                while (m != 0u) {
                    int idx[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        idx[e] = m != 0u ? 64 * w + __builtin_ctzll(m) : -1;
                        m &= m - 1u;
                    }
                    float v[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = block_elem_sel(block, max(idx[e], 0), my_word, my_sel);
#pragma unroll
                    for (int e = 0; e < 8; ++e) sum += idx[e] >= 0 ? v[e] : 0.0f;
                }
            }
            const uint32_t c = cnt > 0 ? f32_to_bf16(__fdiv_rn(sum, static_cast<float>(cnt))) : 0u;
            dst[s * kHeadDim] = static_cast<uint16_t>(f32_to_bf16(__uint_as_float(c << 16) * qk_scale_log2));
        }
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
