// IBCS stage 3 on gfx950: pair-LSE of every (centroid, KV4 block) with
// per-centroid online normalisers (reference: csrc/ibcs.cu:329-489).
//
//   l_sj = fp16( mx + log2(1 + 2^(mn - mx)) ),  {mx, mn} = {max, min}(t0 + 1, t1 + 1)
//   t_r  = c_s . k_(j,r)     (scaled bf16 centroid, bf16 pooled key rep r)
//   M_s  = max_j l_sj,  D_s = sum_j 2^(l_sj - M_s)
//
// exp2(a-mx) + exp2(b-mx) == 1 + exp2(-|a-b|) because exp2(0) == 1; the
// reference's max(sum, 1e-20) floor never binds for finite inputs (sum >= 1).
// D is accumulated from the fp16-rounded values against a lazily moved
// reference and rebased on the exact maximum at the end, which matches the
// reference up to fp32 rounding order. The reference moves under one
// wave-uniform branch per chunk (rarely taken), and the head's last chunk is
// handled outside the main loop, so the loop body is a single path.
//
// This file is compiled with -fno-honor-nans: every input is finite, and
// without NaNs fmaxf/fminf of MFMA results are single instructions.
//
// One workgroup = 4 waves = 8 query blocks (64 centroid rows) of one head.
// The head's KV4 blocks are taken in chunks of 16; in round i wave w handles
// chunk 4i + w, so every pooled key is read by exactly one wave. A chunk (32
// pooled rows, 8 KiB) reaches the wave's LDS buffer by global_load_lds_dwordx4;
// the wave reads it into registers in MFMA layout (rows swizzled so that the
// reads are conflict free) and at once starts the transfer of its next chunk
// into the same buffer, which then overlaps the whole computation. 48 KiB of
// LDS and at most 168 VGPRs let three workgroups share a CU.
// Per chunk and 16-row centroid tile, v_mfma_f32_16x16x32_bf16 computes
// D = R C^T with A = 16 pooled rows (block j0+i, rep r) and B = 16 centroid
// rows (kept in VGPRs), so lane l holds blocks j0 + 4(l/16) .. +3 of
// centroid row l%16. The accumulator starts at 1.0, which adds the
// reference's +1 to both pair dot products. The fp16 results of a round
// (64 rows x 64 blocks) are gathered in LDS and written out as whole
// 128-byte rows.
#include <cfloat>
#include <type_traits>

#include "common.hpp"

namespace ab {

int64_t lse_stride(int64_t fb);  // ibcs.hip

namespace {

constexpr int kLseThreads = 256;
constexpr int kLseQBlocks = 8;   // query blocks per workgroup
constexpr int kLseRows = kLseQBlocks * kCentroids;
constexpr int kLseChunk = 16;    // KV4 blocks per wave step
constexpr int kLseChunkBytes = kLseChunk * kReps * kHeadDim * 2;  // 8 KiB
constexpr int kLseInBytes = 4 * kLseChunkBytes;                   // one buffer per wave
constexpr int kLseOutBytes = kLseRows * 4 * kLseChunk * 2;        // 8 KiB per round
constexpr int kLseLdsBytes = kLseInBytes + 2 * kLseOutBytes;      // 48 KiB
// Largest 2^(l - ref) allowed before the normaliser's reference is moved.
constexpr float kLseSlack = 8.0f;

static_assert(3 * kLseLdsBytes <= 160 * 1024, "three workgroups per CU must fit in LDS");

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes per lane from base + voffset into LDS bytes [lds + 16j, +16) for
// lane j, counted by vmcnt. Nothing else in this kernel keeps m0 live.
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t voffset, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voffset), "s"(base)
                 : "memory", "m0");
}
// The same, after waiting for every earlier LDS access of this wave (the
// transfer overwrites a buffer this wave has just read).
__device__ __forceinline__ void lds_dma16_after_reads(const void* base, uint32_t voffset, uint32_t lds) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voffset),
                 "s"(base)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ void combine_pair(float& m, float& d, float om, float od) {
    const float nm = fmaxf(m, om);
    d = d * fast_exp2(m - nm) + od * fast_exp2(om - nm);
    m = nm;
}

__global__ __launch_bounds__(kLseThreads, 3) void lse_kernel(
    const uint16_t* __restrict__ centroids, const uint16_t* __restrict__ pooled,
    _Float16* __restrict__ lse, float* __restrict__ lse_max, float* __restrict__ lse_den,
    int64_t qb, int fb, int64_t ld, int groups_per_head, int total_groups) {
    extern __shared__ __align__(16) unsigned char smem[];

    // XCD-aware order: hardware deals workgroups round-robin over 8 XCDs, so
    // consecutive logical groups (same head) are given to one XCD.
    const int hw = blockIdx.x;
    const int per_xcd = (total_groups + 7) / 8;
    const int logical = (hw & 7) * per_xcd + (hw >> 3);
    if (logical >= total_groups) return;
    const int64_t bh = logical / groups_per_head;
    const int64_t qgroup = logical % groups_per_head;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, quad = lane >> 4;

    // B operand: centroid row 16*rt + col (query block 2rt + col/8 of the
    // group, centroid col%8), dims 32s + 8*quad .. +8.
    bf16x8 cen[4][4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
        const int64_t qbk = qgroup * kLseQBlocks + 2 * rt + (col >> 3);
        const int64_t crow = (bh * qb + min(qbk, qb - 1)) * kCentroids + (col & 7);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            u32x4 v = *reinterpret_cast<const u32x4*>(centroids + crow * kHeadDim + 32 * s + 8 * quad);
            if (qbk >= qb) v = u32x4{0u, 0u, 0u, 0u};
            cen[rt][s] = __builtin_bit_cast(bf16x8, v);
        }
    }

    const uint16_t* keys = pooled + bh * int64_t(fb) * kReps * kHeadDim;
    const int chunks = (fb + kLseChunk - 1) / kLseChunk;
    const int rounds = (chunks + 3) / 4;
    const uint32_t lds0 = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)smem));
    const uint32_t in_base = lds0 + wave * kLseChunkBytes;

    // Chunk c -> this wave's buffer: 8 transfers of 4 pooled rows. LDS row p
    // (= 2*col + rep) holds its 16-byte chunk k at position k ^ (p/2 % 16);
    // rows past the head's end re-read its last row (never used).
    const int last_row = 2 * fb - 1;
    // Chunks wholly inside the head use a wave-uniform chunk base and the
    // lane's fixed offsets (no per-transfer address arithmetic); only the
    // head's last chunk clamps its rows.
    uint32_t chunk_off[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int p = 4 * k + (lane >> 4);
        chunk_off[k] = uint32_t(p) * 256u + 16u * uint32_t((lane & 15) ^ ((p >> 1) & 15));
    }
    auto issue_chunk = [&](int c) {
        if ((c + 1) * kLseChunk * kReps <= last_row + 1) {
            const uint16_t* base = keys + int64_t(c) * kLseChunk * kReps * kHeadDim;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (k == 0)
                    lds_dma16_after_reads(base, chunk_off[k], in_base + k * 1024);
                else
                    lds_dma16(base, chunk_off[k], in_base + k * 1024);
            }
            return;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int p = 4 * k + (lane >> 4);
            const int row = min(c * kLseChunk * kReps + p, last_row);
            const uint32_t src = uint32_t(row) * 256u + 16u * uint32_t((lane & 15) ^ ((p >> 1) & 15));
            if (k == 0)
                lds_dma16_after_reads(keys, src, in_base + k * 1024);
            else
                lds_dma16(keys, src, in_base + k * 1024);
        }
    };
    // A operand reads: row p = 2*col + r, chunk 4s + quad.
    int a_off[2][4];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int s = 0; s < 4; ++s) a_off[r][s] = (2 * col + r) * 256 + 16 * ((4 * s + quad) ^ col);
    // Round output staging: fp16 [64 rows][64 blocks]; the 16-byte unit U of
    // row R sits at position U ^ ((R >> 1) & 7).
    unsigned char* out_stage = smem + kLseInBytes;

    // Per 16-row tile: exact maximum, normaliser and its reference.
    float top[4], den[4], ref[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
        top[rt] = -FLT_MAX;
        den[rt] = 0.0f;
        ref[rt] = -FLT_MAX;
    }

    const unsigned char* in = smem + (in_base - lds0);
    auto read_chunk = [&](bf16x8 (&a)[2][4]) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                a[r][s] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(in + a_off[r][s]));
    };
    auto compute = [&](int c, int i, const bf16x8 (&a)[2][4], auto tail_tag) {
        constexpr bool kTail = decltype(tail_tag)::value;
        unsigned char* ostage = out_stage + (i & 1) * kLseOutBytes;
        const int jq = c * kLseChunk + 4 * quad;  // first block of this lane
        // fp16 pair-LSEs of each row tile, blocks (0, 1) and (2, 3) (non-tail
        // path). Kept as whole f16x2 values: bit casts of single elements of
        // an ext_vector read element 0 with this compiler.
        f16x2 tile01[4], tile23[4];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            f32x4 acc[2];
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                f32x4 cc = {1.f, 1.f, 1.f, 1.f};
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    cc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[r][s], cen[rt][s], cc, 0, 0, 0);
                acc[r] = cc;
            }
            float l[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float x = acc[0][v], y = acc[1][v];
                l[v] = fmaxf(x, y) + fast_log2(1.0f + fast_exp2(-__builtin_fabsf(x - y)));
            }
            const f16x2 h01 = __builtin_convertvector(f32x2{l[0], l[1]}, f16x2);
            const f16x2 h23 = __builtin_convertvector(f32x2{l[2], l[3]}, f16x2);
            const u32x2 packed = {__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)};
            const int R = 16 * rt + col, u = 4 * wave + quad;  // 8-byte unit of the round row
            *reinterpret_cast<u32x2*>(ostage + R * 128 + 16 * ((u >> 1) ^ ((R >> 1) & 7)) + 8 * (u & 1)) = packed;

            if (kTail) {
                float f[4] = {static_cast<float>(h01[0]), static_cast<float>(h01[1]), static_cast<float>(h23[0]),
                              static_cast<float>(h23[1])};
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (jq + v >= fb) f[v] = -INFINITY;
                const float tmax = fmaxf(fmaxf(f[0], f[1]), fmaxf(f[2], f[3]));
                top[rt] = fmaxf(top[rt], tmax);
                const bool grow = tmax > ref[rt] + kLseSlack;
                if (__any(grow)) {
                    const float nr = grow ? tmax : ref[rt];
                    den[rt] *= fast_exp2(ref[rt] - nr);
                    ref[rt] = nr;
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) den[rt] += fast_exp2(f[v] - ref[rt]);
            } else {
                tile01[rt] = h01;
                tile23[rt] = h23;
            }
        }
        if (!kTail) {
            // The maximum of each tile's four fp16 values in fp16 (exact).
            // One wave-uniform branch per chunk moves the references of every
            // row tile that needs it (rare); tiles and lanes that do not grow
            // take nr == ref, and den * 2^0 leaves den unchanged.
            float tmax[4];
            bool grow_any = false;
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const f16x2 m2 = __builtin_elementwise_max(tile01[rt], tile23[rt]);
                tmax[rt] = static_cast<float>(m2[0] > m2[1] ? m2[0] : m2[1]);
                top[rt] = fmaxf(top[rt], tmax[rt]);
                grow_any |= tmax[rt] > ref[rt] + kLseSlack;
            }
            if (__any(grow_any)) {
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    const float nr = tmax[rt] > ref[rt] + kLseSlack ? tmax[rt] : ref[rt];
                    den[rt] *= fast_exp2(ref[rt] - nr);
                    ref[rt] = nr;
                }
            }
            // f - ref straight from the fp16 halves with v_fma_mix_f32
            // (f16 -> f32 is exact, so this is the rounded f - ref).
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const uint32_t lo = __builtin_bit_cast(uint32_t, tile01[rt]);
                const uint32_t hi = __builtin_bit_cast(uint32_t, tile23[rt]);
                den[rt] += fast_exp2(f16_minus<false>(lo, ref[rt]));
                den[rt] += fast_exp2(f16_minus<true>(lo, ref[rt]));
                den[rt] += fast_exp2(f16_minus<false>(hi, ref[rt]));
                den[rt] += fast_exp2(f16_minus<true>(hi, ref[rt]));
            }
        }
    };

    // Whole rows of round j: thread t writes 16 bytes of rows t/8 and t/8 + 32
    // (blocks past fb land in the row padding, never read). The rows of a
    // wave belong to query blocks w and w + 4 of the group, so the number of
    // stores a wave issues (n_st) is uniform.
    const int n_st = int(qgroup * kLseQBlocks + wave < qb) + int(qgroup * kLseQBlocks + wave + 4 < qb);
    auto store_round = [&](int j) {
        const unsigned char* ostage = out_stage + (j & 1) * kLseOutBytes;
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int R = (tid >> 3) + 32 * h2, U = tid & 7;
            const int64_t qbk = qgroup * kLseQBlocks + R / kCentroids;
            const u32x4 val = *reinterpret_cast<const u32x4*>(ostage + R * 128 + 16 * (U ^ ((R >> 1) & 7)));
            // Streaming store: the pair-LSEs are read back only by the next
            // kernel, and allocating them in the caches would evict the
            // pooled keys that every workgroup of the head re-reads.
            if (qbk < qb)
                __builtin_nontemporal_store(
                    val, reinterpret_cast<u32x4*>(lse + ((bh * qb + qbk) * kCentroids + R % kCentroids) * ld +
                                                  64 * j + 8 * U));
        }
    };

    // Round i: write out round i-1, wait for chunk c (the stores issued after
    // its transfer may stay outstanding), read it into registers, start the
    // transfer of chunk c + 4 into the same buffer, compute chunk c into the
    // staging buffer of round i.
    auto wait_chunk = [&](int i) {
        switch (i > 0 ? n_st : 0) {
            case 2: wait_vmcnt<2>(); break;
            case 1: wait_vmcnt<1>(); break;
            default: wait_vmcnt<0>(); break;
        }
    };
    if (wave < chunks) issue_chunk(wave);
    // Every round but the last: each wave's chunk c = 4i + wave <= 4 rounds - 5
    // is complete and not the head's last (chunks > 4 (rounds - 1)), so the
    // loop body has one path.
    for (int i = 0; i + 1 < rounds; ++i) {
        const int c = 4 * i + wave;
        if (i > 0) store_round(i - 1);
        wait_chunk(i);
        bf16x8 a[2][4];
        read_chunk(a);
        if (c + 4 < chunks) issue_chunk(c + 4);
        compute(c, i, a, std::false_type{});
        lds_barrier();
    }
    if (rounds > 0) {
        const int i = rounds - 1, c = 4 * i + wave;
        if (i > 0) store_round(i - 1);
        wait_chunk(i);
        if (c < chunks) {
            bf16x8 a[2][4];
            read_chunk(a);
            if (c < chunks - 1)
                compute(c, i, a, std::false_type{});
            else
                compute(c, i, a, std::true_type{});
        }
        lds_barrier();
        store_round(rounds - 1);
    }

    // Rebase each lane's normaliser on its exact maximum, then merge the four
    // lanes (quads) of each centroid row and the four waves.
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) den[rt] *= fast_exp2(ref[rt] - top[rt]);
#pragma unroll
    for (int off = 16; off < 64; off <<= 1)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const float om = __shfl_xor(top[rt], off);
            const float od = __shfl_xor(den[rt], off);
            combine_pair(top[rt], den[rt], om, od);
        }
    __syncthreads();  // the staging area is reused below
    float* s_max = reinterpret_cast<float*>(smem + kLseInBytes);
    float* s_den = s_max + 4 * kLseRows;
    if (quad == 0) {
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            s_max[wave * kLseRows + 16 * rt + col] = top[rt];
            s_den[wave * kLseRows + 16 * rt + col] = den[rt];
        }
    }
    __syncthreads();
    if (tid < kLseRows) {
        float m = s_max[tid], d = s_den[tid];
#pragma unroll
        for (int w = 1; w < 4; ++w) combine_pair(m, d, s_max[w * kLseRows + tid], s_den[w * kLseRows + tid]);
        const int64_t qbk = qgroup * kLseQBlocks + tid / kCentroids;
        if (qbk < qb) {
            const int64_t slot = (bh * qb + qbk) * kCentroids + tid % kCentroids;
            lse_max[slot] = m;
            lse_den[slot] = d;
        }
    }
}

}  // namespace

int launch_lse(const void* centroids, const void* pooled, int64_t bh, int64_t n, void* lse,
               float* lse_max, float* lse_den, hipStream_t stream) {
    const int64_t qb = (n + kQueryBlock - 1) / kQueryBlock;
    const int64_t fb = n / kKvBlock;
    const int groups_per_head = static_cast<int>((qb + kLseQBlocks - 1) / kLseQBlocks);
    const int64_t total = groups_per_head * bh;
    if (total > (int64_t(1) << 30)) return set_error(1, "ibcs: too many query blocks (%lld)", (long long)total);
    const int per_xcd = static_cast<int>((total + 7) / 8);
    if (int rc = ensure_lds_limit(reinterpret_cast<const void*>(lse_kernel), kLseLdsBytes)) return rc;
    hipLaunchKernelGGL(lse_kernel, dim3(static_cast<unsigned>(per_xcd * 8)), dim3(kLseThreads), kLseLdsBytes,
                       stream, static_cast<const uint16_t*>(centroids), static_cast<const uint16_t*>(pooled),
                       static_cast<_Float16*>(lse), lse_max, lse_den, qb, static_cast<int>(fb), lse_stride(fb),
                       groups_per_head, static_cast<int>(total));
    return check_launch("lse_kernel");
}

}  // namespace ab
