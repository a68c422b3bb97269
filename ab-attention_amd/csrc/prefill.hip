// Weighted paged sparse prefill on gfx950 (bf16 MFMA flash attention).
//
// Computes, for every 128-query row of the plan and every valid query i,
//   z_t = q_i . k_t * log2(e)/sqrt(128) + w_j      (key t in KV4 block j)
//   o_i = sum_t 2^(z_t - m) v_t / sum_t 2^(z_t - m),  lse_i = m + log2(sum_t 2^(z_t - m))
// over exactly the row's S sampled KV4 blocks (4S keys). This is the
// ABSipAttention variant of the reference's FlashInfer prefill
// (ab_attention/flashinfer_backend.py:30-59): logits + w / (sm_scale*log2 e),
// then an online softmax in base 2 with scale sm_scale*log2 e.
//
// Kernel shape: one workgroup (4 waves) per row; wave w owns queries
// 32w..32w+31. The row's pages are streamed in tiles of 16 KV4 blocks (64
// keys): each tile's K rows and transposed V are staged in LDS (double
// buffered, global loads of tile t+1 in flight while tile t computes).
//   S^T = K Q^T  : v_mfma_f32_32x32x16_bf16, A = K rows from LDS, B = Q in VGPRs
//                  -> each lane holds one query and 16 keys per 32-key half,
//                     in 4-key groups that are exactly one KV4 block.
//   O^T += V^T P^T: A = V^T read from the row-major V tile with the
//                  transposing LDS read ds_read_b64_tr_b16, B = P straight
//                  from the S^T accumulators (bf16); the key order of each
//                  MFMA k-step is chosen so no cross-lane movement is needed.
// LDS tiles (16 KiB each, double buffered) are swizzled so that both the
// 16-byte stores from the loader and the operand reads are bank-conflict free:
//   K: [key][16 chunks of 16 B], chunk position = chunk ^ (key & 15);
//   V: per page 8 blocks of 4 keys x 16 dims (128 B); inside block m the row
//      of key r sits at position r ^ ((m >> 1) & 3), so each 16-lane group of
//      a transposing read fetches one whole 128-byte block.
#include "common.hpp"

namespace ab {
namespace {

constexpr int kPfThreads = 256;
constexpr int kTilePages = 16;
constexpr int kTileKeys = kTilePages * kKvBlock;              // 64
constexpr int kTileBytes = kTileKeys * kHeadDim * 2;         // 16 KiB
constexpr int kStageBytes = 2 * kTileBytes + 128;             // K, V, weights
// Largest p = 2^(y) allowed before the running reference is moved.
constexpr float kSlack = 8.0f;

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Transposing LDS read: within each 16-lane group, lane i receives element
// i%4 of the 8 bytes read by lanes 4r + i/4, for r = 0..3 (so the group reads
// a 4 x 16 tile of 16-bit values, row r from lanes 4r..4r+3, and each lane
// gets one column).
__device__ __forceinline__ i16x4 lds_read_tr16(const unsigned char* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

__global__ __launch_bounds__(kPfThreads, 2) void prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const int32_t* __restrict__ ids, const float* __restrict__ logw, uint16_t* __restrict__ out,
    float* __restrict__ lse, int64_t n, int64_t qb, int64_t rows, int fb, int samples, float scale_log2) {
    extern __shared__ __align__(16) unsigned char smem[];

    // XCD-aware row order. The hardware deals workgroups round-robin over the
    // 8 XCDs, so workgroup w runs on XCD w % 8. Slot w / 8 walks the heads in
    // order: at any time all XCDs work on the same head (its K/V stay in the
    // shared last-level cache), each on a contiguous eighth of its query
    // blocks (neighbouring blocks share most sampled pages in the XCD's L2).
    const int64_t hw = blockIdx.x;
    const int64_t xcd = hw & 7, slot = hw >> 3;
    const int64_t per_xcd = (qb + 7) / 8;
    const int64_t bh = slot / per_xcd;
    const int64_t blk = xcd * per_xcd + slot % per_xcd;
    if (bh >= rows / qb || blk >= qb) return;
    const int64_t row = bh * qb + blk;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int qi = lane & 31, half = lane >> 5;
    const int64_t token = blk * kQueryBlock + wave * 32 + qi;
    const bool valid_q = token < n;

    // Q as the B operand of S^T = K Q^T: dims 16s + 8*half .. +8.
    bf16x8 bq[8];
    {
        const uint16_t* qrow = q + (bh * n + (valid_q ? token : 0)) * kHeadDim + 8 * half;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            u32x4 val = {0u, 0u, 0u, 0u};
            if (valid_q) val = *reinterpret_cast<const u32x4*>(qrow + 16 * s);
            bq[s] = __builtin_bit_cast(bf16x8, val);
        }
    }

    const int32_t* row_ids = ids + row * int64_t(samples);
    const float* row_w = logw + row * int64_t(samples);
    const u32x4* kbase = reinterpret_cast<const u32x4*>(k + bh * n * kHeadDim);
    const u32x4* vbase = reinterpret_cast<const u32x4*>(v + bh * n * kHeadDim);
    const int tiles = samples / kTilePages;

    // Loader role: page lp = tid/16 of the tile, 16-byte chunk lc = tid%16.
    const int lp = tid >> 4, lc = tid & 15;
    u32x4 kreg[4], vreg[4];
    float wreg = 0.f;
    auto load_tile = [&](int tile) {
        // Clamp so a malformed plan can never address outside the head.
        const int64_t j = min(max(row_ids[tile * kTilePages + lp], 0), fb - 1);
        const int64_t first = (4 * j) * 16 + lc;  // in 16-byte units
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            kreg[i] = kbase[first + 16 * i];
            vreg[i] = vbase[first + 16 * i];
        }
        wreg = row_w[tile * kTilePages + lp];
    };
    // Loader's LDS offsets (key 4*lp + i, 16-byte chunk lc).
    const int v_store = lp * 1024 + (lc >> 1) * 128 + (lc & 1) * 16;
    const int v_swz = (lc >> 2) & 3;  // (block >> 1) & 3 with block = lc >> 1
    auto store_tile = [&](unsigned char* st) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = 4 * lp + i;
            *reinterpret_cast<u32x4*>(st + key * 256 + 16 * (lc ^ (key & 15))) = kreg[i];
            *reinterpret_cast<u32x4*>(st + kTileBytes + v_store + 32 * (i ^ v_swz)) = vreg[i];
        }
        if (lc == 0) {
            // weights ordered [half][kt][g] for page 8kt + 2g + half
            const int h = lp & 1, kt = lp >> 3, g = (lp >> 1) & 3;
            reinterpret_cast<float*>(st + 2 * kTileBytes)[h * 8 + kt * 4 + g] = wreg;
        }
    };

    // Operand-read offsets of this lane (stage-relative).
    int k_off[8];  // S^T A operand: key qi (+32kt), chunk 2s + half
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) k_off[s8] = qi * 256 + 16 * ((2 * s8 + half) ^ (qi & 15));
    int v_off[4];  // PV A operand, transposing read: page half (+4ks + 2t), block 2dt + (lane>>4)&1
    {
        const int gd = (lane >> 4) & 1, r = (lane >> 2) & 3, q = lane & 3;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
            v_off[dt] = kTileBytes + half * 1024 + (2 * dt + gd) * 128 + 32 * (r ^ dt) + 8 * q;
    }

    f32x16 o_acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[dt][r] = 0.f;
    float m_run = 0.f, l_run = 0.f;  // reference set by the first tile

    load_tile(0);
    store_tile(smem);
    __syncthreads();

    for (int tile = 0; tile < tiles; ++tile) {
        const bool more = tile + 1 < tiles;
        if (more) load_tile(tile + 1);
        const unsigned char* st = smem + (tile & 1) * kStageBytes;
        const float* ws = reinterpret_cast<const float*>(st + 2 * kTileBytes);

        // S^T for the two 32-key halves.
        f32x16 sacc[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            f32x16 c;
#pragma unroll
            for (int r = 0; r < 16; ++r) c[r] = 0.f;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const bf16x8 a = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4*>(st + k_off[s] + kt * 32 * 256));
                c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bq[s], c, 0, 0, 0);
            }
            sacc[kt] = c;
        }

        // Logits in base 2 with the block weights; lane register r holds key
        // 8*(r/4) + 4*half + r%4 of its half, i.e. page 8kt + 2(r/4) + half.
        // Scores are kept relative to the running reference m_run:
        //   y = s * log2(e)/sqrt(d) + (w - m_run),   p = 2^y.
        float wm[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) wm[i] = ws[half * 8 + i] - m_run;
        float tmax = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float y = __builtin_fmaf(sacc[kt][r], scale_log2, wm[kt * 4 + (r >> 2)]);
                sacc[kt][r] = y;
                tmax = fmaxf(tmax, y);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        // Lazy rescaling: the reference moves only when the tile maximum exceeds
        // it by more than kSlack (so p <= 2^kSlack); the branch is wave-uniform.
        const bool grow = tile == 0 || tmax > kSlack;
        if (__any(grow)) {
            const float shift = grow ? tmax : 0.f;
            const float alpha = fast_exp2(-shift);
            m_run += shift;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o_acc[dt][r] *= alpha;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) sacc[kt][r] -= shift;
        }
        float psum = 0.f;
        uint32_t pw[2][4][2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float p[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    p[i] = fast_exp2(sacc[kt][4 * g + i]);
                    psum += p[i];
                }
                pw[kt][g][0] = pack_bf16(p[0], p[1]);
                pw[kt][g][1] = pack_bf16(p[2], p[3]);
            }
        l_run += psum;

        // O^T += V^T P^T over 4 k-steps of 16 keys. MFMA k-index 8*half + 4t + r
        // of k-step ks is key r of tile page 4*ks + 2t + half, on both operands.
        // A operand of lane (group g = lane/16, i = lane%16): two transposing
        // reads; the source lane 4r + q addresses key r of that page, dims
        // 32dt + 16(g%2) + 4q .. +3, so lane i receives dim 32dt + 16(g%2) + i.
#pragma unroll
        for (int ks4 = 0; ks4 < 4; ++ks4) {
            const int kt = ks4 >> 1, g0 = 2 * (ks4 & 1);
            const u32x4 bw = {pw[kt][g0][0], pw[kt][g0][1], pw[kt][g0 + 1][0], pw[kt][g0 + 1][1]};
            const bf16x8 b = __builtin_bit_cast(bf16x8, bw);
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const unsigned char* p0 = st + v_off[dt] + ks4 * 4096;
                const i16x4 lo = lds_read_tr16(p0);
                const i16x4 hi = lds_read_tr16(p0 + 2048);
                const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                o_acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, o_acc[dt], 0, 0, 0);
            }
        }

        if (more) store_tile(smem + ((tile + 1) & 1) * kStageBytes);
        __syncthreads();
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32);
    if (valid_q) {
        const float inv = 1.0f / l_tot;
        uint16_t* orow = out + (bh * n + token) * kHeadDim;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const u32x2 pk = {pack_bf16(o_acc[dt][4 * g] * inv, o_acc[dt][4 * g + 1] * inv),
                                  pack_bf16(o_acc[dt][4 * g + 2] * inv, o_acc[dt][4 * g + 3] * inv)};
                *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * g + 4 * half) = pk;
            }
        if (lse != nullptr && half == 0) lse[bh * n + token] = m_run + log2f(l_tot);
    }
}

}  // namespace

int launch_prefill(const void* q, const void* k, const void* v, int64_t bh, int64_t n, const int32_t* ids,
                   const float* logw, int64_t samples, void* out, float* lse, hipStream_t stream) {
    const int64_t qb = (n + kQueryBlock - 1) / kQueryBlock;
    const int64_t rows = bh * qb;
    if (samples % kTilePages != 0)
        return set_error(1, "prefill: samples (%lld) must be a multiple of %d", (long long)samples, kTilePages);
    const float scale_log2 = static_cast<float>(1.4426950408889634 / 11.313708498984761);  // log2(e)/sqrt(128)
    const int64_t per_xcd = (qb + 7) / 8;
    const size_t lds = 2 * kStageBytes;
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(prefill_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        attr_set = true;
    }
    if (rows == 0) return 0;
    hipLaunchKernelGGL(prefill_kernel, dim3(static_cast<unsigned>(per_xcd * 8 * bh)), dim3(kPfThreads), lds, stream,
                       static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                       static_cast<const uint16_t*>(v), ids, logw, static_cast<uint16_t*>(out), lse, n, qb, rows,
                       static_cast<int>(n / kKvBlock), static_cast<int>(samples), scale_log2);
    return check_launch("prefill_kernel");
}

}  // namespace ab
