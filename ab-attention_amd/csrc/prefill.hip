// Weighted paged sparse prefill on gfx950 (bf16 MFMA flash attention).
//
// Computes, for every 128-query row of the plan and every valid query i,
//   z_t = q_i . k_t * log2(e)/sqrt(128) + w_j      (key t in KV4 block j)
//   o_i = sum_t 2^(z_t - m) v_t / sum_t 2^(z_t - m),  lse_i = m + log2(sum_t 2^(z_t - m))
// over exactly the row's S listed KV4 blocks (4S keys) of the head's K/V,
// which may be longer or shorter than Q (n_kv tokens). This is the
// ABSipAttention variant of the reference's FlashInfer prefill
// (ab_attention/flashinfer_backend.py:30-59): logits + w / (sm_scale*log2 e),
// then an online softmax in base 2 with scale sm_scale*log2 e.
//
// Kernel shape: one workgroup (4 waves) per row, two workgroups per CU; wave
// w owns queries 32w..32w+31. The row's pages are streamed in tiles of 8 KV4
// blocks (32 keys) through two rings of 4 LDS stages, one for K and one for
// V, that the hardware fills directly from global memory
// (global_load_lds_dwordx4: no staging registers). Each wave moves one
// quarter of every tile and waits only for its own transfers (s_waitcnt
// vmcnt) before the workgroup barrier that publishes them; every transfer
// has three steps to land. The page ids and weights of the row reach LDS the
// same way, 64 tiles at a time, so the loop issues no other global or scalar
// loads; ids and weights are read from LDS one step before their use.
// The loop is software pipelined (see step below): each step issues 16 MFMAs
// of two different tiles and places the softmax VALU work, the LDS operand
// reads and the transfers of other tiles between them, so the MFMA pipe of
// each SIMD is fed while LDS and the vector memory path are busy.
//   S^T = K Q^T  : v_mfma_f32_32x32x16_bf16, A = K rows from LDS, B = Q in VGPRs
//                  -> each lane holds one query and 16 keys, in 4-key groups
//                     that are exactly one KV4 block.
//   O^T += V^T P^T: A = V^T read from the row-major V tile with the
//                  transposing LDS read ds_read_b64_tr_b16, B = P straight
//                  from the S^T accumulators (bf16); the key order of each
//                  MFMA k-step is chosen so no cross-lane movement is needed.
// Softmax reference. A row first runs a fast pass: the reference m of each
// query is the maximum of its logits in the first tile (over both lanes that
// hold the query), and every later tile is exponentiated against it; the
// loop keeps only the running maximum of the logits. p = 2^(z - m) <= 2^64
// then keeps every sum of products far inside the float range, and a term
// more than 2^126 below m is below the resolution of a sum that holds a 1,
// so the result is the normalised softmax. If a query has no finite logit in
// the first tile, or a later logit exceeds m by more than 64, the workgroup
// (after a vote through LDS) discards the pass and runs the row again with a
// moving reference: lazy rescaling, where the reference moves only when a
// tile maximum exceeds it by more than 8. The fast loop carries no rescale
// branch and no per-step exchange between lanes, which leaves more of each
// step's issue slots to the MFMAs (5-6 % less time at the benchmark
// configurations). Where no later tile maximum passes the first tile's by
// more than 8, the lazy pass never moves its reference either, and the two
// passes give the same bits.
// LDS tiles are swizzled so that the operand reads are bank-conflict free. A
// transfer instruction writes 1 KiB contiguously (lane j at +16j), so the
// swizzle is realised by the choice of each lane's source address:
//   K: [key][16 chunks of 16 B], chunk position = chunk ^ (key & 15);
//   V: per page 8 blocks of 4 keys x 16 dims (128 B); inside block m the row
//      of key r sits at position r ^ ((m >> 1) & 3), so each 16-lane group of
//      a transposing read fetches one whole 128-byte block.
// Dense attention (every KV4 block at weight 0, no page list) runs on
// dense_kernel: the same rings, pipeline and two passes on
// v_mfma_f32_16x16x32_bf16 tiles (see there).
#include <algorithm>
#include <type_traits>

#include "common.hpp"

namespace ab {
namespace {

constexpr int kPfThreads = 256;
constexpr int kRing = 4;                                       // stages per ring (K and V)
constexpr int kTilePages = 8;                                  // KV4 blocks per tile
constexpr int kPageBytes = kKvBlock * kHeadDim * 2;            // 1 KiB of K (or V)
constexpr int kTileBytes = kTilePages * kPageBytes;            // 8 KiB: K (or V) of one tile
constexpr int kKRing = 0;
constexpr int kVRing = kRing * kTileBytes;
constexpr int kBatchTiles = 64;                                // ids/weights per LDS batch
constexpr int kBatchBytes = kBatchTiles * kTilePages * 4;      // 2 KiB
constexpr int kIdsOffset = 2 * kRing * kTileBytes;             // 2 batch buffers of ids
constexpr int kWeightsOffset = kIdsOffset + 2 * kBatchBytes;   // 2 batch buffers of weights
constexpr int kVoteOffset = kWeightsOffset + 2 * kBatchBytes;  // 4 words: fast-pass votes
constexpr int kLdsBytes = kVoteOffset + 16;                    // 72 KiB + 16 B
constexpr int kGroupOps = 4;                                   // transfers per wave per step
constexpr int64_t kRowsPerLaunch = 11000;                      // see launch_prefill
// Largest p = 2^(y) allowed before the running reference is moved.
constexpr float kSlack = 8.0f;
// Largest logit above the first tile's maximum that the fast pass accepts:
// p <= 2^64 keeps every product and sum far from the float range.
constexpr float kFastRange = 64.0f;

// The dense kernel's LDS: the two rings and the votes.
constexpr int kDenseVoteOffset = 2 * kRing * kTileBytes;
constexpr int kDenseLdsBytes = kDenseVoteOffset + 16;          // 64 KiB + 16 B

static_assert(kLdsBytes * 2 <= 160 * 1024, "two workgroups per CU must fit in LDS");
static_assert(kDenseLdsBytes * 2 <= 160 * 1024, "two dense workgroups per CU must fit in LDS");

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) unsigned char lds_u8;

// Transposing LDS read: within each 16-lane group, lane i receives element
// i%4 of the 8 bytes read by lanes 4r + i/4, for r = 0..3 (so the group reads
// a 4 x 16 tile of 16-bit values, row r from lanes 4r..4r+3, and each lane
// gets one column). lds is an absolute LDS byte address.
__device__ __forceinline__ i16x4 lds_read_tr16(uint32_t lds) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_i16x4*>(static_cast<uintptr_t>(lds)));
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes per lane from base + voffset straight into LDS: lane j writes LDS
// bytes [lds + 16j, lds + 16j + 16). The transfer is counted by vmcnt. The
// kernel holds nothing in m0 across these statements.
__device__ __forceinline__ void dma16(const void* base, uint32_t voffset, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voffset), "s"(base)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt with vmcnt(N) and lgkmcnt(0) (expcnt left open), then a workgroup
// barrier that the compiler cannot move memory accesses across.
template <int N>
__device__ __forceinline__ void wait_and_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
    asm volatile("s_barrier" ::: "memory");
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// v_max_f32 without the NaN quieting the compiler adds around fmaxf of values
// it cannot prove canonical (logits are finite or -inf).
__device__ __forceinline__ float vmax(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
#pragma clang diagnostic pop

// Maxima of a (query 0) and b (query 1) over the four lanes i, 16 + i,
// 32 + i, 48 + i that hold a query in dense_kernel: three swaps of 16-lane
// rows (rows of the results: a01 b01 a23 b23, then a b a b, then all a / all b).
__device__ __forceinline__ void max_over_rows(float& a, float& b) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    const float m = vmax(__uint_as_float(s[0]), __uint_as_float(s[1]));
    const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    const float m2 = vmax(__uint_as_float(t[0]), __uint_as_float(t[1]));
    const auto u = __builtin_amdgcn_permlane16_swap(__float_as_uint(m2), __float_as_uint(m2), false, false);
    a = __uint_as_float(u[0]);
    b = __uint_as_float(u[1]);
}

// XCD-aware row order of the prefill kernels. The hardware deals workgroups
// round-robin over the 8 XCDs, so workgroup w runs on XCD w % 8. Slot w / 8
// walks the heads in order: at any time all XCDs work on the same head (its
// K/V stay in the shared last-level cache), each on a contiguous eighth of its
// query blocks (neighbouring blocks share most sampled pages in the XCD's L2).
// Within an XCD, slots s and s + 32 of each full generation of 64 slots run
// on the same CU (two workgroups per CU), so they take adjacent query blocks:
// their sampled pages overlap and they sweep them in step, which turns part of
// the gathers into L1 hits. A launch covers the slots from slot_base (a
// multiple of 64) on, on every XCD. False for a slot past the rows.
struct RowSlot {
    int64_t bh, blk, row;
};
__device__ __forceinline__ bool row_slot(int64_t slot_base, int64_t qb, int64_t rows, RowSlot& rs) {
    const int64_t hw = blockIdx.x;
    const int64_t xcd = hw & 7, slot0 = slot_base + (hw >> 3);
    const int64_t per_xcd = (qb + 7) / 8;
    const int64_t generation = slot0 >> 6, s64 = slot0 & 63;
    const int64_t slot = (generation + 1) * 64 <= per_xcd * (rows / qb)
                             ? generation * 64 + 2 * (s64 & 31) + (s64 >> 5)
                             : slot0;
    rs.bh = slot / per_xcd;
    rs.blk = xcd * per_xcd + slot % per_xcd;
    if (rs.bh >= rows / qb || rs.blk >= qb) return false;
    rs.row = rs.bh * qb + rs.blk;
    return true;
}

// The sparse prefill: the row's listed KV4 blocks, with their log weights.
__global__ __launch_bounds__(kPfThreads, 2) void prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const int32_t* __restrict__ ids, const float* __restrict__ logw, uint16_t* __restrict__ out,
    float* __restrict__ lse, int64_t n, int64_t n_kv, int64_t qb, int64_t rows, int fb, int samples,
    float scale_log2, const int32_t* __restrict__ order, int64_t slot_base) {
    extern __shared__ __align__(16) unsigned char smem[];

    RowSlot rs;
    if (!row_slot(slot_base, qb, rows, rs)) return;
    const int64_t bh = rs.bh, blk = rs.blk, row = rs.row;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qi = lane & 31, half = lane >> 5;
    const int64_t token = blk * kQueryBlock + wave * 32 + qi;
    const bool valid_q = token < n;
    // Row of Q / out / lse holding this token: the token itself, or
    // order[token] for a permuted token layout (clamped into the head).
    const int64_t qrow_index = !valid_q ? 0 : order ? min<int64_t>(max(order[token], 0), n - 1) : token;
    const int tiles = samples / kTilePages;

    // Q as the B operand of S^T = K Q^T: dims 16s + 8*half .. +8.
    bf16x8 bq[8];
    {
        const uint16_t* qrow = q + (bh * n + qrow_index) * kHeadDim + 8 * half;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            u32x4 val = {0u, 0u, 0u, 0u};
            if (valid_q) val = *reinterpret_cast<const u32x4*>(qrow + 16 * s);
            bq[s] = __builtin_bit_cast(bf16x8, val);
        }
    }

    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8*)smem));
    const int32_t* row_ids = ids + row * int64_t(samples);
    const float* row_w = logw + row * int64_t(samples);
    const uint16_t* kbase = k + bh * n_kv * kHeadDim;
    const uint16_t* vbase = v + bh * n_kv * kHeadDim;

    // Batch b of ids and weights (tiles 64b .. 64b+63) into buffer b & 1, by
    // wave 0: two 1 KiB transfers each. Lanes past the row's end re-read its
    // last 16 bytes (those entries are never used).
    const uint32_t row_bytes = static_cast<uint32_t>(samples) * 4u;
    auto issue_batch = [&](int b) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t src = min(uint32_t(b) * kBatchBytes + i * 1024u + 16u * lane, row_bytes - 16u);
            const uint32_t dst = (b & 1) * kBatchBytes + i * 1024u;
            dma16(row_ids, src, lds0 + kIdsOffset + dst);
            dma16(row_w, src, lds0 + kWeightsOffset + dst);
        }
    };

    // Transfers of this wave: pages 2w and 2w+1 of a K tile and of a V tile.
    // Source offsets inside a page (1 KiB = 4 keys x 256 B) for lane j:
    //   K: key r = j/16 at LDS chunk position j%16 holds chunk pos ^ (key & 15);
    //   V: block m = j/8, row slot (j/2)%4 holds key slot ^ ((m>>1)&3), dims 16m + 8(j%2).
    uint32_t k_src[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int r = lane >> 4, pos = lane & 15;
        const int key = 4 * (2 * wave + e) + r;
        k_src[e] = uint32_t(r * 16 + (pos ^ (key & 15))) * 16u;
    }
    const uint32_t v_src = [&] {
        const int m = lane >> 3, sl = (lane >> 1) & 3, h = lane & 1;
        return uint32_t((sl ^ ((m >> 1) & 3)) * 16 + 2 * m + h) * 16u;
    }();
    // This wave's two page ids of tile u, clamped into the head (a malformed
    // plan can never address outside it); tiles past the row's end read its
    // last tile (their transfers only keep the per-step count uniform).
    auto load_ids = [&](int u) {
        const int uc = min(u, tiles - 1);
        const u32x2 raw = *reinterpret_cast<const u32x2*>(smem + kIdsOffset + ((uc / kBatchTiles) & 1) * kBatchBytes +
                                                          ((uc % kBatchTiles) * kTilePages + 2 * wave) * 4);
        const u32x2 c = {uint32_t(min(max(static_cast<int>(raw[0]), 0), fb - 1)),
                         uint32_t(min(max(static_cast<int>(raw[1]), 0), fb - 1))};
        return c;
    };
    auto dma_k = [&](int u, uint32_t id, int e) {
        dma16(kbase, id * kPageBytes + k_src[e], lds0 + kKRing + (u & (kRing - 1)) * kTileBytes + (2 * wave + e) * kPageBytes);
    };
    auto dma_v = [&](int u, uint32_t id, int e) {
        dma16(vbase, id * kPageBytes + v_src, lds0 + kVRing + (u & (kRing - 1)) * kTileBytes + (2 * wave + e) * kPageBytes);
    };
    // The four block weights of this lane's keys in tile u: lane register r
    // holds key 8*(r/4) + 4*half + r%4, i.e. page 2(r/4) + half.
    auto load_weights = [&](int u, float (&wv)[4]) {
        const int uc = min(u, tiles - 1);
        const float* ws = reinterpret_cast<const float*>(smem + kWeightsOffset +
                                                         ((uc / kBatchTiles) & 1) * kBatchBytes) +
                          (uc % kBatchTiles) * kTilePages;
#pragma unroll
        for (int g = 0; g < 4; ++g) wv[g] = ws[2 * g + half];
    };

    // Operand-read offsets of this lane (stage-relative).
    int k_off[8];  // S^T A operand: key qi, chunk 2s + half
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) k_off[s8] = qi * 256 + 16 * ((2 * s8 + half) ^ (qi & 15));
    int v_off[4];  // PV A operand, transposing read: page half (+4ks + 2t), block 2dt + (lane>>4)&1
    {
        const int gd = (lane >> 4) & 1, r = (lane >> 2) & 3, q4 = lane & 3;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) v_off[dt] = half * 1024 + (2 * dt + gd) * 128 + 32 * (r ^ dt) + 8 * q4;
    }
    // The same as absolute LDS addresses, so every operand read is one
    // register plus the instruction's constant offset (the dynamic-LDS base
    // is not a compile-time constant and would cost an add per read).
    uint32_t k_abs[8], v_abs[4];
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) k_abs[s8] = lds0 + kKRing + k_off[s8];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) v_abs[dt] = lds0 + kVRing + v_off[dt];
    auto read_k = [&](int u, int j) {
        return *reinterpret_cast<const lds_u32x4*>(
            static_cast<uintptr_t>(k_abs[j] + (u & (kRing - 1)) * kTileBytes));
    };
    // PV A operand j of tile u: V^T for k-step j/4, dims 32(j%4) .. +31. MFMA
    // k-index 8*half + 4t + r of k-step ks is key r of tile page 4*ks + 2t +
    // half, on both operands. Lane (group g = lane/16, i = lane%16) does two
    // transposing reads; the source lane 4r + q addresses key r of that page,
    // dims 32dt + 16(g%2) + 4q .. +3, so lane i receives dim 32dt + 16(g%2) + i.
    auto read_v = [&](int u, int j) {
        const uint32_t a0 = v_abs[j & 3] + (u & (kRing - 1)) * kTileBytes + (j >> 2) * 4096;
        const i16x4 lo = lds_read_tr16(a0), hi = lds_read_tr16(a0 + 2048);
        return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };

    f32x16 o_acc[4];
    // Reference, running sum and state of this lane's query; mx is the same
    // in both lane halves of a query after the exchange, so they are too.
    float m_run, l_run;
    bool started;

    // Step t works on three tiles at once, so that every MFMA of the wave has
    // independent VALU and LDS work beside it. Entering step t, sc holds the
    // logits y = s*log2(e)/sqrt(d) + (w - m_run) of S(t).
    //   phase A: S(t+1) = K(t+1) Q^T (K(t+1) already in registers), beside
    //            p = 2^y of S(t), the reads of V(t) and this step's four
    //            transfers;
    //   phase B: O += V(t)^T P(t)^T, beside the logits of S(t+1) and the
    //            reads of K(t+2) for the next step.
    // Fast pass (kSafe false): the reference stays where the first tile put
    // it and mx is the running maximum of every logit of the lane, checked
    // after the loop. Safe pass: mx is the maximum of S(t) over this lane's
    // keys and the reference moves only when a tile maximum exceeds it by
    // more than kSlack (so p <= 2^kSlack), decided per wave at the start of
    // the step that exponentiates the tile.
    // Rings: K(u) is read in step u-2 and V(u) in step u. Step t transfers
    // K(t+5) into the stage of K(t+1) and V(t+3) into the stage of V(t-1),
    // both read in step t-1; the barrier at the top of step t retires those
    // reads and publishes K(t+2) and V(t) (transferred in step t-3), so every
    // transfer has three steps. Transfers past the row's end keep the count
    // uniform (4 per wave per step) and land in stages nobody reads again.
    auto step = [&](auto safe, int t, f32x16& sc, f32x16& sn, float& mx, u32x4 (&ka)[8], float (&wn)[4],
                    u32x2& idk, u32x2& idv) {
        constexpr bool kSafe = decltype(safe)::value;
        wait_and_barrier<2 * kGroupOps>();
        if (wave == 0 && t % kBatchTiles == kBatchTiles / 2 && (t / kBatchTiles + 1) * kBatchTiles < tiles)
            issue_batch(t / kBatchTiles + 1);
        if constexpr (kSafe) {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
            mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
            const bool was_started = started;
            const bool grow = was_started ? mx > kSlack : mx > -INFINITY;
            started = was_started || grow;
            if (__any(grow)) {
                const float shift = grow ? mx : 0.f;
                // l_run and O are still zero before the first move, so alpha is
                // left at 1 there (2^-mx could overflow for a very negative mx).
                const float alpha = was_started ? fast_exp2(-shift) : 1.f;
                m_run += shift;
                l_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o_acc[dt][r] *= alpha;
#pragma unroll
                for (int r = 0; r < 16; ++r) sc[r] -= shift;
            }
        }
        uint32_t pw[4][2];
        float psum = 0.f;
        bf16x8 va[8];
#pragma unroll
        for (int r = 0; r < 16; ++r) sn[r] = 0.f;
        __builtin_amdgcn_sched_barrier(0);
        // Phase A runs at wave priority 1, phase B at 0: when the SIMD's two
        // waves compete for issue, the one computing the next tile's logits
        // goes first (0.9 % faster at c2 than equal priorities; priority 3,
        // or raising it from the barrier on, was slower).
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            sn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ka[j]), bq[j], sn, 0, 0, 0);
            const float p0 = fast_exp2(sc[2 * j]), p1 = fast_exp2(sc[2 * j + 1]);
            psum = j == 0 ? p0 + p1 : (psum + p0) + p1;
            pw[j >> 1][j & 1] = pack_bf16(p0, p1);
            va[j] = read_v(t, j);
            if (j == 1) dma_k(t + 5, idk[0], 0);
            if (j == 3) dma_k(t + 5, idk[1], 1);
            if (j == 5) dma_v(t + 3, idv[0], 0);
            if (j == 7) dma_v(t + 3, idv[1], 1);
            if (j == 2) load_weights(t + 1, wn);
            __builtin_amdgcn_sched_barrier(0);
        }
        l_run += psum;
        float wm[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) wm[g] = wn[g] - m_run;
        if constexpr (kSafe) mx = -INFINITY;
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int ks = j >> 2;
            const u32x4 bw = {pw[2 * ks][0], pw[2 * ks][1], pw[2 * ks + 1][0], pw[2 * ks + 1][1]};
            o_acc[j & 3] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[j], __builtin_bit_cast(bf16x8, bw), o_acc[j & 3], 0, 0, 0);
            ka[j] = read_k(t + 2, j);
            const float y0 = __builtin_fmaf(sn[2 * j], scale_log2, wm[j >> 1]);
            const float y1 = __builtin_fmaf(sn[2 * j + 1], scale_log2, wm[j >> 1]);
            sn[2 * j] = y0;
            sn[2 * j + 1] = y1;
            mx = fmaxf(fmaxf(mx, y0), y1);  // one v_max3_f32
            if (j == 6) idk = load_ids(t + 6);
            if (j == 7) idv = load_ids(t + 4);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // One pass over the row's tiles. The fast pass returns whether the
    // workgroup must run the safe pass instead (its result is then
    // discarded): a query with no finite logit in the first tile, or a logit
    // above its reference by more than kFastRange.
    auto pass = [&](auto safe) -> bool {
        constexpr bool kSafe = decltype(safe)::value;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o_acc[dt][r] = 0.f;
        m_run = 0.f;
        l_run = 0.f;
        started = false;
        // Prologue: batch 0 of ids/weights (this also completes the Q loads);
        // K(0..3) and V(0..2); S(0) and K(1) into registers once K(0) and K(1)
        // are in; K(4) goes into K(0)'s stage only after every wave has read
        // it. The last eight transfers before step 0 are then K(3), V(1), V(2),
        // K(4), as step 0's wait expects.
        if (wave == 0) issue_batch(0);
        wait_and_barrier<0>();
        {
#pragma unroll
            for (int u = 0; u < 3; ++u) {
                const u32x2 ik = load_ids(u);
                dma_k(u, ik[0], 0);
                dma_k(u, ik[1], 1);
            }
            const u32x2 iv0 = load_ids(0);
            dma_v(0, iv0[0], 0);
            dma_v(0, iv0[1], 1);
            const u32x2 ik3 = load_ids(3);
            dma_k(3, ik3[0], 0);
            dma_k(3, ik3[1], 1);
            const u32x2 iv1 = load_ids(1), iv2 = load_ids(2);
            dma_v(1, iv1[0], 0);
            dma_v(1, iv1[1], 1);
            dma_v(2, iv2[0], 0);
            dma_v(2, iv2[1], 1);
        }
        const u32x2 ik4 = load_ids(4);
        u32x2 idk = load_ids(5), idv = load_ids(3);
        wait_and_barrier<10>();  // K(0), K(1) in; 10 newer transfers may be in flight
        f32x16 s0, s1;
        u32x4 ka[8];
        {
#pragma unroll
            for (int j = 0; j < 8; ++j) ka[j] = read_k(0, j);
#pragma unroll
            for (int r = 0; r < 16; ++r) s0[r] = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ka[j]), bq[j], s0, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 8; ++j) ka[j] = read_k(1, j);
        }
        wait_and_barrier<63>();  // every wave's reads of K(0) are done (no transfer wait)
        dma_k(4, ik4[0], 0);
        dma_k(4, ik4[1], 1);
        // Logits of S(0) (against reference 0).
        float w0[4], mx = -INFINITY;
        load_weights(0, w0);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s0[r] = __builtin_fmaf(s0[r], scale_log2, w0[r >> 2]);
            mx = fmaxf(mx, s0[r]);
        }
        if constexpr (!kSafe) {
            // The query's reference is the maximum of its first tile, over
            // both lane halves; a query without a finite logit there fails the
            // pass.
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
            mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
            started = mx > -INFINITY;
            m_run = started ? mx : 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) s0[r] -= m_run;
            mx = started ? -INFINITY : INFINITY;
        }
        // Four steps per iteration: t is a multiple of 4 there, so every ring
        // stage (u & 3) is a compile-time constant and the LDS addresses fold
        // into the instructions' offsets.
        int t = 0;
        for (; t + 3 < tiles; t += 4) {
            step(safe, t, s0, s1, mx, ka, w0, idk, idv);
            step(safe, t + 1, s1, s0, mx, ka, w0, idk, idv);
            step(safe, t + 2, s0, s1, mx, ka, w0, idk, idv);
            step(safe, t + 3, s1, s0, mx, ka, w0, idk, idv);
        }
        for (; t + 1 < tiles; t += 2) {
            step(safe, t, s0, s1, mx, ka, w0, idk, idv);
            step(safe, t + 1, s1, s0, mx, ka, w0, idk, idv);
        }
        if (t < tiles) step(safe, t, s0, s1, mx, ka, w0, idk, idv);
        // No transfer may still be landing when the workgroup's LDS is
        // released or the rings are refilled.
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
        if constexpr (kSafe) return false;
        // Workgroup vote: every wave publishes its flag, then all read all.
        const uint32_t bad = __any(mx > kFastRange) ? 1u : 0u;
        uint32_t* votes = reinterpret_cast<uint32_t*>(smem + kVoteOffset);
        if (lane == 0) votes[wave] = bad;
        wait_and_barrier<0>();
        const u32x4 all = *reinterpret_cast<const u32x4*>(votes);
        return (all[0] | all[1] | all[2] | all[3]) != 0u;
    };
    if (pass(std::false_type{})) pass(std::true_type{});

    const auto lsw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    const float l_tot = __uint_as_float(lsw[0]) + __uint_as_float(lsw[1]);
    if (valid_q) {
        // A query whose every listed block has weight -inf gets o = 0 and
        // lse = -inf.
        const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
        uint16_t* orow = out + (bh * n + qrow_index) * kHeadDim;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const u32x2 pk = {pack_bf16(o_acc[dt][4 * g] * inv, o_acc[dt][4 * g + 1] * inv),
                                  pack_bf16(o_acc[dt][4 * g + 2] * inv, o_acc[dt][4 * g + 3] * inv)};
                *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * g + 4 * half) = pk;
            }
        if (lse != nullptr && half == 0) lse[bh * n + qrow_index] = started ? m_run + log2f(l_tot) : -INFINITY;
    }
}

// Dense attention: every KV4 block of K/V in order (tile u holds blocks
// 8u .. 8u+7) at weight 0, blocks past the end at -inf, with no page list in
// memory. Every row of a head reads the same pages in the same order, so the
// gathers come from L2 and the MFMAs bound it; it runs on
// v_mfma_f32_16x16x32_bf16, which takes less energy per FLOP than the
// 32x32x16 form (the sparse kernel, bound by its gathers, keeps that one).
// Same rings, transfers, pipeline and two passes as prefill_kernel; the LDS
// holds the two rings and the votes (no page ids or weights).
//
// MFMA mapping (lane l = 16g + i, i < 16, g < 4): wave w owns queries
// 32w + 16j + i (j = 0, 1).
//   S^T = K Q^T : A = 16 keys x 32 dims (lane: key i, dims 8g..+7 of the
//                 k-step), B = 32 dims x 16 queries (lane: query i, the same
//                 dims); the lane gets keys 4g..4g+3 of each 16-key half kt of
//                 the tile for query i: one whole KV4 block, page 4kt + g.
//   O^T += V^T P^T: A = 16 dims x 32 keys, B = 32 keys x 16 queries; the
//                 MFMA k-index 8g + 4kt + r is key r of page 4kt + g on both
//                 operands, so P goes from the S^T accumulators to the B
//                 operand unmoved, and the A operand is two transposing reads
//                 (pages g and 4 + g).
// A query spans the four lanes i, 16 + i, 32 + i, 48 + i; its maximum and sum
// are combined over them with permlane swaps. V's dim blocks are placed by
// the page's parity (position m ^ (page & 1), through the transfer's source
// addresses): the four 16-lane groups of a transposing read fetch the same
// dim block of four different pages, which then fall in opposite halves of
// the banks.
__global__ __launch_bounds__(kPfThreads, 2) void dense_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    uint16_t* __restrict__ out, float* __restrict__ lse, int64_t n, int64_t n_kv, int64_t qb, int64_t rows, int fb,
    int samples, float scale_log2, int64_t slot_base) {
    extern __shared__ __align__(16) unsigned char smem[];
    RowSlot rs;
    if (!row_slot(slot_base, qb, rows, rs)) return;
    const int64_t bh = rs.bh, blk = rs.blk;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15, lg = lane >> 4;
    const int tiles = samples / kTilePages;
    auto token_of = [&](int j) { return blk * kQueryBlock + wave * 32 + 16 * j + li; };

    // Q as the B operand of S^T = K Q^T: query 16j + li, dims 32ks + 8lg .. +8.
    bf16x8 bq[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int64_t token = token_of(j);
        const uint16_t* qrow = q + (bh * n + min<int64_t>(token, n - 1)) * kHeadDim + 8 * lg;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            u32x4 val = {0u, 0u, 0u, 0u};
            if (token < n) val = *reinterpret_cast<const u32x4*>(qrow + 32 * ks);
            bq[j][ks] = __builtin_bit_cast(bf16x8, val);
        }
    }

    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8*)smem));
    const uint16_t* kbase = k + bh * n_kv * kHeadDim;
    const uint16_t* vbase = v + bh * n_kv * kHeadDim;

    // Transfers of this wave: pages 2w + e (e = 0, 1) of a K tile and of a V
    // tile. Source offsets inside a page (1 KiB = 4 keys x 256 B) for lane j:
    //   K: key r = j/16 at LDS chunk position j%16 holds chunk pos ^ (key & 15);
    //   V: 128-byte position P = j/8 holds dim block m = P ^ e, key (j/2)%4,
    //      dims 16m + 8(j%2).
    uint32_t k_src[2], v_src[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int r = lane >> 4, pos = lane & 15;
        const int key = 4 * (2 * wave + e) + r;
        k_src[e] = uint32_t(r * 16 + (pos ^ (key & 15))) * 16u;
        const int P = lane >> 3, sl = (lane >> 1) & 3, h = lane & 1;
        v_src[e] = uint32_t(sl * 256 + (2 * (P ^ e) + h) * 16);
    }
    // This wave's two pages of tile u, clamped into the head; tiles past the
    // row's end read its last tile (their transfers only keep the per-step
    // count uniform).
    auto load_ids = [&](int u) {
        const int id = min(u, tiles - 1) * kTilePages + 2 * wave;
        const u32x2 c = {uint32_t(min(id, fb - 1)), uint32_t(min(id + 1, fb - 1))};
        return c;
    };
    auto dma_k = [&](int u, uint32_t id, int e) {
        dma16(kbase, id * kPageBytes + k_src[e], lds0 + kKRing + (u & (kRing - 1)) * kTileBytes + (2 * wave + e) * kPageBytes);
    };
    auto dma_v = [&](int u, uint32_t id, int e) {
        dma16(vbase, id * kPageBytes + v_src[e], lds0 + kVRing + (u & (kRing - 1)) * kTileBytes + (2 * wave + e) * kPageBytes);
    };
    // The weights of this lane's keys in tile u: pages lg and 4 + lg, 0 inside
    // K/V and -inf past its end.
    auto load_weights = [&](int u, float (&wv)[2]) {
        const int uc = min(u, tiles - 1);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) wv[kt] = uc * kTilePages + 4 * kt + lg < fb ? 0.f : -INFINITY;
    };

    // Operand-read addresses of this lane, absolute in LDS, so every read is
    // one register plus the instruction's constant offset (ring stage, key
    // half, dim block). K (A of S^T): key 16kt + li, chunk 4ks + lg at
    // position chunk ^ li. V (A of O^T, transposing read): page lg (+4), dim
    // block dt at position dt ^ (lg & 1), key li/4, dims 4(li%4) .. +3, so
    // lane li receives dim 16dt + li of the page's four keys.
    uint32_t k_abs[4], v_abs[2];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) k_abs[ks] = lds0 + kKRing + li * 256 + 16 * ((4 * ks + lg) ^ li);
    {
        const int par = lg & 1, base = kVRing + lg * kPageBytes + 32 * (li >> 2) + 8 * (li & 3);
        v_abs[0] = lds0 + base + par * 128;  // even dt: position dt + par
        v_abs[1] = lds0 + base - par * 128;  // odd dt: position dt - par
    }
    auto read_k = [&](int u, int f) {  // f = 4kt + ks
        return *reinterpret_cast<const lds_u32x4*>(
            static_cast<uintptr_t>(k_abs[f & 3] + (u & (kRing - 1)) * kTileBytes + (f >> 2) * 4096));
    };
    auto read_v_half = [&](int u, int dt, int h) {
        const uint32_t a = v_abs[dt & 1] + (u & (kRing - 1)) * kTileBytes + dt * 128 + h * 4 * kPageBytes;
        return lds_read_tr16(a);
    };

    // O^T accumulators: o[dt][j] holds dims 16dt + 4lg .. +3 of query 16j + li.
    f32x4 o_acc[8][2];
    // Reference, running sum and state of query j. thr[j] is -inf until the
    // query's first finite logit, kSlack after.
    float m_run[2], l_run[2], thr[2];

    // Step t, as in prefill_kernel: phase A computes S(t+1) beside p = 2^y of
    // S(t) (sc[2kt + j]: key half kt, query j), the reads of V(t) and this
    // step's four transfers; phase B computes O += V(t)^T P(t)^T beside the
    // logits of S(t+1) and the reads of K(t+2). Fast pass: mx[0] is the
    // running maximum of every logit of the lane. Safe pass: mx[j] is the
    // maximum of query j over this lane's keys of S(t), and the reference
    // moves lazily (kSlack). Rings and transfer lead as in prefill_kernel.
    auto step = [&](auto safe, int t, f32x4 (&sc)[4], f32x4 (&sn)[4], float (&mx)[2], u32x4 (&ka)[8],
                    float (&wn)[2], u32x2& idk, u32x2& idv) {
        constexpr bool kSafe = decltype(safe)::value;
        wait_and_barrier<2 * kGroupOps>();
        if constexpr (kSafe) {
            max_over_rows(mx[0], mx[1]);
            const bool grow0 = mx[0] > thr[0], grow1 = mx[1] > thr[1];
            if (__any(grow0 || grow1)) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const bool grow = j ? grow1 : grow0;
                    const bool was_started = thr[j] == kSlack;
                    const float shift = grow ? mx[j] : 0.f;
                    // l_run and O are still zero before the first move, so alpha
                    // is left at 1 there (2^-mx could overflow for a very
                    // negative mx).
                    const float alpha = was_started ? fast_exp2(-shift) : 1.f;
                    thr[j] = grow ? kSlack : thr[j];
                    m_run[j] += shift;
                    l_run[j] *= alpha;
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) o_acc[dt][j][r] *= alpha;
#pragma unroll
                    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) sc[2 * kt + j][r] -= shift;
                }
            }
        }
        uint32_t pw[2][4];
        float psum[2], p_prev = 0.f;
        bf16x8 va[8];
        i16x4 v_lo = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) sn[c][r] = 0.f;
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int x = 0; x < 16; ++x) {
            const int ks = x >> 2, kt = (x >> 1) & 1, j = x & 1;
            sn[2 * kt + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[4 * kt + ks]),
                                                                     bq[j][ks], sn[2 * kt + j], 0, 0, 0);
            // p of element x of S(t): sc[c][r], c = x/4 = 2kt' + j', r = x%4.
            const int c = x >> 2, r = x & 3;
            const float p = fast_exp2(sc[c][r]);
            if (r == 0) psum[c & 1] = (c >> 1) == 0 ? p : psum[c & 1] + p;
            else psum[c & 1] += p;
            if (x & 1) pw[c & 1][2 * (c >> 1) + (r >> 1)] = pack_bf16(p_prev, p);
            p_prev = p;
            const i16x4 vh = read_v_half(t, x >> 1, x & 1);
            if (x & 1) va[x >> 1] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(v_lo, vh, 0, 1, 2, 3, 4, 5, 6, 7));
            else v_lo = vh;
            if (x == 2) dma_k(t + 5, idk[0], 0);
            if (x == 6) dma_k(t + 5, idk[1], 1);
            if (x == 10) dma_v(t + 3, idv[0], 0);
            if (x == 14) dma_v(t + 3, idv[1], 1);
            if (x == 4) load_weights(t + 1, wn);
            __builtin_amdgcn_sched_barrier(0);
        }
        l_run[0] += psum[0];
        l_run[1] += psum[1];
        float wm[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) wm[c] = wn[c >> 1] - m_run[c & 1];
        if constexpr (kSafe) {
            mx[0] = -INFINITY;
            mx[1] = -INFINITY;
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int x = 0; x < 16; ++x) {
            const int dt = x >> 1, j = x & 1;
            const u32x4 bw = {pw[j][0], pw[j][1], pw[j][2], pw[j][3]};
            o_acc[dt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], __builtin_bit_cast(bf16x8, bw), o_acc[dt][j], 0, 0, 0);
            // The K reads for the next step go out in the first half, so they
            // have landed by the next step's barrier (which waits for them).
            if (x < 8) ka[x] = read_k(t + 2, x);
            if (x & 1) {
                // Logits of elements x-1 and x of S(t+1): sn[c][r], c = x/4.
                const int c = x >> 2, r = x & 3;
                const float y0 = __builtin_fmaf(sn[c][r - 1], scale_log2, wm[c]);
                const float y1 = __builtin_fmaf(sn[c][r], scale_log2, wm[c]);
                sn[c][r - 1] = y0;
                sn[c][r] = y1;
                float& m = mx[kSafe ? (c & 1) : 0];
                m = fmaxf(fmaxf(m, y0), y1);  // one v_max3_f32
            }
            if (x == 12) idk = load_ids(t + 6);
            if (x == 14) idv = load_ids(t + 4);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // One pass over the row's tiles, as in prefill_kernel.
    auto pass = [&](auto safe) -> bool {
        constexpr bool kSafe = decltype(safe)::value;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) o_acc[dt][j][r] = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            m_run[j] = 0.f;
            l_run[j] = 0.f;
            thr[j] = -INFINITY;
        }
        // Prologue: K(0..3) and V(0..2); S(0) and K(1) into registers once
        // K(0) and K(1) are in; K(4) goes into K(0)'s stage only after every
        // wave has read it. The last eight transfers before step 0 are then
        // K(3), V(1), V(2), K(4), as step 0's wait expects.
        wait_and_barrier<0>();
        {
#pragma unroll
            for (int u = 0; u < 3; ++u) {
                const u32x2 ik = load_ids(u);
                dma_k(u, ik[0], 0);
                dma_k(u, ik[1], 1);
            }
            const u32x2 iv0 = load_ids(0);
            dma_v(0, iv0[0], 0);
            dma_v(0, iv0[1], 1);
            const u32x2 ik3 = load_ids(3);
            dma_k(3, ik3[0], 0);
            dma_k(3, ik3[1], 1);
            const u32x2 iv1 = load_ids(1), iv2 = load_ids(2);
            dma_v(1, iv1[0], 0);
            dma_v(1, iv1[1], 1);
            dma_v(2, iv2[0], 0);
            dma_v(2, iv2[1], 1);
        }
        const u32x2 ik4 = load_ids(4);
        u32x2 idk = load_ids(5), idv = load_ids(3);
        wait_and_barrier<10>();  // K(0), K(1) in; 10 newer transfers may be in flight
        f32x4 s0[4], s1[4];
        u32x4 ka[8];
        {
#pragma unroll
            for (int f = 0; f < 8; ++f) ka[f] = read_k(0, f);
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) s0[c][r] = 0.f;
#pragma unroll
            for (int x = 0; x < 16; ++x) {
                const int ks = x >> 2, kt = (x >> 1) & 1, j = x & 1;
                s0[2 * kt + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[4 * kt + ks]),
                                                                         bq[j][ks], s0[2 * kt + j], 0, 0, 0);
            }
#pragma unroll
            for (int f = 0; f < 8; ++f) ka[f] = read_k(1, f);
        }
        wait_and_barrier<63>();  // every wave's reads of K(0) are done (no transfer wait)
        dma_k(4, ik4[0], 0);
        dma_k(4, ik4[1], 1);
        // Logits of S(0) (against reference 0).
        float w0[2], mx[2] = {-INFINITY, -INFINITY};
        load_weights(0, w0);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s0[c][r] = __builtin_fmaf(s0[c][r], scale_log2, w0[c >> 1]);
                mx[c & 1] = fmaxf(mx[c & 1], s0[c][r]);
            }
        }
        if constexpr (!kSafe) {
            // Each query's reference is the maximum of its first tile, over its
            // four lanes; a query without a finite logit there fails the pass.
            max_over_rows(mx[0], mx[1]);
            bool all_started = true;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const bool started = mx[j] > -INFINITY;
                all_started = all_started && started;
                m_run[j] = started ? mx[j] : 0.f;
                thr[j] = started ? kSlack : -INFINITY;
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) s0[2 * kt + j][r] -= m_run[j];
            }
            mx[0] = all_started ? -INFINITY : INFINITY;
        }
        int t = 0;
        for (; t + 3 < tiles; t += 4) {
            step(safe, t, s0, s1, mx, ka, w0, idk, idv);
            step(safe, t + 1, s1, s0, mx, ka, w0, idk, idv);
            step(safe, t + 2, s0, s1, mx, ka, w0, idk, idv);
            step(safe, t + 3, s1, s0, mx, ka, w0, idk, idv);
        }
        for (; t + 1 < tiles; t += 2) {
            step(safe, t, s0, s1, mx, ka, w0, idk, idv);
            step(safe, t + 1, s1, s0, mx, ka, w0, idk, idv);
        }
        if (t < tiles) step(safe, t, s0, s1, mx, ka, w0, idk, idv);
        // No transfer may still be landing when the workgroup's LDS is
        // released or the rings are refilled.
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
        if constexpr (kSafe) return false;
        // Workgroup vote: every wave publishes its flag, then all read all.
        const uint32_t bad = __any(mx[0] > kFastRange) ? 1u : 0u;
        uint32_t* votes = reinterpret_cast<uint32_t*>(smem + kDenseVoteOffset);
        if (lane == 0) votes[wave] = bad;
        wait_and_barrier<0>();
        const u32x4 all = *reinterpret_cast<const u32x4*>(votes);
        return (all[0] | all[1] | all[2] | all[3]) != 0u;
    };
    if (pass(std::false_type{})) pass(std::true_type{});

#pragma unroll
    for (int j = 0; j < 2; ++j) {
        // Sum over the query's four lanes, in the same order in each of them.
        const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(l_run[j]), __float_as_uint(l_run[j]), false, false);
        const float l16 = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
        const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(l16), __float_as_uint(l16), false, false);
        const float l_tot = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
        const int64_t token = token_of(j);
        if (token < n) {
            // A query whose every block has weight -inf (none here while K/V
            // is not empty) gets o = 0 and lse = -inf.
            const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
            uint16_t* orow = out + (bh * n + token) * kHeadDim + 4 * lg;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
                const u32x2 pk = {pack_bf16(o_acc[dt][j][0] * inv, o_acc[dt][j][1] * inv),
                                  pack_bf16(o_acc[dt][j][2] * inv, o_acc[dt][j][3] * inv)};
                *reinterpret_cast<u32x2*>(orow + 16 * dt) = pk;
            }
            if (lse != nullptr && lg == 0) lse[bh * n + token] = thr[j] == kSlack ? m_run[j] + log2f(l_tot) : -INFINITY;
        }
    }
}

// Plan ids of a permuted token layout -> KV4 pages of the stored layout:
// out[i] = map[clamp(ids[i])], 4 ids per thread.
__global__ __launch_bounds__(256) void remap_ids_kernel(const int32_t* __restrict__ ids, int64_t count,
                                                        const int32_t* __restrict__ map, int map_len,
                                                        int32_t* __restrict__ out) {
    const int64_t i0 = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t i = i0 + e;
        if (i < count) out[i] = map[min(max(ids[i], 0), map_len - 1)];
    }
}

// Merge of two attention states over disjoint key sets (base-2 LSEs), as
// FlashInfer's merge_state: m = max(s_a, s_b), w = 2^(s - m),
// o = (o_a w_a + o_b w_b) / (w_a + w_b), s = m + log2(w_a + w_b), in fp32.
// One thread per 8 dims (16 bytes) of one query's 128-dim row.
__global__ __launch_bounds__(256) void merge_kernel(const uint16_t* __restrict__ oa, const float* __restrict__ sa,
                                                   const uint16_t* __restrict__ ob, const float* __restrict__ sb,
                                                   int64_t count, uint16_t* __restrict__ out,
                                                   float* __restrict__ s_out) {
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t row = idx >> 4, part = idx & 15;
    if (row >= count) return;
    const float a = sa[row], b = sb[row];
    const float m = fmaxf(a, b);
    const float wa = fast_exp2(a - m), wb = fast_exp2(b - m);
    const float d = wa + wb, inv = 1.0f / d;
    const u32x4 va = reinterpret_cast<const u32x4*>(oa + row * kHeadDim)[part];
    const u32x4 vb = reinterpret_cast<const u32x4*>(ob + row * kHeadDim)[part];
    u32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float lo = (bf16_lo(va[e]) * wa + bf16_lo(vb[e]) * wb) * inv;
        const float hi = (bf16_hi(va[e]) * wa + bf16_hi(vb[e]) * wb) * inv;
        r[e] = pack_bf16(lo, hi);
    }
    reinterpret_cast<u32x4*>(out + row * kHeadDim)[part] = r;
    if (s_out != nullptr && part == 0) s_out[row] = m + log2f(d);
}

}  // namespace

int launch_merge(const void* oa, const float* sa, const void* ob, const float* sb, int64_t count, void* out,
                 float* s_out, hipStream_t stream) {
    if (count == 0) return 0;
    const int64_t threads = count * 16;
    hipLaunchKernelGGL(merge_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(oa), sa, static_cast<const uint16_t*>(ob), sb, count,
                       static_cast<uint16_t*>(out), s_out);
    return check_launch("merge_kernel");
}

int launch_remap_ids(const int32_t* ids, int64_t count, const int32_t* map, int64_t map_len, int32_t* out,
                     hipStream_t stream) {
    if (count == 0) return 0;
    const int64_t threads = (count + 3) / 4;
    hipLaunchKernelGGL(remap_ids_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, stream, ids,
                       count, map, static_cast<int>(map_len), out);
    return check_launch("remap_ids_kernel");
}

// Row slots per XCD that one prefill launch covers (a whole number of
// generations of 64 slots): the rows of a call are split into launches of
// about kRowsPerLaunch rows each.
int64_t prefill_launch_slots(int64_t bh, int64_t n) {
    const int64_t qb = (n + kQueryBlock - 1) / kQueryBlock;
    const int64_t rows = bh * qb;
    const int64_t generations = ((qb + 7) / 8 * bh + 63) / 64;
    const int64_t launches = std::max<int64_t>(1, (rows + kRowsPerLaunch - 1) / kRowsPerLaunch);
    return (generations + launches - 1) / launches * 64;
}

int launch_prefill(const void* q, const void* k, const void* v, bool dense, int64_t bh, int64_t n, int64_t n_kv,
                   const int32_t* ids, const float* logw, int64_t samples, void* out, float* lse,
                   const int32_t* order, hipStream_t stream) {
    const int64_t qb = (n + kQueryBlock - 1) / kQueryBlock;
    const int64_t rows = bh * qb;
    if (samples % kTilePages != 0)
        return set_error(1, "prefill: samples (%lld) must be a multiple of %d", (long long)samples, kTilePages);
    if (!dense && ((reinterpret_cast<uintptr_t>(ids) & 15u) || (reinterpret_cast<uintptr_t>(logw) & 15u)))
        return set_error(1, "prefill: ids and log_weights must be 16-byte aligned");
    if (n_kv * kHeadDim * 2 > int64_t(0xffffffff))
        return set_error(1, "prefill: one head of K/V must be under 4 GiB");
    const float scale_log2 = static_cast<float>(1.4426950408889634 / 11.313708498984761);  // log2(e)/sqrt(128)
    const int64_t per_xcd = (qb + 7) / 8;
    if (rows == 0) return 0;
    const void* kernel = dense ? reinterpret_cast<const void*>(dense_kernel) : reinterpret_cast<const void*>(prefill_kernel);
    const int lds_bytes = dense ? kDenseLdsBytes : kLdsBytes;
    if (int rc = ensure_lds_limit(kernel, lds_bytes)) return rc;
    // The rows are launched in chunks of about kRowsPerLaunch, each a whole
    // number of generations (64 row slots per XCD; a generation is what the
    // chip holds at once, two workgroups per CU). The rows resident on an XCD
    // sweep their (ascending) page lists at the same pace only while they
    // started together; over a long launch their start times spread out, the
    // pages they touch at one moment spread over the whole head and the XCD's
    // L2 stops serving them. A new launch lines them up again (at c2, one
    // launch: 25.0 ms; five launches of whole heads: 23.9 ms, bit-identical),
    // and whole generations leave no half-empty generation in each launch.
    const int64_t slots = per_xcd * bh;                    // row slots per XCD
    const int64_t per_launch = prefill_launch_slots(bh, n);
    for (int64_t slot_base = 0; slot_base < slots; slot_base += per_launch) {
        const int64_t count = std::min(per_launch, slots - slot_base);
        const dim3 grid(static_cast<unsigned>(count * 8)), block(kPfThreads);
        const int fb = static_cast<int>(n_kv / kKvBlock), s = static_cast<int>(samples);
        if (dense) {
            hipLaunchKernelGGL(dense_kernel, grid, block, lds_bytes, stream, static_cast<const uint16_t*>(q),
                               static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                               static_cast<uint16_t*>(out), lse, n, n_kv, qb, rows, fb, s, scale_log2, slot_base);
            if (int rc = check_launch("dense_kernel")) return rc;
        } else {
            hipLaunchKernelGGL(prefill_kernel, grid, block, lds_bytes, stream, static_cast<const uint16_t*>(q),
                               static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), ids, logw,
                               static_cast<uint16_t*>(out), lse, n, n_kv, qb, rows, fb, s, scale_log2, order,
                               slot_base);
            if (int rc = check_launch("prefill_kernel")) return rc;
        }
    }
    return 0;
}

}  // namespace ab
