// SIP on gfx950: inclusion probabilities pi = min(1, tau * m_j) with
// sum(pi) = S, certainty blocks first (ascending, weight 0), then Madow
// systematic draws with log2(1/pi) weights. One workgroup of 1,024 (or 512)
// threads per row, 256 of whose threads play the reference's CUB block.
//
// Bit-exact restatement of csrc/sip.cu:33-167. Every fp64 sum keeps the
// reference's association, which the reference gets from CUB:
//   - BlockReduce (WARP_REDUCTIONS): per 32-thread group a shfl_down tree with
//     offsets 1,2,4,8,16, then thread 0 folds the 8 group totals left to right;
//   - BlockScan (RAKING) exclusive sum: 32 raking threads fold 8 consecutive
//     partials, a 32-lane Kogge-Stone (shfl_up 1..16), shift by one lane, and
//     each segment rescanned from its prefix.
// A wave64 holds two of these 32-thread groups; shuffles use width 32.
// The walk's `mass += value * scale` is one fused multiply-add (as nvcc
// contracts it); every other product is rounded before its sum, which the
// build enforces with -ffp-contract=off.
//
// Workgroups have 1024 threads (16 waves) per row; the fused kernel gives
// rows small enough for two per CU 512-thread workgroups. The 256 "logical
// threads" that define CUB's association (threads 0..255) own the ordered
// folds and the chunk chains; the association-free phases (staging, marking,
// the last residual, the draws) use all the workgroup's threads, which keeps
// enough waves per SIMD to hide LDS and fp64 latency.
//
// Two storage schemes, same bits:
//   - sip_lds_kernel (rows whose masses and fp64 prefixes fit in LDS):
//     persistent workgroups walk rows r, r + grid, ...; while a row is
//     processed out of LDS, the next row's masses are loaded into registers,
//     and they are written to LDS as soon as the row's last draw has read it
//     (before the row's results are stored). Certainty is marked by the sign
//     bit of the LDS copy, as the reference negates its copy.
//   - sip_global_kernel (larger rows): one row per workgroup, the row is
//     re-read from L2 by each pass, LDS holds the prefixes and a certainty
//     bitmask.
// The fused plan (sip_fused_kernel, below) computes each row's masses into
// LDS from the pair-LSEs and samples it there; rows too large for the full
// prefix array keep a power-of-two number of prefixes per chunk
// (coarse_draws).
#include <algorithm>

#include "common.hpp"
#include "masses.hpp"

namespace ab {
namespace {

constexpr int kSipThreads = 256;   // logical threads of the reference's CUB blocks
constexpr int kSipWorkers = 1024;  // hardware threads per row
constexpr int kBucket = 4;
constexpr int kUnroll = 8;
constexpr int kDraws = 2;

// Row accessors. raw(i) is the stored value of mass i, x_of() turns it into
// the reference's clamped mass fmaxf(m, 1e-30f), certain_of() tells whether
// the element is certain, weight_mass(i) is fmax((double)m, 1e-30) for the
// log-weight. raw8(i0) fetches masses i0 .. i0+7 without bounds checks (the
// storage is padded; callers discard indices >= population).

// Masses held in LDS: negative and NaN masses are stored as +0 (the clamps
// above map them to the same values), so the sign bit is free to mark
// certainty, as the reference marks it by negating its copy.
struct LdsRow {
    float* values;  // 16-byte aligned, population + 8 entries
    __device__ __forceinline__ float raw(int i) const { return values[i]; }
    __device__ __forceinline__ void raw8(int i0, float (&r)[8]) const {  // i0 % 4 == 0
        const f32x4 a = *reinterpret_cast<const f32x4*>(values + i0);
        const f32x4 b = *reinterpret_cast<const f32x4*>(values + i0 + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            r[e] = a[e];
            r[e + 4] = b[e];
        }
    }
    // fmaxf(|r|, 1e-30f) on the bit patterns: both are non-negative, non-NaN.
    __device__ __forceinline__ static float x_of(float r) {
        return __uint_as_float(max(__float_as_uint(r) & 0x7fffffffu, __float_as_uint(1e-30f)));
    }
    // x_of for a row with no element marked: every stored value has its sign
    // bit clear, so the mask is not needed.
    __device__ __forceinline__ static float x_unmarked(float r) {
        return __uint_as_float(max(__float_as_uint(r), __float_as_uint(1e-30f)));
    }
    __device__ __forceinline__ bool certain_of(int, float r) const { return (__float_as_uint(r) >> 31) != 0u; }
    __device__ __forceinline__ float x(int i) const { return x_of(values[i]); }
    __device__ __forceinline__ bool certain(int i) const { return certain_of(i, values[i]); }
    __device__ __forceinline__ void mark(int i) { values[i] = -fabsf(values[i]); }
    __device__ __forceinline__ double weight_mass(int i) const {
        return fmax(static_cast<double>(fabsf(values[i])), 1e-30);
    }
    __device__ __forceinline__ void set_any_certain(bool) {}
};

// Raw masses in global memory, certainty in an LDS bitmask.
struct GlobalRow {
    const float* input;
    uint32_t* marks;
    bool any_certain;
    int last;  // population - 1
    __device__ __forceinline__ float raw(int i) const { return input[i]; }
    __device__ __forceinline__ void raw8(int i0, float (&r)[8]) const {
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = input[min(i0 + e, last)];
    }
    __device__ __forceinline__ static float x_of(float r) { return fmaxf(r, 1e-30f); }
    __device__ __forceinline__ static float x_unmarked(float r) { return x_of(r); }
    __device__ __forceinline__ bool certain_of(int i, float) const {
        return any_certain && ((marks[i >> 5] >> (i & 31)) & 1u);
    }
    __device__ __forceinline__ float x(int i) const { return x_of(input[i]); }
    __device__ __forceinline__ bool certain(int i) const { return certain_of(i, 0.f); }
    __device__ __forceinline__ void mark(int i) { atomicOr(&marks[i >> 5], 1u << (i & 31)); }
    __device__ __forceinline__ double weight_mass(int i) const { return fmax(static_cast<double>(input[i]), 1e-30); }
    __device__ __forceinline__ void set_any_certain(bool v) { any_certain = v; }
};

// LDS layout of the row kernels: fp64 bucket prefixes [buckets + 1], then
// (16-byte aligned) the masses or the certainty bitmask.
__host__ __device__ constexpr size_t sip_values_offset(int64_t buckets) {
    return (size_t(buckets + 1) * 8 + 15) / 16 * 16;
}

struct SipShared {
    double part[kSipThreads];
    double group_max[kSipThreads / 32];
    double scale;
    int added, pass, last;
    int wave_count[kSipThreads / 64];
    int exact;  // coarse prefixes: the row needs the reference's probe sequence
};

constexpr size_t kSipLdsLimit = 160 * 1024;

// LDS layout of the fused kernel for rows whose full prefix array does not
// fit: the masses (16-byte aligned), then the kept prefixes.
__host__ __device__ constexpr size_t sip_fused_coarse_offset(int64_t population) {
    return (size_t(population + 8) * 4 + 15) / 16 * 16;
}

// Prefixes each chunk keeps, its first (the scan value) included: the largest
// power of two (at most 32, a chunk's bucket count at the largest rows) that
// fits the LDS left after the masses, and at least 2.
__host__ __device__ constexpr int coarse_keep(int64_t population) {
    const size_t used = sizeof(SipShared) + sip_fused_coarse_offset(population);
    const size_t room = used < kSipLdsLimit ? (kSipLdsLimit - used) / (kSipThreads * sizeof(double)) : 0;
    int keep = 2;
    while (keep < 32 && size_t(2 * keep) <= room) keep *= 2;
    return keep;
}

// Thread-strided partial (sum, max) over the non-certain masses: thread t
// folds i = t, t+256, ... in order (sip.cu:63-71). The kUnroll loads of a
// step are issued together (clamped indices), then folded. With
// kNoCertain (the first pass, before any block is marked) steps that lie
// wholly inside the row need no per-element tests: every element is added.
template <bool kNoCertain, class R>
__device__ __forceinline__ void strided_partials(const R& rv, int pop, double& sum, double& mx) {
    const int t = threadIdx.x;
    sum = 0.0;
    // The maximum is order free: kept as the bit pattern of the largest
    // (positive) clamped mass, converted once at the end.
    uint32_t top = 0u;
    int i0 = t;
    if (kNoCertain) {
        for (; i0 + (kUnroll - 1) * kSipThreads < pop; i0 += kSipThreads * kUnroll) {
            float r[kUnroll];
#pragma unroll
            for (int e = 0; e < kUnroll; ++e) r[e] = rv.raw(i0 + e * kSipThreads);
#pragma unroll
            for (int e = 0; e < kUnroll; ++e) {
                const float x = R::x_unmarked(r[e]);
                sum = sum + static_cast<double>(x);
                top = max(top, __float_as_uint(x));
            }
        }
    }
    for (; i0 < pop; i0 += kSipThreads * kUnroll) {
        float r[kUnroll];
#pragma unroll
        for (int e = 0; e < kUnroll; ++e) r[e] = rv.raw(min(i0 + e * kSipThreads, pop - 1));
#pragma unroll
        for (int e = 0; e < kUnroll; ++e) {
            const int i = i0 + e * kSipThreads;
            const bool ok = i < pop && !rv.certain_of(i, r[e]);
            const float x = R::x_of(r[e]);
            sum = sum + (ok ? static_cast<double>(x) : 0.0);  // + 0.0 leaves a positive sum unchanged
            top = max(top, ok ? __float_as_uint(x) : 0u);
        }
    }
    mx = static_cast<double>(__uint_as_float(top));
}

// Bucket prefixes and draws from kept prefixes (the tail of sip_row for
// kCoarse). The reference's bucket prefixes (sip.cu:131-142) are one fp64
// chain per chunk of 4*cb blocks: prefix[b] = R (residual count) if bucket b
// starts past the last non-certain block, else the chain E[c] + the chunk's
// masses before bucket b, added in order. Each chunk keeps `keep` of them
// (coarse_keep: as many as the LDS holds after the masses, a power of two):
// its first (E[c] = sh.part[c] after the scan) and those at buckets
// c*cb + j*step, step = ceil(cb / keep); a slot whose bucket lies past the
// chunk holds the next chunk's first prefix. Any other prefix is the same
// chain continued from the nearest kept one, which gives the same bits.
// A draw with threshold th (sip.cu:144-166) needs the bucket the reference's
// binary search returns. Chains only grow, so the prefix array can fall only
// where a chunk's last prefix exceeds the next chunk's first (rounding of the
// scan against the chain) or where it drops to R (no threshold reaches R).
// If no threshold lies in such a drop at a chunk boundary, exactly one bucket
// b has prefix[b] <= th < prefix[b + 1], and the binary search returns it
// whatever its probes: the draw then finds it with a binary search over the
// kept prefixes and a walk of fewer than `step` buckets. Each chunk checks
// its boundary; a row where some threshold lands in a drop (sh.exact) makes
// the reference's probes instead, each prefix rebuilt from the kept ones.
template <int kWorkers, class R, class StageNext>
__device__ __forceinline__ void coarse_draws(R& rv, double* coarse, SipShared& sh, float offset_u,
                                             int32_t* __restrict__ out_ids, float* __restrict__ out_w, int pop,
                                             int residuals, int certainty, int last, double scale, int chunk,
                                             StageNext stage_next) {
    const int t = threadIdx.x;
    const int buckets = (pop + kBucket - 1) / kBucket;
    const int cb = chunk / kBucket;  // buckets per chunk
    const int keep = coarse_keep(pop);
    const int keep_log2 = __builtin_ctz(keep);
    const int step = (cb + keep - 1) / keep;  // buckets between kept prefixes
    const double rd = static_cast<double>(residuals);
    const double offset = static_cast<double>(offset_u);
    double* kept = coarse;  // [256][keep]: chunk c's prefixes at buckets c*cb + j*step
    auto chunk_end = [&](int c) { return min((c + 1) * cb, buckets); };
    // prefix[c * cb]: the chunk's scan value, or R past the last residual
    // (and for the terminal bucket).
    auto first_prefix = [&](int c) -> double {
        if (c >= kSipThreads || c * cb >= buckets || kBucket * (c * cb) > last) return rd;
        return sh.part[c];
    };
    // The chain over the 4 blocks of bucket b (sip.cu:137-140).
    auto add_bucket = [&](int b, double cum) -> double {
        float r[8];
        rv.raw8(b * kBucket, r);
#pragma unroll
        for (int e = 0; e < kBucket; ++e) {
            const int i = b * kBucket + e;
            const bool ok = i < pop && !rv.certain_of(i, r[e]);
            const double m = static_cast<double>(R::x_of(r[e])) * scale;
            cum = cum + (ok ? m : 0.0);
        }
        return cum;
    };

    // Kept prefixes: the same chain walk as the reference's prefix pass,
    // recording the prefix at every step-th bucket of the chunk.
    if (t < kSipThreads) {
        const int begin = t * chunk, end = min(begin + chunk, pop);
        double* mine = kept + t * keep;
        mine[0] = first_prefix(t);
        int slot = 1;          // kept prefixes of this chunk recorded so far
        int at = step;         // chunk-relative bucket of the next one
        double vlast = rd;     // the prefix at the chunk's last bucket
        if (begin < pop) {
            double cumulative = sh.part[t];
            int i0 = begin;
            if (certainty == 0) {
                for (; i0 + 8 <= end; i0 += 8) {
                    float r[8];
                    rv.raw8(i0, r);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        if (e % kBucket == 0) {
                            if ((i0 + e) / kBucket - t * cb == at) {
                                mine[slot++] = cumulative;
                                at += step;
                            }
                            vlast = cumulative;
                        }
                        cumulative = cumulative + static_cast<double>(R::x_unmarked(r[e])) * scale;
                    }
                }
            }
            for (; i0 < end; i0 += 8) {
                float r[8];
                rv.raw8(i0, r);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int i = i0 + e;
                    if (e % kBucket == 0 && i < end) {
                        const double v = i > last ? rd : cumulative;
                        if (i / kBucket - t * cb == at) {
                            mine[slot++] = v;
                            at += step;
                        }
                        vlast = v;
                    }
                    const bool ok = i < end && !rv.certain_of(i, r[e]);
                    const double m = static_cast<double>(R::x_of(r[e])) * scale;
                    cumulative = cumulative + (ok ? m : 0.0);
                }
            }
            // A drop at the boundary with the next chunk: does some threshold
            // offset + s (0 <= s < residuals, exact in fp64) lie in it?
            const double next = first_prefix(t + 1);
            if (vlast > next) {
                double s = ceil(next - offset);
                while (s > 0.0 && offset + (s - 1.0) >= next) s -= 1.0;
                while (offset + s < next) s += 1.0;
                s = fmax(s, 0.0);
                if (s < rd && offset + s < vlast && offset + s >= next) atomicOr(&sh.exact, 1);
            }
        }
        // Slots whose bucket lies past the chunk: the next chunk's first prefix.
        const double next_first = first_prefix(t + 1);
        for (; slot < keep; ++slot) mine[slot] = next_first;
    }
    lds_barrier();

    // Kept prefixes in bucket order: entry k is slot k % keep of chunk k / keep.
    auto kept_value = [&](int k) -> double { return kept[k]; };
    auto kept_bucket = [&](int k) -> int {
        if (k >= kSipThreads * keep) return buckets;
        const int c = k >> keep_log2, j = k & (keep - 1);
        return min(c * cb + j * step, chunk_end(c));
    };
    // prefix[b] rebuilt from the nearest kept prefix at or before it.
    auto prefix_at = [&](int b) -> double {
        if (b >= buckets || kBucket * b > last) return rd;
        const int c = b / cb, j = (b - c * cb) / step;
        double cum = kept[c * keep + j];
        for (int bb = c * cb + j * step; bb < b; ++bb) cum = add_bucket(bb, cum);
        return cum;
    };
    const bool exact = sh.exact != 0;
    const int per_round = kWorkers * kDraws;
    const int rounds = (residuals + per_round - 1) / per_round;
    for (int round = 0; round < rounds; ++round) {
        const int slot0 = t + round * per_round;
        double threshold[kDraws];
        int bucket[kDraws];
        double base[kDraws];
#pragma unroll
        for (int d = 0; d < kDraws; ++d) threshold[d] = offset + static_cast<double>(slot0 + d * kWorkers);
        if (!exact) {
            // Binary search over the kept prefixes, the draws in lockstep,
            // then each walks its segment to the crossing bucket.
            int lower[kDraws], upper[kDraws];
#pragma unroll
            for (int d = 0; d < kDraws; ++d) {
                lower[d] = 0;
                upper[d] = slot0 + d * kWorkers < residuals ? kSipThreads * keep - 1 : 0;
            }
            bool busy = true;
            while (busy) {
                busy = false;
#pragma unroll
                for (int d = 0; d < kDraws; ++d)
                    if (lower[d] < upper[d]) {
                        const int middle = (lower[d] + upper[d] + 1) / 2;
                        if (kept_value(middle) <= threshold[d]) lower[d] = middle;
                        else upper[d] = middle - 1;
                        busy = true;
                    }
            }
#pragma unroll
            for (int d = 0; d < kDraws; ++d) {
                int b = kept_bucket(lower[d]);
                double cum = kept_value(lower[d]);
                const int bend = kept_bucket(lower[d] + 1);
                while (b + 1 < bend) {
                    const double nxt = add_bucket(b, cum);
                    if ((kBucket * (b + 1) > last ? rd : nxt) > threshold[d]) break;
                    cum = nxt;
                    ++b;
                }
                bucket[d] = min(b, buckets - 1);
                base[d] = cum;
            }
        } else {
#pragma unroll
            for (int d = 0; d < kDraws; ++d) {
                int lower = 0, upper = slot0 + d * kWorkers < residuals ? buckets : 0;
                while (lower < upper) {
                    const int middle = (lower + upper + 1) / 2;
                    if (prefix_at(middle) <= threshold[d]) lower = middle;
                    else upper = middle - 1;
                }
                bucket[d] = min(lower, buckets - 1);
                base[d] = prefix_at(bucket[d]);
            }
        }
        int selected[kDraws];
        float weight[kDraws];
#pragma unroll
        for (int d = 0; d < kDraws; ++d) {
            double mass = base[d];
            int sel = last;
            float r[8];
            rv.raw8(bucket[d] * kBucket, r);
#pragma unroll
            for (int e = 0; e < kBucket; ++e) {
                const int i = bucket[d] * kBucket + e;
                if (i >= pop || rv.certain_of(i, r[e])) continue;
                sel = i;
                mass = fma(static_cast<double>(R::x_of(r[e])), scale, mass);
                if (mass > threshold[d]) break;
            }
            selected[d] = sel;
            weight[d] = static_cast<float>(-log2(rv.weight_mass(sel) * scale));
        }
        if (round + 1 == rounds) {
            lds_barrier();
            stage_next();
        }
#pragma unroll
        for (int d = 0; d < kDraws; ++d) {
            const int slot = slot0 + d * kWorkers;
            if (slot < residuals) {
                out_ids[certainty + slot] = selected[d];
                out_w[certainty + slot] = weight[d];
            }
        }
    }
    if (rounds == 0) {
        lds_barrier();
        stage_next();
    }
}

// Everything after the first pass's thread partials are known: certainty
// iteration, certain ids, chunk scan, bucket prefixes and the draws. Inlined:
// a called function starts by waiting for every outstanding memory access,
// which would stall on the next row's prefetch.
template <int kWorkers, bool kCoarse, class R, class StageNext>
__device__ __forceinline__ void sip_row(R& rv, double sum, double mx, double* prefix, SipShared& sh, float offset_u,
                                        int32_t* __restrict__ out_ids, float* __restrict__ out_w, int pop,
                                        int samples, StageNext stage_next, int exact_init = 0) {
    const int t = threadIdx.x;
    const bool logical = t < kSipThreads;
    const int buckets = (pop + kBucket - 1) / kBucket;

    // Certainty passes (sip.cu:62-96).
    int certainty = 0;
    double scale;
    for (int pass = 0;; ++pass) {
        if (logical) {
            if (pass > 0) strided_partials<false>(rv, pop, sum, mx);
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) {
                const double os = __shfl_down(sum, off, 32);
                const double om = __shfl_down(mx, off, 32);
                sum = sum + os;
                mx = fmax(mx, om);
            }
            if ((t & 31) == 0) {
                sh.part[t >> 5] = sum;
                sh.group_max[t >> 5] = mx;
            }
        }
        lds_barrier();
        if (t == 0) {
            double total = sh.part[0], maximum = sh.group_max[0];
            for (int w = 1; w < kSipThreads / 32; ++w) {
                total = total + sh.part[w];
                maximum = fmax(maximum, sh.group_max[w]);
            }
            const double sc = static_cast<double>(samples - certainty) / total;
            sh.scale = sc;
            sh.pass = maximum * sc >= 1.0;
            sh.added = 0;
        }
        lds_barrier();
        scale = sh.scale;
        if (sh.pass) {
            int count = 0;
            for (int i = t; i < pop; i += kWorkers)
                if (!rv.certain(i) && static_cast<double>(rv.x(i)) * scale >= 1.0) {
                    rv.mark(i);
                    ++count;
                }
            if (count) atomicAdd(&sh.added, count);
        }
        lds_barrier();
        const int added = sh.added;
        certainty += added;
        rv.set_any_certain(certainty != 0);
        lds_barrier();
        if (added == 0) break;
    }

    // Last residual (non-certain) index: the last element unless marked.
    int last = pop - 1;
    if (certainty != 0) {
        if (t == 0) sh.last = -1;
        lds_barrier();
        int mine = -1;
        for (int i = t; i < pop; i += kWorkers)
            if (!rv.certain(i)) mine = i;
        if (mine >= 0) atomicMax(&sh.last, mine);
        lds_barrier();
        last = sh.last;
    }

    const int chunk = ((buckets + kSipThreads - 1) / kSipThreads) * kBucket;  // sip.cu:99-101
    const int begin = t * chunk;
    const int end = logical ? min(begin + chunk, pop) : begin;

    // Certain ids first, ascending, weight 0 (sip.cu:108-124): chunk counts,
    // an exclusive scan over the 256 chunks (integer, order free), then
    // each chunk writes its certain ids in order.
    if (certainty != 0) {
        int count = 0;
        for (int i = begin; i < end; ++i) count += rv.certain(i);
        int inc = count;
        if (logical) {
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int o = __shfl_up(inc, off);
                if ((t & 63) >= off) inc += o;
            }
            if ((t & 63) == 63) sh.wave_count[t >> 6] = inc;
        }
        lds_barrier();
        if (logical) {
            int slot = inc - count;
            for (int w = 0; w < (t >> 6); ++w) slot += sh.wave_count[w];
            for (int i = begin; i < end; ++i)
                if (rv.certain(i)) {
                    out_ids[slot] = i;
                    out_w[slot++] = 0.f;
                }
        }
        lds_barrier();
    }

    // Chunk masses and their CUB-ordered exclusive scan (sip.cu:126-130).
    // A chunk starts at a multiple of 4; its masses are fetched 8 at a time.
    // Positions past the chunk and certain blocks add 0.0, which leaves the
    // (non-negative) running sum unchanged.
    // Without certain blocks, groups of 8 wholly inside the chunk add every
    // element (no tests).
    if (logical) {
        double chunk_mass = 0.0;
        int i0 = begin;
        if (certainty == 0) {
            for (; i0 + 8 <= end; i0 += 8) {
                float r[8];
                rv.raw8(i0, r);
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    chunk_mass = chunk_mass + static_cast<double>(R::x_unmarked(r[e])) * scale;
            }
        }
        for (; i0 < end; i0 += 8) {
            float r[8];
            rv.raw8(i0, r);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const bool ok = i0 + e < end && !rv.certain_of(i0 + e, r[e]);
                const double m = static_cast<double>(R::x_of(r[e])) * scale;
                chunk_mass = chunk_mass + (ok ? m : 0.0);
            }
        }
        sh.part[t] = chunk_mass;
    }
    if (kCoarse && t == 0) sh.exact = exact_init;
    lds_barrier();
    if (t < 32) {
        double seg = sh.part[8 * t];
#pragma unroll
        for (int i = 1; i < 8; ++i) seg = seg + sh.part[8 * t + i];
        double inc = seg;
#pragma unroll
        for (int off = 1; off < 32; off <<= 1) {
            const double o = __shfl_up(inc, off, 32);
            if (t >= off) inc = o + inc;
        }
        inc = 0.0 + inc;
        const double up = __shfl_up(inc, 1, 32);
        double ex = (t == 0) ? 0.0 : up;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const double in = sh.part[8 * t + i];
            sh.part[8 * t + i] = ex;
            ex = ex + in;
        }
    }
    lds_barrier();

    const int residuals = samples - certainty;
    if constexpr (kCoarse) {
        coarse_draws<kWorkers>(rv, prefix, sh, offset_u, out_ids, out_w, pop, residuals, certainty, last, scale,
                               chunk, stage_next);
        return;
    }

    // Bucket prefixes (sip.cu:131-142).
    if (t == 0) prefix[buckets] = static_cast<double>(residuals);
    if (logical) {
        double cumulative = sh.part[t];
        int i0 = begin;
        if (certainty == 0) {
            // No certain blocks: last = pop - 1, so no bucket start lies past
            // it, and every element of a whole group of 8 is added.
            for (; i0 + 8 <= end; i0 += 8) {
                float r[8];
                rv.raw8(i0, r);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (e % kBucket == 0) prefix[(i0 + e) / kBucket] = cumulative;
                    cumulative = cumulative + static_cast<double>(R::x_unmarked(r[e])) * scale;
                }
            }
        }
        for (; i0 < end; i0 += 8) {
            float r[8];
            rv.raw8(i0, r);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int i = i0 + e;
                if (e % kBucket == 0 && i < end)
                    prefix[i / kBucket] = i > last ? static_cast<double>(residuals) : cumulative;
                const bool ok = i < end && !rv.certain_of(i, r[e]);
                const double m = static_cast<double>(R::x_of(r[e])) * scale;
                cumulative = cumulative + (ok ? m : 0.0);
            }
        }
    }
    lds_barrier();

    // Systematic draws (sip.cu:144-166). Each thread runs up to kDraws
    // independent searches in lockstep (their LDS reads overlap); every search
    // makes exactly the reference's probes. The results of the last round are
    // stored only after stage_next() has refilled LDS with the next row (once
    // every thread is done reading this one), so that the next row's prefetch
    // never waits behind these stores.
    const double offset = static_cast<double>(offset_u);
    const int per_round = kWorkers * kDraws;
    const int rounds = (residuals + per_round - 1) / per_round;
    for (int round = 0; round < rounds; ++round) {
        const int slot0 = t + round * per_round;
        int lower[kDraws], upper[kDraws];
        double threshold[kDraws];
#pragma unroll
        for (int d = 0; d < kDraws; ++d) {
            const int slot = slot0 + d * kWorkers;
            threshold[d] = offset + static_cast<double>(slot);
            lower[d] = 0;
            upper[d] = slot < residuals ? buckets : 0;
        }
        bool busy = true;
        while (busy) {
            busy = false;
#pragma unroll
            for (int d = 0; d < kDraws; ++d)
                if (lower[d] < upper[d]) {
                    const int middle = (lower[d] + upper[d] + 1) / 2;
                    if (prefix[middle] <= threshold[d]) lower[d] = middle;
                    else upper[d] = middle - 1;
                    busy = true;
                }
        }
        int selected[kDraws];
        float weight[kDraws];
#pragma unroll
        for (int d = 0; d < kDraws; ++d) {
            const int bucket = min(lower[d], buckets - 1);
            double mass = prefix[bucket];
            int sel = last;
            float r[8];
            rv.raw8(bucket * kBucket, r);
#pragma unroll
            for (int e = 0; e < kBucket; ++e) {
                const int i = bucket * kBucket + e;
                if (i >= pop || rv.certain_of(i, r[e])) continue;
                sel = i;
                mass = fma(static_cast<double>(R::x_of(r[e])), scale, mass);
                if (mass > threshold[d]) break;
            }
            selected[d] = sel;
            weight[d] = static_cast<float>(-log2(rv.weight_mass(sel) * scale));
        }
        if (round + 1 == rounds) {
            lds_barrier();
            stage_next();
        }
#pragma unroll
        for (int d = 0; d < kDraws; ++d) {
            const int slot = slot0 + d * kWorkers;
            if (slot < residuals) {
                out_ids[certainty + slot] = selected[d];
                out_w[certainty + slot] = weight[d];
            }
        }
    }
    if (rounds == 0) {
        lds_barrier();
        stage_next();
    }
}

// Persistent kernel, row in LDS. Each of the 1024 threads prefetches up to
// kPer >= ceil(population / 1024) masses of the next row into registers.
template <int kPer>
__global__ __launch_bounds__(kSipWorkers) void sip_lds_kernel(
    const float* __restrict__ masses, const float* __restrict__ offsets, int32_t* __restrict__ ids,
    float* __restrict__ logw, int population, int samples, int64_t rows) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ SipShared sh;
    const int t = threadIdx.x;
    const int pop = population;
    const int buckets = (pop + kBucket - 1) / kBucket;
    double* prefix = reinterpret_cast<double*>(smem);
    float* values = reinterpret_cast<float*>(smem + sip_values_offset(buckets));

    float next[kPer];
    // Load k of a row reads element t + 1024k through a wave-uniform base
    // pointer, so no per-load offsets stay live across the row (spilled
    // offsets would be reloaded from scratch, and each reload's wait would
    // also wait for the prefetch loads already issued).
    auto prefetch = [&](int64_t r) {
        const float* in = masses + r * int64_t(pop);
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const float* base = in + k * kSipWorkers;
            next[k] = t + k * kSipWorkers < pop ? base[t] : 0.0f;
        }
    };
    auto stage = [&] {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int i = t + k * kSipWorkers;
            if (i < pop) values[i] = next[k] > 0.0f ? next[k] : 0.0f;  // NaN, negatives -> +0
        }
    };
    int64_t row = blockIdx.x;
    if (row < rows) {
        prefetch(row);
        stage();
    }
    for (; row < rows; row += gridDim.x) {
        const int64_t following = row + gridDim.x;
        if (following < rows) prefetch(following);
        lds_barrier();  // this row is staged
        LdsRow rv{values};
        double sum = 0.0, mx = 0.0;
        if (t < kSipThreads) strided_partials<true>(rv, pop, sum, mx);
        sip_row<kSipWorkers, false>(rv, sum, mx, prefix, sh, offsets[row], ids + row * int64_t(samples),
                                    logw + row * int64_t(samples), pop, samples, [&] {
                                        if (following < rows) stage();
                                    });
    }
}

// Fused masses + SIP for rows whose masses fit in LDS: each persistent
// workgroup computes its row's masses from the fp16 pair-LSEs [8, ld]
// straight into LDS (RowMasses: the arithmetic of masses_kernel, so the same
// bits as the scores that kernel writes), then samples the row as
// sip_lds_kernel does. The scores never go to global memory. A row's
// pair-LSEs are loaded two groups of 8 blocks per thread at a time (16 loads
// in flight).
// kCoarse = false: LDS holds the fp64 bucket prefixes and the masses (c2:
//   113 KB, one workgroup per CU).
// kCoarse = true, for rows whose full prefix array does not fit (c3's 29,700
//   blocks): LDS holds the masses and coarse_keep(pop) kept prefixes per
//   chunk (coarse_draws).
// Two 512-thread workgroups per CU with kept prefixes were tried at c2
// (81.9 KB each): 4.89 ms against 4.14 ms for this layout.
template <int kWorkers, bool kCoarse>
__global__ __launch_bounds__(kWorkers) void sip_fused_kernel(
    const _Float16* __restrict__ lse, const float* __restrict__ pops, const float* __restrict__ lse_max,
    const float* __restrict__ lse_den, int64_t ld, const float* __restrict__ offsets, int32_t* __restrict__ ids,
    float* __restrict__ logw, int population, int samples, int64_t rows, int force_exact) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ SipShared sh;
    const int t = threadIdx.x;
    const int pop = population;
    const int buckets = (pop + kBucket - 1) / kBucket;
    const int groups = (pop + 7) / 8;
    double* prefix = reinterpret_cast<double*>(kCoarse ? smem + sip_fused_coarse_offset(pop) : smem);
    float* values = reinterpret_cast<float*>(kCoarse ? smem : smem + sip_values_offset(buckets));
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        // The previous row's last reads of values[] finished before the
        // barrier ahead of its stores, so the row can be written over.
        RowMasses rm;
        rm.load(pops, lse_max, lse_den, row);
        const _Float16* src = lse + row * kCentroids * ld;
        for (int g0 = t; g0 < groups; g0 += 2 * kWorkers) {
            f16x8 h[2][kCentroids];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int g = min(g0 + u * kWorkers, groups - 1);
#pragma unroll
                for (int c = 0; c < kCentroids; ++c) h[u][c] = *reinterpret_cast<const f16x8*>(src + c * ld + 8 * g);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int g = g0 + u * kWorkers;
                if (g < groups) {
                    // Whole groups of 8: the masses of a last partial group
                    // past the population land in values[]' 8 padding
                    // entries, which no reader uses.
                    float m[8];
                    rm.eight(h[u], m);
                    f32x4 lo, hi;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        lo[e] = m[e] > 0.0f ? m[e] : 0.0f;  // NaN, negatives -> +0
                        hi[e] = m[e + 4] > 0.0f ? m[e + 4] : 0.0f;
                    }
                    *reinterpret_cast<f32x4*>(values + 8 * g) = lo;
                    *reinterpret_cast<f32x4*>(values + 8 * g + 4) = hi;
                }
            }
        }
        lds_barrier();
        LdsRow rv{values};
        double sum = 0.0, mx = 0.0;
        if (t < kSipThreads) strided_partials<true>(rv, pop, sum, mx);
        sip_row<kWorkers, kCoarse>(rv, sum, mx, prefix, sh, offsets[row], ids + row * int64_t(samples),
                                      logw + row * int64_t(samples), pop, samples, [] {}, force_exact);
    }
}

__global__ __launch_bounds__(kSipWorkers) void sip_global_kernel(
    const float* __restrict__ masses, const float* __restrict__ offsets, int32_t* __restrict__ ids,
    float* __restrict__ logw, int population, int samples) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ SipShared sh;
    const int t = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int pop = population;
    const int buckets = (pop + kBucket - 1) / kBucket;
    double* prefix = reinterpret_cast<double*>(smem);
    GlobalRow rv{masses + row * int64_t(pop), reinterpret_cast<uint32_t*>(prefix + buckets + 1), false, pop - 1};
    for (int w = t; w < (pop + 31) / 32; w += kSipWorkers) rv.marks[w] = 0u;
    lds_barrier();
    double sum = 0.0, mx = 0.0;
    if (t < kSipThreads) strided_partials<true>(rv, pop, sum, mx);
    sip_row<kSipWorkers, false>(rv, sum, mx, prefix, sh, offsets[row], ids + row * int64_t(samples),
                                logw + row * int64_t(samples), pop, samples, [] {});
}

template <int kPer>
int launch_lds(const float* scores, const float* offsets, int64_t rows, int pop, int samples, int32_t* ids,
               float* logw, size_t bytes, hipStream_t stream) {
    const void* fn = reinterpret_cast<const void*>(sip_lds_kernel<kPer>);
    if (int rc = ensure_lds_limit(fn, static_cast<int>(bytes))) return rc;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kSipWorkers, bytes) != hipSuccess || per_cu < 1)
        per_cu = 1;
    const int64_t grid = std::min<int64_t>(rows, int64_t(device_cu_count()) * per_cu);
    hipLaunchKernelGGL(sip_lds_kernel<kPer>, dim3(static_cast<unsigned>(grid)), dim3(kSipWorkers), bytes, stream,
                       scores, offsets, ids, logw, pop, samples, rows);
    return check_launch("sip_lds_kernel");
}

}  // namespace

constexpr size_t kSipStaticLds = sizeof(SipShared);
constexpr size_t kLdsLimit = kSipLdsLimit;

size_t sip_lds_bytes(int64_t population, bool lds_values) {
    const int64_t buckets = (population + kBucket - 1) / kBucket;
    const size_t base = sip_values_offset(buckets);
    return lds_values ? base + size_t(population + 8) * 4 : base + size_t((population + 31) / 32) * 4;
}

bool sip_fits(int64_t population) { return sip_lds_bytes(population, false) + kSipStaticLds <= kLdsLimit; }

// The fused kernel's LDS: the bucket prefixes and the masses, or (rows too
// large for that) the masses and coarse_keep kept prefixes per chunk.
size_t sip_fused_lds_bytes(int64_t population, bool coarse) {
    return coarse ? sip_fused_coarse_offset(population) + size_t(kSipThreads) * coarse_keep(population) *
                                                                 sizeof(double)
                  : sip_lds_bytes(population, true);
}

bool sip_fused_fits(int64_t population) {
    return sip_fused_lds_bytes(population, true) + kSipStaticLds <= kLdsLimit;
}
static_assert(sip_fused_coarse_offset(kMaxKvBlocks) + coarse_keep(kMaxKvBlocks) * kSipThreads * sizeof(double) +
                      kSipStaticLds <= kLdsLimit,
              "every row the API accepts fits the fused kernel's LDS");

namespace {

template <int kWorkers, bool kCoarse>
int launch_fused(const _Float16* lse, const float* pops, const float* lse_max, const float* lse_den, int64_t ld,
                 const float* offsets, int64_t rows, int pop, int samples, int32_t* ids, float* logw,
                 int force_exact, hipStream_t stream) {
    const size_t bytes = sip_fused_lds_bytes(pop, kCoarse);
    const void* fn = reinterpret_cast<const void*>(sip_fused_kernel<kWorkers, kCoarse>);
    if (int rc = ensure_lds_limit(fn, static_cast<int>(bytes))) return rc;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kWorkers, bytes) != hipSuccess || per_cu < 1)
        per_cu = 1;
    const int64_t grid = std::min<int64_t>(rows, int64_t(device_cu_count()) * per_cu);
    hipLaunchKernelGGL((sip_fused_kernel<kWorkers, kCoarse>), dim3(static_cast<unsigned>(grid)), dim3(kWorkers), bytes,
                       stream, lse, pops, lse_max, lse_den, ld, offsets, ids, logw, pop, samples, rows,
                       force_exact);
    return check_launch("sip_fused_kernel");
}

}  // namespace

// force_exact: every row sampled with kept prefixes takes the reference's
// probe sequence (the path otherwise used only when a threshold lands in a
// rounding drop of the prefix array, which tests cannot construct); the bits
// are the same either way.
int launch_sip_fused(const void* lse, const float* pops, const float* lse_max, const float* lse_den, int64_t ld,
                     const float* offsets, int64_t rows, int64_t population, int64_t samples, int32_t* ids,
                     float* logw, int force_exact, hipStream_t stream) {
    if (!sip_fused_fits(population))
        return set_error(1, "sip: population %lld does not fit the fused kernel's LDS", (long long)population);
    if (rows == 0) return 0;
    const _Float16* h = static_cast<const _Float16*>(lse);
    const int pop = static_cast<int>(population), s = static_cast<int>(samples);
    const size_t full = sip_fused_lds_bytes(population, false) + kSipStaticLds;
    // Rows small enough for two per CU (c1's 8,190 blocks: 49 KB) take
    // 512-thread workgroups: a CU then samples two rows at once, where one
    // 1,024-thread workgroup (16 waves x 93 VGPRs) would hold it alone.
    if (2 * full <= kLdsLimit)
        return launch_fused<kSipWorkers / 2, false>(h, pops, lse_max, lse_den, ld, offsets, rows, pop, s, ids, logw,
                                                    force_exact, stream);
    if (full <= kLdsLimit)
        return launch_fused<kSipWorkers, false>(h, pops, lse_max, lse_den, ld, offsets, rows, pop, s, ids, logw,
                                                force_exact, stream);
    return launch_fused<kSipWorkers, true>(h, pops, lse_max, lse_den, ld, offsets, rows, pop, s, ids, logw,
                                           force_exact, stream);
}

int launch_sip(const float* scores, const float* offsets, int64_t rows, int64_t population, int64_t samples,
               int32_t* ids, float* logw, hipStream_t stream) {
    if (!sip_fits(population))
        return set_error(1, "sip: population %lld exceeds single-workgroup LDS capacity", (long long)population);
    if (rows == 0) return 0;
    const int pop = static_cast<int>(population), s = static_cast<int>(samples);
    const size_t lds_bytes = sip_lds_bytes(population, true);
    const int per_thread = (pop + kSipWorkers - 1) / kSipWorkers;
    if (lds_bytes + kSipStaticLds <= kLdsLimit) {
        if (per_thread <= 4) return launch_lds<4>(scores, offsets, rows, pop, s, ids, logw, lds_bytes, stream);
        if (per_thread <= 8) return launch_lds<8>(scores, offsets, rows, pop, s, ids, logw, lds_bytes, stream);
        if (per_thread <= 16) return launch_lds<16>(scores, offsets, rows, pop, s, ids, logw, lds_bytes, stream);
        if (per_thread <= 24) return launch_lds<24>(scores, offsets, rows, pop, s, ids, logw, lds_bytes, stream);
    }
    const size_t bytes = sip_lds_bytes(population, false);
    if (int rc = ensure_lds_limit(reinterpret_cast<const void*>(sip_global_kernel), static_cast<int>(bytes)))
        return rc;
    hipLaunchKernelGGL(sip_global_kernel, dim3(static_cast<unsigned>(rows)), dim3(kSipWorkers), bytes, stream,
                       scores, offsets, ids, logw, pop, s);
    return check_launch("sip_global_kernel");
}

}  // namespace ab
