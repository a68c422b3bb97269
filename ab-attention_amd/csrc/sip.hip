// SIP on gfx950: inclusion probabilities pi = min(1, tau * m_j) with
// sum(pi) = S, certainty blocks first (ascending, weight 0), then Madow
// systematic draws with log2(1/pi) weights. One 256-thread workgroup per row.
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
// Row storage: when the row fits, the clamped masses live in LDS with the
// certainty mark in their sign (as the reference does); otherwise they are
// re-read from global memory and certainty is an LDS bitmask. Both give the
// same bits.
#include "common.hpp"

namespace ab {
namespace {

constexpr int kSipThreads = 256;
constexpr int kBucket = 4;

template <bool kLdsValues>
struct RowView {
    const float* input;
    float* values;      // LDS copy (kLdsValues)
    uint32_t* marks;    // LDS bitmask (!kLdsValues)

    __device__ __forceinline__ float x(int i) const {
        if constexpr (kLdsValues) return fabsf(values[i]);
        else return fmaxf(input[i], 1e-30f);
    }
    __device__ __forceinline__ bool certain(int i) const {
        if constexpr (kLdsValues) return values[i] < 0.f;
        else return (marks[i >> 5] >> (i & 31)) & 1u;
    }
    __device__ __forceinline__ void mark(int i) {
        if constexpr (kLdsValues) values[i] = -values[i];
        else atomicOr(&marks[i >> 5], 1u << (i & 31));
    }
};

template <bool kLdsValues>
__global__ __launch_bounds__(kSipThreads) void sip_kernel(
    const float* __restrict__ masses, const float* __restrict__ offsets,
    int32_t* __restrict__ ids, float* __restrict__ logw, int population, int samples) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ double part[kSipThreads];
    __shared__ double group_max[kSipThreads / 32];
    __shared__ double s_scale;
    __shared__ int s_new, s_pass, s_last;
    __shared__ int s_count[kSipThreads];

    const int t = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int pop = population;
    const int buckets = (pop + kBucket - 1) / kBucket;
    double* prefix = reinterpret_cast<double*>(smem);
    const int mask_words = (pop + 31) / 32;
    RowView<kLdsValues> rv;
    rv.input = masses + row * int64_t(pop);
    rv.marks = reinterpret_cast<uint32_t*>(prefix + buckets + 1);
    rv.values = reinterpret_cast<float*>(rv.marks + mask_words);

    if constexpr (kLdsValues) {
        for (int i = t; i < pop; i += kSipThreads) rv.values[i] = fmaxf(rv.input[i], 1e-30f);
    } else {
        for (int w = t; w < mask_words; w += kSipThreads) rv.marks[w] = 0u;
    }
    __syncthreads();

    // Certainty passes (sip.cu:62-96).
    int certainty = 0;
    double scale;
    for (;;) {
        double sum = 0.0, mx = 0.0;
        for (int i = t; i < pop; i += kSipThreads)
            if (!rv.certain(i)) {
                const double v = static_cast<double>(rv.x(i));
                sum = sum + v;
                mx = fmax(mx, v);
            }
#pragma unroll
        for (int off = 1; off < 32; off <<= 1) {
            const double os = __shfl_down(sum, off, 32);
            const double om = __shfl_down(mx, off, 32);
            sum = sum + os;
            mx = fmax(mx, om);
        }
        if ((t & 31) == 0) {
            part[t >> 5] = sum;
            group_max[t >> 5] = mx;
        }
        __syncthreads();
        if (t == 0) {
            double total = part[0], maximum = group_max[0];
            for (int w = 1; w < kSipThreads / 32; ++w) {
                total = total + part[w];
                maximum = fmax(maximum, group_max[w]);
            }
            const double sc = static_cast<double>(samples - certainty) / total;
            s_scale = sc;
            s_pass = maximum * sc >= 1.0;
            s_new = 0;
        }
        __syncthreads();
        scale = s_scale;
        if (s_pass) {
            int count = 0;
            for (int i = t; i < pop; i += kSipThreads)
                if (!rv.certain(i) && static_cast<double>(rv.x(i)) * scale >= 1.0) {
                    rv.mark(i);
                    ++count;
                }
            if (count) atomicAdd(&s_new, count);
        }
        __syncthreads();
        const int added = s_new;
        certainty += added;
        __syncthreads();
        if (added == 0) break;
    }

    // Last residual (non-certain) index; a max is order independent.
    if (t == 0) s_last = -1;
    __syncthreads();
    {
        int last = -1;
        for (int i = t; i < pop; i += kSipThreads)
            if (!rv.certain(i)) last = i;
        if (last >= 0) atomicMax(&s_last, last);
    }
    __syncthreads();
    const int last = s_last;

    const int chunk = ((buckets + kSipThreads - 1) / kSipThreads) * kBucket;  // sip.cu:99-101
    const int begin = t * chunk;
    const int end = min(begin + chunk, pop);
    int32_t* out_ids = ids + row * int64_t(samples);
    float* out_w = logw + row * int64_t(samples);

    // Certain ids first, ascending, weight 0 (sip.cu:108-124).
    if (certainty != 0) {
        int count = 0;
        for (int i = begin; i < end; ++i) count += rv.certain(i);
        s_count[t] = count;
        __syncthreads();
        int slot = 0;
        for (int u = 0; u < t; ++u) slot += s_count[u];
        for (int i = begin; i < end; ++i)
            if (rv.certain(i)) {
                out_ids[slot] = i;
                out_w[slot++] = 0.f;
            }
        __syncthreads();
    }

    // Chunk masses and their CUB-ordered exclusive scan (sip.cu:126-130).
    double chunk_mass = 0.0;
    for (int i = begin; i < end; ++i)
        chunk_mass = chunk_mass + (rv.certain(i) ? 0.0 : static_cast<double>(rv.x(i)) * scale);
    part[t] = chunk_mass;
    __syncthreads();
    if (t < 32) {
        double seg = part[8 * t];
#pragma unroll
        for (int i = 1; i < 8; ++i) seg = seg + part[8 * t + i];
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
            const double in = part[8 * t + i];
            part[8 * t + i] = ex;
            ex = ex + in;
        }
    }
    __syncthreads();
    double cumulative = part[t];

    // Bucket prefixes (sip.cu:131-142).
    const int residuals = samples - certainty;
    if (t == 0) prefix[buckets] = static_cast<double>(residuals);
    for (int i = begin; i < end; ++i) {
        if (i % kBucket == 0) prefix[i / kBucket] = i > last ? static_cast<double>(residuals) : cumulative;
        cumulative = cumulative + (rv.certain(i) ? 0.0 : static_cast<double>(rv.x(i)) * scale);
    }
    __syncthreads();

    // Systematic draws (sip.cu:144-166).
    const double offset = static_cast<double>(offsets[row]);
    for (int slot = t; slot < residuals; slot += kSipThreads) {
        const double threshold = offset + static_cast<double>(slot);
        int lower = 0, upper = buckets;
        while (lower < upper) {
            const int middle = (lower + upper + 1) / 2;
            if (prefix[middle] <= threshold) lower = middle;
            else upper = middle - 1;
        }
        const int bucket = min(lower, buckets - 1);
        double mass = prefix[bucket];
        int selected = last;
        const int stop = min((bucket + 1) * kBucket, pop);
        for (int i = bucket * kBucket; i < stop; ++i) {
            if (rv.certain(i)) continue;
            selected = i;
            mass = fma(static_cast<double>(rv.x(i)), scale, mass);
            if (mass > threshold) break;
        }
        out_ids[certainty + slot] = selected;
        out_w[certainty + slot] =
            static_cast<float>(-log2(fmax(static_cast<double>(rv.input[selected]), 1e-30) * scale));
    }
}

}  // namespace

size_t sip_lds_bytes(int64_t population, bool lds_values) {
    const int64_t buckets = (population + kBucket - 1) / kBucket;
    const int64_t words = (population + 31) / 32;
    size_t bytes = size_t(buckets + 1) * 8 + size_t(words) * 4;
    if (lds_values) bytes += size_t(population) * 4;
    return bytes;
}

// Static LDS of sip_kernel: part (2 KiB) + group_max + scalars + s_count (1 KiB).
constexpr size_t kSipStaticLds = kSipThreads * 8 + 8 * 8 + 8 + 12 + kSipThreads * 4;
constexpr size_t kLdsLimit = 160 * 1024;

bool sip_fits(int64_t population) { return sip_lds_bytes(population, false) + kSipStaticLds <= kLdsLimit; }

int launch_sip(const float* scores, const float* offsets, int64_t rows, int64_t population, int64_t samples,
               int32_t* ids, float* logw, hipStream_t stream) {
    const bool lds_values = sip_lds_bytes(population, true) + kSipStaticLds <= kLdsLimit;
    const size_t bytes = sip_lds_bytes(population, lds_values);
    if (bytes + kSipStaticLds > kLdsLimit)
        return set_error(1, "sip: population %lld exceeds single-workgroup LDS capacity", (long long)population);
    const void* fn = lds_values ? reinterpret_cast<const void*>(sip_kernel<true>)
                                : reinterpret_cast<const void*>(sip_kernel<false>);
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (rows == 0) return 0;
    if (lds_values)
        hipLaunchKernelGGL(sip_kernel<true>, dim3(static_cast<unsigned>(rows)), dim3(kSipThreads), bytes, stream,
                           scores, offsets, ids, logw, static_cast<int>(population), static_cast<int>(samples));
    else
        hipLaunchKernelGGL(sip_kernel<false>, dim3(static_cast<unsigned>(rows)), dim3(kSipThreads), bytes, stream,
                           scores, offsets, ids, logw, static_cast<int>(population), static_cast<int>(samples));
    return check_launch("sip_kernel");
}

}  // namespace ab
