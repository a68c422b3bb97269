// Shared definitions for the gfx950 AB-Attention kernels.
//
// Geometry is fixed by the reference (csrc/ibcs.cu:32-36,
// ab_attention/flashinfer_backend.py:19-21): head dim 128, 128-query blocks,
// 4-key (KV4) blocks, 8 centroids per query block, 2 key representatives per
// KV4 block, 32 KV4 blocks per sample page.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ab {

constexpr int kHeadDim = 128;
constexpr int kQueryBlock = 128;
constexpr int kKvBlock = 4;
constexpr int kCentroids = 8;
constexpr int kReps = 2;
constexpr int kBlocksPerPage = 32;
constexpr int64_t kMaxKvBlocks = 32768;  // csrc/ibcs.cu:567-568

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_lo(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t bits) { return __uint_as_float(uint32_t(bits) << 16); }

// Round-to-nearest-even float -> bfloat16 bits (NaN kept quiet).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// Two floats -> packed bf16 pair with one v_cvt_pk_bf16_f32 (round to nearest
// even, the same rounding as f32_to_bf16 for every non-NaN input).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Hardware base-2 exponential and logarithm (v_exp_f32 / v_log_f32).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

__device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// (float)half - ref for the low (kHigh = false) or high half of a packed
// fp16 pair, in one v_fma_mix_f32: half * 1.0 + (-ref), rounded once. The
// conversion is exact, so this equals (float)half - ref rounded, in one
// instruction instead of a conversion and a subtraction.
template <bool kHigh>
__device__ __forceinline__ float f16_minus(uint32_t packed, float ref) {
    float r;
    if (kHigh)
        asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(packed), "v"(ref));
    else
        asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(packed), "v"(ref));
    return r;
}
// The same with a wave-uniform ref held in an SGPR (no copy to a VGPR).
template <bool kHigh>
__device__ __forceinline__ float f16_minus_uniform(uint32_t packed, float ref) {
    float r;
    if (kHigh)
        asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(packed), "s"(ref));
    else
        asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(packed), "s"(ref));
    return r;
}
#pragma clang diagnostic pop

// Workgroup barrier for LDS traffic only: waits for this wave's LDS accesses
// (lgkmcnt(0)) but leaves its outstanding global loads in flight. HIP's
// __syncthreads() also waits for every outstanding global load (vmcnt(0)),
// which would drain a prefetch issued before the barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
    asm volatile("s_barrier" ::: "memory");
}

}  // namespace ab

// Error reporting shared by every C-ABI entry point (api.hip).
namespace ab {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Raises the dynamic-LDS limit of kernel `fn` on the current device to at
// least `bytes`. The attribute is per device; each (kernel, device) pair is
// set once, so later launches (including launches recorded into a HIP graph)
// make no attribute call. Returns 0, or a nonzero status on failure.
int ensure_lds_limit(const void* fn, int bytes);
// Compute units of the current device (cached per device).
int device_cu_count();
// ab_ibcs_sip's argument checks except the workspace (shape, sample count,
// pointers, alignment); `what` prefixes the error message.
int check_ibcs_sip_args(const char* what, const void* q, const void* k, int64_t batch_heads, int64_t tokens,
                        const float* offsets, int64_t samples, const int32_t* ids, const float* log_weights);
}  // namespace ab
