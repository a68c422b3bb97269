// ab_ibcs_sip_static: the fused plan (ab_ibcs_sip) for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc). The IBCS intermediates of ab_ibcs_sip's
// workspace live instead in `scratch`, a file-scope device array of
// kScratchBytes that each GPU this library runs on holds until the process
// ends. Heads are processed in chunks that fit it; one head must fit.
//
// This file is built into a library of its own, libab_attention_static.so,
// which links against libab_attention_hip.so. The array is part of this
// library's code object only, so a process that never loads this library
// never reserves it.
//
// The array's name is a host-side stand-in, not a device address: host code
// uses only the address hipGetSymbolAddress returns for the current device,
// resolved once per device on the first call there, after every argument
// check has passed. Every call on a GPU shares that GPU's array: calls that
// overlap on one GPU (other streams, other threads) race. No part of the
// scratch needs to start at zero: every kernel of the chain writes what the
// next one reads.
#include <algorithm>
#include <mutex>

#include "../../include/ab_attention.h"
#include "../../include/ab_attention_static.h"
#include "common.hpp"

namespace ab {
namespace {

constexpr size_t kScratchBytes = AB_STATIC_SCRATCH_BYTES;  // 512 MiB per GPU
constexpr int kMaxScratchDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The scratch array's address on the current device (nullptr and an error
// message on failure).
void* scratch_on_current_device() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxScratchDevices) {
        set_error(AB_ERR_LAUNCH, "ibcs_sip_static: no usable current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device] == nullptr) {
        void* ptr = nullptr;
        const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || ptr == nullptr) {
            set_error(AB_ERR_LAUNCH, "ibcs_sip_static: resolving the static scratch on device %d failed: %s", device,
                      hipGetErrorString(err));
            return nullptr;
        }
        g_scratch_ptr[device] = ptr;
    }
    return g_scratch_ptr[device];
}

}  // namespace
}  // namespace ab

using namespace ab;

extern "C" int ab_ibcs_sip_static(const void* q, const void* k, const int32_t* order, int64_t batch_heads,
                                  int64_t tokens, const float* offsets, int64_t samples, int32_t* ids,
                                  float* log_weights, void* stream) {
    // The checks of ab_ibcs_sip, then the scratch capacity, all before the
    // first runtime call.
    if (int rc = check_ibcs_sip_args("ibcs_sip_static", q, k, batch_heads, tokens, offsets, samples, ids,
                                     log_weights))
        return rc;
    const size_t one_head = ab_ibcs_sip_workspace_bytes(1, tokens);
    if (one_head == 0 || one_head > kScratchBytes)
        return set_error(AB_ERR_INVALID,
                         "ibcs_sip_static: one head of %lld tokens needs %zu bytes of scratch, more than the "
                         "%zu-byte static scratch (ab_ibcs_sip with a caller workspace takes heads of up to "
                         "131,072 tokens)",
                         (long long)tokens, one_head, kScratchBytes);
    int64_t chunk = std::min<int64_t>(batch_heads, int64_t(kScratchBytes / one_head));
    while (chunk > 1 && ab_ibcs_sip_workspace_bytes(chunk, tokens) > kScratchBytes) --chunk;
    void* ws = scratch_on_current_device();
    if (ws == nullptr) return AB_ERR_LAUNCH;
    const int64_t qb = (tokens + kQueryBlock - 1) / kQueryBlock;
    const size_t head_bytes = size_t(tokens) * kHeadDim * 2;
    for (int64_t h0 = 0; h0 < batch_heads; h0 += chunk) {
        const int64_t heads = std::min(chunk, batch_heads - h0);
        const int64_t row0 = h0 * qb;
        if (int rc = ab_ibcs_sip(static_cast<const char*>(q) + h0 * head_bytes,
                                 static_cast<const char*>(k) + h0 * head_bytes, order, heads, tokens, offsets + row0,
                                 samples, ws, kScratchBytes, ids + row0 * samples, log_weights + row0 * samples,
                                 stream))
            return rc;
    }
    return AB_OK;
}
