// C-ABI of the gfx950 AB-Attention library (declared in include/ab_attention.h).
//
// Every entry point validates its sizes before any launch, enqueues on the
// caller's stream, never synchronises and never allocates: buffers, including
// workspace, belong to the caller. Failures return a nonzero status and leave
// a message for ab_last_error().
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <map>
#include <mutex>
#include <utility>

#include "../../include/ab_attention.h"
#include "common.hpp"

namespace ab {

int64_t lse_stride(int64_t fb);
int launch_cluster_pool(const void* q, const void* k, int64_t bh, int64_t n, void* centroids, float* pops,
                        void* pooled, float qk_scale_log2, const int32_t* order, hipStream_t stream);
int launch_lse(const void* centroids, const void* pooled, int64_t bh, int64_t n, void* lse, float* lse_max,
               float* lse_den, hipStream_t stream);
int launch_masses(const void* lse, const float* pops, const float* lse_max, const float* lse_den, int64_t rows,
                  int64_t fb, float* scores, hipStream_t stream);
int launch_sip(const float* scores, const float* offsets, int64_t rows, int64_t population, int64_t samples,
               int32_t* ids, float* logw, hipStream_t stream);
bool sip_fits(int64_t population);
bool sip_fused_fits(int64_t population);
int launch_sip_fused(const void* lse, const float* pops, const float* lse_max, const float* lse_den, int64_t ld,
                     const float* offsets, int64_t rows, int64_t population, int64_t samples, int32_t* ids,
                     float* logw, int force_exact, hipStream_t stream);
int launch_prefill(const void* q, const void* k, const void* v, bool dense, int64_t bh, int64_t n, int64_t n_kv,
                   const int32_t* ids, const float* logw, int64_t samples, void* out, float* lse,
                   const int32_t* order, hipStream_t stream);
int64_t prefill_launch_slots(int64_t bh, int64_t n);
int launch_remap_ids(const int32_t* ids, int64_t count, const int32_t* map, int64_t map_len, int32_t* out,
                     hipStream_t stream);
int launch_merge(const void* oa, const float* sa, const void* ob, const float* sb, int64_t count, void* out,
                 float* s_out, hipStream_t stream);

namespace {
thread_local char g_error[512] = "";

// float(128^-0.5 * log2(e)) as computed by the reference host code
// (csrc/ibcs.cu:601-602).
float qk_scale_log2() { return static_cast<float>(std::pow(128.0, -0.5) * 1.4426950408889634); }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct IbcsLayout {
    int64_t qb, fb, rows, ld;
    size_t centroids, pops, pooled, lse, lse_max, lse_den, total;
};

IbcsLayout ibcs_layout(int64_t bh, int64_t n) {
    IbcsLayout L;
    L.qb = (n + kQueryBlock - 1) / kQueryBlock;
    L.fb = n / kKvBlock;
    L.rows = bh * L.qb;
    L.ld = lse_stride(L.fb);
    size_t off = 0;
    L.centroids = off;
    off = align256(off + size_t(L.rows) * kCentroids * kHeadDim * 2);
    L.pops = off;
    off = align256(off + size_t(L.rows) * kCentroids * 4);
    L.pooled = off;
    off = align256(off + size_t(bh) * L.fb * kReps * kHeadDim * 2);
    L.lse = off;
    off = align256(off + size_t(L.rows) * kCentroids * L.ld * 2);
    L.lse_max = off;
    off = align256(off + size_t(L.rows) * kCentroids * 4);
    L.lse_den = off;
    off = align256(off + size_t(L.rows) * kCentroids * 4);
    L.total = off;
    return L;
}

int check_qk_shape(const char* what, int64_t bh, int64_t n) {
    if (bh <= 0 || n <= 0) return set_error(AB_ERR_INVALID, "%s: batch_heads and tokens must be positive", what);
    if (n % kKvBlock) return set_error(AB_ERR_INVALID, "%s: sequence length must be divisible by 4", what);
    if (n / kKvBlock > kMaxKvBlocks)
        return set_error(AB_ERR_INVALID, "%s: KV4 block count must be in [1, 32768]", what);
    const int64_t qb = (n + kQueryBlock - 1) / kQueryBlock;
    if (qb > 65535 || bh > 65535) return set_error(AB_ERR_INVALID, "%s: grid too large", what);
    return AB_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
}  // namespace

int set_error(int code, const char* fmt, ...) {
    va_list args;
    va_start(args, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, args);
    va_end(args);
    return code;
}

int check_launch(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_error(AB_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(err));
    return AB_OK;
}

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_attr_mutex;
std::map<std::pair<const void*, int>, int> g_lds_limit;  // (kernel, device) -> bytes set
std::atomic<int> g_cu_count[kMaxDevices];
}  // namespace

int ensure_lds_limit(const void* fn, int bytes) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return set_error(AB_ERR_LAUNCH, "no current HIP device");
    std::lock_guard<std::mutex> lock(g_attr_mutex);
    int& done = g_lds_limit[{fn, device}];
    if (done >= bytes) return AB_OK;
    const hipError_t err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (err != hipSuccess)
        return set_error(AB_ERR_LAUNCH, "setting a %d-byte LDS limit failed: %s", bytes, hipGetErrorString(err));
    done = bytes;
    return AB_OK;
}

int device_cu_count() {
    int device = 0;
    (void)hipGetDevice(&device);
    if (device < 0 || device >= kMaxDevices) device = 0;
    int cus = g_cu_count[device].load(std::memory_order_relaxed);
    if (cus == 0) {
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        cus = std::max(cus, 1);
        g_cu_count[device].store(cus, std::memory_order_relaxed);
    }
    return cus;
}

}  // namespace ab

using namespace ab;

extern "C" {

const char* ab_last_error(void) { return g_error; }

int ab_abi_version(void) { return AB_ABI_VERSION; }

int64_t ab_ibcs_lse_stride(int64_t tokens) { return lse_stride(tokens / kKvBlock); }

size_t ab_ibcs_workspace_bytes(int64_t batch_heads, int64_t tokens) {
    if (batch_heads <= 0 || tokens <= 0) return 0;
    return ibcs_layout(batch_heads, tokens).total;
}

int ab_ibcs_cluster_pool(const void* q, const void* k, int64_t batch_heads, int64_t tokens, void* centroids,
                         float* populations, void* pooled_keys, void* stream) {
    if (int rc = check_qk_shape("ibcs", batch_heads, tokens)) return rc;
    if (!q || !k || !centroids || !populations || !pooled_keys)
        return set_error(AB_ERR_INVALID, "ibcs: null pointer");
    if (!aligned16(q) || !aligned16(k) || !aligned16(pooled_keys))
        return set_error(AB_ERR_INVALID, "ibcs: q, k and pooled keys must be 16-byte aligned");
    return launch_cluster_pool(q, k, batch_heads, tokens, centroids, populations, pooled_keys, qk_scale_log2(),
                               nullptr, static_cast<hipStream_t>(stream));
}

int ab_ibcs_lse(const void* centroids, const void* pooled_keys, int64_t batch_heads, int64_t tokens,
                void* block_lse, float* lse_max, float* lse_den, void* stream) {
    if (int rc = check_qk_shape("ibcs", batch_heads, tokens)) return rc;
    if (!centroids || !pooled_keys || !block_lse || !lse_max || !lse_den)
        return set_error(AB_ERR_INVALID, "ibcs: null pointer");
    if (!aligned16(centroids) || !aligned16(pooled_keys) || !aligned16(block_lse))
        return set_error(AB_ERR_INVALID, "ibcs: centroids, pooled keys and block LSE must be 16-byte aligned");
    return launch_lse(centroids, pooled_keys, batch_heads, tokens, block_lse, lse_max, lse_den,
                      static_cast<hipStream_t>(stream));
}

int ab_ibcs_masses(const void* block_lse, const float* populations, const float* lse_max, const float* lse_den,
                   int64_t rows, int64_t kv_blocks, float* scores, void* stream) {
    if (rows < 0 || kv_blocks <= 0 || kv_blocks > kMaxKvBlocks)
        return set_error(AB_ERR_INVALID, "ibcs: bad masses shape");
    if (!block_lse || !populations || !lse_max || !lse_den || !scores)
        return set_error(AB_ERR_INVALID, "ibcs: null pointer");
    if (!aligned16(block_lse)) return set_error(AB_ERR_INVALID, "ibcs: block LSE must be 16-byte aligned");
    if (rows == 0) return AB_OK;
    return launch_masses(block_lse, populations, lse_max, lse_den, rows, kv_blocks, scores,
                         static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {
// The whole IBCS chain, with the query/key tokens read through `order`
// (nullptr: the stored order).
int ibcs_chain(const void* q, const void* k, const int32_t* order, int64_t batch_heads, int64_t tokens,
               void* workspace, size_t workspace_bytes, float* scores, void* stream) {
    if (int rc = check_qk_shape("ibcs", batch_heads, tokens)) return rc;
    if (!q || !k || !workspace || !scores) return set_error(AB_ERR_INVALID, "ibcs: null pointer");
    if (!aligned16(q) || !aligned16(k)) return set_error(AB_ERR_INVALID, "ibcs: q and k must be 16-byte aligned");
    const IbcsLayout L = ibcs_layout(batch_heads, tokens);
    if (workspace_bytes < L.total)
        return set_error(AB_ERR_INVALID, "ibcs: workspace of %zu bytes is smaller than the %zu required",
                         workspace_bytes, L.total);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
        return set_error(AB_ERR_INVALID, "ibcs: workspace must be 256-byte aligned");
    char* ws = static_cast<char*>(workspace);
    if (int rc = launch_cluster_pool(q, k, batch_heads, tokens, ws + L.centroids,
                                     reinterpret_cast<float*>(ws + L.pops), ws + L.pooled, qk_scale_log2(), order,
                                     static_cast<hipStream_t>(stream)))
        return rc;
    if (int rc = ab_ibcs_lse(ws + L.centroids, ws + L.pooled, batch_heads, tokens, ws + L.lse,
                             reinterpret_cast<float*>(ws + L.lse_max), reinterpret_cast<float*>(ws + L.lse_den),
                             stream))
        return rc;
    return ab_ibcs_masses(ws + L.lse, reinterpret_cast<const float*>(ws + L.pops),
                          reinterpret_cast<const float*>(ws + L.lse_max),
                          reinterpret_cast<const float*>(ws + L.lse_den), L.rows, L.fb, scores, stream);
}
}  // namespace

extern "C" {

int ab_ibcs(const void* q, const void* k, int64_t batch_heads, int64_t tokens, void* workspace,
            size_t workspace_bytes, float* scores, void* stream) {
    return ibcs_chain(q, k, nullptr, batch_heads, tokens, workspace, workspace_bytes, scores, stream);
}

int ab_ibcs_ordered(const void* q, const void* k, const int32_t* order, int64_t batch_heads, int64_t tokens,
                    void* workspace, size_t workspace_bytes, float* scores, void* stream) {
    if (!order) return set_error(AB_ERR_INVALID, "ibcs: null token order");
    return ibcs_chain(q, k, order, batch_heads, tokens, workspace, workspace_bytes, scores, stream);
}

size_t ab_ibcs_sip_workspace_bytes(int64_t batch_heads, int64_t tokens) {
    if (batch_heads <= 0 || tokens <= 0 || tokens % kKvBlock) return 0;
    // The fused kernel samples every row in LDS (rows of up to 32,768 blocks
    // fit), so the workspace holds only the IBCS intermediates.
    return ibcs_layout(batch_heads, tokens).total;
}

}  // extern "C"

namespace ab {
// Every check of ab_ibcs_sip except the workspace's: shape, sample count,
// pointers and alignment. Shared with the static-scratch entry point, which
// runs it before it touches the device.
int check_ibcs_sip_args(const char* what, const void* q, const void* k, int64_t batch_heads, int64_t tokens,
                        const float* offsets, int64_t samples, const int32_t* ids, const float* log_weights) {
    if (int rc = check_qk_shape(what, batch_heads, tokens)) return rc;
    const int64_t fb = tokens / kKvBlock;
    if (!(samples > 0 && samples < fb))
        return set_error(AB_ERR_INVALID, "%s: sample count must be inside the population", what);
    if (!sip_fused_fits(fb))
        return set_error(AB_ERR_INVALID, "%s: population exceeds the fused kernel's LDS capacity", what);
    if (!q || !k || !offsets || !ids || !log_weights) return set_error(AB_ERR_INVALID, "%s: null pointer", what);
    if (!aligned16(q) || !aligned16(k)) return set_error(AB_ERR_INVALID, "%s: q and k must be 16-byte aligned", what);
    return AB_OK;
}
}  // namespace ab

namespace {
// ab_ibcs_sip; force_exact selects the reference's probe sequence for every
// row sampled with kept prefixes (same bits, testing only).
int ibcs_sip_impl(const void* q, const void* k, const int32_t* order, int64_t batch_heads, int64_t tokens,
                  const float* offsets, int64_t samples, void* workspace, size_t workspace_bytes, int32_t* ids,
                  float* log_weights, int force_exact, void* stream) {
    if (int rc = check_ibcs_sip_args("ibcs_sip", q, k, batch_heads, tokens, offsets, samples, ids, log_weights))
        return rc;
    const IbcsLayout L = ibcs_layout(batch_heads, tokens);
    if (!workspace) return set_error(AB_ERR_INVALID, "ibcs_sip: null pointer");
    const size_t need = ab_ibcs_sip_workspace_bytes(batch_heads, tokens);
    if (workspace_bytes < need)
        return set_error(AB_ERR_INVALID, "ibcs_sip: workspace of %zu bytes is smaller than the %zu required",
                         workspace_bytes, need);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
        return set_error(AB_ERR_INVALID, "ibcs_sip: workspace must be 256-byte aligned");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    float* pops = reinterpret_cast<float*>(ws + L.pops);
    float* lse_max = reinterpret_cast<float*>(ws + L.lse_max);
    float* lse_den = reinterpret_cast<float*>(ws + L.lse_den);
    if (int rc = launch_cluster_pool(q, k, batch_heads, tokens, ws + L.centroids, pops, ws + L.pooled,
                                     qk_scale_log2(), order, st))
        return rc;
    if (int rc = launch_lse(ws + L.centroids, ws + L.pooled, batch_heads, tokens, ws + L.lse, lse_max, lse_den, st))
        return rc;
    return launch_sip_fused(ws + L.lse, pops, lse_max, lse_den, L.ld, offsets, L.rows, L.fb, samples, ids,
                            log_weights, force_exact, st);
}
}  // namespace

extern "C" {

int ab_ibcs_sip(const void* q, const void* k, const int32_t* order, int64_t batch_heads, int64_t tokens,
                const float* offsets, int64_t samples, void* workspace, size_t workspace_bytes, int32_t* ids,
                float* log_weights, void* stream) {
    return ibcs_sip_impl(q, k, order, batch_heads, tokens, offsets, samples, workspace, workspace_bytes, ids,
                         log_weights, 0, stream);
}

int ab_ibcs_sip_exact_draws(const void* q, const void* k, const int32_t* order, int64_t batch_heads,
                            int64_t tokens, const float* offsets, int64_t samples, void* workspace,
                            size_t workspace_bytes, int32_t* ids, float* log_weights, void* stream) {
    return ibcs_sip_impl(q, k, order, batch_heads, tokens, offsets, samples, workspace, workspace_bytes, ids,
                         log_weights, 1, stream);
}

int ab_sip(const float* scores, const float* offsets, int64_t rows, int64_t population, int64_t samples,
           int32_t* ids, float* log_weights, void* stream) {
    if (rows < 0) return set_error(AB_ERR_INVALID, "sip: negative row count");
    if (!(samples > 0 && samples < population))
        return set_error(AB_ERR_INVALID, "sip: sample count must be inside the population");
    if (population > (int64_t(1) << 30)) return set_error(AB_ERR_INVALID, "sip: population too large");
    if (!sip_fits(population))
        return set_error(AB_ERR_INVALID, "sip: population exceeds single-workgroup LDS capacity");
    if (rows > 0 && (!scores || !offsets || !ids || !log_weights))
        return set_error(AB_ERR_INVALID, "sip: null pointer");
    if (rows > 0xffffffffll) return set_error(AB_ERR_INVALID, "sip: too many rows");
    return launch_sip(scores, offsets, rows, population, samples, ids, log_weights,
                      static_cast<hipStream_t>(stream));
}

int ab_paged_prefill(const void* q, const void* k, const void* v, int64_t batch_heads, int64_t tokens,
                     const int32_t* ids, const float* log_weights, int64_t samples, void* out, float* lse,
                     void* stream) {
    if (int rc = check_qk_shape("paged_prefill", batch_heads, tokens)) return rc;
    if (samples <= 0 || samples % kBlocksPerPage)
        return set_error(AB_ERR_INVALID, "paged_prefill: samples must be a positive multiple of 32");
    return ab_paged_prefill_kv(q, k, v, batch_heads, tokens, tokens, ids, log_weights, samples, out, lse, stream);
}

namespace {
// Shared validation of the prefill entry points. dense: every KV4 block of
// K/V at weight 0 (ids and log_weights are not read; samples is derived).
int paged_prefill_checked(const void* q, const void* k, const void* v, bool dense, const int32_t* order,
                          int64_t batch_heads, int64_t q_tokens, int64_t kv_tokens, const int32_t* ids,
                          const float* log_weights, int64_t samples, void* out, float* lse, void* stream) {
    if (batch_heads <= 0 || q_tokens <= 0 || kv_tokens <= 0)
        return set_error(AB_ERR_INVALID, "paged_prefill: batch_heads and token counts must be positive");
    if (kv_tokens % kKvBlock)
        return set_error(AB_ERR_INVALID, "paged_prefill: key/value length must be divisible by 4");
    if (kv_tokens * kHeadDim * 2 > int64_t(0xffffffff))
        return set_error(AB_ERR_INVALID, "paged_prefill: one head of K/V must be under 4 GiB");
    const int64_t qb = (q_tokens + kQueryBlock - 1) / kQueryBlock;
    if (batch_heads > 65535 || qb > 65535) return set_error(AB_ERR_INVALID, "paged_prefill: grid too large");
    if (dense) samples = (kv_tokens / kKvBlock + 7) / 8 * 8;
    if (samples <= 0 || samples % 8)
        return set_error(AB_ERR_INVALID, "paged_prefill: samples must be a positive multiple of 8");
    if (!q || !k || !v || !out || (!dense && (!ids || !log_weights)))
        return set_error(AB_ERR_INVALID, "paged_prefill: null pointer");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || (reinterpret_cast<uintptr_t>(out) & 7u))
        return set_error(AB_ERR_INVALID, "paged_prefill: q/k/v must be 16-byte and out 8-byte aligned");
    if (!dense && (!aligned16(ids) || !aligned16(log_weights)))
        return set_error(AB_ERR_INVALID, "paged_prefill: ids and log_weights must be 16-byte aligned");
    const int64_t rows = batch_heads * qb;
    if (rows * samples > (int64_t(1) << 40)) return set_error(AB_ERR_INVALID, "paged_prefill: plan too large");
    return launch_prefill(q, k, v, dense, batch_heads, q_tokens, kv_tokens, ids, log_weights, samples, out, lse,
                          order, static_cast<hipStream_t>(stream));
}
}  // namespace

int ab_paged_prefill_kv(const void* q, const void* k, const void* v, int64_t batch_heads, int64_t q_tokens,
                        int64_t kv_tokens, const int32_t* ids, const float* log_weights, int64_t samples,
                        void* out, float* lse, void* stream) {
    return paged_prefill_checked(q, k, v, false, nullptr, batch_heads, q_tokens, kv_tokens, ids, log_weights,
                                 samples, out, lse, stream);
}

int ab_dense_prefill(const void* q, const void* k, const void* v, int64_t batch_heads, int64_t q_tokens,
                     int64_t kv_tokens, void* out, float* lse, void* stream) {
    return paged_prefill_checked(q, k, v, true, nullptr, batch_heads, q_tokens, kv_tokens, nullptr, nullptr, 0,
                                 out, lse, stream);
}

int ab_paged_prefill_ordered(const void* q, const void* k, const void* v, const int32_t* order,
                             int64_t batch_heads, int64_t tokens, const int32_t* ids, const float* log_weights,
                             int64_t samples, void* out, float* lse, void* stream) {
    if (!order) return set_error(AB_ERR_INVALID, "paged_prefill: null token order");
    if (int rc = check_qk_shape("paged_prefill", batch_heads, tokens)) return rc;
    if (samples <= 0 || samples % kBlocksPerPage)
        return set_error(AB_ERR_INVALID, "paged_prefill: samples must be a positive multiple of 32");
    return paged_prefill_checked(q, k, v, false, order, batch_heads, tokens, tokens, ids, log_weights, samples,
                                 out, lse, stream);
}

int64_t ab_prefill_launch_slots(int64_t batch_heads, int64_t q_tokens) {
    if (batch_heads <= 0 || q_tokens <= 0) return 0;
    return prefill_launch_slots(batch_heads, q_tokens);
}

int ab_remap_ids(const int32_t* ids, int64_t count, const int32_t* map, int64_t map_len, int32_t* out,
                 void* stream) {
    if (count < 0 || map_len <= 0 || map_len > kMaxKvBlocks)
        return set_error(AB_ERR_INVALID, "remap_ids: bad count or map length");
    if (count > 0 && (!ids || !map || !out)) return set_error(AB_ERR_INVALID, "remap_ids: null pointer");
    if (count > (int64_t(1) << 40)) return set_error(AB_ERR_INVALID, "remap_ids: too many ids");
    return launch_remap_ids(ids, count, map, map_len, out, static_cast<hipStream_t>(stream));
}

int ab_merge_states(const void* o_a, const float* lse_a, const void* o_b, const float* lse_b, int64_t count,
                    void* out, float* lse_out, void* stream) {
    if (count < 0) return set_error(AB_ERR_INVALID, "merge_states: negative count");
    if (count > 0 && (!o_a || !lse_a || !o_b || !lse_b || !out))
        return set_error(AB_ERR_INVALID, "merge_states: null pointer");
    if (!aligned16(o_a) || !aligned16(o_b) || !aligned16(out))
        return set_error(AB_ERR_INVALID, "merge_states: states must be 16-byte aligned");
    if (count > (int64_t(1) << 35)) return set_error(AB_ERR_INVALID, "merge_states: too many rows");
    return launch_merge(o_a, lse_a, o_b, lse_b, count, out, lse_out, static_cast<hipStream_t>(stream));
}

}  // extern "C"
