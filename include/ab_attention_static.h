/*
 * C ABI of libab_attention_static.so: the fused plan without allocation.
 *
 * No counterpart in the reference; for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). This library links against libab_attention_hip.so
 * (include/ab_attention.h), whose ab_last_error() reports its failures.
 *
 * ab_ibcs_sip_static is ab_ibcs_sip with the same arguments minus the
 * workspace, giving the same bits. The IBCS intermediates live in a static
 * device array of AB_STATIC_SCRATCH_BYTES in this library's code object: a
 * GPU holds it from the moment the HIP runtime loads that code object there
 * until the process ends. With ROCm 7's deferred code-object loading that is
 * the first ab_ibcs_sip_static call on the device, not the library's load
 * (measured on an MI355X: loading took 0 MiB of device memory, the first
 * call 512 MiB). A process that never loads this library holds no such
 * array; libab_attention_hip.so has none. Heads run in chunks that fit
 * the array, and a shape whose single head needs more (tokens above 128,768)
 * is rejected with AB_ERR_INVALID. Every argument is checked, with
 * ab_ibcs_sip's checks and messages, before any runtime call. The call
 * allocates nothing (no hipMalloc, no hipFree). Calls that overlap on one GPU
 * (other streams or threads) race on the array. The first call on a device
 * resolves the array's address, a runtime call: make it outside graph
 * capture.
 */
#ifndef AB_ATTENTION_STATIC_H
#define AB_ATTENTION_STATIC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AB_STATIC_SCRATCH_BYTES ((size_t)512 << 20)
int ab_ibcs_sip_static(const void *q, const void *k, const int32_t *order, int64_t batch_heads, int64_t tokens,
                       const float *offsets, int64_t samples, int32_t *ids, float *log_weights, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* AB_ATTENTION_STATIC_H */
