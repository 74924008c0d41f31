/* Diagnostic entry point of libkcr_hip.so with no counterpart in the
 * reference: a streaming kernel that measures the HBM rate the bandwidth-bound
 * ops can reach on this device (the practical ceiling beside the 8 TB/s peak),
 * and calibrates the FETCH_SIZE / WRITE_SIZE counters on a known byte count.
 * Only the benchmark calls it. */
#ifndef KCR_PROBE_H
#define KCR_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reads == 1: dst[i] = src[i] over `words` 16-byte words (read 16·words bytes,
 * write 16·words bytes).
 * reads == 2: dst[i] = src[i] ^ src[words + i] (read 32·words, write 16·words):
 * the 2:1 read:write mix of the gated activations.
 * src and dst must be 16-byte aligned device pointers and must not overlap.
 * Asynchronous on `stream`. Returns a kcr_status. */
int32_t kcr_hbm_stream_probe(void* dst, const void* src, int64_t words, int32_t reads, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KCR_PROBE_H */
