/*
 * llmik_diag.h — measurement floors of libllmik_diag.so, a library of its
 * own beside libllmik_hip.so. No counterpart in the reference and no part
 * of the product's ABI: these kernels calibrate the roofline figures of
 * the entry points in llmik.h (bench.py --floors, the profile summaries
 * that quote the floors). Status codes are llmik.h's.
 */
#ifndef LLMIK_DIAG_H
#define LLMIK_DIAG_H

#include "llmik.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The message of this library's last failed call on the calling thread. */
LLMIK_API const char* llmik_diag_last_error(void);

/*
 * llmik_diag_empty: one launch of an empty kernel, n_workgroups x 512 threads.
 *
 * llmik_diag_read: a streaming read of `bytes` bytes at src (16-byte aligned,
 * bytes % 16 == 0, bytes <= 3 GiB) by n_workgroups x 8 waves, each wave
 * reading units of loads_per_lane (4, 8 or 16) KiB round robin, with
 * loads_per_lane non-temporal 16-byte loads per lane in flight. Wave w
 * writes the xor of the 32-bit words it read to ((uint32_t*)sink)[w]; sink
 * must hold n_workgroups * 8 values, and their xor is the xor of every word.
 */
LLMIK_API llmik_status llmik_diag_empty(int n_workgroups, void* stream);
LLMIK_API llmik_status llmik_diag_read(const void* src, size_t bytes, void* sink, int n_workgroups,
                                       int loads_per_lane, void* stream);
/*
 * llmik_diag_read_write: the read of llmik_diag_read (loads_per_lane 4 or 8)
 * with a write stream of write_bytes_per_16 (4, 8 or 16) bytes per 16 bytes
 * read: 16-byte chunk j of src gives its first write_bytes_per_16 bytes to
 * dst at j * write_bytes_per_16 (src, dst 16-byte aligned; dst holds
 * bytes / 16 * write_bytes_per_16 bytes). The KV writers' stream shape.
 */
LLMIK_API llmik_status llmik_diag_read_write(const void* src, size_t bytes, void* dst, int write_bytes_per_16,
                                             int n_workgroups, int loads_per_lane, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LLMIK_DIAG_H */
