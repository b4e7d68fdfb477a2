/* probe.h — C ABI of libanehip_probe.so, the measurement-only library that
 * bench.py loads beside libanehip.so.  No counterpart in the reference and
 * not part of the product library: the measured floor under a
 * bandwidth-bound launch of a given size and grid, timed on a libanehip
 * context's stream like the kernels it bounds.
 *
 * anehip_probe_read streams nbytes (a positive multiple of 16) from device
 * memory src in 16-byte loads on workgroups x threads threads (threads a
 * multiple of 64, at most 1024), depth (1, 2, 4 or 8) loads in flight per
 * thread; sink (device, at least workgroups * threads * 4 bytes) is written
 * only in the unlikely case that a thread's XOR of its loads equals a fixed
 * constant.  anehip_probe_empty launches an empty kernel of that grid.  Both
 * return 0 or a negative ANEHIP_E* code with the message in
 * anehip_last_error(ctx). */
#pragma once
#include "../../include/anehip.h"

#ifdef __cplusplus
extern "C" {
#endif

int anehip_probe_read(anehip_ctx *ctx, const void *src, size_t nbytes, uint32_t workgroups, uint32_t threads,
                      uint32_t depth, void *sink);
int anehip_probe_empty(anehip_ctx *ctx, uint32_t workgroups, uint32_t threads);

#ifdef __cplusplus
}
#endif
