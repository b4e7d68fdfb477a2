// common.h — shared definitions of libanehip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/anehip.h"

namespace anehip {

// Per-context error slot.  Context-free failures use a thread-local slot.
struct ErrorSlot {
    std::string msg;
};

ErrorSlot &global_error();

int set_error(ErrorSlot &slot, int code, const char *fmt, ...) __attribute__((format(printf, 3, 4)));

#define ANEHIP_HIP_TRY(slot, expr)                                                            \
    do {                                                                                      \
        hipError_t _e = (expr);                                                               \
        if (_e != hipSuccess)                                                                 \
            return ::anehip::set_error((slot), ANEHIP_EHIP, "%s failed: %s (%s:%d)", #expr,   \
                                       hipGetErrorString(_e), __FILE__, __LINE__);            \
    } while (0)

// A device buffer owned by a context.
struct DevBuf {
    void *ptr = nullptr;
    size_t bytes = 0;
};

// Device workspace used by split-K reductions: partial sums and per-tile
// arrival counters.  Counters are returned to zero by the kernel that uses
// them, so the workspace needs clearing only once, at allocation.
struct Workspace {
    float *partial = nullptr;      // split-K partial sums
    size_t partial_floats = 0;
    uint32_t *counters = nullptr;  // per-row-tile arrival counters
    size_t n_counters = 0;
};

}  // namespace anehip

struct anehip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    anehip::ErrorSlot err;
    anehip::Workspace ws;
    std::vector<void *> user_allocs;
    struct Model *model = nullptr;  // decode-step state (decode.hip)
    int cu_count = 0;
};

namespace anehip {

// Ensures the split-K workspace holds at least `floats` partials and
// `counters` counters (grown with hipMalloc, cleared once).
int ensure_workspace(anehip_ctx *ctx, size_t floats, size_t counters);

// GEMM dispatch used by the public entry point and by the decode step.
// All pointers are device pointers; work is queued on `stream`.
int launch_quant_gemm(anehip_ctx *ctx, hipStream_t stream, uint32_t ggml_type, const void *w,
                      uint32_t m, uint32_t n, const float *x, uint32_t batch, float *y);

}  // namespace anehip
