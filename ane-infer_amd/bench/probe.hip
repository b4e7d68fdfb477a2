// Roofline probes (libanehip_probe.so, loaded by bench.py only; not part of
// the product library): the floor a bandwidth-bound launch of a given size and
// grid can reach on this device, measured with the same launch path, stream
// and timers as the kernels it bounds.  probe_read_kernel streams a buffer in 16-byte loads
// (grid-stride, DEPTH independent loads in flight per thread, the values
// folded into one XOR so the loads stay live); probe_empty_kernel does
// nothing, which gives the fixed cost of one launch of that grid.
#include "../csrc/common.h"
#include "probe.h"

namespace anehip {
namespace {

template <int DEPTH>
__global__ void probe_read_kernel(const uint4 *__restrict__ src, size_t n16, uint32_t *__restrict__ sink) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (size_t)(DEPTH - 1) * stride < n16; i += (size_t)DEPTH * stride) {
        uint4 v[DEPTH];
#pragma unroll
        for (int k = 0; k < DEPTH; k++) v[k] = src[i + (size_t)k * stride];
#pragma unroll
        for (int k = 0; k < DEPTH; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    for (; i < n16; i += stride) {
        const uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    // a store that depends on every load (and almost never happens)
    if (acc == 0x9E3779B9u) sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

__global__ void probe_empty_kernel() {}

}  // namespace
}  // namespace anehip

using namespace anehip;

#define NEED_CTX(ctx, name)                                                                    \
    do {                                                                                       \
        if (!(ctx)) return set_error(global_error(), ANEHIP_EINVAL, name ": ctx is NULL");      \
    } while (0)

extern "C" {

int anehip_probe_read(anehip_ctx *ctx, const void *src, size_t nbytes, uint32_t workgroups, uint32_t threads,
                      uint32_t depth, void *sink) {
    NEED_CTX(ctx, "probe_read");
    if (!src || !sink) return set_error(ctx->err, ANEHIP_EINVAL, "probe_read: null pointer");
    if (nbytes == 0 || nbytes % 16)
        return set_error(ctx->err, ANEHIP_EINVAL, "probe_read: nbytes %zu not a positive multiple of 16", nbytes);
    if (workgroups == 0 || workgroups > (1u << 20) || threads == 0 || threads > 1024 || threads % 64)
        return set_error(ctx->err, ANEHIP_EINVAL, "probe_read: grid %u x %u unsupported", workgroups, threads);
    const size_t n16 = nbytes / 16;
    const uint4 *s = static_cast<const uint4 *>(src);
    uint32_t *k = static_cast<uint32_t *>(sink);
    switch (depth) {
        case 1: hipLaunchKernelGGL(probe_read_kernel<1>, dim3(workgroups), dim3(threads), 0, ctx->stream, s, n16, k); break;
        case 2: hipLaunchKernelGGL(probe_read_kernel<2>, dim3(workgroups), dim3(threads), 0, ctx->stream, s, n16, k); break;
        case 4: hipLaunchKernelGGL(probe_read_kernel<4>, dim3(workgroups), dim3(threads), 0, ctx->stream, s, n16, k); break;
        case 8: hipLaunchKernelGGL(probe_read_kernel<8>, dim3(workgroups), dim3(threads), 0, ctx->stream, s, n16, k); break;
        default: return set_error(ctx->err, ANEHIP_EINVAL, "probe_read: depth %u not 1, 2, 4 or 8", depth);
    }
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

int anehip_probe_empty(anehip_ctx *ctx, uint32_t workgroups, uint32_t threads) {
    NEED_CTX(ctx, "probe_empty");
    if (workgroups == 0 || workgroups > (1u << 20) || threads == 0 || threads > 1024 || threads % 64)
        return set_error(ctx->err, ANEHIP_EINVAL, "probe_empty: grid %u x %u unsupported", workgroups, threads);
    hipLaunchKernelGGL(probe_empty_kernel, dim3(workgroups), dim3(threads), 0, ctx->stream);
    ANEHIP_HIP_TRY(ctx->err, hipGetLastError());
    return ANEHIP_OK;
}

}  // extern "C"
