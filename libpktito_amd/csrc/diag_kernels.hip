/* Measurement aids: the floors a small product's time is read against. An
 * empty kernel (the cost of a launch), and a streaming read of a buffer by
 * one 16-byte load a thread over as many workgroups as the bytes need, every
 * load in flight at once, folded so that none is dropped; nothing is written
 * unless the fold meets a fixed 32-bit constant. */
#include "pk_hip.h"
#include "q8_internal.h"

namespace pkq8 {

__global__ __launch_bounds__(256) void empty_kernel() {}

__global__ __launch_bounds__(256) void stream_read_kernel(const uint4 *__restrict__ p, uint64_t n16,
                                                          uint32_t *__restrict__ sink) {
    uint32_t f = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * 256) {
        const uint4 v = p[i];
        f ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (f == 0x9E3779B9u)
        *sink = f;
}

int launch_empty(hipStream_t s) {
    empty_kernel<<<1, 64, 0, s>>>();
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

int launch_stream_read(const void *p, uint64_t bytes, uint32_t *sink, hipStream_t s) {
    const uint64_t n16 = bytes / 16;
    if (n16 == 0)
        return 0;
    const uint64_t wg = (n16 + 255) / 256;
    stream_read_kernel<<<(uint32_t)(wg < 8192 ? wg : 8192), 256, 0, s>>>((const uint4 *)p, n16, sink);
    return hipPeekAtLastError() == hipSuccess ? 0 : -1;
}

}  // namespace pkq8
