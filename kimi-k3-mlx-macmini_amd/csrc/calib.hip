// HBM calibration kernels: a streaming read and a streaming copy of a known byte count.
// They have no counterpart in the reference.  The benchmark uses them to measure the
// bandwidth one launch of a given size can reach on this device (the practical ceiling
// beside the 8 TB/s spec), and the profiler runs use them to scale the FETCH_SIZE /
// WRITE_SIZE counters (bytes the counters report per byte actually moved).
#include <algorithm>

#include "k3_common.h"

namespace k3 {
namespace {

// Each block streams one contiguous chunk of 16-byte words, 8 loads in flight per lane.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4 *__restrict__ src, int64_t n16, int64_t chunk,
                                                          uint32_t *__restrict__ sink) {
    const int64_t start = static_cast<int64_t>(blockIdx.x) * chunk;
    const int64_t end = min(start + chunk, n16);
    uint32_t acc = 0;
    for (int64_t base = start + threadIdx.x; base < end; base += 256 * 8) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t i = base + static_cast<int64_t>(u) * 256;
            v[u] = i < end ? src[i] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    // keeps the loads live; the sink word is written only for one data-dependent value
    if (acc == 0x9e3779b9u) sink[blockIdx.x & 1023] = acc;
}

__global__ __launch_bounds__(256) void stream_copy_kernel(uint4 *__restrict__ dst, const uint4 *__restrict__ src,
                                                          int64_t n16, int64_t chunk) {
    const int64_t start = static_cast<int64_t>(blockIdx.x) * chunk;
    const int64_t end = min(start + chunk, n16);
    for (int64_t base = start + threadIdx.x; base < end; base += 256 * 8) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t i = base + static_cast<int64_t>(u) * 256;
            if (i < end) v[u] = src[i];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t i = base + static_cast<int64_t>(u) * 256;
            if (i < end) dst[i] = v[u];
        }
    }
}

int grid_for(int64_t n16, int64_t *chunk) {
    // 2048 blocks (8 per CU) measured best for 7.8 MB .. 280 MB single-launch reads
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(2048, cdiv(n16, 256)));
    *chunk = cdiv(n16, blocks);
    return static_cast<int>(cdiv(n16, *chunk));
}

}  // namespace
}  // namespace k3

using namespace k3;

extern "C" int k3_stream_read(const void *src, int64_t bytes, void *sink, void *stream) {
    if (!src || !sink) return set_error(K3_ERR_NULL, "stream read: null pointer");
    if (bytes < 0 || bytes % 16 || !aligned16(src))
        return set_error(K3_ERR_SHAPE, "stream read: bytes must be a multiple of 16 and src 16-byte aligned");
    if (bytes == 0) return K3_OK;
    int64_t chunk;
    const int blocks = grid_for(bytes / 16, &chunk);
    stream_read_kernel<<<dim3(blocks), 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint4 *>(src), bytes / 16, chunk, static_cast<uint32_t *>(sink));
    return check_hip(hipGetLastError(), "stream read launch");
}

extern "C" int k3_stream_copy(void *dst, const void *src, int64_t bytes, void *stream) {
    if (!src || !dst) return set_error(K3_ERR_NULL, "stream copy: null pointer");
    if (bytes < 0 || bytes % 16 || !aligned16(src) || !aligned16(dst))
        return set_error(K3_ERR_SHAPE, "stream copy: bytes must be a multiple of 16, pointers 16-byte aligned");
    if (bytes == 0) return K3_OK;
    int64_t chunk;
    const int blocks = grid_for(bytes / 16, &chunk);
    stream_copy_kernel<<<dim3(blocks), 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<uint4 *>(dst), static_cast<const uint4 *>(src), bytes / 16, chunk);
    return check_hip(hipGetLastError(), "stream copy launch");
}
