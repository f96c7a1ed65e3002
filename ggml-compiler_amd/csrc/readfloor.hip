// readfloor.hip - gcq_stream_read: one launch that reads a device buffer once and computes
// nothing, the floor a kernel streaming the same bytes in one launch cannot beat. The benchmark
// times it beside each decode projection (same bytes, same launch method) to separate what the
// launch and the memory system cost from what a kernel adds.
//
// Each wavefront reads a contiguous range (1 KiB per load instruction, 16 B per lane), `U` loads
// in flight before any is consumed; the XOR of the words is stored only if it equals a constant,
// which keeps the loads without writing anything in practice.
#include "gcq_common.h"

#include "../../include/gcq.h"

namespace gcq {
int cu_count();
namespace {

template <int U>
__global__ __launch_bounds__(256) void k_stream_read(const uint8_t * __restrict__ src, int64_t bytes, int64_t per_wave,
                                                     uint32_t * __restrict__ sink) {
    const int64_t wave = ((int64_t) blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t w0 = wave * per_wave;
    const int64_t w1 = w0 + per_wave < bytes ? w0 + per_wave : bytes;
    uint32_t acc = 0;
    for (int64_t a = w0; a < w1; a += U * 1024) {
        uint4 r[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t o = a + u * 1024 + lane * 16;
            r[u] = o + 16 <= w1 ? *reinterpret_cast<const uint4 *>(src + o) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= r[u].x ^ r[u].y ^ r[u].z ^ r[u].w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace
}  // namespace gcq

using namespace gcq;

extern "C" int gcq_stream_read(const void * src, size_t bytes, int waves_per_cu, int unroll, uint32_t * sink,
                               void * stream) {
    return guarded([&] {
        require(src != nullptr && sink != nullptr, "stream_read: src or sink is NULL");
        require(((uintptr_t) src & 15u) == 0 && bytes % 16 == 0, "stream_read: src and bytes must be 16-byte aligned");
        require(bytes > 0 && bytes < ((size_t) 1 << 40), "stream_read: bytes out of range");
        require(waves_per_cu == 4 || waves_per_cu == 8 || waves_per_cu == 16 || waves_per_cu == 32,
                "stream_read: waves_per_cu must be 4, 8, 16 or 32");
        require(unroll == 1 || unroll == 2 || unroll == 4, "stream_read: unroll must be 1, 2 or 4");
        const int64_t waves = (int64_t) cu_count() * waves_per_cu;
        const int64_t per_wave = ((int64_t) ((bytes + waves - 1) / waves) + 1023) / 1024 * 1024;
        const int grid = (int) (waves / 4);
        const hipStream_t s = as_stream(stream);
        const uint8_t * p = static_cast<const uint8_t *>(src);
        if (unroll == 1) k_stream_read<1><<<grid, 256, 0, s>>>(p, (int64_t) bytes, per_wave, sink);
        else if (unroll == 2) k_stream_read<2><<<grid, 256, 0, s>>>(p, (int64_t) bytes, per_wave, sink);
        else k_stream_read<4><<<grid, 256, 0, s>>>(p, (int64_t) bytes, per_wave, sink);
        check_hip(hipGetLastError(), "stream_read launch");
    });
}
