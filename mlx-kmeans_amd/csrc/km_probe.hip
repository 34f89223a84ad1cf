// Streaming-read probe: the HBM read rate a plain kernel reaches on this device, the floor a pass's time is judged
// against beside the published peak (quick_bench.py:48-63 measures the same on Apple GPUs with a grid-stride
// read of one large array).
//
// Each thread reads 16-byte vectors in a grid-stride loop with UNROLL loads in flight and writes one float per
// thread, so no load can be dropped; the output (grid x 4 bytes) is negligible against the array.
#include "km_internal.h"

namespace {

template <int UNROLL>
__global__ __launch_bounds__(256) void k_stream_read(const float4 *__restrict__ x, int64_t n4, float *__restrict__ out) {
    const int64_t T = (int64_t)gridDim.x * blockDim.x;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t i = t;
    float s = 0.0f;
    for (; i + (UNROLL - 1) * T < n4; i += UNROLL * T) {
        float4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) v[u] = x[i + u * T];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) s += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
    for (; i < n4; i += T) {
        const float4 v = x[i];
        s += (v.x + v.y) + (v.z + v.w);
    }
    out[t] = s;
}

}  // namespace

hipError_t km_launch_stream_read(const void *x, int64_t bytes, float *out, int blocks, hipStream_t s) {
    if (blocks < 1 || bytes % 16 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_stream_read<4>, dim3(blocks), dim3(256), 0, s, (const float4 *)x, bytes / 16, out);
    return hipGetLastError();
}
