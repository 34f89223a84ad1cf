// Streaming-read probe: the HBM read rate a plain kernel reaches on this device, the floor a pass's time is judged
// against beside the published peak (quick_bench.py:48-63 measures the same on Apple GPUs with a grid-stride
// read of one large array).
//
// Each block reads one contiguous range of the array, its 256 threads taking consecutive 16-byte vectors with
// UNROLL loads in flight, non-temporal (the data is read once); each thread writes one float, so no load can be
// dropped, and the output (grid x 4 bytes) is negligible against the array. On MI355X this reaches 7.0-7.1 TB/s;
// the same read without the non-temporal hint, or as a grid-stride loop, 6.0-6.3.
#include "km_internal.h"

namespace {

typedef float probe_f4 __attribute__((ext_vector_type(4)));

template <int UNROLL>
__global__ __launch_bounds__(256) void k_stream_read(const probe_f4 *__restrict__ x, int64_t n4, float *__restrict__ out) {
    const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
    const int64_t b0 = (int64_t)blockIdx.x * per;
    const int64_t b1 = b0 + per < n4 ? b0 + per : n4;
    int64_t i = b0 + threadIdx.x;
    float s = 0.0f;
    for (; i + (UNROLL - 1) * 256 < b1; i += UNROLL * 256) {
        probe_f4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) v[u] = __builtin_nontemporal_load(x + i + u * 256);
#pragma unroll
        for (int u = 0; u < UNROLL; u++) s += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
    for (; i < b1; i += 256) {
        const probe_f4 v = __builtin_nontemporal_load(x + i);
        s += (v.x + v.y) + (v.z + v.w);
    }
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace

hipError_t km_launch_stream_read(const void *x, int64_t bytes, float *out, int blocks, hipStream_t s) {
    if (blocks < 1 || bytes % 16 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_stream_read<8>, dim3(blocks), dim3(256), 0, s, (const probe_f4 *)x, bytes / 16, out);
    return hipGetLastError();
}
