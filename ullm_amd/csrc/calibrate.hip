// Read-bandwidth calibration kernel: the floor a read-only HBM stream of a
// given size reaches on this GPU, measured beside the attention kernels.
//
// The decode op reads its K/V bytes once and writes little, so its roofline
// is a pure read.  For small layers (4 MiB at 4K context) the time of one
// launch in a graph, not the 8 TB/s peak, bounds it: this kernel gives that
// bound at the same size, with the same launch path (one graph node).
#include "common.hpp"

namespace ullm {

// Workgroup w reads its contiguous slice [w*per, (w+1)*per) of 16-byte
// chunks (the last slice takes the remainder); the result is stored only if
// it matches a value the data never folds to, so the loads stay live.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4 *__restrict__ p, int64_t n16,
                                                          uint32_t *__restrict__ sink) {
    const int64_t per = n16 / gridDim.x;
    const int64_t lo = per * blockIdx.x;
    const int64_t hi = blockIdx.x + 1 == gridDim.x ? n16 : lo + per;
    uint32_t acc = 0;
#pragma unroll 8
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
        const u32x4 v = p[i];
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

}  // namespace ullm

using namespace ullm;

extern "C" int ullm_hip_stream_read(const void *src, size_t bytes, int workgroups,
                                    uint32_t *sink, void *stream) {
    if (!src || !sink || bytes < 16 || workgroups < 1 || ((uintptr_t)src & 15))
        return set_error(ULLM_HIP_E_INVALID, "stream_read: bad arguments");
    const int64_t n16 = (int64_t)(bytes / 16);
    hipLaunchKernelGGL(stream_read_kernel, dim3(workgroups), dim3(256), 0, (hipStream_t)stream,
                       (const u32x4 *)src, n16, sink);
    return check_hip(hipGetLastError(), "stream_read launch");
}
