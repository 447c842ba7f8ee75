// Ceiling probe of the hash-grid gradient scatter: the device's rate of fp32
// atomic-add requests to random 64-byte lines (graft_diag.h).
#include "abi_error.h"
#include "common.h"
#include "graft_diag.h"

#include <stdexcept>

namespace graft {
namespace {

// 32-bit integer finalizer (xor-shift / multiply rounds) spreading
// consecutive inputs over the line range.
__device__ __forceinline__ uint32_t mix32(uint32_t x)
{
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// Lane j of group g (dwords lanes per group) adds to dword j of line
// mix32(...) & line_mask, once per iteration: one line request per group per
// instruction.  line_mask + 1 lines of 16 floats fit the buffer.
__global__ __launch_bounds__(256) void atomic_lines_kernel(float* __restrict__ buf, uint32_t line_mask, int dwords,
                                                           int iters)
{
    const int lane = threadIdx.x & 63;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int grp = lane / dwords, j = lane - grp * dwords;
    for (int it = 0; it < iters; it++) {
        const uint32_t line = mix32(wave * 7919u + (uint32_t)it * 64u + (uint32_t)grp) & line_mask;
        atomic_add_f32(buf + (size_t)line * 16 + j, 1.0f);
    }
}

struct Event {
    hipEvent_t e = nullptr;
    ~Event()
    {
        if (e) (void)hipEventDestroy(e);
    }
};

}  // namespace
}  // namespace graft

extern "C" int graft_diag_atomic_line_rate(float* d_buf, size_t bytes, int dwords_per_line, double* requests_per_s,
                                           hipStream_t stream)
{
    return graft::guarded("graft_diag_atomic_line_rate", [&] {
        if (d_buf == nullptr || requests_per_s == nullptr) throw std::runtime_error("null argument");
        if (dwords_per_line < 1 || dwords_per_line > 16 || (dwords_per_line & (dwords_per_line - 1)))
            throw std::runtime_error("dwords_per_line must be 1, 2, 4, 8 or 16");
        if (bytes < (size_t)64 << 10) throw std::runtime_error("buffer must hold at least 64 KiB");
        size_t lines = 1;
        while (lines * 2 * 64 <= bytes && lines < ((size_t)1 << 31)) lines *= 2;
        const int blocks = graft::num_cus();
        const long long lanes_per_iter = (long long)blocks * 256;
        const int iters = (int)std::max(1LL, ((1LL << 24) * dwords_per_line) / lanes_per_iter);
        graft::Event a, b;
        GRAFT_HIP_CHECK(hipEventCreate(&a.e));
        GRAFT_HIP_CHECK(hipEventCreate(&b.e));
        const uint32_t mask = (uint32_t)(lines - 1);
        hipLaunchKernelGGL(graft::atomic_lines_kernel, dim3(blocks), dim3(256), 0, stream, d_buf, mask,
                           dwords_per_line, iters);
        GRAFT_LAUNCH_CHECK();
        const int reps = 5;
        GRAFT_HIP_CHECK(hipEventRecord(a.e, stream));
        for (int r = 0; r < reps; r++)
            hipLaunchKernelGGL(graft::atomic_lines_kernel, dim3(blocks), dim3(256), 0, stream, d_buf, mask,
                               dwords_per_line, iters);
        GRAFT_LAUNCH_CHECK();
        GRAFT_HIP_CHECK(hipEventRecord(b.e, stream));
        GRAFT_HIP_CHECK(hipEventSynchronize(b.e));
        float ms = 0.f;
        GRAFT_HIP_CHECK(hipEventElapsedTime(&ms, a.e, b.e));
        const double requests = (double)lanes_per_iter * iters * reps / dwords_per_line;
        *requests_per_s = requests / (ms * 1e-3);
    });
}
