// Device-ceiling probes of bench.py (bench_probes.so, built beside bench.py
// by __graft_entry__.build(); not part of lib3dmaker_amd.so).  Each measures
// a rate that a kernel of the training step is priced against where no
// published peak applies, on the caller's stream, and blocks until done.
//
//   probe_stream_copy        a hand-written grid-stride float4 copy: the
//                            achievable streaming bandwidth (read + write)
//   probe_random_lines       one 4-byte load per lane from a pseudo-random
//                            64-byte line of a table: the achievable rate of
//                            the hash encode's corner gathers, over the whole
//                            table or with each XCD's workgroups confined to
//                            their eighth of it (as the encode deals levels)
//   probe_atomic_lines       fire-and-forget fp32 atomic adds to random
//                            64-byte lines: the rate that bounds a scatter of
//                            one global atomic per product
//
// Functions return 0, or non-zero with a message in probe_last_error().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <string>

namespace {

std::string g_err;

int fail(const std::string& m)
{
    g_err = m;
    return 1;
}

#define PROBE_CHECK(expr)                                                                      \
    do {                                                                                       \
        hipError_t _e = (expr);                                                                \
        if (_e != hipSuccess) return fail(std::string(#expr) + ": " + hipGetErrorString(_e)); \
    } while (0)

__device__ __forceinline__ uint32_t mix32(uint32_t x)
{
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

typedef float v4f __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ v4f ld(const v4f* p)
{
    if constexpr (NT) return __builtin_nontemporal_load(p);
    return *p;
}

template <bool NT>
__device__ __forceinline__ void st(v4f* p, v4f v)
{
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

template <bool NT>
__global__ __launch_bounds__(256) void copy_kernel(const v4f* __restrict__ src, v4f* __restrict__ dst, size_t n)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n; i += 4 * stride) {
        const v4f a = ld<NT>(src + i), b = ld<NT>(src + i + stride), c = ld<NT>(src + i + 2 * stride),
                  d = ld<NT>(src + i + 3 * stride);
        st<NT>(dst + i, a);
        st<NT>(dst + i + stride, b);
        st<NT>(dst + i + 2 * stride, c);
        st<NT>(dst + i + 3 * stride, d);
    }
    for (; i < n; i += stride) st<NT>(dst + i, ld<NT>(src + i));
}

// Lane loads dword (h & 15) of line (h >> 4) & mask within its region; the
// addresses do not depend on loaded data, so loads of successive iterations
// are in flight together.  XCD partition: workgroup b runs on XCD b mod 8 and
// reads only lines [x * lines/8, (x + 1) * lines/8).
__global__ __launch_bounds__(256) void lines_kernel(const uint32_t* __restrict__ table, uint32_t line_mask,
                                                    int xcd_partition, int iters, uint32_t* __restrict__ sink)
{
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t base = 0, mask = line_mask;
    if (xcd_partition) {
        const uint32_t per = (line_mask + 1) / 8;
        base = (blockIdx.x % 8) * per;
        mask = per - 1;
    }
    uint32_t acc = 0;
#pragma unroll 8
    for (int it = 0; it < iters; it++) {
        const uint32_t h = mix32(gid * 0x9E3779B9u + (uint32_t)it * 0x85EBCA6Bu);
        const uint32_t line = base + ((h >> 4) & mask);
        acc ^= table[(size_t)line * 16 + (h & 15u)];
    }
    sink[gid] = acc;
}

__global__ __launch_bounds__(256) void atomic_lines_kernel(float* __restrict__ buf, uint32_t line_mask, int dwords,
                                                           int iters)
{
    const int lane = threadIdx.x & 63;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int grp = lane / dwords, j = lane - grp * dwords;
    for (int it = 0; it < iters; it++) {
        const uint32_t line = mix32(wave * 7919u + (uint32_t)it * 64u + (uint32_t)grp) & line_mask;
        __hip_atomic_fetch_add(buf + (size_t)line * 16 + j, 1.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

int num_cus(int* out)
{
    int dev = 0;
    PROBE_CHECK(hipGetDevice(&dev));
    PROBE_CHECK(hipDeviceGetAttribute(out, hipDeviceAttributeMultiprocessorCount, dev));
    return 0;
}

// Milliseconds of `launch` repeated `reps` times after one warm-up, on `s`.
template <class F>
int time_ms(hipStream_t s, int reps, F&& launch, float* ms)
{
    hipEvent_t a, b;
    PROBE_CHECK(hipEventCreate(&a));
    PROBE_CHECK(hipEventCreate(&b));
    launch();
    PROBE_CHECK(hipGetLastError());
    PROBE_CHECK(hipEventRecord(a, s));
    for (int r = 0; r < reps; r++) launch();
    PROBE_CHECK(hipGetLastError());
    PROBE_CHECK(hipEventRecord(b, s));
    PROBE_CHECK(hipEventSynchronize(b));
    PROBE_CHECK(hipEventElapsedTime(ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return 0;
}

uint32_t lines_pow2(size_t bytes)
{
    uint32_t lines = 1;
    while ((size_t)lines * 2 * 64 <= bytes && lines < (1u << 31)) lines *= 2;
    return lines;
}

}  // namespace

extern "C" {

const char* probe_last_error(void) { return g_err.c_str(); }

// Bytes read + written per second by a float4 copy of n_bytes (a multiple of
// 16) from src to dst: the best of 4, 8, 16 and 32 workgroups per CU, with
// ordinary and with non-temporal accesses, each the mean of `reps` launches.
int probe_stream_copy(const void* src, void* dst, size_t n_bytes, int reps, double* bytes_per_s, hipStream_t s)
{
    if (!src || !dst || n_bytes < 16 || n_bytes % 16 || reps < 1 || !bytes_per_s) return fail("bad arguments");
    int cus = 0;
    if (num_cus(&cus)) return 1;
    const size_t n = n_bytes / 16;
    const auto* s4 = static_cast<const v4f*>(src);
    auto* d4 = static_cast<v4f*>(dst);
    double best = 0.0;
    for (int nt = 0; nt < 2; nt++) {
        for (int per_cu = 4; per_cu <= 32; per_cu *= 2) {
            const int blocks = cus * per_cu;
            float ms = 0.f;
            if (time_ms(s, reps, [&] {
                    if (nt) hipLaunchKernelGGL(copy_kernel<true>, dim3(blocks), dim3(256), 0, s, s4, d4, n);
                    else hipLaunchKernelGGL(copy_kernel<false>, dim3(blocks), dim3(256), 0, s, s4, d4, n);
                }, &ms))
                return 1;
            best = std::max(best, 2.0 * (double)n_bytes * reps / (ms * 1e-3));
        }
    }
    *bytes_per_s = best;
    return 0;
}

// 64-byte-line loads per second: `lanes_loads` loads per lane, 16 workgroups
// of 256 lanes per CU, each load from a pseudo-random line among the largest
// power of two of lines that fits table_bytes (>= 64 KiB).  sink receives one
// word per lane (>= 16 * 256 * CUs words).
int probe_random_lines(const void* table, size_t table_bytes, int xcd_partition, int lane_loads, void* sink,
                       size_t sink_bytes, double* lines_per_s, hipStream_t s)
{
    if (!table || table_bytes < (64u << 10) || lane_loads < 1 || !sink || !lines_per_s) return fail("bad arguments");
    int cus = 0;
    if (num_cus(&cus)) return 1;
    const int blocks = cus * 16;
    if (sink_bytes < (size_t)blocks * 256 * 4) return fail("sink too small");
    const uint32_t lines = lines_pow2(table_bytes);
    float ms = 0.f;
    const int reps = 5;
    if (time_ms(s, reps, [&] {
            hipLaunchKernelGGL(lines_kernel, dim3(blocks), dim3(256), 0, s, static_cast<const uint32_t*>(table),
                               lines - 1, xcd_partition, lane_loads, static_cast<uint32_t*>(sink));
        }, &ms))
        return 1;
    *lines_per_s = (double)blocks * 256 * lane_loads * reps / (ms * 1e-3);
    return 0;
}

// Atomic line requests per second: groups of dwords_per_line (1, 2, 4, 8 or
// 16) lanes add to consecutive dwords of one pseudo-random line; one
// workgroup per CU, about 2^24 requests per launch, 5 timed launches.
int probe_atomic_lines(float* buf, size_t bytes, int dwords_per_line, double* requests_per_s, hipStream_t s)
{
    if (!buf || bytes < (64u << 10) || !requests_per_s) return fail("bad arguments");
    if (dwords_per_line < 1 || dwords_per_line > 16 || (dwords_per_line & (dwords_per_line - 1)))
        return fail("dwords_per_line must be 1, 2, 4, 8 or 16");
    int cus = 0;
    if (num_cus(&cus)) return 1;
    const uint32_t lines = lines_pow2(bytes);
    const long long lanes = (long long)cus * 256;
    const int iters = (int)std::max<long long>(1, ((1LL << 24) * dwords_per_line) / lanes);
    float ms = 0.f;
    const int reps = 5;
    if (time_ms(s, reps, [&] {
            hipLaunchKernelGGL(atomic_lines_kernel, dim3(cus), dim3(256), 0, s, buf, lines - 1, dwords_per_line,
                               iters);
        }, &ms))
        return 1;
    *requests_per_s = (double)lanes / dwords_per_line * iters * reps / (ms * 1e-3);
    return 0;
}

}  // extern "C"
