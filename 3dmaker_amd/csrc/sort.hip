// Stable pair sort for the legacy Morton-ordered compaction (processRaysChunk,
// processRays.cu:357-464, which sorts with cub::DeviceRadixSort::SortPairs over
// all 32 key bits): rocPRIM's LSD radix sort, kept in its own translation unit
// because its templates dominate compile time.
#include "nerf.h"

#include <mutex>

#include <rocprim/device/device_radix_sort.hpp>

namespace graft {

namespace {
std::mutex g_sort_mu;
void* g_sort_tmp = nullptr;
size_t g_sort_bytes = 0;
}  // namespace

void sort_pairs_u32(const uint32_t* keys_in, uint32_t* keys_out, const uint32_t* values_in, uint32_t* values_out,
                    uint32_t n, hipStream_t s)
{
    if (n == 0) return;
    size_t bytes = 0;
    GRAFT_HIP_CHECK(rocprim::radix_sort_pairs(nullptr, bytes, keys_in, keys_out, values_in, values_out, n, 0u, 32u, s));
    std::lock_guard<std::mutex> lk(g_sort_mu);
    if (bytes > g_sort_bytes) {
        if (g_sort_tmp) GRAFT_HIP_CHECK(hipFree(g_sort_tmp));
        g_sort_tmp = nullptr;
        g_sort_bytes = 0;
        GRAFT_HIP_CHECK(hipMalloc(&g_sort_tmp, bytes));
        g_sort_bytes = bytes;
    }
    size_t have = g_sort_bytes;
    GRAFT_HIP_CHECK(
        rocprim::radix_sort_pairs(g_sort_tmp, have, keys_in, keys_out, values_in, values_out, n, 0u, 32u, s));
    // the temporary storage is shared by every caller: it is released to the
    // next one only after this sort has finished
    GRAFT_HIP_CHECK(hipStreamSynchronize(s));
}

}  // namespace graft
