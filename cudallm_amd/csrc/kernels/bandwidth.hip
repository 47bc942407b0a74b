// Measured HBM stream-read bandwidth of this GPU: the second denominator of the roofline fractions
// (the first is MI355X's published 8 TB/s).  The quantity is the reference's "measured peak"
// (src/tools/cudallm_bandwidth.cpp:19-68, read_gbps_best); the kernel is this file's own.
//
// Each workgroup reads one contiguous slice of the buffer (consecutive DRAM pages per workgroup),
// every thread keeping U independent 128-bit non-temporal loads in flight.  The words are XOR-folded
// and written only if they hit a value that never occurs in the fill pattern, so the loads cannot be
// removed and the kernel writes nothing.
#include <algorithm>
#include <vector>

#include <hip/hip_ext.h>

#include "../kernels.h"
#include "device.h"

namespace cllm {
namespace {

constexpr int kBwThreads = 256;

template <int U>
__global__ void __launch_bounds__(kBwThreads) stream_read_kernel(const u32x4* src, size_t n16, size_t per_block,
                                                                 unsigned* sink) {
    const size_t begin = static_cast<size_t>(blockIdx.x) * per_block;
    const size_t end = begin + per_block < n16 ? begin + per_block : n16;
    unsigned acc = 0;
    for (size_t i = begin + threadIdx.x; i < end; i += static_cast<size_t>(kBwThreads) * U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t j = i + static_cast<size_t>(u) * kBwThreads;
            v[u] = j < end ? load_stream(src + j) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;  // never true for the 0x5a fill: keeps the loads
}

}  // namespace

void launch_stream_read(const void* src, size_t bytes, int blocks_per_cu, unsigned* sink, size_t sink_words,
                        hipStream_t s) {
    CLLM_REQUIRE(src && sink, "stream read: src and sink are required");
    CLLM_REQUIRE(bytes >= (1u << 20) && bytes % 16 == 0, "stream read: bytes must be >= 1 MiB and a multiple of 16");
    CLLM_REQUIRE(blocks_per_cu == 4 || blocks_per_cu == 8 || blocks_per_cu == 16, "stream read: blocks_per_cu is 4, 8 or 16");
    const int grid = blocks_per_cu * device_cu_count();
    CLLM_REQUIRE(sink_words >= static_cast<size_t>(grid), "stream read: sink needs blocks_per_cu x CUs words");
    const size_t n16 = bytes / 16, per_block = (n16 + grid - 1) / grid;
    const u32x4* p = static_cast<const u32x4*>(src);
    const KernelEvents ev = take_kernel_events();
    if (ev.start)
        hipExtLaunchKernelGGL(stream_read_kernel<8>, dim3(grid), dim3(kBwThreads), 0, s, ev.start, ev.stop, 0u, p, n16,
                              per_block, sink);
    else
        hipLaunchKernelGGL(stream_read_kernel<8>, dim3(grid), dim3(kBwThreads), 0, s, p, n16, per_block, sink);
    CLLM_HIP(hipGetLastError());
}

ReadBandwidth measure_read_bandwidth(size_t bytes, int reps) {
    CLLM_REQUIRE(bytes >= (64u << 20) && bytes % 16 == 0, "read bandwidth: bytes must be >= 64 MiB and a multiple of 16");
    CLLM_REQUIRE(reps >= 1 && reps <= 1000, "read bandwidth: reps must be 1..1000");
    const int cus = device_cu_count();
    const size_t n16 = bytes / 16;
    void* buf = nullptr;
    unsigned* sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    ReadBandwidth best{};
    auto cleanup = [&] {
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        if (buf) (void)hipFree(buf);
        if (sink) (void)hipFree(sink);
    };
    try {
        CLLM_HIP(hipMalloc(&buf, bytes));
        CLLM_HIP(hipMalloc(&sink, sizeof(unsigned) * 64 * static_cast<size_t>(cus)));
        CLLM_HIP(hipMemset(buf, 0x5a, bytes));
        CLLM_HIP(hipEventCreate(&e0));
        CLLM_HIP(hipEventCreate(&e1));
        const u32x4* src = static_cast<const u32x4*>(buf);
        // Launch shapes swept: workgroups per CU x loads in flight per thread.
        for (int per_cu : {4, 8, 16}) {
            for (int unroll : {4, 8}) {
                const int grid = per_cu * cus;
                const size_t per_block = (n16 + grid - 1) / grid;
                auto launch = [&] {
                    if (unroll == 4)
                        hipLaunchKernelGGL(stream_read_kernel<4>, dim3(grid), dim3(kBwThreads), 0, nullptr, src, n16,
                                           per_block, sink);
                    else
                        hipLaunchKernelGGL(stream_read_kernel<8>, dim3(grid), dim3(kBwThreads), 0, nullptr, src, n16,
                                           per_block, sink);
                    CLLM_HIP(hipGetLastError());
                };
                for (int w = 0; w < 2; ++w) launch();
                std::vector<double> gbps;
                for (int r = 0; r < reps; ++r) {
                    CLLM_HIP(hipEventRecord(e0, nullptr));
                    launch();
                    CLLM_HIP(hipEventRecord(e1, nullptr));
                    CLLM_HIP(hipEventSynchronize(e1));
                    float ms = 0.f;
                    CLLM_HIP(hipEventElapsedTime(&ms, e0, e1));
                    gbps.push_back(static_cast<double>(bytes) / (ms * 1e-3) / 1e9);
                }
                std::sort(gbps.begin(), gbps.end());
                if (gbps.back() > best.best_gbps) {
                    best.best_gbps = gbps.back();
                    best.median_gbps = gbps[gbps.size() / 2];
                    best.blocks_per_cu = per_cu;
                    best.loads_in_flight = unroll;
                }
            }
        }
    } catch (...) {
        cleanup();
        throw;
    }
    cleanup();
    return best;
}

}  // namespace cllm
