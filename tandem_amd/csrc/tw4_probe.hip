// Streaming-read probe: the plain-read ceiling the bandwidth-bound decode kernels are measured
// against. It reads `bytes` from `src` with 16-byte non-temporal loads (each wavefront instruction
// 1 KB contiguous, 8 loads in flight per lane) and does no other work; the loaded words are XOR-folded
// and written to sink[0] only if the fold equals `key`, so the loads cannot be dropped and, for any
// other key, nothing is stored. Two orders: grid-stride (consecutive wavefronts of the whole grid
// read consecutive KB) and chunked (each workgroup reads one contiguous span, its wavefronts taking
// the span's KB blocks in turn: the order of the decode kernels, where a workgroup streams its row
// tiles' contiguous blocks).
#include "tw4_common.h"

namespace tw4 {

constexpr int kProbeThreads = 256;
constexpr int kProbeInflight = 8;  // 16-byte loads in flight per lane

__global__ void __launch_bounds__(kProbeThreads) read_probe_kernel(const u4* __restrict__ src, int64_t n16,
                                                                    uint32_t key, uint32_t* __restrict__ sink) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeThreads;
    uint32_t fold = 0;
    int64_t i = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
    for (; i + (kProbeInflight - 1) * stride < n16; i += kProbeInflight * stride) {
        u4 v[kProbeInflight];
#pragma unroll
        for (int j = 0; j < kProbeInflight; ++j) v[j] = load_stream(src + i + j * stride);
#pragma unroll
        for (int j = 0; j < kProbeInflight; ++j) fold ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    for (; i < n16; i += stride) {
        const u4 v = load_stream(src + i);
        fold ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (fold == key) sink[0] = fold;
}

__global__ void __launch_bounds__(kProbeThreads) read_probe_chunked_kernel(const u4* __restrict__ src, int64_t n16,
                                                                            int64_t span16, uint32_t key,
                                                                            uint32_t* __restrict__ sink) {
    constexpr int kWaves = kProbeThreads / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * span16;
    const int64_t hi = min(lo + span16, n16);
    uint32_t fold = 0;
    int64_t i = lo + 64 * wave + lane;  // 1 KB block (wave + kWaves j) of the span
    for (; i + (kProbeInflight - 1) * 64 * kWaves < hi; i += kProbeInflight * 64 * kWaves) {
        u4 v[kProbeInflight];
#pragma unroll
        for (int j = 0; j < kProbeInflight; ++j) v[j] = load_stream(src + i + j * 64 * kWaves);
#pragma unroll
        for (int j = 0; j < kProbeInflight; ++j) fold ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    for (; i < hi; i += 64 * kWaves) {
        const u4 v = load_stream(src + i);
        fold ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (fold == key) sink[0] = fold;
}

}  // namespace tw4

using namespace tw4;

extern "C" int tw4_read_probe(const void* src, int64_t bytes, int workgroups, int chunked, uint32_t key,
                              uint32_t* sink, void* stream) {
    TW4_REQUIRE(src && sink, TW4_EINVAL, "read_probe: null pointer");
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(src) % 16 == 0 && bytes > 0 && bytes % 16 == 0, TW4_EINVAL,
                "read_probe: src 16-byte aligned and bytes a positive multiple of 16");
    TW4_REQUIRE(workgroups >= 1 && workgroups <= (1 << 20), TW4_EINVAL, "read_probe: 1 <= workgroups <= 2^20");
    TW4_REQUIRE(chunked == 0 || chunked == 1, TW4_EINVAL, "read_probe: chunked 0 or 1");
    const int64_t n16 = bytes / 16;
    if (chunked) {
        const int64_t span16 = (n16 + workgroups - 1) / workgroups;
        read_probe_chunked_kernel<<<workgroups, kProbeThreads, 0, static_cast<hipStream_t>(stream)>>>(
            static_cast<const u4*>(src), n16, span16, key, sink);
    } else {
        read_probe_kernel<<<workgroups, kProbeThreads, 0, static_cast<hipStream_t>(stream)>>>(
            static_cast<const u4*>(src), n16, key, sink);
    }
    TW4_LAUNCH_CHECK("read_probe: launch");
    return TW4_OK;
}
