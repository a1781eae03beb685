// Streaming-read probe: the plain-read ceiling the bandwidth-bound decode kernels are measured
// against. It reads `bytes` from `src` with 16-byte non-temporal loads (each wavefront instruction
// 1 KB contiguous, D = 1, 2, 4 or 8 loads in flight per lane) and does no other work; the loaded words are XOR-folded
// and written to sink[0] only if the fold equals `key`, so the loads cannot be dropped and, for any
// other key, nothing is stored. Two orders: grid-stride (consecutive wavefronts of the whole grid
// read consecutive KB) and chunked (each workgroup reads one contiguous span, its wavefronts taking
// the span's KB blocks in turn: the order of the decode kernels, where a workgroup streams its row
// tiles' contiguous blocks).
#include "tw4_common.h"

namespace tw4 {

constexpr int kProbeThreads = 256;

// Every lane issues its next D loads before it folds any of them; a load past the end reads the last
// vector (a valid address) and is not folded, so there is no branch around a load and a lane with
// fewer vectors than D still has them all in flight at once.
template <int D>
__device__ __forceinline__ uint32_t probe_round(const u4* __restrict__ src, int64_t i, int64_t step, int64_t hi) {
    u4 v[D];
#pragma unroll
    for (int j = 0; j < D; ++j) v[j] = load_stream(src + min(i + j * step, hi - 1));
    uint32_t fold = 0;
#pragma unroll
    for (int j = 0; j < D; ++j) fold ^= i + j * step < hi ? v[j].x ^ v[j].y ^ v[j].z ^ v[j].w : 0u;
    return fold;
}

template <int D>
__global__ void __launch_bounds__(kProbeThreads) read_probe_kernel(const u4* __restrict__ src, int64_t n16,
                                                                    uint32_t key, uint32_t* __restrict__ sink) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeThreads;
    uint32_t fold = 0;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x; i < n16; i += D * stride)
        fold ^= probe_round<D>(src, i, stride, n16);
    if (fold == key) sink[0] = fold;
}

template <int D>
__global__ void __launch_bounds__(kProbeThreads) read_probe_chunked_kernel(const u4* __restrict__ src, int64_t n16,
                                                                            int64_t span16, uint32_t key,
                                                                            uint32_t* __restrict__ sink) {
    constexpr int kWaves = kProbeThreads / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * span16;
    const int64_t hi = min(lo + span16, n16);
    uint32_t fold = 0;
    // 1 KB blocks wave, wave + kWaves, ... of the span
    for (int64_t i = lo + 64 * wave + lane; i < hi; i += D * 64 * kWaves) fold ^= probe_round<D>(src, i, 64 * kWaves, hi);
    if (fold == key) sink[0] = fold;
}

template <int D>
void probe_launch(const u4* src, int64_t n16, int workgroups, int chunked, uint32_t key, uint32_t* sink,
                  hipStream_t stream) {
    if (chunked)
        read_probe_chunked_kernel<D><<<workgroups, kProbeThreads, 0, stream>>>(src, n16, (n16 + workgroups - 1) / workgroups,
                                                                             key, sink);
    else
        read_probe_kernel<D><<<workgroups, kProbeThreads, 0, stream>>>(src, n16, key, sink);
}

}  // namespace tw4

using namespace tw4;

extern "C" int tw4_read_probe(const void* src, int64_t bytes, int workgroups, int chunked, int inflight,
                              uint32_t key, uint32_t* sink, void* stream) {
    TW4_REQUIRE(src && sink, TW4_EINVAL, "read_probe: null pointer");
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(src) % 16 == 0 && bytes > 0 && bytes % 16 == 0, TW4_EINVAL,
                "read_probe: src 16-byte aligned and bytes a positive multiple of 16");
    TW4_REQUIRE(workgroups >= 1 && workgroups <= (1 << 20), TW4_EINVAL, "read_probe: 1 <= workgroups <= 2^20");
    TW4_REQUIRE(chunked == 0 || chunked == 1, TW4_EINVAL, "read_probe: chunked 0 or 1");
    const int64_t n16 = bytes / 16;
    const auto src16 = static_cast<const u4*>(src);
    const auto st = static_cast<hipStream_t>(stream);
    switch (inflight) {
        case 1: probe_launch<1>(src16, n16, workgroups, chunked, key, sink, st); break;
        case 2: probe_launch<2>(src16, n16, workgroups, chunked, key, sink, st); break;
        case 4: probe_launch<4>(src16, n16, workgroups, chunked, key, sink, st); break;
        case 8: probe_launch<8>(src16, n16, workgroups, chunked, key, sink, st); break;
        default: tw4host::set_error("read_probe: inflight 1, 2, 4 or 8 (got %d)", inflight); return TW4_EINVAL;
    }
    TW4_LAUNCH_CHECK("read_probe: launch");
    return TW4_OK;
}
