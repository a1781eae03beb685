// tw4_gemm_noalloc: the fused-dequant GEMM with its split-K workspace in a static device array, for
// callers that cannot allocate (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc). The kernels are tw4_gemm's; only where the partial sums and the tile counters live
// changes.
//
// `scratch` is one static device array per GPU the library runs on, held until the process ends:
//   [0, kScratchLockBytes)                int32 tile counters (kScratchLocks), zero between calls
//   [kScratchLockBytes, kScratchBytes)    fp32 split-K partial sums (kScratchFloats)
// In host code the name `scratch` only stands for the symbol: its device address comes from
// hipGetSymbolAddress, once per device with that device current, and only that address is used
// (kernel arguments, the counter clear). Every call on a GPU shares that GPU's array: calls that
// overlap on one GPU (two streams, or two host threads) race on it and must be serialized by the
// caller. The counters are cleared once, at set-up, by a fill kernel; each call's last arriver
// returns them to zero, so the array's float contents from the last call are never read again.
#include <mutex>

#include "tw4_common.h"

namespace tw4 {

constexpr int kScratchLocks = TW4_NOALLOC_COUNTERS;       // tiles a split call may use
constexpr int64_t kScratchFloats = TW4_NOALLOC_FLOATS;    // fp32 partials (32 MiB, the default workspace)
constexpr int64_t kScratchLockBytes = kScratchLocks * 4;
constexpr int64_t kScratchBytes = kScratchLockBytes + kScratchFloats * 4;
static_assert(kScratchLockBytes % 256 == 0, "partials stay 256-byte aligned");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
static void* g_scratch[kMaxScratchDevices];  // device address of `scratch` per GPU, null until set up
static std::mutex g_scratch_mu;

__global__ void clear_words(int* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

// Set-up for the current device `dev`: the array's address and its counters cleared on `stream`
// (ordered before any later launch on it). Called by tw4_init (outside graph capture, null stream,
// then synchronized) or by the first tw4_gemm_noalloc call on a device.
static int scratch_setup(int dev, hipStream_t stream, bool sync) {
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return tw4host::hip_fail(e, "noalloc: hipGetSymbolAddress(scratch)");
    TW4_REQUIRE(ptr != nullptr && reinterpret_cast<uintptr_t>(ptr) % 256 == 0, TW4_EHIP,
                "noalloc: scratch has no aligned device address");
    clear_words<<<16, 256, 0, stream>>>(static_cast<int*>(ptr), kScratchLocks);
    TW4_LAUNCH_CHECK("noalloc: clear counters");
    if (sync) {
        e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return tw4host::hip_fail(e, "noalloc: clear counters");
    }
    g_scratch[dev] = ptr;
    return TW4_OK;
}

}  // namespace tw4

using namespace tw4;

// tw4_init's part: called with `dev` current.
int tw4_noalloc_prepare_device(int dev) {
    TW4_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, TW4_EINVAL, "noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev]) return TW4_OK;
    return scratch_setup(dev, nullptr, true);
}

extern "C" int tw4_gemm_noalloc(const uint16_t* x, const int32_t* packed, const uint16_t* scales,
                                const uint16_t* zeros, uint16_t* y, int M, int N, int K, int mt, int nt, int warps_n,
                                int warps_k, int stages, int splits, int act, void* stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return tw4host::hip_fail(e, "noalloc: hipGetDevice");
    TW4_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, TW4_EINVAL, "noalloc: device %d out of range", dev);
    auto st = static_cast<hipStream_t>(stream);
    void* base = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (!g_scratch[dev]) {
            hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
            e = hipStreamIsCapturing(st, &cap);
            if (e != hipSuccess) return tw4host::hip_fail(e, "noalloc: hipStreamIsCapturing");
            TW4_REQUIRE(cap == hipStreamCaptureStatusNone, TW4_EINVAL,
                        "noalloc: call tw4_init(%d) before capturing tw4_gemm_noalloc (its scratch is set up there)",
                        dev);
            const int rc = scratch_setup(dev, st, false);
            if (rc) return rc;
        }
        base = g_scratch[dev];
    }
    int32_t* locks = static_cast<int32_t*>(base);
    float* ws = reinterpret_cast<float*>(static_cast<unsigned char*>(base) + kScratchLockBytes);
    const int rc = tw4_gemm(x, packed, scales, zeros, y, ws, locks, kScratchFloats, kScratchLocks, M, N, K, mt, nt,
                            warps_n, warps_k, stages, splits, act, stream);
    if (rc == TW4_ESPACE)
        tw4host::set_error("noalloc: split-K needs more than the static scratch (%lld fp32 partials, %d tile "
                           "counters) for M %d N %d K %d splits %d: use fewer splits, or tw4_gemm with a workspace",
                           static_cast<long long>(kScratchFloats), kScratchLocks, M, N, K, splits);
    return rc;
}
