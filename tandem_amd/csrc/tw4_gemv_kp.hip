// The vector-ALU GEMV (M <= 4) compiled a second time with its kernel arguments preloaded into SGPRs
// (gfx950 loads the first kernel-argument dwords into user SGPRs before the wavefront starts, so its
// first instructions do not wait for an s_load of the arguments; tandem_amd/build.py passes
// -amdgpu-kernarg-preload-count for this file only). The kernel is tw4_decode.h's gemv_kernel; the
// copy only changes how a wavefront starts. Measured on MI355X it takes the small grids faster (Qwen3-8B
// qkv at M = 1 4.75 -> 4.40 us, o 3.79 -> 3.66 us) and the large ones level or slower (gate_up 10.2 ->
// 10.3 us), so the tables name it, as ("gemvk", warps_k, unroll, ntile), only where it won.
#include "tw4_decode.h"

namespace tw4 {

static int g_kp_ready[kMaxDevices];

// The same LDS set-up as the plain GEMV's (decode_prepare): x rows of large K need more than 64 KB.
int gemv_kp_prepare(int dev) {
    if (dev < 0 || dev >= kMaxDevices) {
        tw4host::set_error("init: device %d out of range", dev);
        return TW4_EINVAL;
    }
    if (g_kp_ready[dev]) return TW4_OK;
    int rc = TW4_OK;
#define TW4_KP_PREP(WK, U, T)                                                   \
    if (rc == TW4_OK) rc = allow_lds(gemv_kernel<1, WK, U, T, false, true>); \
    if (rc == TW4_OK) rc = allow_lds(gemv_kernel<2, WK, U, T, false, true>); \
    if (rc == TW4_OK) rc = allow_lds(gemv_kernel<3, WK, U, T, false, true>); \
    if (rc == TW4_OK) rc = allow_lds(gemv_kernel<4, WK, U, T, false, true>);
    TW4_DECODE_CONFIGS(TW4_KP_PREP)
#undef TW4_KP_PREP
    if (rc == TW4_OK) g_kp_ready[dev] = 1;
    return rc;
}

}  // namespace tw4

using namespace tw4;

int tw4_gemv_kp_prepare_device(int dev) { return gemv_kp_prepare(dev); }

extern "C" int tw4_gemv_kp(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                           uint16_t* y, int M, int N, int K, int warps_k, int unroll, int ntile, int act,
                           void* stream) {
    int rc = check_operands("gemv_kp", x, packed, scales, zeros, y, M, N, K);
    if (rc) return rc;
    TW4_REQUIRE(M >= 1 && M <= 4, TW4_EINVAL, "gemv_kp: 1 <= M <= 4 (M = %d; larger M: mma)", M);
    TW4_REQUIRE(K <= 65536, TW4_EINVAL, "gemv_kp: K <= 65536 (K = %d; larger K: mma)", K);
    TW4_REQUIRE(act == 0 || (act == 1 && N % 16 == 0), TW4_EINVAL,
                "gemv_kp: act 0, or 1 (SwiGLU) with N %% 16 == 0 (act = %d, N = %d)", act, N);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return tw4host::hip_fail(e, "gemv_kp: hipGetDevice");
    rc = gemv_kp_prepare(dev);
    if (rc) return rc;
    auto xp = reinterpret_cast<const h1*>(x);
    auto wp = reinterpret_cast<const u4*>(packed);
    auto sp = reinterpret_cast<const h1*>(scales);
    auto zp = reinterpret_cast<const h1*>(zeros);
    auto yp = reinterpret_cast<h1*>(y);
    auto st = static_cast<hipStream_t>(stream);
    const NormIn none{nullptr, nullptr, nullptr, 0.0f};
    switch (M) {
        case 1: return gemv_dispatch<1, false, true>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, none, st);
        case 2: return gemv_dispatch<2, false, true>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, none, st);
        case 3: return gemv_dispatch<3, false, true>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, none, st);
        default: return gemv_dispatch<4, false, true>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, none, st);
    }
}
