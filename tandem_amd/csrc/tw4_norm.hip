// RMSNorm and residual-add + RMSNorm of the decoder layer around the W4A16 projections, fp16 rows
// of K values (K % 512 == 0, K <= 8192), fp32 math:
//
//   tw4_rms_norm:      y = fp16(x rstd w),                  rstd = rsqrt(mean(x^2) + eps)
//   tw4_add_rms_norm:  s = x + r (fp32); r <- fp16(s); x <- fp16(s rstd w),  rstd from s (in place)
//
// One wavefront per row: lane l holds chunks (8 halves, 16 bytes) l, l + 64, ... of the row, all
// loaded before any math (J = K / 512 chunks per lane, kept in registers for the second pass). The
// sum of squares follows the fixed order of norm_rstd (per chunk, per quant group of 16 chunks, then
// over the groups), the same order as the decode kernels' fused norm prologue, so a fused
// projection sees the very bits this kernel writes. A decode batch is a few rows: the kernel is
// latency-bound (two dependent memory round trips), 4 rows per workgroup.
#include "tw4_common.h"

namespace tw4 {

constexpr int kNormMaxGroups = 64;  // K <= 8192

template <bool ADD, int J>
__global__ void __launch_bounds__(256) rms_norm_kernel(h1* x, h1* r, const h1* __restrict__ w, h1* y, int M, int K,
                                                       float eps) {  // y may be x: every store follows every load
    __shared__ float gsum[4][kNormMaxGroups];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + wave;
    if (row >= M) return;  // whole wavefronts; no workgroup barrier below
    const int64_t base = static_cast<int64_t>(row) * (K >> 3);
    u4* xr = reinterpret_cast<u4*>(x) + base;
    u4* rr = reinterpret_cast<u4*>(r) + base;
    const u4* wr = reinterpret_cast<const u4*>(w);
    u4 xv[J], rv[J], wv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        xv[j] = xr[64 * j + lane];
        if constexpr (ADD) rv[j] = rr[64 * j + lane];
        wv[j] = wr[64 * j + lane];
    }
    float* gs = gsum[wave];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        float s[8];
        chunk_to_f32(xv[j], s);
        if constexpr (ADD) {
            float b[8];
            chunk_to_f32(rv[j], b);
#pragma unroll
            for (int i = 0; i < 8; ++i) s[i] += b[i];
        }
        const float q = row16_sum(sumsq8(s));  // group 4 j + lane / 16
        if ((lane & 15) == 0) gs[4 * j + (lane >> 4)] = q;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float rstd = norm_rstd(gs, K >> 7, K, eps, lane);
    u4* yr = reinterpret_cast<u4*>(y) + base;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        float s[8], g[8];
        chunk_to_f32(xv[j], s);
        if constexpr (ADD) {
            float b[8];
            chunk_to_f32(rv[j], b);
#pragma unroll
            for (int i = 0; i < 8; ++i) s[i] += b[i];
            rr[64 * j + lane] = f32_to_chunk(s);
        }
        chunk_to_f32(wv[j], g);
#pragma unroll
        for (int i = 0; i < 8; ++i) s[i] = s[i] * rstd * g[i];
        yr[64 * j + lane] = f32_to_chunk(s);
    }
}

template <bool ADD>
int norm_launch(h1* x, h1* r, const h1* w, h1* y, int M, int K, float eps, hipStream_t st) {
    const unsigned grid = static_cast<unsigned>((M + 3) / 4);
    switch (K >> 9) {
#define TW4_NORM_CASE(J) \
    case J: rms_norm_kernel<ADD, J><<<grid, 256, 0, st>>>(x, r, w, y, M, K, eps); break;
        TW4_NORM_CASE(1) TW4_NORM_CASE(2) TW4_NORM_CASE(3) TW4_NORM_CASE(4) TW4_NORM_CASE(5)
        TW4_NORM_CASE(6) TW4_NORM_CASE(7) TW4_NORM_CASE(8) TW4_NORM_CASE(10) TW4_NORM_CASE(12)
        TW4_NORM_CASE(14) TW4_NORM_CASE(16)
#undef TW4_NORM_CASE
        default:
            tw4host::set_error("rms_norm: K = %d is not compiled (K / 512 in 1..8, 10, 12, 14, 16)", K);
            return TW4_EINVAL;
    }
    TW4_LAUNCH_CHECK("rms_norm: launch");
    return TW4_OK;
}

int norm_check(const void* x, const void* r, const void* w, const void* y, int M, int K, const char* who) {
    TW4_REQUIRE(x && r && w && y, TW4_EINVAL, "%s: null pointer", who);
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(r) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(w) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0,
                TW4_EINVAL, "%s: rows must be 16-byte aligned", who);
    TW4_REQUIRE(M >= 0, TW4_EINVAL, "%s: M >= 0 (M = %d)", who, M);
    TW4_REQUIRE(K >= 512 && K % 512 == 0 && K <= 8192, TW4_EINVAL, "%s: K %% 512 == 0 and K <= 8192 (K = %d)", who,
                K);
    return TW4_OK;
}

}  // namespace tw4

using namespace tw4;

extern "C" int tw4_rms_norm(const uint16_t* x, const uint16_t* weight, uint16_t* y, int M, int K, float eps,
                            void* stream) {
    int rc = norm_check(x, x, weight, y, M, K, "rms_norm");
    if (rc || M == 0) return rc;
    auto xp = const_cast<h1*>(reinterpret_cast<const h1*>(x));  // read only (ADD = false)
    return norm_launch<false>(xp, xp, reinterpret_cast<const h1*>(weight), reinterpret_cast<h1*>(y), M, K, eps,
                              static_cast<hipStream_t>(stream));
}

extern "C" int tw4_add_rms_norm(uint16_t* x, uint16_t* residual, const uint16_t* weight, int M, int K, float eps,
                                void* stream) {
    int rc = norm_check(x, residual, weight, x, M, K, "add_rms_norm");
    if (rc || M == 0) return rc;
    auto xp = reinterpret_cast<h1*>(x);
    return norm_launch<true>(xp, reinterpret_cast<h1*>(residual), reinterpret_cast<const h1*>(weight), xp, M, K, eps,
                             static_cast<hipStream_t>(stream));
}
