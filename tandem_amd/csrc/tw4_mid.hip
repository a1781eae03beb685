// Fused-dequant GEMM for batched decode, M <= 64 (tw4_gemm with stages = 1): HBM-bound like the
// decode kernels, with 1 to 4 token tiles per weight fragment and no x staging.
//
// Work unit = (tile group of NT row tiles, split s of `splits` contiguous quant-group ranges); one
// workgroup of WK wavefronts per unit, the wavefronts splitting the unit's groups into contiguous
// sub-ranges. Per group, a wavefront
//   - streams the NT weight blocks (one 16-byte non-temporal buffer load per lane and block, block
//     offset g * 1 KB in the scalar operand) and one 2-byte scale or zero per lane and tile (the
//     lanes of even kb load the scale, of odd kb the zero; v_permlane16_swap hands each lane both),
//   - loads the B fragments of x straight from L2 (x is M K 2 bytes, at most 1.5 MB here: it stays
//     resident in every XCD's L2), coalesced: load j of token tile b gives lane (kb, r) the 16 bytes
//     of token 16 b + r at k = 128 g + 32 j + 8 kb, so the four lanes of a token read 64 contiguous
//     bytes (one buffer load per (j, b), the group offset g * 256 bytes in the scalar operand); a
//     4 x 4 transpose across the lanes r, r + 16, r + 32, r + 48 (v_permlane32_swap, then
//     v_permlane16_swap, 16 per token tile and group) turns that into the MFMA order, lane (kb, r)
//     step s <-> k = 128 g + 32 kb + 8 s. (Loading the MFMA order directly spreads each load over
//     64 separate 64-byte segments of 16 rows, four times the L2 requests; measured, those loads
//     cost more than everything else of the kernel but the weight stream.)
//   - dequantizes word s of each block into A = fp16_rne((q - z) s) (16 rows x 32 k) and issues NT x
//     MT v_mfma_f32_16x16x32_f16 per step: every x fragment feeds NT tiles, every weight fragment MT
//     token tiles.
// The next group's weights, parameters AND x fragments are issued before the current group's math
// (two register sets, the loop unrolled by two so they swap roles without copies), so neither the
// HBM stream nor the L2 reads of x wait behind the math, and there is no workgroup barrier before
// the end. No LDS holds x: the unit needs no staging phase, and the grid is sized by the table to
// fill the GPU once.
// At the end the WK wavefronts add their sums in LDS (wavefront 0 keeps the total); with splits > 1
// the unit's fp32 partial goes to the split-K workspace and the last arriver of the tile group adds
// the partials in split order (finish_unit: deterministic, counters back to zero).
#include "tw4_common.h"

namespace tw4 {

template <int U, int NT, int MT>
struct MidSet {           // one chunk (U groups) of a wavefront's loads, per lane
    u4 w[U][NT];          // weight words (kb, r, s = 0..3) of each tile's block
    uint16_t p[U][NT];    // the row's scale (even kb) or zero (odd kb)
    u4 x[U][4][MT];       // x as loaded: load j of token tile b, token 16 b + r, k = 128 g + 32 j + 8 kb .. + 7
};

template <int NT, int MT>
struct MidStreams {
    __amdgpu_buffer_rsrc_t w[NT];  // tile's weight blocks: block g at byte g * 1024
    __amdgpu_buffer_rsrc_t x;      // x [M, K] fp16
    const uint16_t* p[NT];         // this lane's scale (even kb) or zero (odd kb) of (tile, group 0)
    int prow_stride[NT];           // scale / zero elements between consecutive groups of the tile
    int xoff[MT];                  // byte offset of (token 16 b + r, k = 8 kb) in x
    int lane;
};

// Even kb lanes hold the row's scale, odd kb lanes its zero: v_permlane16_swap exchanges rows 0 <-> 1
// and 2 <-> 3 of two copies, leaving the scales in the first result and the zeros in the second.
__device__ __forceinline__ GroupQ mid_group_q(uint16_t p, bool valid) {
    const auto sz = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(p), static_cast<uint32_t>(p), false, false);
    return group_q(valid ? as_h1(sz[0]) : static_cast<h1>(0.0f), as_h1(sz[1]));
}

// Lane (kb, r) holds v[j] = k octet 4 j + kb of its token (as loaded); afterwards v[s] = octet 4 kb + s.
// Two stages of 2 x 2 block swaps: lanes kb, kb + 2 exchange v[j + 2] / v[j] (v_permlane32_swap: the
// upper 32 lanes of the first operand with the lower 32 of the second), then lanes kb, kb + 1 exchange
// v[j + 1] / v[j] (v_permlane16_swap: odd rows of the first with even rows of the second).
__device__ __forceinline__ void octet_transpose(u4 (&v)[4]) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const auto p = __builtin_amdgcn_permlane32_swap(v[j][c], v[j + 2][c], false, false);
            v[j][c] = p[0];
            v[j + 2][c] = p[1];
        }
#pragma unroll
    for (int j = 0; j < 4; j += 2)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const auto p = __builtin_amdgcn_permlane16_swap(v[j][c], v[j + 1][c], false, false);
            v[j][c] = p[0];
            v[j + 1][c] = p[1];
        }
}

template <int U, int NT, int MT>
__device__ __forceinline__ void mid_load(MidSet<U, NT, MT>& d, const MidStreams<NT, MT>& ms, int g0, int glast) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int g = min(g0 + u, glast);  // past the range: a valid group, given scale 0 at use
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            d.w[u][t] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(ms.w[t], ms.lane * 16,
                                                                                     g * (kBlockU4 * 16), 2));
            d.p[u][t] = ms.p[t][static_cast<int64_t>(g) * ms.prow_stride[t]];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < MT; ++b)
                d.x[u][j][b] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(ms.x, ms.xoff[b] + 64 * j,
                                                                                            g * 256, 0));
    }
}

// One chunk: issue the next chunk's loads (PF), then the math of this one. FULL: all U groups of the
// chunk are in the wavefront's range.
template <bool PF, bool FULL, int U, int NT, int MT>
__device__ __forceinline__ void mid_chunk(const MidSet<U, NT, MT>& cur, MidSet<U, NT, MT>& nxt,
                                          const MidStreams<NT, MT>& ms, int g0, int ge, f4 (&acc)[NT][MT],
                                          uint32_t magic) {
    if constexpr (PF) mid_load<U, NT, MT>(nxt, ms, g0 + U, ge - 1);
    __builtin_amdgcn_sched_barrier(0);  // keep the loads above the math: the scheduler would sink them
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const bool valid = FULL || g0 + u < ge;
        GroupQ p[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) p[t] = mid_group_q(cur.p[u][t], valid);
        u4 xb[MT][4];  // B fragments: xb[b][s] = token 16 b + r, k = 128 g + 32 kb + 8 s .. + 7
#pragma unroll
        for (int b = 0; b < MT; ++b) {
#pragma unroll
            for (int j = 0; j < 4; ++j) xb[b][j] = cur.x[u][j][b];
            octet_transpose(xb[b]);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const h8 a = dequant_word(word_of(cur.w[u][t], s), p[t], magic);
#pragma unroll
                for (int b = 0; b < MT; ++b) acc[t][b] = mfma16x16x32(a, bitcast<h8>(xb[b][s]), acc[t][b]);
            }
        }
    }
}

template <int MT, int NT, int U, int WK>
__global__ void __launch_bounds__(WK * 64) mid_kernel(const h1* __restrict__ x, const u4* __restrict__ w,
                                                     const h1* __restrict__ scales, const h1* __restrict__ zeros,
                                                     h1* __restrict__ y, float* __restrict__ ws,
                                                     int* __restrict__ locks, int M, int N, int K, int splits,
                                                     int act) {
    extern __shared__ u4 lds[];  // [WK - 1][NT][MT][64] f4 partial sums, then the split-K flag
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, kb = lane >> 4;
    const int G = K >> 7, tiles = (N + 15) >> 4;
    const int unit = xcd_remap(blockIdx.x, gridDim.x);
    const int tg = unit / splits, split = unit - tg * splits;
    const int tile0 = tg * NT;
    const int glo = static_cast<int>(static_cast<int64_t>(split) * G / splits);
    const int R = static_cast<int>(static_cast<int64_t>(split + 1) * G / splits) - glo;
    const int gw = (R + WK - 1) / WK, gb = glo + min(wave * gw, R), ge = glo + min(wave * gw + gw, R);
    const int nch = (ge - gb + U - 1) / U;

    MidStreams<NT, MT> ms;
    ms.lane = lane;
    const uint16_t* pbase = reinterpret_cast<const uint16_t*>((lane & 16) ? zeros : scales);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int tt = min(tile0 + t, tiles - 1);  // tiles past the end recompute the last one; never stored
        const int rows_t = tile_rows(tt, N);
        ms.w[t] = __builtin_amdgcn_make_buffer_rsrc(const_cast<u4*>(w + static_cast<int64_t>(tt) * G * kBlockU4), 0,
                                                    G * kBlockU4 * 16, kBufferFlags);
        ms.p[t] = pbase + static_cast<int64_t>(16) * tt * G + min(r, rows_t - 1);
        ms.prow_stride[t] = rows_t;
    }
    // M K 2 < 2^31 (checked on the host), so every x offset fits the 32-bit buffer offsets
    ms.x = __builtin_amdgcn_make_buffer_rsrc(const_cast<h1*>(x), 0, M * K * 2, kBufferFlags);
#pragma unroll
    for (int b = 0; b < MT; ++b) ms.xoff[b] = (min(16 * b + r, M - 1) * K + 8 * kb) * 2;  // rows past M: the last
    const uint32_t magic = magic_reg();

    f4 acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int b = 0; b < MT; ++b) acc[t][b] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    MidSet<U, NT, MT> a, b2;
    mid_load<U, NT, MT>(a, ms, gb, max(ge - 1, glo));  // unconditional: an empty range loads a valid group
    int i = 0;
    for (; i + 2 < nch; i += 2) {
        mid_chunk<true, true, U, NT, MT>(a, b2, ms, gb + U * i, ge, acc, magic);
        mid_chunk<true, true, U, NT, MT>(b2, a, ms, gb + U * (i + 1), ge, acc, magic);
    }
    if (i + 2 == nch) {
        mid_chunk<true, true, U, NT, MT>(a, b2, ms, gb + U * i, ge, acc, magic);
        mid_chunk<false, false, U, NT, MT>(b2, a, ms, gb + U * (i + 1), ge, acc, magic);
    } else if (i + 1 == nch) {
        mid_chunk<false, false, U, NT, MT>(a, b2, ms, gb + U * i, ge, acc, magic);
    }

    if constexpr (WK > 1) {  // wavefront 0 collects the K sub-range sums
        f4* red = reinterpret_cast<f4*>(lds);
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int b = 0; b < MT; ++b) red[(((wave - 1) * NT + t) * MT + b) * 64 + lane] = acc[t][b];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int v = 0; v < WK - 1; ++v)
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int b = 0; b < MT; ++b) acc[t][b] += red[((v * NT + t) * MT + b) * 64 + lane];
        }
    }
    int* last_flag = reinterpret_cast<int*>(lds + (WK - 1) * NT * MT * 64);
    finish_unit<MT, NT, 1>(acc, wave == 0, 0, lane, tid, splits, tg, unit, ws, locks, *last_flag, y, M, N, 0, tile0,
                           tiles, act);
}

// Compiled configurations (MT, NT, U, WK).
#define TW4_MID_CONFIGS(X)                                                                                   \
    X(1, 2, 2, 8) X(1, 4, 1, 8) X(1, 4, 2, 4) X(1, 4, 2, 8) X(1, 8, 1, 8)                                   \
    X(2, 2, 1, 4) X(2, 2, 1, 8) X(2, 2, 2, 4) X(2, 2, 2, 8) X(2, 3, 1, 8) X(2, 4, 1, 4) X(2, 4, 1, 8) \
    X(2, 6, 1, 8) X(4, 2, 1, 4) X(4, 2, 1, 8)

template <int MT, int NT, int U, int WK>
constexpr int mid_lds_bytes() {
    return ((WK - 1) * NT * MT * 64 + 1) * 16;
}

template <int MT, int NT, int U, int WK>
int mid_prepare_one() {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(mid_kernel<MT, NT, U, WK>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, mid_lds_bytes<MT, NT, U, WK>());
    return e == hipSuccess ? TW4_OK : tw4host::hip_fail(e, "init: hipFuncSetAttribute (stages 1)");
}

template <int MT, int NT, int U, int WK>
int mid_launch(const h1* x, const u4* w, const h1* s, const h1* z, h1* y, float* ws, int* locks, int64_t ws_floats,
               int64_t n_locks, int M, int N, int K, int splits, int cus, int act, hipStream_t stream) {
    const int G = K >> 7, tiles = (N + 15) >> 4, groups = (tiles + NT - 1) / NT;
    TW4_REQUIRE(M <= 16 * MT, TW4_EINVAL, "gemm (stages 1): M %d > 16 mt = %d", M, 16 * MT);
    TW4_REQUIRE(static_cast<int64_t>(M) * K < (1LL << 30), TW4_EINVAL, "gemm (stages 1): M K < 2^30");
    constexpr int64_t kPart = static_cast<int64_t>(NT) * MT * 256;  // floats of one unit's partial
    int sp = splits;
    if (sp == 0) {  // enough units to give every CU one, within the default workspace (never the caller's)
        sp = 1;
        while (static_cast<int64_t>(groups) * sp < cus && sp < G &&
               static_cast<int64_t>(groups) * (sp + 1) * kPart <= TW4_AUTO_SPLIT_FLOATS &&
               groups <= TW4_AUTO_SPLIT_COUNTERS)
            ++sp;
    }
    TW4_REQUIRE(sp >= 1 && sp <= G, TW4_EINVAL, "gemm (stages 1): splits %d for %d groups", sp, G);
    if (sp > 1) {
        TW4_REQUIRE(ws && locks, TW4_EINVAL, "gemm: split-K needs a workspace and counters");
        TW4_REQUIRE(static_cast<int64_t>(groups) * sp * kPart <= ws_floats && groups <= n_locks, TW4_ESPACE,
                    "gemm: split-K workspace too small for %d tiles x %d splits", groups, sp);
    }
    const int64_t blocks = static_cast<int64_t>(groups) * sp;
    TW4_REQUIRE(blocks < (1LL << 31), TW4_EINVAL, "gemm: grid too large");
    mid_kernel<MT, NT, U, WK><<<static_cast<unsigned>(blocks), WK * 64, mid_lds_bytes<MT, NT, U, WK>(), stream>>>(
        x, w, s, z, y, ws, locks, M, N, K, sp, act);
    TW4_LAUNCH_CHECK("gemm (stages 1): launch");
    return TW4_OK;
}

}  // namespace tw4

using namespace tw4;

int tw4_gemm_mid_prepare(int /*dev*/) {
    int rc = TW4_OK;
#define TW4_MID_PREP(MT, NT, U, WK) \
    if (rc == TW4_OK) rc = mid_prepare_one<MT, NT, U, WK>();
    TW4_MID_CONFIGS(TW4_MID_PREP)
#undef TW4_MID_PREP
    return rc;
}

// Called by tw4_gemm for stages == 1 (warps_n is then U, the groups per prefetch chunk).
int tw4_gemm_mid_dispatch(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                          uint16_t* y, float* ws, int32_t* locks, int64_t ws_floats, int64_t n_locks, int M, int N,
                          int K, int mt, int nt, int unroll, int warps_k, int splits, int cus, int act, void* stream) {
    auto xp = reinterpret_cast<const h1*>(x);
    auto wp = reinterpret_cast<const u4*>(packed);
    auto sp = reinterpret_cast<const h1*>(scales);
    auto zp = reinterpret_cast<const h1*>(zeros);
    auto yp = reinterpret_cast<h1*>(y);
    auto st = static_cast<hipStream_t>(stream);
#define TW4_MID_CASE(MT, NT, U, WK)                                                                               \
    if (mt == MT && nt == NT && unroll == U && warps_k == WK)                                                     \
        return mid_launch<MT, NT, U, WK>(xp, wp, sp, zp, yp, ws, locks, ws_floats, n_locks, M, N, K, splits, cus, act, \
                                         st);
    TW4_MID_CONFIGS(TW4_MID_CASE)
#undef TW4_MID_CASE
    tw4host::set_error("gemm: unsupported stages-1 config mt / nt / unroll / warps_k %d / %d / %d / %d", mt, nt, unroll,
                       warps_k);
    return TW4_ECONFIG;
}

int tw4_gemm_mid_configs(int* out, int max_configs, int start) {
    int n = 0;
#define TW4_MID_LIST(MT, NT, U, WK)                  \
    if (out && start + n < max_configs) {            \
        out[5 * (start + n)] = MT;                   \
        out[5 * (start + n) + 1] = NT;               \
        out[5 * (start + n) + 2] = U;                \
        out[5 * (start + n) + 3] = WK;               \
        out[5 * (start + n) + 4] = 1;                \
    }                                                \
    ++n;
    TW4_MID_CONFIGS(TW4_MID_LIST)
#undef TW4_MID_LIST
    return n;
}
