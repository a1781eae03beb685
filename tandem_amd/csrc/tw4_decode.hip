// Decode kernels, M <= 16: y[M, N] = x[M, K] @ dequant(W)^T, bandwidth-bound on the int4 weights.
//
// A workgroup owns NT row tiles (16 rows each) and its WK wavefronts split K by quant groups:
// iteration i of wave w covers groups w + WK (u + UNROLL i), u = 0 .. UNROLL-1. Lane
// l = 16 kb + r streams the 16 bytes (kb, r, s = 0..3) of each (row tile, group) block with one
// non-temporal global_load_dwordx4: weights k = 128 g + 32 kb .. + 31 of row r. Weight blocks
// and their scales / zeros are loaded one iteration ahead into a second register set (the loop
// is unrolled by two so the sets swap roles without copies). Loads retire in issue order
// (vmcnt), so each iteration first issues what it needs now (x), then the next iteration's
// weights, then computes: waiting for x never waits for the prefetch. The partial sums of the
// WK wavefronts are added in LDS at the end.
//
//   gemv: vector ALUs, M <= 4. x [M, K] is copied to LDS once per workgroup (all 16 lanes of a
//         kb slice read the same 16 bytes: a broadcast). (q - z) is unpacked exactly to fp16
//         pairs and multiplied with x pairs by v_dot2_f32_f16 (fp32 accumulation); the group's
//         scale multiplies the lane's fp32 partial sum once per group. Row sums are finished
//         with two cross-lane exchanges (lanes r, r + 16, r + 32, r + 48 hold the four 32-k
//         slices of a group).
//   mma:  matrix cores, M <= 16. v_mfma_f32_16x16x32_f16 with the dequantized weights
//         fp16_rne((q - z) s) as A (16 rows x 32 k) and x as B (32 k x 16 batch columns, columns
//         >= M are zero). Step s of a block uses word s of every lane: lane (kb, r) feeds A row r
//         and B column r the weights / activations k = 128 g + 32 kb + 8 s .. + 7, the same k
//         permutation for both operands, so each MFMA sums 32 distinct k of the group. D holds
//         output rows 4 kb + i (i = 0..3) of batch column r in lane (kb, r).
//   act = 1 (mma): rows are in interleave_gate_up order, so the gate rows 4 kb + i (kb = 0, 1)
//         and up rows 8 + 4 kb + i of a feature sit in lanes l and l + 32; one cross-lane
//         exchange pairs them and the lane writes silu(gate) * up.
#include "tw4_common.h"

namespace tw4 {

template <int U, int NT>
struct WeightSet {  // one iteration's weight blocks and group parameters, per lane
    u4 w[U][NT];
    uint32_t s[U][NT], z[U][NT];
};

template <int U, int NT>
struct DecodeRows {
    const u4* wb[NT];   // this lane's 16-byte vector of group 0 of each row tile
    int64_t sb[NT];     // index of (row, group 0) in scales / zeros
};

template <int WK, int U, int NT>
__device__ __forceinline__ void load_weights(WeightSet<U, NT>& ws, const DecodeRows<U, NT>& rows,
                                             const h1* __restrict__ scales, const h1* __restrict__ zeros,
                                             int wave, int iter, int G) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int g = min(wave + WK * (u + U * iter), G - 1);  // clamped: loaded, never used
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            ws.w[u][t] = load_stream(rows.wb[t] + static_cast<int64_t>(g) * kBlockU4);
            ws.s[u][t] = load_u16(scales + rows.sb[t] + g);
            ws.z[u][t] = load_u16(zeros + rows.sb[t] + g);
        }
    }
}

// Rows past N (the zero padding of the last row tile) read row N - 1's scale and zero: loaded
// from a valid address, multiplied with zero weights, never stored.
template <int U, int NT>
__device__ __forceinline__ DecodeRows<U, NT> decode_rows(const u4* w, int tile0, int tiles, int N, int G, int lane) {
    DecodeRows<U, NT> rows;
    const int r = lane & 15;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int tt = min(tile0 + t, tiles - 1);  // tiles past the end recompute the last one; not stored
        rows.wb[t] = w + static_cast<int64_t>(tt) * G * kBlockU4 + lane;
        rows.sb[t] = static_cast<int64_t>(min(16 * tt + r, N - 1)) * G;
    }
    return rows;
}

// ------------------------------------------------------------------------------------ gemv
template <bool PF, int M, int WK, int U, int NT>
__device__ __forceinline__ void gemv_step(const WeightSet<U, NT>& cur, WeightSet<U, NT>& nxt,
                                          const DecodeRows<U, NT>& rows, const u4* xs, const h1* scales,
                                          const h1* zeros, float (&acc)[NT][M], int wave, int iter, int G,
                                          int K, int kb, uint32_t magic) {
    if constexpr (PF) load_weights<WK, U, NT>(nxt, rows, scales, zeros, wave, iter + 1, G);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch above the math: the scheduler would sink it
#pragma unroll
    for (int u = 0; u < U; ++u) {  // no branch: a group past G (the wavefront's last iteration) gets scale 0
        const int graw = wave + WK * (u + U * iter);
        const bool valid = graw < G;
        const int g = min(graw, G - 1);
        GroupQ p[NT];
        float part[NT][M];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            p[t] = group_q(as_h1(cur.s[u][t]), as_h1(cur.z[u][t]));
#pragma unroll
            for (int m = 0; m < M; ++m) part[t][m] = 0.0f;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            u4 xq[M];  // x[m][128 g + 32 kb + 8 s .. + 7]
#pragma unroll
            for (int m = 0; m < M; ++m) xq[m] = xs[m * (K >> 3) + 16 * g + 4 * kb + s];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                h2 d[4];
                unpack_qz(word_of(cur.w[u][t], s), p[t], magic, d);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    part[t][m] = __builtin_amdgcn_fdot2(d[0], bitcast<h2>(xq[m].x), part[t][m], false);
                    part[t][m] = __builtin_amdgcn_fdot2(d[1], bitcast<h2>(xq[m].y), part[t][m], false);
                    part[t][m] = __builtin_amdgcn_fdot2(d[2], bitcast<h2>(xq[m].z), part[t][m], false);
                    part[t][m] = __builtin_amdgcn_fdot2(d[3], bitcast<h2>(xq[m].w), part[t][m], false);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float sc = valid ? static_cast<float>(as_h1(cur.s[u][t])) : 0.0f;
#pragma unroll
            for (int m = 0; m < M; ++m) acc[t][m] = __builtin_fmaf(part[t][m], sc, acc[t][m]);
        }
    }
}

template <int M, int WK, int U, int NT>
__global__ void __launch_bounds__(WK * 64) gemv_kernel(const h1* __restrict__ x, const u4* __restrict__ w,
                                                      const h1* __restrict__ scales, const h1* __restrict__ zeros,
                                                      h1* __restrict__ y, int N, int K) {
    extern __shared__ u4 xs[];  // x [M][K] as 16-byte chunks
    __shared__ float red[WK][NT * M][16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, kb = lane >> 4;
    const int G = K >> 7, tiles = (N + 15) >> 4;
    const int tile0 = blockIdx.x * NT;
    const uint32_t magic = magic_reg();
    const DecodeRows<U, NT> rows = decode_rows<U, NT>(w, tile0, tiles, N, G, lane);
    const int iters = wave < G ? (G - wave + WK * U - 1) / (WK * U) : 0;

    WeightSet<U, NT> a, b;
    load_weights<WK, U, NT>(a, rows, scales, zeros, wave, 0, G);
    const int chunks = M * (K >> 3);
    for (int c = threadIdx.x; c < chunks; c += WK * 64) xs[c] = reinterpret_cast<const u4*>(x)[c];
    __syncthreads();

    float acc[NT][M];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[t][m] = 0.0f;
    // steady state: every step prefetches (no branch around the loads, so the waits stay exact);
    // the last step of the wavefront prefetches nothing
    int i = 0;
    for (; i + 2 < iters; i += 2) {
        gemv_step<true, M, WK, U, NT>(a, b, rows, xs, scales, zeros, acc, wave, i, G, K, kb, magic);
        gemv_step<true, M, WK, U, NT>(b, a, rows, xs, scales, zeros, acc, wave, i + 1, G, K, kb, magic);
    }
    if (i + 2 == iters) {
        gemv_step<true, M, WK, U, NT>(a, b, rows, xs, scales, zeros, acc, wave, i, G, K, kb, magic);
        gemv_step<false, M, WK, U, NT>(b, a, rows, xs, scales, zeros, acc, wave, i + 1, G, K, kb, magic);
    } else if (i + 1 == iters) {
        gemv_step<false, M, WK, U, NT>(a, b, rows, xs, scales, zeros, acc, wave, i, G, K, kb, magic);
    }
    // lanes r, r + 16, r + 32, r + 48 hold the four k slices of row r
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float v = acc[t][m];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            acc[t][m] = v;
        }
    if (WK > 1) {
        if (kb == 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int m = 0; m < M; ++m) red[wave][t * M + m][r] = acc[t][m];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int v = 1; v < WK; ++v)
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int m = 0; m < M; ++m) acc[t][m] += red[v][t * M + m][r];
    }
    if (kb != 0) return;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int row = 16 * (tile0 + t) + r;
        if (row >= N) continue;
#pragma unroll
        for (int m = 0; m < M; ++m) y[static_cast<int64_t>(m) * N + row] = static_cast<h1>(acc[t][m]);
    }
}

// ------------------------------------------------------------------------------------- mma
template <bool PF, int WK, int U, int NT>
__device__ __forceinline__ void mma_step(const WeightSet<U, NT>& cur, WeightSet<U, NT>& nxt,
                                         const DecodeRows<U, NT>& rows, const h8* xl,
                                         const h1* scales, const h1* zeros, f4 (&acc)[NT], int wave, int iter,
                                         int G, uint32_t magic) {
    h8 xb[U][4];  // issued first: waiting for it never waits for the prefetch below
#pragma unroll
    for (int u = 0; u < U; ++u) {
        // k = 128 g + 32 kb + 8 s .. + 7. Lanes past M read row 0: B column r only feeds D column
        // r, which is not stored for r >= M. A group past G (the wavefront's last iteration)
        // reads group G - 1 and gets scale 0 below. No selects or branches around the loads, so
        // the waits for x stay exact.
        const int g = min(wave + WK * (u + U * iter), G - 1);
#pragma unroll
        for (int s = 0; s < 4; ++s) xb[u][s] = xl[16 * g + s];
    }
    if constexpr (PF) load_weights<WK, U, NT>(nxt, rows, scales, zeros, wave, iter + 1, G);
    __builtin_amdgcn_sched_barrier(0);  // keep the loads above the math: the scheduler would sink them
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const bool valid = wave + WK * (u + U * iter) < G;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const GroupQ p = group_q(valid ? as_h1(cur.s[u][t]) : static_cast<h1>(0.0f), as_h1(cur.z[u][t]));
#pragma unroll
            for (int s = 0; s < 4; ++s)
                acc[t] = mfma16x16x32(dequant_word(word_of(cur.w[u][t], s), p, magic), xb[u][s], acc[t]);
        }
    }
}

template <int WK, int U, int NT>
__global__ void __launch_bounds__(WK * 64) mma_kernel(const h1* __restrict__ x, const u4* __restrict__ w,
                                                     const h1* __restrict__ scales, const h1* __restrict__ zeros,
                                                     h1* __restrict__ y, int M, int N, int K, int act) {
    __shared__ f4 red[WK > 1 ? WK - 1 : 1][NT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, kb = lane >> 4;
    const int G = K >> 7, tiles = (N + 15) >> 4;
    const int tile0 = blockIdx.x * NT;
    const uint32_t magic = magic_reg();
    const DecodeRows<U, NT> rows = decode_rows<U, NT>(w, tile0, tiles, N, G, lane);
    const int iters = wave < G ? (G - wave + WK * U - 1) / (WK * U) : 0;
    const h8* xl = reinterpret_cast<const h8*>(x + static_cast<int64_t>(r < M ? r : 0) * K + 32 * kb);

    WeightSet<U, NT> a, b;
    load_weights<WK, U, NT>(a, rows, scales, zeros, wave, 0, G);
    f4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    int i = 0;
    for (; i + 2 < iters; i += 2) {
        mma_step<true, WK, U, NT>(a, b, rows, xl, scales, zeros, acc, wave, i, G, magic);
        mma_step<true, WK, U, NT>(b, a, rows, xl, scales, zeros, acc, wave, i + 1, G, magic);
    }
    if (i + 2 == iters) {
        mma_step<true, WK, U, NT>(a, b, rows, xl, scales, zeros, acc, wave, i, G, magic);
        mma_step<false, WK, U, NT>(b, a, rows, xl, scales, zeros, acc, wave, i + 1, G, magic);
    } else if (i + 1 == iters) {
        mma_step<false, WK, U, NT>(a, b, rows, xl, scales, zeros, acc, wave, i, G, magic);
    }
    if (WK > 1) {
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t) red[wave - 1][t][lane] = acc[t];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int v = 0; v < WK - 1; ++v)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] += red[v][t][lane];
    }
    const int m = r;
    if (act) {  // N % 16 == 0 (checked on the host)
        const int half_n = N >> 1;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            f4 up;
            up.x = __shfl_xor(acc[t].x, 32);
            up.y = __shfl_xor(acc[t].y, 32);
            up.z = __shfl_xor(acc[t].z, 32);
            up.w = __shfl_xor(acc[t].w, 32);
            const int tt = tile0 + t;
            if (kb >= 2 || m >= M || tt >= tiles) continue;
            const int f = 8 * tt + 4 * kb;  // features f .. f + 3 of the [M, N/2] output
            const h4 o = h4{static_cast<h1>(silu(acc[t].x) * up.x), static_cast<h1>(silu(acc[t].y) * up.y),
                            static_cast<h1>(silu(acc[t].z) * up.z), static_cast<h1>(silu(acc[t].w) * up.w)};
            *reinterpret_cast<h4*>(y + static_cast<int64_t>(m) * half_n + f) = o;
        }
        return;
    }
    if (m >= M) return;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int n = 16 * (tile0 + t) + 4 * kb;  // N % 8 == 0: n < N implies n + 3 < N
        if (n >= N) continue;
        const h4 o = h4{static_cast<h1>(acc[t].x), static_cast<h1>(acc[t].y), static_cast<h1>(acc[t].z),
                        static_cast<h1>(acc[t].w)};
        *reinterpret_cast<h4*>(y + static_cast<int64_t>(m) * N + n) = o;
    }
}

// Compiled decode configurations (warps_k, unroll, ntile).
#define TW4_DECODE_CONFIGS(X) \
    X(1, 2, 1) X(1, 4, 1) X(2, 2, 1) X(2, 4, 1) X(4, 1, 1) X(4, 2, 1) X(4, 4, 1) X(8, 1, 1) X(8, 2, 1) \
    X(2, 2, 2) X(4, 1, 2) X(4, 2, 2) X(8, 1, 2) X(8, 2, 2) X(4, 4, 2) X(2, 4, 2) X(16, 1, 1) X(16, 2, 1)

constexpr int kMaxDevices = 64;
constexpr int kGemvMaxLds = 160 * 1024;  // gfx950 LDS per workgroup
static int g_decode_ready[kMaxDevices];

template <int M>
int gemv_prepare() {
#define TW4_GEMV_ATTR(WK, U, T)                                                                          \
    {                                                                                                    \
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gemv_kernel<M, WK, U, T>),      \
                                           hipFuncAttributeMaxDynamicSharedMemorySize,                   \
                                           kGemvMaxLds - static_cast<int>(sizeof(float)) * WK * T * M * 16); \
        if (e != hipSuccess) return tw4host::hip_fail(e, "init: gemv hipFuncSetAttribute");             \
    }
    TW4_DECODE_CONFIGS(TW4_GEMV_ATTR)
#undef TW4_GEMV_ATTR
    return TW4_OK;
}

int decode_prepare(int dev) {
    if (dev < 0 || dev >= kMaxDevices) {
        tw4host::set_error("init: device %d out of range", dev);
        return TW4_EINVAL;
    }
    if (g_decode_ready[dev]) return TW4_OK;
    int rc = gemv_prepare<1>();
    if (rc == TW4_OK) rc = gemv_prepare<2>();
    if (rc == TW4_OK) rc = gemv_prepare<3>();
    if (rc == TW4_OK) rc = gemv_prepare<4>();
    if (rc == TW4_OK) g_decode_ready[dev] = 1;
    return rc;
}

template <int M>
int gemv_dispatch(const h1* x, const u4* w, const h1* s, const h1* z, h1* y, int N, int K, int wk, int un, int nt,
                  hipStream_t st) {
    const int tiles = (N + 15) >> 4;
    const size_t lds = static_cast<size_t>(M) * K * 2;
#define TW4_GEMV_CASE(WK, U, T)                                                                     \
    if (wk == WK && un == U && nt == T) {                                                           \
        TW4_REQUIRE(lds + sizeof(float) * WK * T * M * 16 <= static_cast<size_t>(kGemvMaxLds), TW4_EINVAL, \
                    "gemv: x [%d, %d] does not fit in LDS (use mma)", M, K);                        \
        gemv_kernel<M, WK, U, T><<<(tiles + T - 1) / T, WK * 64, lds, st>>>(x, w, s, z, y, N, K);   \
        TW4_LAUNCH_CHECK("gemv: launch");                                                           \
        return TW4_OK;                                                                              \
    }
    TW4_DECODE_CONFIGS(TW4_GEMV_CASE)
#undef TW4_GEMV_CASE
    tw4host::set_error("gemv: unsupported warps_k / unroll / ntile %d / %d / %d", wk, un, nt);
    return TW4_ECONFIG;
}

int check_operands(const char* who, const void* x, const int32_t* packed, const uint16_t* scales,
                   const uint16_t* zeros, const void* y, int M, int N, int K) {
    TW4_REQUIRE(x && packed && scales && zeros && y, TW4_EINVAL, "%s: null pointer", who);
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0, TW4_EINVAL, "%s: x must be 16-byte aligned", who);
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(packed) % 16 == 0, TW4_EINVAL, "%s: packed must be 16-byte aligned", who);
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(y) % 8 == 0, TW4_EINVAL, "%s: y must be 8-byte aligned", who);
    TW4_REQUIRE(K > 0 && K % 128 == 0, TW4_EINVAL, "%s: K %% 128 == 0 (K = %d)", who, K);
    TW4_REQUIRE(N > 0 && N % 8 == 0, TW4_EINVAL, "%s: N %% 8 == 0 (N = %d)", who, N);
    return TW4_OK;
}

}  // namespace tw4

using namespace tw4;

int tw4_decode_prepare_device(int dev) { return decode_prepare(dev); }

extern "C" int tw4_gemv(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                        uint16_t* y, int M, int N, int K, int warps_k, int unroll, int ntile, void* stream) {
    int rc = check_operands("gemv", x, packed, scales, zeros, y, M, N, K);
    if (rc) return rc;
    TW4_REQUIRE(M >= 1 && M <= 4, TW4_EINVAL, "gemv: 1 <= M <= 4 (M = %d; larger M: mma)", M);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return tw4host::hip_fail(e, "gemv: hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices || !g_decode_ready[dev]) {
        rc = decode_prepare(dev);
        if (rc) return rc;
    }
    auto xp = reinterpret_cast<const h1*>(x);
    auto wp = reinterpret_cast<const u4*>(packed);
    auto sp = reinterpret_cast<const h1*>(scales);
    auto zp = reinterpret_cast<const h1*>(zeros);
    auto yp = reinterpret_cast<h1*>(y);
    auto st = static_cast<hipStream_t>(stream);
    switch (M) {
        case 1: return gemv_dispatch<1>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, st);
        case 2: return gemv_dispatch<2>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, st);
        case 3: return gemv_dispatch<3>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, st);
        default: return gemv_dispatch<4>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, st);
    }
}

extern "C" int tw4_mma(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                       uint16_t* y, int M, int N, int K, int warps_k, int unroll, int ntile, int act, void* stream) {
    int rc = check_operands("mma", x, packed, scales, zeros, y, M, N, K);
    if (rc) return rc;
    TW4_REQUIRE(M >= 1 && M <= 16, TW4_EINVAL, "mma: 1 <= M <= 16 (M = %d)", M);
    TW4_REQUIRE(act == 0 || (act == 1 && N % 16 == 0), TW4_EINVAL,
                "mma: act 0, or 1 (SwiGLU) with N %% 16 == 0 (act = %d, N = %d)", act, N);
    auto xp = reinterpret_cast<const h1*>(x);
    auto wp = reinterpret_cast<const u4*>(packed);
    auto sp = reinterpret_cast<const h1*>(scales);
    auto zp = reinterpret_cast<const h1*>(zeros);
    auto yp = reinterpret_cast<h1*>(y);
    auto st = static_cast<hipStream_t>(stream);
    const int tiles = (N + 15) >> 4;
#define TW4_MMA_CASE(WK, U, T)                                                                               \
    if (warps_k == WK && unroll == U && ntile == T) {                                                        \
        mma_kernel<WK, U, T><<<(tiles + T - 1) / T, WK * 64, 0, st>>>(xp, wp, sp, zp, yp, M, N, K, act);     \
        TW4_LAUNCH_CHECK("mma: launch");                                                                     \
        return TW4_OK;                                                                                       \
    }
    TW4_DECODE_CONFIGS(TW4_MMA_CASE)
#undef TW4_MMA_CASE
    tw4host::set_error("mma: unsupported warps_k / unroll / ntile %d / %d / %d", warps_k, unroll, ntile);
    return TW4_ECONFIG;
}
