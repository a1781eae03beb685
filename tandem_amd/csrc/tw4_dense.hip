// Dense fp16 GEMV for small batches (the lm_head of a W4A16 model and other fp16 projections):
// y[M, N] = x[M, K] @ w[N, K]^T, M <= 8, w row-major (nn.Linear layout), fp32 accumulation.
//
// Bound by streaming w once. A workgroup owns a contiguous block of rows; each wavefront takes
// RB rows at a time and reads each row as K / 512 fully coalesced 1 KB wavefront loads (lane l
// holds chunks l, l + 64, ... of 8 halves, non-temporal). The next RB rows are in flight (second
// register set, loop unrolled by two) while the current ones are reduced. x is staged in LDS once
// per workgroup; lane l reads the same x chunks for every row, so per row it costs M LDS reads of
// 16 bytes per 16 weight bytes (x chunks are read once per row block and shared by its RB rows).
// Each lane accumulates its chunks with v_dot2_f32_f16; a row's 64 partial sums are added with
// DPP (within rows of 16 lanes) and two permlane swaps, and lane 0 writes the RB x M results.
//
// For M = 5 .. 8 the v_dot2 form reads M x 16 bytes of x from LDS per 16 weight bytes, which makes
// it LDS-bound; the matrix-core form (rows_inflight = 16 or 32: one or two 128-k chunks per step in
// flight) takes 16-row tiles of w as the A operand of v_mfma_f32_16x16x32_f16 and x as B, so one
// 16-byte B fragment serves 16 rows.
#include "tw4_common.h"

namespace tw4 {

// Sum over all 64 lanes, in every lane.
__device__ __forceinline__ float wave_sum(float v) {
    v += lane_xor1(v);
    v += lane_xor2(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
    return sum_rows(v);
}

template <int RB, int J>
struct RowSet {
    u4 w[RB][J];
};

template <int RB, int J>
__device__ __forceinline__ void load_rows(RowSet<RB, J>& rs, const u4* w, int64_t kc, int row, int last_row, int lane) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const u4* p = w + static_cast<int64_t>(min(row + rb, last_row)) * kc + lane;  // past the end: a valid row
#pragma unroll
        for (int j = 0; j < J; ++j) rs.w[rb][j] = load_stream(p + 64 * j);
    }
}

// Rows [row, row + RB) against x (LDS, [MT][K / 8] chunks; rows past M repeat row M - 1): lane 0
// stores y for tokens < M and rows < row_end.
template <bool PF, int M, int RB, int J>
__device__ __forceinline__ void rows_step(const RowSet<RB, J>& cur, RowSet<RB, J>& nxt, const u4* w, int64_t kc,
                                          const u4* xs, h1* y, int N, int Mx, int row, int row_end, int last_row,
                                          int lane) {
    if constexpr (PF) load_rows<RB, J>(nxt, w, kc, row + RB, last_row, lane);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch above the math
    float acc[RB][M];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[rb][m] = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const u4 xv = xs[m * kc + 64 * j + lane];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const u4 wv = cur.w[rb][j];
                float a = acc[rb][m];
                a = __builtin_amdgcn_fdot2(bitcast<h2>(wv.x), bitcast<h2>(xv.x), a, false);
                a = __builtin_amdgcn_fdot2(bitcast<h2>(wv.y), bitcast<h2>(xv.y), a, false);
                a = __builtin_amdgcn_fdot2(bitcast<h2>(wv.z), bitcast<h2>(xv.z), a, false);
                a = __builtin_amdgcn_fdot2(bitcast<h2>(wv.w), bitcast<h2>(xv.w), a, false);
                acc[rb][m] = a;
            }
        }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float v = wave_sum(acc[rb][m]);
            if (lane == 0 && m < Mx && row + rb < row_end) y[static_cast<int64_t>(m) * N + row + rb] = static_cast<h1>(v);
        }
}

// J = K / 512 chunk loads per lane and row (K <= 4096 here); M tokens of x in LDS, 1 <= Mx <= M.
template <int M, int RB, int J>
__global__ void __launch_bounds__(256) dense_gemv_kernel(const h1* __restrict__ x, const u4* __restrict__ w,
                                                         h1* __restrict__ y, int Mx, int N, int rows_per_wave) {
    extern __shared__ u4 xs[];
    constexpr int kc = 64 * J;  // 16-byte chunks per row
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = (blockIdx.x * 4 + wave) * rows_per_wave;
    const int row_end = min(row0 + rows_per_wave, N);
    const int nblk = row_end > row0 ? (row_end - row0 + RB - 1) / RB : 0;

    RowSet<RB, J> a, b;
    if (nblk > 0) load_rows<RB, J>(a, w, kc, row0, N - 1, lane);
    // x -> LDS, all waves of the workgroup (M kc chunks)
    const u4* xg = reinterpret_cast<const u4*>(x);
    for (int c = threadIdx.x; c < M * kc; c += 256) {
        const int m = c / kc;  // kc is a power of two
        xs[c] = xg[static_cast<int64_t>(min(m, Mx - 1)) * kc + (c - m * kc)];
    }
    __syncthreads();

    int i = 0;
    for (; i + 2 < nblk; i += 2) {
        rows_step<true, M, RB, J>(a, b, w, kc, xs, y, N, Mx, row0 + RB * i, row_end, N - 1, lane);
        rows_step<true, M, RB, J>(b, a, w, kc, xs, y, N, Mx, row0 + RB * (i + 1), row_end, N - 1, lane);
    }
    if (i + 2 == nblk) {
        rows_step<true, M, RB, J>(a, b, w, kc, xs, y, N, Mx, row0 + RB * i, row_end, N - 1, lane);
        rows_step<false, M, RB, J>(b, a, w, kc, xs, y, N, Mx, row0 + RB * (i + 1), row_end, N - 1, lane);
    } else if (i + 1 == nblk) {
        rows_step<false, M, RB, J>(a, b, w, kc, xs, y, N, Mx, row0 + RB * i, row_end, N - 1, lane);
    }
}

// ------------------------------------------------------------------------- matrix cores, M <= 8
// A wavefront owns rows_per_wave rows (whole 16-row tiles) and walks them tile by tile, each over
// all of K in chunks of 128 k. Lane (kb, r) loads, for word s = 0..3 of a chunk, the 16 bytes of
// row r at k = 128 c + 8 (4 s + kb) .. + 7 (one instruction per s: 64 contiguous bytes per row), and
// feeds them as A row r; the B fragment of token r is x at the same k from LDS, so each MFMA sums 32
// distinct k of the chunk. D chunks form a step: the next step's D chunks (possibly the next tile's
// first) are in flight in a second register set while the current ones are multiplied, 4 D KB per
// wavefront. D holds rows 4 kb + i of token r in lane (kb, r).
// x: 8 token rows in LDS (rows past M repeat row M - 1; B columns r >= 8 read row 7 and feed D
// columns that are never stored), row stride K / 8 + 1 chunks so the 16 rows of a fragment read hit
// different banks. Staged once per workgroup, its loads issued before the first weight chunks.
constexpr int kMmaWaves = 8;  // wavefronts per workgroup of the matrix-core form (one x copy each)

template <int D>
struct ChunkSet {
    u4 w[D][4];
};

// Plain (cached) loads: an instruction reads 64 bytes of each of 16 rows, half of a 128-byte line whose
// other half the next word's load reads (with non-temporal loads the tile ran 2 % slower).
template <int D>
__device__ __forceinline__ void load_chunks16(ChunkSet<D>& cs, const u4* wrow, int c, int kb) {
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int s = 0; s < 4; ++s) cs.w[d][s] = wrow[16 * (c + d) + 4 * s + kb];
}

template <bool PF, int D>
__device__ __forceinline__ void mma16_step(const ChunkSet<D>& cur, ChunkSet<D>& nxt, const u4* nrow, int nc,
                                           const u4* xr, int c, int kb, f4& acc) {
    if constexpr (PF) load_chunks16<D>(nxt, nrow, nc, kb);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch above the math
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int s = 0; s < 4; ++s)
            acc = mfma16x16x32(bitcast<h8>(cur.w[d][s]), bitcast<h8>(xr[16 * (c + d) + 4 * s + kb]), acc);
}

// J = K / 512 x chunks per thread for the staging (K <= 4096: at most 8); D = chunks per step, with
// 2 D <= 4 J (the K / 128 chunks of a row are a whole, even number of steps).
template <int J, int D>
__global__ void __launch_bounds__(kMmaWaves * 64) dense_mma_kernel(const h1* __restrict__ x, const u4* __restrict__ w,
                                                                   h1* __restrict__ y, int Mx, int N,
                                                                   int rows_per_wave) {
    extern __shared__ u4 xs[];
    constexpr int kc = 64 * J;  // 16-byte chunks per row of x and w
    constexpr int C = kc / 16;  // 128-k chunks per row
    static_assert(C % (2 * D) == 0, "a row is an even number of D-chunk steps");
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, kb = lane >> 4;
    const int row0 = (blockIdx.x * kMmaWaves + wave) * rows_per_wave;
    const int tiles = (max(min(rows_per_wave, N - row0), 0) + 15) >> 4;  // the last one may be partial
    const int last_tile = max(tiles - 1, 0);
    auto wrow = [&](int t) {  // this lane's row of tile t (rows past N read row N - 1)
        return w + static_cast<int64_t>(min(row0 + 16 * t + r, N - 1)) * kc;
    };

    // x staging: thread i takes chunks i, i + 512, ... (J of them) of the 8 x kc token-row image
    const u4* xg = reinterpret_cast<const u4*>(x);
    u4 xv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int f = threadIdx.x + kMmaWaves * 64 * j;  // < 8 kc
        const int m = f / kc;                            // kc is a power of two
        xv[j] = xg[static_cast<int64_t>(min(m, Mx - 1)) * kc + (f - m * kc)];
    }
    __builtin_amdgcn_sched_barrier(0);
    ChunkSet<D> a, b;
    load_chunks16<D>(a, wrow(0), 0, kb);  // tiles == 0: a valid row, never used
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int f = threadIdx.x + kMmaWaves * 64 * j;
        const int m = f / kc;
        xs[m * (kc + 1) + (f - m * kc)] = xv[j];
    }
    __syncthreads();

    const u4* xr = xs + min(r, 7) * (kc + 1);
    for (int t = 0; t < tiles; ++t) {
        const u4* cr = wrow(t);
        const u4* nr = wrow(min(t + 1, last_tile));  // the last tile prefetches its own first step: unused
        f4 acc = f4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int c = 0; c < C - 2 * D; c += 2 * D) {
            mma16_step<true, D>(a, b, cr, c + D, xr, c, kb, acc);
            mma16_step<true, D>(b, a, cr, c + 2 * D, xr, c + D, kb, acc);
        }
        mma16_step<true, D>(a, b, cr, C - D, xr, C - 2 * D, kb, acc);
        mma16_step<true, D>(b, a, nr, 0, xr, C - D, kb, acc);
        const int n = row0 + 16 * t + 4 * kb;
        if (r < Mx && n < N) {
            h1* yp = y + static_cast<int64_t>(r) * N + n;
            if (n + 3 < N && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0) {
                *reinterpret_cast<h4*>(yp) = h4{static_cast<h1>(acc.x), static_cast<h1>(acc.y),
                                                static_cast<h1>(acc.z), static_cast<h1>(acc.w)};
            } else {
                const float v[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (n + i < N) yp[i] = static_cast<h1>(v[i]);
            }
        }
    }
}

// Compiled (rows in flight RB, rows per wavefront) configurations.
#define TW4_DENSE_CONFIGS(X) X(1, 16) X(1, 32) X(2, 16) X(2, 32) X(2, 64) X(4, 32) X(4, 64)
// Matrix-core form (rows_inflight 16 D: 16-row tiles, D chunks of 128 k per step in flight): rows
// per wavefront, whole 16-row tiles.
// (4 chunks per step ran 5-30 % slower on the Qwen3 lm_heads: no configuration compiled.)
#define TW4_DENSE_MMA_CONFIGS(X) X(16, 16) X(16, 32) X(16, 64) X(16, 128) X(32, 16) X(32, 32)

template <int M, int RB, int J>
int dense_launch(const h1* x, const u4* w, h1* y, int Mx, int N, int rows_per_wave, hipStream_t st) {
    const int64_t waves = (static_cast<int64_t>(N) + rows_per_wave - 1) / rows_per_wave;
    const unsigned grid = static_cast<unsigned>((waves + 3) / 4);
    const size_t lds = static_cast<size_t>(M) * 64 * J * 16;  // <= 64 KB
    dense_gemv_kernel<M, RB, J><<<grid, 256, lds, st>>>(x, w, y, Mx, N, rows_per_wave);
    TW4_LAUNCH_CHECK("gemv_f16: launch");
    return TW4_OK;
}

template <int M, int RB>
int dense_by_k(const h1* x, const u4* w, h1* y, int Mx, int N, int K, int rows_per_wave, hipStream_t st) {
    switch (K >> 9) {
        case 1: return dense_launch<M, RB, 1>(x, w, y, Mx, N, rows_per_wave, st);
        case 2: return dense_launch<M, RB, 2>(x, w, y, Mx, N, rows_per_wave, st);
        case 4: return dense_launch<M, RB, 4>(x, w, y, Mx, N, rows_per_wave, st);
        case 8: return dense_launch<M, RB, 8>(x, w, y, Mx, N, rows_per_wave, st);
        default: break;
    }
    tw4host::set_error("gemv_f16: K = %d (K in 512, 1024, 2048, 4096)", K);
    return TW4_EINVAL;
}

template <int J, int D>
int dense_mma_launch(const h1* x, const u4* w, h1* y, int Mx, int N, int rows_per_wave, hipStream_t st) {
    const int64_t waves = (static_cast<int64_t>(N) + rows_per_wave - 1) / rows_per_wave;
    const unsigned grid = static_cast<unsigned>((waves + kMmaWaves - 1) / kMmaWaves);
    const size_t lds = static_cast<size_t>(8) * (64 * J + 1) * 16;  // <= 65.7 KB
    dense_mma_kernel<J, D><<<grid, kMmaWaves * 64, lds, st>>>(x, w, y, Mx, N, rows_per_wave);
    TW4_LAUNCH_CHECK("gemv_f16: launch");
    return TW4_OK;
}

template <int D>
int dense_mma(const h1* x, const u4* w, h1* y, int M, int N, int K, int rows_per_wave, hipStream_t st) {
    if (K / 128 < 2 * D) {
        tw4host::set_error("gemv_f16: rows in flight %d need K >= %d (K = %d)", 16 * D, 256 * D, K);
        return TW4_ECONFIG;
    }
    switch (K >> 9) {
        case 1: if constexpr (D <= 2) return dense_mma_launch<1, D>(x, w, y, M, N, rows_per_wave, st); break;
        case 2: return dense_mma_launch<2, D>(x, w, y, M, N, rows_per_wave, st);
        case 4: return dense_mma_launch<4, D>(x, w, y, M, N, rows_per_wave, st);
        case 8: return dense_mma_launch<8, D>(x, w, y, M, N, rows_per_wave, st);
        default: break;
    }
    tw4host::set_error("gemv_f16: K = %d (K in 512, 1024, 2048, 4096)", K);
    return TW4_EINVAL;
}

template <int RB>
int dense_by_m(const h1* x, const u4* w, h1* y, int M, int N, int K, int rows_per_wave, hipStream_t st) {
    if (M == 1) return dense_by_k<1, RB>(x, w, y, M, N, K, rows_per_wave, st);
    if (M == 2) return dense_by_k<2, RB>(x, w, y, M, N, K, rows_per_wave, st);
    if (M <= 4) return dense_by_k<4, RB>(x, w, y, M, N, K, rows_per_wave, st);
    return dense_by_k<8, RB>(x, w, y, M, N, K, rows_per_wave, st);  // token rows past M repeat row M - 1
}

}  // namespace tw4

using namespace tw4;

extern "C" int tw4_gemv_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, int M, int N, int K, int rows_inflight,
                            int rows_per_wave, void* stream) {
    TW4_REQUIRE(x && w && y, TW4_EINVAL, "gemv_f16: null pointer");
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0, TW4_EINVAL,
                "gemv_f16: x and w must be 16-byte aligned");
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(y) % 2 == 0, TW4_EINVAL, "gemv_f16: y must be 2-byte aligned");
    TW4_REQUIRE(M >= 1 && M <= 8, TW4_EINVAL, "gemv_f16: 1 <= M <= 8 (M = %d)", M);
    TW4_REQUIRE(N >= 1, TW4_EINVAL, "gemv_f16: N >= 1 (N = %d)", N);
    TW4_REQUIRE(K == 512 || K == 1024 || K == 2048 || K == 4096, TW4_EINVAL,
                "gemv_f16: K in 512, 1024, 2048, 4096 (K = %d)", K);
    auto xp = reinterpret_cast<const h1*>(x);
    auto wp = reinterpret_cast<const u4*>(w);
    auto yp = reinterpret_cast<h1*>(y);
    auto st = static_cast<hipStream_t>(stream);
#define TW4_DENSE_CASE(RB, RPW) \
    if (rows_inflight == RB && rows_per_wave == RPW) return dense_by_m<RB>(xp, wp, yp, M, N, K, RPW, st);
    TW4_DENSE_CONFIGS(TW4_DENSE_CASE)
#undef TW4_DENSE_CASE
#define TW4_DENSE_MMA_CASE(RB, RPW) \
    if (rows_inflight == RB && rows_per_wave == RPW) return dense_mma<RB / 16>(xp, wp, yp, M, N, K, RPW, st);
    TW4_DENSE_MMA_CONFIGS(TW4_DENSE_MMA_CASE)
#undef TW4_DENSE_MMA_CASE
    tw4host::set_error("gemv_f16: unsupported rows in flight / rows per wavefront %d / %d", rows_inflight,
                       rows_per_wave);
    return TW4_ECONFIG;
}

extern "C" int tw4_gemv_f16_configs(int* out, int max_configs) {
    int n = 0;
#define TW4_LIST(RB, RPW)                 \
    if (out && n < max_configs) {         \
        out[2 * n] = RB;                  \
        out[2 * n + 1] = RPW;             \
    }                                     \
    ++n;
    TW4_DENSE_CONFIGS(TW4_LIST)
    TW4_DENSE_MMA_CONFIGS(TW4_LIST)
#undef TW4_LIST
    return n;
}
