// Fused-dequant GEMM, M > 16 (prefill and batched decode): y[M, N] = x[M, K] @ dequant(W)^T.
//
// Workgroup tile: BM = 16 MT tokens x BN = 16 NT WN weight rows. Wavefront (wn, wk) owns the
// NT row tiles (nblk WN + wn) NT .. + NT - 1 and, of every K step, quant group step WK + wk.
//   x:       the workgroup's BM x 128 tile of each group goes global -> registers -> LDS, double
//            buffered (the next step's global loads are in flight while the current step
//            computes), one barrier per step. All WN wavefronts read it, so LDS carries the reuse.
//            16-byte chunk c of token row rho is stored at chunk c ^ (rho & 15): the 16 lanes of a
//            ds_read_b128 (rows rho = 16 b + r, same chunk) then touch 16 different chunks.
//   weights: each wavefront streams its own (row tile, group) blocks with one non-temporal
//            global_load_dwordx4 per lane, one step ahead in registers; no other wavefront of
//            the workgroup reads them, so they skip LDS.
//   math:    v_mfma_f32_16x16x32_f16, A = dequantized weights fp16_rne((q - z) s) (16 rows x
//            32 k), B = x (32 k x 16 tokens), the same k permutation as the decode kernels:
//            lane (kb, r), step s <-> k = 128 g + 32 kb + 8 s .. + 7. D lane (kb, r) = rows
//            4 kb + i of token r.
//   WK = 2:  the two K wavefronts add their sums in LDS at the end.
//   split-K: work units 0 .. dp - 1 are whole tiles; each later tile is shared by `splits` units
//            that take contiguous ranges of K steps. A unit stores its fp32 partial tile to ws
//            (agent-scope stores that write through the XCD's L2), then one agent-scope atomic on
//            the tile's counter tells the last arriver, which adds
//            the `splits` partials in split order (the result does not depend on arrival order),
//            writes y and returns the counter to zero for the next call.
//   act = 1: SwiGLU epilogue as in the decode kernel (gate rows 4 kb + i and up rows 8 + 4 kb + i
//            sit in lanes l and l + 32).
//   grid:    work units are re-numbered so that each XCD (workgroups are dealt to the 8 XCDs
//            round-robin) runs a contiguous range; tiles are ordered in bands of 8 token blocks,
//            token block fastest, so concurrently running workgroups of one XCD share weight
//            tiles in its L2.
#include <algorithm>
#include <type_traits>

#include "tw4_common.h"

// tw4_mid.hip: the stages-1 kernel (batched decode, 16 < M <= 64)
int tw4_gemm_mid_prepare(int dev);
int tw4_gemm_mid_dispatch(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                          uint16_t* y, float* ws, int32_t* locks, int64_t ws_floats, int64_t n_locks, int M, int N,
                          int K, int mt, int nt, int unroll, int warps_k, int splits, int cus, int act, void* stream);
int tw4_gemm_mid_configs(int* out, int max_configs, int start);

namespace tw4 {

template <int MT, int NT, int WN, int WK, int ST>
struct GemmCfg {
    static constexpr int BM = 16 * MT;
    static constexpr int BN = 16 * NT * WN;
    static constexpr int THREADS = WN * WK * 64;
    static constexpr int XCH = BM * 16;         // 16-byte chunks of one group's x tile
    static constexpr int STEP_CH = WK * XCH;    // chunks of one K step
    static constexpr int XIT = (STEP_CH + THREADS - 1) / THREADS;
    static constexpr int RING = 2 * STEP_CH * 16;
    static constexpr int RED = (WK - 1) * WN * NT * MT * 64 * 16;
    static constexpr int LDS = RING > RED ? RING : RED;
};


template <int MT, int NT, int WN, int WK, int ST>
__global__ void __launch_bounds__(WN * WK * 64) gemm_kernel(
    const h1* __restrict__ x, const u4* __restrict__ w, const h1* __restrict__ scales, const h1* __restrict__ zeros,
    h1* __restrict__ y, float* __restrict__ ws, int* __restrict__ locks, int M, int N, int K, int mb, int nb, int dp,
    int splits, int act) {
    using C = GemmCfg<MT, NT, WN, WK, ST>;
    extern __shared__ u4 lds[];
    __shared__ int last_flag;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave % WN, wk = wave / WN;
    const int r = lane & 15, kb = lane >> 4;
    const int G = K >> 7, tiles_n = (N + 15) >> 4;
    const int steps = (G + WK - 1) / WK;

    const int unit = xcd_remap(blockIdx.x, gridDim.x);
    const bool whole = unit < dp;
    const int su = unit - dp;
    const int tile = whole ? unit : dp + su / splits;
    const int split = whole ? 0 : su % splits;
    const int nsplit = whole ? 1 : splits;
    const int step0 = static_cast<int>(static_cast<int64_t>(split) * steps / nsplit);
    const int nst = static_cast<int>(static_cast<int64_t>(split + 1) * steps / nsplit) - step0;
    const int band = tile / (8 * nb), band_rows = min(mb - band * 8, 8), rin = tile - band * 8 * nb;
    const int mblk = band * 8 + rin % band_rows, nblk = rin / band_rows;
    const int m0 = mblk * C::BM;
    const int wt0 = (nblk * WN + wn) * NT;

    // x chunks of this thread: source offset (fp16 elements, group 0) and LDS slot offset (u4)
    int64_t xsrc[C::XIT];
    int xdst[C::XIT], xgrp[C::XIT];
#pragma unroll
    for (int it = 0; it < C::XIT; ++it) {
        const int c = min(it * C::THREADS + tid, C::STEP_CH - 1);
        const int u = c / C::XCH, cc = c % C::XCH, rho = cc >> 4, ch = cc & 15;
        xsrc[it] = static_cast<int64_t>(min(m0 + rho, M - 1)) * K + 8 * ch;
        xdst[it] = u * C::XCH + rho * 16 + (ch ^ (rho & 15));
        xgrp[it] = u;
    }
    // weight blocks and group parameters of this wavefront's row tiles
    const u4* wb[NT];
    int64_t sb[NT];  // tile-major scale / zero offset of group 0 (row r clamped to the tile: padding rows
    int srows[NT];   // have zero weights and are never stored), and the stride between groups
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int tt = min(wt0 + t, tiles_n - 1);
        wb[t] = w + static_cast<int64_t>(tt) * G * kBlockU4 + lane;
        srows[t] = tile_rows(tt, N);
        sb[t] = static_cast<int64_t>(16) * tt * G + min(r, srows[t] - 1);
    }
    const uint32_t magic = magic_reg();

    u4 xr[C::XIT];
    auto load_x = [&](int step) {
#pragma unroll
        for (int it = 0; it < C::XIT; ++it) {
            const int g = min(step * WK + xgrp[it], G - 1);
            xr[it] = *reinterpret_cast<const u4*>(x + xsrc[it] + 128 * g);
        }
    };
    auto store_x = [&](int slot) {
        u4* dst = lds + slot * C::STEP_CH;
#pragma unroll
        for (int it = 0; it < C::XIT; ++it)
            if (C::STEP_CH % C::THREADS == 0 || it * C::THREADS + tid < C::STEP_CH) dst[xdst[it]] = xr[it];
    };
    struct WSet {
        u4 w[NT];
        uint32_t s[NT], z[NT];
    };
    auto load_w = [&](int step, WSet& ws) {
        const int g = min(step * WK + wk, G - 1);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            ws.w[t] = load_stream(wb[t] + static_cast<int64_t>(g) * kBlockU4);
            ws.s[t] = load_u16(scales + sb[t] + static_cast<int64_t>(g) * srows[t]);
            ws.z[t] = load_u16(zeros + sb[t] + static_cast<int64_t>(g) * srows[t]);
        }
    };

    f4 acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int b = 0; b < MT; ++b) acc[t][b] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // One K step: issue the next step's x (then weight) loads, compute this step from LDS and
    // registers, park the next x tile in the other LDS slot, barrier. x is issued first, so the
    // wait before store_x does not wait for the weight prefetch.
    auto step_fn = [&](auto prefetch, int ls, const WSet& cur, WSet& nxt) {
        constexpr bool more = decltype(prefetch)::value;
        const int step = step0 + ls;
        if constexpr (more) {
            load_x(step + 1);
            load_w(step + 1, nxt);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch above the math: the scheduler would sink it
        {  // no branch: a group past G (WK = 2, odd G) gets scale 0
            const bool valid = step * WK + wk < G;
            const u4* xs = lds + (ls & 1) * C::STEP_CH + wk * C::XCH;
            GroupQ p[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t)
                p[t] = group_q(valid ? as_h1(cur.s[t]) : static_cast<h1>(0.0f), as_h1(cur.z[t]));
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                h8 xb[MT];
#pragma unroll
                for (int b = 0; b < MT; ++b) xb[b] = bitcast<h8>(xs[(16 * b + r) * 16 + ((4 * kb + s) ^ r)]);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const h8 a = dequant_word(word_of(cur.w[t], s), p[t], magic);
#pragma unroll
                    for (int b = 0; b < MT; ++b) acc[t][b] = mfma16x16x32(a, xb[b], acc[t][b]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (more) store_x((ls + 1) & 1);
        __syncthreads();
    };
    const std::true_type pf;
    const std::false_type last;

    WSet wa, wb2;
    load_x(step0);
    load_w(step0, wa);
    store_x(0);
    __syncthreads();
    // steady state: every step prefetches (no branch around the loads, so the waits stay exact);
    // the unit's last step prefetches nothing
    int ls = 0;
    for (; ls + 2 < nst; ls += 2) {
        step_fn(pf, ls, wa, wb2);
        step_fn(pf, ls + 1, wb2, wa);
    }
    if (ls + 2 == nst) {
        step_fn(pf, ls, wa, wb2);
        step_fn(last, ls + 1, wb2, wa);
    } else if (ls + 1 == nst) {
        step_fn(last, ls, wa, wb2);
    }

    if constexpr (WK > 1) {  // fold the K wavefronts wk > 0 into wk = 0 (the ring is free after the last barrier)
        f4* red = reinterpret_cast<f4*>(lds);
        if (wk > 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int b = 0; b < MT; ++b) red[((((wk - 1) * WN + wn) * NT + t) * MT + b) * 64 + lane] = acc[t][b];
        }
        __syncthreads();
        if (wk == 0) {
#pragma unroll
            for (int v = 1; v < WK; ++v)
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int b = 0; b < MT; ++b) acc[t][b] += red[((((v - 1) * WN + wn) * NT + t) * MT + b) * 64 + lane];
        }
    }

    finish_unit<MT, NT, WN>(acc, wk == 0, wn, lane, tid, nsplit, tile - dp, su, ws, locks, last_flag, y, M, N, m0, wt0,
                            tiles_n, act);
}

// ------------------------------------------------------------------------ resident-x streaming
// stages = 0: small-M variant. A work unit is one BM x BN output tile over one of `splits`
// contiguous K ranges (every tile is split). The unit's x rows (only the M - m0 that exist) over
// its whole K range are staged in LDS once, behind a single barrier; then every wavefront streams
// its NT row tiles' weight blocks over its own contiguous sub-range of groups (WK wavefronts split
// the unit's range) with U groups in flight ahead of the math in a second register set, like the
// decode kernels, and no further barrier. Each lane loads either the scale (even kb) or the zero
// (odd kb) of its row, one 2-byte load per tile and group; v_permlane16_swap hands every lane both.
// LDS x image: row rho, group j, 16-byte chunk c at ((rho R + j) 16 + (c ^ (rho & 15))), R groups per
// row, so the 16 rows of a B fragment read 16 different chunks.
template <int U, int NT>
struct StreamSet {
    u4 w[U][NT];
    uint16_t p[U][NT];  // scale (even kb) or zero (odd kb) of the lane's row (16 bits: no zero-extension
                        // that the compiler could place, with a wait for the load, before the main loop)
};

template <int MT, int NT, int WN, int WK, int U>
struct StreamCfg {
    static constexpr int BM = 16 * MT;
    static constexpr int BN = 16 * NT * WN;
    static constexpr int THREADS = WN * WK * 64;
    static constexpr int RED = (WK - 1) * WN * NT * MT * 64;  // u4 (f4) of the K-wavefront reduction
    static constexpr int XB = 8;                              // x chunks in flight per thread while staging
};

// LDS (u4) of a unit with `rows` x rows over `groups` groups.
template <int MT, int NT, int WN, int WK, int U>
__host__ __device__ __forceinline__ int stream_lds_u4(int rows, int groups) {
    using C = StreamCfg<MT, NT, WN, WK, U>;
    const int x = rows * groups * 16;
    return x > C::RED ? x : C::RED;
}

template <int U, int NT>
__device__ __forceinline__ void stream_load(StreamSet<U, NT>& ws, const u4* const (&wb)[NT], const uint16_t* const (&pb)[NT],
                                            const int (&srows)[NT], int g0, int glast) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int g = min(g0 + u, glast);  // past the range: a valid block, given scale 0 below
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            ws.w[u][t] = load_stream(wb[t] + static_cast<int64_t>(g) * kBlockU4);
            ws.p[u][t] = pb[t][static_cast<int64_t>(g) * srows[t]];
        }
    }
}

template <bool PF, int MT, int NT, int U>
__device__ __forceinline__ void stream_chunk(const StreamSet<U, NT>& cur, StreamSet<U, NT>& nxt, const u4* const (&wb)[NT],
                                             const uint16_t* const (&pb)[NT], const int (&srows)[NT],
                                             const u4* const (&xrow)[MT], const int (&xsw)[MT], int g0, int ge, int glo,
                                             f4 (&acc)[NT][MT], int kb, uint32_t magic) {
    if constexpr (PF) stream_load<U, NT>(nxt, wb, pb, srows, g0 + U, ge - 1);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch above the math: the scheduler would sink it
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int graw = g0 + u;
        const bool valid = graw < ge;
        const int j = min(graw, ge - 1) - glo;  // group within the unit's range
        GroupQ p[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const auto sz = __builtin_amdgcn_permlane16_swap(cur.p[u][t], cur.p[u][t], false, false);
            p[t] = group_q(valid ? as_h1(sz[0]) : static_cast<h1>(0.0f), as_h1(sz[1]));
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            h8 xb[MT];
#pragma unroll
            for (int b = 0; b < MT; ++b) xb[b] = bitcast<h8>(xrow[b][j * 16 + ((4 * kb + s) ^ xsw[b])]);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const h8 a = dequant_word(word_of(cur.w[u][t], s), p[t], magic);
#pragma unroll
                for (int b = 0; b < MT; ++b) acc[t][b] = mfma16x16x32(a, xb[b], acc[t][b]);
            }
        }
    }
}

template <int MT, int NT, int WN, int WK, int U>
__global__ void __launch_bounds__(WN * WK * 64) stream_kernel(
    const h1* __restrict__ x, const u4* __restrict__ w, const h1* __restrict__ scales, const h1* __restrict__ zeros,
    h1* __restrict__ y, float* __restrict__ ws, int* __restrict__ locks, int M, int N, int K, int mb, int nb,
    int splits, int act) {
    using C = StreamCfg<MT, NT, WN, WK, U>;
    extern __shared__ u4 lds[];
    __shared__ int last_flag;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave % WN, wk = wave / WN;
    const int r = lane & 15, kb = lane >> 4;
    const int G = K >> 7, tiles_n = (N + 15) >> 4;

    const int unit = xcd_remap(blockIdx.x, gridDim.x);
    const int tile = unit / splits, split = unit - tile * splits;
    const int glo = static_cast<int>(static_cast<int64_t>(split) * G / splits);
    const int ghi = static_cast<int>(static_cast<int64_t>(split + 1) * G / splits);
    const int R = ghi - glo;
    const int band = tile / (8 * nb), band_rows = min(mb - band * 8, 8), rin = tile - band * 8 * nb;
    const int mblk = band * 8 + rin % band_rows, nblk = rin / band_rows;
    const int m0 = mblk * C::BM;
    const int rows = min(C::BM, M - m0);  // x rows that exist
    const int wt0 = (nblk * WN + wn) * NT;

    // this wavefront's groups and weight / parameter streams
    const int gw = (R + WK - 1) / WK, gb = glo + min(wk * gw, R), ge = glo + min(wk * gw + gw, R);
    const int nch = (ge - gb + U - 1) / U;
    const u4* wb[NT];
    const uint16_t* pb[NT];
    int srows[NT];
    const uint16_t* pbase = reinterpret_cast<const uint16_t*>((lane & 16) ? zeros : scales);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int tt = min(wt0 + t, tiles_n - 1);  // tiles past the end recompute the last one; not stored
        wb[t] = w + static_cast<int64_t>(tt) * G * kBlockU4 + lane;
        srows[t] = tile_rows(tt, N);
        pb[t] = pbase + static_cast<int64_t>(16) * tt * G + min(r, srows[t] - 1);
    }
    const u4* xrow[MT];  // B column r of batch tile b = token row 16 b + r (rows past M read the last one)
    int xsw[MT];         // that row's chunk swizzle
#pragma unroll
    for (int b = 0; b < MT; ++b) {
        const int rho = min(16 * b + r, rows - 1);
        xrow[b] = lds + rho * R * 16;
        xsw[b] = rho & 15;
    }
    const uint32_t magic = magic_reg();

    // stage x[m0 .. m0 + rows - 1][groups glo .. ghi - 1]: flat chunk f -> (row f / (16 R), chunk
    // f % (16 R)); XB loads in flight per thread before their stores. The wavefront's first weight
    // chunk is issued right behind the first x batch, so its memory latency overlaps the staging
    // (loads retire in order: waiting for that batch never waits for the weights). No branch sits
    // around these loads; an empty group range loads a valid block that is never used.
    StreamSet<U, NT> a, b2;
    {
        const int r16 = 16 * R, total = rows * r16;
        const uint32_t magic16 = 0xFFFFFFFFu / static_cast<uint32_t>(r16) + 1u;  // f / r16 = umulhi(f, magic16)
        const u4* xg = reinterpret_cast<const u4*>(x);
        const int kx = K >> 3;
        auto load_batch = [&](int f0, u4 (&v)[C::XB], int (&dst)[C::XB]) {
#pragma unroll
            for (int i = 0; i < C::XB; ++i) {
                const int f = min(f0 + i * C::THREADS, total - 1);  // past the end: repeat the last chunk
                const int rho = static_cast<int>(__umulhi(static_cast<uint32_t>(f), magic16));
                const int c = f - rho * r16;
                v[i] = xg[static_cast<int64_t>(m0 + rho) * kx + 16 * glo + c];
                dst[i] = (rho * R + (c >> 4)) * 16 + ((c & 15) ^ (rho & 15));
            }
        };
        u4 v[C::XB];
        int dst[C::XB];
        load_batch(tid, v, dst);
        __builtin_amdgcn_sched_barrier(0);
        stream_load<U, NT>(a, wb, pb, srows, gb, max(ge - 1, 0));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < C::XB; ++i) lds[dst[i]] = v[i];
        for (int f0 = tid + C::XB * C::THREADS; f0 - tid < total; f0 += C::XB * C::THREADS) {  // uniform trip count
            load_batch(f0, v, dst);
#pragma unroll
            for (int i = 0; i < C::XB; ++i) lds[dst[i]] = v[i];
        }
    }
    __syncthreads();  // x staged

    f4 acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int bb = 0; bb < MT; ++bb) acc[t][bb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    int i = 0;
    for (; i + 2 < nch; i += 2) {
        stream_chunk<true, MT, NT, U>(a, b2, wb, pb, srows, xrow, xsw, gb + U * i, ge, glo, acc, kb, magic);
        stream_chunk<true, MT, NT, U>(b2, a, wb, pb, srows, xrow, xsw, gb + U * (i + 1), ge, glo, acc, kb, magic);
    }
    if (i + 2 == nch) {
        stream_chunk<true, MT, NT, U>(a, b2, wb, pb, srows, xrow, xsw, gb + U * i, ge, glo, acc, kb, magic);
        stream_chunk<false, MT, NT, U>(b2, a, wb, pb, srows, xrow, xsw, gb + U * (i + 1), ge, glo, acc, kb, magic);
    } else if (i + 1 == nch) {
        stream_chunk<false, MT, NT, U>(a, b2, wb, pb, srows, xrow, xsw, gb + U * i, ge, glo, acc, kb, magic);
    }

    if constexpr (WK > 1) {  // fold wavefronts wk > 0 into wk = 0 (x is no longer read after the barrier)
        __syncthreads();
        f4* red = reinterpret_cast<f4*>(lds);
        if (wk > 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int bb = 0; bb < MT; ++bb) red[((((wk - 1) * WN + wn) * NT + t) * MT + bb) * 64 + lane] = acc[t][bb];
        }
        __syncthreads();
        if (wk == 0) {
#pragma unroll
            for (int v = 1; v < WK; ++v)
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int bb = 0; bb < MT; ++bb)
                        acc[t][bb] += red[((((v - 1) * WN + wn) * NT + t) * MT + bb) * 64 + lane];
        }
    }
    finish_unit<MT, NT, WN>(acc, wk == 0, wn, lane, tid, splits, tile, unit, ws, locks, last_flag, y, M, N, m0, wt0,
                            tiles_n, act);
}

// Compiled GEMM configurations (MT, NT, WN, WK, ST).
#define TW4_GEMM_CONFIGS(X)                                                                               \
    X(1, 1, 4, 1, 2) X(1, 2, 4, 1, 2) X(2, 1, 4, 1, 2) X(2, 2, 4, 1, 2) X(2, 1, 4, 2, 2) X(2, 2, 4, 2, 2) \
    X(4, 1, 4, 1, 2) X(4, 2, 4, 1, 2) X(4, 2, 4, 2, 2) X(4, 4, 4, 1, 2) X(8, 1, 4, 1, 2) X(8, 2, 4, 1, 2) \
    X(8, 4, 4, 1, 2) X(8, 2, 2, 1, 2) X(4, 4, 2, 1, 2)

// Compiled resident-x streaming configurations (MT, NT, WN, WK), stages = 0; kStreamU groups in flight.
#define TW4_STREAM_CONFIGS(X)                                                                              \
    X(1, 2, 4, 1) X(1, 4, 4, 1) X(1, 2, 4, 2) X(2, 2, 4, 1) X(2, 4, 4, 1) X(2, 2, 4, 2) X(4, 2, 4, 1) X(4, 4, 4, 1) \
    X(4, 2, 4, 2) X(1, 2, 8, 1) X(2, 2, 8, 1)
constexpr int kStreamU = 2;
constexpr int kStreamAutoLds = 64 * 1024;  // splits = 0: the x slice of a unit stays within this
constexpr int kMaxLdsBytes = 160 * 1024 - 256;  // dynamic LDS: gfx950 has 160 KB per workgroup, minus the static flag

constexpr int kMaxDevices = 64;
#define TW4_COUNT(MT, NT, WN, WK, ST) +1
constexpr int kGemmConfigs = 0 TW4_GEMM_CONFIGS(TW4_COUNT);
#undef TW4_COUNT

struct DeviceInfo {
    int ready;
    int cus;
    int occupancy[kGemmConfigs];  // resident workgroups per CU
};
static DeviceInfo g_dev[kMaxDevices];

template <int MT, int NT, int WN, int WK, int ST>
int gemm_prepare(int dev, int index) {
    using C = GemmCfg<MT, NT, WN, WK, ST>;
    auto kern = gemm_kernel<MT, NT, WN, WK, ST>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
    if (e != hipSuccess) return tw4host::hip_fail(e, "init: hipFuncSetAttribute");
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, C::THREADS, C::LDS);
    if (e != hipSuccess) return tw4host::hip_fail(e, "init: hipOccupancyMaxActiveBlocksPerMultiprocessor");
    g_dev[dev].occupancy[index] = per_cu > 0 ? per_cu : 1;
    return TW4_OK;
}

thread_local int g_last_blocks = 0, g_last_dp = 0, g_last_splits = 0;

template <int MT, int NT, int WN, int WK, int ST>
int gemm_launch(int dev, int index, const h1* x, const u4* w, const h1* s, const h1* z, h1* y, float* ws,
                int* locks, int64_t ws_floats, int64_t n_locks, int M, int N, int K, int splits, int act,
                hipStream_t stream) {
    using C = GemmCfg<MT, NT, WN, WK, ST>;
    const int G = K >> 7, steps = (G + WK - 1) / WK;
    const int mb = (M + C::BM - 1) / C::BM, tiles_n = (N + 15) >> 4;
    const int nb = (tiles_n * 16 + C::BN - 1) / C::BN;
    const int64_t tiles64 = static_cast<int64_t>(mb) * nb;
    TW4_REQUIRE(tiles64 < (1LL << 30), TW4_EINVAL, "gemm: too many tiles (%lld)", static_cast<long long>(tiles64));
    const int tiles = static_cast<int>(tiles64);
    const int64_t tile_floats = static_cast<int64_t>(C::BM) * C::BN;
    int dp = tiles, sp = 1;
    if (splits == 0) {  // whole tiles for the full waves; split the last, partial wave along K
        const int slots = g_dev[dev].occupancy[index] * g_dev[dev].cus;
        const int rem = tiles % slots;
        double best = 1.0;  // s = 1: one more wave of whole tiles, in units of one tile's time
        for (int c = 2; c <= 8 && c <= steps && rem > 0; ++c) {
            // the budget is the default workspace, not the caller's, so the choice (and the bits) never
            // depend on the workspace size; one too small for it is refused below
            if (static_cast<int64_t>(rem) * c * tile_floats > TW4_AUTO_SPLIT_FLOATS || rem > TW4_AUTO_SPLIT_COUNTERS)
                break;
            // the split wave's time in tile units, plus a fix-up cost per extra split
            const double t = static_cast<double>((static_cast<int64_t>(rem) * c + slots - 1) / slots) / c + 0.02 * c;
            if (t < best) best = t, sp = c;
        }
        if (sp > 1) {
            dp = tiles - rem;
            TW4_REQUIRE(ws && locks, TW4_EINVAL, "gemm: split-K needs a workspace and counters");
            TW4_REQUIRE(static_cast<int64_t>(rem) * sp * tile_floats <= ws_floats && rem <= n_locks, TW4_ESPACE,
                        "gemm: split-K workspace too small for %d tiles x %d splits", rem, sp);
        }
    } else if (splits > 1) {
        TW4_REQUIRE(splits <= steps, TW4_EINVAL, "gemm: splits %d > K steps %d", splits, steps);
        TW4_REQUIRE(static_cast<int64_t>(tiles) * splits * tile_floats <= ws_floats && tiles <= n_locks, TW4_ESPACE,
                    "gemm: split-K workspace too small for %d tiles x %d splits", tiles, splits);
        dp = 0, sp = splits;
    }
    const int64_t blocks = dp + static_cast<int64_t>(tiles - dp) * sp;
    TW4_REQUIRE(blocks < (1LL << 31), TW4_EINVAL, "gemm: grid too large");
    g_last_blocks = static_cast<int>(blocks), g_last_dp = dp, g_last_splits = sp;
    gemm_kernel<MT, NT, WN, WK, ST><<<static_cast<unsigned>(blocks), C::THREADS, C::LDS, stream>>>(
        x, w, s, z, y, ws, locks, M, N, K, mb, nb, dp, sp, act);
    TW4_LAUNCH_CHECK("gemm: launch");
    return TW4_OK;
}

template <int MT, int NT, int WN, int WK>
int stream_prepare() {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(stream_kernel<MT, NT, WN, WK, kStreamU>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLdsBytes);
    if (e != hipSuccess) return tw4host::hip_fail(e, "init: hipFuncSetAttribute (stream)");
    return TW4_OK;
}

template <int MT, int NT, int WN, int WK>
int stream_launch(int dev, const h1* x, const u4* w, const h1* s, const h1* z, h1* y, float* ws, int* locks,
                  int64_t ws_floats, int64_t n_locks, int M, int N, int K, int splits, int act, hipStream_t stream) {
    using C = StreamCfg<MT, NT, WN, WK, kStreamU>;
    const int G = K >> 7;
    const int mb = (M + C::BM - 1) / C::BM, tiles_n = (N + 15) >> 4;
    const int nb = (tiles_n * 16 + C::BN - 1) / C::BN;
    const int64_t tiles64 = static_cast<int64_t>(mb) * nb;
    TW4_REQUIRE(tiles64 < (1LL << 26), TW4_EINVAL, "gemm: too many tiles (%lld)", static_cast<long long>(tiles64));
    const int tiles = static_cast<int>(tiles64);
    const int rows = M < C::BM ? M : C::BM;
    int sp = splits;
    if (sp == 0) {  // the fewest splits whose x slice fits the auto budget, then enough units for the GPU
        sp = 1;
        while (sp < G && 16LL * stream_lds_u4<MT, NT, WN, WK, kStreamU>(rows, (G + sp - 1) / sp) > kStreamAutoLds) ++sp;
        while (sp < G && static_cast<int64_t>(tiles) * sp < 2LL * g_dev[dev].cus) ++sp;
    }
    TW4_REQUIRE(sp >= 1 && sp <= G, TW4_EINVAL, "gemm: splits %d for %d groups", sp, G);
    const size_t lds = 16 * static_cast<size_t>(stream_lds_u4<MT, NT, WN, WK, kStreamU>(rows, (G + sp - 1) / sp));
    TW4_REQUIRE(lds <= static_cast<size_t>(kMaxLdsBytes), TW4_ECONFIG,
                "gemm: the x slice of %d rows x %d groups does not fit in LDS (stages 0: use more splits)", rows,
                (G + sp - 1) / sp);
    if (sp > 1) {
        TW4_REQUIRE(ws && locks, TW4_EINVAL, "gemm: split-K needs a workspace and counters");
        TW4_REQUIRE(static_cast<int64_t>(tiles) * sp * C::BM * C::BN <= ws_floats && tiles <= n_locks, TW4_ESPACE,
                    "gemm: split-K workspace too small for %d tiles x %d splits", tiles, sp);
    }
    const int64_t blocks = static_cast<int64_t>(tiles) * sp;
    g_last_blocks = static_cast<int>(blocks), g_last_dp = 0, g_last_splits = sp;
    stream_kernel<MT, NT, WN, WK, kStreamU><<<static_cast<unsigned>(blocks), C::THREADS, lds, stream>>>(
        x, w, s, z, y, ws, locks, M, N, K, mb, nb, sp, act);
    TW4_LAUNCH_CHECK("gemm: launch");
    return TW4_OK;
}

int device_prepare(int dev) {
    if (dev < 0 || dev >= kMaxDevices) {
        tw4host::set_error("init: device %d out of range", dev);
        return TW4_EINVAL;
    }
    if (g_dev[dev].ready) return TW4_OK;
    int cus = 0;
    hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return tw4host::hip_fail(e, "init: multiprocessor count");
    g_dev[dev].cus = cus;
    int index = 0, rc = TW4_OK;
#define TW4_PREP(MT, NT, WN, WK, ST) \
    if (rc == TW4_OK) rc = gemm_prepare<MT, NT, WN, WK, ST>(dev, index); \
    ++index;
    TW4_GEMM_CONFIGS(TW4_PREP)
#undef TW4_PREP
#define TW4_SPREP(MT, NT, WN, WK) \
    if (rc == TW4_OK) rc = stream_prepare<MT, NT, WN, WK>();
    TW4_STREAM_CONFIGS(TW4_SPREP)
#undef TW4_SPREP
    if (rc == TW4_OK) rc = tw4_gemm_mid_prepare(dev);
    if (rc == TW4_OK) g_dev[dev].ready = 1;
    return rc;
}

}  // namespace tw4

using namespace tw4;

int tw4_gemm_prepare_device(int dev) { return device_prepare(dev); }

// tw4_gemm_lds.hip: the stages-3 GEMM (weights and x staged in LDS by direct-to-LDS loads)
int tw4_gemm_lds_dispatch(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                          uint16_t* y, float* ws, int32_t* locks, int64_t ws_floats, int64_t n_locks, int M, int N,
                          int K, int mt, int nt, int warps_n, int warps_m, int splits, int cus, int act, void* stream);
int tw4_gemm_lds_configs(int* out, int max_configs, int start);

extern "C" int tw4_gemm(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                        uint16_t* y, float* ws, int32_t* locks, int64_t ws_floats, int64_t n_locks, int M, int N,
                        int K, int mt, int nt, int warps_n, int warps_k, int stages, int splits, int act,
                        void* stream) {
    TW4_REQUIRE(x && packed && scales && zeros && y, TW4_EINVAL, "gemm: null pointer");
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0, TW4_EINVAL, "gemm: x must be 16-byte aligned");
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(packed) % 16 == 0, TW4_EINVAL, "gemm: packed must be 16-byte aligned");
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(y) % 8 == 0, TW4_EINVAL, "gemm: y must be 8-byte aligned");
    TW4_REQUIRE(K > 0 && K % 128 == 0, TW4_EINVAL, "gemm: K %% 128 == 0 (K = %d)", K);
    TW4_REQUIRE(N > 0 && N % 8 == 0, TW4_EINVAL, "gemm: N %% 8 == 0 (N = %d)", N);
    TW4_REQUIRE(M >= 0, TW4_EINVAL, "gemm: M >= 0 (M = %d)", M);
    TW4_REQUIRE(act == 0 || (act == 1 && N % 16 == 0), TW4_EINVAL,
                "gemm: act 0, or 1 (SwiGLU) with N %% 16 == 0 (act = %d, N = %d)", act, N);
    TW4_REQUIRE(splits >= 0 && splits <= 16, TW4_EINVAL, "gemm: splits 0 (split the last wave) or 1 .. 16");
    TW4_REQUIRE(splits <= 1 || (ws && locks), TW4_EINVAL, "gemm: split-K needs a workspace and counters");
    TW4_REQUIRE(ws_floats >= 0 && n_locks >= 0, TW4_EINVAL, "gemm: workspace sizes must be >= 0");
    ws_floats = ws_floats < kMaxPartialFloats ? ws_floats : kMaxPartialFloats;  // the part split-K may use
    if (M == 0) return TW4_OK;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return tw4host::hip_fail(e, "gemm: hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices || !g_dev[dev].ready) {
        int rc = device_prepare(dev);
        if (rc) return rc;
    }
    if (splits == 0 && !(ws && locks)) splits = 1;
    if (stages == 1)
        return tw4_gemm_mid_dispatch(x, packed, scales, zeros, y, ws, locks, ws_floats, n_locks, M, N, K, mt, nt,
                                     warps_n, warps_k, splits, g_dev[dev].cus, act, stream);
    if (stages == 3)
        return tw4_gemm_lds_dispatch(x, packed, scales, zeros, y, ws, locks, ws_floats, n_locks, M, N, K, mt, nt,
                                     warps_n, warps_k, splits, g_dev[dev].cus, act, stream);
    auto xp = reinterpret_cast<const h1*>(x);
    auto wp = reinterpret_cast<const u4*>(packed);
    auto sp = reinterpret_cast<const h1*>(scales);
    auto zp = reinterpret_cast<const h1*>(zeros);
    auto yp = reinterpret_cast<h1*>(y);
    auto st = static_cast<hipStream_t>(stream);
    if (stages == 0) {
#define TW4_STREAM_CASE(MT, NT, WN, WK)                                                                       \
    if (mt == MT && nt == NT && warps_n == WN && warps_k == WK)                                                 \
        return stream_launch<MT, NT, WN, WK>(dev, xp, wp, sp, zp, yp, ws, locks, ws_floats, n_locks, M, N, K, splits, \
                                             act, st);
        TW4_STREAM_CONFIGS(TW4_STREAM_CASE)
#undef TW4_STREAM_CASE
    }
    int index = 0;
#define TW4_GEMM_CASE(MT, NT, WN, WK, ST)                                                                        \
    if (mt == MT && nt == NT && warps_n == WN && warps_k == WK && stages == ST)                                  \
        return gemm_launch<MT, NT, WN, WK, ST>(dev, index, xp, wp, sp, zp, yp, ws, locks, ws_floats, n_locks, M, \
                                               N, K, splits, act, st);                                           \
    ++index;
    TW4_GEMM_CONFIGS(TW4_GEMM_CASE)
#undef TW4_GEMM_CASE
    tw4host::set_error("gemm: unsupported mt / nt / warps_n / warps_k / stages %d / %d / %d / %d / %d", mt, nt,
                       warps_n, warps_k, stages);
    return TW4_ECONFIG;
}

extern "C" int tw4_gemm_last_grid(int* blocks, int* dp_tiles, int* splits) {
    if (blocks) *blocks = g_last_blocks;
    if (dp_tiles) *dp_tiles = g_last_dp;
    if (splits) *splits = g_last_splits;
    return TW4_OK;
}

extern "C" int tw4_gemm_configs(int* out, int max_configs) {
    int n = 0;
#define TW4_LIST(MT, NT, WN, WK, ST)      \
    if (out && n < max_configs) {         \
        out[5 * n] = MT;                  \
        out[5 * n + 1] = NT;              \
        out[5 * n + 2] = WN;              \
        out[5 * n + 3] = WK;              \
        out[5 * n + 4] = ST;              \
    }                                     \
    ++n;
    TW4_GEMM_CONFIGS(TW4_LIST)
#undef TW4_LIST
#define TW4_SLIST(MT, NT, WN, WK) TW4_LIST(MT, NT, WN, WK, 0)
#define TW4_LIST(MT, NT, WN, WK, ST)      \
    if (out && n < max_configs) {         \
        out[5 * n] = MT;                  \
        out[5 * n + 1] = NT;              \
        out[5 * n + 2] = WN;              \
        out[5 * n + 3] = WK;              \
        out[5 * n + 4] = ST;              \
    }                                     \
    ++n;
    TW4_STREAM_CONFIGS(TW4_SLIST)
#undef TW4_LIST
#undef TW4_SLIST
    n += tw4_gemm_lds_configs(out, max_configs, n);
    return n + tw4_gemm_mid_configs(out, max_configs, n);
}
