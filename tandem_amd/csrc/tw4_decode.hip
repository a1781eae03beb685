// Decode kernels, M <= 64, and their C entry points: the matrix-core GEMV (gemvm) and decode kernel
// (mma, with its split-K and persistent forms), the host set-up, and tw4_gemv / tw4_gemv_act /
// tw4_decode_norm over the vector-ALU GEMV. tw4_decode.h holds the shared streaming code, the GEMV and
// the description of the kernels' layout and arithmetic.
#include "tw4_decode.h"

namespace tw4 {

// ----------------------------------------------------------------------------------- gemvm
// The GEMV's arithmetic on the matrix cores, M <= 16. A = the raw magic halves of a word (1024 + q,
// or 1024 + 16 q for the high nibbles: no zero point, no scale), B = x' (pairs 2, 3, 6, 7 divided
// by 16), so one v_mfma_f32_16x16x32_f16 does the 32 products that take 16 v_dot2 per batch row
// on the vector ALUs. The bias and the zero point come off in the accumulator's start value,
// D0 = -1024 A_g - z B_g (A_g / B_g: the group's sums of x' / x), and the group's scale after its
// four MFMAs: acc += s (D0 + sum (1024 + q) x'). The weights are exact (q - z) as in the GEMV
// (not the fp16-rounded (q - z) s of the mma kernel), so this is a GEMV-class kernel for tolerance
// purposes. Lane (kb, r) holds D rows 4 kb + i of batch column r: it loads the scales and zeros of
// rows 4 kb .. 4 kb + 3 with two 8-byte loads per group.
template <int U, int NT>
struct WeightSetM {
    u4 w[U][NT];
    u2 s[U][NT];  // fp16 scales of rows 4 kb .. 4 kb + 3
    u2 z[U][NT];  // fp16 zeros of the same rows
};

template <int U, int NT>
__device__ __forceinline__ void load_chunk_m(WeightSetM<U, NT>& ws, const TileStreams<NT>& ts, const uint16_t* s16,
                                             const uint16_t* z16, int g0, int glast, int kb) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int g = min(g0 + u, glast);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            ws.w[u][t] = load_block(ts.w[t], g, ts.lane);
            // rows 4 kb .. 4 kb + 3 of the tile; a short last tile (8 rows) reads rows 4 .. 7 for kb >= 2
            const int row0 = min(4 * kb, ts.rows[t] - 4);
            const int64_t off = ts.p[t] + static_cast<int64_t>(g) * ts.rows[t] + row0;
            ws.s[u][t] = *reinterpret_cast<const u2*>(s16 + off);
            ws.z[u][t] = *reinterpret_cast<const u2*>(z16 + off);
        }
    }
}

__host__ __device__ __forceinline__ int gemvm_gcorr_u4(int M, int K) { return (M * (K >> 7) * 8 + 15) / 16; }

// After staging: the group sums (-1024 A_g, B_g) of the wavefront's groups from the slice sums.
__device__ __forceinline__ void group_corr(const float2* corr, float2* gcorr, int G, int gb, int ge, int M, int lane) {
    const int n = (ge - gb) * M;
    for (int j = lane; j < n; j += 64) {
        const int m = j / (ge - gb), g = gb + (j - m * (ge - gb));
        const float2* c = corr + (m * G + g) * 4;
        gcorr[m * G + g] = float2{(c[0].x + c[1].x) + (c[2].x + c[3].x), (c[0].y + c[1].y) + (c[2].y + c[3].y)};
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <bool PF, int U, int NT>
__device__ __forceinline__ void gemvm_chunk(const WeightSetM<U, NT>& cur, WeightSetM<U, NT>& nxt,
                                            const TileStreams<NT>& ts, const uint16_t* s16, const uint16_t* z16,
                                            const u4* lx, const float2* gcorr, const DecodeLds& l, f4 (&acc)[NT],
                                            int xrow, int g0, int ge, int G, int kb, uint32_t magic) {
    if constexpr (PF) load_chunk_m<U, NT>(nxt, ts, s16, z16, g0 + U, ge - 1, kb);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch above the math
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int graw = g0 + u;  // a chunk that prefetches is not the last: all its groups are in range
        const bool valid = PF || graw < ge;
        const int g = PF ? graw : min(graw, ge - 1);
        const float2 gc = gcorr[xrow * G + g];
        h8 xb[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) xb[s] = bitcast<h8>(lx[xrow * l.xs + 16 * g + 4 * kb + s]);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const h4 z4 = bitcast<h4>(cur.z[u][t]);
            f4 d;
            d.x = __builtin_fmaf(-static_cast<float>(z4.x), gc.y, gc.x);
            d.y = __builtin_fmaf(-static_cast<float>(z4.y), gc.y, gc.x);
            d.z = __builtin_fmaf(-static_cast<float>(z4.z), gc.y, gc.x);
            d.w = __builtin_fmaf(-static_cast<float>(z4.w), gc.y, gc.x);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                h2 q[4];
                unpack_raw(word_of(cur.w[u][t], s), magic, q);
                const h8 a = h8{q[0].x, q[0].y, q[1].x, q[1].y, q[2].x, q[2].y, q[3].x, q[3].y};
                d = mfma16x16x32(a, xb[s], d);
            }
            if (valid) {
                const h4 s4 = bitcast<h4>(cur.s[u][t]);
                acc[t].x = __builtin_fmaf(static_cast<float>(s4.x), d.x, acc[t].x);
                acc[t].y = __builtin_fmaf(static_cast<float>(s4.y), d.y, acc[t].y);
                acc[t].z = __builtin_fmaf(static_cast<float>(s4.z), d.z, acc[t].z);
                acc[t].w = __builtin_fmaf(static_cast<float>(s4.w), d.w, acc[t].w);
            }
        }
    }
}

// M (1 .. 16, the columns of one B tile) is a kernel argument; ONE: M == 1, where the x staging needs
// no division by the row length.
template <bool ONE, int WK, int U, int NT>
__global__ void __launch_bounds__(WK * 64) gemvm_kernel(const h1* __restrict__ x, const u4* __restrict__ w,
                                                       const h1* __restrict__ scales, const h1* __restrict__ zeros,
                                                       h1* __restrict__ y, int M, int N, int K, int act) {
    extern __shared__ u4 smem[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: SGPR
    const int r = lane & 15, kb = lane >> 4;
    const int G = K >> 7, tiles = (N + 15) >> 4;
    const int tile0 = xcd_rotated_block((tiles + NT - 1) / NT) * NT;  // the launch's grid
    const DecodeLds l = decode_lds(true, M, K, gemv_corr_u4(M, K) + gemvm_gcorr_u4(M, K), (WK - 1) * NT * 64);
    const uint32_t magic = magic_reg();
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(scales);
    const uint16_t* z16 = reinterpret_cast<const uint16_t*>(zeros);
    TileStreams<NT> ts = tile_streams<NT>(w, s16, z16, tile0, tiles, N, G, lane);
    const int gw = (G + WK - 1) / WK, gb = min(wave * gw, G), ge = min(gb + gw, G);
    const int nch = (ge - gb + U - 1) / U;
    float2* corr = reinterpret_cast<float2*>(smem + l.corr);
    float2* gcorr = reinterpret_cast<float2*>(smem + l.corr + gemv_corr_u4(M, K));
    const int xrow = min(r, M - 1);  // B columns past M: any valid row, their D columns are not stored

    const int kx = K >> 3;
    const u4* xg = reinterpret_cast<const u4*>(x);
    const XSlice xsl = x_slice(gb, ge, M);
    WeightSetM<U, NT> a, b;
    {  // no branch around the first loads (see gemv_kernel); an empty slice reads valid addresses
        u4 xfirst[kXB];
        load_x_batch<ONE>(xfirst, xg, kx, xsl, lane);
        __builtin_amdgcn_sched_barrier(0);
        load_chunk_m<U, NT>(a, ts, s16, z16, gb, max(ge - 1, 0), kb);
        __builtin_amdgcn_sched_barrier(0);
        stage_x<true, ONE>(smem, l, corr, xg, kx, xsl, xfirst, lane);
        group_corr(corr, gcorr, G, gb, ge, M, lane);
    }

    f4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    int i = 0;
    for (; i + 2 < nch; i += 2) {
        gemvm_chunk<true, U, NT>(a, b, ts, s16, z16, smem, gcorr, l, acc, xrow, gb + U * i, ge, G, kb, magic);
        gemvm_chunk<true, U, NT>(b, a, ts, s16, z16, smem, gcorr, l, acc, xrow, gb + U * (i + 1), ge, G, kb, magic);
    }
    if (i + 2 == nch) {
        gemvm_chunk<true, U, NT>(a, b, ts, s16, z16, smem, gcorr, l, acc, xrow, gb + U * i, ge, G, kb, magic);
        gemvm_chunk<false, U, NT>(b, a, ts, s16, z16, smem, gcorr, l, acc, xrow, gb + U * (i + 1), ge, G, kb, magic);
    } else if (i + 1 == nch) {
        gemvm_chunk<false, U, NT>(a, b, ts, s16, z16, smem, gcorr, l, acc, xrow, gb + U * i, ge, G, kb, magic);
    }
    if (WK > 1) {
        f4* red = reinterpret_cast<f4*>(smem + l.red);  // [WK - 1][NT][64]
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t) red[((wave - 1) * NT + t) * 64 + lane] = acc[t];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int v = 0; v < WK - 1; ++v)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] += red[(v * NT + t) * 64 + lane];
    }
    if (act) {  // N % 16 == 0: gate rows 4 kb + i (kb = 0, 1) in lane l, up rows 8 + 4 kb + i in lane l + 32
        const int half_n = N >> 1;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int tt = tile0 + t;
            f4 up;
            up.x = lane_xor32(acc[t].x, lane);
            up.y = lane_xor32(acc[t].y, lane);
            up.z = lane_xor32(acc[t].z, lane);
            up.w = lane_xor32(acc[t].w, lane);
            if (kb >= 2 || r >= M || tt >= tiles) continue;
            const f4 g4 = acc[t];
            *reinterpret_cast<h4*>(y + static_cast<int64_t>(r) * half_n + 8 * tt + 4 * kb) =
                h4{static_cast<h1>(silu(g4.x) * up.x), static_cast<h1>(silu(g4.y) * up.y),
                   static_cast<h1>(silu(g4.z) * up.z), static_cast<h1>(silu(g4.w) * up.w)};
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int n = 16 * (tile0 + t) + 4 * kb;  // N % 8 == 0: n < N implies n + 3 < N
        if (n >= N || r >= M) continue;
        const f4 a4 = acc[t];
        *reinterpret_cast<h4*>(y + static_cast<int64_t>(r) * N + n) =
            h4{static_cast<h1>(a4.x), static_cast<h1>(a4.y), static_cast<h1>(a4.z), static_cast<h1>(a4.w)};
    }
}

// ------------------------------------------------------------------------------------- mma
// MT batch tiles of 16 columns (M <= 16 MT): lane (kb, r) feeds B column r of tile b = token
// 16 b + r, and D tile (t, b) holds rows 4 kb + i of that token. Each dequantized A fragment feeds
// MT MFMAs.
// Where the mma kernel reads its B fragments (x): straight from global memory at the start of each
// chunk, or from an LDS image staged once per wavefront, in batches of 2 (kXLds) or 8 (kXLdsWide)
// 16-byte chunks per lane. A batch is loaded before the first weight chunk; a later batch waits for
// that chunk too (loads retire in order), so the host takes the wide batch where a lane's share of the
// slice is more than 2 chunks and the narrow one where the extra, repeated loads would cost.
enum XMode { kXGlobal = 0, kXLds = 1, kXLdsWide = 2 };

// PF: load the next chunk, groups pg .. pg + U - 1 of the streams pts (the next chunk of this tile, or
// the first of the workgroup's next tile group), into nxt. FULL: all U groups of this chunk are in
// range (every chunk but a tile's last).
template <bool PF, int XM, int U, int NT, int MT, bool FULL = PF>
__device__ __forceinline__ void mma_chunk(const WeightSet<U, NT>& cur, WeightSet<U, NT>& nxt, const TileStreams<NT>& pts,
                                          int pg, const uint16_t* s16, const uint16_t* z16, const u4* smem,
                                          const DecodeLds& l, const h8* const (&xl)[MT], int xrow, f4 (&acc)[NT][MT],
                                          int g0, int ge, int glo, int kb, uint32_t magic) {
    h8 xb[XM == kXGlobal ? U : 1][4][MT];
    if constexpr (XM == kXGlobal) {  // issued first: waiting for x never waits for the prefetch below
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int g = min(g0 + u, ge - 1);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int b = 0; b < MT; ++b) xb[u][s][b] = xl[b][16 * g + s];  // k = 128 g + 32 kb + 8 s .. + 7
        }
    }
    if constexpr (PF) load_chunk<U, NT>(nxt, pts, s16, z16, pg, ge - 1);
    __builtin_amdgcn_sched_barrier(0);  // keep the loads above the math: the scheduler would sink them
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int graw = g0 + u;
        const bool valid = FULL || graw < ge;
        const int g = FULL ? graw : min(graw, ge - 1);
        GroupQ p[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            uint32_t s_raw, z_raw;
            scale_zero(cur.p[u][t], s_raw, z_raw);
            p[t] = group_q_raw(s_raw, z_raw, valid);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            h8 xv[MT];
#pragma unroll
            for (int b = 0; b < MT; ++b) {
                if constexpr (XM != kXGlobal)
                    xv[b] = bitcast<h8>(smem[xrow * l.xs + 16 * (g - glo) + 4 * kb + s]);
                else
                    xv[b] = xb[u][s][b];
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const h8 wa = dequant_word(word_of(cur.w[u][t], s), p[t], magic);
#pragma unroll
                for (int b = 0; b < MT; ++b) acc[t][b] = mfma16x16x32(wa, xv[b], acc[t][b]);
            }
        }
    }
}

// splits > 1: workgroup (tile group tg, split s) covers quant groups [s G / splits, (s + 1) G / splits)
// only, with x in LDS over that range alone, and the splits partial sums of a tile group are added by
// the last arriver (finish_unit: ws / locks, the GEMM's counter protocol).
// PERSIST: a grid smaller than the tile groups; workgroup u takes tile groups u, u + nunits, ...
// with x staged once, each wavefront prefetching the next tile group's first chunk during its last
// one. Two workgroup barriers per tile group guard the reduction buffer.
// The arguments the prologue needs (x, the weights, M, N, K, nsplit and nunits = gridDim.x) come first:
// they fill the 13 argument dwords preloaded into SGPRs, so no wavefront waits on a scalar load before
// its first weight load; y, act, the norm inputs and the split-K buffers are read later.
template <int WK, int U, int NT, int MT, int XM, bool NORM = false, bool SPLIT = false, bool PERSIST = false>
__global__ void __launch_bounds__(WK * 64) mma_kernel(const h1* __restrict__ x, const u4* __restrict__ w,
                                                     const h1* __restrict__ scales, const h1* __restrict__ zeros,
                                                     int M, int N, int K, int nsplit, int nunits,
                                                     h1* __restrict__ y, int act, NormIn nin,
                                                     float* __restrict__ ws, int* __restrict__ locks) {
    constexpr bool XLDS = XM != kXGlobal;
    constexpr int XB = XM == kXLdsWide ? 8 : 2;
    static_assert(!XLDS || MT == 1, "x in LDS: one batch tile");
    static_assert(!NORM || XLDS, "the fused norm stages x in LDS");
    static_assert(!SPLIT || (MT == 1 && !NORM), "split-K: one batch tile, no fused norm");
    static_assert(!PERSIST || (XLDS && !NORM && !SPLIT), "persistent: x in LDS, no fused norm, no split-K");
    const int splits = SPLIT ? nsplit : 1;  // a constant 1 where split-K is not compiled in
    if constexpr (U * MT > 4 && MT > 1) {
        return;  // register budget: never launched (tw4_mma rejects U * MT > 4 for M > 16)
    } else {
    extern __shared__ u4 smem[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: SGPR
    const int r = lane & 15, kb = lane >> 4;
    const int G = K >> 7, tiles = (N + 15) >> 4;
    const int unit = xcd_rotated_block(nunits), split = unit % splits;
    int tg = unit / splits;
    int tile0 = tg * NT;
    const int glo = split * G / splits, R = (split + 1) * G / splits - glo;  // this workgroup's quant groups
    const DecodeLds l = decode_lds(XLDS, M, 128 * R, 0, (WK - 1) * NT * MT * 64, NORM);
    const uint32_t magic = magic_reg();
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(scales);
    const uint16_t* z16 = reinterpret_cast<const uint16_t*>(zeros);
    TileStreams<NT> ts = tile_streams<NT>(w, s16, z16, tile0, tiles, N, G, lane);
    const int xrow = min(r, M - 1);  // B columns past M: any valid row, their D columns are not stored
    const h8* xl[MT];
#pragma unroll
    for (int b = 0; b < MT; ++b)
        xl[b] = reinterpret_cast<const h8*>(x + static_cast<int64_t>(min(16 * b + r, M - 1)) * K + 32 * kb);
    const int gw = (R + WK - 1) / WK, gb = glo + min(wave * gw, R), ge = glo + min(wave * gw + gw, R);
    const int nch = (ge - gb + U - 1) / U;

    WeightSet<U, NT> a, b;
    const int kx = K >> 3;
    const u4* xg = reinterpret_cast<const u4*>(x) + 16 * glo;  // the LDS image starts at group glo
    const XSlice xsl = x_slice(gb - glo, ge - glo, M);
    if constexpr (XLDS) {
        if constexpr (NORM) {  // no branch around these loads (see stage_x_norm)
            u4 fx[kXB], fr[kXB], fw[kXB];
            load_norm_batch<false, true>(fx, fr, fw, xg, nin.r ? reinterpret_cast<const u4*>(nin.r) : xg,
                                         reinterpret_cast<const u4*>(nin.w), kx, xsl, lane);
            __builtin_amdgcn_sched_barrier(0);
            load_chunk<U, NT>(a, ts, s16, z16, gb, max(ge - 1, 0));
            __builtin_amdgcn_sched_barrier(0);
            stage_x_norm<false, false, kNormMaxRows>(smem, l, nullptr, xg, kx, xsl, nin, M, G, K, fx, fr, fw, lane);
        } else {  // no branch around the first loads (see gemv_kernel)
            u4 xfirst[XB];
            load_x_batch<false, XB>(xfirst, xg, kx, xsl, lane);
            __builtin_amdgcn_sched_barrier(0);
            load_chunk<U, NT>(a, ts, s16, z16, gb, max(ge - 1, 0));
            __builtin_amdgcn_sched_barrier(0);
            stage_x<false, false, XB>(smem, l, nullptr, xg, kx, xsl, xfirst, lane);
        }
    } else {
        load_chunk<U, NT>(a, ts, s16, z16, gb, max(ge - 1, 0));
    }

    const int ngroups = (tiles + NT - 1) / NT;
    for (int pass = 0;; ++pass) {  // one pass per tile group (PERSIST: several)
    const int tg_next = tg + nunits;
    const bool more = PERSIST && tg_next < ngroups;  // uniform across the workgroup
    // The streams the pass's last chunk prefetches from. Last pass: weight blocks of an empty buffer
    // range (out-of-range buffer loads return zeros without a memory access) and the group
    // parameters the chunk itself has just loaded (cache hits).
    TileStreams<NT> tsn = ts;
    if constexpr (PERSIST) {
        if (more) {
            tsn = tile_streams<NT>(w, s16, z16, tg_next * NT, tiles, N, G, lane);
        } else {
#pragma unroll
            for (int t = 0; t < NT; ++t)
                tsn.w[t] = __builtin_amdgcn_make_buffer_rsrc(const_cast<u4*>(w), 0, 0, kBufferFlags);
        }
    }
    f4 acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int bb = 0; bb < MT; ++bb) acc[t][bb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    int i = 0;
    for (; i + 2 < nch; i += 2) {
        mma_chunk<true, XM, U, NT, MT>(a, b, ts, gb + U * (i + 1), s16, z16, smem, l, xl, xrow, acc, gb + U * i, ge,
                                       glo, kb, magic);
        mma_chunk<true, XM, U, NT, MT>(b, a, ts, gb + U * (i + 2), s16, z16, smem, l, xl, xrow, acc, gb + U * (i + 1),
                                       ge, glo, kb, magic);
    }
    // A tile's last chunk. PERSIST: it prefetches the next tile group's first chunk, which the next
    // pass finds in a (on the last pass: nothing from memory, see tsn).
    if (i + 2 == nch) {
        mma_chunk<true, XM, U, NT, MT>(a, b, ts, gb + U * (i + 1), s16, z16, smem, l, xl, xrow, acc, gb + U * i, ge,
                                       glo, kb, magic);
        mma_chunk<PERSIST, XM, U, NT, MT, false>(b, a, tsn, more ? gb : gb + U * (i + 1), s16, z16, smem, l, xl, xrow,
                                                 acc, gb + U * (i + 1), ge, glo, kb, magic);
    } else if (i + 1 == nch) {
        mma_chunk<PERSIST, XM, U, NT, MT, false>(a, b, tsn, more ? gb : gb + U * i, s16, z16, smem, l, xl, xrow, acc,
                                                 gb + U * i, ge, glo, kb, magic);
        if constexpr (PERSIST) a = b;
    }
    if constexpr (NORM) write_residual<false>(xg, nin, kx, xsl, lane);
    if (WK > 1) {
        f4* red = reinterpret_cast<f4*>(smem + l.red);  // [WK - 1][NT][MT][64]
        if (PERSIST && pass > 0) __syncthreads();  // wavefront 0 has read the previous tile group's sums
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int bb = 0; bb < MT; ++bb) red[(((wave - 1) * NT + t) * MT + bb) * 64 + lane] = acc[t][bb];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int v = 0; v < WK - 1; ++v)
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int bb = 0; bb < MT; ++bb) acc[t][bb] += red[((v * NT + t) * MT + bb) * 64 + lane];
        }
    }
    if constexpr (SPLIT) {  // every thread takes part (the epilogue has workgroup barriers)
        int* last_flag = reinterpret_cast<int*>(smem + l.total);  // one u4 past the layout
        finish_unit<MT, NT, 1>(acc, wave == 0, 0, lane, threadIdx.x, splits, tg, unit, ws, locks, *last_flag, y, M, N,
                               0, tile0, tiles, act);
        return;
    }
    if (wave == 0 && act) {  // N % 16 == 0 (checked on the host)
        const int half_n = N >> 1;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int tt = tile0 + t;
#pragma unroll
            for (int bb = 0; bb < MT; ++bb) {
                f4 up;
                up.x = lane_xor32(acc[t][bb].x, lane);
                up.y = lane_xor32(acc[t][bb].y, lane);
                up.z = lane_xor32(acc[t][bb].z, lane);
                up.w = lane_xor32(acc[t][bb].w, lane);
                const int m = 16 * bb + r;
                if (kb >= 2 || m >= M || tt >= tiles) continue;
                const int f = 8 * tt + 4 * kb;  // features f .. f + 3 of the [M, N/2] output
                const f4 g4 = acc[t][bb];
                const h4 o = h4{static_cast<h1>(silu(g4.x) * up.x), static_cast<h1>(silu(g4.y) * up.y),
                                static_cast<h1>(silu(g4.z) * up.z), static_cast<h1>(silu(g4.w) * up.w)};
                *reinterpret_cast<h4*>(y + static_cast<int64_t>(m) * half_n + f) = o;
            }
        }
    } else if (wave == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int n = 16 * (tile0 + t) + 4 * kb;  // N % 8 == 0: n < N implies n + 3 < N
            if (n >= N) continue;
#pragma unroll
            for (int bb = 0; bb < MT; ++bb) {
                const int m = 16 * bb + r;
                if (m >= M) continue;
                const f4 a4 = acc[t][bb];
                *reinterpret_cast<h4*>(y + static_cast<int64_t>(m) * N + n) =
                    h4{static_cast<h1>(a4.x), static_cast<h1>(a4.y), static_cast<h1>(a4.z), static_cast<h1>(a4.w)};
            }
        }
    }
    if (!more) return;
    ts = tsn;
    tg = tg_next;
    tile0 = tg * NT;
    }
    }
}

// One chunk's x fragments read from global memory (k = 128 g + 32 kb + 8 s .. + 7 of batch rows
// 16 b + r), per lane.
template <int U, int MT>
struct XFrags {
    h8 v[U][4][MT];
};

template <int U, int MT>
__device__ __forceinline__ void load_x_frags(XFrags<U, MT>& xf, const h8* const (&xl)[MT], int g0, int glast) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int g = min(g0 + u, glast);  // past the range: a valid address; the group is not added
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int b = 0; b < MT; ++b) xf.v[u][s][b] = xl[b][16 * g + s];
    }
}

// mma_chunk's arithmetic with the chunk's x fragments loaded one chunk ahead, beside its weights:
// PF loads the next chunk's weights and x together, so the x loads' L2 round trip is hidden behind
// this chunk's math like the weights' instead of being waited for at the start of every chunk. The
// same sums in the same order as mma_chunk (the same bits). Used by the six-row-tile configuration,
// whose grid has one wavefront per SIMD on Qwen3-8B gate_up (no other wavefront's math covers that
// round trip): M = 16-32 3-4 % faster. With two or three row tiles (two wavefronts per SIMD) it was
// level at M = 8 and 2-5 % slower at M = 16-32, so those keep mma_chunk.
template <bool PF, int U, int NT, int MT>
__device__ __forceinline__ void mma_chunk_gx(const WeightSet<U, NT>& cur, WeightSet<U, NT>& nxt,
                                             const XFrags<U, MT>& xcur, XFrags<U, MT>& xnxt,
                                             const TileStreams<NT>& ts, const h8* const (&xl)[MT], const uint16_t* s16,
                                             const uint16_t* z16, f4 (&acc)[NT][MT], int g0, int ge, uint32_t magic) {
    if constexpr (PF) {
        load_chunk<U, NT>(nxt, ts, s16, z16, g0 + U, ge - 1);
        load_x_frags<U, MT>(xnxt, xl, g0 + U, ge - 1);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the loads above the math: the scheduler would sink them
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const bool valid = PF || g0 + u < ge;  // a chunk that prefetches has all its groups in range
        GroupQ p[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            uint32_t s_raw, z_raw;
            scale_zero(cur.p[u][t], s_raw, z_raw);
            p[t] = group_q_raw(s_raw, z_raw, valid);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const h8 wa = dequant_word(word_of(cur.w[u][t], s), p[t], magic);
#pragma unroll
                for (int b = 0; b < MT; ++b) acc[t][b] = mfma16x16x32(wa, xcur.v[u][s][b], acc[t][b]);
            }
    }
}

// The row-tile-wide configurations (TW4_MMA_WIDE_CONFIGS) in a kernel of their own: x from global
// memory, one tile group of NT row tiles per workgroup, the epilogue chosen at compile time (ACT:
// SwiGLU). Its chunks are mma_chunk's (mma_chunk_gx's at six row tiles); it has none of mma_kernel's
// other forms (x in LDS, the fused norm, split-K, the persistent loop), whose state changed the
// compiler's schedule of the same chunk loop: that kernel's loop waited for two more loads per group
// than this one's, and ran Qwen3-8B gate_up at M = 24 in 17.6 us kernel-only against 16.2 us here.
template <int WK, int U, int NT, int MT, bool ACT>
__global__ void __launch_bounds__(WK * 64) mma_wide_kernel(const h1* __restrict__ x, const u4* __restrict__ w,
                                                          const h1* __restrict__ scales, const h1* __restrict__ zeros,
                                                          int M, int N, int K, int nunits, h1* __restrict__ y) {
    if constexpr (U * MT > 4 && MT > 1) {
        return;  // register budget: never launched (tw4_mma rejects U * MT > 4 for M > 16)
    } else {
    extern __shared__ u4 smem[];  // [WK - 1][NT][MT][64] f4 partial sums
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: SGPR
    const int r = lane & 15, kb = lane >> 4;
    const int G = K >> 7, tiles = (N + 15) >> 4;
    const int tile0 = xcd_rotated_block(nunits) * NT;
    const uint32_t magic = magic_reg();
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(scales);
    const uint16_t* z16 = reinterpret_cast<const uint16_t*>(zeros);
    const TileStreams<NT> ts = tile_streams<NT>(w, s16, z16, tile0, tiles, N, G, lane);
    const h8* xl[MT];
#pragma unroll
    for (int b = 0; b < MT; ++b)
        xl[b] = reinterpret_cast<const h8*>(x + static_cast<int64_t>(min(16 * b + r, M - 1)) * K + 32 * kb);
    const int gw = (G + WK - 1) / WK, gb = min(wave * gw, G), ge = min(gb + gw, G);
    const int nch = (ge - gb + U - 1) / U;
    WeightSet<U, NT> a, b;
    load_chunk<U, NT>(a, ts, s16, z16, gb, max(ge - 1, 0));
    f4 acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int bb = 0; bb < MT; ++bb) acc[t][bb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    int i = 0;
    if constexpr (NT >= 6) {  // x one chunk ahead (mma_chunk_gx)
        XFrags<U, MT> xa, xb;
        load_x_frags<U, MT>(xa, xl, gb, max(ge - 1, 0));
        for (; i + 2 < nch; i += 2) {
            mma_chunk_gx<true, U, NT, MT>(a, b, xa, xb, ts, xl, s16, z16, acc, gb + U * i, ge, magic);
            mma_chunk_gx<true, U, NT, MT>(b, a, xb, xa, ts, xl, s16, z16, acc, gb + U * (i + 1), ge, magic);
        }
        if (i + 2 == nch) {
            mma_chunk_gx<true, U, NT, MT>(a, b, xa, xb, ts, xl, s16, z16, acc, gb + U * i, ge, magic);
            mma_chunk_gx<false, U, NT, MT>(b, a, xb, xa, ts, xl, s16, z16, acc, gb + U * (i + 1), ge, magic);
        } else if (i + 1 == nch) {
            mma_chunk_gx<false, U, NT, MT>(a, b, xa, xb, ts, xl, s16, z16, acc, gb + U * i, ge, magic);
        }
    } else {  // x at the start of each chunk (mma_chunk)
        const DecodeLds l{};  // unused by the global-x chunks
        for (; i + 2 < nch; i += 2) {
            mma_chunk<true, kXGlobal, U, NT, MT>(a, b, ts, gb + U * (i + 1), s16, z16, smem, l, xl, 0, acc,
                                                 gb + U * i, ge, 0, kb, magic);
            mma_chunk<true, kXGlobal, U, NT, MT>(b, a, ts, gb + U * (i + 2), s16, z16, smem, l, xl, 0, acc,
                                                 gb + U * (i + 1), ge, 0, kb, magic);
        }
        if (i + 2 == nch) {
            mma_chunk<true, kXGlobal, U, NT, MT>(a, b, ts, gb + U * (i + 1), s16, z16, smem, l, xl, 0, acc,
                                                 gb + U * i, ge, 0, kb, magic);
            mma_chunk<false, kXGlobal, U, NT, MT>(b, a, ts, 0, s16, z16, smem, l, xl, 0, acc, gb + U * (i + 1), ge,
                                                  0, kb, magic);
        } else if (i + 1 == nch) {
            mma_chunk<false, kXGlobal, U, NT, MT>(a, b, ts, 0, s16, z16, smem, l, xl, 0, acc, gb + U * i, ge, 0, kb,
                                                  magic);
        }
    }
    if (WK > 1) {
        f4* red = reinterpret_cast<f4*>(smem);
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int bb = 0; bb < MT; ++bb) red[(((wave - 1) * NT + t) * MT + bb) * 64 + lane] = acc[t][bb];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int v = 0; v < WK - 1; ++v)
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int bb = 0; bb < MT; ++bb) acc[t][bb] += red[((v * NT + t) * MT + bb) * 64 + lane];
    }
    if constexpr (ACT) {  // N % 16 == 0 (checked on the host): gate rows 4 kb + i, up rows in lane + 32
        const int half_n = N >> 1;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int tt = tile0 + t;
#pragma unroll
            for (int bb = 0; bb < MT; ++bb) {
                f4 up;
                up.x = lane_xor32(acc[t][bb].x, lane);
                up.y = lane_xor32(acc[t][bb].y, lane);
                up.z = lane_xor32(acc[t][bb].z, lane);
                up.w = lane_xor32(acc[t][bb].w, lane);
                const int m = 16 * bb + r;
                if (kb >= 2 || m >= M || tt >= tiles) continue;
                const f4 g4 = acc[t][bb];
                *reinterpret_cast<h4*>(y + static_cast<int64_t>(m) * half_n + 8 * tt + 4 * kb) =
                    h4{static_cast<h1>(silu(g4.x) * up.x), static_cast<h1>(silu(g4.y) * up.y),
                       static_cast<h1>(silu(g4.z) * up.z), static_cast<h1>(silu(g4.w) * up.w)};
            }
        }
    } else {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int n = 16 * (tile0 + t) + 4 * kb;  // N % 8 == 0: n < N implies n + 3 < N
            if (n >= N) continue;
#pragma unroll
            for (int bb = 0; bb < MT; ++bb) {
                const int m = 16 * bb + r;
                if (m >= M) continue;
                const f4 a4 = acc[t][bb];
                *reinterpret_cast<h4*>(y + static_cast<int64_t>(m) * N + n) =
                    h4{static_cast<h1>(a4.x), static_cast<h1>(a4.y), static_cast<h1>(a4.z), static_cast<h1>(a4.w)};
            }
        }
    }
}
}

static int g_decode_ready[kMaxDevices];
static int g_decode_cus[kMaxDevices];


int decode_prepare(int dev) {
    if (dev < 0 || dev >= kMaxDevices) {
        tw4host::set_error("init: device %d out of range", dev);
        return TW4_EINVAL;
    }
    if (g_decode_ready[dev]) return TW4_OK;
    int cus = 0;
    hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return tw4host::hip_fail(e, "init: multiprocessor count");
    g_decode_cus[dev] = cus;
    int rc = TW4_OK;
#define TW4_ATTR_GEMV(WK, U, T, NORM)                                        \
    if (rc == TW4_OK) rc = allow_lds(gemv_kernel<1, WK, U, T, NORM>);        \
    if (rc == TW4_OK) rc = allow_lds(gemv_kernel<2, WK, U, T, NORM>);        \
    if (rc == TW4_OK) rc = allow_lds(gemv_kernel<3, WK, U, T, NORM>);        \
    if (rc == TW4_OK) rc = allow_lds(gemv_kernel<4, WK, U, T, NORM>);
#define TW4_ATTR(WK, U, T)                                                   \
    TW4_ATTR_GEMV(WK, U, T, false)                                           \
    TW4_ATTR_GEMV(WK, U, T, true)                                            \
    if (rc == TW4_OK) rc = allow_lds(gemvm_kernel<true, WK, U, T>);          \
    if (rc == TW4_OK) rc = allow_lds(gemvm_kernel<false, WK, U, T>);         \
    if (rc == TW4_OK) rc = allow_lds(mma_kernel<WK, U, T, 1, kXLds>);         \
    if (rc == TW4_OK) rc = allow_lds(mma_kernel<WK, U, T, 1, kXLds, true>);   \
    if (rc == TW4_OK) rc = allow_lds(mma_kernel<WK, U, T, 1, kXLdsWide>);     \
    if (rc == TW4_OK) rc = allow_lds(mma_kernel<WK, U, T, 1, kXGlobal>);      \
    if (rc == TW4_OK) rc = allow_lds(mma_kernel<WK, U, T, 1, kXLds, false, true>);     \
    if (rc == TW4_OK) rc = allow_lds(mma_kernel<WK, U, T, 1, kXLdsWide, false, true>); \
    if (rc == TW4_OK) rc = allow_lds(mma_kernel<WK, U, T, 1, kXGlobal, false, true>);  \
    if (rc == TW4_OK) rc = allow_lds(mma_kernel<WK, U, T, 2, kXGlobal>);      \
    if (rc == TW4_OK) rc = allow_lds(mma_kernel<WK, U, T, 4, kXGlobal>);
    TW4_DECODE_CONFIGS(TW4_ATTR)
#define TW4_ATTR_WIDE_ACT(WK, U, T, A)                                       \
    if (rc == TW4_OK) rc = allow_lds(mma_wide_kernel<WK, U, T, 1, A>);        \
    if (rc == TW4_OK) rc = allow_lds(mma_wide_kernel<WK, U, T, 2, A>);        \
    if (rc == TW4_OK) rc = allow_lds(mma_wide_kernel<WK, U, T, 4, A>);
#define TW4_ATTR_WIDE(WK, U, T) TW4_ATTR_WIDE_ACT(WK, U, T, false) TW4_ATTR_WIDE_ACT(WK, U, T, true)
    TW4_MMA_WIDE_CONFIGS(TW4_ATTR_WIDE)
#undef TW4_ATTR_WIDE
#undef TW4_ATTR_WIDE_ACT
#undef TW4_ATTR
#undef TW4_ATTR_GEMV
    if (rc == TW4_OK) g_decode_ready[dev] = 1;
    return rc;
}

int ensure_prepared() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return tw4host::hip_fail(e, "decode: hipGetDevice");
    if (dev >= 0 && dev < kMaxDevices && g_decode_ready[dev]) return TW4_OK;
    return decode_prepare(dev);
}

int gemvm_dispatch(const h1* x, const u4* w, const h1* s, const h1* z, h1* y, int M, int N, int K, int wk, int un,
                   int nt, int act, hipStream_t st) {
    const int tiles = (N + 15) >> 4;
#define TW4_GEMVM_CASE(WK, U, T)                                                                             \
    if (wk == WK && un == U && nt == T) {                                                                    \
        const size_t lds = 16 * static_cast<size_t>(                                                         \
                                    decode_lds(true, M, K, gemv_corr_u4(M, K) + gemvm_gcorr_u4(M, K), (WK - 1) * T * 64).total); \
        TW4_REQUIRE(lds <= static_cast<size_t>(kMaxLds), TW4_EINVAL,                                        \
                    "gemv_mfma: x [%d, %d] does not fit in LDS (use mma)", M, K);                            \
        if (M == 1)                                                                                          \
            gemvm_kernel<true, WK, U, T><<<(tiles + T - 1) / T, WK * 64, lds, st>>>(x, w, s, z, y, M, N, K, act); \
        else                                                                                                 \
            gemvm_kernel<false, WK, U, T><<<(tiles + T - 1) / T, WK * 64, lds, st>>>(x, w, s, z, y, M, N, K, act); \
        TW4_LAUNCH_CHECK("gemv_mfma: launch");                                                               \
        return TW4_OK;                                                                                       \
    }
    TW4_DECODE_CONFIGS(TW4_GEMVM_CASE)
#undef TW4_GEMVM_CASE
    tw4host::set_error("gemv_mfma: unsupported warps_k / unroll / ntile %d / %d / %d", wk, un, nt);
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

extern "C" int tw4_gemv_act(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                            uint16_t* y, int M, int N, int K, int warps_k, int unroll, int ntile, int act,
                            void* stream) {
    int rc = check_operands("gemv", x, packed, scales, zeros, y, M, N, K);
    if (rc) return rc;
    TW4_REQUIRE(M >= 1 && M <= 4, TW4_EINVAL, "gemv: 1 <= M <= 4 (M = %d; larger M: mma)", M);
    TW4_REQUIRE(K <= 65536, TW4_EINVAL, "gemv: K <= 65536 (K = %d; larger K: mma)", K);
    TW4_REQUIRE(act == 0 || (act == 1 && N % 16 == 0), TW4_EINVAL,
                "gemv: act 0, or 1 (SwiGLU) with N %% 16 == 0 (act = %d, N = %d)", act, N);
    rc = ensure_prepared();
    if (rc) return rc;
    auto xp = reinterpret_cast<const h1*>(x);
    auto wp = reinterpret_cast<const u4*>(packed);
    auto sp = reinterpret_cast<const h1*>(scales);
    auto zp = reinterpret_cast<const h1*>(zeros);
    auto yp = reinterpret_cast<h1*>(y);
    auto st = static_cast<hipStream_t>(stream);
    const NormIn none{nullptr, nullptr, nullptr, 0.0f};
    switch (M) {
        case 1: return gemv_dispatch<1, false>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, none, st);
        case 2: return gemv_dispatch<2, false>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, none, st);
        case 3: return gemv_dispatch<3, false>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, none, st);
        default: return gemv_dispatch<4, false>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, none, st);
    }
}

extern "C" int tw4_gemv_mfma(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                             uint16_t* y, int M, int N, int K, int warps_k, int unroll, int ntile, int act,
                             void* stream) {
    int rc = check_operands("gemv_mfma", x, packed, scales, zeros, y, M, N, K);
    if (rc) return rc;
    TW4_REQUIRE(M >= 1 && M <= 16, TW4_EINVAL, "gemv_mfma: 1 <= M <= 16 (M = %d; larger M: mma)", M);
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(scales) % 8 == 0 && reinterpret_cast<uintptr_t>(zeros) % 8 == 0,
                TW4_EINVAL, "gemv_mfma: scales and zeros must be 8-byte aligned");
    TW4_REQUIRE(K <= 65536, TW4_EINVAL, "gemv_mfma: K <= 65536 (K = %d; larger K: mma)", K);
    TW4_REQUIRE(act == 0 || (act == 1 && N % 16 == 0), TW4_EINVAL,
                "gemv_mfma: act 0, or 1 (SwiGLU) with N %% 16 == 0 (act = %d, N = %d)", act, N);
    rc = ensure_prepared();
    if (rc) return rc;
    auto xp = reinterpret_cast<const h1*>(x);
    auto wp = reinterpret_cast<const u4*>(packed);
    auto sp = reinterpret_cast<const h1*>(scales);
    auto zp = reinterpret_cast<const h1*>(zeros);
    auto yp = reinterpret_cast<h1*>(y);
    auto st = static_cast<hipStream_t>(stream);
    return gemvm_dispatch(xp, wp, sp, zp, yp, M, N, K, warps_k, unroll, ntile, act, st);
}

extern "C" int tw4_gemv(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                        uint16_t* y, int M, int N, int K, int warps_k, int unroll, int ntile, void* stream) {
    return tw4_gemv_act(x, packed, scales, zeros, y, M, N, K, warps_k, unroll, ntile, 0, stream);
}

namespace tw4 {

// One mma launch; nin (not null): the fused norm prologue, which needs x in LDS. splits > 1: split-K
// over workgroups (ws / locks: the partial sums and counters, zero before the first call).
// per_cu > 0: the persistent form, at most per_cu workgroups per CU, each streaming several tile groups.
int mma_launch(const h1* xp, const u4* wp, const h1* sp, const h1* zp, h1* yp, int M, int N, int K, int warps_k,
               int unroll, int ntile, int act, const NormIn* nin, float* ws, int* locks, int64_t ws_floats,
               int64_t n_locks, int splits, hipStream_t st, int per_cu = 0) {
    const int mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
    TW4_REQUIRE(mt == 1 || unroll * mt <= 4, TW4_ECONFIG,
                "mma: M = %d takes %d batch tiles; unroll %d x %d tiles > 4 is not compiled", M, mt, unroll, mt);
    const int G = K >> 7, tiles = (N + 15) >> 4;
    TW4_REQUIRE(splits >= 1 && splits <= 16 && splits <= G, TW4_EINVAL,
                "mma: splits in 1 .. min(16, K / 128) (splits = %d, K = %d)", splits, K);
    TW4_REQUIRE(splits == 1 || !nin, TW4_EINVAL, "mma: the fused norm needs whole rows (splits = 1)");
    TW4_REQUIRE(splits == 1 || mt == 1, TW4_EINVAL, "mma: split-K for M <= 16 only (M = %d)", M);
    const int R = (G + splits - 1) / splits;  // the most quant groups a workgroup covers
    const size_t x_bytes = static_cast<size_t>(M) * (16 * R + 1) * 16;
    const bool xlds_small = mt == 1 && x_bytes <= static_cast<size_t>(kXLdsLimit);
    const int gw = (R + warps_k - 1) / max(warps_k, 1);
    const bool wide = M * gw > 8;  // a lane's share of the staged slice, M gw / 4 chunks, is more than 2
    TW4_REQUIRE(!nin || xlds_small, TW4_ECONFIG,
                "mma: the fused norm stages x in LDS: M (K + 8) 2 bytes <= %d (M = %d, K = %d)", kXLdsLimit, M, K);
    const NormIn none{nullptr, nullptr, nullptr, 0.0f};
    const int64_t groups = (tiles + ntile - 1) / max(ntile, 1);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = 0;
    TW4_REQUIRE(per_cu >= 0 && per_cu <= 8, TW4_EINVAL, "mma: per_cu in 0 .. 8 (per_cu = %d)", per_cu);
    TW4_REQUIRE(per_cu == 0 || (splits == 1 && !nin && mt == 1), TW4_EINVAL,
                "mma: the persistent form takes M <= 16, no split-K and no fused norm");
    const int64_t cap = static_cast<int64_t>(per_cu) * g_decode_cus[dev];
    const int64_t units = per_cu > 0 ? (groups < cap ? groups : cap) : groups * splits;
    // x in LDS past kXLdsLimit (one workgroup per CU) only where the grid fits the CUs at once
    const bool few = units <= g_decode_cus[dev];
    if (splits > 1) {
        TW4_REQUIRE(ws && locks, TW4_EINVAL, "mma: split-K needs a workspace and counters");
        TW4_REQUIRE(groups * splits * ntile * mt * 256 <= ws_floats && groups <= n_locks, TW4_ESPACE,
                    "mma: split-K workspace too small for %lld tile groups x %d splits", static_cast<long long>(groups),
                    splits);
    }
// mma_kernel's arguments in its order; the grid (nunits) is the number of units launched.
#define TW4_MMA_ARGS(NIN) xp, wp, sp, zp, M, N, K, splits, static_cast<int>(grid), yp, act, NIN, ws, locks
#define TW4_MMA_CASE(WK, U, T)                                                                                            \
    if (warps_k == WK && unroll == U && ntile == T) {                                                                     \
        const int red_u4 = (WK - 1) * T * mt * 64;                                                                        \
        const bool xlds = xlds_small || (mt == 1 && few && x_bytes <= static_cast<size_t>(kXLdsBig) &&                    \
                                         16 * (static_cast<size_t>(decode_lds(true, M, 128 * R, 0, red_u4).total) + 1) <= \
                                             static_cast<size_t>(kMaxLds));                                               \
        const size_t lds = 16 * (static_cast<size_t>(                                                                     \
                                     decode_lds(xlds, M, 128 * R, 0, red_u4, nin != nullptr).total) +                     \
                                 1); /* + the split-K flag */                                                             \
        const unsigned grid = static_cast<unsigned>(units);                                                               \
        TW4_REQUIRE(per_cu == 0 || xlds, TW4_ECONFIG, "mma: the persistent form stages x in LDS (M = %d, K = %d)",        \
                    M, K);                                                                                                \
        if (per_cu > 0 && wide)                                                                                           \
            mma_kernel<WK, U, T, 1, kXLdsWide, false, false, true><<<grid, WK * 64, lds, st>>>(TW4_MMA_ARGS(none));       \
        else if (per_cu > 0)                                                                                              \
            mma_kernel<WK, U, T, 1, kXLds, false, false, true><<<grid, WK * 64, lds, st>>>(TW4_MMA_ARGS(none));           \
        else if (splits > 1 && xlds && wide)                                                                              \
            mma_kernel<WK, U, T, 1, kXLdsWide, false, true><<<grid, WK * 64, lds, st>>>(TW4_MMA_ARGS(none));              \
        else if (splits > 1 && xlds)                                                                                      \
            mma_kernel<WK, U, T, 1, kXLds, false, true><<<grid, WK * 64, lds, st>>>(TW4_MMA_ARGS(none));                  \
        else if (splits > 1)                                                                                              \
            mma_kernel<WK, U, T, 1, kXGlobal, false, true><<<grid, WK * 64, lds, st>>>(TW4_MMA_ARGS(none));               \
        else if (nin)                                                                                                     \
            mma_kernel<WK, U, T, 1, kXLds, true><<<grid, WK * 64, lds, st>>>(TW4_MMA_ARGS(*nin));                         \
        else if (xlds && wide)                                                                                            \
            mma_kernel<WK, U, T, 1, kXLdsWide><<<grid, WK * 64, lds, st>>>(TW4_MMA_ARGS(none));                           \
        else if (xlds)                                                                                                    \
            mma_kernel<WK, U, T, 1, kXLds><<<grid, WK * 64, lds, st>>>(TW4_MMA_ARGS(none));                               \
        else if (mt == 1)                                                                                                 \
            mma_kernel<WK, U, T, 1, kXGlobal><<<grid, WK * 64, lds, st>>>(TW4_MMA_ARGS(none));                            \
        else if (mt == 2)                                                                                                 \
            mma_kernel<WK, U, T, 2, kXGlobal><<<grid, WK * 64, lds, st>>>(TW4_MMA_ARGS(none));                            \
        else                                                                                                              \
            mma_kernel<WK, U, T, 4, kXGlobal><<<grid, WK * 64, lds, st>>>(TW4_MMA_ARGS(none));                            \
        TW4_LAUNCH_CHECK("mma: launch");                                                                                  \
        return TW4_OK;                                                                                                    \
    }
    TW4_DECODE_CONFIGS(TW4_MMA_CASE)
#undef TW4_MMA_CASE
// The row-tile-wide configurations: x from global memory at any M, one workgroup per tile group.
#define TW4_WIDE_LAUNCH(WK, U, T, MTV, A)                                                                     \
    mma_wide_kernel<WK, U, T, MTV, A><<<grid, WK * 64, lds, st>>>(xp, wp, sp, zp, M, N, K, static_cast<int>(grid), yp)
#define TW4_MMA_WIDE_CASE(WK, U, T)                                                                           \
    if (warps_k == WK && unroll == U && ntile == T) {                                                         \
        TW4_REQUIRE(splits == 1 && per_cu == 0 && !nin, TW4_ECONFIG,                                         \
                    "mma: (%d, %d, %d) reads x from global memory: no split-K, persistent form or fused norm", \
                    WK, U, T);                                                                                \
        const size_t lds = 16 * static_cast<size_t>((WK - 1) * T * mt * 64);                                  \
        const unsigned grid = static_cast<unsigned>(units);                                                   \
        if (mt == 1 && act)                                                                                   \
            TW4_WIDE_LAUNCH(WK, U, T, 1, true);                                                               \
        else if (mt == 1)                                                                                     \
            TW4_WIDE_LAUNCH(WK, U, T, 1, false);                                                              \
        else if (mt == 2 && act)                                                                              \
            TW4_WIDE_LAUNCH(WK, U, T, 2, true);                                                               \
        else if (mt == 2)                                                                                     \
            TW4_WIDE_LAUNCH(WK, U, T, 2, false);                                                              \
        else if (act)                                                                                         \
            TW4_WIDE_LAUNCH(WK, U, T, 4, true);                                                               \
        else                                                                                                  \
            TW4_WIDE_LAUNCH(WK, U, T, 4, false);                                                              \
        TW4_LAUNCH_CHECK("mma: launch");                                                                      \
        return TW4_OK;                                                                                        \
    }
    TW4_MMA_WIDE_CONFIGS(TW4_MMA_WIDE_CASE)
#undef TW4_MMA_WIDE_CASE
#undef TW4_WIDE_LAUNCH
#undef TW4_MMA_ARGS
    tw4host::set_error("mma: unsupported warps_k / unroll / ntile %d / %d / %d", warps_k, unroll, ntile);
    return TW4_ECONFIG;
}

}  // namespace tw4

extern "C" int tw4_mma(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                       uint16_t* y, int M, int N, int K, int warps_k, int unroll, int ntile, int act, void* stream) {
    int rc = check_operands("mma", x, packed, scales, zeros, y, M, N, K);
    if (rc) return rc;
    TW4_REQUIRE(M >= 1 && M <= 64, TW4_EINVAL, "mma: 1 <= M <= 64 (M = %d)", M);
    TW4_REQUIRE(act == 0 || (act == 1 && N % 16 == 0), TW4_EINVAL,
                "mma: act 0, or 1 (SwiGLU) with N %% 16 == 0 (act = %d, N = %d)", act, N);
    rc = ensure_prepared();
    if (rc) return rc;
    return mma_launch(reinterpret_cast<const h1*>(x), reinterpret_cast<const u4*>(packed),
                      reinterpret_cast<const h1*>(scales), reinterpret_cast<const h1*>(zeros), reinterpret_cast<h1*>(y),
                      M, N, K, warps_k, unroll, ntile, act, nullptr, nullptr, nullptr, 0, 0, 1,
                      static_cast<hipStream_t>(stream));
}

extern "C" int tw4_mma_persist(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                               uint16_t* y, int M, int N, int K, int warps_k, int unroll, int ntile, int per_cu, int act,
                               void* stream) {
    int rc = check_operands("mma", x, packed, scales, zeros, y, M, N, K);
    if (rc) return rc;
    TW4_REQUIRE(M >= 1 && M <= 16, TW4_EINVAL, "mma: the persistent form takes 1 <= M <= 16 (M = %d)", M);
    TW4_REQUIRE(per_cu >= 1 && per_cu <= 8, TW4_EINVAL, "mma: per_cu in 1 .. 8 (per_cu = %d)", per_cu);
    TW4_REQUIRE(act == 0 || (act == 1 && N % 16 == 0), TW4_EINVAL,
                "mma: act 0, or 1 (SwiGLU) with N %% 16 == 0 (act = %d, N = %d)", act, N);
    rc = ensure_prepared();
    if (rc) return rc;
    return mma_launch(reinterpret_cast<const h1*>(x), reinterpret_cast<const u4*>(packed),
                      reinterpret_cast<const h1*>(scales), reinterpret_cast<const h1*>(zeros), reinterpret_cast<h1*>(y),
                      M, N, K, warps_k, unroll, ntile, act, nullptr, nullptr, nullptr, 0, 0, 1,
                      static_cast<hipStream_t>(stream), per_cu);
}

extern "C" int tw4_mma_splitk(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                              uint16_t* y, float* ws, int32_t* locks, int64_t ws_floats, int64_t n_locks, int M, int N,
                              int K, int warps_k, int unroll, int ntile, int splits, int act, void* stream) {
    int rc = check_operands("mma", x, packed, scales, zeros, y, M, N, K);
    if (rc) return rc;
    TW4_REQUIRE(M >= 1 && M <= 64, TW4_EINVAL, "mma: 1 <= M <= 64 (M = %d)", M);
    TW4_REQUIRE(act == 0 || (act == 1 && N % 16 == 0), TW4_EINVAL,
                "mma: act 0, or 1 (SwiGLU) with N %% 16 == 0 (act = %d, N = %d)", act, N);
    TW4_REQUIRE(ws_floats >= 0 && n_locks >= 0, TW4_EINVAL, "mma: workspace sizes must be >= 0");
    TW4_REQUIRE(splits >= 1 && splits <= 16 && splits <= K / 128, TW4_EINVAL,
                "mma: splits in 1 .. min(16, K / 128) (splits = %d, K = %d)", splits, K);
    TW4_REQUIRE(splits == 1 || M <= 16, TW4_EINVAL, "mma: split-K for M <= 16 only (M = %d)", M);
    TW4_REQUIRE(splits == 1 || (ws && locks), TW4_EINVAL, "mma: split-K needs a workspace and counters");
    ws_floats = ws_floats < kMaxPartialFloats ? ws_floats : kMaxPartialFloats;  // the part split-K may use
    rc = ensure_prepared();
    if (rc) return rc;
    return mma_launch(reinterpret_cast<const h1*>(x), reinterpret_cast<const u4*>(packed),
                      reinterpret_cast<const h1*>(scales), reinterpret_cast<const h1*>(zeros), reinterpret_cast<h1*>(y),
                      M, N, K, warps_k, unroll, ntile, act, nullptr, ws, reinterpret_cast<int*>(locks), ws_floats,
                      n_locks, splits, static_cast<hipStream_t>(stream));
}

extern "C" int tw4_decode_norm(const uint16_t* x, const uint16_t* residual, uint16_t* residual_out,
                               const uint16_t* norm_weight, float eps, const int32_t* packed, const uint16_t* scales,
                               const uint16_t* zeros, uint16_t* y, int M, int N, int K, int kind, int warps_k,
                               int unroll, int ntile, int act, void* stream) {
    int rc = check_operands("decode_norm", x, packed, scales, zeros, y, M, N, K);
    if (rc) return rc;
    TW4_REQUIRE(norm_weight && reinterpret_cast<uintptr_t>(norm_weight) % 16 == 0, TW4_EINVAL,
                "decode_norm: norm_weight must be a 16-byte aligned pointer");
    TW4_REQUIRE(!residual || (residual_out && reinterpret_cast<uintptr_t>(residual) % 16 == 0 &&
                              reinterpret_cast<uintptr_t>(residual_out) % 16 == 0),
                TW4_EINVAL, "decode_norm: residual and residual_out must be 16-byte aligned pointers");
    TW4_REQUIRE(!residual || (residual_out != residual && residual_out != x), TW4_EINVAL,
                "decode_norm: residual_out must not alias residual or x (other workgroups still read them)");
    TW4_REQUIRE(M >= 1 && M <= kNormMaxRows, TW4_EINVAL, "decode_norm: 1 <= M <= %d (M = %d)", kNormMaxRows, M);
    TW4_REQUIRE(kind == 0 || kind == 1, TW4_EINVAL, "decode_norm: kind 0 (gemv) or 1 (mma), not %d", kind);
    TW4_REQUIRE(kind == 1 || M <= 4, TW4_EINVAL, "decode_norm: gemv: 1 <= M <= 4 (M = %d)", M);
    TW4_REQUIRE(K <= 65536, TW4_EINVAL, "decode_norm: K <= 65536 (K = %d)", K);
    TW4_REQUIRE(act == 0 || (act == 1 && N % 16 == 0), TW4_EINVAL,
                "decode_norm: act 0, or 1 (SwiGLU) with N %% 16 == 0 (act = %d, N = %d)", act, N);
    rc = ensure_prepared();
    if (rc) return rc;
    const NormIn nin{reinterpret_cast<const h1*>(residual), reinterpret_cast<h1*>(residual_out),
                     reinterpret_cast<const h1*>(norm_weight), eps};
    auto xp = reinterpret_cast<const h1*>(x);
    auto wp = reinterpret_cast<const u4*>(packed);
    auto sp = reinterpret_cast<const h1*>(scales);
    auto zp = reinterpret_cast<const h1*>(zeros);
    auto yp = reinterpret_cast<h1*>(y);
    auto st = static_cast<hipStream_t>(stream);
    if (kind == 1) return mma_launch(xp, wp, sp, zp, yp, M, N, K, warps_k, unroll, ntile, act, &nin, nullptr, nullptr, 0, 0, 1,
                                     st);
    switch (M) {
        case 1: return gemv_dispatch<1, true>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, nin, st);
        case 2: return gemv_dispatch<2, true>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, nin, st);
        case 3: return gemv_dispatch<3, true>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, nin, st);
        default: return gemv_dispatch<4, true>(xp, wp, sp, zp, yp, N, K, warps_k, unroll, ntile, act, nin, st);
    }
}

#define TW4_LIST(WK, U, T)                  \
    if (out && n < max_configs) {           \
        out[3 * n] = WK;                    \
        out[3 * n + 1] = U;                 \
        out[3 * n + 2] = T;                 \
    }                                       \
    ++n;

extern "C" int tw4_decode_configs(int* out, int max_configs) {
    int n = 0;
    TW4_DECODE_CONFIGS(TW4_LIST)
    return n;
}

extern "C" int tw4_mma_wide_configs(int* out, int max_configs) {
    int n = 0;
    TW4_MMA_WIDE_CONFIGS(TW4_LIST)
    return n;
}
#undef TW4_LIST
