// Building blocks of the decode kernels (tw4_decode.hip): the streaming helpers, x staging, the fused
// norm prologue and the vector-ALU GEMV (its launcher gemv_dispatch too), and the compiled decode
// configurations. Everything here is a template or inline.
//
// Decode kernels, M <= 64: y[M, N] = x[M, K] @ dequant(W)^T, bound by streaming the int4 weights.
//
// A workgroup owns NT row tiles (16 rows each); its WK wavefronts split K into WK contiguous ranges
// of quant groups. Lane l = 16 kb + r streams the 16 bytes (kb, r, s = 0..3) of every (row tile,
// group) block of its range with one non-temporal global_load_dwordx4 (weights k = 128 g + 32 kb
// .. + 31 of row r), and the block's scale and zero with two 2-byte loads: scales and zeros are
// stored tile-major, so the 16 rows of a group are one 32-byte segment. Ranges are walked in chunks
// of UNROLL groups; the next chunk's weights, scales and zeros are in flight (a second register
// set; the loop is unrolled by two so the sets swap roles without copies) while the current chunk is
// computed. Loads retire in issue order, so a chunk issues what it needs now first, then the
// prefetch, and no branch sits around a load: every wait is exact.
//
// x goes to LDS when it fits (row stride K + 8 halves, so the 16 rows of a B-fragment read hit 16
// different bank groups): each wavefront stages only its own groups' slice, while its first chunk
// is in flight, with no workgroup barrier. The WK partial sums are added in LDS at the end.
//
//   gemv: vector ALUs, M <= 4, x always in LDS, stored as x' (pairs 2, 3 and 6, 7 of every 8 k
//         divided by 16) with per-slice sums of x' and x (fill_x_biased). A word becomes four
//         fp16 pairs of "magic" values (1024 + q, or 1024 + 16 q for the high nibbles) with four
//         v_and_or_b32 and one shift, and v_dot2_f32_f16 multiplies them with x' pairs (fp32
//         accumulation); the 1024 bias and the zero point come off once per group and slice
//         (dot - 1024 sum x' - z sum x), then the group's scale. Row sums are finished with two
//         cross-lane exchanges (lanes r, r + 16, r + 32, r + 48 hold the four 32-k slices).
//   mma:  matrix cores, M <= 64 (MT = ceil(M / 16) batch tiles of 16 columns). v_mfma_f32_16x16x32_f16 with the dequantized weights
//         fp16_rne((q - z) s) as A (16 rows x 32 k) and x as B (32 k x 16 batch columns). Step s
//         of a block uses word s of every lane: lane (kb, r) feeds A row r and B column r the
//         weights / activations k = 128 g + 32 kb + 8 s .. + 7, the same k permutation for both
//         operands, so each MFMA sums 32 distinct k of the group. B columns r >= M read row
//         M - 1: they only feed D columns that are never stored. D holds output rows 4 kb + i
//         (i = 0..3) of batch column r in lane (kb, r). x comes from LDS when M (K + 8) 2 bytes
//         fit in 80 KB, else straight from global memory (issued before the prefetch). Split-K
//         form (M <= 16): each workgroup covers 1 / splits of the quant groups, so only that part
//         of x has to fit in LDS, and the last arriver of a row-tile group adds the partial sums.
//   act = 1: rows are in interleave_gate_up order (gate rows 0..7 of a tile, then its up rows).
//         mma: the gate rows 4 kb + i (kb = 0, 1) and up rows 8 + 4 kb + i of a feature sit in
//         lanes l and l + 32; gemv: in lanes i and i + 8. One cross-lane exchange pairs them and
//         the lane writes silu(gate) * up.
#pragma once

#include "tw4_common.h"

namespace tw4 {


template <int U, int NT>
struct WeightSet {  // one chunk's weight blocks and group parameters, per lane
    u4 w[U][NT];
    uint16_t p[U][NT];  // the row's scale (lanes of rows kb = 0, 2) or zero (kb = 1, 3): see scale_zero
};

// Lanes 16 kb + r of even kb load row r's scale, of odd kb its zero: one 2-byte load per lane and
// group instead of two. v_permlane16_swap exchanges rows 0 <-> 1 and 2 <-> 3 of two copies, which
// leaves the even rows' values (scales) in the first result and the odd rows' (zeros) in the second.
__device__ __forceinline__ void scale_zero(uint32_t p, uint32_t& s, uint32_t& z) {
    const auto sz = __builtin_amdgcn_permlane16_swap(p, p, false, false);
    s = sz[0];
    z = sz[1];
}

// Workgroups are dealt to the 8 XCDs round robin (workgroup b runs on XCD b mod 8). Within each full
// group of 8 workgroups the tile index is rotated by b / 8, so the tiles one XCD streams do not all
// share the same low address bits: measured on MI355X, the XCDs then finish closer together (the
// M = 1 GEMV on gate_up 10.3 vs 10.4-10.6 us). A permutation of 0 .. nblocks - 1.
// nblocks is the launch's gridDim.x. The kernels that know it from their explicit arguments pass it
// computed from them: gridDim.x is a hidden kernel argument placed after the explicit ones, past the
// argument dwords preloaded into SGPRs, so reading it costs every wavefront a scalar load and a wait
// before its first weight load (the M = 1 GEMV on gate_up measured 10.2 -> 9.9 us without it).
__device__ __forceinline__ int xcd_rotated_block(int nblocks) {
    const int b = blockIdx.x, full = nblocks & ~7;
    return b < full ? (b & ~7) | (((b & 7) + (b >> 3)) & 7) : b;
}

// The workgroup's row tiles. Everything but `lane` and `prow` is uniform across the wavefront (the
// tile index comes from blockIdx), so tile and group offsets stay in scalar registers and each
// load is one scalar base + the lane's fixed vector offset.
template <int NT>
struct TileStreams {
    __amdgpu_buffer_rsrc_t w[NT];  // the tile's weight blocks (G KB): block g at byte g * 1024
    int64_t p[NT];       // scale / zero offset of (tile, group 0) in the tile-major order
    int rows[NT];        // rows of the tile: the scale / zero stride between groups
    int prow[NT];        // this lane's row in the tile (clamped: padding rows have zero weights)
    int lane;
    const uint16_t* pb;  // scales (even kb) or zeros (odd kb)
};

template <int NT>
__device__ __forceinline__ TileStreams<NT> tile_streams(const u4* w, const uint16_t* s16, const uint16_t* z16, int tile0,
                                                       int tiles, int N, int G, int lane) {
    TileStreams<NT> ts;
    const int r = lane & 15;
    ts.lane = lane;
    ts.pb = (lane & 16) ? z16 : s16;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int tt = min(tile0 + t, tiles - 1);  // tiles past the end recompute the last one; not stored
        ts.w[t] = __builtin_amdgcn_make_buffer_rsrc(const_cast<u4*>(w + static_cast<int64_t>(tt) * G * kBlockU4), 0,
                                                    G * kBlockU4 * 16, kBufferFlags);
        ts.rows[t] = tile_rows(tt, N);
        ts.p[t] = static_cast<int64_t>(16) * tt * G;
        ts.prow[t] = min(r, ts.rows[t] - 1);
    }
    return ts;
}

// LDS layout of a decode workgroup (offsets in 16-byte units): [x rows][corr][norm][reduction].
struct DecodeLds {
    int xs;    // x row stride (u4): K / 8 + 1
    int corr;  // gemv: per (m, group, slice) sums of x' and x (float2)
    int norm;  // fused norm prologue: per (m, group) sums of squares (float [M][G])
    int red;   // cross-wavefront reduction
    int total;
};

__host__ __device__ __forceinline__ DecodeLds decode_lds(bool xlds, int M, int K, int corr_u4, int red_u4,
                                                         bool norm = false) {
    DecodeLds l;
    l.xs = (K >> 3) + 1;
    l.corr = xlds ? M * l.xs : 0;
    l.norm = l.corr + corr_u4;
    l.red = l.norm + (norm ? (M * (K >> 7) + 3) / 4 : 0);
    l.total = l.red + red_u4;
    return l;
}

__host__ __device__ __forceinline__ int gemv_corr_u4(int M, int K) { return M * (K >> 7) * 2; }  // float2 [M][G][4]
__host__ __device__ __forceinline__ int gemv_red_u4(int M, int WK, int NT) { return (WK * NT * M * 16 + 3) / 4; }

// One word -> its four magic halves, no zero applied: (1024 + q) for weights 0, 1 and 4, 5,
// (1024 + 16 q) for weights 2, 3 and 6, 7 (see fill_x_biased).
__device__ __forceinline__ void unpack_raw(uint32_t w, uint32_t magic, h2 (&d)[4]) {
    const uint32_t w8 = w >> 8;
    d[0] = bitcast<h2>((w & 0x000F000Fu) | magic);
    d[1] = bitcast<h2>((w & 0x00F000F0u) | magic);
    d[2] = bitcast<h2>((w8 & 0x000F000Fu) | magic);
    d[3] = bitcast<h2>((w8 & 0x00F000F0u) | magic);
}

template <int U, int NT>
__device__ __forceinline__ void load_chunk(WeightSet<U, NT>& ws, const TileStreams<NT>& ts, const uint16_t* s16,
                                           const uint16_t* z16, int g0, int glast) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int g = min(g0 + u, glast);  // past the range: a valid block, given scale 0 below
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            ws.w[u][t] = load_block(ts.w[t], g, ts.lane);
            const int64_t pg = ts.p[t] + static_cast<int64_t>(g) * ts.rows[t];
            ws.p[u][t] = (ts.pb + pg)[ts.prow[t]];
        }
    }
}

// Per-wavefront x staging. A wavefront reads x only over its own quant groups [gb, ge), so it stages
// just that slice of every row into the workgroup's LDS image of x (rows of K + 8 halves) and needs
// no workgroup barrier: its lanes write, then read, their own slice. The slice is M rows of n16
// chunks of 16 bytes (from column c0), walked as one flat index f = m n16 + c: lane l takes chunks
// l, l + 64, ... in batches of kXB, all of a batch's loads before its stores. Chunks past the end
// repeat the last one (identical duplicate writes), so no branch sits around a load or a store. The
// first batch is loaded before the first weight chunk is issued, so waiting for it never waits for
// the weights (loads retire in order).
constexpr int kXB = 2;

struct XSlice {
    int c0;          // first chunk column: 16 gb
    int n16;         // chunks per row: 16 (ge - gb), a multiple of 4
    int n;           // M n16
    uint32_t magic;  // ceil(2^32 / n16): f / n16 == umulhi(f, magic) for f < 16 n16 <= 2^17 (K <= 65536)
};

// An empty slice (gb == ge == G) gets c0 = 0, so the unconditional loads of the fused norm
// prologue read chunk 0 of row 0 (16 gb would be one chunk past the end of x and of the weight).
__device__ __forceinline__ XSlice x_slice(int gb, int ge, int M) {
    const int n16 = 16 * (ge - gb);
    return XSlice{n16 > 0 ? 16 * gb : 0, n16, M * n16,
                  n16 > 0 ? static_cast<uint32_t>(0xFFFFFFFFu / static_cast<uint32_t>(n16)) + 1u : 0u};
}

struct XPos {
    int m, c;
};

// Flat chunk f -> (row, chunk in row); f past the slice -> its last chunk. ONE_ROW: M == 1 known at
// compile time, no division (magic is 0 for an empty slice, so m = 0 there too).
template <bool ONE_ROW>
__device__ __forceinline__ XPos x_pos(const XSlice& xs, int f) {
    f = max(min(f, xs.n - 1), 0);  // an empty slice (n = 0) reads chunk 0 of row 0: a valid address
    if constexpr (ONE_ROW) return XPos{0, f};
    const int m = static_cast<int>(__umulhi(static_cast<uint32_t>(f), xs.magic));
    return XPos{m, f - m * xs.n16};
}

__device__ __forceinline__ u4 x_chunk(const u4* xg, int kx, const XSlice& xs, XPos p) {
    return xg[static_cast<int64_t>(p.m) * kx + xs.c0 + p.c];
}

template <bool ONE_ROW, int XB = kXB>
__device__ __forceinline__ void load_x_batch(u4 (&v)[XB], const u4* xg, int kx, const XSlice& xs, int f0) {
#pragma unroll
    for (int j = 0; j < XB; ++j) v[j] = x_chunk(xg, kx, xs, x_pos<ONE_ROW>(xs, f0 + 64 * j));
}

// Flat chunk f into LDS. BIASED: as x' (pairs k = 8 j + 2, 3 and 8 j + 6, 7 divided by 16: exact, a
// power-of-two scale, rounded only where x / 16 is below fp16's normal range) plus, per (m, group,
// 32-k slice kb), the float sums -1024 A (A = sum x') and B = sum x of the slice (corr[(m G + g) 4 + kb],
// float2). A word's four magic halves (1024 + q for weights 8 j + 0, 1 and 8 j + 4, 5; 1024 + 16 q
// for 8 j + 2, 3 and 8 j + 6, 7) dotted with x' give sum q x + 1024 sum x', so
// sum (q - z) x = dot - 1024 A - z B. The four chunks of a 32-k slice are lanes 4 i .. 4 i + 3 of
// one call (n16 and the lane offsets are multiples of 4); past the slice end all four or none.
template <bool BIASED, bool ONE_ROW>
__device__ __forceinline__ void store_x_chunk(u4* smem, const DecodeLds& l, float2* corr, int kx, const XSlice& xs,
                                              u4 v, int f) {
    const XPos p = x_pos<ONE_ROW>(xs, f);
    const int col = xs.c0 + p.c;
    if constexpr (!BIASED) {
        smem[p.m * l.xs + col] = v;
    } else {
        const h2 lo = h2{static_cast<h1>(1.0f), static_cast<h1>(1.0f)};
        const h2 hi = h2{static_cast<h1>(0.0625f), static_cast<h1>(0.0625f)};
        const h2 x0 = bitcast<h2>(v.x), x1 = bitcast<h2>(v.y), x2 = bitcast<h2>(v.z), x3 = bitcast<h2>(v.w);
        const h2 y0 = x0 * lo, y1 = x1 * hi, y2 = x2 * lo, y3 = x3 * hi;
        float a = __builtin_amdgcn_fdot2(y0, lo, 0.0f, false);  // sums on v_dot2 (exact products by 1)
        a = __builtin_amdgcn_fdot2(y1, lo, a, false);
        a = __builtin_amdgcn_fdot2(y2, lo, a, false);
        a = __builtin_amdgcn_fdot2(y3, lo, a, false);
        float b = __builtin_amdgcn_fdot2(x0, lo, 0.0f, false);
        b = __builtin_amdgcn_fdot2(x1, lo, b, false);
        b = __builtin_amdgcn_fdot2(x2, lo, b, false);
        b = __builtin_amdgcn_fdot2(x3, lo, b, false);
        a += lane_xor1(a);
        b += lane_xor1(b);
        a += lane_xor2(a);
        b += lane_xor2(b);
        smem[p.m * l.xs + col] =
            u4{bitcast<uint32_t>(y0), bitcast<uint32_t>(y1), bitcast<uint32_t>(y2), bitcast<uint32_t>(y3)};
        if ((col & 3) == 0 && f < xs.n) corr[p.m * (kx >> 2) + (col >> 2)] = float2{-1024.0f * a, b};
    }
}

// Stores the first batch (already loaded), then loads and stores the rest of the slice batch by
// batch; ends with the wavefront's LDS writes ordered before its reads.
template <bool BIASED, bool ONE_ROW, int XB = kXB>
__device__ __forceinline__ void stage_x(u4* smem, const DecodeLds& l, float2* corr, const u4* xg, int kx,
                                        const XSlice& xs, const u4 (&first)[XB], int lane) {
#pragma unroll
    for (int j = 0; j < XB; ++j) store_x_chunk<BIASED, ONE_ROW>(smem, l, corr, kx, xs, first[j], lane + 64 * j);
    for (int f0 = lane + 64 * XB; f0 - lane < xs.n; f0 += 64 * XB) {  // wavefront-uniform trip count
        u4 v[XB];
        load_x_batch<ONE_ROW, XB>(v, xg, kx, xs, f0);
#pragma unroll
        for (int j = 0; j < XB; ++j) store_x_chunk<BIASED, ONE_ROW>(smem, l, corr, kx, xs, v[j], f0 + 64 * j);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Fused norm prologue: x is replaced by a = fp16(s rstd w) with s = x + r (fp32; r = 0 without a
// residual) and rstd = rsqrt(mean(s^2) + eps) over the whole row, the bits tw4_add_rms_norm /
// tw4_rms_norm would write, then staged as above. The workgroup's wavefronts together cover every
// quant group of K, so each adds its slice's group sums of squares (norm_rstd's order: sumsq8 per
// chunk, row16_sum over the 16 chunks of a group, held by lanes 16 i .. 16 i + 15 of one batch)
// into LDS, and after one workgroup barrier every wavefront reads all G sums of a row. Workgroup 0
// writes the residual sum fp16(s) to r_out after its main loop (never in place: other workgroups
// still read r). Every load up to the end of staging is unconditional (a missing residual is read
// as x and not added; an empty slice reads chunk 0) and no store is issued, so each wait for x
// counts exactly and never waits for the weight chunk issued behind it.
struct NormIn {
    const h1* r;  // residual [M, K], or null: plain RMSNorm of x
    h1* r_out;    // fp16(x + r) [M, K] (when r)
    const h1* w;  // norm weight [K]
    float eps;
};

constexpr int kNormMaxRows = 16;

// s = x + r per element, as one fma on the fp16 operands (v_fma_mix_f32: no conversions): r * rw + x
// with rw = 1 (a residual) or 0 (none: rv then holds x, and x + x * 0 = x). The same bits as
// converting both and adding in fp32.
__device__ __forceinline__ void norm_sum(const u4& xv, const u4& rv, float rw, float (&s)[8]) {
    const h2 x[4] = {bitcast<h2>(xv.x), bitcast<h2>(xv.y), bitcast<h2>(xv.z), bitcast<h2>(xv.w)};
    const h2 r[4] = {bitcast<h2>(rv.x), bitcast<h2>(rv.y), bitcast<h2>(rv.z), bitcast<h2>(rv.w)};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s[2 * i] = __builtin_fmaf(static_cast<float>(r[i].x), rw, static_cast<float>(x[i].x));
        s[2 * i + 1] = __builtin_fmaf(static_cast<float>(r[i].y), rw, static_cast<float>(x[i].y));
    }
}

// rg: the residual, or x itself when there is none (loaded, not added).
template <bool ONE_ROW, bool W>
__device__ __forceinline__ void load_norm_batch(u4 (&xv)[kXB], u4 (&rv)[kXB], u4 (&wv)[kXB], const u4* xg,
                                                const u4* rg, const u4* wg, int kx, const XSlice& xs, int f0) {
#pragma unroll
    for (int j = 0; j < kXB; ++j) {
        const XPos p = x_pos<ONE_ROW>(xs, f0 + 64 * j);
        xv[j] = x_chunk(xg, kx, xs, p);
        rv[j] = x_chunk(rg, kx, xs, p);
        if constexpr (W) wv[j] = wg[xs.c0 + p.c];
    }
}

template <bool ONE_ROW>
__device__ __forceinline__ void norm_group_sums(float* gsum, const u4 (&xv)[kXB], const u4 (&rv)[kXB], float rw,
                                                const XSlice& xs, int G, int f0, int lane) {
#pragma unroll
    for (int j = 0; j < kXB; ++j) {
        float sv[8];
        norm_sum(xv[j], rv[j], rw, sv);
        const float q = row16_sum(sumsq8(sv));
        const int f = f0 + 64 * j;
        const XPos p = x_pos<ONE_ROW>(xs, f);
        if ((lane & 15) == 0 && f < xs.n) gsum[p.m * G + ((xs.c0 + p.c) >> 4)] = q;
    }
}

template <bool BIASED, bool ONE_ROW, int MR>
__device__ __forceinline__ void norm_store_batch(u4* smem, const DecodeLds& l, float2* corr, int kx, const XSlice& xs,
                                                 const u4 (&xv)[kXB], const u4 (&rv)[kXB], const u4 (&wv)[kXB],
                                                 float rw, const float (&rstd)[MR], int f0) {
#pragma unroll
    for (int j = 0; j < kXB; ++j) {
        const int f = f0 + 64 * j;
        const XPos p = x_pos<ONE_ROW>(xs, f);
        float sv[8];
        norm_sum(xv[j], rv[j], rw, sv);
        float rs = rstd[0];
#pragma unroll
        for (int m = 1; m < MR; ++m) rs = p.m == m ? rstd[m] : rs;
        const h2 g[4] = {bitcast<h2>(wv[j].x), bitcast<h2>(wv[j].y), bitcast<h2>(wv[j].z), bitcast<h2>(wv[j].w)};
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // (s rstd) g: the product with the fp16 g as an fma with -0 (exact)
            sv[2 * i] = __builtin_fmaf(sv[2 * i] * rs, static_cast<float>(g[i].x), -0.0f);
            sv[2 * i + 1] = __builtin_fmaf(sv[2 * i + 1] * rs, static_cast<float>(g[i].y), -0.0f);
        }
        store_x_chunk<BIASED, ONE_ROW>(smem, l, corr, kx, xs, f32_to_chunk(sv), f);
    }
}

// Called by every wavefront of the workgroup (it holds a workgroup barrier); a wavefront with an
// empty slice only takes part in the barrier. fx / fr / fw: the slice's first batch, already loaded.
template <bool BIASED, bool ONE_ROW, int MR>
__device__ __forceinline__ void stage_x_norm(u4* smem, const DecodeLds& l, float2* corr, const u4* xg, int kx,
                                             const XSlice& xs, const NormIn& nin, int M, int G, int K,
                                             const u4 (&fx)[kXB], const u4 (&fr)[kXB], const u4 (&fw)[kXB],
                                             int lane) {
    float* gsum = reinterpret_cast<float*>(smem + l.norm);  // [M][G]
    const bool has_r = nin.r != nullptr;
    const u4* rg = has_r ? reinterpret_cast<const u4*>(nin.r) : xg;
    const float rw = has_r ? 1.0f : 0.0f;
    const u4* wg = reinterpret_cast<const u4*>(nin.w);
    if (xs.n > 0) {
        norm_group_sums<ONE_ROW>(gsum, fx, fr, rw, xs, G, lane, lane);
        for (int f0 = lane + 64 * kXB; f0 - lane < xs.n; f0 += 64 * kXB) {  // wavefront-uniform trip count
            u4 xv[kXB], rv[kXB], wv[kXB];
            load_norm_batch<ONE_ROW, false>(xv, rv, wv, xg, rg, wg, kx, xs, f0);
            norm_group_sums<ONE_ROW>(gsum, xv, rv, rw, xs, G, f0, lane);
        }
    }
    __syncthreads();
    float rstd[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m)
        rstd[m] = m < M ? norm_rstd(gsum + m * G, G, K, nin.eps, lane) : 0.0f;  // wavefront-uniform branch
    if (xs.n > 0) {
        norm_store_batch<BIASED, ONE_ROW, MR>(smem, l, corr, kx, xs, fx, fr, fw, rw, rstd, lane);
        for (int f0 = lane + 64 * kXB; f0 - lane < xs.n; f0 += 64 * kXB) {
            u4 xv[kXB], rv[kXB], wv[kXB];
            load_norm_batch<ONE_ROW, true>(xv, rv, wv, xg, rg, wg, kx, xs, f0);
            norm_store_batch<BIASED, ONE_ROW, MR>(smem, l, corr, kx, xs, xv, rv, wv, rw, rstd, f0);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup 0, after its main loop: fp16(x + r) of the wavefront's slice into r_out.
template <bool ONE_ROW>
__device__ __forceinline__ void write_residual(const u4* xg, const NormIn& nin, int kx, const XSlice& xs, int lane) {
    if (nin.r == nullptr || blockIdx.x != 0) return;
    const u4* rg = reinterpret_cast<const u4*>(nin.r);
    u4* rog = reinterpret_cast<u4*>(nin.r_out);
    for (int f0 = lane; f0 - lane < xs.n; f0 += 64 * kXB) {
        u4 xv[kXB], rv[kXB], wv[kXB];
        load_norm_batch<ONE_ROW, false>(xv, rv, wv, xg, rg, nullptr, kx, xs, f0);
#pragma unroll
        for (int j = 0; j < kXB; ++j) {
            const int f = f0 + 64 * j;
            const XPos p = x_pos<ONE_ROW>(xs, f);
            float sv[8];
            norm_sum(xv[j], rv[j], 1.0f, sv);
            if (f < xs.n) rog[static_cast<int64_t>(p.m) * kx + xs.c0 + p.c] = f32_to_chunk(sv);
        }
    }
}

__device__ __forceinline__ GroupQ group_q_raw(uint32_t s, uint32_t z, bool valid) {
    return group_q(valid ? as_h1(s) : static_cast<h1>(0.0f), as_h1(z));
}

// ------------------------------------------------------------------------------------ gemv
// The group's dot products run on the raw magic halves against x' (fill_x_biased): 4 v_and_or_b32,
// one shift and 4 v_dot2 per word; the zero point and the 1024 bias come off once per group:
// acc += s (dot - 1024 A - z B).
template <bool PF, int M, int U, int NT, int DIST = 1>
__device__ __forceinline__ void gemv_chunk(const WeightSet<U, NT>& cur, WeightSet<U, NT>& nxt, const TileStreams<NT>& ts,
                                           const uint16_t* s16, const uint16_t* z16, const u4* lx, const float2* corr,
                                           const DecodeLds& l, float (&acc)[NT][M], int g0, int ge, int G, int kb,
                                           uint32_t magic) {
    if constexpr (PF) load_chunk<U, NT>(nxt, ts, s16, z16, g0 + DIST * U, ge - 1);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch above the math: the scheduler would sink it
#pragma unroll
    for (int u = 0; u < U; ++u) {
        // a chunk that prefetches is not the wavefront's last: all its groups are in range
        const int graw = g0 + u;
        const bool valid = PF || graw < ge;
        const int g = PF ? graw : min(graw, ge - 1);
        // the slice's sums start at -1024 A (the bias correction, precomputed) and take the dots
        float part[NT][M];
        float2 c[M];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            c[m] = corr[(m * G + g) * 4 + kb];
#pragma unroll
            for (int t = 0; t < NT; ++t) part[t][m] = c[m].x;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            u4 xq[M];  // x'[m][128 g + 32 kb + 8 s .. + 7]
#pragma unroll
            for (int m = 0; m < M; ++m) xq[m] = lx[m * l.xs + 16 * g + 4 * kb + s];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                h2 d[4];
                unpack_raw(word_of(cur.w[u][t], s), magic, d);
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
            uint32_t s_raw, z_raw;
            scale_zero(cur.p[u][t], s_raw, z_raw);
            const float sc = static_cast<float>(as_h1(s_raw));
            const float zf = static_cast<float>(as_h1(z_raw));
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float v = __builtin_fmaf(-zf, c[m].y, part[t][m]);
                acc[t][m] = valid ? __builtin_fmaf(v, sc, acc[t][m]) : acc[t][m];
            }
        }
    }
}

template <int M, int WK, int U, int NT, bool NORM>
__global__ void __launch_bounds__(WK * 64) gemv_kernel(const h1* __restrict__ x, const u4* __restrict__ w,
                                                      const h1* __restrict__ scales, const h1* __restrict__ zeros,
                                                      h1* __restrict__ y, int N, int K, int act, NormIn nin) {
    extern __shared__ u4 smem[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: SGPR
    const int r = lane & 15, kb = lane >> 4;
    const int G = K >> 7, tiles = (N + 15) >> 4;
    const int tile0 = xcd_rotated_block((tiles + NT - 1) / NT) * NT;  // the launch's grid
    const DecodeLds l = decode_lds(true, M, K, gemv_corr_u4(M, K), gemv_red_u4(M, WK, NT), NORM);
    const uint32_t magic = magic_reg();
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(scales);
    const uint16_t* z16 = reinterpret_cast<const uint16_t*>(zeros);
    TileStreams<NT> ts = tile_streams<NT>(w, s16, z16, tile0, tiles, N, G, lane);
    const int gw = (G + WK - 1) / WK, gb = min(wave * gw, G), ge = min(gb + gw, G);
    const int nch = (ge - gb + U - 1) / U;
    float2* corr = reinterpret_cast<float2*>(smem + l.corr);

    const int kx = K >> 3;
    const u4* xg = reinterpret_cast<const u4*>(x);
    const XSlice xsl = x_slice(gb, ge, M);
    WeightSet<U, NT> a, b;
    if constexpr (NORM) {  // no branch around these loads (see stage_x_norm); ge - 1 >= 0 is a valid group
        u4 fx[kXB], fr[kXB], fw[kXB];
        load_norm_batch<M == 1, true>(fx, fr, fw, xg, nin.r ? reinterpret_cast<const u4*>(nin.r) : xg,
                                      reinterpret_cast<const u4*>(nin.w), kx, xsl, lane);
        __builtin_amdgcn_sched_barrier(0);
        load_chunk<U, NT>(a, ts, s16, z16, gb, max(ge - 1, 0));
        __builtin_amdgcn_sched_barrier(0);
        stage_x_norm<true, M == 1, M>(smem, l, corr, xg, kx, xsl, nin, M, G, K, fx, fr, fw, lane);
    } else {  // unconditional as well: a branch here makes the compiler wait for the whole first chunk
        u4 xfirst[kXB];
        load_x_batch<M == 1>(xfirst, xg, kx, xsl, lane);
        __builtin_amdgcn_sched_barrier(0);
        load_chunk<U, NT>(a, ts, s16, z16, gb, max(ge - 1, 0));
        __builtin_amdgcn_sched_barrier(0);
        stage_x<true, M == 1>(smem, l, corr, xg, kx, xsl, xfirst, lane);
    }

    float acc[NT][M];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[t][m] = 0.0f;
    int i = 0;
    if constexpr (U == 1) {
        // three one-group sets: chunk j computes set j % 3 and prefetches chunk j + 2 into set
        // (j + 2) % 3, two groups in flight while one is computed; the last two chunks prefetch nothing.
        // Against one group ahead (the loop below at U = 1), measured on the Qwen3-8B shapes at
        // M = 1: qkv (8, 1, 1) 4.59 -> 4.34 us, o (8, 1, 1) 4.06 -> 3.51, down (8, 1, 1) 7.50 -> 6.89;
        // the last chunk's arithmetic stays one group, where a two-group chunk (U = 2) doubles it.
        WeightSet<U, NT> c;
        load_chunk<U, NT>(b, ts, s16, z16, gb + 1, max(ge - 1, 0));
        for (; i + 4 < nch; i += 3) {
            gemv_chunk<true, M, U, NT, 2>(a, c, ts, s16, z16, smem, corr, l, acc, gb + i, ge, G, kb, magic);
            gemv_chunk<true, M, U, NT, 2>(b, a, ts, s16, z16, smem, corr, l, acc, gb + i + 1, ge, G, kb, magic);
            gemv_chunk<true, M, U, NT, 2>(c, b, ts, s16, z16, smem, corr, l, acc, gb + i + 2, ge, G, kb, magic);
        }
        const int rem = nch - i;
        if (rem == 4) {
            gemv_chunk<true, M, U, NT, 2>(a, c, ts, s16, z16, smem, corr, l, acc, gb + i, ge, G, kb, magic);
            gemv_chunk<true, M, U, NT, 2>(b, a, ts, s16, z16, smem, corr, l, acc, gb + i + 1, ge, G, kb, magic);
            gemv_chunk<false, M, U, NT>(c, b, ts, s16, z16, smem, corr, l, acc, gb + i + 2, ge, G, kb, magic);
            gemv_chunk<false, M, U, NT>(a, b, ts, s16, z16, smem, corr, l, acc, gb + i + 3, ge, G, kb, magic);
        } else if (rem == 3) {
            gemv_chunk<true, M, U, NT, 2>(a, c, ts, s16, z16, smem, corr, l, acc, gb + i, ge, G, kb, magic);
            gemv_chunk<false, M, U, NT>(b, a, ts, s16, z16, smem, corr, l, acc, gb + i + 1, ge, G, kb, magic);
            gemv_chunk<false, M, U, NT>(c, b, ts, s16, z16, smem, corr, l, acc, gb + i + 2, ge, G, kb, magic);
        } else if (rem == 2) {
            gemv_chunk<false, M, U, NT>(a, c, ts, s16, z16, smem, corr, l, acc, gb + i, ge, G, kb, magic);
            gemv_chunk<false, M, U, NT>(b, c, ts, s16, z16, smem, corr, l, acc, gb + i + 1, ge, G, kb, magic);
        } else if (rem == 1) {
            gemv_chunk<false, M, U, NT>(a, c, ts, s16, z16, smem, corr, l, acc, gb + i, ge, G, kb, magic);
        }
    } else {
    // steady state: every chunk prefetches the next; the wavefront's last chunk prefetches nothing
    for (; i + 2 < nch; i += 2) {
        gemv_chunk<true, M, U, NT>(a, b, ts, s16, z16, smem, corr, l, acc, gb + U * i, ge, G, kb, magic);
        gemv_chunk<true, M, U, NT>(b, a, ts, s16, z16, smem, corr, l, acc, gb + U * (i + 1), ge, G, kb, magic);
    }
    if (i + 2 == nch) {
        gemv_chunk<true, M, U, NT>(a, b, ts, s16, z16, smem, corr, l, acc, gb + U * i, ge, G, kb, magic);
        gemv_chunk<false, M, U, NT>(b, a, ts, s16, z16, smem, corr, l, acc, gb + U * (i + 1), ge, G, kb, magic);
    } else if (i + 1 == nch) {
        gemv_chunk<false, M, U, NT>(a, b, ts, s16, z16, smem, corr, l, acc, gb + U * i, ge, G, kb, magic);
    }
    }
    if constexpr (NORM) write_residual<M == 1>(xg, nin, kx, xsl, lane);
    // lanes r, r + 16, r + 32, r + 48 hold the four k slices of row r
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            acc[t][m] = sum_rows(acc[t][m]);
        }
    if (WK > 1) {
        float* red = reinterpret_cast<float*>(smem + l.red);  // [WK][NT * M][16]
        if (kb == 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int m = 0; m < M; ++m) red[(wave * NT * M + t * M + m) * 16 + r] = acc[t][m];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int v = 1; v < WK; ++v)
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int m = 0; m < M; ++m) acc[t][m] += red[(v * NT * M + t * M + m) * 16 + r];
    }
    if (act) {  // N % 16 == 0 (checked on the host): gate row i of the tile in lane i, up row 8 + i in lane i + 8
        const int half_n = N >> 1;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int tt = tile0 + t;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float up = __int_as_float(
                    __builtin_amdgcn_update_dpp(0, __float_as_int(acc[t][m]), 0x128, 0xF, 0xF, false));  // row_ror:8
                if (kb == 0 && r < 8 && tt < tiles)
                    y[static_cast<int64_t>(m) * half_n + 8 * tt + r] = static_cast<h1>(silu(acc[t][m]) * up);
            }
        }
        return;
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

// Compiled decode configurations (warps_k, unroll, ntile).
#define TW4_DECODE_CONFIGS(X)                                                                            \
    X(1, 4, 1) X(1, 8, 1) X(2, 4, 1) X(2, 8, 1) X(4, 1, 1) X(4, 2, 1) X(4, 4, 1) X(4, 8, 1) X(8, 1, 1) \
    X(8, 2, 1) X(8, 4, 1) X(16, 1, 1) X(16, 2, 1) X(2, 4, 2) X(4, 2, 2) X(4, 4, 2) X(8, 1, 2) X(8, 2, 2)

// Row-tile-wide configurations of the matrix-core decode kernel only (warps_k, unroll, ntile): up to
// six row tiles per workgroup, x read from global memory (L2) at every chunk and never staged in LDS,
// so each wavefront's x fragments feed ntile weight blocks and no workgroup pays a staging phase. For
// projections with many row tiles (gate_up): measured on Qwen3-8B gate_up, (4, 1, 6) at M = 32 took
// 17.9-18.6 us against 20.2-21.2 us for the x-ring GEMM, (4, 1, 3) at M = 8 12.5 against 13.1 us.
#define TW4_MMA_WIDE_CONFIGS(X) X(4, 1, 2) X(4, 1, 3) X(4, 1, 6) X(4, 2, 3)

constexpr int kMaxDevices = 64;
constexpr int kMaxLds = 160 * 1024;      // gfx950 LDS per workgroup
constexpr int kXLdsLimit = 80 * 1024;    // mma keeps x in LDS up to this size (M = 8 at K = 4096)
constexpr int kXLdsBig = 136 * 1024;     // ... and up to this one when the grid has at most one workgroup per CU

// Launch the vector-ALU GEMV (M <= 4) of one compiled configuration. LDS beyond 64 KB needs the
// kernel's hipFuncSetAttribute (tw4_init / the first call).
template <int M, bool NORM>
int gemv_dispatch(const h1* x, const u4* w, const h1* s, const h1* z, h1* y, int N, int K, int wk, int un, int nt,
                  int act, const NormIn& nin, hipStream_t st) {
    const int tiles = (N + 15) >> 4;
#define TW4_GEMV_CASE(WK, U, T)                                                                              \
    if (wk == WK && un == U && nt == T) {                                                                    \
        const size_t lds =                                                                                   \
            16 * static_cast<size_t>(decode_lds(true, M, K, gemv_corr_u4(M, K), gemv_red_u4(M, WK, T), NORM).total); \
        TW4_REQUIRE(lds <= static_cast<size_t>(kMaxLds), TW4_EINVAL,                                        \
                    "gemv: x [%d, %d] does not fit in LDS (use mma)", M, K);                                 \
        gemv_kernel<M, WK, U, T, NORM><<<(tiles + T - 1) / T, WK * 64, lds, st>>>(x, w, s, z, y, N, K, act, nin); \
        TW4_LAUNCH_CHECK("gemv: launch");                                                                    \
        return TW4_OK;                                                                                       \
    }
    TW4_DECODE_CONFIGS(TW4_GEMV_CASE)
#undef TW4_GEMV_CASE
    tw4host::set_error("gemv: unsupported warps_k / unroll / ntile %d / %d / %d", wk, un, nt);
    return TW4_ECONFIG;
}

template <typename Kern>
int allow_lds(Kern kern) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       kMaxLds);
    return e == hipSuccess ? TW4_OK : tw4host::hip_fail(e, "init: decode hipFuncSetAttribute");
}

// Host-side argument checks shared by the decode entry points (tw4_decode.hip).
int check_operands(const char* who, const void* x, const int32_t* packed, const uint16_t* scales,
                   const uint16_t* zeros, const void* y, int M, int N, int K);

}  // namespace tw4
