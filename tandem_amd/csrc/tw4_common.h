// Shared device helpers and host plumbing of libtandem_w4.so (gfx950 only).
//
// Tile layout (see include/tandem_w4.h): row tile T (16 rows) x quant group g is one 1 KB block
// of 256 int32 words ordered [kb 4][r 16][s 4]; word (kb, r, s) holds weights
// k = 128 g + 32 kb + 8 s + o of row 16 T + r, weight o = 2 q + e in nibble q + 4 e.
// Lane l = 16 kb + r of a wavefront loads the 16 bytes (kb, r, s = 0..3) of a block with one
// global_load_dwordx4, so a wavefront load of a block is 1 KB contiguous.
//
// The k order inside a word is the one that lets four v_and_or_b32 turn a word into four
// half2 values with no integer-to-float conversion (the fp16 "magic number" trick: an fp16 with
// bit pattern 0x6400 | m, m < 1024, has the value 1024 + m; published with FasterTransformer's
// and Marlin's int4 dequantization). Pair q of the word, (weights 2q, 2q + 1), is nibbles
// (q, q + 4): bits 4q .. 4q+3 and 16 + 4q .. 16 + 4q + 3.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tandem_w4.h"

namespace tw4 {

typedef _Float16 h1;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kGroup = 128;       // quant group (k values per scale / zero)
constexpr int kTileRows = 16;     // rows per row tile
constexpr int kBlockWords = 256;  // int32 words per (row tile, group) block
constexpr int kBlockU4 = 64;      // 16-byte vectors per block (one per lane)

template <typename T, typename F>
__device__ __forceinline__ T bitcast(F v) {
    return __builtin_bit_cast(T, v);
}

// Per (row, group) constants of the in-register dequantization.
struct GroupQ {
    h2 zlo;  // -(1024 + z): subtracted from a low-nibble magic half (1024 + q)
    h2 zhi;  // -(64 + z):   added to a high-nibble magic half times 1/16 ((1024 + 16 q) / 16)
    h2 s;    // scale
};

__device__ __forceinline__ GroupQ group_q(h1 s, h1 z) {
    GroupQ p;
    const h1 lo = -(z + static_cast<h1>(1024.0f));
    const h1 hi = -(z + static_cast<h1>(64.0f));
    p.zlo = h2{lo, lo};
    p.zhi = h2{hi, hi};
    p.s = h2{s, s};
    return p;
}

// The magic constant 0x64006400 must live in a VGPR for the compiler to fuse the mask and the
// or into one v_and_or_b32 (a gfx9 VOP3 instruction encodes no 32-bit literal): kernels create
// it once with magic_reg() and pass it down.
__device__ __forceinline__ uint32_t magic_reg() {
    uint32_t m = 0x64006400u;
    asm volatile("" : "+v"(m));
    return m;
}

// One word -> its 8 weights (q - z), exact in fp16 (integers -15 .. 15), in k order.
__device__ __forceinline__ void unpack_qz(uint32_t w, const GroupQ& p, uint32_t magic, h2 (&d)[4]) {
    const uint32_t w8 = w >> 8;
    const h2 sixteenth = h2{static_cast<h1>(0.0625f), static_cast<h1>(0.0625f)};
    d[0] = bitcast<h2>((w & 0x000F000Fu) | magic) + p.zlo;               // k 0, 1
    d[1] = bitcast<h2>((w & 0x00F000F0u) | magic) * sixteenth + p.zhi;   // k 2, 3
    d[2] = bitcast<h2>((w8 & 0x000F000Fu) | magic) + p.zlo;              // k 4, 5
    d[3] = bitcast<h2>((w8 & 0x00F000F0u) | magic) * sixteenth + p.zhi;  // k 6, 7
}

// One word -> its 8 dequantized weights fp16_rne((q - z) * s) in k order: the exact integer
// (q - z) times s is a single rounding, so the bits equal fp32 (q - z) * s rounded to fp16.
__device__ __forceinline__ h8 dequant_word(uint32_t w, const GroupQ& p, uint32_t magic) {
    h2 d[4];
    unpack_qz(w, p, magic, d);
    d[0] *= p.s;
    d[1] *= p.s;
    d[2] *= p.s;
    d[3] *= p.s;
    return h8{d[0].x, d[0].y, d[1].x, d[1].y, d[2].x, d[2].y, d[3].x, d[3].y};
}

// Scales and zeros are loaded as raw 16-bit values into 32-bit registers, and only turned into
// fp16 where they are used: the compiler then has no reason to touch a prefetched value (and
// wait for its load) before the step that needs it.
__device__ __forceinline__ uint32_t load_u16(const h1* p) { return *reinterpret_cast<const uint16_t*>(p); }
__device__ __forceinline__ h1 as_h1(uint32_t v) { return bitcast<h1>(static_cast<uint16_t>(v)); }

__device__ __forceinline__ uint32_t word_of(const u4& v, int i) {  // i constant after unrolling
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ u4 load_stream(const u4* p) {  // weights: read once, do not keep
    return __builtin_nontemporal_load(p);
}

// Raw buffer resource word 3 for gfx9-family data loads (32-bit data format, no swizzle).
constexpr int kBufferFlags = 0x00020000;

// Lane `lane`'s 16 bytes of weight block g of a tile, through the tile's buffer resource: the
// block offset g * 1024 goes in the scalar offset and the lane offset in the vector one, so a
// stream of blocks costs no per-lane 64-bit address arithmetic. Non-temporal (aux = 2: nt).
__device__ __forceinline__ u4 load_block(__amdgpu_buffer_rsrc_t rs, int g, int lane) {
    return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, g * (kBlockU4 * 16), 2));
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

// Cross-lane exchanges on the VALU (DPP and gfx950's permlane swaps) instead of the LDS crossbar.
// DPP quad_perm [1, 0, 3, 2] and [2, 3, 0, 1]: the value of lane l ^ 1 and of lane l ^ 2.
__device__ __forceinline__ float lane_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}

// v_permlane16_swap / v_permlane32_swap on two copies of v leave rows {0, 2} / {1, 3} (resp. the
// lower / upper 32 lanes) of v in every lane of the first / second result. Sum of lanes r, r + 16,
// r + 32, r + 48 in every lane, added as (v0 + v1) + (v2 + v3).
__device__ __forceinline__ float sum_rows(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Sum of the 16 lanes of each row (lanes 16 i .. 16 i + 15), the same bits in all 16 lanes: every
// step adds the values of a lane pair that exchange with each other (l ^ 1, l ^ 2, then DPP
// row_half_mirror and row_mirror), and floating-point addition is commutative.
__device__ __forceinline__ float row16_sum(float v) {
    v += lane_xor1(v);
    v += lane_xor2(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // half mirror
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));  // row mirror
    return v;
}

// Sum over the 64 lanes, the same bits in every lane: (R0 + R1) + (R2 + R3) of the row sums.
__device__ __forceinline__ float wave_total(float v) { return sum_rows(row16_sum(v)); }

// Sum of squares of 8 fp32 values in a fixed order (all fma, so no contraction choice is left to
// the compiler).
__device__ __forceinline__ float sumsq8(const float (&s)[8]) {
    float q = __builtin_fmaf(s[0], s[0], 0.0f);
#pragma unroll
    for (int i = 1; i < 8; ++i) q = __builtin_fmaf(s[i], s[i], q);
    return q;
}

// 8 halves of a 16-byte chunk as fp32, and 8 fp32 values rounded (RNE) into a chunk.
__device__ __forceinline__ void chunk_to_f32(const u4& v, float (&f)[8]) {
    const h2 a = bitcast<h2>(v.x), b = bitcast<h2>(v.y), c = bitcast<h2>(v.z), d = bitcast<h2>(v.w);
    f[0] = a.x, f[1] = a.y, f[2] = b.x, f[3] = b.y, f[4] = c.x, f[5] = c.y, f[6] = d.x, f[7] = d.y;
}
__device__ __forceinline__ u4 f32_to_chunk(const float (&f)[8]) {
    return u4{bitcast<uint32_t>(h2{static_cast<h1>(f[0]), static_cast<h1>(f[1])}),
              bitcast<uint32_t>(h2{static_cast<h1>(f[2]), static_cast<h1>(f[3])}),
              bitcast<uint32_t>(h2{static_cast<h1>(f[4]), static_cast<h1>(f[5])}),
              bitcast<uint32_t>(h2{static_cast<h1>(f[6]), static_cast<h1>(f[7])})};
}

// RMS normalisation with its sum of squares in one fixed order, shared by the norm kernels and the
// decode kernels' fused norm prologue, so both produce the same bits. For a row of K halves
// (K % 128 == 0): chunk c = values 8 c .. 8 c + 7 gives q_c = sumsq8; quant group g (chunks
// 16 g .. 16 g + 15, held by lanes 16 i .. 16 i + 15 of one row of a wavefront) gives
// S_g = row16_sum(q); lane l of one wavefront adds S_l, S_(l+64), ... in increasing order and
// wave_total adds the lanes. rstd = rsqrt(total / K + eps).
__device__ __forceinline__ float norm_rstd(const float* gsum, int G, int K, float eps, int lane) {
    float t = 0.0f;
    for (int g = lane; g < G; g += 64) t += gsum[g];
    return rsqrtf(wave_total(t) / static_cast<float>(K) + eps);
}

// The value of lane l ^ 32.
__device__ __forceinline__ float lane_xor32(float v, int lane) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(lane < 32 ? a[1] : a[0]);
}

__device__ __forceinline__ f4 mfma16x16x32(const h8& a, const h8& b, const f4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Scales and zeros are [N, K/128] fp16 buffers stored tile-major: the values of row tile T are
// [group][row in tile], so the 16 rows of one group are 32 contiguous bytes (one load by a
// wavefront touches one segment). Row tile T holds rows_t = min(16, N - 16 T) rows (only the last
// tile of an N % 16 != 0 matrix has 8), and every earlier tile is full:
//     offset(n, g) = 16 T G + g rows_t + (n - 16 T),   T = n / 16.
__host__ __device__ __forceinline__ int tile_rows(int t, int n) { return min(16, n - 16 * t); }
__host__ __device__ __forceinline__ int64_t param_offset(int row, int g, int n, int G) {
    const int t = row >> 4;
    return static_cast<int64_t>(16) * t * G + static_cast<int64_t>(g) * tile_rows(t, n) + (row & 15);
}

// Row of the interleave_gate_up order: destination row n' = 16 T + 8 h + i holds source row
// h * N/2 + 8 T + i.
__host__ __device__ __forceinline__ int interleaved_source_row(int nprime, int n) {
    const int t = nprime >> 4, h = (nprime >> 3) & 1, i = nprime & 7;
    return h * (n >> 1) + 8 * t + i;
}
__host__ __device__ __forceinline__ int interleaved_dest_row(int src, int n) {
    const int half = n >> 1, h = src >= half ? 1 : 0, rem = src - h * half;
    return 16 * (rem >> 3) + 8 * h + (rem & 7);
}

// Workgroups are dealt to the 8 XCDs round robin (workgroup b runs on XCD b mod 8); renumbering them so
// that XCD x gets a contiguous range of work units keeps the units that share weight or x tiles in one
// XCD's L2. A permutation of 0 .. n - 1 (the first n mod 8 XCDs take one unit more).
__device__ __forceinline__ int xcd_remap(int b, int n) {
    if (n < 16) return b;
    const int q = n >> 3, rr = n & 7, xcd = b & 7, idx = b >> 3;
    return xcd < rr ? xcd * (q + 1) + idx : rr * (q + 1) + (xcd - rr) * q + idx;
}

// The end of a work unit, run by every thread of the workgroup. Wavefronts with `holder` set hold
// the unit's fp32 tiles (rows 16 (wt0 + t) .., tokens m0 + 16 b ..) in acc. nsplit > 1: each stores
// its partial to split slot su of ws; one agent-scope counter per split tile (st) tells the last
// arriver, which adds the nsplit partials of the tile in split order (the result does not depend
// on arrival order), returns the counter to zero for the next call and writes y. Each wavefront
// partial is stored [fragment][lane][component]: one 16-byte store or load per lane and fragment,
// 1 KB contiguous per instruction. Stores and loads carry sc1, the cache policy of agent-scope
// atomics on gfx950 (the compiler's relaxed agent-scope load / store): they are coherent across
// the XCDs' L2s without a cache-wide write-back or invalidate. s_waitcnt vmcnt(0) + barrier order
// the stores before the count; the last arriver issues its loads only after it has seen the count
// reach nsplit. The last arriver loads the partials of VB splits at a time (one memory round trip
// per VB splits) and adds them in split order. act = 1: SwiGLU epilogue (gate rows 4 kb + i and up
// rows 8 + 4 kb + i sit in lanes l and l + 32).
constexpr int kCoherentAux = 16;  // buffer-instruction cache policy: sc1
constexpr int64_t kMaxPartialFloats = int64_t(1) << 29;  // split-K workspace used: byte offsets < 2^31

template <int MT, int NT, int WN, int PART_FLOATS = 64>
__device__ __forceinline__ void finish_unit(f4 (&acc)[NT][MT], bool holder, int wn, int lane, int tid, int nsplit,
                                            int st, int su, float* __restrict__ ws, int* __restrict__ locks,
                                            int& last_flag, h1* __restrict__ y, int M, int N, int m0, int wt0,
                                            int tiles_n, int act) {
    const int r = lane & 15, kb = lane >> 4;
    if (nsplit > 1) {
        constexpr int V = NT * MT * 4 * 64;  // floats per wavefront partial
        // byte offsets below 2^31: the launchers use at most kMaxPartialFloats of the workspace
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(ws, 0, 0x7FFFFFFF, kBufferFlags);
        if (holder) {
            const int mine = static_cast<int>((static_cast<int64_t>(su) * WN + wn) * V * 4);
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int b = 0; b < MT; ++b)
                    __builtin_amdgcn_raw_buffer_store_b128(bitcast<u4>(acc[t][b]), rs, ((t * MT + b) * 64 + lane) * 16,
                                                           mine, kCoherentAux);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(locks + st, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_flag = old == nsplit - 1;
        }
        __syncthreads();
        if (!last_flag) return;
        if (holder) {
            constexpr int F = NT * MT;                        // 16-byte fragments per lane of one partial
            constexpr int VB = 4 * F >= PART_FLOATS ? 1 : PART_FLOATS / (4 * F);  // splits per round
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int b = 0; b < MT; ++b) acc[t][b] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            for (int v0 = 0; v0 < nsplit; v0 += VB) {
                f4 part[VB][F];
#pragma unroll
                for (int j = 0; j < VB; ++j) {
                    const int v = min(v0 + j, nsplit - 1);  // past the last split: re-read it, not added
                    const int other = static_cast<int>(((static_cast<int64_t>(st) * nsplit + v) * WN + wn) * V * 4);
#pragma unroll
                    for (int i = 0; i < F; ++i)
                        part[j][i] = bitcast<f4>(__builtin_amdgcn_raw_buffer_load_b128(rs, (i * 64 + lane) * 16, other,
                                                                                       kCoherentAux));
                }
#pragma unroll
                for (int j = 0; j < VB; ++j) {
                    if (v0 + j >= nsplit) break;  // uniform
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int b = 0; b < MT; ++b) acc[t][b] += part[j][t * MT + b];
                }
            }
        }
        if (tid == 0) __hip_atomic_store(locks + st, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!holder) return;

    if (act) {  // N % 16 == 0 (checked on the host)
        const int half_n = N >> 1;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int tt = wt0 + t;
#pragma unroll
            for (int b = 0; b < MT; ++b) {
                f4 up;
                up.x = lane_xor32(acc[t][b].x, lane);
                up.y = lane_xor32(acc[t][b].y, lane);
                up.z = lane_xor32(acc[t][b].z, lane);
                up.w = lane_xor32(acc[t][b].w, lane);
                const int m = m0 + 16 * b + r;
                if (kb >= 2 || m >= M || tt >= tiles_n) continue;
                const f4 g = acc[t][b];
                const h4 o = h4{static_cast<h1>(silu(g.x) * up.x), static_cast<h1>(silu(g.y) * up.y),
                                static_cast<h1>(silu(g.z) * up.z), static_cast<h1>(silu(g.w) * up.w)};
                *reinterpret_cast<h4*>(y + static_cast<int64_t>(m) * half_n + 8 * tt + 4 * kb) = o;
            }
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int n = 16 * (wt0 + t) + 4 * kb;  // N % 8 == 0: n < N implies n + 3 < N
        if (n >= N) continue;
#pragma unroll
        for (int b = 0; b < MT; ++b) {
            const int m = m0 + 16 * b + r;
            if (m >= M) continue;
            const f4 a = acc[t][b];
            *reinterpret_cast<h4*>(y + static_cast<int64_t>(m) * N + n) =
                h4{static_cast<h1>(a.x), static_cast<h1>(a.y), static_cast<h1>(a.z), static_cast<h1>(a.w)};
        }
    }
}

}  // namespace tw4

// ------------------------------------------------------------------------------- host plumbing
namespace tw4host {

void set_error(const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);

}  // namespace tw4host

#define TW4_REQUIRE(cond, code, ...)          \
    do {                                      \
        if (!(cond)) {                        \
            tw4host::set_error(__VA_ARGS__);  \
            return (code);                    \
        }                                     \
    } while (0)

#define TW4_LAUNCH_CHECK(what)                                           \
    do {                                                                 \
        hipError_t e_ = hipGetLastError();                               \
        if (e_ != hipSuccess) return tw4host::hip_fail(e_, (what));      \
    } while (0)
