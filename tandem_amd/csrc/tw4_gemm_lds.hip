// Fused-dequant GEMM for large M (prefill): y[M, N] = x[M, K] @ dequant(W)^T, with BOTH operand
// tiles staged through LDS by gfx950's direct-to-LDS loads (global_load_lds_dwordx4), a 3-deep ring.
//
// Workgroup tile BM x BN = (WM wavefronts x 16 MT tokens) x (WN wavefronts x 16 NT rows); wavefront
// (wm, wn) computes 16 MT tokens x 16 NT rows. A stage is half a quant group (BK = 64 k): stage s
// covers k = 64 s .. 64 s + 63 of group s / 2.
//   x:       the BM x 64 fp16 tile, 128 B per token row, 8 rows per load instruction. LDS slot
//            (row rho, position p) holds 16-byte chunk p ^ (rho & 7) of the row, so the 16 lanes of a
//            B-fragment read (16 rows, one chunk) hit 8 different bank groups per 8 lanes.
//   weights: the int4 tile as it sits in HBM: the k half of each (row tile, group) 1 KB block is 512
//            contiguous bytes (words kb = 2 h, 2 h + 1 of [kb][r][s]), two row tiles per instruction.
//            Every weight byte is read from HBM once per workgroup; the WM wavefronts that share a
//            row tile each read it from LDS as int4 (a quarter of the fp16 bytes) and dequantize the
//            words they need in registers.
//   params:  each wavefront's NT tiles' 16 scales and 16 zeros of the group (64 B per tile).
//   math:    v_mfma_f32_16x16x32_f16, A = dequantized weights fp16_rne((q - z) s) (16 rows x 32 k),
//            B = x (32 k x 16 tokens). Substep j (0, 1) of a stage: lane (q, r) feeds A row r and B
//            column r the k values of word (kb = 2 h + (q >> 1), s = 2 j + (q & 1)), i.e.
//            k = 64 s + 32 (q >> 1) + 16 j + 8 (q & 1) + 0..7, the same permutation for both operands.
//            D lane (q, r) = rows 4 q + i of token r, the layout finish_unit stores.
//   ring:    R = 3 or 4 slots. Stage i waits for its own loads (vmcnt), one workgroup barrier, issues
//            stage i + R - 1 into the slot stage i - 1 used, then computes from LDS, so R - 1 stages of
//            loads are in flight under every stage's math.
//   split-K: work units (tile, split) take contiguous stage ranges; the epilogue is the other GEMM's
//            finish_unit (deterministic last-arriver reduction, counters returned to zero).
#include "tw4_common.h"

namespace tw4 {

typedef __attribute__((address_space(3))) const void lds_void;

// Direct-to-LDS load of BYTES (4 or 16) per lane: lane l's BYTES at global `src` go to LDS byte address
// `lds_addr` (wavefront-uniform) + l BYTES. Issued as inline assembly so that the compiler, which cannot tell the
// ring's slots apart for these loads, does not add a wait for every load in flight before each LDS
// read; the ring waits with explicit vmcnt counts instead, and the loop holds no other vector memory
// operation. M0 (the LDS base operand) is saved and restored around the load, one wait state after
// writing it (the M0 -> LDS-DMA hazard).
template <int BYTES>
__device__ __forceinline__ void lds_dma(const void* src, uint32_t lds_addr) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr);
    uint32_t saved;
    if constexpr (BYTES == 16)
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(src), "s"(base) : "memory");
    else
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(src), "s"(base) : "memory");
}

template <int MT, int NT, int WM, int WN>
struct LdsGemmCfg {
    static constexpr int BM = 16 * MT * WM;
    static constexpr int BN = 16 * NT * WN;
    static constexpr int WAVES = WM * WN;
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int X_U4 = BM * 8;               // x tile: BM rows x 8 chunks
    static constexpr int W_U4 = BN / 16 * 32;         // weights: BN / 16 half-blocks of 512 B
    static constexpr int P_U4 = WAVES * NT * 4;       // params: per wavefront NT x (16 scales, 16 zeros)
    static constexpr int SLOT_U4 = X_U4 + W_U4 + P_U4;
    static constexpr int X_INSTR = BM / 8 / WAVES;    // x loads per wavefront per stage (8 rows each)
    static constexpr int W_INSTR = BN / 32 / WAVES;   // weight loads per wavefront per stage (2 half-blocks)
    static constexpr int P_INSTR = NT / 4;            // params loads per wavefront (4 tiles x 64 B each)
    static constexpr int LOADS = X_INSTR + W_INSTR + P_INSTR;
    static_assert(BM % (8 * WAVES) == 0, "x rows split evenly over the wavefronts");
    static_assert(BN % (32 * WAVES) == 0, "weight half-blocks split evenly over the wavefronts");
    static_assert(NT % 4 == 0, "params loads of 64 lanes x 4 bytes: 4 tiles x 64 B each");
    static_assert(3 * LOADS < 64, "s_waitcnt vmcnt immediate");
};

// s_waitcnt with only vmcnt limited (expcnt and lgkmcnt at their maxima); gfx9's 6-bit vmcnt is
// split over bits 3:0 and 15:14 of the immediate.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// A workgroup barrier that orders no memory by itself (the LDS data it guards was waited for with
// wait_vmcnt): s_barrier between two compiler-only fences, so no LDS access moves across it.
__device__ __forceinline__ void ring_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int MT, int NT, int WM, int WN>
struct LdsGemmArgs {
    const h1* x;
    const u4* w;
    const uint16_t* s16;
    const uint16_t* z16;
    int M, K, G, m0, tile0;  // tile0: the workgroup's first row tile
    int tile_last;           // the matrix's last row tile: tiles past it read it again (never stored)
};

// Issue the direct-to-LDS loads of stage `st` into `slot`. Every wavefront issues exactly LOADS
// instructions, so each can wait for a stage with one vmcnt.
template <int MT, int NT, int WM, int WN>
__device__ __forceinline__ void issue_stage(uint32_t slot, const LdsGemmArgs<MT, NT, WM, WN>& a, int st, int wave,
                                            int lane) {
    using C = LdsGemmCfg<MT, NT, WM, WN>;
    const int g = st >> 1, h = st & 1;
    // x: rows 8 j .. 8 j + 7 of the tile for instruction j = wave X_INSTR + i
#pragma unroll
    for (int i = 0; i < C::X_INSTR; ++i) {
        const int j = wave * C::X_INSTR + i;
        const int rho = 8 * j + (lane >> 3), p = lane & 7, c = p ^ (rho & 7);
        const int row = min(a.m0 + rho, a.M - 1);  // rows past M repeat the last one; never stored
        const h1* src = a.x + static_cast<int64_t>(row) * a.K + 128 * g + 64 * h + 8 * c;
        lds_dma<16>(src, slot + 16 * 64 * j);
    }
    // weights: half-blocks of row tiles 2 j, 2 j + 1 of the workgroup
#pragma unroll
    for (int i = 0; i < C::W_INSTR; ++i) {
        const int j = wave * C::W_INSTR + i;
        const int t = min(a.tile0 + 2 * j + (lane >> 5), a.tile_last);
        const u4* src = a.w + (static_cast<int64_t>(t) * a.G + g) * kBlockU4 + 32 * h + (lane & 31);
        lds_dma<16>(src, slot + 16 * (C::X_U4 + 64 * j));
    }
    // params of this wavefront's NT tiles, 4 bytes per lane with every lane active (no branch around the
    // load): lane 16 t' + 8 kind + p of load i holds rows 2 p, 2 p + 1 of tile 4 i + t''s scales (kind 0)
    // or zeros
    {
        const int wn = wave % WN;
        const int kind = (lane >> 3) & 1, p = lane & 7;
        const uint16_t* base = kind ? a.z16 : a.s16;
#pragma unroll
        for (int i = 0; i < C::P_INSTR; ++i) {
            const int tile = min(a.tile0 + wn * NT + 4 * i + (lane >> 4), a.tile_last);
            const uint16_t* src = base + static_cast<int64_t>(16) * tile * a.G + 16 * g + 2 * p;
            lds_dma<4>(src, slot + 16 * (C::X_U4 + C::W_U4 + wave * NT * 4 + 16 * i));
        }
    }
}

// One stage's math from `slot`: two substeps of NT x MT MFMAs.
template <int MT, int NT, int WM, int WN>
__device__ __forceinline__ void compute_stage(const u4* slot, f4 (&acc)[NT][MT], int wave, int wm, int wn, int lane,
                                              uint32_t magic) {
    using C = LdsGemmCfg<MT, NT, WM, WN>;
    const int r = lane & 15, q = lane >> 4;
    const u4* xs = slot;
    const u4* ws = slot + C::X_U4;
    const uint16_t* ps = reinterpret_cast<const uint16_t*>(slot + C::X_U4 + C::W_U4 + wave * NT * 4);
    // lane (q, r) needs words s = q & 1 and 2 + (q & 1) of (kb = 2 h + (q >> 1), r): one ds_read2_b32
    uint32_t wv[NT][2];
    GroupQ pq[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const uint32_t* wp = reinterpret_cast<const uint32_t*>(ws + (wn * NT + t) * 32 + (q >> 1) * 16 + r) + (q & 1);
        wv[t][0] = wp[0];
        wv[t][1] = wp[2];
        pq[t] = group_q(as_h1(ps[(2 * t) * 16 + r]), as_h1(ps[(2 * t + 1) * 16 + r]));
    }
    // both substeps' B fragments are read up front, so the second substep's LDS latency hides under the
    // first substep's MFMAs
    h8 xb[2][MT];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int c = 4 * (q >> 1) + 2 * j + (q & 1);
#pragma unroll
        for (int b = 0; b < MT; ++b) {
            const int rho = wm * 16 * MT + 16 * b + r;
            xb[j][b] = bitcast<h8>(xs[rho * 8 + (c ^ (rho & 7))]);
        }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const h8 a = dequant_word(wv[t][j], pq[t], magic);
#pragma unroll
            for (int b = 0; b < MT; ++b) acc[t][b] = mfma16x16x32(a, xb[j][b], acc[t][b]);
        }
    }
}

// One step of a ring of R slots with compile-time slot S: wait for stage i (leaving the later stages
// already issued in flight: up to R - 2 of them), barrier, issue stage i + R - 1 into the slot
// (S + R - 1) % R that stage i - 1 used, compute stage i from slot S.
template <int S, int R, int MT, int NT, int WM, int WN>
__device__ __forceinline__ void ring_step(const u4* ring, uint32_t ring_addr, const LdsGemmArgs<MT, NT, WM, WN>& a,
                                          int i, int nst, int st0, f4 (&acc)[NT][MT], int wave, int wm, int wn,
                                          int lane, uint32_t magic) {
    using C = LdsGemmCfg<MT, NT, WM, WN>;
    const int ahead = min(nst - 1 - i, R - 2);  // stages after i already in flight
    if constexpr (R == 4) {
        if (ahead >= 2)
            wait_vmcnt<2 * C::LOADS>();
        else if (ahead == 1)
            wait_vmcnt<C::LOADS>();
        else
            wait_vmcnt<0>();
    } else {
        if (ahead >= 1)
            wait_vmcnt<C::LOADS>();
        else
            wait_vmcnt<0>();
    }
    ring_barrier();
    if (i + R - 1 < nst)
        issue_stage<MT, NT, WM, WN>(ring_addr + 16 * ((S + R - 1) % R) * C::SLOT_U4, a, st0 + i + R - 1, wave, lane);
    compute_stage<MT, NT, WM, WN>(ring + S * C::SLOT_U4, acc, wave, wm, wn, lane, magic);
    __builtin_amdgcn_sched_barrier(0);  // one stage's registers at a time: no scheduling across steps
}

template <int MT, int NT, int WM, int WN, int R>
__global__ void __launch_bounds__(64 * WM * WN) gemm_lds_kernel(const h1* __restrict__ x, const u4* __restrict__ w,
                                                               const h1* __restrict__ scales,
                                                               const h1* __restrict__ zeros, h1* __restrict__ y,
                                                               float* __restrict__ ws, int* __restrict__ locks, int M,
                                                               int N, int K, int mb, int nb, int splits, int act) {
    using C = LdsGemmCfg<MT, NT, WM, WN>;
    static_assert(R == 3 || R == 4, "ring of 3 or 4 slots");
    __shared__ u4 ring[R * C::SLOT_U4];
    __shared__ int last_flag;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave % WN, wm = wave / WN;
    const int G = K >> 7, tiles_n = (N + 15) >> 4, stages = 2 * G;

    // work unit -> (tile, split); tiles in bands of 8 token blocks, each XCD a contiguous range
    const int unit = xcd_remap(blockIdx.x, gridDim.x);
    const int tile = unit / splits, split = unit - tile * splits;
    const int band = tile / (8 * nb), band_rows = min(mb - band * 8, 8), rin = tile - band * 8 * nb;
    const int mblk = band * 8 + rin % band_rows, nblk = rin / band_rows;
    const int st0 = static_cast<int>(static_cast<int64_t>(split) * stages / splits);
    const int nst = static_cast<int>(static_cast<int64_t>(split + 1) * stages / splits) - st0;

    LdsGemmArgs<MT, NT, WM, WN> a;
    a.x = x;
    a.w = w;
    a.s16 = reinterpret_cast<const uint16_t*>(scales);
    a.z16 = reinterpret_cast<const uint16_t*>(zeros);
    a.M = M;
    a.K = K;
    a.G = G;
    a.m0 = mblk * C::BM;
    a.tile0 = nblk * (C::BN / 16);
    a.tile_last = tiles_n - 1;

    const uint32_t magic = magic_reg();
    f4 acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int b = 0; b < MT; ++b) acc[t][b] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // the ring's LDS byte address, taken once from the array itself (the direct-to-LDS loads take it in M0)
    const uint32_t ring_addr = static_cast<uint32_t>(reinterpret_cast<size_t>((lds_void*)ring));
#pragma unroll
    for (int p = 0; p < R - 1; ++p)
        if (p < nst) issue_stage<MT, NT, WM, WN>(ring_addr + 16 * p * C::SLOT_U4, a, st0 + p, wave, lane);
    for (int i = 0; i < nst; i += R) {
        ring_step<0, R>(ring, ring_addr, a, i, nst, st0, acc, wave, wm, wn, lane, magic);
        if (i + 1 < nst) ring_step<1, R>(ring, ring_addr, a, i + 1, nst, st0, acc, wave, wm, wn, lane, magic);
        if (i + 2 < nst) ring_step<2, R>(ring, ring_addr, a, i + 2, nst, st0, acc, wave, wm, wn, lane, magic);
        if constexpr (R == 4)
            if (i + 3 < nst) ring_step<3, R>(ring, ring_addr, a, i + 3, nst, st0, acc, wave, wm, wn, lane, magic);
    }

    finish_unit<MT, NT, WM * WN>(acc, true, wave, lane, tid, splits, tile, unit, ws, locks, last_flag, y, M, N,
                                 a.m0 + wm * 16 * MT, a.tile0 + wn * NT, tiles_n, act);
}

// Compiled configurations (MT, NT, WM, WN, ring slots).
#define TW4_LDS_GEMM_CONFIGS(X) X(8, 4, 2, 4, 3) X(16, 4, 1, 4, 3) X(4, 4, 2, 4, 3) X(8, 4, 2, 2, 3)

template <int MT, int NT, int WM, int WN, int R>
int lds_gemm_launch(const h1* x, const u4* w, const h1* s, const h1* z, h1* y, float* ws, int* locks,
                    int64_t ws_floats, int64_t n_locks, int M, int N, int K, int splits, int cus, int act,
                    hipStream_t stream) {
    using C = LdsGemmCfg<MT, NT, WM, WN>;
    TW4_REQUIRE(N % 16 == 0, TW4_EINVAL, "gemm (stages 3): N %% 16 == 0 (N = %d)", N);
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(s) % 16 == 0 && reinterpret_cast<uintptr_t>(z) % 16 == 0, TW4_EINVAL,
                "gemm (stages 3): scales and zeros must be 16-byte aligned");
    const int G = K >> 7, stages = 2 * G;
    const int mb = (M + C::BM - 1) / C::BM, nb = (N + C::BN - 1) / C::BN;
    const int64_t tiles64 = static_cast<int64_t>(mb) * nb;
    TW4_REQUIRE(tiles64 < (1LL << 30), TW4_EINVAL, "gemm: too many tiles (%lld)", static_cast<long long>(tiles64));
    const int tiles = static_cast<int>(tiles64);
    int sp = splits;
    if (sp == 0) {  // enough units to fill the GPU once, within the workspace
        sp = 1;
        while (static_cast<int64_t>(tiles) * sp < cus && 2 * (sp + 1) <= stages &&
               static_cast<int64_t>(tiles) * (sp + 1) * C::BM * C::BN <= ws_floats && tiles <= n_locks)
            ++sp;
    }
    TW4_REQUIRE(sp >= 1 && sp <= stages, TW4_EINVAL, "gemm: splits %d for %d stages", sp, stages);
    if (sp > 1) {
        TW4_REQUIRE(ws && locks, TW4_EINVAL, "gemm: split-K needs a workspace and counters");
        TW4_REQUIRE(static_cast<int64_t>(tiles) * sp * C::BM * C::BN <= ws_floats && tiles <= n_locks, TW4_ESPACE,
                    "gemm: split-K workspace too small for %d tiles x %d splits", tiles, sp);
    }
    const int64_t blocks = static_cast<int64_t>(tiles) * sp;
    TW4_REQUIRE(blocks < (1LL << 31), TW4_EINVAL, "gemm: grid too large");
    gemm_lds_kernel<MT, NT, WM, WN, R><<<static_cast<unsigned>(blocks), C::THREADS, 0, stream>>>(
        x, w, s, z, y, ws, locks, M, N, K, mb, nb, sp, act);
    TW4_LAUNCH_CHECK("gemm (stages 3): launch");
    return TW4_OK;
}

}  // namespace tw4

using namespace tw4;

// Called by tw4_gemm for stages == 3 (warps_k is then WM, the wavefronts along M).
int tw4_gemm_lds_dispatch(const uint16_t* x, const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                          uint16_t* y, float* ws, int32_t* locks, int64_t ws_floats, int64_t n_locks, int M, int N,
                          int K, int mt, int nt, int warps_n, int warps_m, int splits, int cus, int act,
                          void* stream) {
    auto xp = reinterpret_cast<const h1*>(x);
    auto wp = reinterpret_cast<const u4*>(packed);
    auto sp = reinterpret_cast<const h1*>(scales);
    auto zp = reinterpret_cast<const h1*>(zeros);
    auto yp = reinterpret_cast<h1*>(y);
    auto st = static_cast<hipStream_t>(stream);
#define TW4_LDS_CASE(MT, NT, WM, WN, R)                                                                           \
    if (mt == MT && nt == NT && warps_m == WM && warps_n == WN)                                                      \
        return lds_gemm_launch<MT, NT, WM, WN, R>(xp, wp, sp, zp, yp, ws, locks, ws_floats, n_locks, M, N, K, splits, \
                                                  cus, act, st);
    TW4_LDS_GEMM_CONFIGS(TW4_LDS_CASE)
#undef TW4_LDS_CASE
    tw4host::set_error("gemm: unsupported stages-3 config mt / nt / warps_n / warps_m %d / %d / %d / %d", mt, nt,
                       warps_n, warps_m);
    return TW4_ECONFIG;
}

int tw4_gemm_lds_configs(int* out, int max_configs, int start) {
    int n = 0;
#define TW4_LDS_LIST(MT, NT, WM, WN, R)              \
    if (out && start + n < max_configs) {            \
        out[5 * (start + n)] = MT;                   \
        out[5 * (start + n) + 1] = NT;               \
        out[5 * (start + n) + 2] = WN;               \
        out[5 * (start + n) + 3] = WM;               \
        out[5 * (start + n) + 4] = 3;                \
    }                                                \
    ++n;
    TW4_LDS_GEMM_CONFIGS(TW4_LDS_LIST)
#undef TW4_LDS_LIST
    return n;
}
