// Fused-dequant GEMM for large M (prefill): y[M, N] = x[M, K] @ dequant(W)^T, with BOTH operand
// tiles staged through LDS by gfx950's direct-to-LDS loads (global_load_lds_dwordx4), a 3-deep ring.
//
// Workgroup tile BM x BN = (WM wavefronts x 16 MT tokens) x (WN wavefronts x 16 NT rows); wavefront
// (wm, wn) computes 16 MT tokens x 16 NT rows. A stage is half a quant group (BK = 64 k): stage s
// covers k = 64 s .. 64 s + 63 of group s / 2.
//   x:       the BM x 64 fp16 tile, 128 B per token row, 8 rows per load instruction. LDS slot
//            (row rho, position p) holds 16-byte chunk p ^ ((rho >> 1) & 7) of the row. Two rows fill
//            the 64 banks, even rows the lower 32, odd rows the upper 32; the swizzle gives the 8
//            even (and the 8 odd) rows of a B-fragment read (16 rows, one chunk) 8 different 16-byte
//            positions, so its 16 lanes touch every bank once (with rho & 7, each position came
//            twice: a 2-way bank conflict on every x read).
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
// The global address is a wavefront-uniform 64-bit base in SGPRs (`sbase`, the part that moves with the
// stage) plus this lane's 32-bit byte offset `voff` (fixed for the whole kernel), the instruction's
// scalar-base form: no per-lane 64-bit address arithmetic per load.
template <int BYTES>
__device__ __forceinline__ void lds_dma(const void* sbase, uint32_t voff, uint32_t lds_addr) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr);
    uint32_t saved;
    if constexpr (BYTES == 16)
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(voff), "s"(sbase), "s"(base) : "memory");
    else
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(voff), "s"(sbase), "s"(base) : "memory");
}

template <int MT, int NT, int WM, int WN>
struct LdsGemmCfg {
    static constexpr int BM = 16 * MT * WM;
    static constexpr int BN = 16 * NT * WN;
    static constexpr int WAVES = WM * WN;
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int X_U4 = BM * 8;               // x tile: BM rows x 8 chunks
    static constexpr int W_U4 = BN / 16 * 32;         // weights: BN / 16 half-blocks of 512 B
    static constexpr int P_U4 = WAVES * 32;           // params: per wavefront 8 tiles' 16 scales, then their zeros
    static constexpr int SLOT_U4 = X_U4 + W_U4 + P_U4;
    static constexpr int X_INSTR = BM / 8 / WAVES;    // x loads per wavefront per stage (8 rows each)
    static constexpr int W_INSTR = BN / 32 / WAVES;   // weight loads per wavefront per stage (2 half-blocks)
    static constexpr int P_INSTR = 2;                 // params loads per wavefront: scales, zeros (8 tiles x 32 B)
    static constexpr int LOADS = X_INSTR + W_INSTR + P_INSTR;
    // registers for two wavefronts per SIMD (at most 256 each) where the accumulators allow it and two
    // wavefronts per SIMD can be resident: 8 wavefronts per workgroup, or 4 with a ring small enough
    // (BM = 128) that two workgroups share a CU and run out of phase
    static constexpr int MIN_WAVES_PER_SIMD = MT * NT <= 32 && (WAVES >= 8 || BM <= 128) ? 2 : 1;
    static_assert(BM % (8 * WAVES) == 0, "x rows split evenly over the wavefronts");
    static_assert(BN % (32 * WAVES) == 0, "weight half-blocks split evenly over the wavefronts");
    static_assert(NT == 4 || NT == 8, "params: one dword load covers 8 tiles' 16 values (NT = 4 loads 4 twice)");
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
    using C = LdsGemmCfg<MT, NT, WM, WN>;
    const char* x;  // byte bases; a stage adds its k offset to them (scalar) and each lane its offset below
    const char* w;
    const char* s16;
    const char* z16;
    uint32_t xoff[C::X_INSTR];  // this lane's byte offsets, fixed for the kernel (see lds_gemm_offsets)
    uint32_t woff[C::W_INSTR];
    uint32_t poff;              // scales and zeros share it
};

// Per-lane byte offsets of the direct-to-LDS loads (everything but the stage's k position):
//   x load i (rows 8 j .. 8 j + 7 of the tile, j = wave X_INSTR + i): lane l takes row rho = 8 j + l / 8
//     (rows past M read the last row; never stored), 16-byte chunk (l & 7) ^ ((rho >> 1) & 7);
//   weight load i (row tiles 2 j, 2 j + 1 of the workgroup, j = wave W_INSTR + i): lane l the 16 bytes
//     l & 31 of the k half of tile 2 j + l / 32's block (tiles past the matrix read its last tile);
//   params: lane l the values of rows 2 (l & 7), + 1 of the wavefront's tile l / 8 (of NT; NT = 4 repeats).
template <int MT, int NT, int WM, int WN>
__device__ __forceinline__ void lds_gemm_offsets(LdsGemmArgs<MT, NT, WM, WN>& a, int M, int K, int G, int m0,
                                                 int tile0, int tile_last, int wave, int wn, int lane) {
    using C = LdsGemmCfg<MT, NT, WM, WN>;
#pragma unroll
    for (int i = 0; i < C::X_INSTR; ++i) {
        const int j = wave * C::X_INSTR + i;
        const int rho = 8 * j + (lane >> 3), c = (lane & 7) ^ ((rho >> 1) & 7);
        const int row = min(m0 + rho, M - 1);
        a.xoff[i] = static_cast<uint32_t>(row) * static_cast<uint32_t>(K) * 2u + 16u * c;
    }
#pragma unroll
    for (int i = 0; i < C::W_INSTR; ++i) {
        const int j = wave * C::W_INSTR + i;
        const int t = min(tile0 + 2 * j + (lane >> 5), tile_last);
        a.woff[i] = static_cast<uint32_t>(t) * static_cast<uint32_t>(G) * 1024u + 16u * (lane & 31);
    }
    const int t = min(tile0 + wn * NT + (lane >> 3) % NT, tile_last);
    a.poff = (static_cast<uint32_t>(t) * 16u * static_cast<uint32_t>(G) + 2u * (lane & 7)) * 2u;
}

// Issue the direct-to-LDS loads of stage `st` into `slot`. Every wavefront issues exactly LOADS
// instructions, so each can wait for a stage with one vmcnt. Stage st = (group g, k half h) moves the
// bases only: x by (128 g + 64 h) halves, the weights by block g and half h (g * 1024 + h * 512 bytes),
// the scales and zeros by group g (16 g halves of every tile).
template <int MT, int NT, int WM, int WN>
__device__ __forceinline__ void issue_stage(uint32_t slot, const LdsGemmArgs<MT, NT, WM, WN>& a, int st, int wave) {
    using C = LdsGemmCfg<MT, NT, WM, WN>;
    const int g = st >> 1, h = st & 1;
    const char* xb = a.x + (256 * g + 128 * h);
#pragma unroll
    for (int i = 0; i < C::X_INSTR; ++i) lds_dma<16>(xb, a.xoff[i], slot + 16 * 64 * (wave * C::X_INSTR + i));
    const char* wb = a.w + (1024 * g + 512 * h);
#pragma unroll
    for (int i = 0; i < C::W_INSTR; ++i)
        lds_dma<16>(wb, a.woff[i], slot + 16 * (C::X_U4 + 64 * (wave * C::W_INSTR + i)));
    const uint32_t pslot = slot + 16 * (C::X_U4 + C::W_U4 + wave * 32);
    lds_dma<4>(a.s16 + 32 * g, a.poff, pslot);         // scales [8 tiles][16 rows]
    lds_dma<4>(a.z16 + 32 * g, a.poff, pslot + 256);   // zeros, the same order
}

// One stage's math from `slot`: two substeps of NT x MT MFMAs.
template <int MT, int NT, int WM, int WN>
__device__ __forceinline__ void compute_stage(const u4* slot, f4 (&acc)[NT][MT], int wave, int wm, int wn, int lane,
                                              uint32_t magic) {
    using C = LdsGemmCfg<MT, NT, WM, WN>;
    // One wavefront along M: let the scheduler interleave the MFMAs with the LDS reads and the dequant
    // (LLVM's IGroupLP strategy 0). Measured on the 128 x 256 tile at M = 2048 / 4096: gate_up 364.6 ->
    // 360.1 / 706.3 -> 696.7 us, down 204.1 -> 200.8 / 336.3 -> 334.4 us; on the WM = 2 tiles it was
    // slower, so they keep the default schedule. The MFMA order per accumulator is unchanged.
    if constexpr (WM == 1) __builtin_amdgcn_iglp_opt(0);
    const int r = lane & 15, q = lane >> 4;
    const u4* xs = slot;
    const u4* ws = slot + C::X_U4;
    const uint16_t* ps = reinterpret_cast<const uint16_t*>(slot + C::X_U4 + C::W_U4 + wave * 32);  // [2][8][16]
    // lane (q, r) needs words s = q & 1 and 2 + (q & 1) of (kb = 2 h + (q >> 1), r): one ds_read2_b32
    uint32_t wv[NT][2];
    GroupQ pq[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const uint32_t* wp = reinterpret_cast<const uint32_t*>(ws + (wn * NT + t) * 32 + (q >> 1) * 16 + r) + (q & 1);
        wv[t][0] = wp[0];
        wv[t][1] = wp[2];
        pq[t] = group_q(as_h1(ps[t * 16 + r]), as_h1(ps[128 + t * 16 + r]));
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
            xb[j][b] = bitcast<h8>(xs[rho * 8 + (c ^ ((rho >> 1) & 7))]);
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
        issue_stage<MT, NT, WM, WN>(ring_addr + 16 * ((S + R - 1) % R) * C::SLOT_U4, a, st0 + i + R - 1, wave);
    compute_stage<MT, NT, WM, WN>(ring + S * C::SLOT_U4, acc, wave, wm, wn, lane, magic);
    __builtin_amdgcn_sched_barrier(0);  // one stage's registers at a time: no scheduling across steps
}

template <int MT, int NT, int WM, int WN, int R>
__global__ void __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(LdsGemmCfg<MT, NT, WM, WN>::MIN_WAVES_PER_SIMD))) gemm_lds_kernel(const h1* __restrict__ x, const u4* __restrict__ w,
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

    const int m0 = mblk * C::BM, tile0 = nblk * (C::BN / 16);
    LdsGemmArgs<MT, NT, WM, WN> a;
    a.x = reinterpret_cast<const char*>(x);
    a.w = reinterpret_cast<const char*>(w);
    a.s16 = reinterpret_cast<const char*>(scales);
    a.z16 = reinterpret_cast<const char*>(zeros);
    lds_gemm_offsets<MT, NT, WM, WN>(a, M, K, G, m0, tile0, tiles_n - 1, wave, wn, lane);

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
        if (p < nst) issue_stage<MT, NT, WM, WN>(ring_addr + 16 * p * C::SLOT_U4, a, st0 + p, wave);
    for (int i = 0; i < nst; i += R) {
        ring_step<0, R>(ring, ring_addr, a, i, nst, st0, acc, wave, wm, wn, lane, magic);
        if (i + 1 < nst) ring_step<1, R>(ring, ring_addr, a, i + 1, nst, st0, acc, wave, wm, wn, lane, magic);
        if (i + 2 < nst) ring_step<2, R>(ring, ring_addr, a, i + 2, nst, st0, acc, wave, wm, wn, lane, magic);
        if constexpr (R == 4)
            if (i + 3 < nst) ring_step<3, R>(ring, ring_addr, a, i + 3, nst, st0, acc, wave, wm, wn, lane, magic);
    }

    finish_unit<MT, NT, WM * WN>(acc, true, wave, lane, tid, splits, tile, unit, ws, locks, last_flag, y, M, N,
                                 m0 + wm * 16 * MT, tile0 + wn * NT, tiles_n, act);
}

// Compiled configurations (MT, NT, WM, WN, ring slots).
#define TW4_LDS_GEMM_CONFIGS(X) X(8, 4, 2, 4, 3) X(16, 4, 1, 4, 3) X(4, 4, 2, 4, 3) X(8, 4, 2, 2, 3) X(8, 8, 1, 4, 4) X(8, 4, 1, 4, 3)

template <int MT, int NT, int WM, int WN, int R>
int lds_gemm_launch(const h1* x, const u4* w, const h1* s, const h1* z, h1* y, float* ws, int* locks,
                    int64_t ws_floats, int64_t n_locks, int M, int N, int K, int splits, int cus, int act,
                    hipStream_t stream) {
    using C = LdsGemmCfg<MT, NT, WM, WN>;
    TW4_REQUIRE(N % 16 == 0, TW4_EINVAL, "gemm (stages 3): N %% 16 == 0 (N = %d)", N);
    // the loads' per-lane byte offsets are 32-bit: x (M K 2 bytes) and the weights (N K / 2 bytes)
    TW4_REQUIRE(static_cast<int64_t>(M) * K < (1LL << 31) && static_cast<int64_t>(N) * K < (1LL << 33), TW4_EINVAL,
                "gemm (stages 3): M K < 2^31 and N K < 2^33 (M %d, N %d, K %d)", M, N, K);
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(s) % 16 == 0 && reinterpret_cast<uintptr_t>(z) % 16 == 0, TW4_EINVAL,
                "gemm (stages 3): scales and zeros must be 16-byte aligned");
    const int G = K >> 7, stages = 2 * G;
    const int mb = (M + C::BM - 1) / C::BM, nb = (N + C::BN - 1) / C::BN;
    const int64_t tiles64 = static_cast<int64_t>(mb) * nb;
    TW4_REQUIRE(tiles64 < (1LL << 30), TW4_EINVAL, "gemm: too many tiles (%lld)", static_cast<long long>(tiles64));
    const int tiles = static_cast<int>(tiles64);
    int sp = splits;
    if (sp == 0) {  // enough units to fill the GPU once, within the default workspace (never the caller's)
        sp = 1;
        while (static_cast<int64_t>(tiles) * sp < cus && 2 * (sp + 1) <= stages &&
               static_cast<int64_t>(tiles) * (sp + 1) * C::BM * C::BN <= TW4_AUTO_SPLIT_FLOATS &&
               tiles <= TW4_AUTO_SPLIT_COUNTERS)
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
