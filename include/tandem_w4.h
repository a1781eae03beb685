/*
 * tandem_w4.h - C ABI of the MI355X (gfx950) AWQ W4A16 linear library, libtandem_w4.so.
 *
 * y[M, N] = x[M, K] @ dequant(W)[N, K]^T with AutoAWQ 4-bit weights (group 128), fp16 activations,
 * fp32 accumulation. Every pointer is a device pointer; every launch goes on the caller's HIP
 * stream (`stream`, a hipStream_t passed as void*; NULL = the null stream). Launches allocate
 * nothing, never synchronize and read no device memory from the host, so they may be captured
 * in a HIP graph once tw4_init() has run for the device.
 *
 * Status: every entry point returns TW4_OK (0) or a nonzero TW4_E* code; tw4_last_error()
 * returns the calling thread's last message (the reference raises RuntimeError from
 * TORCH_CHECK with the same conditions, python/tandem/csrc/w4_gemv.cu:568-579).
 *
 * Weight layout ("tile layout", produced by tw4_repack_awq, consumed by every kernel):
 *   packed  int32 [Npad/16][K/128][4 kb][16 r][4 s]   Npad = N rounded up to 16
 *           word (kb, r, s) of row tile T and quant group g holds the 8 consecutive weights
 *           k = 128 g + 32 kb + 8 s + o (o = 2 q + e, q = 0..3, e = 0..1) of row n = 16 T + r,
 *           weight o in nibble q + 4 e. One row tile x one group is 1 KB: one 16-byte load per
 *           lane of a 64-lane wavefront (lane 16 kb + r takes words s = 0..3). Rows n >= N
 *           are zero.
 *   scales  fp16 [N, K/128]    s[n, g], stored tile-major: at 16 T G + g rows_T + (n - 16 T),
 *                              T = n / 16, rows_T = min(16, N - 16 T)
 *   zeros   fp16 [N, K/128]    z[n, g], the integer zero point (exact), same order
 *   w[n, k] = fp16_rne((q[n, k] - z[n, k/128]) * s[n, k/128]).
 * N is the number of output features (the rows of scales); packed must hold Npad * K / 8 words.
 * The host view of `packed` is [Npad, K/8] int32: the same buffer size as the reference's
 * post-finalize `packed` (python/tandem/layers/awq.py:49-68, 243-246), a different word order.
 */
#ifndef TANDEM_W4_H
#define TANDEM_W4_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TW4_OK = 0,
    TW4_EINVAL = 1,    /* bad shape, alignment, size or argument */
    TW4_ECONFIG = 2,   /* kernel configuration not compiled in */
    TW4_EHIP = 3,      /* HIP runtime error (launch, attribute, device query) */
    TW4_ESPACE = 4     /* split-K workspace or counters too small */
};

/* Library version string, e.g. "tandem_w4 0.1.0 gfx950". No reference counterpart (the
 * reference's extension is a JIT torch module, python/tandem/layers/w4_cuda.py:44-62). */
const char* tw4_version(void);

/* Offload architecture the device code was compiled for ("gfx950"). */
const char* tw4_arch(void);

/* The calling thread's last error message ("" if none). Replaces the TORCH_CHECK messages of
 * python/tandem/csrc/w4_gemv.cu:568-579, 599, 608, 624-625, 647, 654-661, 681. */
const char* tw4_last_error(void);

/* One-time set-up for `device`, before any graph capture: checks the device is gfx950, sets the
 * dynamic-LDS limit of every GEMM configuration and records its occupancy for the last-wave
 * split-K model. Replaces the first-launch static of gemm_launch (python/tandem/csrc/
 * w4_gemv.cu:539-544) and the build-before-capture step of W4Linear.finalize
 * (python/tandem/layers/awq.py:247-251). Safe to call repeatedly. */
int tw4_init(int device);

/* AutoAWQ "gemm" tensors -> tile layout, on the device.
 *   qweight int32 [K, N/8], qzeros int32 [K/128, N/8] (AWQ nibble order 0,2,4,6,1,3,5,7),
 *   scales fp16 [K/128, N]  ->  packed [Npad/16 * K/128 * 256] int32, scales_out / zeros_out
 *   fp16 [N, K/128]. packed must be zero-filled by the caller (its rows >= N stay zero).
 * interleave = 1 reorders rows as interleave_gate_up (gate rows 8T..8T+7 then up rows
 * N/2+8T..N/2+8T+7 in row tile T; N % 16 == 0).
 * Replaces repack_awq + interleave_gate_up (python/tandem/layers/awq.py:42-75, 235-241). */
int tw4_repack_awq(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                   int32_t* packed, uint16_t* scales_out, uint16_t* zeros_out,
                   int K, int N, int interleave, void* stream);

/* Tile layout -> dense fp16 out [N, K] (nn.Linear layout), bit-exact fp16_rne((q - z) * s).
 * deinterleave = 1 undoes interleave_gate_up on the rows. Replaces the Triton
 * _w4_dequant_kernel / w4_dequant (python/tandem/layers/awq.py:89-133). */
int tw4_dequant(const int32_t* packed, const uint16_t* scales, const uint16_t* zeros,
                uint16_t* out, int N, int K, int deinterleave, void* stream);

/* Decode GEMV on the vector ALUs, 1 <= M <= 4: y fp16 [M, N]. x fp16 [M, K] contiguous and
 * 16-byte aligned. Config: warps_k wavefronts split K into contiguous group ranges inside a
 * workgroup, unroll quant groups per chunk (one chunk in flight ahead of the math), ntile row
 * tiles (16 rows) per workgroup.
 * Replaces w4_gemv (python/tandem/csrc/w4_gemv.cu:96-153, 581-617). */
int tw4_gemv(const uint16_t* x, const int32_t* packed, const uint16_t* scales,
             const uint16_t* zeros, uint16_t* y, int M, int N, int K,
             int warps_k, int unroll, int ntile, void* stream);

/* tw4_gemv with tw4_mma's act argument: act = 1 writes y = silu(gate) * up, [M, N/2], rows in
 * interleave_gate_up order (N % 16 == 0); act = 0 is tw4_gemv. The reference's GEMV has no
 * SwiGLU epilogue (python/tandem/csrc/w4_gemv.cu:96-153), so its SwiGLU gate_up takes w4_mma at
 * every decode M (python/tandem/layers/awq.py:253-270); this entry lets a W4Linear table send
 * M <= 4 SwiGLU gate_up to the GEMV. */
int tw4_gemv_act(const uint16_t* x, const int32_t* packed, const uint16_t* scales,
                 const uint16_t* zeros, uint16_t* y, int M, int N, int K,
                 int warps_k, int unroll, int ntile, int act, void* stream);

/* The GEMV's arithmetic on the matrix cores, 1 <= M <= 16 (one 16-column B tile): raw magic halves
 * (1024 + q) times x' on v_mfma_f32_16x16x32_f16, the bias and the zero point in the accumulator's
 * start value, the scale per group; exact (q - z) weights like tw4_gemv (so the GEMV's tolerance).
 * Same configs and act as tw4_gemv_act; x' of M rows and its per-group sums must fit in LDS
 * (TW4_EINVAL otherwise: K = 4096 takes M <= 16, K = 12288 M <= 4); scales and zeros 8-byte aligned.
 * No reference counterpart: an alternative kernel for the (N, K, M) decode-table entries of w4_gemv
 * and w4_mma (python/tandem/layers/awq.py:136-160). */
int tw4_gemv_mfma(const uint16_t* x, const int32_t* packed, const uint16_t* scales,
                  const uint16_t* zeros, uint16_t* y, int M, int N, int K,
                  int warps_k, int unroll, int ntile, int act, void* stream);

/* The decoder layer's add + RMSNorm fused into a decode kernel's x staging: the kernel
 * (kind 0: tw4_gemv_act, 1 <= M <= 4; kind 1: tw4_mma with x in LDS, 1 <= M <= 16 and
 * M (K + 8) 2 <= 80 KB) runs on a = fp16((x + residual) * rsqrt(mean((x + residual)^2) + eps)
 * * norm_weight), the fp32 sum s = x + residual, and writes residual_out = fp16(s) (not in
 * place). residual = NULL: plain RMSNorm of x, residual_out unused. y and residual_out are
 * bit-identical to tw4_add_rms_norm (or tw4_rms_norm) followed by the same kernel and config.
 * norm_weight fp16 [K]; x, residual, residual_out fp16 [M, K], 16-byte aligned.
 * Replaces the unfused pair ops.fused_add_rms_norm + projection of the reference's decoder layer
 * (python/tandem/models/llama_family.py:58-65; its fused-prologue GEMV,
 * python/tandem/layers/triton_gemv.py:92-178, 330-415, is the same idea for fp16 weights). */
int tw4_decode_norm(const uint16_t* x, const uint16_t* residual, uint16_t* residual_out,
                    const uint16_t* norm_weight, float eps, const int32_t* packed,
                    const uint16_t* scales, const uint16_t* zeros, uint16_t* y, int M, int N,
                    int K, int kind, int warps_k, int unroll, int ntile, int act, void* stream);

/* Decode on the matrix cores (v_mfma_f32_16x16x32_f16, weights as the A operand, the batch on
 * the 16-column side, ceil(M / 16) column tiles), 1 <= M <= 64; unroll * ceil(M / 16) <= 4.
 * act = 1: y = silu(gate) * up, [M, N/2], rows in interleave_gate_up order (N % 16 == 0);
 * act = 0: y [M, N]. Configurations: those of tw4_decode_configs, and the row-tile-wide ones of
 * tw4_mma_wide_configs (up to six row tiles per workgroup, x read from global memory at every
 * chunk instead of staged in LDS; tw4_mma only: tw4_mma_splitk with splits > 1, tw4_mma_persist and
 * tw4_decode_norm refuse them with TW4_ECONFIG).
 * Replaces w4_mma (python/tandem/csrc/w4_gemv.cu:166-295, 619-648). */
int tw4_mma(const uint16_t* x, const int32_t* packed, const uint16_t* scales,
            const uint16_t* zeros, uint16_t* y, int M, int N, int K,
            int warps_k, int unroll, int ntile, int act, void* stream);

/* tw4_mma with K split over `splits` workgroups per row-tile group, M <= 16, 2 <= splits <=
 * min(16, K / 128): a workgroup covers 1 / splits of the quant groups, with x in LDS over that
 * range only, and the last arriver of a tile group adds the splits partial sums in split order
 * (deterministic) and writes y. ws / locks: tw4_gemm's caller-owned fp32 workspace (at least
 * ceil(ceil(N / 16) / ntile) x splits x ntile x 256 floats) and int32 counters (one per tile group),
 * zero before the first call and returned to zero by every call; calls that share them must not
 * overlap. No counterpart in the reference: it extends w4_mma (csrc/w4_gemv.cu:619-648) for M = 4 .. 16
 * with a large K, where each workgroup would otherwise read all of x from L2. */
int tw4_mma_splitk(const uint16_t* x, const int32_t* packed, const uint16_t* scales,
                   const uint16_t* zeros, uint16_t* y, float* ws, int32_t* locks,
                   int64_t ws_floats, int64_t n_locks, int M, int N, int K,
                   int warps_k, int unroll, int ntile, int splits, int act, void* stream);

/* tw4_mma's persistent form, M <= 16, per_cu in 1 .. 8: at most per_cu workgroups per CU, each
 * staging x (in LDS) once and streaming row-tile groups b, b + grid, ... with the next group's first
 * chunk prefetched during the current group's last one; the same bits as tw4_mma with the same
 * (warps_k, unroll, ntile). Needs M (K + 8) 2 bytes of x in LDS: up to 80 KB, or 136 KB where the grid
 * has at most one workgroup per CU. No counterpart in the reference: it extends w4_mma
 * (csrc/w4_gemv.cu:619-648) for the decode batches where staging x per workgroup costs more than
 * the tile itself. */
int tw4_mma_persist(const uint16_t* x, const int32_t* packed, const uint16_t* scales,
                    const uint16_t* zeros, uint16_t* y, int M, int N, int K,
                    int warps_k, int unroll, int ntile, int per_cu, int act, void* stream);

/* Fused-dequant GEMM for M > 16 (any M >= 1 works): x tiles double-buffered through LDS,
 * weights dequantized in registers into MFMA fragments, fp32 accumulation, optional split-K
 * across workgroups with a deterministic last-arriver reduction.
 *   mt      16-token column tiles per workgroup (BM = 16 mt)
 *   nt      16-row weight tiles per wavefront
 *   warps_n wavefronts along N (BN = 16 nt warps_n)
 *   warps_k wavefronts splitting each K step (1 or 2)
 *   stages  2: x tiles through a double-buffered LDS ring, one barrier per K step;
 *           0: small M: the unit's x rows over its whole K range resident in LDS (one barrier),
 *           each wavefront streams its weight blocks with two groups in flight (every tile is
 *           split: splits = 0 picks the fewest splits whose x slice fits, then enough units to
 *           fill the GPU; a slice that cannot fit is refused with TW4_ECONFIG)
 *           1: batched decode, M <= 16 mt (mt 1, 2 or 4): no x staging; each wavefront streams its
 *           nt row tiles' weights and reads its x fragments from L2 (coalesced, then a cross-lane
 *           transpose), both one quant group ahead of the math; warps_n is then the groups per
 *           prefetch chunk (1 or 2) and warps_k the wavefronts splitting each unit's groups (4 or 8);
 *           splits = 0 picks enough K splits to give every CU a unit
 *           3: large M: x AND the int4 weight tiles staged through LDS by direct-to-LDS loads
 *           (global_load_lds_dwordx4) in a 3-deep ring of half-group (64 k) stages; warps_k is then
 *           the number of wavefronts along M (BM = 16 mt warps_k, BN = 16 nt warps_n); N % 16 == 0,
 *           scales and zeros 16-byte aligned; splits = 0 picks enough K splits to fill the GPU
 *   splits  0: split only the last, partial wave of tiles along K; 1: no split; s > 1: every
 *           tile split s ways. The partial-wave rule counts tile waves, not bytes: where the whole
 *           grid fits in one wave it splits every tile, and on a bandwidth-bound shape the fp32
 *           partials can cost more than the split saves (Qwen3-8B gate_up at M = 32 with
 *           (2, 1, 4, 2, 2, 0) moved 1.64x its algorithmic bytes). The gfx950 tables name the split.
 * ws (fp32, ws_floats) and locks (int32, n_locks, zero before the first call) are the split-K
 * workspace; the kernel returns every counter to zero, so graph replays stay correct. Calls
 * that share a workspace must not overlap. splits = 0 chooses its split from the tiles and the
 * CU count within a fixed budget of TW4_AUTO_SPLIT_FLOATS partials and TW4_AUTO_SPLIT_COUNTERS
 * counters (the default workspace's size), never from ws_floats / n_locks: a given config and
 * shape always runs the same split and gives the same bits, and a workspace smaller than that
 * split needs is refused with TW4_ESPACE.
 * Replaces w4_gemm / gemm_launch (python/tandem/csrc/w4_gemv.cu:312-566, 650-683) and the
 * workspace contract of python/tandem/layers/w4_cuda.py:24-41. */
#define TW4_AUTO_SPLIT_FLOATS (1LL << 23)
#define TW4_AUTO_SPLIT_COUNTERS (1 << 15)
int tw4_gemm(const uint16_t* x, const int32_t* packed, const uint16_t* scales,
             const uint16_t* zeros, uint16_t* y, float* ws, int32_t* locks,
             int64_t ws_floats, int64_t n_locks, int M, int N, int K,
             int mt, int nt, int warps_n, int warps_k, int stages, int splits, int act,
             void* stream);

/* tw4_gemm without a caller workspace, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. Same kernels, arguments (minus ws / locks / sizes), results and errors as tw4_gemm
 * called with a workspace of TW4_NOALLOC_FLOATS fp32 values and TW4_NOALLOC_COUNTERS counters, which
 * is the default workspace's size and the budget splits = 0 chooses within: every call tw4_gemm
 * accepts with that workspace runs the same split here and gives the same bits. The split-K
 * partial sums and tile counters live in a static device array of the library, one per GPU, held
 * until the process ends. A call whose split-K needs more is refused with TW4_ESPACE. The function
 * allocates nothing and never synchronizes. tw4_init(device) sets the array up
 * (its address and cleared counters); without it the first call on a device does, and then must not
 * be under graph capture (TW4_EINVAL). All calls on one GPU share the array: calls that overlap on a
 * GPU (other streams or threads) race and must be serialized by the caller. */
#define TW4_NOALLOC_FLOATS TW4_AUTO_SPLIT_FLOATS
#define TW4_NOALLOC_COUNTERS TW4_AUTO_SPLIT_COUNTERS
int tw4_gemm_noalloc(const uint16_t* x, const int32_t* packed, const uint16_t* scales,
                     const uint16_t* zeros, uint16_t* y, int M, int N, int K,
                     int mt, int nt, int warps_n, int warps_k, int stages, int splits, int act,
                     void* stream);

/* Dense fp16 GEMV for small batches: y [M, N] = x [M, K] @ w [N, K]^T (w row-major, nn.Linear
 * layout), 1 <= M <= 8, K in {512, 1024, 2048, 4096}, fp32 accumulation; x and w 16-byte aligned.
 * Config: rows_inflight rows per wavefront in flight (plus the next block prefetched), rows_per_wave
 * contiguous rows per wavefront; rows_inflight 16 or 32 selects the matrix-core form (16-row tiles on
 * v_mfma_f32_16x16x32_f16 with one or two 128-k chunks per step in flight, rows_per_wave a multiple
 * of 16), for M = 5 .. 8. For the fp16 lm_head of
 * a W4A16 model.
 * Replaces gemv / _gemv_kernel (python/tandem/layers/triton_gemv.py:26-61, 180-218). */
int tw4_gemv_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, int M, int N, int K,
                 int rows_inflight, int rows_per_wave, void* stream);

/* Compiled (rows_inflight, rows_per_wave) configurations of tw4_gemv_f16; returns how many. */
int tw4_gemv_f16_configs(int* out, int max_configs);

/* RMSNorm of the decoder layer around the projections, fp16 rows [M, K], fp32 math, K % 512 == 0,
 * K <= 8192, rows 16-byte aligned. y = fp16(x * rsqrt(mean(x^2) + eps) * weight).
 * Replaces ops.rms_norm of the GPU path (python/tandem/layers/ops.py:107-109, FlashInfer's
 * rmsnorm: fp32 math, one rounding). */
int tw4_rms_norm(const uint16_t* x, const uint16_t* weight, uint16_t* y, int M, int K, float eps,
                 void* stream);

/* Residual add + RMSNorm, in place: s = x + residual in fp32; residual <- fp16(s);
 * x <- fp16(s * rsqrt(mean(s^2) + eps) * weight). Same limits as tw4_rms_norm.
 * Replaces ops.fused_add_rms_norm (python/tandem/layers/ops.py:111-120; the Triton kernel of
 * python/tandem/layers/triton_ops.py:101-124 and FlashInfer's fused_add_rmsnorm). The sum of
 * squares is taken in the same fixed order as the decode kernels' fused norm prologue. */
int tw4_add_rms_norm(uint16_t* x, uint16_t* residual, const uint16_t* weight, int M, int K,
                     float eps, void* stream);

/* Streaming-read probe: reads `bytes` (a multiple of 16) from the device buffer `src` with 16-byte
 * non-temporal loads (1 KB per wavefront instruction, `inflight` = 1, 2, 4 or 8 issued per lane
 * before any is used) over `workgroups`
 * workgroups of 256 threads, grid-stride (chunked = 0) or one contiguous span per workgroup (chunked =
 * 1, the decode kernels' order), and does nothing else: it writes sink[0] only if the XOR of every
 * loaded word equals `key`. The plain-read ceiling against which the decode kernels' bandwidth is
 * judged. No reference counterpart (the reference calibrated with a device copy,
 * docs/P0基线报告.md:33). */
int tw4_read_probe(const void* src, int64_t bytes, int workgroups, int chunked, int inflight, uint32_t key,
                   uint32_t* sink, void* stream);

/* Compiled configurations, for sweeps and tests (the reference lists them in its host code,
 * python/tandem/csrc/w4_gemv.cu:596-597, 641-645, 676-679). Each writes up to max_configs
 * tuples into out and returns how many exist: tw4_decode_configs (warps_k, unroll, ntile) for
 * tw4_gemv and tw4_mma; tw4_gemm_configs (mt, nt, warps_n, warps_k, stages) for tw4_gemm (for
 * stages 3 the fourth value is the wavefronts along M). */
int tw4_decode_configs(int* out, int max_configs);
int tw4_gemm_configs(int* out, int max_configs);

/* The row-tile-wide (warps_k, unroll, ntile) configurations tw4_mma takes besides
 * tw4_decode_configs' (see tw4_mma). The reference's w4_mma compiles ntile 1 and 2 only
 * (python/tandem/csrc/w4_gemv.cu:641-645): (4, 1, 3), (4, 1, 6) and (4, 2, 3) have no counterpart
 * there; (4, 1, 2) is one of its configurations, which this library runs in the row-tile-wide
 * form. */
int tw4_mma_wide_configs(int* out, int max_configs);

/* Grid the last tw4_gemm call on this thread launched: workgroups, data-parallel tiles and
 * split factor (for benchmarks and tests; the reference keeps these internal,
 * python/tandem/csrc/w4_gemv.cu:545-563). */
int tw4_gemm_last_grid(int* blocks, int* dp_tiles, int* splits);

#ifdef __cplusplus
}
#endif

#endif /* TANDEM_W4_H */
