// Load-time repack (AutoAWQ "gemm" tensors -> tile layout) and the dense dequantization
// (tile layout -> fp16 [N, K]).
//
// AutoAWQ packs output columns c = 0..7 of an int32 in nibble order [0, 2, 4, 6, 1, 3, 5, 7],
// so column c sits in nibble kAwqReverse[c] (python/tandem/layers/awq.py:38-46).
#include "tw4_common.h"

namespace tw4 {

__constant__ int kAwqReverse[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// One thread per (8 k, 8 columns): reads the 8 AWQ words qweight[8 kq + o][c8] (o = 0..7) and
// writes the 8 tile-layout words of columns 8 c8 .. 8 c8 + 7 for those 8 k (an 8 x 8 nibble
// transpose in registers).
__global__ void repack_weights_kernel(const int32_t* __restrict__ qweight, uint32_t* __restrict__ packed,
                                      int K, int N, int interleave) {
    const int n8 = N >> 3, kq_count = K >> 3;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<int64_t>(n8) * kq_count) return;
    const int c8 = static_cast<int>(idx % n8), kq = static_cast<int>(idx / n8);
    uint32_t src[8];
#pragma unroll
    for (int o = 0; o < 8; ++o) src[o] = static_cast<uint32_t>(qweight[static_cast<int64_t>(8 * kq + o) * n8 + c8]);
    const int G = K >> 7, g = kq >> 4, kb = (kq >> 2) & 3, s = kq & 3;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int shift = 4 * kAwqReverse[c];
        uint32_t word = 0;
#pragma unroll
        for (int o = 0; o < 8; ++o) {
            const uint32_t q = (src[o] >> shift) & 0xFu;
            word |= q << (4 * ((o >> 1) + 4 * (o & 1)));  // weight o = 2 q' + e in nibble q' + 4 e
        }
        const int n = 8 * c8 + c;
        const int dst = interleave ? interleaved_dest_row(n, N) : n;
        const int64_t block = static_cast<int64_t>(dst >> 4) * G + g;
        packed[block * kBlockWords + (kb * 16 + (dst & 15)) * 4 + s] = word;
    }
}

// One thread per (group, column): scales [G, N] -> tile-major [N, G] (param_offset); qzeros nibble ->
// exact fp16 zero.
__global__ void repack_group_params_kernel(const int32_t* __restrict__ qzeros, const h1* __restrict__ scales,
                                          h1* __restrict__ s_out, h1* __restrict__ z_out, int K, int N,
                                          int interleave) {
    const int G = K >> 7;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<int64_t>(G) * N) return;
    const int n = static_cast<int>(idx % N), g = static_cast<int>(idx / N);
    const uint32_t zw = static_cast<uint32_t>(qzeros[static_cast<int64_t>(g) * (N >> 3) + (n >> 3)]);
    const int z = static_cast<int>((zw >> (4 * kAwqReverse[n & 7])) & 0xFu);
    const int dst = interleave ? interleaved_dest_row(n, N) : n;
    const int64_t o = param_offset(dst, g, N, G);
    s_out[o] = scales[idx];
    z_out[o] = static_cast<h1>(static_cast<float>(z));
}

// One thread per 16-byte vector of the tile layout (lane l = 16 kb + r of its block): writes the
// 32 dequantized weights k = 128 g + 32 kb .. + 31 of row 16 T + r as four 16-byte stores.
__global__ void dequant_kernel(const u4* __restrict__ packed, const h1* __restrict__ scales,
                               const h1* __restrict__ zeros, h1* __restrict__ out, int N, int K,
                               int deinterleave) {
    const int G = K >> 7, tiles = (N + 15) >> 4;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<int64_t>(tiles) * G * kBlockU4) return;
    const int lane = static_cast<int>(idx & 63);
    const int64_t block = idx >> 6;
    const int g = static_cast<int>(block % G), t = static_cast<int>(block / G);
    const int r = lane & 15, kb = lane >> 4;
    const int row = 16 * t + r;
    if (row >= N) return;
    const uint32_t magic = magic_reg();
    const u4 v = packed[idx];
    const int64_t sidx = param_offset(row, g, N, G);
    const GroupQ p = group_q(scales[sidx], zeros[sidx]);
    const int dst = deinterleave ? interleaved_source_row(row, N) : row;
    h8* o = reinterpret_cast<h8*>(out + static_cast<int64_t>(dst) * K + 128 * g + 32 * kb);
    o[0] = dequant_word(v.x, p, magic);
    o[1] = dequant_word(v.y, p, magic);
    o[2] = dequant_word(v.z, p, magic);
    o[3] = dequant_word(v.w, p, magic);
}

}  // namespace tw4

using namespace tw4;

extern "C" int tw4_repack_awq(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                              int32_t* packed, uint16_t* scales_out, uint16_t* zeros_out, int K, int N,
                              int interleave, void* stream) {
    TW4_REQUIRE(K > 0 && K % 128 == 0, TW4_EINVAL, "repack_awq: K %% 128 == 0 (K = %d, group 128 only)", K);
    TW4_REQUIRE(N > 0 && N % 8 == 0, TW4_EINVAL, "repack_awq: N %% 8 == 0 (N = %d)", N);
    TW4_REQUIRE(!interleave || N % 16 == 0, TW4_EINVAL, "repack_awq: interleave needs N %% 16 == 0 (N = %d)", N);
    TW4_REQUIRE(qweight && qzeros && scales && packed && scales_out && zeros_out, TW4_EINVAL,
                "repack_awq: null pointer");
    auto st = static_cast<hipStream_t>(stream);
    const int64_t words = static_cast<int64_t>(N >> 3) * (K >> 3);
    const int64_t params = static_cast<int64_t>(K >> 7) * N;
    repack_weights_kernel<<<static_cast<unsigned>((words + 255) / 256), 256, 0, st>>>(
        qweight, reinterpret_cast<uint32_t*>(packed), K, N, interleave);
    TW4_LAUNCH_CHECK("repack_awq: weight launch");
    repack_group_params_kernel<<<static_cast<unsigned>((params + 255) / 256), 256, 0, st>>>(
        qzeros, reinterpret_cast<const h1*>(scales), reinterpret_cast<h1*>(scales_out),
        reinterpret_cast<h1*>(zeros_out), K, N, interleave);
    TW4_LAUNCH_CHECK("repack_awq: group-parameter launch");
    return TW4_OK;
}

extern "C" int tw4_dequant(const int32_t* packed, const uint16_t* scales, const uint16_t* zeros, uint16_t* out,
                           int N, int K, int deinterleave, void* stream) {
    TW4_REQUIRE(K > 0 && K % 128 == 0, TW4_EINVAL, "dequant: K %% 128 == 0 (K = %d)", K);
    TW4_REQUIRE(N > 0 && N % 8 == 0, TW4_EINVAL, "dequant: N %% 8 == 0 (N = %d)", N);
    TW4_REQUIRE(!deinterleave || N % 16 == 0, TW4_EINVAL, "dequant: deinterleave needs N %% 16 == 0 (N = %d)", N);
    TW4_REQUIRE(packed && scales && zeros && out, TW4_EINVAL, "dequant: null pointer");
    TW4_REQUIRE(reinterpret_cast<uintptr_t>(packed) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
                TW4_EINVAL, "dequant: packed and out must be 16-byte aligned");
    const int64_t vecs = static_cast<int64_t>((N + 15) >> 4) * (K >> 7) * kBlockU4;
    dequant_kernel<<<static_cast<unsigned>((vecs + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        reinterpret_cast<const u4*>(packed), reinterpret_cast<const h1*>(scales), reinterpret_cast<const h1*>(zeros),
        reinterpret_cast<h1*>(out), N, K, deinterleave);
    TW4_LAUNCH_CHECK("dequant: launch");
    return TW4_OK;
}
