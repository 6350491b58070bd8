// tq_mfma.h -- fp32 matrix-core chains shared by the encoders and decoders (gfx950).
//
// v_mfma_f32_16x16x4_f32 adds the four products of its k = 0..3 to the accumulator one after
// another, each with one rounding (an fma chain in k order), so a chain of 32 of them over
// k-steps s = 0..31 covering d = 4s + k is the fma chain d = 0..127, bit for bit, denormals
// and signed zeros included.
//
// A wave works on a tile of 16 vectors.  Lane l = 16 g + v (v = l % 16, g = l / 16) holds
// element 4s + g of vector v for s = 0..31: the B operand (k = g, column v) of every product;
// a product's accumulator comes back to the lanes of its column v.  The matrix is the A
// operand, read from an LDS image laid out per (16-row tile t, k-step block sb): 64 lanes x 4
// consecutive k-steps, one 16-byte read per lane per block, lane slots xor-swizzled
// (slot = l ^ (l >> 4)).  In the CONTIG row order, row m = 4q + i of tile t is output index
// 32q + 4t + i, so lane g ends up holding outputs [32g, 32g + 32) of its vector.

#pragma once

#include <cstdint>

#include "tq_common.h"

namespace tqmx {

constexpr int MXD = TQ_DIM;

typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int MQ_WAVES = 8;                 // waves per workgroup, each on its own tiles
constexpr int MQ_THREADS = 64 * MQ_WAVES;

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// floor(n / d) = (n * m) >> s for 0 <= n < 2^31 and 1 <= d < 2^31, with l = ceil(log2 d),
// s = 31 + l and m = ceil(2^s / d) < 2^32: then 2^s <= m d <= 2^s + 2^l (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994, Theorem 4.2).
struct FastDiv {
    uint32_t m, s;
};
inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    return {(uint32_t)(((1ull << (31 + l)) + d - 1) / d), 31 + l};
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) {
    return (uint32_t)(((uint64_t)n * f.m) >> f.s);
}

// Rotation / QJL products of one tile: acc[t][i] = chain over d of b[d] * M[row(t, 4g + i)][d],
// with b held as described above (b[s] = element 4s + g) and `a` this lane's slot of image M.
// NT < 8 computes the row tiles t = 0..NT-1 of an image pointer advanced by t0 * 8 * 64.
template <int NT = 8>
__device__ __forceinline__ void image_products(const float4* __restrict__ a, const float* b, f32x4* acc) {
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // two register sets of A values: block sb + 1 is read while block sb's products run; the
    // scheduling barriers keep the compiler from hoisting every block's reads to the top
    float4 cur[NT], nxt[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) cur[t] = a[t * 8 * 64];
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) {
        if (sb + 1 < 8) {
#pragma unroll
            for (int t = 0; t < NT; ++t) nxt[t] = a[(t * 8 + sb + 1) * 64];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float ae = e == 0 ? cur[t].x : e == 1 ? cur[t].y : e == 2 ? cur[t].z : cur[t].w;
                acc[t] = mfma_f32(ae, b[4 * sb + e], acc[t]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NT; ++t) cur[t] = nxt[t];
    }
}

// CONTIG image of M^T for a matrix M of `rows` <= MXD rows of MXD floats: row r of the image
// is column r of M, and its k-index d is row d - (MXD - rows) of M, the first MXD - rows
// k-indices zero.  A chain over the image then starts with that many zero products, which
// leave its +0 start unchanged (+0 plus a zero of either sign is +0), so it is the fma chain
// over M's rows, bit for bit.
__device__ __forceinline__ void build_image_transposed(float* img, const float* __restrict__ M, int rows = MXD) {
    const int pad = MXD - rows;
    for (int idx = threadIdx.x; idx < MXD * MXD; idx += MQ_THREADS) {
        const int d = idx / MXD, r = idx % MXD;  // consecutive threads read along one row of M
        const int q = r >> 5, t = (r >> 2) & 7, m = 4 * q + (r & 3);
        const int s = d >> 2, k = d & 3;
        img[(t * 8 + (s >> 2)) * 256 + (s & 3) + 4 * ((16 * k + m) ^ k)] =
            d >= pad ? M[(size_t)(d - pad) * MXD + r] : 0.0f;
    }
}

}  // namespace tqmx
