// tq_group.hip -- channel-group (outlier split) encoder and decoder kernels for gfx950.
//
// A channel group is a sorted subset of the D = 128 head channels with its own
// rotation, codebook, bit width (1..8) and, for Q_prod keys, QJL matrix, all of the
// group's dimension d.  Reference: PackedMSELayer._encode_split /
// _encode_keys_split_qjl (runtime/packed_qmse_cache.py:481-496, 437-454) gather
// tensor[..., idx] and run _encode_group / _encode_keys_qjl_group (:376-402,
// :285-310) on the d-dimensional sub-vectors; _decode_merge / _decode_keys_merge_qjl
// (:498-515, :456-479) decode each group (:404-435, :312-330) and scatter it back
// into the full row.
//
// The kernels never gather.  One lane owns one token vector and holds the whole
// 128-channel row with the channels outside the group set to zero; the group's d x d
// matrices arrive in channel space (tq_group_matrix: row j < d carries the group
// matrix row j at the group's channels, every other entry 0).  Every fp32 reduction is
// an fma chain over the channels in ascending order, the group's channels ascend, and
// an fma whose product is zero returns its addend (up to the sign of a zero sum), so
// each chain equals the chain over the gathered d-dimensional sub-vector term for
// term.  Rows j >= d are skipped.  Codes, norms, signs and the decoded values are
// therefore bit-identical to the plain encoder / decoder run at D = d on the gathered
// sub-vectors, which is how the CPU oracle states them.
//
// The decoder of groups wider than 24 channels runs on the fp32 matrix cores instead
// (dequantize_group_mfma_kernel below, with the chains of tq_mfma.h): same chains, same
// bits.
//
// Packed rows are ceil(d*bits/8) code bytes and ceil(d/8) sign bytes per token, LSB
// first, zero padded (runtime/packed_qmse_cache.py:13-43, 148-154); lanes write them
// byte by byte, so no alignment is required of those buffers.

#include <math.h>

#include <algorithm>
#include <type_traits>

#include "tq_common.h"
#include "tq_mfma.h"

namespace {

constexpr int D = TQ_DIM;
constexpr int GBLOCK = 256;  // lanes (= vectors) per workgroup
constexpr int MAX_BITS = 8;

// Channel c is in the group iff bit c is set.  Passed by value: uniform (SGPR) words,
// and with c a compile-time constant after unrolling each test is a scalar bit test.
struct ChanMask {
    uint32_t w[D / 32];
};

__device__ __forceinline__ bool in_group(const ChanMask& m, int c) { return (m.w[c >> 5] >> (c & 31)) & 1u; }

// Channels 8i..8i+7 of the lane's row, those outside the group zeroed, bf16 -> fp32.
__device__ __forceinline__ void load_masked8(const uint16_t* xv, int i, const ChanMask& m, float* o) {
    const uint4 w = reinterpret_cast<const uint4*>(xv)[i];
    const uint32_t h[8] = {w.x & 0xFFFFu, w.x >> 16, w.y & 0xFFFFu, w.y >> 16,
                           w.z & 0xFFFFu, w.z >> 16, w.w & 0xFFFFu, w.w >> 16};
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = in_group(m, 8 * i + k) ? tq::bf16_to_f32(h[k]) : 0.0f;
}

__device__ __forceinline__ void load_masked(const uint16_t* xv, const ChanMask& m, float* o) {
#pragma unroll
    for (int i = 0; i < D / 8; ++i) load_masked8(xv, i, m, o + 8 * i);
}

// #{i : b[i] < z} (torch.bucketize right=False) by binary search over the sorted
// boundaries in LDS: the predicate holds on a prefix, `bits` probes.
__device__ __forceinline__ uint32_t bucket_lds(float z, const float* s_b, int bits) {
    uint32_t c = 0;
    for (uint32_t s = 1u << (bits - 1); s > 0; s >>= 1) c += (s_b[c + s - 1] < z) ? s : 0u;
    return c;
}

// LSB-first bit stream written byte by byte into the lane's own row.
struct ByteWriter {
    uint8_t* dst;
    uint32_t acc = 0;
    int fill = 0;
    __device__ __forceinline__ explicit ByteWriter(uint8_t* d) : dst(d) {}
    __device__ __forceinline__ void put(uint32_t v, int nbits) {  // nbits <= 8: at most one byte
        acc |= v << fill;
        fill += nbits;
        if (fill >= 8) {
            *dst++ = (uint8_t)acc;
            acc >>= 8;
            fill -= 8;
        }
    }
    __device__ __forceinline__ void flush() {
        if (fill > 0) *dst = (uint8_t)acc;
    }
};

template <bool PROD>
__global__ __launch_bounds__(GBLOCK) void quantize_group_kernel(
    const uint16_t* __restrict__ x, int heads, int64_t tokens, int64_t n_vec, int64_t x_sb, int64_t x_sh,
    int64_t x_st, ChanMask mask, int sub_dim, int bits, const float* __restrict__ R,
    const float* __restrict__ centers, const float* __restrict__ boundaries, const float* __restrict__ S,
    uint8_t* __restrict__ codes, uint16_t* __restrict__ norms, uint8_t* __restrict__ signs,
    uint16_t* __restrict__ rnorms, int64_t out_cap, int64_t out_offset) {
    __shared__ float s_bound[(1 << MAX_BITS) - 1];
    __shared__ float s_centers[PROD ? (1 << MAX_BITS) : 1];
    __shared__ uint8_t s_code[PROD ? D : 1][GBLOCK];  // PROD: codes of each lane, column per lane
    const int nb = (1 << bits) - 1;
    for (int i = threadIdx.x; i < nb; i += GBLOCK) s_bound[i] = boundaries[i];
    if (PROD)
        for (int i = threadIdx.x; i <= nb; i += GBLOCK) s_centers[i] = centers[i];
    __syncthreads();

    const int64_t v = (int64_t)blockIdx.x * GBLOCK + threadIdx.x;
    if (v >= n_vec) return;  // no barrier below this point
    const int64_t t = v % tokens;
    const int64_t gh = v / tokens;
    const int64_t h = gh % heads;
    const int64_t b = gh / heads;
    const uint16_t* xv = x + b * x_sb + h * x_sh + t * x_st;
    const int64_t slot = gh * out_cap + out_offset + t;

    // ---- norm and direction of the group's sub-vector
    float u[D];
    load_masked(xv, mask, u);
    float ss = 0.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) ss = __builtin_fmaf(u[d], u[d], ss);
    float n = tq::sqrt_rn(ss);
    if (!(n > 0.0f)) n = 1.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) u[d] = tq::div_rn(u[d], n);
    const uint32_t n16 = tq::f32_to_f16(n);
    norms[slot] = (uint16_t)n16;

    // ---- rotate (rows j < d), bucketize, pack
    ByteWriter bw(codes + slot * (int64_t)((sub_dim * bits + 7) >> 3));
    for (int j = 0; j < sub_dim; ++j) {
        const float* rj = R + j * D;
        float z = 0.0f;
#pragma unroll
        for (int d = 0; d < D; ++d) z = __builtin_fmaf(u[d], rj[d], z);
        const uint32_t c = bucket_lds(z, s_bound, bits);
        bw.put(c, bits);
        if (PROD) s_code[j][threadIdx.x] = (uint8_t)c;
    }
    bw.flush();

    if constexpr (PROD) {
        // ---- residual decode khat = bf16((C[code] @ R) * f32(f16(n))), rows j < d
        float* acc = u;  // u is dead after the rotation
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int j = 0; j < sub_dim; ++j) {
            const float cj = s_centers[s_code[j][threadIdx.x]];
            const float* rj = R + j * D;
#pragma unroll
            for (int d = 0; d < D; ++d) acc[d] = __builtin_fmaf(cj, rj[d], acc[d]);
        }
        const float nf = tq::f16_to_f32(n16);
        __asm__ volatile("" ::: "memory");  // x is re-read here, 16 bytes at a time, not held
        float rs = 0.0f;
#pragma unroll
        for (int i = 0; i < D / 8; ++i) {
            float xr[8];
            load_masked8(xv, i, mask, xr);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int d = 8 * i + k;
                const float kh = tq::bf16_to_f32(tq::f32_to_bf16(acc[d] * nf));
                acc[d] = xr[k] - kh;  // 0 - 0 outside the group: R's columns there are zero
                rs = __builtin_fmaf(acc[d], acc[d], rs);
            }
        }
        float rho = tq::sqrt_rn(rs);
        if (!(rho > 0.0f)) rho = 1.0f;
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = tq::div_rn(acc[d], rho);
        rnorms[slot] = (uint16_t)tq::f32_to_f16(rho);
        ByteWriter sw(signs + slot * (int64_t)((sub_dim + 7) >> 3));
        for (int i = 0; i < sub_dim; ++i) {
            const float* si = S + i * D;
            float p = 0.0f;
#pragma unroll
            for (int d = 0; d < D; ++d) p = __builtin_fmaf(acc[d], si[d], p);
            sw.put(p >= 0.0f ? 1u : 0u, 1);
        }
        sw.flush();
    }
}

// Decode-append sizes (below GQ_SMALL vectors): a workgroup encodes GAV vectors with D threads
// each.  Thread (v, j) runs output j's chains of vector v -- z_j and p_j for j < d, khat_j for
// every channel j -- and every thread of a vector runs the two norm chains over the masked row
// held in LDS (the same operands in the same order: one value in all of them).  These are the
// lane kernel's chains term for term, so the outputs are bit-identical to it.  The channel-space
// matrices are staged in LDS with a row stride of GMS = 132 floats (rows read 16 bytes at a time
// and columns read one float at a time both spread over the banks).
constexpr int GAV = 4;                 // vectors per workgroup
constexpr int GAT = GAV * D;           // threads per workgroup
constexpr int GMS = D + 4;             // LDS row stride of a staged matrix, floats
constexpr int64_t GQ_SMALL = 8192;     // below this many vectors the small-batch kernel runs

template <bool PROD>
__global__ __launch_bounds__(GAT) void quantize_group_small_kernel(
    const uint16_t* __restrict__ x, int heads, int64_t tokens, int64_t n_vec, int64_t x_sb, int64_t x_sh,
    int64_t x_st, ChanMask mask, int sub_dim, int bits, const float* __restrict__ R,
    const float* __restrict__ centers, const float* __restrict__ boundaries, const float* __restrict__ S,
    uint8_t* __restrict__ codes, uint16_t* __restrict__ norms, uint8_t* __restrict__ signs,
    uint16_t* __restrict__ rnorms, int64_t out_cap, int64_t out_offset) {
    __shared__ float4 sR[D * GMS / 4];
    __shared__ float4 sS[PROD ? D * GMS / 4 : 1];
    __shared__ float4 sx[GAV][D / 4];   // the masked vector, later rhat
    __shared__ float4 su[GAV][D / 4];   // u = x / n, later the residual
    __shared__ float sc[GAV][D];        // C[code_j], j < d
    __shared__ uint8_t scode[GAV][D];
    __shared__ float s_bound[(1 << MAX_BITS) - 1];
    __shared__ float s_centers[PROD ? (1 << MAX_BITS) : 1];

    const int tid = threadIdx.x;
    const int vi = tid / D, j = tid % D;  // vector of the workgroup (two whole waves), output index
    const int64_t v = (int64_t)blockIdx.x * GAV + vi;
    const bool active = v < n_vec;        // threads of missing vectors compute on unused LDS, store nothing
    float* const fx = reinterpret_cast<float*>(sx[vi]);
    float* const fu = reinterpret_cast<float*>(su[vi]);
    const int nb = (1 << bits) - 1;
    for (int i = tid; i < nb; i += GAT) s_bound[i] = boundaries[i];
    if (PROD)
        for (int i = tid; i <= nb; i += GAT) s_centers[i] = centers[i];

    int64_t slot = 0;
    if (active) {
        const int64_t t = v % tokens, gh = v / tokens;
        const int64_t h = gh % heads, b = gh / heads;
        const uint32_t mw = j < 32 ? mask.w[0] : j < 64 ? mask.w[1] : j < 96 ? mask.w[2] : mask.w[3];
        fx[j] = ((mw >> (j & 31)) & 1u) ? tq::bf16_to_f32(x[b * x_sb + h * x_sh + t * x_st + j]) : 0.0f;
        slot = gh * out_cap + out_offset + t;
    }
    for (int k = tid; k < D * D / 4; k += GAT) {
        const int r = k / (D / 4), c4 = k % (D / 4);
        sR[r * (GMS / 4) + c4] = reinterpret_cast<const float4*>(R)[k];
        if constexpr (PROD) sS[r * (GMS / 4) + c4] = reinterpret_cast<const float4*>(S)[k];
    }
    __syncthreads();

    // ---- norm of the group's sub-vector, u = x / n
    float ss = 0.0f;
#pragma unroll
    for (int d4 = 0; d4 < D / 4; ++d4) {
        const float4 e = sx[vi][d4];
        ss = __builtin_fmaf(e.x, e.x, ss);
        ss = __builtin_fmaf(e.y, e.y, ss);
        ss = __builtin_fmaf(e.z, e.z, ss);
        ss = __builtin_fmaf(e.w, e.w, ss);
    }
    float n = tq::sqrt_rn(ss);
    if (!(n > 0.0f)) n = 1.0f;
    const float xj = fx[j];
    fu[j] = tq::div_rn(xj, n);
    const uint32_t n16 = tq::f32_to_f16(n);
    if (active && j == 0) norms[slot] = (uint16_t)n16;
    __syncthreads();

    // ---- z_j (rows j < d), code_j
    float z = 0.0f;
    {
        const float4* rj = sR + j * (GMS / 4);
#pragma unroll
        for (int d4 = 0; d4 < D / 4; ++d4) {
            const float4 uu = su[vi][d4], rr = rj[d4];
            z = __builtin_fmaf(uu.x, rr.x, z);
            z = __builtin_fmaf(uu.y, rr.y, z);
            z = __builtin_fmaf(uu.z, rr.z, z);
            z = __builtin_fmaf(uu.w, rr.w, z);
        }
    }
    const uint32_t code = j < sub_dim ? bucket_lds(z, s_bound, bits) : 0u;
    scode[vi][j] = (uint8_t)code;
    if constexpr (PROD) sc[vi][j] = s_centers[code];
    __syncthreads();

    // ---- the code row, ceil(d bits / 8) bytes: thread j builds byte j (stream bits [8 j, 8 j + 8))
    const int rb = (sub_dim * bits + 7) >> 3;
    if (active && j < rb) {
        const int b0 = 8 * j;
        const int k1 = (b0 + 7) / bits < sub_dim - 1 ? (b0 + 7) / bits : sub_dim - 1;
        uint32_t acc = 0;
        for (int k = b0 / bits; k <= k1; ++k) acc |= (uint32_t)scode[vi][k] << (k * bits - b0 + 8);  // shift in [9 - bits, 15]
        codes[slot * rb + j] = (uint8_t)(acc >> 8);
    }

    if constexpr (PROD) {
        // ---- residual: khat_c = bf16((fma chain jj < d of C[code_jj] R[jj][c]) * f32(f16(n))), c = j
        const float* fR = reinterpret_cast<const float*>(sR);
        float acc = 0.0f;
        for (int jj = 0; jj < sub_dim; ++jj) acc = __builtin_fmaf(sc[vi][jj], fR[jj * GMS + j], acc);
        const float kh = tq::bf16_to_f32(tq::f32_to_bf16(acc * tq::f16_to_f32(n16)));
        const float r = xj - kh;  // 0 - 0 outside the group: R's columns there are zero
        fu[j] = r;                // u was last read by the rotation, before the barrier above
        __syncthreads();
        float rs = 0.0f;
#pragma unroll
        for (int d4 = 0; d4 < D / 4; ++d4) {
            const float4 e = su[vi][d4];
            rs = __builtin_fmaf(e.x, e.x, rs);
            rs = __builtin_fmaf(e.y, e.y, rs);
            rs = __builtin_fmaf(e.z, e.z, rs);
            rs = __builtin_fmaf(e.w, e.w, rs);
        }
        float rho = tq::sqrt_rn(rs);
        if (!(rho > 0.0f)) rho = 1.0f;
        fx[j] = tq::div_rn(r, rho);  // x was last read before the first barrier
        if (active && j == 0) rnorms[slot] = (uint16_t)tq::f32_to_f16(rho);
        __syncthreads();
        // ---- sign_i (i = j < d): fma chain over the channels of rhat_c S[i][c]
        float p = 0.0f;
        const float4* si = sS + j * (GMS / 4);
#pragma unroll
        for (int d4 = 0; d4 < D / 4; ++d4) {
            const float4 hh = sx[vi][d4], ww = si[d4];
            p = __builtin_fmaf(hh.x, ww.x, p);
            p = __builtin_fmaf(hh.y, ww.y, p);
            p = __builtin_fmaf(hh.z, ww.z, p);
            p = __builtin_fmaf(hh.w, ww.w, p);
        }
        const uint64_t sb = __builtin_amdgcn_ballot_w64(j < sub_dim && p >= 0.0f);  // bit l: index 64 (j / 64) + l
        const int l = j & 63, byte = 8 * (j >> 6) + l;  // lanes 0..7 of a wave write its 8 bytes
        if (active && l < 8 && byte < ((sub_dim + 7) >> 3))
            signs[slot * ((sub_dim + 7) >> 3) + byte] = (uint8_t)(sb >> (8 * l));
    }
}

// out = bf16((C[code] @ R) * f32(norm)) on the group's channels; with QJL (Q_prod keys)
// corr = bf16(((s @ S) * rnorm) * qs), out = bf16(f32(khat) + f32(corr)).  Channels
// outside the group are zeroed, or kept from `out` when `merge` is set.
template <bool QJL>
__global__ __launch_bounds__(GBLOCK) void dequantize_group_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ norms, const uint8_t* __restrict__ signs,
    const uint16_t* __restrict__ rnorms, int64_t tokens, int64_t cap, int64_t n_vec, ChanMask mask, int sub_dim,
    int bits, const float* __restrict__ R, const float* __restrict__ centers, const float* __restrict__ S, float qs,
    int merge, uint16_t* __restrict__ out) {
    __shared__ float s_centers[1 << MAX_BITS];
    for (int i = threadIdx.x; i < (1 << bits); i += GBLOCK) s_centers[i] = centers[i];
    __syncthreads();
    const int64_t v = (int64_t)blockIdx.x * GBLOCK + threadIdx.x;
    if (v >= n_vec) return;
    const int64_t g = v / tokens, t = v % tokens;
    const int64_t slot = g * cap + t;
    const uint8_t* row = codes + slot * (int64_t)((sub_dim * bits + 7) >> 3);
    const uint32_t cmask = (1u << bits) - 1u;
    float acc[D];
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] = 0.0f;
    for (int j = 0; j < sub_dim; ++j) {
        const int pos = j * bits;
        uint32_t pair = row[pos >> 3];
        if ((pos & 7) + bits > 8) pair |= (uint32_t)row[(pos >> 3) + 1] << 8;
        const float cj = s_centers[(pair >> (pos & 7)) & cmask];
        const float* rj = R + j * D;
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = __builtin_fmaf(cj, rj[d], acc[d]);
    }
    const float nf = tq::f16_to_f32(norms[slot]);
    uint32_t kh[D / 2];  // bf16 pairs
#pragma unroll
    for (int i = 0; i < D / 2; ++i)
        kh[i] = tq::f32_to_bf16(acc[2 * i] * nf) | (tq::f32_to_bf16(acc[2 * i + 1] * nf) << 16);
#pragma unroll
    for (int i = 0; i < D / 2; ++i) __asm__("" : "+v"(kh[i]));  // packed here: acc dies before the QJL part
    if constexpr (QJL) {
        // the correction in two halves of D/2 channels (each channel's fma chain is unchanged)
        const uint8_t* srow = signs + slot * (int64_t)((sub_dim + 7) >> 3);
        const float rn = tq::f16_to_f32(rnorms[slot]);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float cacc[D / 2];
#pragma unroll
            for (int d = 0; d < D / 2; ++d) cacc[d] = 0.0f;
            for (int i = 0; i < sub_dim; ++i) {
                const float si = ((srow[i >> 3] >> (i & 7)) & 1u) ? 1.0f : -1.0f;
                const float* Si = S + i * D + half * (D / 2);
#pragma unroll
                for (int d = 0; d < D / 2; ++d) cacc[d] = __builtin_fmaf(si, Si[d], cacc[d]);
            }
#pragma unroll
            for (int i = 0; i < D / 4; ++i) {
                const int p = half * (D / 4) + i;
                const float c0 = tq::bf16_to_f32(tq::f32_to_bf16((cacc[2 * i] * rn) * qs));
                const float c1 = tq::bf16_to_f32(tq::f32_to_bf16((cacc[2 * i + 1] * rn) * qs));
                const float k0 = tq::bf16_to_f32(kh[p] & 0xFFFFu) + c0;
                const float k1 = tq::bf16_to_f32(kh[p] >> 16) + c1;
                kh[p] = tq::f32_to_bf16(k0) | (tq::f32_to_bf16(k1) << 16);
            }
        }
    }
    uint4* o4 = reinterpret_cast<uint4*>(out + v * D);
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
        uint32_t m[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            m[k] = (in_group(mask, 8 * i + 2 * k) ? 0x0000FFFFu : 0u) |
                   (in_group(mask, 8 * i + 2 * k + 1) ? 0xFFFF0000u : 0u);
        if (merge && (m[0] | m[1] | m[2] | m[3]) == 0u) continue;  // no channel of the group: kept as is
        uint4 w = make_uint4(kh[4 * i] & m[0], kh[4 * i + 1] & m[1], kh[4 * i + 2] & m[2], kh[4 * i + 3] & m[3]);
        if (merge) {
            const uint4 old = o4[i];
            w.x |= old.x & ~m[0];
            w.y |= old.y & ~m[1];
            w.z |= old.z & ~m[2];
            w.w |= old.w & ~m[3];
        }
        o4[i] = w;
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Validates a group's channel list (host memory): 1 <= sub_dim <= dim, strictly
// ascending, within [0, dim).  dim must be the kernels' D.
int group_mask(const int32_t* channels, int sub_dim, int dim, ChanMask* m) {
    if (!channels || sub_dim < 1 || dim < 1 || sub_dim > dim) return TQ_ERR_INVALID_ARGUMENT;
    if (dim != D) return TQ_ERR_UNSUPPORTED;
    for (int k = 0; k < D / 32; ++k) m->w[k] = 0;
    for (int i = 0; i < sub_dim; ++i) {
        const int32_t c = channels[i];
        if (c < 0 || c >= dim || (i > 0 && c <= channels[i - 1])) return TQ_ERR_INVALID_ARGUMENT;
        m->w[c >> 5] |= 1u << (c & 31);
    }
    return TQ_OK;
}

}  // namespace

extern "C" int tq_group_matrix(const float* sub, int sub_dim, const int32_t* channels, int dim, float* out) {
    if (!sub || !out || !channels || sub_dim < 1 || dim < 1 || sub_dim > dim) return TQ_ERR_INVALID_ARGUMENT;
    for (int i = 0; i < sub_dim; ++i)
        if (channels[i] < 0 || channels[i] >= dim || (i > 0 && channels[i] <= channels[i - 1]))
            return TQ_ERR_INVALID_ARGUMENT;
    for (int64_t k = 0; k < (int64_t)dim * dim; ++k) out[k] = 0.0f;
    for (int j = 0; j < sub_dim; ++j)
        for (int i = 0; i < sub_dim; ++i) out[(int64_t)j * dim + channels[i]] = sub[(int64_t)j * sub_dim + i];
    return TQ_OK;
}

extern "C" int tq_quantize_group(const uint16_t* x, int batch, int heads, int64_t tokens, int dim, int64_t x_sb,
                                 int64_t x_sh, int64_t x_st, const int32_t* channels, int sub_dim, int bits,
                                 const float* rotation, const float* centers, const float* boundaries,
                                 const float* qjl, uint8_t* codes, uint16_t* norms, uint8_t* signs,
                                 uint16_t* rnorms, int64_t out_cap, int64_t out_offset, void* stream) {
    if (!x || batch < 0 || heads < 0 || tokens < 0 || out_offset < 0 || out_offset + tokens > out_cap)
        return TQ_ERR_INVALID_ARGUMENT;
    ChanMask mask;
    int st = group_mask(channels, sub_dim, dim, &mask);
    if (st != TQ_OK) return st;
    if (bits < 1 || bits > MAX_BITS) return TQ_ERR_INVALID_ARGUMENT;
    const bool prod = qjl != nullptr;
    if (!rotation || !boundaries || !codes || !norms) return TQ_ERR_INVALID_ARGUMENT;
    if (prod && (!centers || !signs || !rnorms)) return TQ_ERR_INVALID_ARGUMENT;
    if (!aligned16(x) || (x_sb % 8) || (x_sh % 8) || (x_st % 8)) return TQ_ERR_UNSUPPORTED;
    const int64_t n_vec = (int64_t)batch * heads * tokens;
    if (n_vec == 0) return TQ_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!aligned16(rotation) || (prod && !aligned16(qjl))) return TQ_ERR_UNSUPPORTED;
    if (n_vec < GQ_SMALL) {
        const int64_t sblocks = (n_vec + GAV - 1) / GAV;
        if (prod)
            hipLaunchKernelGGL((quantize_group_small_kernel<true>), dim3((unsigned)sblocks), dim3(GAT), 0, s, x,
                               heads, tokens, n_vec, x_sb, x_sh, x_st, mask, sub_dim, bits, rotation, centers,
                               boundaries, qjl, codes, norms, signs, rnorms, out_cap, out_offset);
        else
            hipLaunchKernelGGL((quantize_group_small_kernel<false>), dim3((unsigned)sblocks), dim3(GAT), 0, s, x,
                               heads, tokens, n_vec, x_sb, x_sh, x_st, mask, sub_dim, bits, rotation, nullptr,
                               boundaries, nullptr, codes, norms, nullptr, nullptr, out_cap, out_offset);
        TQ_CHECK_LAUNCH();
        return TQ_OK;
    }
    const int64_t blocks = (n_vec + GBLOCK - 1) / GBLOCK;
    if (prod)
        hipLaunchKernelGGL((quantize_group_kernel<true>), dim3((unsigned)blocks), dim3(GBLOCK), 0, s, x, heads,
                           tokens, n_vec, x_sb, x_sh, x_st, mask, sub_dim, bits, rotation, centers, boundaries, qjl,
                           codes, norms, signs, rnorms, out_cap, out_offset);
    else
        hipLaunchKernelGGL((quantize_group_kernel<false>), dim3((unsigned)blocks), dim3(GBLOCK), 0, s, x, heads,
                           tokens, n_vec, x_sb, x_sh, x_st, mask, sub_dim, bits, rotation, nullptr, boundaries,
                           nullptr, codes, norms, nullptr, nullptr, out_cap, out_offset);
    TQ_CHECK_LAUNCH();
    return TQ_OK;
}

namespace {
using namespace tqmx;

// ------------------------------------------------------------------ matrix-core decoder
// The decoder above on the fp32 matrix cores, as the unsplit decoders: output channel c is the
// chain j = 0..d-1 of C[code_j] * R[j][c] (of sign_j * S[j][c] for the correction), with R the
// group's d x D matrix in channel space.  Its image holds R^T behind 128 - d zero k-indices, and
// the B operand is zero there too, so every chain starts with zero products that leave its +0
// start unchanged.  Code and sign rows (ceil(d b / 8) and ceil(d / 8) bytes, not aligned) are
// staged per wave in LDS through range-checked dword buffer loads; lane 16 g + v then takes
// the fields of indices 4s + g - (128 - d) from row v.  Lane 16 g + v ends with channels
// [32g, 32g + 32) of vector v and stores them as 64 bytes, the other group's channels zeroed
// or, with `merge`, kept.
// Groups of at most this many channels decode one lane per vector (dequantize_group_kernel):
// its chains are d terms long, where the matrix-core chains are padded to 128 (at a C2 layer
// the lane kernel is faster below about 24 channels for values, 34 for QJL keys).
constexpr int GDQ_LANE_MAX_DIM = 24;
constexpr int GRW = 34;  // staged dwords per code row: up to 128 bytes, a misaligned start, one spare
constexpr int GSW = 6;   // staged dwords per sign row: up to 16 bytes, a misaligned start, one spare

__device__ __forceinline__ __amdgpu_buffer_rsrc_t group_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Bits [bit, bit + n) (n <= 8) of the LDS dword array w.
__device__ __forceinline__ uint32_t staged_bits(const uint32_t* w, uint32_t bit, uint32_t n) {
    const uint32_t i = bit >> 5;
    return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(w[i + 1], w[i], bit & 31), 0, n);
}

// Row v's bytes [b0, b0 + r) as dwords from the one holding b0 into dst (the four lanes of a
// vector share the loads); returns b0's bit offset in dst.  `limit` is the buffer's extent in
// bytes (the descriptor's range): a dword that crosses it is assembled from byte loads, since
// a dword load past the range reads as zero whole, and bytes past it read as zero.
__device__ __forceinline__ uint32_t stage_row(uint32_t* dst, __amdgpu_buffer_rsrc_t rs, uint32_t limit, uint32_t b0,
                                              int r, int nw, int g, bool live) {
    const uint32_t a0 = b0 & ~3u;
    const int n = (int)((b0 + (uint32_t)r - a0 + 3) >> 2);
    for (int i = g; i < nw; i += 4) {
        const uint32_t off = a0 + 4u * (uint32_t)i;
        uint32_t w = 0u;
        if (live && i < n) {
            if (off + 4u <= limit) {
                w = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
            } else {
#pragma unroll
                for (uint32_t k = 0; k < 4; ++k)
                    if (off + k < limit) w |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, off + k, 0, 0) << (8 * k);
            }
        }
        dst[i] = w;
    }
    return 8 * (b0 - a0);
}

template <bool QJL, int PARTS>
__global__ __launch_bounds__(MQ_THREADS) void dequantize_group_mfma_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ norms, const uint8_t* __restrict__ signs,
    const uint16_t* __restrict__ rnorms, int64_t tokens, int64_t cap, int64_t n_vec, uint32_t code_bytes,
    uint32_t sign_bytes, ChanMask mask, int sub_dim, int bits, const float* __restrict__ R,
    const float* __restrict__ centers, const float* __restrict__ S, float qs, int merge, uint16_t* __restrict__ out,
    FastDiv tok_div) {
    __shared__ float4 s_img[(QJL ? 2 : 1) * D * D / 4];  // R^T image (+ S^T image)
    __shared__ float s_cent[1 << MAX_BITS];
    __shared__ uint32_t s_code[MQ_WAVES][16][GRW];
    __shared__ uint32_t s_sign[QJL ? MQ_WAVES : 1][16][GSW];
    float* img = reinterpret_cast<float*>(s_img);
    build_image_transposed(img, R, sub_dim);
    if constexpr (QJL) build_image_transposed(img + D * D, S, sub_dim);
    for (int i = threadIdx.x; i < (1 << bits); i += MQ_THREADS) s_cent[i] = centers[i];
    __syncthreads();  // the only barrier: each wave then works on its own tiles

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int v = lane & 15, g = lane >> 4;
    const float4* a_img = s_img + (lane ^ g);
    const int pad = D - sub_dim;
    const int rb = (sub_dim * bits + 7) >> 3, sbytes = (sub_dim + 7) >> 3;
    const __amdgpu_buffer_rsrc_t rc = group_rsrc(codes, code_bytes);
    const __amdgpu_buffer_rsrc_t rsg = group_rsrc(QJL ? signs : codes, QJL ? sign_bytes : 0u);
    const uint32_t mw = g == 0 ? mask.w[0] : g == 1 ? mask.w[1] : g == 2 ? mask.w[2] : mask.w[3];
    constexpr int NT = 8 / PARTS;  // row tiles (16 output channels each) per work item
    const int64_t n_items = (n_vec + 15) / 16 * PARTS;

    // work item = (tile of 16 vectors, part): part p computes row tiles [p NT, p NT + NT), the
    // channels 32g + [4 p NT, 4 p NT + 4 NT) of lane 16 g + v's vector
    for (int64_t item = (int64_t)blockIdx.x * MQ_WAVES + wave; item < n_items;
         item += (int64_t)gridDim.x * MQ_WAVES) {
        const int64_t tile = item / PARTS;
        const int t0 = (int)(item % PARTS) * NT;
        const uint32_t vi = (uint32_t)tile * 16u + (uint32_t)v;  // n_vec < 2^31
        const bool live = vi < (uint64_t)n_vec;
        uint32_t slot = 0;  // slot * row bytes < 2^31 (checked on the host)
        if (live) {
            const uint32_t gh = fdiv(vi, tok_div);
            slot = gh * (uint32_t)cap + (vi - gh * (uint32_t)tokens);
        }
        uint32_t* crow = s_code[wave][v];
        const uint32_t cbit = stage_row(crow, rc, code_bytes, slot * (uint32_t)rb, rb, GRW, g, live);
        uint32_t* srow = QJL ? s_sign[wave][v] : nullptr;
        uint32_t sbit = 0;
        if constexpr (QJL) sbit = stage_row(srow, rsg, sign_bytes, slot * (uint32_t)sbytes, sbytes, GSW, g, live);
        // the wave's LDS accesses complete in issue order; keep the compiler from moving the
        // reads above the writes (or the next tile's writes above these reads)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float cv[32];
#pragma unroll
        for (int s = 0; s < 32; ++s) {
            const int j = 4 * s + g - pad;
            cv[s] = j >= 0 ? s_cent[staged_bits(crow, cbit + (uint32_t)(j * bits), (uint32_t)bits)] : 0.0f;
        }
        f32x4 acc[NT];
        image_products<NT>(a_img + t0 * 8 * 64, cv, acc);
        const float nf = live ? tq::f16_to_f32(norms[slot]) : 0.0f;
        uint32_t kh[2 * NT];  // bf16 pairs of channels 32g + 4 t0 + 2p, + 2p + 1
#pragma unroll
        for (int p = 0; p < 2 * NT; ++p)
            kh[p] = tq::f32_to_bf16(acc[p >> 1][2 * (p & 1)] * nf) |
                    (tq::f32_to_bf16(acc[p >> 1][2 * (p & 1) + 1] * nf) << 16);
        if constexpr (QJL) {
            float sv[32];
#pragma unroll
            for (int s = 0; s < 32; ++s) {
                const int j = 4 * s + g - pad;
                sv[s] = j < 0 ? 0.0f : staged_bits(srow, sbit + (uint32_t)j, 1u) ? 1.0f : -1.0f;
            }
            f32x4 pacc[NT];
            image_products<NT>(a_img + D * D / 4 + t0 * 8 * 64, sv, pacc);
            const float rn = live ? tq::f16_to_f32(rnorms[slot]) : 0.0f;
#pragma unroll
            for (int p = 0; p < 2 * NT; ++p) {
                const float c0 = tq::bf16_to_f32(tq::f32_to_bf16((pacc[p >> 1][2 * (p & 1)] * rn) * qs));
                const float c1 = tq::bf16_to_f32(tq::f32_to_bf16((pacc[p >> 1][2 * (p & 1) + 1] * rn) * qs));
                const float k0 = tq::bf16_to_f32(kh[p] & 0xFFFFu) + c0;
                const float k1 = tq::bf16_to_f32(kh[p] >> 16) + c1;
                kh[p] = tq::f32_to_bf16(k0) | (tq::f32_to_bf16(k1) << 16);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (live) {
            uint4* o4 = reinterpret_cast<uint4*>(out + (int64_t)vi * D + 32 * g + 4 * t0);
#pragma unroll
            for (int i = 0; i < NT / 2; ++i) {
                uint32_t m[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int p = 2 * t0 + 4 * i + k;  // channel pair of the lane's 32 channels
                    m[k] = (((mw >> (2 * p)) & 1u) ? 0x0000FFFFu : 0u) | (((mw >> (2 * p + 1)) & 1u) ? 0xFFFF0000u : 0u);
                }
                if (merge && (m[0] | m[1] | m[2] | m[3]) == 0u) continue;  // no channel of the group
                uint4 w = make_uint4(kh[4 * i] & m[0], kh[4 * i + 1] & m[1], kh[4 * i + 2] & m[2], kh[4 * i + 3] & m[3]);
                if (merge) {
                    const uint4 old = o4[i];
                    w.x |= old.x & ~m[0];
                    w.y |= old.y & ~m[1];
                    w.z |= old.z & ~m[2];
                    w.w |= old.w & ~m[3];
                }
                o4[i] = w;
            }
        }
    }
}

int64_t group_decoder_groups(bool qjl) {
    static std::atomic<int64_t> cached[2][tq::MAX_DEVICES];
    return tq::once_per_device(cached[qjl ? 1 : 0], 256, [qjl](int dev) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 256;
        const hipError_t e = qjl ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                                       &per_cu, dequantize_group_mfma_kernel<true, 1>, MQ_THREADS, 0)
                                 : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                                       &per_cu, dequantize_group_mfma_kernel<false, 1>, MQ_THREADS, 0);
        if (e != hipSuccess || per_cu < 1) per_cu = 1;
        return (int64_t)cus * per_cu;
    });
}
}  // namespace

extern "C" int tq_dequantize_group(const uint8_t* codes, const uint16_t* norms, const uint8_t* signs,
                                   const uint16_t* rnorms, int64_t groups, int64_t tokens, int64_t cap, int dim,
                                   const int32_t* channels, int sub_dim, int bits, const float* rotation,
                                   const float* centers, const float* qjl, int merge, uint16_t* out,
                                   void* stream) {
    if (!codes || !norms || !rotation || !centers || !out || groups < 0 || tokens < 0 || tokens > cap)
        return TQ_ERR_INVALID_ARGUMENT;
    ChanMask mask;
    int st = group_mask(channels, sub_dim, dim, &mask);
    if (st != TQ_OK) return st;
    if (bits < 1 || bits > MAX_BITS) return TQ_ERR_INVALID_ARGUMENT;
    const bool has_qjl = qjl != nullptr;
    if (has_qjl && (!signs || !rnorms)) return TQ_ERR_INVALID_ARGUMENT;
    if (!aligned16(out)) return TQ_ERR_UNSUPPORTED;
    const int64_t n_vec = groups * tokens;
    if (n_vec == 0) return TQ_OK;
    // byte extents from `codes` / `signs` to the last row read: the staging loads are
    // range-checked against them, and 32-bit row offsets cover them
    const int64_t last = (groups - 1) * cap + tokens;
    const int64_t rb = (sub_dim * bits + 7) >> 3, sbytes = (sub_dim + 7) >> 3;
    if (n_vec >= ((int64_t)1 << 31) || last * rb >= ((int64_t)1 << 31) || cap >= ((int64_t)1 << 31))
        return TQ_ERR_UNSUPPORTED;
    // sqrt(pi/2)/d in double, rounded once to fp32 (the reference multiplies an fp32
    // tensor by this Python float)
    const float qs = (float)(sqrt(M_PI / 2.0) / (double)sub_dim);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (sub_dim <= GDQ_LANE_MAX_DIM) {
        const int64_t blocks = (n_vec + GBLOCK - 1) / GBLOCK;
        if (has_qjl)
            hipLaunchKernelGGL((dequantize_group_kernel<true>), dim3((unsigned)blocks), dim3(GBLOCK), 0, s, codes,
                               norms, signs, rnorms, tokens, cap, n_vec, mask, sub_dim, bits, rotation, centers, qjl,
                               qs, merge != 0, out);
        else
            hipLaunchKernelGGL((dequantize_group_kernel<false>), dim3((unsigned)blocks), dim3(GBLOCK), 0, s, codes,
                               norms, nullptr, nullptr, tokens, cap, n_vec, mask, sub_dim, bits, rotation, centers,
                               nullptr, qs, merge != 0, out);
        TQ_CHECK_LAUNCH();
        return TQ_OK;
    }
    // a call with fewer tiles than the device holds waves splits each tile's row tiles over
    // 2 or 4 waves (the same chains)
    const int64_t tiles = (n_vec + 15) / 16;
    const int64_t resident = group_decoder_groups(has_qjl);
    const int parts = 4 * tiles <= resident * MQ_WAVES ? 4 : 2 * tiles <= resident * MQ_WAVES ? 2 : 1;
    const int64_t wgs = std::min<int64_t>((tiles * parts + MQ_WAVES - 1) / MQ_WAVES, resident);
    const FastDiv td = make_fastdiv((uint32_t)tokens);
    const uint32_t cbytes = (uint32_t)(last * rb), sgbytes = has_qjl ? (uint32_t)(last * sbytes) : 0u;
    auto launch = [&](auto qjl_c, auto parts_c) {
        constexpr bool Q = decltype(qjl_c)::value;
        constexpr int PP = decltype(parts_c)::value;
        hipLaunchKernelGGL((dequantize_group_mfma_kernel<Q, PP>), dim3((unsigned)wgs), dim3(MQ_THREADS), 0, s, codes,
                           norms, Q ? signs : nullptr, Q ? rnorms : nullptr, tokens, cap, n_vec, cbytes, sgbytes, mask,
                           sub_dim, bits, rotation, centers, Q ? qjl : nullptr, qs, merge != 0, out, td);
    };
    using T = std::true_type;
    using F = std::false_type;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    using P4 = std::integral_constant<int, 4>;
    if (has_qjl) {
        if (parts == 4) launch(T{}, P4{});
        else if (parts == 2) launch(T{}, P2{});
        else launch(T{}, P1{});
    } else {
        if (parts == 4) launch(F{}, P4{});
        else if (parts == 2) launch(F{}, P2{});
        else launch(F{}, P1{});
    }
    TQ_CHECK_LAUNCH();
    return TQ_OK;
}
