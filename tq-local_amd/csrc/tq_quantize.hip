// tq_quantize.hip -- TurboQuant encoder kernels for gfx950 (prefill and decode-append).
//
// Every kernel evaluates the encoder in one fixed fp32 order (the CPU oracle restates the
// reference in the same order), so their outputs are bit-identical to it and to each other:
//
//   norm^2 = fma chain d=0..127 of x_d*x_d;  n = sqrt_rn;  n==0 -> 1
//   u_d    = x_d /_rn n
//   z_j    = fma chain d=0..127 of u_d*R[j][d]          (z = u @ R^T)
//   code_j = #{i : boundaries_i < z_j}                   (torch.bucketize right=False)
//   Q_prod residual:  khat_d = bf16((fma chain j=0..127 of C[code_j]*R[j][d]) * f32(f16(n)))
//                     r = x - khat;  rho = sqrt_rn(fma chain r_d^2) (0 -> 1);  rhat = r /_rn rho
//                     sign_i = (fma chain d of rhat_d*S[i][d]) >= 0
//
// Two encoders: the matrix-core kernel for calls of at least MQ_MIN_VECTORS vectors (prefill)
// and a small-batch kernel with one thread per output index of each vector (decode-append).
//
// Reference: runtime/packed_qmse_cache.py:376-402 (_encode_group), :285-310
// (_encode_keys_qjl_group), :404-435 (_decode_group), :13-43 (_pack_indices),
// :148-154 (_pack_qjl_signs).

#include <algorithm>
#include <type_traits>
#include <utility>

#include "tq_common.h"
#include "tq_mfma.h"

namespace {

using namespace tqmx;
constexpr int D = TQ_DIM;

struct QuantArgs {
    const uint16_t* x;
    int heads;
    int64_t tokens;
    int64_t n_vec;
    int64_t x_sb, x_sh, x_st;
    const float* R;
    const float* centers;
    const float* boundaries;
    const float* S;
    uint8_t* codes;
    uint16_t* norms;
    uint8_t* signs;
    uint16_t* rnorms;
    int64_t out_cap, out_offset;
};

// Appends `nbits` bits to a 64-bit staging register; full 32-bit words are
// written to `dst` (the lane's own output row).
struct BitWriter {
    uint64_t acc = 0;
    int fill = 0;
    int wi = 0;
    __device__ __forceinline__ void put(uint32_t v, int nbits, uint32_t* dst) {
        acc |= (uint64_t)v << fill;
        fill += nbits;
        if (fill >= 32) {
            dst[wi++] = (uint32_t)acc;
            acc >>= 32;
            fill -= 32;
        }
    }
};

// #{i : b[i] < z} (torch.bucketize right=False): one compare and one add-with-carry per
// boundary; the empty asm keeps the count a plain running sum (no bitmask reassociation).
template <int NB>
__device__ __forceinline__ uint32_t bucket_count(float z, const float* __restrict__ b) {
    uint32_t c = 0;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        c += (b[i] < z) ? 1u : 0u;
        __asm__("" : "+v"(c));
    }
    return c;
}

// The same count by binary search over the sorted boundaries (the predicate b[i] < z holds on
// a prefix): BITS compares, and at level l a select tree over the 2^l candidate thresholds
// driven by the earlier outcomes (2^BITS - BITS - 1 selects in all, against 2^BITS - 1
// compare/add pairs for the linear count).
template <int BITS>
__device__ __forceinline__ uint32_t bucket_search(float z, const float* __restrict__ b) {
    bool p[BITS];
    uint32_t c = 0;
#pragma unroll
    for (int lvl = 0; lvl < BITS; ++lvl) {
        const int s = 1 << (BITS - 1 - lvl);
        float cand[1 << (BITS - 1)];
#pragma unroll
        for (int m = 0; m < (1 << lvl); ++m) cand[m] = b[s - 1 + 2 * s * m];
        // candidate m = sum_q p[q] 2^(lvl - 1 - q): reduce by the last outcome first
#pragma unroll
        for (int q = lvl - 1; q >= 0; --q) {
            const int half = 1 << q;  // entries left after this step
#pragma unroll
            for (int m = 0; m < half; ++m) cand[m] = p[q] ? cand[2 * m + 1] : cand[2 * m];
        }
        p[lvl] = cand[0] < z;
        c |= p[lvl] ? (uint32_t)s : 0u;
    }
    return c;
}

// ------------------------------------------------------------------ small-batch encoder
// Below MQ_MIN_VECTORS vectors (decode-append encodes B * Hkv of them per step) a workgroup
// encodes AV vectors with D threads each: thread (v, j) owns output index j of vector v in
// every matrix-vector product and runs that output's fma chain alone, in the fixed order
// above, so the result is bit for bit the chain of the oracle and of the matrix-core kernel.
// The matrices are staged in LDS with a row stride of MS = 132 floats: thread j reading row j
// 16 bytes at a time (the rotation and the QJL projection) touches 4 j + 4 k mod 64, distinct
// banks for the 16 lanes of an LDS pass, and thread d reading column d (the residual decode)
// touches consecutive banks.  The norms are fma chains over the vector held in LDS, run by
// every thread of the vector (the same operands in the same order: one value in all of them).
constexpr int AV = 4;          // vectors per workgroup
constexpr int AT = AV * D;     // threads per workgroup
constexpr int MS = D + 4;      // LDS row stride of a staged matrix, floats

template <int BITS, bool PROD>
__global__ __launch_bounds__(AT) void append_kernel(
    const uint16_t* __restrict__ x, int heads, int64_t tokens, int64_t n_vec, int64_t x_sb, int64_t x_sh,
    int64_t x_st, const float* __restrict__ R, const float* __restrict__ centers,
    const float* __restrict__ boundaries, const float* __restrict__ S, uint8_t* __restrict__ codes,
    uint16_t* __restrict__ norms, uint8_t* __restrict__ signs, uint16_t* __restrict__ rnorms, int64_t out_cap,
    int64_t out_offset) {
    __shared__ float4 sR[D * MS / 4];
    __shared__ float4 sS[PROD ? D * MS / 4 : 1];
    __shared__ float4 sx[AV][D / 4];    // the vector in fp32, later rhat
    __shared__ float4 su[AV][D / 4];    // u = x / n, later the residual
    __shared__ float4 sc[AV][D / 4];    // C[code_j]
    __shared__ uint8_t scode[AV][D];
    __shared__ float scent[1 << BITS];

    const int tid = threadIdx.x;
    const int vi = tid / D, j = tid % D;  // vector of the workgroup (two whole waves), output index
    const int64_t v = (int64_t)blockIdx.x * AV + vi;
    const bool active = v < n_vec;        // threads of missing vectors compute on unused LDS, store nothing
    float* const fx = reinterpret_cast<float*>(sx[vi]);
    float* const fu = reinterpret_cast<float*>(su[vi]);
    float* const fc = reinterpret_cast<float*>(sc[vi]);

    // ---- the vector, the codebook and the matrices into LDS (row r of a matrix at r * MS)
    int64_t slot = 0;
    if (active) {
        const int64_t t = v % tokens, gh = v / tokens;
        const int64_t h = gh % heads, b = gh / heads;
        fx[j] = tq::bf16_to_f32(x[b * x_sb + h * x_sh + t * x_st + j]);
        slot = gh * out_cap + out_offset + t;
    }
    if (PROD && tid < (1 << BITS)) scent[tid] = centers[tid];
    for (int k = tid; k < D * D / 4; k += AT) {
        const int r = k / (D / 4), c4 = k % (D / 4);
        sR[r * (MS / 4) + c4] = reinterpret_cast<const float4*>(R)[k];
        if constexpr (PROD) sS[r * (MS / 4) + c4] = reinterpret_cast<const float4*>(S)[k];
    }
    __syncthreads();

    // ---- norm, u = x / n
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

    // ---- z_j = fma chain d of u_d R[j][d]; code_j
    float z = 0.0f;
    {
        const float4* rj = sR + j * (MS / 4);
#pragma unroll
        for (int d4 = 0; d4 < D / 4; ++d4) {
            const float4 uu = su[vi][d4], rr = rj[d4];
            z = __builtin_fmaf(uu.x, rr.x, z);
            z = __builtin_fmaf(uu.y, rr.y, z);
            z = __builtin_fmaf(uu.z, rr.z, z);
            z = __builtin_fmaf(uu.w, rr.w, z);
        }
    }
    const uint32_t code = bucket_count<(1 << BITS) - 1>(z, boundaries);
    scode[vi][j] = (uint8_t)code;
    if constexpr (PROD) fc[j] = scent[code];
    __syncthreads();

    // ---- the code row: thread j < ROW / 4 assembles dword j (stream bits [32 j, 32 j + 32))
    constexpr int ROW = D * BITS / 8;
    if (active && j < ROW / 4) {
        const int b0 = 32 * j;
        uint64_t acc = 0;
        for (int k = b0 / BITS; k <= (b0 + 31) / BITS; ++k)
            acc |= (uint64_t)scode[vi][k] << (k * BITS - b0 + 32);  // shift in [33 - BITS, 63]
        reinterpret_cast<uint32_t*>(codes + slot * ROW)[j] = (uint32_t)(acc >> 32);
    }

    if constexpr (PROD) {
        // ---- residual: khat_d = bf16((fma chain jj of C[code_jj] R[jj][d]) * f32(f16(n))), d = j
        const float* fR = reinterpret_cast<const float*>(sR);
        float acc = 0.0f;
#pragma unroll
        for (int k4 = 0; k4 < D / 4; ++k4) {
            const float4 cc = sc[vi][k4];
            acc = __builtin_fmaf(cc.x, fR[(4 * k4 + 0) * MS + j], acc);
            acc = __builtin_fmaf(cc.y, fR[(4 * k4 + 1) * MS + j], acc);
            acc = __builtin_fmaf(cc.z, fR[(4 * k4 + 2) * MS + j], acc);
            acc = __builtin_fmaf(cc.w, fR[(4 * k4 + 3) * MS + j], acc);
        }
        const float kh = tq::bf16_to_f32(tq::f32_to_bf16(acc * tq::f16_to_f32(n16)));
        const float r = xj - kh;
        fu[j] = r;  // u was last read by the rotation, before the barrier above
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
        // ---- sign_i = (fma chain d of rhat_d S[i][d]) >= 0, i = j; a wave holds 64 of them
        float p = 0.0f;
        const float4* si = sS + j * (MS / 4);
#pragma unroll
        for (int d4 = 0; d4 < D / 4; ++d4) {
            const float4 hh = sx[vi][d4], ww = si[d4];
            p = __builtin_fmaf(hh.x, ww.x, p);
            p = __builtin_fmaf(hh.y, ww.y, p);
            p = __builtin_fmaf(hh.z, ww.z, p);
            p = __builtin_fmaf(hh.w, ww.w, p);
        }
        const uint64_t sb = __builtin_amdgcn_ballot_w64(p >= 0.0f);  // bit l: index 64 (j / 64) + l
        if (active && (j & 63) == 0)
            reinterpret_cast<uint2*>(signs + slot * (D / 8))[j >> 6] = make_uint2((uint32_t)sb, (uint32_t)(sb >> 32));
    }
}

// ------------------------------------------------------------------ matrix-core encoder
// The same encoder with its three D x D matrix-vector products on the fp32 matrix cores:
// v_mfma_f32_16x16x4_f32 adds the four products of its k = 0..3 to the accumulator one
// after another, each with one rounding (an fma chain in k order), so a chain of 32 of them
// over k-steps s = 0..31 covering d = 4s + k is the fma chain d = 0..127 above, bit for bit,
// denormals and signed zeros included.  The norms come out of the same instruction: with
// both operands equal to the tile of vectors, the diagonal of the 16 x 16 product is each
// vector's own fma chain of x_d * x_d.
//
// A wave encodes a tile of 16 vectors at a time.  Lane l = 16 g + v (v = l % 16, g = l / 16)
// holds element 4s + g of vector v for s = 0..31: that is the B operand (k = g, column v) of
// every product, and a product's accumulator comes back to the lanes of its column v, so a
// vector never leaves its four lanes.  The matrices are the A operands, read from an LDS
// image laid out per (16-row tile t, k-step block sb): 64 lanes x 4 consecutive k-steps, one
// 16-byte read per lane per block, lane slots xor-swizzled (slot = l ^ (l >> 4)) so that
// the transposed 4-byte reads of the Q_prod residual stage are bank-conflict free as well.
//
// Which output index a row m = 4q + i of tile t computes is a free choice (each output is
// its own chain); it sets which lane ends up holding it:
//   CONTIG  (Q_mse codes, QJL signs): index 32q + 4t + i -> lane g holds [32g, 32g + 32),
//           packed and stored by that lane directly;
//   STRIDED (Q_prod codes): index 4(4t + i) + q -> lane g holds the indices 4s + g, the
//           B-operand layout of the residual decode that consumes them; one LDS round trip
//           regroups them for packing.
constexpr int64_t MQ_MIN_VECTORS = 4096;    // below this the small-batch encoder is used
constexpr int LUT_MAX = 512;                // cells of the bucketize grid

// ---- bucketize through a uniform grid
// code(z) = #{i : b_i < z} for the NB sorted boundaries.  Cells of width w = (smallest gap
// between neighbouring boundaries) / 4 start at e0 = b_0 - 2w; cell k stores
// c0 = #{i : b_i < e0 + (k - 1) w} and b_{c0} (+inf when c0 = NB).  z goes to the cell
// k = clamp(floor((z - e0) / w), 0, cells - 1), and code(z) = c0 + [b_{c0} < z].  Exact, not
// approximate: the computed (z - e0) / w is within 1e-3 of the real quotient (both |e0| / w and
// |b_NB-1| / w are kept below 4096), so e0 + (k - 1) w < z < e0 + (k + 2) w, a window of 3w
// that holds no two boundaries (the gap is 4w).  Every b_i below the window's start is < z,
// b_{c0 + 1} >= b_{c0} + 4w is above its end, and b_{c0} decides the rest.  The two clamped
// ends: k = 0 covers z < b_0 - w and NaN (c0 = 0, [b_0 < z] false), and the last cell starts
// more than w above b_NB-1 (c0 = NB).  A boundary set without that geometry (unsorted,
// repeated, or too many cells) uses bucket_search instead.
struct BucketGrid {
    float scale, offset, top;  // f = z * scale + offset; cells = top + 1
    float w, e0;
    int cells;
    bool ok;
};
template <int NB>
__device__ __forceinline__ BucketGrid bucket_grid(const float* __restrict__ b) {
    BucketGrid g{0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0, false};
    if constexpr (NB > 1) {
        float gap = b[1] - b[0];
        bool sorted = gap > 0.0f;
#pragma unroll
        for (int i = 2; i < NB; ++i) {
            const float d = b[i] - b[i - 1];
            sorted = sorted && d > 0.0f;
            gap = fminf(gap, d);
        }
        const float w = gap * 0.25f;
        const float e0 = b[0] - 2.0f * w;
        const float span = (b[NB - 1] - e0) / w;
        g.w = w;
        g.e0 = e0;
        g.scale = 1.0f / w;
        g.offset = -e0 * g.scale;
        g.ok = sorted && w > 0.0f && span < (float)(LUT_MAX - 5) && fabsf(g.offset) < 4096.0f &&
               fabsf(b[NB - 1] * g.scale) < 4096.0f;
        g.cells = g.ok ? (int)ceilf(span) + 4 : 0;
        g.top = (float)(g.cells - 1);
    }
    return g;
}
template <int NB>
__device__ __forceinline__ void fill_bucket_grid(float2* lut, const BucketGrid& g, const float* __restrict__ b) {
    for (int k = threadIdx.x; k < g.cells; k += MQ_THREADS) {
        const float start = g.e0 + (float)(k - 1) * g.w;
        uint32_t c0 = 0;
#pragma unroll
        for (int i = 0; i < NB; ++i) c0 += b[i] < start ? 1u : 0u;
        lut[k] = make_float2(c0 < NB ? b[c0] : __builtin_inff(), __uint_as_float(c0));
    }
}
__device__ __forceinline__ uint32_t bucket_lookup(float z, const float2* lut, const BucketGrid& g) {
    float f = __builtin_fmaf(z, g.scale, g.offset);
    f = fminf(fmaxf(f, 0.0f), g.top);  // NaN -> 0
    const float2 e = lut[(uint32_t)f];
    return __float_as_uint(e.y) + (e.x < z ? 1u : 0u);
}

// LDS image of the D x D matrix M (row = output index, column = d) for A-operand reads.
template <bool STRIDED>
__device__ __forceinline__ void build_image(float* img, const float* __restrict__ M) {
    for (int idx = threadIdx.x; idx < D * D / 4; idx += MQ_THREADS) {
        const int row = idx >> 5, s = idx & 31;  // columns 4s .. 4s + 3
        const float4 val = reinterpret_cast<const float4*>(M)[idx];
        int t, q, i;
        if (STRIDED) {
            t = row >> 4, i = (row >> 2) & 3, q = row & 3;
        } else {
            q = row >> 5, t = (row >> 2) & 7, i = row & 3;
        }
        const int m = 4 * q + i;
        float* blk = img + (t * 8 + (s >> 2)) * 256 + (s & 3);
        const float e[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) blk[4 * ((16 * k + m) ^ k)] = e[k];
    }
}

// The 16 diagonal entries of a Gram accumulator (lane 16 g + v, register i holds row 4g + i,
// column v), returned to every lane of column v.
__device__ __forceinline__ float gram_diag(const f32x4& acc, int v) {
    const int r = v & 3;
    const float mine = r == 0 ? acc[0] : r == 1 ? acc[1] : r == 2 ? acc[2] : acc[3];
    return __shfl(mine, v + 16 * (v >> 2));
}

template <int BITS>
__device__ __forceinline__ void store_row(uint8_t* dst, const uint32_t* w) {
    if constexpr (BITS == 4) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    } else if constexpr (BITS == 2) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
    } else {
#pragma unroll
        for (int k = 0; k < BITS; ++k) reinterpret_cast<uint32_t*>(dst)[k] = w[k];
    }
}

template <int BITS, bool PROD>
__global__ __launch_bounds__(MQ_THREADS) void quantize_mfma_kernel(
    const uint16_t* __restrict__ x, int heads, int64_t tokens, int64_t n_vec, int64_t x_sb, int64_t x_sh,
    int64_t x_st, const float* __restrict__ R, const float* __restrict__ centers,
    const float* __restrict__ boundaries, const float* __restrict__ S, uint8_t* __restrict__ codes,
    uint16_t* __restrict__ norms, uint8_t* __restrict__ signs, uint16_t* __restrict__ rnorms, int64_t out_cap,
    int64_t out_offset, FastDiv tok_div, FastDiv head_div) {
    __shared__ float4 s_img[(PROD ? 2 : 1) * D * D / 4];                // R image (+ S image)
    __shared__ uint32_t s_stage[PROD ? MQ_WAVES * 16 * 4 * 8 : 1];      // Q_prod code regrouping
    __shared__ float s_cent[PROD ? (1 << BITS) : 1];
    constexpr int NB = (1 << BITS) - 1;
    __shared__ float2 s_lut[NB > 1 ? LUT_MAX : 1];
    const BucketGrid grid = bucket_grid<NB>(boundaries);
    const bool use_grid = __builtin_amdgcn_readfirstlane(grid.ok ? 1 : 0) != 0;
    if (NB > 1 && use_grid) fill_bucket_grid<NB>(s_lut, grid, boundaries);
    float* img = reinterpret_cast<float*>(s_img);
    build_image<PROD>(img, R);
    if constexpr (PROD) {
        build_image<false>(img + D * D, S);
        if (threadIdx.x < (1 << BITS)) s_cent[threadIdx.x] = centers[threadIdx.x];
    }
    __syncthreads();  // the only barrier: each wave then works on its own tiles

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int v = lane & 15, g = lane >> 4;
    // v_perm_b32 selector: bf16 element g of a 4-element group -> high half of an fp32
    const uint32_t sel = ((2u * g + 1u) << 24) | ((2u * g) << 16) | 0x0c0cu;
    const float4* a_rot = s_img + (lane ^ g);
    constexpr int ROW = D * BITS / 8;
    const int64_t n_tiles = (n_vec + 15) / 16;

    for (int64_t tile = (int64_t)blockIdx.x * MQ_WAVES + wave; tile < n_tiles;
         tile += (int64_t)gridDim.x * MQ_WAVES) {
        const uint32_t vi = (uint32_t)tile * 16u + (uint32_t)v;  // n_vec < 2^31
        const bool live = vi < (uint64_t)n_vec;
        int64_t slot = 0;
        float xs[32];  // xs[s] = x[v][4s + g]
        {
            uint4 w[16];
            if (live) {
                const uint32_t gh = fdiv(vi, tok_div), t = vi - gh * (uint32_t)tokens;
                const uint32_t b = fdiv(gh, head_div), h = gh - b * (uint32_t)heads;
                slot = (int64_t)gh * out_cap + out_offset + t;
                const uint4* x4 =
                    reinterpret_cast<const uint4*>(x + (int64_t)b * x_sb + (int64_t)h * x_sh + (int64_t)t * x_st);
#pragma unroll
                for (int c = 0; c < 16; ++c) w[c] = x4[c];
            } else {
#pragma unroll
                for (int c = 0; c < 16; ++c) w[c] = make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                xs[2 * c] = __uint_as_float(__builtin_amdgcn_perm(w[c].y, w[c].x, sel));
                xs[2 * c + 1] = __uint_as_float(__builtin_amdgcn_perm(w[c].w, w[c].z, sel));
            }
        }
        // ---- norm: Gram diagonal; u = x / n
        f32x4 gacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 32; ++s) gacc = mfma_f32(xs[s], xs[s], gacc);
        float n = tq::sqrt_rn(gram_diag(gacc, v));
        if (!(n > 0.0f)) n = 1.0f;
        float u[32];
#pragma unroll
        for (int s = 0; s < 32; ++s) u[s] = tq::div_rn(xs[s], n);
        const uint32_t n16 = tq::f32_to_f16(n);
        if (live && g == 0) norms[slot] = (uint16_t)n16;
        // Q_prod: the input elements again at the residual, held as bf16 pairs meanwhile
        uint32_t xp[PROD ? 16 : 1];
        if constexpr (PROD) {
#pragma unroll
            for (int c = 0; c < 16; ++c)
                xp[c] = __builtin_amdgcn_perm(__float_as_uint(xs[2 * c + 1]), __float_as_uint(xs[2 * c]), 0x07060302u);
        }

        // ---- rotation and codes
        f32x4 acc[8];
        image_products(a_rot, u, acc);
        uint32_t out[BITS];
        BitWriter bw;
        auto code_of = [&](float z, auto grid_path) -> uint32_t {
            if constexpr (NB == 1) return boundaries[0] < z ? 1u : 0u;
            else if constexpr (decltype(grid_path)::value) return bucket_lookup(z, s_lut, grid);
            else return bucket_search<BITS>(z, boundaries);
        };
        if constexpr (!PROD) {
            auto pack = [&](auto grid_path) {
#pragma unroll
                for (int t = 0; t < 8; ++t)
#pragma unroll
                    for (int i = 0; i < 4; ++i) bw.put(code_of(acc[t][i], grid_path), BITS, out);
            };
            if (use_grid) pack(std::true_type{});
            else pack(std::false_type{});
            if (live) store_row<BITS>(codes + slot * ROW + 4 * BITS * g, out);
        } else {
            // codes of indices 4s + g; regroup through LDS into [32g, 32g + 32) for packing
            uint32_t cw[8];
            float cv[32];  // C[code] of index 4s + g: the residual decode's B operand
#pragma unroll
            for (int k = 0; k < 8; ++k) cw[k] = 0u;
            auto codes_of = [&](auto grid_path) {
#pragma unroll
                for (int t = 0; t < 8; ++t)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int s = 4 * t + i;
                        const uint32_t c = code_of(acc[t][i], grid_path);
                        cw[s >> 2] |= c << (8 * (s & 3));
                        cv[s] = s_cent[c];
                    }
            };
            if (use_grid) codes_of(std::true_type{});
            else codes_of(std::false_type{});
            uint32_t* stg = s_stage + wave * (16 * 4 * 8);
            uint4* st4 = reinterpret_cast<uint4*>(stg + (v * 4 + g) * 8);
            st4[0] = make_uint4(cw[0], cw[1], cw[2], cw[3]);
            st4[1] = make_uint4(cw[4], cw[5], cw[6], cw[7]);
            // the wave's LDS accesses complete in issue order; keep the compiler from moving
            // the reads above the writes (or the next tile's writes above these reads)
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            uint2 rd[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) rd[q] = reinterpret_cast<const uint2*>(stg + (v * 4 + q) * 8)[g];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int a = 0; a < 8; ++a)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t wd = a < 4 ? rd[q].x : rd[q].y;
                    bw.put((wd >> (8 * (a & 3))) & 0xFFu, BITS, out);
                }
            if (live) store_row<BITS>(codes + slot * ROW + 4 * BITS * g, out);

            // ---- residual decode khat = C[code] @ R: A = R transposed, read from the STRIDED
            // image 4 bytes at a time; output row 4g + i of tile t is dim 4(4t + i) + g
            const int qv = v >> 2, iv = v & 3;
            int off[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) off[c] = 4 * (16 * qv + 4 * g + (c ^ qv)) + iv;
            f32x4 kacc[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) kacc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            // k-step block sb covers s' = 4 sb + e; its 32 A values are read one block ahead
            float ka[8][4], kn[8][4];
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) ka[t][e] = img[t * 256 + off[e]];
#pragma unroll
            for (int sb = 0; sb < 8; ++sb) {
                if (sb + 1 < 8) {
#pragma unroll
                    for (int t = 0; t < 8; ++t)
#pragma unroll
                        for (int e = 0; e < 4; ++e) kn[t][e] = img[((sb + 1) * 8 + t) * 256 + off[e]];
                }
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int t = 0; t < 8; ++t) kacc[t] = mfma_f32(ka[t][e], cv[4 * sb + e], kacc[t]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int t = 0; t < 8; ++t)
#pragma unroll
                    for (int e = 0; e < 4; ++e) ka[t][e] = kn[t][e];
            }
            const float nf = tq::f16_to_f32(n16);
            float r[32];
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int s = 4 * t + i;
                    const float x = __uint_as_float((s & 1) ? (xp[s >> 1] & 0xFFFF0000u) : (xp[s >> 1] << 16));
                    r[s] = x - tq::bf16_to_f32(tq::f32_to_bf16(kacc[t][i] * nf));
                }
            f32x4 racc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 32; ++s) racc = mfma_f32(r[s], r[s], racc);
            float rho = tq::sqrt_rn(gram_diag(racc, v));
            if (!(rho > 0.0f)) rho = 1.0f;
#pragma unroll
            for (int s = 0; s < 32; ++s) r[s] = tq::div_rn(r[s], rho);
            if (live && g == 0) rnorms[slot] = (uint16_t)tq::f32_to_f16(rho);

            // ---- QJL signs of rhat @ S^T (CONTIG image): lane g holds signs [32g, 32g + 32)
            f32x4 pacc[8];
            image_products(a_rot + D * D / 4, r, pacc);
            uint32_t sb = 0u;
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) sb |= (pacc[t][i] >= 0.0f ? 1u : 0u) << (4 * t + i);
            if (live) reinterpret_cast<uint32_t*>(signs + slot * (D / 8))[g] = sb;
        }
    }
}

// ------------------------------------------------------------------- decoders
// out = bf16((C[code] @ R) * f32(norm)); with QJL (keys of Q_prod) the reference's
// correction is added in bf16: corr = bf16(((s @ S) * rnorm) * sqrt(pi/2)/D),
// out = bf16(f32(khat) + f32(corr))   (runtime/packed_qmse_cache.py:312-330, 404-435).
// Output dim d is the fma chain j = 0..127 of C[code_j] * R[j][d] (of sign_j * S[j][d] for
// the correction), the residual decode's order.  On the matrix cores these are the image
// products above with A = R^T (S^T): a CONTIG image of the transposed matrix leaves dims
// [32g, 32g + 32) of vector v in lane 16 g + v, which stores them as 64 contiguous bytes.
// The B operand is C[code] of index 4s + g; each of a vector's four lanes loads the whole
// code row and takes its own indices from it.

// cv[s] = C[code of index 4s + g] for s = 0..31.  Index 4s + g sits at bit (4s + g) BITS of the
// code row w, inside the 64-bit window that starts at word 4s BITS / 32 (its field ends within
// 16 bits of bit 4s BITS); w has one zero word past the row's end.  The word indices are
// template constants so that the row stays in registers.
template <int BITS, int... S>
__device__ __forceinline__ void centers_of(const uint32_t* w, int g, const float* cent, float* cv,
                                           std::integer_sequence<int, S...>) {
    constexpr uint32_t MASK = (1u << BITS) - 1u;
    ((cv[S] = cent[(uint32_t)(((uint64_t)w[(4 * S * BITS) >> 5] | ((uint64_t)w[((4 * S * BITS) >> 5) + 1] << 32)) >>
                               (((4 * S * BITS) & 31) + g * BITS)) &
                   MASK]),
     ...);
}

template <int BITS, bool QJL, int PARTS>
__global__ __launch_bounds__(MQ_THREADS) void dequantize_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ norms, const uint8_t* __restrict__ signs,
    const uint16_t* __restrict__ rnorms, int64_t tokens, int64_t cap, int64_t n_vec, const float* __restrict__ R,
    const float* __restrict__ centers, const float* __restrict__ S, uint16_t* __restrict__ out, FastDiv tok_div) {
    __shared__ float4 s_img[(QJL ? 2 : 1) * D * D / 4];  // R^T image (+ S^T image)
    __shared__ float s_cent[1 << BITS];
    float* img = reinterpret_cast<float*>(s_img);
    build_image_transposed(img, R);
    if constexpr (QJL) build_image_transposed(img + D * D, S);
    if (threadIdx.x < (1 << BITS)) s_cent[threadIdx.x] = centers[threadIdx.x];
    __syncthreads();  // the only barrier: each wave then works on its own tiles

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int v = lane & 15, g = lane >> 4;
    constexpr int NT = 8 / PARTS;  // row tiles (16 output dims each) per work item
    constexpr int ROW = D * BITS / 8;  // code bytes per vector
    constexpr int RW = ROW / 4;
    const int64_t n_items = (n_vec + 15) / 16 * PARTS;

    // work item = (tile of 16 vectors, part): part p computes row tiles [p NT, p NT + NT), the
    // dims 32g + [4 p NT, 4 p NT + 4 NT) of each of lane 16 g + v's vector
    for (int64_t item = (int64_t)blockIdx.x * MQ_WAVES + wave; item < n_items;
         item += (int64_t)gridDim.x * MQ_WAVES) {
        const int64_t tile = item / PARTS;
        const int t0 = (int)(item % PARTS) * NT;
        const float4* a_img = s_img + t0 * 8 * 64 + (lane ^ g);
        const uint32_t vi = (uint32_t)tile * 16u + (uint32_t)v;  // n_vec < 2^31
        const bool live = vi < (uint64_t)n_vec;
        int64_t slot = 0;
        if (live) {
            const uint32_t gh = fdiv(vi, tok_div);
            slot = (int64_t)gh * cap + (vi - gh * (uint32_t)tokens);
        }
        // the code row (a lane past the end reads slot 0's, which exists, and stores nothing),
        // one zero word past its end
        uint32_t w[RW + 1];
        {
            const uint4* c4 = reinterpret_cast<const uint4*>(codes + slot * ROW);
#pragma unroll
            for (int c = 0; c < BITS; ++c) {
                const uint4 q = c4[c];
                w[4 * c] = q.x, w[4 * c + 1] = q.y, w[4 * c + 2] = q.z, w[4 * c + 3] = q.w;
            }
            w[RW] = 0u;
        }
        float cv[32];
        centers_of<BITS>(w, g, s_cent, cv, std::make_integer_sequence<int, 32>{});
        f32x4 acc[NT];
        image_products<NT>(a_img, cv, acc);
        const float nf = live ? tq::f16_to_f32(norms[slot]) : 0.0f;
        uint32_t kh[2 * NT];  // bf16 pairs of dims 32g + 4 t0 + 2p, + 2p + 1
#pragma unroll
        for (int p = 0; p < 2 * NT; ++p)
            kh[p] = tq::f32_to_bf16(acc[p >> 1][2 * (p & 1)] * nf) |
                    (tq::f32_to_bf16(acc[p >> 1][2 * (p & 1) + 1] * nf) << 16);
        if constexpr (QJL) {
            // sign of index 4s + g: word s / 8, bit 4 (s % 8) + g of the 16-byte sign row
            uint4 sw = make_uint4(0u, 0u, 0u, 0u);
            float rn = 0.0f;
            if (live) {
                sw = reinterpret_cast<const uint4*>(signs + slot * (D / 8))[0];
                rn = tq::f16_to_f32(rnorms[slot]);
            }
            const uint32_t sws[4] = {sw.x, sw.y, sw.z, sw.w};
            float sv[32];
#pragma unroll
            for (int s = 0; s < 32; ++s) sv[s] = ((sws[s >> 3] >> (4 * (s & 7) + g)) & 1u) ? 1.0f : -1.0f;
            f32x4 pacc[NT];
            image_products<NT>(a_img + D * D / 4, sv, pacc);
            const float qs = 1.2533141373155003f / D;  // sqrt(pi/2)/D rounded to fp32
#pragma unroll
            for (int p = 0; p < 2 * NT; ++p) {
                const float c0 = tq::bf16_to_f32(tq::f32_to_bf16((pacc[p >> 1][2 * (p & 1)] * rn) * qs));
                const float c1 = tq::bf16_to_f32(tq::f32_to_bf16((pacc[p >> 1][2 * (p & 1) + 1] * rn) * qs));
                const float k0 = tq::bf16_to_f32(kh[p] & 0xFFFFu) + c0;
                const float k1 = tq::bf16_to_f32(kh[p] >> 16) + c1;
                kh[p] = tq::f32_to_bf16(k0) | (tq::f32_to_bf16(k1) << 16);
            }
        }
        if (live) {
            uint4* o4 = reinterpret_cast<uint4*>(out + (int64_t)vi * D + 32 * g + 4 * t0);
#pragma unroll
            for (int i = 0; i < NT / 2; ++i) o4[i] = make_uint4(kh[4 * i], kh[4 * i + 1], kh[4 * i + 2], kh[4 * i + 3]);
        }
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_common(const uint16_t* x, int batch, int heads, int64_t tokens, int dim, int64_t x_sb, int64_t x_sh,
                 int64_t x_st, int64_t out_cap, int64_t out_offset) {
    if (!x || batch < 0 || heads < 0 || tokens < 0 || out_offset < 0) return TQ_ERR_INVALID_ARGUMENT;
    if (out_offset + tokens > out_cap) return TQ_ERR_INVALID_ARGUMENT;
    if (dim != TQ_DIM) return TQ_ERR_UNSUPPORTED;
    if (!aligned16(x) || (x_sb % 8) || (x_sh % 8) || (x_st % 8)) return TQ_ERR_UNSUPPORTED;
    return TQ_OK;
}

// Workgroups of a matrix-core kernel that fit on the device at once (each loops over tiles,
// so more would only repeat the LDS image set-up).
template <auto KERNEL>
int64_t resident_groups() {
    static std::atomic<int64_t> cached[tq::MAX_DEVICES];
    return tq::once_per_device(cached, 256, [](int dev) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, KERNEL, MQ_THREADS, 0) != hipSuccess || per_cu < 1)
            per_cu = 1;
        return (int64_t)cus * per_cu;
    });
}

template <int BITS, bool PROD>
int launch_quantize(const QuantArgs& a, hipStream_t s) {
    if (a.n_vec >= MQ_MIN_VECTORS && a.n_vec < ((int64_t)1 << 31)) {
        const int64_t tiles = (a.n_vec + 15) / 16;
        const int64_t groups = std::min<int64_t>((tiles + MQ_WAVES - 1) / MQ_WAVES, resident_groups<quantize_mfma_kernel<BITS, PROD>>());
        hipLaunchKernelGGL((quantize_mfma_kernel<BITS, PROD>), dim3((unsigned)groups), dim3(MQ_THREADS), 0, s, a.x,
                           a.heads, a.tokens, a.n_vec, a.x_sb, a.x_sh, a.x_st, a.R, a.centers, a.boundaries, a.S,
                           a.codes, a.norms, a.signs, a.rnorms, a.out_cap, a.out_offset,
                           make_fastdiv((uint32_t)a.tokens), make_fastdiv((uint32_t)a.heads));
        TQ_CHECK_LAUNCH();
        return TQ_OK;
    }
    const int64_t blocks = (a.n_vec + AV - 1) / AV;
    if (blocks == 0) return TQ_OK;
    hipLaunchKernelGGL((append_kernel<BITS, PROD>), dim3((unsigned)blocks), dim3(AT), 0, s, a.x, a.heads,
                       a.tokens, a.n_vec, a.x_sb, a.x_sh, a.x_st, a.R, a.centers, a.boundaries, a.S, a.codes,
                       a.norms, a.signs, a.rnorms, a.out_cap, a.out_offset);
    TQ_CHECK_LAUNCH();
    return TQ_OK;
}

}  // namespace

extern "C" int tq_quantize_mse(const uint16_t* x, int batch, int heads, int64_t tokens, int dim, int64_t x_sb,
                               int64_t x_sh, int64_t x_st, int bits, const float* rotation,
                               const float* boundaries, uint8_t* codes, uint16_t* norms, int64_t out_cap,
                               int64_t out_offset, void* stream) {
    int st = check_common(x, batch, heads, tokens, dim, x_sb, x_sh, x_st, out_cap, out_offset);
    if (st != TQ_OK) return st;
    if (!rotation || !boundaries || !codes || !norms) return TQ_ERR_INVALID_ARGUMENT;
    if (!aligned16(codes) || !aligned16(rotation)) return TQ_ERR_UNSUPPORTED;
    QuantArgs a{x, heads, tokens, (int64_t)batch * heads * tokens, x_sb, x_sh, x_st, rotation, nullptr,
                boundaries, nullptr, codes, norms, nullptr, nullptr, out_cap, out_offset};
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (bits) {
        case 1: return launch_quantize<1, false>(a, s);
        case 2: return launch_quantize<2, false>(a, s);
        case 3: return launch_quantize<3, false>(a, s);
        case 4: return launch_quantize<4, false>(a, s);
        default: return TQ_ERR_INVALID_ARGUMENT;
    }
}

extern "C" int tq_quantize_prod(const uint16_t* x, int batch, int heads, int64_t tokens, int dim, int64_t x_sb,
                                int64_t x_sh, int64_t x_st, int mse_bits, const float* rotation,
                                const float* centers, const float* boundaries, const float* qjl, uint8_t* codes,
                                uint16_t* norms, uint8_t* signs, uint16_t* rnorms, int64_t out_cap,
                                int64_t out_offset, void* stream) {
    int st = check_common(x, batch, heads, tokens, dim, x_sb, x_sh, x_st, out_cap, out_offset);
    if (st != TQ_OK) return st;
    if (!rotation || !centers || !boundaries || !qjl || !codes || !norms || !signs || !rnorms)
        return TQ_ERR_INVALID_ARGUMENT;
    if (!aligned16(codes) || !aligned16(signs) || !aligned16(rotation) || !aligned16(qjl)) return TQ_ERR_UNSUPPORTED;
    QuantArgs a{x, heads, tokens, (int64_t)batch * heads * tokens, x_sb, x_sh, x_st, rotation, centers,
                boundaries, qjl, codes, norms, signs, rnorms, out_cap, out_offset};
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (mse_bits) {
        case 1: return launch_quantize<1, true>(a, s);
        case 2: return launch_quantize<2, true>(a, s);
        case 3: return launch_quantize<3, true>(a, s);
        default: return TQ_ERR_INVALID_ARGUMENT;
    }
}

namespace {

template <int BITS, bool QJL, int PARTS>
int launch_dequantize_parts(const uint8_t* codes, const uint16_t* norms, const uint8_t* signs,
                            const uint16_t* rnorms, int64_t tokens, int64_t cap, int64_t n_vec,
                            const float* rotation, const float* centers, const float* qjl, uint16_t* out,
                            hipStream_t s) {
    const int64_t items = (n_vec + 15) / 16 * PARTS;
    const int64_t wgs = std::min<int64_t>((items + MQ_WAVES - 1) / MQ_WAVES,
                                          resident_groups<dequantize_kernel<BITS, QJL, PARTS>>());
    hipLaunchKernelGGL((dequantize_kernel<BITS, QJL, PARTS>), dim3((unsigned)wgs), dim3(MQ_THREADS), 0, s, codes,
                       norms, signs, rnorms, tokens, cap, n_vec, rotation, centers, qjl, out,
                       make_fastdiv((uint32_t)tokens));
    TQ_CHECK_LAUNCH();
    return TQ_OK;
}

// A call with fewer tiles than the device holds waves splits each tile's row tiles over 2 or 4
// waves: the same chains, each wave running a half or a quarter of a tile's MFMAs.
template <int BITS, bool QJL>
int run_dequantize(const uint8_t* codes, const uint16_t* norms, const uint8_t* signs, const uint16_t* rnorms,
                   int64_t tokens, int64_t cap, int64_t n_vec, const float* rotation, const float* centers,
                   const float* qjl, uint16_t* out, hipStream_t s) {
    const int64_t tiles = (n_vec + 15) / 16;
    const int64_t waves = resident_groups<dequantize_kernel<BITS, QJL, 1>>() * MQ_WAVES;
    if (4 * tiles <= waves)
        return launch_dequantize_parts<BITS, QJL, 4>(codes, norms, signs, rnorms, tokens, cap, n_vec, rotation,
                                                     centers, qjl, out, s);
    if (2 * tiles <= waves)
        return launch_dequantize_parts<BITS, QJL, 2>(codes, norms, signs, rnorms, tokens, cap, n_vec, rotation,
                                                     centers, qjl, out, s);
    return launch_dequantize_parts<BITS, QJL, 1>(codes, norms, signs, rnorms, tokens, cap, n_vec, rotation, centers,
                                                 qjl, out, s);
}

template <bool QJL>
int launch_dequantize(const uint8_t* codes, const uint16_t* norms, const uint8_t* signs, const uint16_t* rnorms,
                      int64_t groups, int64_t tokens, int64_t cap, int dim, int bits, const float* rotation,
                      const float* centers, const float* qjl, uint16_t* out, void* stream) {
    if (!codes || !norms || !rotation || !centers || !out || groups < 0 || tokens < 0 || tokens > cap)
        return TQ_ERR_INVALID_ARGUMENT;
    if (QJL && (!signs || !rnorms || !qjl)) return TQ_ERR_INVALID_ARGUMENT;
    if (dim != TQ_DIM) return TQ_ERR_UNSUPPORTED;
    if (!aligned16(codes) || !aligned16(out) || (QJL && !aligned16(signs))) return TQ_ERR_UNSUPPORTED;
    if (bits < 1 || bits > 4) return TQ_ERR_INVALID_ARGUMENT;
    const int64_t n_vec = groups * tokens;
    if (n_vec == 0) return TQ_OK;
    if (n_vec >= ((int64_t)1 << 31)) return TQ_ERR_UNSUPPORTED;
    auto run = [&](auto b) {
        return run_dequantize<decltype(b)::value, QJL>(codes, norms, signs, rnorms, tokens, cap, n_vec, rotation,
                                                        centers, qjl, out, static_cast<hipStream_t>(stream));
    };
    switch (bits) {
        case 1: return run(std::integral_constant<int, 1>{});
        case 2: return run(std::integral_constant<int, 2>{});
        case 3: return run(std::integral_constant<int, 3>{});
        default: return run(std::integral_constant<int, 4>{});
    }
}

}  // namespace

extern "C" int tq_dequantize_mse(const uint8_t* codes, const uint16_t* norms, int64_t groups, int64_t tokens,
                                 int64_t cap, int dim, int bits, const float* rotation, const float* centers,
                                 uint16_t* out, void* stream) {
    return launch_dequantize<false>(codes, norms, nullptr, nullptr, groups, tokens, cap, dim, bits, rotation,
                                    centers, nullptr, out, stream);
}

extern "C" int tq_dequantize_prod(const uint8_t* codes, const uint16_t* norms, const uint8_t* signs,
                                  const uint16_t* rnorms, int64_t groups, int64_t tokens, int64_t cap, int dim,
                                  int mse_bits, const float* rotation, const float* centers, const float* qjl,
                                  uint16_t* out, void* stream) {
    if (mse_bits > 3) return TQ_ERR_INVALID_ARGUMENT;
    return launch_dequantize<true>(codes, norms, signs, rnorms, groups, tokens, cap, dim, mse_bits, rotation,
                                   centers, qjl, out, stream);
}
