// tq_quantize.hip -- TurboQuant encoder kernels for gfx950 (prefill and decode-append).
//
// One lane owns one token vector (D = 128): the bf16 vector is held in
// VGPRs, and the rotation / QJL matrix rows are uniform across the wave, so
// every multiply-add takes its matrix operand from an SGPR (scalar loads)
// and its vector operand from a VGPR.  The fp32 evaluation order is fixed
// (see the reference restatement in the CPU oracle):
//
//   norm^2 = fma chain d=0..127 of x_d*x_d;  n = sqrt_rn;  n==0 -> 1
//   u_d    = x_d /_rn n
//   z_j    = fma chain d=0..127 of u_d*R[j][d]          (z = u @ R^T)
//   code_j = #{i : boundaries_i < z_j}                   (torch.bucketize right=False)
//   Q_prod residual:  khat_d = bf16((fma chain j=0..127 of C[code_j]*R[j][d]) * f32(f16(n)))
//                     r = x - khat;  rho = sqrt_rn(fma chain r_d^2) (0 -> 1);  rhat = r /_rn rho
//                     sign_i = (fma chain d of rhat_d*S[i][d]) >= 0
//
// Reference: runtime/packed_qmse_cache.py:376-402 (_encode_group), :285-310
// (_encode_keys_qjl_group), :404-435 (_decode_group), :13-43 (_pack_indices),
// :148-154 (_pack_qjl_signs).

#include "tq_common.h"

namespace {

constexpr int D = TQ_DIM;
constexpr int QBLOCK = 256;  // lanes (= vectors) per workgroup

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

// ---- matrix rows through SGPRs, double-buffered
// Every multiply-add takes its matrix element from an SGPR (the row is uniform across the
// wave).  Scalar loads return out of order, so a compiler-placed wait for one chunk also
// waits for any chunk issued after it; the rows are therefore streamed by hand in CH-float
// chunks through two SGPR buffers: wait for chunk k, issue chunk k + 1, compute on chunk k.
// Each wait then covers a load that was issued one chunk of compute earlier.  The kernels
// using this must not spill SGPRs (a spill copy could read a buffer before its wait).
typedef float sf16 __attribute__((ext_vector_type(16)));
template <int CH>
struct SChunk {
    sf16 a[CH / 16];
    __device__ __forceinline__ float operator[](int k) const { return a[k >> 4][k & 15]; }
};
__device__ __forceinline__ void sload(SChunk<16>& c, const float* p) {
    asm volatile("s_load_dwordx16 %0, %1, 0x0" : "=&s"(c.a[0]) : "s"(p) : "memory");
}
__device__ __forceinline__ void sload(SChunk<32>& c, const float* p) {
    asm volatile("s_load_dwordx16 %0, %2, 0x0\n\ts_load_dwordx16 %1, %2, 0x40"
                 : "=&s"(c.a[0]), "=&s"(c.a[1])
                 : "s"(p)
                 : "memory");
}
// completes every outstanding scalar load (and LDS access); c is valid afterwards
__device__ __forceinline__ void swait(SChunk<16>& c) { asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(c.a[0])); }
__device__ __forceinline__ void swait(SChunk<32>& c) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(c.a[0]), "+s"(c.a[1]));
}

// Streams the D rows of the row-major D x D matrix M (uniform pointer): chunk(d0, C) is
// called for d0 = 0, CH, 2 CH, ... with C[k] = M[j][d0 + k], then row_end(j).
template <int CH, typename ChunkFn, typename RowFn>
__device__ __forceinline__ void stream_rows(const float* M, ChunkFn&& chunk, RowFn&& row_end) {
    constexpr int NC = D / CH;  // chunks per row (even)
    SChunk<CH> A, B;
    sload(A, M);
    for (int j = 0; j < D; ++j) {
        const float* mj = M + j * D;
        const float* next = M + (j + 1 < D ? j + 1 : j) * D;  // the last row reloads itself
#pragma unroll
        for (int c = 0; c < NC; c += 2) {
            swait(A);
            sload(B, mj + (c + 1) * CH);
            chunk(c * CH, A);
            swait(B);
            sload(A, c + 2 < NC ? mj + (c + 2) * CH : next);
            chunk((c + 1) * CH, B);
        }
        row_end(j);
    }
    swait(A);  // no scalar load may still be writing registers the caller reuses
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
        float cand[1 << lvl];
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

template <int BITS, bool PROD>
__global__ __launch_bounds__(QBLOCK) void quantize_kernel(
    const uint16_t* __restrict__ x, int heads, int64_t tokens, int64_t n_vec, int64_t x_sb, int64_t x_sh,
    int64_t x_st, const float* __restrict__ R, const float* __restrict__ centers,
    const float* __restrict__ boundaries, const float* __restrict__ S, uint8_t* __restrict__ codes,
    uint16_t* __restrict__ norms, uint8_t* __restrict__ signs, uint16_t* __restrict__ rnorms, int64_t out_cap,
    int64_t out_offset) {
    __shared__ uint8_t s_code[D][QBLOCK];  // PROD only: codes of each lane, column per lane
    __shared__ float s_centers[1 << BITS];
    if (PROD && threadIdx.x < (1 << BITS)) s_centers[threadIdx.x] = centers[threadIdx.x];
    if (PROD) __syncthreads();

    const int64_t v = (int64_t)blockIdx.x * QBLOCK + threadIdx.x;
    if (v >= n_vec) return;  // no barrier below this point
    const int64_t t = v % tokens;
    const int64_t gh = v / tokens;
    const int64_t h = gh % heads;
    const int64_t b = gh / heads;
    const uint16_t* xv = x + b * x_sb + h * x_sh + t * x_st;
    const int64_t slot = gh * out_cap + out_offset + t;

    // ---- load x, norm
    const uint4* x4 = reinterpret_cast<const uint4*>(xv);
    auto unpack8 = [](const uint4& w, float* o) {
        o[0] = tq::bf16_to_f32(w.x & 0xFFFFu);
        o[1] = tq::bf16_to_f32(w.x >> 16);
        o[2] = tq::bf16_to_f32(w.y & 0xFFFFu);
        o[3] = tq::bf16_to_f32(w.y >> 16);
        o[4] = tq::bf16_to_f32(w.z & 0xFFFFu);
        o[5] = tq::bf16_to_f32(w.z >> 16);
        o[6] = tq::bf16_to_f32(w.w & 0xFFFFu);
        o[7] = tq::bf16_to_f32(w.w >> 16);
    };
    float u[D];
    float ss = 0.0f;
    if constexpr (PROD) {
        // the norm from one streamed pass over x, then x read again into u / n: the raw vector
        // and u are never live together (keeps the Q_prod kernel at three waves per SIMD)
#pragma unroll
        for (int i = 0; i < D / 8; ++i) {
            float e[8];
            unpack8(x4[i], e);
#pragma unroll
            for (int k = 0; k < 8; ++k) ss = __builtin_fmaf(e[k], e[k], ss);
        }
        __asm__ volatile("" ::: "memory");  // a second read, not a copy held from the first
    } else {
#pragma unroll
        for (int i = 0; i < D / 8; ++i) unpack8(x4[i], &u[8 * i]);
#pragma unroll
        for (int d = 0; d < D; ++d) ss = __builtin_fmaf(u[d], u[d], ss);
    }
    float n = tq::sqrt_rn(ss);
    if (!(n > 0.0f)) n = 1.0f;
    if constexpr (PROD) {
#pragma unroll
        for (int i = 0; i < D / 8; ++i) {
            unpack8(x4[i], &u[8 * i]);
#pragma unroll
            for (int k = 0; k < 8; ++k) u[8 * i + k] = tq::div_rn(u[8 * i + k], n);
        }
    } else {
#pragma unroll
        for (int d = 0; d < D; ++d) u[d] = tq::div_rn(u[d], n);
    }
    const uint32_t n16 = tq::f32_to_f16(n);
    norms[slot] = (uint16_t)n16;

    // ---- rotate, bucketize, pack
    constexpr int NB = (1 << BITS) - 1;
    constexpr int ROW = D * BITS / 8;
    uint32_t* crow = reinterpret_cast<uint32_t*>(codes + slot * ROW);
    BitWriter bw;
    if constexpr (PROD) {
        for (int j = 0; j < D; ++j) {
            const float* rj = R + j * D;
            float z = 0.0f;
#pragma unroll
            for (int d = 0; d < D; ++d) z = __builtin_fmaf(u[d], rj[d], z);
            const uint32_t c = bucket_search<BITS>(z, boundaries);
            bw.put(c, BITS, crow);
            s_code[j][threadIdx.x] = (uint8_t)c;
        }
    } else {
    float z = 0.0f;
    constexpr int CH = 32;
    stream_rows<CH>(
        R,
        [&](int d0, const SChunk<CH>& C) {
#pragma unroll
            for (int k = 0; k < CH; ++k) z = __builtin_fmaf(u[d0 + k], C[k], z);
        },
        [&](int j) {
            const uint32_t c = bucket_count<NB>(z, boundaries);
            z = 0.0f;
            bw.put(c, BITS, crow);
        });
    }

    if constexpr (PROD) {
        // ---- residual decode khat = bf16((C[code] @ R) * f32(f16(n))), accumulated row by row
        float* acc = u;  // u is dead after the rotation: one 128-register array
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int j = 0; j < D; ++j) {
            const float cj = s_centers[s_code[j][threadIdx.x]];
            const float* rj = R + j * D;
#pragma unroll
            for (int d = 0; d < D; ++d) acc[d] = __builtin_fmaf(cj, rj[d], acc[d]);
        }
        const float nf = tq::f16_to_f32(n16);
        __asm__ volatile("" ::: "memory");  // x is re-read here, not held across the loop above
        float rs = 0.0f;
#pragma unroll
        for (int i = 0; i < D / 8; ++i) {
            uint4 w = x4[i];
            uint32_t xs[8] = {w.x & 0xFFFFu, w.x >> 16, w.y & 0xFFFFu, w.y >> 16,
                              w.z & 0xFFFFu, w.z >> 16, w.w & 0xFFFFu, w.w >> 16};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int d = 8 * i + k;
                const float kh = tq::bf16_to_f32(tq::f32_to_bf16(acc[d] * nf));
                acc[d] = tq::bf16_to_f32(xs[k]) - kh;
                rs = __builtin_fmaf(acc[d], acc[d], rs);
            }
        }
        float rho = tq::sqrt_rn(rs);
        if (!(rho > 0.0f)) rho = 1.0f;
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = tq::div_rn(acc[d], rho);
        rnorms[slot] = (uint16_t)tq::f32_to_f16(rho);
        uint32_t* srow = reinterpret_cast<uint32_t*>(signs + slot * (D / 8));
        BitWriter sw;
        for (int i = 0; i < D; ++i) {
            const float* si = S + i * D;
            float p = 0.0f;
#pragma unroll
            for (int d = 0; d < D; ++d) p = __builtin_fmaf(acc[d], si[d], p);
            sw.put(p >= 0.0f ? 1u : 0u, 1, srow);
        }
    }
}

// ------------------------------------------------------------------- dequantise
// out = bf16((C[code] @ R) * f32(norm)); with QJL (keys of Q_prod) the reference's
// correction is added in bf16: corr = bf16(((s @ S) * rnorm) * sqrt(pi/2)/D),
// out = bf16(f32(khat) + f32(corr))   (runtime/packed_qmse_cache.py:312-330, 404-435).
template <int BITS, bool QJL>
__global__ __launch_bounds__(QBLOCK) void dequantize_kernel(const uint8_t* __restrict__ codes,
                                                            const uint16_t* __restrict__ norms,
                                                            const uint8_t* __restrict__ signs,
                                                            const uint16_t* __restrict__ rnorms,
                                                            int64_t tokens, int64_t cap, int64_t n_vec,
                                                            const float* __restrict__ R,
                                                            const float* __restrict__ centers,
                                                            const float* __restrict__ S,
                                                            uint16_t* __restrict__ out) {
    __shared__ float s_centers[1 << BITS];
    if (threadIdx.x < (1 << BITS)) s_centers[threadIdx.x] = centers[threadIdx.x];
    __syncthreads();
    const int64_t v = (int64_t)blockIdx.x * QBLOCK + threadIdx.x;
    if (v >= n_vec) return;
    const int64_t g = v / tokens, t = v % tokens;
    const int64_t slot = g * cap + t;
    constexpr int ROW = D * BITS / 8;
    const uint8_t* row = codes + slot * ROW;
    float acc[D];
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] = 0.0f;
    for (int j = 0; j < D; ++j) {
        const int pos = j * BITS;
        uint32_t pair = row[pos >> 3];
        if ((pos & 7) + BITS > 8) pair |= (uint32_t)row[(pos >> 3) + 1] << 8;
        const float cj = s_centers[(pair >> (pos & 7)) & ((1u << BITS) - 1u)];
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
        // the correction in two halves of D/2 dims (each dim's fma chain over i is unchanged):
        // the packed k^ and one half-width accumulator stay live instead of a full one
        const uint8_t* srow = signs + slot * (D / 8);
        const float rn = tq::f16_to_f32(rnorms[slot]);
        const float qs = 1.2533141373155003f / D;  // sqrt(pi/2)/D rounded to fp32
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float cacc[D / 2];
#pragma unroll
            for (int d = 0; d < D / 2; ++d) cacc[d] = 0.0f;
            for (int i = 0; i < D; ++i) {
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
    for (int i = 0; i < D / 8; ++i) o4[i] = make_uint4(kh[4 * i], kh[4 * i + 1], kh[4 * i + 2], kh[4 * i + 3]);
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

template <int BITS, bool PROD>
int launch_quantize(const QuantArgs& a, hipStream_t s) {
    const int64_t blocks = (a.n_vec + QBLOCK - 1) / QBLOCK;
    if (blocks == 0) return TQ_OK;
    hipLaunchKernelGGL((quantize_kernel<BITS, PROD>), dim3((unsigned)blocks), dim3(QBLOCK), 0, s, a.x, a.heads,
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
    if (!aligned16(codes)) return TQ_ERR_UNSUPPORTED;
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
    if (!aligned16(codes) || !aligned16(signs)) return TQ_ERR_UNSUPPORTED;
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

template <bool QJL>
int launch_dequantize(const uint8_t* codes, const uint16_t* norms, const uint8_t* signs, const uint16_t* rnorms,
                      int64_t groups, int64_t tokens, int64_t cap, int dim, int bits, const float* rotation,
                      const float* centers, const float* qjl, uint16_t* out, void* stream) {
    if (!codes || !norms || !rotation || !centers || !out || groups < 0 || tokens < 0 || tokens > cap)
        return TQ_ERR_INVALID_ARGUMENT;
    if (QJL && (!signs || !rnorms || !qjl)) return TQ_ERR_INVALID_ARGUMENT;
    if (dim != TQ_DIM) return TQ_ERR_UNSUPPORTED;
    if (!aligned16(codes) || !aligned16(out)) return TQ_ERR_UNSUPPORTED;
    const int64_t n_vec = groups * tokens;
    const int64_t blocks = (n_vec + QBLOCK - 1) / QBLOCK;
    if (blocks == 0) return TQ_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (bits) {
#define TQ_DQ(B)                                                                                             \
    case B:                                                                                                  \
        hipLaunchKernelGGL((dequantize_kernel<B, QJL>), dim3((unsigned)blocks), dim3(QBLOCK), 0, s, codes, norms, \
                           signs, rnorms, tokens, cap, n_vec, rotation, centers, qjl, out);                    \
        break;
        TQ_DQ(1) TQ_DQ(2) TQ_DQ(3) TQ_DQ(4)
#undef TQ_DQ
        default: return TQ_ERR_INVALID_ARGUMENT;
    }
    TQ_CHECK_LAUNCH();
    return TQ_OK;
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
