// tq_attention.hip -- fused decode attention over the packed TurboQuant cache (gfx950).
//
// Two launches per call, on the caller's stream:
//
//   split_kernel  grid (n_split, batch * kv_heads), NW waves per workgroup.  A
//                 workgroup owns a contiguous token range of one (batch row, KV
//                 head); each wave owns a contiguous sub-range and walks it in
//                 blocks of 16 tokens.  All G query heads of the GQA group share
//                 every K/V byte read (reference runtime/triton_kernels.py:84-198
//                 re-reads the tile once per query head).
//   merge_kernel  log-sum-exp merge over splits, normalise, un-rotate by R_v, write
//                 fp32 / bf16 / lse (reference :330-336, 366-368).
//
// Per 16-token block, lane l = (n = l & 15, g = l >> 4):
//
//   key score     v_mfma_f32_16x16x32_bf16, D[row][token] += A[row][k] B[k][token].
//                 A (registers, fixed for the call): rows = (query head, hi|lo part of
//                 q_rot = q R_k^T in bf16), k-slots = (dim, hi|lo part of the codebook
//                 value); B = the dequantised keys, one 8-byte LDS lookup per pair of
//                 codes returning (Ck_hi, Ck_lo) for both.  Every cross product of the
//                 two-term splits is formed, so the score carries ~2^-17 relative error
//                 against fp32 inputs (the fp32 reference rounds at 2^-24; the
//                 tolerance is 2e-3 of |out|).
//   QJL term      v_mfma_i32_16x16x64_i8 on the raw sign bits (bytes of 0/1, two VALU
//                 ops per 4 dims) against q_proj = q S^T in 32-bit fixed point split in
//                 four int8 limbs (rows = (head, limb)); exact integer accumulation.
//   softmax       online, base 2 (scores are pre-multiplied by log2 e), per head.
//   value sum     v_mfma_f32_16x16x32_bf16, D[(head, w hi|lo)][dim] += A B: A = the
//                 softmax weights p |v| split hi/lo, transposed through LDS; B = value
//                 codes dequantised by single-code LDS lookups (Cv_hi, Cv_lo) from a
//                 table small enough to be bank-conflict free.
//
// Everything accumulates in fp32 (MFMA f32 / i32 accumulators); no packed-fp32 VALU.

#include "tq_common.h"

namespace {

constexpr int D = TQ_DIM;
constexpr int NW = 8;          // waves per split workgroup
constexpr int NT = NW * 64;    // threads per split workgroup
constexpr int BLK = 16;        // tokens per block (MFMA N)
constexpr int WT_STRIDE = 20;  // dwords per row of the weight-transpose buffer (bank spread)
constexpr float NEG_INF = -__builtin_huge_valf();
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float QJL_SCALE = 1.2533141373155003f / D;  // sqrt(pi/2) / D

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_bf16(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}
__device__ __forceinline__ i32x4 mfma_i8(const u32x4& a, const u32x4& b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0,
                                                 0);
}

// bf16 (round to nearest even) of x and of the remainder x - bf16(x): x = hi + lo to ~2^-17.
__device__ __forceinline__ void split_bf16(float x, uint32_t& hi, uint32_t& lo) {
    hi = tq::f32_to_bf16(x);
    lo = tq::f32_to_bf16(x - tq::bf16_to_f32(hi));
}
__device__ __forceinline__ uint32_t pack_hilo(float x) {
    uint32_t hi, lo;
    split_bf16(x, hi, lo);
    return hi | (lo << 16);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;  // row_half_mirror (lane i <-> 7 - i within 8)
constexpr int DPP_MIRROR = 0x140;       // row_mirror (lane i <-> 15 - i within 16)

// max / sum over the 16 lanes of a row, result in every lane of the row
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp<DPP_QUAD_XOR2>(v));
    v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
    return fmaxf(v, dpp<DPP_MIRROR>(v));
}
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp<DPP_QUAD_XOR1>(v);
    v += dpp<DPP_QUAD_XOR2>(v);
    v += dpp<DPP_HALF_MIRROR>(v);
    return v + dpp<DPP_MIRROR>(v);
}

// Bits [pos, pos + N) of a little-endian word array held in registers, returned
// shifted left by S (an LDS byte offset into a table of 2^S-byte entries).  pos, N
// and S are compile-time constants after unrolling: two VALU ops per field.
template <int N, int S>
__device__ __forceinline__ uint32_t field_x(const uint32_t* w, int pos) {
    const int wi = pos >> 5, sh = pos & 31;
    constexpr uint32_t M = ((1u << N) - 1u) << S;
    if (sh + N > 32) return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh - S) & M;
    if (sh >= S) return (w[wi] >> (sh - S)) & M;
    return (w[wi] << (S - sh)) & M;
}

struct Ws {
    size_t po, pml, total;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

Ws ws_layout(int batch, int q_heads, int n_split) {
    Ws w;
    const size_t bh = (size_t)batch * q_heads;
    w.po = 0;
    w.pml = align256(w.po + bh * (size_t)n_split * D * sizeof(float));
    w.total = align256(w.pml + bh * (size_t)n_split * 2 * sizeof(float));
    return w;
}

// Upper bound on splits per group for any token count: the grid never exceeds
// MAX_RESIDENT_WGS workgroups (more would queue behind the first wave of them).
constexpr int MAX_RESIDENT_WGS = 256 * 4;

// ------------------------------------------------------------------ split kernel
// GC = 1: at most 4 query heads per KV head; row 4h + x of every MFMA belongs to
//         head h, so lane group g (lanes 16g..16g+15) holds head g everywhere.
// GC = 2: 5..8 heads; rows 2h + x, lane group g holds heads 2g and 2g + 1.
template <int GC>
struct Rows {
    static constexpr int HPL = GC;      // heads per lane group
    static constexpr int NQJ = GC;      // QJL MFMA sets (4 limbs per head in total)
    __host__ __device__ static constexpr int row(int h, int x) { return GC == 1 ? 4 * h + x : 2 * h + x; }
};

template <int KB, int VB, bool QJL, int GC>
struct Smem {
    uint2 ktab[1 << (2 * KB)];          // (Ck hi|lo of c0, Ck hi|lo of c1) per pair of key codes
    uint32_t vtab[1 << VB];             // Cv hi|lo per value code
    uint32_t wt[NW][16][WT_STRIDE];     // per-wave transpose of the softmax weights
    union {
        struct {
            float q[8][D];
            float qr[8][D];             // q R_k^T
            float qp[8][D];             // q S^T, then its fixed-point integer image
            float red[NT / 64];
        } pro;
        struct {
            float o[NW][8][D];
            float m[NW][8];
            float s[NW][8];
        } epi;
    } u;
};

template <int KB, int VB, bool QJL, int GC>
__global__ __launch_bounds__(NT) void split_kernel(
    const uint16_t* __restrict__ q, int q_heads, int kv_heads, int G, const int32_t* __restrict__ seq_starts,
    const int32_t* __restrict__ seq_lens, int64_t n_tokens, int64_t cap, const uint8_t* __restrict__ kc,
    const uint16_t* __restrict__ kn, const uint8_t* __restrict__ ks, const uint16_t* __restrict__ kr,
    const uint8_t* __restrict__ vc, const uint16_t* __restrict__ vn, const float* __restrict__ Rk,
    const float* __restrict__ Ck, const float* __restrict__ S, const float* __restrict__ Cv, float scale,
    int64_t tokens_per_split, int n_split, float* __restrict__ part_o, float* __restrict__ part_ml) {
    using Sm = Smem<KB, VB, QJL, GC>;
    using R = Rows<GC>;
    constexpr int KROW = D * KB / 8;  // bytes per key row
    constexpr int VROW = D * VB / 8;  // bytes per value row
    constexpr int VCH = 8 * VB;       // bits of one lane's 8-dim value chunk
    __shared__ Sm sm;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int split = blockIdx.x, grp = blockIdx.y;
    const int b = grp / kv_heads, kvh = grp - b * kv_heads;
    const int bh0 = b * q_heads + kvh * G;  // first query head of the group

    // ------------------------------------------------------------ prologue
    for (int i = tid; i < (1 << (2 * KB)); i += NT)
        sm.ktab[i] = make_uint2(pack_hilo(Ck[i & ((1 << KB) - 1)]), pack_hilo(Ck[i >> KB]));
    for (int i = tid; i < (1 << VB); i += NT) sm.vtab[i] = pack_hilo(Cv[i]);
    for (int i = tid; i < 8 * D; i += NT) {
        const int h = i / D, d = i % D;
        sm.u.pro.q[h][d] = h < G ? tq::bf16_to_f32(q[(size_t)(bh0 + h) * D + d]) : 0.0f;
    }
    // rows of the weight transpose that never carry a head (GC = 1: rows 4h + 2, 4h + 3)
    for (int i = tid; i < NW * 16 * WT_STRIDE; i += NT) (&sm.wt[0][0][0])[i] = 0u;
    __syncthreads();
    if (tid < 2 * D) {
        // thread -> (matrix, output dim j): q_rot[h][j] = q[h] . R_k[j], q_proj[h][j] = q[h] . S[j]
        const int j = tid & (D - 1);
        const bool proj = tid >= D;
        if (!proj || QJL) {
            const float4* row = reinterpret_cast<const float4*>((proj ? S : Rk) + (size_t)j * D);
            float acc[8];
#pragma unroll
            for (int h = 0; h < 8; ++h) acc[h] = 0.0f;
            for (int d4 = 0; d4 < D / 4; ++d4) {
                const float4 r4 = row[d4];
#pragma unroll
                for (int h = 0; h < 4 * GC; ++h) {
                    const float* qh = sm.u.pro.q[h] + 4 * d4;
                    acc[h] = __builtin_fmaf(qh[0], r4.x, acc[h]);
                    acc[h] = __builtin_fmaf(qh[1], r4.y, acc[h]);
                    acc[h] = __builtin_fmaf(qh[2], r4.z, acc[h]);
                    acc[h] = __builtin_fmaf(qh[3], r4.w, acc[h]);
                }
            }
#pragma unroll
            for (int h = 0; h < 8; ++h) (proj ? sm.u.pro.qp : sm.u.pro.qr)[h][j] = acc[h];
        }
    }
    __syncthreads();

    // fixed-point scale of q_proj: |q_proj * 2^F| <= 2^30, so four balanced int8 limbs hold it
    int F = 0;
    if constexpr (QJL) {
        float mx = 0.0f;
        for (int i = tid; i < 8 * D; i += NT) mx = fmaxf(mx, fabsf((&sm.u.pro.qp[0][0])[i]));
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        if (lane == 0) sm.u.pro.red[wave] = mx;
        __syncthreads();
        mx = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) mx = fmaxf(mx, sm.u.pro.red[w]);
        int e = 0;
        if (mx > 0.0f) (void)frexpf(mx, &e);  // mx < 2^e
        F = 30 - e;
        F = F > 100 ? 100 : F;
    }

    // A operands of the key-score MFMAs (32 VGPRs): lane (i = n, g), MFMA j, VGPR r holds
    // q_x[h][32 g + 4 j + r] twice (k-slots for the hi and lo codebook parts).
    const int h_row = GC == 1 ? n / 4 : n / 2;
    const int x_row = GC == 1 ? n % 4 : n % 2;
    const bool row_live = x_row < 2 && h_row < G;
    u32x4 qa[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            uint32_t v = 0;
            if (row_live) {
                uint32_t hi, lo;
                split_bf16(sm.u.pro.qr[h_row][32 * g + 4 * j + r], hi, lo);
                v = x_row == 0 ? hi : lo;
                v |= v << 16;
            }
            qa[j][r] = v;
        }
    // A operands of the QJL MFMAs: rows = (head, limb); MFMA jj (dims of shift 4 jj + v),
    // VGPR v, byte e <-> dim 32 g + 4 jj + v + 8 e.
    u32x4 qj[R::NQJ][2];
    float sq[R::HPL];  // sum_d q_proj_int[h][d] / 2^F for this lane's heads
#pragma unroll
    for (int i = 0; i < R::HPL; ++i) sq[i] = 0.0f;
    if constexpr (QJL) {
        const float sc = ldexpf(1.0f, F);
#pragma unroll
        for (int set = 0; set < R::NQJ; ++set) {
            const int h = GC == 1 ? n / 4 : n / 2;
            const int limb = GC == 1 ? n % 4 : 2 * set + (n % 2);
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    uint32_t word = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        int x = 0;
                        if (h < G) x = (int)rintf(sm.u.pro.qp[h][32 * g + 4 * jj + v + 8 * e] * sc);
                        // balanced base-256 digits: x = l0 + 256 l1 + 65536 l2 + 2^24 l3, l_i in [-128, 127]
                        int digit = 0;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const int l = ((x + 128) & 255) - 128;
                            if (k == limb) digit = l;
                            x = (x - l) >> 8;
                        }
                        word |= (uint32_t)(digit & 255) << (8 * e);
                    }
                    qj[set][jj][v] = word;
                }
        }
        // per-head sums of the integer images (for the +-1 form of the signs)
#pragma unroll
        for (int i = 0; i < R::HPL; ++i) {
            const int h = R::HPL * g + i;
            double acc = 0.0;
            if (h < G)
                for (int d = 0; d < D; ++d) acc += (double)rintf(sm.u.pro.qp[h][d] * sc);
            sq[i] = (float)(acc * (double)ldexpf(1.0f, -F));
        }
    }
    __syncthreads();  // the prologue area is reused by the epilogue

    // ---------------------------------------------------------- token range
    int64_t len = n_tokens;
    if (seq_lens) {
        const int64_t l = seq_lens[b];
        len = l < n_tokens ? (l < 0 ? 0 : l) : n_tokens;
    }
    int64_t start = 0;
    if (seq_starts) {
        const int64_t st = seq_starts[b];
        start = st < 0 ? 0 : st;
    }
    int64_t r0 = (int64_t)split * tokens_per_split;
    int64_t r1 = r0 + tokens_per_split;
    r0 = r0 > start ? r0 : start;
    r1 = r1 < len ? r1 : len;
    const int64_t span = r1 > r0 ? r1 - r0 : 0;
    const int64_t per_wave = ((span + NW - 1) / NW + BLK - 1) / BLK * BLK;
    const int64_t t0 = r0 + (int64_t)wave * per_wave;
    int64_t t1 = t0 + per_wave;
    t1 = t1 < r1 ? t1 : r1;
    const size_t row0 = (size_t)grp * cap;

    // per-lane softmax state (heads of this lane group) and value accumulators
    float m_run[R::HPL], s_lane[R::HPL];
#pragma unroll
    for (int i = 0; i < R::HPL; ++i) m_run[i] = NEG_INF, s_lane[i] = 0.0f;
    f32x4 acc_v[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) acc_v[m] = f32x4{0.f, 0.f, 0.f, 0.f};

    const float c_mse = scale * LOG2E;
    const float c_qjl = scale * LOG2E * QJL_SCALE;
    const float qfix = ldexpf(1.0f, 1 - F);  // 2 * 2^-F: sum_d qp s_d = 2 (sum_{bit=1} qp) - sum qp
    uint32_t(*wt)[WT_STRIDE] = sm.wt[wave];

    // value chunk of lane n: dims [8n, 8n + 8) = bits [VCH n, VCH n + VCH) of the row
    constexpr int VCH_BYTES_MAX = VROW;
    const int vbit0 = VCH * n;
    const int vdw = vbit0 >> 5;                       // first dword of the chunk
    const int vsh = vbit0 & 31;
    const bool v2 = (vsh + VCH > 32);                 // chunk straddles two dwords (VB = 3 only)
    (void)VCH_BYTES_MAX;

    struct Blk {
        uint32_t kw[KB];     // key codes of token n, dims [32 g, 32 g + 32)
        uint32_t sw;         // sign bits of token n, dims [32 g, 32 g + 32)
        uint32_t kn, kr, vn; // norms (f16 bits) of token n
        uint32_t vw[4][2];   // value codes of tokens 4 g + r, lane n's dword(s)
    };
    auto load = [&](Blk& B, int64_t tb) {
        const int64_t last = t1 - 1;
        int64_t tk = tb + n;
        tk = tk < last ? tk : last;
        const uint32_t* kp = reinterpret_cast<const uint32_t*>(kc + (row0 + tk) * KROW) + KB * g;
#pragma unroll
        for (int i = 0; i < KB; ++i) B.kw[i] = kp[i];
        if constexpr (QJL) {
            B.sw = reinterpret_cast<const uint32_t*>(ks + (row0 + tk) * (D / 8))[g];
            B.kr = kr[row0 + tk];
        } else {
            B.sw = 0u;
            B.kr = 0u;
        }
        B.kn = kn[row0 + tk];
        B.vn = vn[row0 + tk];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int64_t tv = tb + 4 * g + r;
            tv = tv < last ? tv : last;
            const uint32_t* vp = reinterpret_cast<const uint32_t*>(vc + (row0 + tv) * VROW) + vdw;
            B.vw[r][0] = vp[0];
            B.vw[r][1] = v2 ? vp[1] : 0u;  // never past the row: only straddling chunks read on
        }
    };

    auto process = [&](const Blk& B, int64_t tb) {
        // ---- key scores: 8 MFMAs over dims 32 g + 4 j + r
        f32x4 acc_k = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            u32x4 bk;
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const uint32_t off = field_x<2 * KB, 3>(B.kw, (4 * j + 2 * p) * KB);
                const uint2 e = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(sm.ktab) + off);
                bk[2 * p] = e.x;
                bk[2 * p + 1] = e.y;
            }
            acc_k = mfma_bf16(qa[j], bk, acc_k);
        }
        // ---- QJL sums
        i32x4 acc_q[R::NQJ];
        if constexpr (QJL) {
#pragma unroll
            for (int set = 0; set < R::NQJ; ++set) {
                acc_q[set] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    u32x4 bq;
#pragma unroll
                    for (int v = 0; v < 4; ++v) bq[v] = (B.sw >> (4 * jj + v)) & 0x01010101u;
                    acc_q[set] = mfma_i8(qj[set][jj], bq, acc_q[set]);
                }
            }
        }
        // ---- scores (log2 domain) of token n for this lane's heads
        const bool valid = tb + n < t1;
        const float knf = tq::f16_to_f32(B.kn) * c_mse;
        const float krf = QJL ? tq::f16_to_f32(B.kr) * c_qjl : 0.0f;
        const float vnf = tq::f16_to_f32(B.vn);
        float lg[R::HPL];
#pragma unroll
        for (int i = 0; i < R::HPL; ++i) {
            float v = knf * (acc_k[2 * i] + acc_k[2 * i + 1]);
            if constexpr (QJL) {
                float qs;
                if constexpr (GC == 1) {
                    qs = ((float)acc_q[0][0] + 256.0f * (float)acc_q[0][1]) +
                         (65536.0f * (float)acc_q[0][2] + 16777216.0f * (float)acc_q[0][3]);
                } else {
                    qs = ((float)acc_q[0][2 * i] + 256.0f * (float)acc_q[0][2 * i + 1]) +
                         (65536.0f * (float)acc_q[1][2 * i] + 16777216.0f * (float)acc_q[1][2 * i + 1]);
                }
                v = __builtin_fmaf(krf, __builtin_fmaf(qs, qfix, -sq[i]), v);
            }
            lg[i] = valid ? v : NEG_INF;
        }
        // ---- online softmax
        bool grow = false;
        float mnew[R::HPL];
#pragma unroll
        for (int i = 0; i < R::HPL; ++i) {
            mnew[i] = fmaxf(m_run[i], row_max16(lg[i]));
            grow |= mnew[i] > m_run[i];
        }
        if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
            for (int i = 0; i < R::HPL; ++i) {
                const float a = m_run[i] == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(m_run[i] - mnew[i]);
                s_lane[i] *= a;
#pragma unroll
                for (int m = 0; m < 8; ++m) {
                    acc_v[m][2 * i] *= a;
                    acc_v[m][2 * i + 1] *= a;
                }
                m_run[i] = mnew[i];
            }
        }
        uint32_t wq[R::HPL][2];
#pragma unroll
        for (int i = 0; i < R::HPL; ++i) {
            const float mu = m_run[i] == NEG_INF ? 0.0f : m_run[i];
            const float p = __builtin_amdgcn_exp2f(lg[i] - mu);
            s_lane[i] += p;
            uint32_t hi, lo;
            split_bf16(p * vnf, hi, lo);
            wq[i][0] = hi | (hi << 16);
            wq[i][1] = lo | (lo << 16);
        }
        // ---- weights -> A operand of the value MFMAs (transpose through LDS)
#pragma unroll
        for (int i = 0; i < R::HPL; ++i) {
            const int h = R::HPL * g + i;
            wt[R::row(h, 0)][n] = wq[i][0];
            wt[R::row(h, 1)][n] = wq[i][1];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const u32x4 av = *reinterpret_cast<const u32x4*>(&wt[n][4 * g]);
        // ---- value MFMAs: lane (n, g) supplies tokens 4 g + r, dim 8 n + m
        uint32_t vch[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if constexpr (VB == 3)
                vch[r] = __builtin_amdgcn_alignbit(B.vw[r][1], B.vw[r][0], vsh);
            else
                vch[r] = B.vw[r][0] >> vsh;
        }
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            u32x4 bv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t off = field_x<VB, 2>(&vch[r], VB * m);
                bv[r] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(sm.vtab) + off);
            }
            acc_v[m] = mfma_bf16(av, bv, acc_v[m]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    if (t0 < t1) {
        // two blocks in flight: while one is processed the next-but-one is loaded into
        // the register set just consumed, so the roles of A and Bq alternate without copies
        Blk A, Bq;
        int64_t tb = t0;
        load(A, tb);
        if (tb + BLK < t1) load(Bq, tb + BLK);
        while (true) {
            process(A, tb);
            tb += BLK;
            if (tb >= t1) break;
            if (tb + BLK < t1) load(A, tb + BLK);
            process(Bq, tb);
            tb += BLK;
            if (tb >= t1) break;
            if (tb + BLK < t1) load(Bq, tb + BLK);
        }
    }

    // ------------------------------------------------------------ epilogue
    float s_row[R::HPL];
#pragma unroll
    for (int i = 0; i < R::HPL; ++i) s_row[i] = row_sum16(s_lane[i]);
    // lane (n, g): dims 8 n + m of heads R::HPL g + i
#pragma unroll
    for (int i = 0; i < R::HPL; ++i) {
        const int h = R::HPL * g + i;
#pragma unroll
        for (int m = 0; m < 8; ++m) sm.u.epi.o[wave][h][8 * n + m] = acc_v[m][2 * i] + acc_v[m][2 * i + 1];
        if (n == 0) {
            sm.u.epi.m[wave][h] = m_run[i];
            sm.u.epi.s[wave][h] = s_row[i];
        }
    }
    __syncthreads();
    for (int i = tid; i < G * D; i += NT) {
        const int h = i / D, d = i % D;
        float M = NEG_INF;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, sm.u.epi.m[w][h]);
        float o = 0.0f, s = 0.0f;
        if (M != NEG_INF) {
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const float mw = sm.u.epi.m[w][h];
                const float e = mw == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
                o = __builtin_fmaf(e, sm.u.epi.o[w][h][d], o);
                s = __builtin_fmaf(e, sm.u.epi.s[w][h], s);
            }
        }
        const size_t pidx = (size_t)(bh0 + h) * n_split + split;
        part_o[pidx * D + d] = o;
        if (d == 0) {
            part_ml[pidx * 2 + 0] = M;
            part_ml[pidx * 2 + 1] = s;
        }
    }
}

// ----------------------------------------------------------------- merge
// One workgroup per (batch row, query head): merge the split partials (maxima in
// the log2 domain), normalise, un-rotate by R_v.
__global__ __launch_bounds__(D) void merge_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                                  int n_split, const float* __restrict__ Rv,
                                                  float* __restrict__ out_f32, uint16_t* __restrict__ out_bf16,
                                                  float* __restrict__ lse_out) {
    __shared__ float so[D];
    __shared__ float red[2];
    const int bh = blockIdx.x, d = threadIdx.x, lane = d & 63, wv = d >> 6;
    const float* ml = part_ml + (size_t)bh * n_split * 2;
    float M = NEG_INF;
    for (int k = d; k < n_split; k += D) M = fmaxf(M, ml[2 * k]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    if (lane == 0) red[wv] = M;
    __syncthreads();
    M = fmaxf(red[0], red[1]);
    __syncthreads();
    float o = 0.0f, s = 0.0f;
    if (M != NEG_INF) {
        for (int k = 0; k < n_split; ++k) {
            const float mk = ml[2 * k];
            const float e = mk == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mk - M);
            o = __builtin_fmaf(e, part_o[((size_t)bh * n_split + k) * D + d], o);
            s = __builtin_fmaf(e, ml[2 * k + 1], s);
        }
    }
    o = (M != NEG_INF) ? o / fmaxf(s, 1e-8f) : 0.0f;
    if (lse_out && d == 0) lse_out[bh] = (M != NEG_INF) ? M * LN2 + logf(s) : NEG_INF;
    so[d] = o;
    __syncthreads();
    float a = 0.0f;
#pragma unroll 8
    for (int k = 0; k < D; ++k) a = __builtin_fmaf(so[k], Rv[(size_t)k * D + d], a);
    if (out_f32) out_f32[(size_t)bh * D + d] = a;
    if (out_bf16) out_bf16[(size_t)bh * D + d] = (uint16_t)tq::f32_to_bf16(a);
}

struct SplitArgs {
    const uint16_t* q;
    int q_heads, kv_heads, G;
    const int32_t *seq_starts, *seq_lens;
    int64_t n_tokens, cap;
    const uint8_t* kc;
    const uint16_t* kn;
    const uint8_t* ks;
    const uint16_t* kr;
    const uint8_t* vc;
    const uint16_t* vn;
    const float *Rk, *Ck, *S, *Cv;
    float scale;
    int64_t tps;
    int n_split;
    float *po, *pml;
};

int cu_count() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 256;
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) != hipSuccess) return 256;
        cus = p.multiProcessorCount > 0 ? p.multiProcessorCount : 256;
    }
    return cus;
}

template <int KB, int VB, bool QJL, int GC>
int wgs_per_cu() {
    static int occ = 0;
    if (occ == 0) {
        int o = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, split_kernel<KB, VB, QJL, GC>, NT, 0) != hipSuccess || o < 1)
            o = 1;
        occ = o;
    }
    return occ;
}

int choose_split(int groups, int64_t n_tokens, int target_wgs, int64_t* tokens_per_split) {
    const int64_t min_per_split = (int64_t)NW * BLK * 2;  // >= two blocks per wave
    const int64_t max_split = (n_tokens + min_per_split - 1) / min_per_split;
    int64_t want = (target_wgs + groups - 1) / groups;
    const int64_t cap_split = (MAX_RESIDENT_WGS + groups - 1) / groups;
    want = want < cap_split ? want : cap_split;
    int64_t ns = want < max_split ? want : max_split;
    if (ns < 1) ns = 1;
    int64_t per = (n_tokens + ns - 1) / ns;
    per = (per + BLK - 1) / BLK * BLK;
    if (per < BLK) per = BLK;
    *tokens_per_split = per;
    const int64_t got = (n_tokens + per - 1) / per;
    return (int)(got > 0 ? got : 1);
}

template <int KB, int VB, bool QJL, int GC>
int launch_split(const SplitArgs& a, int groups, hipStream_t s, int* n_split_out, int64_t* tps_out) {
    const int target = wgs_per_cu<KB, VB, QJL, GC>() * cu_count();
    int64_t tps;
    const int ns = choose_split(groups, a.n_tokens > 0 ? a.n_tokens : 1, target, &tps);
    *n_split_out = ns;
    *tps_out = tps;
    if (a.po == nullptr) return TQ_OK;  // sizing query only
    hipLaunchKernelGGL((split_kernel<KB, VB, QJL, GC>), dim3(ns, groups), dim3(NT), 0, s, a.q, a.q_heads,
                       a.kv_heads, a.G, a.seq_starts, a.seq_lens, a.n_tokens, a.cap, a.kc, a.kn, a.ks, a.kr, a.vc,
                       a.vn, a.Rk, a.Ck, a.S, a.Cv, a.scale, tps, ns, a.po, a.pml);
    return TQ_OK;
}

template <int KB, int VB, bool QJL>
int launch_split_g(int G, const SplitArgs& a, int groups, hipStream_t s, int* ns, int64_t* tps) {
    if (G <= 4) return launch_split<KB, VB, QJL, 1>(a, groups, s, ns, tps);
    if (G <= 8) return launch_split<KB, VB, QJL, 2>(a, groups, s, ns, tps);
    return TQ_ERR_UNSUPPORTED;
}

int dispatch(int key_bits, int value_bits, int has_qjl, int G, const SplitArgs& a, int groups, hipStream_t s,
             int* ns, int64_t* tps) {
    if (has_qjl) {
        switch (value_bits) {
            case 2: return launch_split_g<1, 2, true>(G, a, groups, s, ns, tps);
            case 3: return launch_split_g<2, 3, true>(G, a, groups, s, ns, tps);
            default: return launch_split_g<3, 4, true>(G, a, groups, s, ns, tps);
        }
    }
    switch (value_bits) {
        case 1: return launch_split_g<1, 1, false>(G, a, groups, s, ns, tps);
        case 2: return launch_split_g<2, 2, false>(G, a, groups, s, ns, tps);
        case 3: return launch_split_g<3, 3, false>(G, a, groups, s, ns, tps);
        default: return launch_split_g<4, 4, false>(G, a, groups, s, ns, tps);
    }
    (void)key_bits;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" size_t tq_decode_attention_workspace_bytes(int batch, int q_heads, int kv_heads, int dim,
                                                      int64_t max_tokens) {
    if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || dim != D || max_tokens < 0) return 0;
    // any n_tokens yields at most ceil(MAX_RESIDENT_WGS / groups) splits
    const int64_t groups = (int64_t)batch * kv_heads;
    const int bound = (int)((MAX_RESIDENT_WGS + groups - 1) / groups);
    return ws_layout(batch, q_heads, bound).total;
}

extern "C" int tq_decode_attention(const uint16_t* q, int batch, int q_heads, int kv_heads, int dim,
                                   const int32_t* seq_starts, const int32_t* seq_lens, int64_t n_tokens, int64_t cap,
                                   const uint8_t* k_codes, const uint16_t* k_norms, const uint8_t* k_signs,
                                   const uint16_t* k_rnorms, const uint8_t* v_codes, const uint16_t* v_norms,
                                   int key_bits, int value_bits, int has_qjl, const float* key_rotation,
                                   const float* key_centers, const float* qjl, const float* value_rotation,
                                   const float* value_centers, float scale, float* out_f32, uint16_t* out_bf16,
                                   float* lse_out, void* workspace, size_t workspace_bytes, void* stream) {
    if (!q || batch <= 0 || q_heads <= 0 || kv_heads <= 0 || n_tokens < 0 || cap < n_tokens)
        return TQ_ERR_INVALID_ARGUMENT;
    if (dim != D) return TQ_ERR_UNSUPPORTED;
    if (q_heads % kv_heads) return TQ_ERR_INVALID_ARGUMENT;
    const int G = q_heads / kv_heads;
    if (G > TQ_MAX_GROUP) return TQ_ERR_UNSUPPORTED;
    if (!key_rotation || !key_centers || !value_rotation || !value_centers) return TQ_ERR_INVALID_ARGUMENT;
    if (!out_f32 && !out_bf16 && !lse_out) return TQ_ERR_INVALID_ARGUMENT;
    if (n_tokens > 0 && (!k_codes || !k_norms || !v_codes || !v_norms)) return TQ_ERR_INVALID_ARGUMENT;
    if (has_qjl && (!qjl || (n_tokens > 0 && (!k_signs || !k_rnorms)))) return TQ_ERR_INVALID_ARGUMENT;
    if ((k_codes && !aligned16(k_codes)) || (k_signs && !aligned16(k_signs)) || (v_codes && !aligned16(v_codes)) ||
        !aligned16(key_rotation) || (qjl && !aligned16(qjl)))
        return TQ_ERR_UNSUPPORTED;
    const bool combo_ok = has_qjl ? (key_bits + 1 == value_bits && value_bits >= 2 && value_bits <= 4)
                                  : (key_bits == value_bits && key_bits >= 1 && key_bits <= 4);
    if (!combo_ok) return TQ_ERR_UNSUPPORTED;
    if (!workspace) return TQ_ERR_WORKSPACE;
    if (!(scale > 0.0f)) scale = 1.0f / sqrtf((float)D);

    hipStream_t s = static_cast<hipStream_t>(stream);
    const int groups = batch * kv_heads;
    SplitArgs a{q, q_heads, kv_heads, G, seq_starts, seq_lens, n_tokens, cap, k_codes, k_norms, k_signs, k_rnorms,
                v_codes, v_norms, key_rotation, key_centers, qjl, value_centers, scale, 0, 0, nullptr, nullptr};
    int n_split = 0;
    int64_t tps = 0;
    int st = dispatch(key_bits, value_bits, has_qjl, G, a, groups, s, &n_split, &tps);  // sizing
    if (st != TQ_OK) return st;
    const Ws w = ws_layout(batch, q_heads, n_split);
    if (workspace_bytes < w.total) return TQ_ERR_WORKSPACE;
    char* base = static_cast<char*>(workspace);
    a.po = reinterpret_cast<float*>(base + w.po);
    a.pml = reinterpret_cast<float*>(base + w.pml);
    st = dispatch(key_bits, value_bits, has_qjl, G, a, groups, s, &n_split, &tps);
    if (st != TQ_OK) return st;
    TQ_CHECK_LAUNCH();
    hipLaunchKernelGGL(merge_kernel, dim3(batch * q_heads), dim3(D), 0, s, a.po, a.pml, n_split, value_rotation,
                       out_f32, out_bf16, lse_out);
    TQ_CHECK_LAUNCH();
    return TQ_OK;
}
