// tq_attention.hip -- fused decode attention over the packed TurboQuant cache (gfx950).
//
// Two launches per call, on the caller's stream:
//
//   split_kernel  grid (n_split, batch * kv_heads), 4 waves per workgroup.  One
//                 workgroup owns a contiguous token range of one (batch row, KV
//                 head); all G query heads of the GQA group share every K/V byte
//                 it reads (reference runtime/triton_kernels.py:84-198, which
//                 re-reads the tile once per query head).
//     prologue    q_rot = q @ R_k^T, q_proj = q @ S^T for the G heads (reference
//                 :289, 305-306); a byte-indexed QJL table
//                 T[pos][byte] = sum_{bit i of byte} q_proj[8 pos + i] (one float per
//                 head); pair tables of codebook values for K and V.
//     key pass    per 16 tokens: lane (token, 32-dim group) unpacks its codes two at
//                 a time through the K pair table and feeds them as the B operand of
//                 v_mfma_f32_4x4x1_16b_f32 (16 independent 4x4 blocks: M = 4 query
//                 heads, N = 4 tokens, K = 1 dim); A is q_rot, held in VGPRs.  The
//                 QJL term is four byte-table lookups.  Group partials are summed
//                 with DPP row rotations.
//     softmax     online, per 64-token tile, max tracked per head.
//     value pass  per 4 tokens: lane (token, 8 dims) unpacks codes through the V
//                 pair table into the B operand; A = p * |v| per head; 8 MFMA chains
//                 (one per dim of the lane's 8) accumulate sum_t w C_v[code].
//     epilogue    waves merge by log-sum-exp in LDS; one (o[D], max, sum) partial
//                 per (query head, split) is written.
//   merge_kernel  log-sum-exp merge over splits, normalise, un-rotate by R_v, write
//                 fp32 / bf16 / lse (reference :330-336, 366-368).
//
// Everything accumulates in fp32 (MFMA f32, VALU f32); no packed-fp32 VALU ops.

#include "tq_common.h"

namespace {

constexpr int D = TQ_DIM;
constexpr int NWAVE = 4;
constexpr int NT = NWAVE * 64;  // threads of a split workgroup
constexpr int MIN_WAVES_PER_SIMD = 2;
constexpr int TILE = 64;        // tokens per wave iteration
constexpr int TARGET_WGS = 512; // two resident 8-wave workgroups on each of 256 CUs
constexpr float NEG_INF = -__builtin_huge_valf();
constexpr float QJL_SCALE = 1.2533141373155003f / D;  // sqrt(pi/2) / D

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma4x4(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int DPP_ROR4 = 0x124;      // row_ror:4
constexpr int DPP_ROR8 = 0x128;      // row_ror:8

__device__ __forceinline__ float swz_xor16(float v) {  // lane ^ 16 within each half-wave
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}

// max over the 16 lanes that differ in bits {0,1,4,5} of the lane id, result uniform
__device__ __forceinline__ float max_tokens(float v) {
    v = fmaxf(v, dpp<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp<DPP_QUAD_XOR2>(v));
    v = fmaxf(v, swz_xor16(v));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    return fmaxf(a, b);
}

__device__ __forceinline__ float sel4(const f4& v, int i) {
    return i == 0 ? v[0] : (i == 1 ? v[1] : (i == 2 ? v[2] : v[3]));
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

int choose_split(int groups, int64_t n_tokens, int64_t* tokens_per_split) {
    const int64_t unit = NWAVE * TILE;
    const int64_t max_split = (n_tokens + unit - 1) / unit;
    const int64_t want = (TARGET_WGS + groups - 1) / groups;
    int64_t n_split = want < max_split ? want : max_split;
    if (n_split < 1) n_split = 1;
    int64_t per = (n_tokens + n_split - 1) / n_split;
    per = (per + unit - 1) / unit * unit;
    if (per < unit) per = unit;
    *tokens_per_split = per;
    const int64_t n = (n_tokens + per - 1) / per;
    return (int)(n > 0 ? n : 1);
}

// ------------------------------------------------------------------ split kernel
template <int KB, int VB, bool QJL, int G>
struct SplitSmem {
    static constexpr int NQ = (G + 3) / 4;
    static constexpr int NH = NQ * 4;
    // the small tables come first so their LDS offsets fit the DS immediate field
    float2 lutk[1 << (2 * KB)];        // (C_k[lo], C_k[hi]) per pair of key codes
    float2 lutv[1 << (2 * VB)];        // (C_v[lo], C_v[hi]) per pair of value codes
    f4 lutq[QJL ? NQ * 16 * 256 : 1];  // QJL byte table, 4 heads per entry
    union {
        struct {
            float q[NH][D];
            float qrot[NH][D];
            float qproj[NH][D];
        } pro;
        float w[NWAVE][TILE][NH];  // p * |v| of the current tile, per wave
        struct {
            float o[NWAVE][NH][D];
            float m[NWAVE][NH];
            float s[NWAVE][NH];
        } epi;
    } u;
};

template <int KB, int VB, bool QJL, int G>
__global__ __launch_bounds__(NT, MIN_WAVES_PER_SIMD) void split_kernel(
    const uint16_t* __restrict__ q, int q_heads, int kv_heads, const int32_t* __restrict__ seq_starts,
    const int32_t* __restrict__ seq_lens, int64_t n_tokens, int64_t cap, const uint8_t* __restrict__ kc,
    const uint16_t* __restrict__ kn, const uint8_t* __restrict__ ks, const uint16_t* __restrict__ kr,
    const uint8_t* __restrict__ vc, const uint16_t* __restrict__ vn, const float* __restrict__ Rk,
    const float* __restrict__ Ck, const float* __restrict__ S, const float* __restrict__ Cv, float scale,
    int64_t tokens_per_split, int n_split, float* __restrict__ part_o, float* __restrict__ part_ml) {
    using Smem = SplitSmem<KB, VB, QJL, G>;
    constexpr int NQ = Smem::NQ;
    constexpr int NH = Smem::NH;
    constexpr int KROW = D * KB / 8;  // bytes per key row
    constexpr int VROW = D * VB / 8;  // bytes per value row
    constexpr int KPAIR = 1 << (2 * KB);
    constexpr int VPAIR = 1 << (2 * VB);
    __shared__ Smem sm;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, grp = blockIdx.y;
    const int b = grp / kv_heads, kvh = grp - b * kv_heads;
    const int bh0 = b * q_heads + kvh * G;  // first query head of the group

    // ------------------------------------------------------------ prologue
    for (int i = tid; i < NH * D; i += NT) {
        const int h = i / D, d = i % D;
        sm.u.pro.q[h][d] = h < G ? tq::bf16_to_f32(q[(size_t)(bh0 + h) * D + d]) : 0.0f;
    }
    for (int i = tid; i < KPAIR; i += NT)
        sm.lutk[i] = make_float2(Ck[i & ((1 << KB) - 1)], Ck[i >> KB]);
    for (int i = tid; i < VPAIR; i += NT)
        sm.lutv[i] = make_float2(Cv[i & ((1 << VB) - 1)], Cv[i >> VB]);
    __syncthreads();
    {
        // thread -> output row j, heads h = hp, hp + HS, ...: q_rot[h][j] = q[h] . Rk[j], q_proj[h][j] = q[h] . S[j]
        constexpr int HS = NT / D;        // head slices (4 with 512 threads)
        constexpr int HPER = (NH + HS - 1) / HS;
        const int j = tid & (D - 1), hp = tid / D;
        float ar[HPER], ap[HPER];
#pragma unroll
        for (int i = 0; i < HPER; ++i) ar[i] = ap[i] = 0.0f;
        const float4* rr = reinterpret_cast<const float4*>(Rk + (size_t)j * D);
        const float4* sr = reinterpret_cast<const float4*>(S + (size_t)j * D);
        for (int d4 = 0; d4 < D / 4; ++d4) {
            const float4 r4 = rr[d4];
            float4 s4 = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (QJL) s4 = sr[d4];
#pragma unroll
            for (int i = 0; i < HPER; ++i) {
                if (hp + HS * i >= NH) break;
                const float* qh = sm.u.pro.q[hp + HS * i] + 4 * d4;
                ar[i] = __builtin_fmaf(qh[0], r4.x, ar[i]);
                ar[i] = __builtin_fmaf(qh[1], r4.y, ar[i]);
                ar[i] = __builtin_fmaf(qh[2], r4.z, ar[i]);
                ar[i] = __builtin_fmaf(qh[3], r4.w, ar[i]);
                if constexpr (QJL) {
                    ap[i] = __builtin_fmaf(qh[0], s4.x, ap[i]);
                    ap[i] = __builtin_fmaf(qh[1], s4.y, ap[i]);
                    ap[i] = __builtin_fmaf(qh[2], s4.z, ap[i]);
                    ap[i] = __builtin_fmaf(qh[3], s4.w, ap[i]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < HPER; ++i) {
            if (hp + HS * i >= NH) break;
            sm.u.pro.qrot[hp + HS * i][j] = ar[i];
            sm.u.pro.qproj[hp + HS * i][j] = ap[i];
        }
    }
    __syncthreads();
    if constexpr (QJL) {
        // byte table of sum_i q_proj[8 pos + i] * (bit_i ? +1 : -1), by doubling:
        // T[0] = -sum_i q_proj[8 pos + i];  T[b] = T[b - 2^k] + 2 q_proj[8 pos + k] for 2^k <= b < 2^(k+1)
        for (int i = tid; i < NQ * 16; i += NT) {
            const int qq = i / 16, pos = i % 16;
            f4 t0 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 8; ++k)
#pragma unroll
                for (int r = 0; r < 4; ++r) t0[r] -= sm.u.pro.qproj[4 * qq + r][8 * pos + k];
            sm.lutq[i * 256] = t0;
        }
        __syncthreads();
#pragma unroll 1
        for (int k = 0; k < 8; ++k) {
            const int span = 1 << k;
            for (int i = tid; i < NQ * 16 * span; i += NT) {
                const int qq = i / (16 * span), rem = i % (16 * span);
                const int pos = rem / span, bb = span + rem % span;
                const int d = 8 * pos + k;
                const f4 add = {2.0f * sm.u.pro.qproj[4 * qq + 0][d], 2.0f * sm.u.pro.qproj[4 * qq + 1][d],
                                2.0f * sm.u.pro.qproj[4 * qq + 2][d], 2.0f * sm.u.pro.qproj[4 * qq + 3][d]};
                sm.lutq[(qq * 16 + pos) * 256 + bb] = sm.lutq[(qq * 16 + pos) * 256 + bb - span] + add;
            }
            __syncthreads();
        }
    }
    // A operands of the key MFMAs: lane (ts, g, j) holds q_rot[4 qq + j][32 g + k], k < 32
    const int kg = (lane >> 2) & 3;  // 32-dim group of this lane in the key pass
    const int kj = lane & 3;         // token within the 4-token MFMA block / head row
    float qa[NQ][32];
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq)
#pragma unroll
        for (int k = 0; k < 32; ++k) qa[qq][k] = sm.u.pro.qrot[4 * qq + kj][32 * kg + k];
    __syncthreads();  // the prologue area is reused for the softmax weights

    // ---------------------------------------------------------- token range
    int64_t len = n_tokens;
    if (seq_lens) {
        const int64_t l = seq_lens[b];
        len = l < n_tokens ? (l < 0 ? 0 : l) : n_tokens;
    }
    int64_t t0 = (int64_t)split * tokens_per_split;
    const int64_t t1 = (t0 + tokens_per_split < len) ? t0 + tokens_per_split : len;
    if (seq_starts) {
        const int64_t st = seq_starts[b];
        if (st > t0) t0 = st;
    }
    const size_t row0 = (size_t)grp * cap;

    f4 m_run[NQ], dv[NQ][8];
    float s_lane[NQ];
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq) {
        m_run[qq] = f4{NEG_INF, NEG_INF, NEG_INF, NEG_INF};
        s_lane[qq] = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) dv[qq][k] = f4{0.f, 0.f, 0.f, 0.f};
    }
    const int kts = lane >> 4;         // 4-token set of this lane in the key pass
    const int vs = lane >> 4;          // token slot of this lane in the value pass
    const int vcnk = lane & 15;        // 8-dim chunk of this lane in the value pass
    const int vboff = vcnk * VB;       // byte offset of the chunk's codes in a value row
    float (*wbuf)[NH] = sm.u.w[wave];

    // Loads are software-pipelined: the key data of tile i+1 is issued before the
    // value pass of tile i, the value data of tile i before its key pass, so every
    // load has half a tile of MFMA/VALU work to arrive.  Addresses are a uniform
    // (SGPR) tile base plus a 32-bit lane offset; only the last, partial tile of a
    // range clamps token indices and masks logits.
    constexpr int VW = (VB == 3) ? 2 : 1;  // dwords per lane per value row (3-bit codes straddle)
    const int64_t step = (int64_t)NWAVE * TILE;
    const int kofs_lane = (4 * kts + kj) * KROW + kg * 4 * KB;   // bytes, within a 16-token sub-tile
    const int sofs_lane = (4 * kts + kj) * (D / 8) + 4 * kg;
    const int nofs_lane = 4 * kts + kj;                          // token, within a sub-tile
    const int vofs_lane = vs * VROW + (vboff & ~3);              // bytes, within a 4-token set
    const bool v_hi = (VW == 2) && ((vboff & 3) + VB > 4);
    uint32_t kw[4][KB], ksw[4], kn16[4], kr16[4], vn16[4];
    uint32_t vw[16][VW];
    auto load_keys = [&](int64_t tb, bool masked) {
        const uint8_t* kb = kc + (row0 + tb) * KROW;
        const uint8_t* sb = ks + (row0 + tb) * (D / 8);
        const uint16_t* nb = kn + row0 + tb;
        const uint16_t* rb = kr + row0 + tb;
        const uint16_t* vb = vn + row0 + tb;
        const int last = (int)(t1 - 1 - tb);
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            int tok = 16 * st + nofs_lane;
            if (masked) tok = tok < last ? tok : last;
            const int d = tok - nofs_lane - 16 * st;  // 0 unless clamped
            const uint32_t* k32 = reinterpret_cast<const uint32_t*>(kb + 16 * st * KROW + kofs_lane + d * KROW);
#pragma unroll
            for (int i = 0; i < KB; ++i) kw[st][i] = k32[i];
            kn16[st] = nb[tok];
            vn16[st] = vb[tok];
            if constexpr (QJL) {
                ksw[st] = *reinterpret_cast<const uint32_t*>(sb + 16 * st * (D / 8) + sofs_lane + d * (D / 8));
                kr16[st] = rb[tok];
            }
        }
    };
    auto load_values = [&](int64_t tb, bool masked) {
        const uint8_t* base = vc + (row0 + tb) * VROW;
        const int last = (int)(t1 - 1 - tb);
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            int ofs = 4 * it * VROW + vofs_lane;
            if (masked && 4 * it + vs > last) ofs = last * VROW + (vboff & ~3);
            const uint32_t* v32 = reinterpret_cast<const uint32_t*>(base + ofs);
            vw[it][0] = v32[0];
            // second dword only where the lane's 3-byte chunk straddles it (never past the row)
            if constexpr (VW == 2) vw[it][1] = v_hi ? v32[1] : 0u;
        }
    };
    auto tile = [&](int64_t tb, bool masked) {
        // ------------------------------------------------------ key pass
        f4 lg[4][NQ];
        float vnorm[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const bool valid = !masked || tb + 16 * st + nofs_lane < t1;
            const float knf = tq::f16_to_f32(kn16[st]) * scale;
            vnorm[st] = tq::f16_to_f32(vn16[st]);
            f4 acc0[NQ], acc1[NQ];
#pragma unroll
            for (int qq = 0; qq < NQ; ++qq) acc0[qq] = acc1[qq] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p = 0; p < 16; ++p) {
                const float2 c = sm.lutk[tq::extract_bits<2 * KB>(kw[st], 2 * KB * p)];
#pragma unroll
                for (int qq = 0; qq < NQ; ++qq) {
                    acc0[qq] = mfma4x4(qa[qq][2 * p], c.x, acc0[qq]);
                    acc1[qq] = mfma4x4(qa[qq][2 * p + 1], c.y, acc1[qq]);
                }
            }
            float qsc = 0.0f;
            if constexpr (QJL) qsc = (QJL_SCALE * scale) * tq::f16_to_f32(kr16[st]);
#pragma unroll
            for (int qq = 0; qq < NQ; ++qq) {
                f4 part = (acc0[qq] + acc1[qq]) * knf;
                if constexpr (QJL) {
                    const uint32_t sw = ksw[st];
                    const f4* tab = sm.lutq + (qq * 16 + 4 * kg) * 256;
                    const f4 qj = (tab[__builtin_amdgcn_ubfe(sw, 0, 8)] + tab[256 + __builtin_amdgcn_ubfe(sw, 8, 8)]) +
                                  (tab[512 + __builtin_amdgcn_ubfe(sw, 16, 8)] + tab[768 + (sw >> 24)]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) part[r] = __builtin_fmaf(qsc, qj[r], part[r]);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = part[r];
                    v += dpp<DPP_ROR4>(v);
                    v += dpp<DPP_ROR8>(v);
                    lg[st][qq][r] = valid ? v : NEG_INF;
                }
            }
        }
        if (tb + step < t1) load_keys(tb + step, tb + step + TILE > t1);
        // ------------------------------------------------------ online softmax
        f4 alpha[NQ];
        bool rescale = false;
#pragma unroll
        for (int qq = 0; qq < NQ; ++qq) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float mt = fmaxf(fmaxf(lg[0][qq][r], lg[1][qq][r]), fmaxf(lg[2][qq][r], lg[3][qq][r]));
                mt = max_tokens(mt);
                const float mn = fmaxf(m_run[qq][r], mt);  // finite: the tile has a valid token
                rescale |= m_run[qq][r] != mn;
                alpha[qq][r] = __expf(m_run[qq][r] - mn);
                m_run[qq][r] = mn;
            }
            // this lane's head in the weight table is 4 qq + kg
            const float mh = sel4(m_run[qq], kg);
            float ps = 0.0f;
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const float p = __expf(sel4(lg[st][qq], kg) - mh);  // exp(-inf) = 0 for invalid tokens
                ps += p;
                wbuf[16 * st + nofs_lane][4 * qq + kg] = (4 * qq + kg < G) ? p * vnorm[st] : 0.0f;
            }
            s_lane[qq] = rescale ? __builtin_fmaf(s_lane[qq], sel4(alpha[qq], kg), ps) : s_lane[qq] + ps;
        }
        if (rescale) {
#pragma unroll
            for (int qq = 0; qq < NQ; ++qq)
#pragma unroll
                for (int k = 0; k < 8; ++k) dv[qq][k] *= alpha[qq];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        // ------------------------------------------------------ value pass
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const int tt = 4 * it + vs;
            uint32_t bits;
            if constexpr (VW == 2) {
                bits = __builtin_amdgcn_alignbit(vw[it][1], vw[it][0], 8 * (vboff & 3));
            } else {
                bits = vw[it][0] >> (8 * (vboff & 3));
            }
            float w[NQ];
#pragma unroll
            for (int qq = 0; qq < NQ; ++qq) w[qq] = wbuf[tt][4 * qq + kj];
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) {
                const float2 c = sm.lutv[__builtin_amdgcn_ubfe(bits, 2 * VB * k2, 2 * VB)];
#pragma unroll
                for (int qq = 0; qq < NQ; ++qq) {
                    dv[qq][2 * k2] = mfma4x4(w[qq], c.x, dv[qq][2 * k2]);
                    dv[qq][2 * k2 + 1] = mfma4x4(w[qq], c.y, dv[qq][2 * k2 + 1]);
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    };
    int64_t tb = t0 + (int64_t)wave * TILE;
    if (tb < t1) load_keys(tb, tb + TILE > t1);
    for (; tb + TILE <= t1; tb += step) {  // full tiles
        load_values(tb, false);
        tile(tb, false);
    }
    if (tb < t1) {  // the partial tile (at most one per wave)
        load_values(tb, true);
        tile(tb, true);
    }

    // ------------------------------------------------------------ epilogue
    // value accumulators: lanes vcnk, +16, +32, +48 hold the same dims (token slots)
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq)
#pragma unroll
        for (int k = 0; k < 8; ++k)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = dv[qq][k][r];
                v += swz_xor16(v);
                v += __shfl_xor(v, 32);
                dv[qq][k][r] = v;
            }
    // running sums: lane holds head 4 qq + kg over its tokens; sum over (kts, kj)
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq) {
        float v = s_lane[qq];
        v += dpp<DPP_QUAD_XOR1>(v);
        v += dpp<DPP_QUAD_XOR2>(v);
        v += swz_xor16(v);
        v += __shfl_xor(v, 32);
        s_lane[qq] = v;
    }
    __syncthreads();  // weight buffers are reused for the wave merge
    if (lane < 16) {
#pragma unroll
        for (int qq = 0; qq < NQ; ++qq)
#pragma unroll
            for (int k = 0; k < 8; ++k)
#pragma unroll
                for (int r = 0; r < 4; ++r) sm.u.epi.o[wave][4 * qq + r][8 * vcnk + k] = dv[qq][k][r];
    }
    if (lane < 4) {  // lanes 0..3 have kg = 0, kj = lane
#pragma unroll
        for (int qq = 0; qq < NQ; ++qq) sm.u.epi.m[wave][4 * qq + lane] = sel4(m_run[qq], lane);
    }
    if ((lane & 3) == 0 && lane < 16) {  // lanes 0, 4, 8, 12 hold kg = 0..3
#pragma unroll
        for (int qq = 0; qq < NQ; ++qq) sm.u.epi.s[wave][4 * qq + kg] = s_lane[qq];
    }
    __syncthreads();
    for (int i = tid; i < G * D; i += NT) {
        const int h = i / D, d = i % D;
        float M = NEG_INF;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, sm.u.epi.m[w][h]);
        float o = 0.0f, s = 0.0f;
        if (M != NEG_INF) {
#pragma unroll
            for (int w = 0; w < NWAVE; ++w) {
                const float e = __expf(sm.u.epi.m[w][h] - M);
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
__global__ __launch_bounds__(D) void merge_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                                  int n_split, const float* __restrict__ Rv,
                                                  float* __restrict__ out_f32, uint16_t* __restrict__ out_bf16,
                                                  float* __restrict__ lse_out) {
    __shared__ float so[D];
    __shared__ float se[D];  // per-split weights (n_split <= D is enforced on the host)
    __shared__ float sM, sS;
    const int bh = blockIdx.x, d = threadIdx.x;
    const float* ml = part_ml + (size_t)bh * n_split * 2;
    float mv = d < n_split ? ml[2 * d] : NEG_INF;
    float M = mv;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    if (d == 0 || d == 64) se[d] = M;
    __syncthreads();
    M = fmaxf(se[0], se[64]);
    __syncthreads();
    float e = (d < n_split && M != NEG_INF) ? __expf(mv - M) : 0.0f;
    float s = d < n_split ? e * ml[2 * d + 1] : 0.0f;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    se[d] = e;
    if (d == 0) sS = s;
    __syncthreads();
    if (d == 64) sS += s;
    __syncthreads();
    const float sum = sS;
    float o = 0.0f;
    for (int k = 0; k < n_split; ++k) o = __builtin_fmaf(se[k], part_o[((size_t)bh * n_split + k) * D + d], o);
    o = (M != NEG_INF) ? o / fmaxf(sum, 1e-8f) : 0.0f;
    if (lse_out && d == 0) lse_out[bh] = (M != NEG_INF) ? M + logf(sum) : NEG_INF;
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
    int q_heads, kv_heads;
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

template <int KB, int VB, bool QJL, int G>
void launch_split(const SplitArgs& a, dim3 grid, hipStream_t s) {
    hipLaunchKernelGGL((split_kernel<KB, VB, QJL, G>), grid, dim3(NT), 0, s, a.q, a.q_heads, a.kv_heads,
                       a.seq_starts, a.seq_lens, a.n_tokens, a.cap, a.kc, a.kn, a.ks, a.kr, a.vc, a.vn, a.Rk, a.Ck,
                       a.S, a.Cv, a.scale, a.tps, a.n_split, a.po, a.pml);
}

template <int KB, int VB, bool QJL>
int launch_split_g(int G, const SplitArgs& a, dim3 grid, hipStream_t s) {
    switch (G) {
        case 1: launch_split<KB, VB, QJL, 1>(a, grid, s); break;
        case 2: launch_split<KB, VB, QJL, 2>(a, grid, s); break;
        case 3: launch_split<KB, VB, QJL, 3>(a, grid, s); break;
        case 4: launch_split<KB, VB, QJL, 4>(a, grid, s); break;
        case 5: launch_split<KB, VB, QJL, 5>(a, grid, s); break;
        case 6: launch_split<KB, VB, QJL, 6>(a, grid, s); break;
        case 7: launch_split<KB, VB, QJL, 7>(a, grid, s); break;
        case 8: launch_split<KB, VB, QJL, 8>(a, grid, s); break;
        default: return TQ_ERR_UNSUPPORTED;
    }
    return TQ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" size_t tq_decode_attention_workspace_bytes(int batch, int q_heads, int kv_heads, int dim,
                                                      int64_t max_tokens) {
    if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || dim != D || max_tokens < 0) return 0;
    // any n_tokens yields at most ceil(TARGET_WGS / groups) splits
    const int64_t groups = (int64_t)batch * kv_heads;
    const int bound = (int)((TARGET_WGS + groups - 1) / groups);
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

    int64_t tps;
    const int n_split = choose_split(batch * kv_heads, n_tokens > 0 ? n_tokens : 1, &tps);
    if (n_split > D) return TQ_ERR_UNSUPPORTED;  // merge kernel keeps one weight per thread
    const Ws w = ws_layout(batch, q_heads, n_split);
    if (workspace_bytes < w.total) return TQ_ERR_WORKSPACE;
    char* base = static_cast<char*>(workspace);
    float* po = reinterpret_cast<float*>(base + w.po);
    float* pml = reinterpret_cast<float*>(base + w.pml);
    hipStream_t s = static_cast<hipStream_t>(stream);

    SplitArgs a{q, q_heads, kv_heads, seq_starts, seq_lens, n_tokens, cap, k_codes, k_norms, k_signs, k_rnorms,
                v_codes, v_norms, key_rotation, key_centers, qjl, value_centers, scale, tps, n_split, po, pml};
    const dim3 grid(n_split, batch * kv_heads);
    int st;
    if (has_qjl) {
        switch (value_bits) {
            case 2: st = launch_split_g<1, 2, true>(G, a, grid, s); break;
            case 3: st = launch_split_g<2, 3, true>(G, a, grid, s); break;
            default: st = launch_split_g<3, 4, true>(G, a, grid, s); break;
        }
    } else {
        switch (value_bits) {
            case 1: st = launch_split_g<1, 1, false>(G, a, grid, s); break;
            case 2: st = launch_split_g<2, 2, false>(G, a, grid, s); break;
            case 3: st = launch_split_g<3, 3, false>(G, a, grid, s); break;
            default: st = launch_split_g<4, 4, false>(G, a, grid, s); break;
        }
    }
    if (st != TQ_OK) return st;
    TQ_CHECK_LAUNCH();
    hipLaunchKernelGGL(merge_kernel, dim3(batch * q_heads), dim3(D), 0, s, po, pml, n_split, value_rotation, out_f32,
                       out_bf16, lse_out);
    TQ_CHECK_LAUNCH();
    return TQ_OK;
}
