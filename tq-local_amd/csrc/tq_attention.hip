// tq_attention.hip -- fused decode attention over the packed TurboQuant cache (gfx950).
//
// Three launches per call, all on the caller's stream:
//   1. prepare_kernel  q_rot = q @ R_k^T and q_proj = q @ S^T for every query head
//                      (reference runtime/triton_kernels.py:289, 305-306)
//   2. split_kernel    one workgroup per (sequence split, batch row, KV head): all G
//                      query heads of the GQA group share each K/V tile it reads.
//                      Key pass (lane = token): unpack codes, codebook lookup in LDS,
//                      MSE logit + QJL correction; value pass (16 lanes per token,
//                      8 dims per lane): unpack, lookup, p * |v| * C_v accumulate.
//                      Online softmax across tiles.  Writes (o[D], max, sum) partials
//                      (reference runtime/triton_kernels.py:84-198).
//   3. merge_kernel    log-sum-exp merge of the split partials, normalise, un-rotate
//                      by R_v, write fp32 and bf16 (reference :330-336, 366-368).
// The q-side rotations are uniform over a workgroup, so the key pass takes them as
// scalar (SGPR) operands straight from the workspace.

#include "tq_common.h"

namespace {

constexpr int D = TQ_DIM;
constexpr int ABLOCK = 256;       // threads of a split workgroup
constexpr int TILE = 256;         // tokens per tile (one per lane in the key pass)
constexpr int VLANES = 16;        // lanes per token in the value pass (8 dims each)
constexpr int TARGET_WGS = 1024;  // aim for >= 4 workgroups per CU on 256 CUs
constexpr float NEG_INF = -__builtin_huge_valf();

struct Ws {
    size_t qr, qp, po, pml, total;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

Ws ws_layout(int batch, int q_heads, int n_split) {
    Ws w;
    const size_t bh = (size_t)batch * q_heads;
    w.qr = 0;
    w.qp = align256(w.qr + bh * D * sizeof(float));
    w.po = align256(w.qp + bh * D * sizeof(float));
    w.pml = align256(w.po + bh * (size_t)n_split * D * sizeof(float));
    w.total = align256(w.pml + bh * (size_t)n_split * 2 * sizeof(float));
    return w;
}

int choose_split(int groups, int64_t n_tokens, int64_t* tokens_per_split) {
    int64_t max_split = (n_tokens + TILE - 1) / TILE;
    int64_t want = (TARGET_WGS + groups - 1) / groups;
    int64_t n_split = want < max_split ? want : max_split;
    if (n_split < 1) n_split = 1;
    int64_t per = (n_tokens + n_split - 1) / n_split;
    per = (per + TILE - 1) / TILE * TILE;
    if (per < TILE) per = TILE;
    *tokens_per_split = per;
    return (int)((n_tokens + per - 1) / per > 0 ? (n_tokens + per - 1) / per : 1);
}

// ----------------------------------------------------------------- prepare
__global__ __launch_bounds__(D) void prepare_kernel(const uint16_t* __restrict__ q, const float* __restrict__ Rk,
                                                    const float* __restrict__ S, int has_qjl,
                                                    float* __restrict__ qr, float* __restrict__ qp) {
    __shared__ float sq[D];
    const int bh = blockIdx.x, j = threadIdx.x;
    sq[j] = tq::bf16_to_f32(q[(size_t)bh * D + j]);
    __syncthreads();
    float a = 0.0f;
    const float* rj = Rk + (size_t)j * D;
#pragma unroll 8
    for (int d = 0; d < D; ++d) a = __builtin_fmaf(sq[d], rj[d], a);
    qr[(size_t)bh * D + j] = a;
    if (has_qjl) {
        float p = 0.0f;
        const float* sj = S + (size_t)j * D;
#pragma unroll 8
        for (int d = 0; d < D; ++d) p = __builtin_fmaf(sq[d], sj[d], p);
        qp[(size_t)bh * D + j] = p;
    }
}

// ------------------------------------------------------------- reductions
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// --------------------------------------------------------------- split
template <int KB, int VB, bool QJL, int G>
__global__ __launch_bounds__(ABLOCK) void split_kernel(
    const float* __restrict__ qr, const float* __restrict__ qp, int q_heads, int kv_heads,
    const int32_t* __restrict__ seq_starts, const int32_t* __restrict__ seq_lens, int64_t n_tokens, int64_t cap,
    const uint8_t* __restrict__ kc,
    const uint16_t* __restrict__ kn, const uint8_t* __restrict__ ks, const uint16_t* __restrict__ kr,
    const uint8_t* __restrict__ vc, const uint16_t* __restrict__ vn, const float* __restrict__ Ck,
    const float* __restrict__ Cv, float scale, int64_t tokens_per_split, int n_split, float* __restrict__ part_o,
    float* __restrict__ part_ml) {
    constexpr int KROW = D * KB / 8;  // bytes per key row
    constexpr int VROW = D * VB / 8;  // bytes per value row
    constexpr int NWAVE = ABLOCK / 64;
    __shared__ float sCk[1 << KB];
    __shared__ float sCv[1 << VB];
    __shared__ float sW[TILE][G];          // p * |v| per token and head
    __shared__ float sRed[NWAVE][G];       // cross-wave reduction scratch
    __shared__ float sO[NWAVE][G][D];      // cross-wave value reduction

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, grp = blockIdx.y;
    const int b = grp / kv_heads, kvh = grp - b * kv_heads;
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

    if (tid < (1 << KB)) sCk[tid] = Ck[tid];
    if (tid < (1 << VB)) sCv[tid] = Cv[tid];

    const int bh0 = b * q_heads + kvh * G;  // first query head of the group
    const float* qrow = qr + (size_t)bh0 * D;
    const float* prow = qp + (size_t)bh0 * D;
    const size_t row0 = (size_t)grp * cap;  // first token slot of this group
    const float qjl_scale = 1.2533141373155003f / D;  // sqrt(pi/2)/D

    float m_run[G], s_lane[G], o[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m_run[h] = NEG_INF;
        s_lane[h] = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) o[h][k] = 0.0f;
    }
    __syncthreads();

    const int vslot = tid / VLANES, vpart = tid % VLANES;
    for (int64_t ts = t0; ts < t1; ts += TILE) {
        // ------------------------------------------------ key pass (lane = token)
        const int64_t t = ts + tid;
        const bool valid = t < t1;
        float logit[G];
        if (valid) {
            uint32_t kw[KROW / 4];
            const uint4* k4 = reinterpret_cast<const uint4*>(kc + (row0 + t) * KROW);
#pragma unroll
            for (int i = 0; i < KROW / 16; ++i) {
                const uint4 w = k4[i];
                kw[4 * i] = w.x; kw[4 * i + 1] = w.y; kw[4 * i + 2] = w.z; kw[4 * i + 3] = w.w;
            }
            uint32_t sw[4] = {0u, 0u, 0u, 0u};
            float rnf = 0.0f;
            if constexpr (QJL) {
                const uint4 w = *reinterpret_cast<const uint4*>(ks + (row0 + t) * (D / 8));
                sw[0] = w.x; sw[1] = w.y; sw[2] = w.z; sw[3] = w.w;
                rnf = tq::f16_to_f32(kr[row0 + t]);
            }
            const float knf = tq::f16_to_f32(kn[row0 + t]);
            float acc[G], qa[G];
#pragma unroll
            for (int h = 0; h < G; ++h) { acc[h] = 0.0f; qa[h] = 0.0f; }
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const float cv = sCk[tq::extract_bits<KB>(kw, d * KB)];
#pragma unroll
                for (int h = 0; h < G; ++h) acc[h] = __builtin_fmaf(qrow[h * D + d], cv, acc[h]);
                if constexpr (QJL) {
                    const float sg = ((sw[d >> 5] >> (d & 31)) & 1u) ? 1.0f : -1.0f;
#pragma unroll
                    for (int h = 0; h < G; ++h) qa[h] = __builtin_fmaf(prow[h * D + d], sg, qa[h]);
                }
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float l = knf * acc[h];
                if constexpr (QJL) l = __builtin_fmaf(qjl_scale * rnf, qa[h], l);
                logit[h] = l * scale;
            }
        } else {
#pragma unroll
            for (int h = 0; h < G; ++h) logit[h] = NEG_INF;
        }
        // tile max per head
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float wm = wave_max(logit[h]);
            if (lane == 0) sRed[wave][h] = wm;
        }
        __syncthreads();
        float alpha[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float tm = sRed[0][h];
#pragma unroll
            for (int w = 1; w < NWAVE; ++w) tm = fmaxf(tm, sRed[w][h]);
            const float m_new = fmaxf(m_run[h], tm);  // finite: the tile has a valid token
            alpha[h] = __expf(m_run[h] - m_new);
            m_run[h] = m_new;
        }
        const float vnf = valid ? tq::f16_to_f32(vn[row0 + t]) : 0.0f;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float p = valid ? __expf(logit[h] - m_run[h]) : 0.0f;
            s_lane[h] = __builtin_fmaf(s_lane[h], alpha[h], p);
            sW[tid][h] = p * vnf;
        }
        __syncthreads();
        // ------------------------------------------------ value pass (16 lanes / token)
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int k = 0; k < 8; ++k) o[h][k] *= alpha[h];
        const int boff = vpart * VB;  // byte offset of this lane's 8 codes
        for (int tt = vslot; tt < TILE; tt += ABLOCK / VLANES) {
            const int64_t tv = ts + tt;
            if (tv >= t1) break;
            const uint8_t* vrow = vc + (row0 + tv) * VROW;
            const uint32_t* v32 = reinterpret_cast<const uint32_t*>(vrow);
            uint64_t pair = v32[boff >> 2];
            if ((boff & 3) + VB > 4) pair |= (uint64_t)v32[(boff >> 2) + 1] << 32;
            const uint32_t bits = (uint32_t)(pair >> (8 * (boff & 3)));
            float w[G];
#pragma unroll
            for (int h = 0; h < G; ++h) w[h] = sW[tt][h];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float cv = sCv[(bits >> (k * VB)) & ((1u << VB) - 1u)];
#pragma unroll
                for (int h = 0; h < G; ++h) o[h][k] = __builtin_fmaf(w[h], cv, o[h][k]);
            }
        }
        __syncthreads();
    }

    // ---------------------------------------------------- reduce and store
    // value accumulators: lanes vpart, vpart+16, +32, +48 of a wave hold the same dims
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            float v = o[h][k];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            o[h][k] = v;
        }
    if (lane < VLANES) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int k = 0; k < 8; ++k) sO[wave][h][vpart * 8 + k] = o[h][k];
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float ws = wave_sum(s_lane[h]);
        if (lane == 0) sRed[wave][h] = ws;
    }
    __syncthreads();
    for (int i = tid; i < G * D; i += ABLOCK) {
        const int h = i / D, d = i % D;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) v += sO[w][h][d];
        part_o[((size_t)(bh0 + h) * n_split + split) * D + d] = v;
    }
    if (tid < G) {
        float st = 0.0f;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) st += sRed[w][tid];
        float mr = NEG_INF;
#pragma unroll
        for (int h = 0; h < G; ++h)
            if (h == tid) mr = m_run[h];
        part_ml[((size_t)(bh0 + tid) * n_split + split) * 2 + 0] = mr;
        part_ml[((size_t)(bh0 + tid) * n_split + split) * 2 + 1] = st;
    }
}

// ----------------------------------------------------------------- merge
__global__ __launch_bounds__(D) void merge_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                                  int n_split, const float* __restrict__ Rv,
                                                  float* __restrict__ out_f32, uint16_t* __restrict__ out_bf16,
                                                  float* __restrict__ lse_out) {
    __shared__ float so[D];
    const int bh = blockIdx.x, d = threadIdx.x;
    const float* ml = part_ml + (size_t)bh * n_split * 2;
    float M = NEG_INF;
    for (int s = 0; s < n_split; ++s) M = fmaxf(M, ml[2 * s]);
    float o = 0.0f, sum = 0.0f;
    if (M != NEG_INF) {
        for (int s = 0; s < n_split; ++s) {
            const float e = __expf(ml[2 * s] - M);
            sum = __builtin_fmaf(e, ml[2 * s + 1], sum);
            o = __builtin_fmaf(e, part_o[((size_t)bh * n_split + s) * D + d], o);
        }
        o = o / fmaxf(sum, 1e-8f);
    }
    if (lse_out && d == 0) lse_out[bh] = (M != NEG_INF) ? M + logf(sum) : NEG_INF;
    so[d] = o;
    __syncthreads();
    float a = 0.0f;
#pragma unroll 8
    for (int k = 0; k < D; ++k) a = __builtin_fmaf(so[k], Rv[(size_t)k * D + d], a);
    if (out_f32) out_f32[(size_t)bh * D + d] = a;
    if (out_bf16) out_bf16[(size_t)bh * D + d] = (uint16_t)tq::f32_to_bf16(a);
}

template <int KB, int VB, bool QJL>
int launch_split_g(int G, dim3 grid, hipStream_t s, const float* qr, const float* qp, int q_heads, int kv_heads,
                   const int32_t* seq_starts, const int32_t* seq_lens, int64_t n_tokens, int64_t cap, const uint8_t* kc, const uint16_t* kn,
                   const uint8_t* ks, const uint16_t* kr, const uint8_t* vc, const uint16_t* vn, const float* Ck,
                   const float* Cv, float scale, int64_t tps, int n_split, float* po, float* pml) {
#define TQ_SPLIT(GG)                                                                                           \
    case GG:                                                                                                   \
        hipLaunchKernelGGL((split_kernel<KB, VB, QJL, GG>), grid, dim3(ABLOCK), 0, s, qr, qp, q_heads, kv_heads, \
                           seq_starts, seq_lens, n_tokens, cap, kc, kn, ks, kr, vc, vn, Ck, Cv, scale, tps, n_split, po, pml); \
        break;
    switch (G) {
        TQ_SPLIT(1) TQ_SPLIT(2) TQ_SPLIT(3) TQ_SPLIT(4) TQ_SPLIT(5) TQ_SPLIT(6) TQ_SPLIT(7) TQ_SPLIT(8)
        default: return TQ_ERR_UNSUPPORTED;
    }
#undef TQ_SPLIT
    return TQ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" size_t tq_decode_attention_workspace_bytes(int batch, int q_heads, int kv_heads, int dim,
                                                      int64_t max_tokens) {
    if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || dim != D || max_tokens < 0) return 0;
    int64_t tps;
    const int n_split = choose_split(batch * kv_heads, max_tokens > 0 ? max_tokens : 1, &tps);
    // any n_tokens <= max_tokens yields at most this many splits
    int64_t want = (TARGET_WGS + batch * kv_heads - 1) / (batch * kv_heads);
    const int bound = (int)(want > n_split ? want : n_split);
    return ws_layout(batch, q_heads, bound).total;
}

extern "C" int tq_decode_attention(const uint16_t* q, int batch, int q_heads, int kv_heads, int dim,
                                   const int32_t* seq_starts, const int32_t* seq_lens, int64_t n_tokens, int64_t cap,
                                   const uint8_t* k_codes,
                                   const uint16_t* k_norms, const uint8_t* k_signs, const uint16_t* k_rnorms,
                                   const uint8_t* v_codes, const uint16_t* v_norms, int key_bits, int value_bits,
                                   int has_qjl, const float* key_rotation, const float* key_centers,
                                   const float* qjl, const float* value_rotation, const float* value_centers,
                                   float scale, float* out_f32, uint16_t* out_bf16, float* lse_out, void* workspace,
                                   size_t workspace_bytes, void* stream) {
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
    if ((k_codes && !aligned16(k_codes)) || (k_signs && !aligned16(k_signs)) || (v_codes && !aligned16(v_codes)))
        return TQ_ERR_UNSUPPORTED;
    const bool combo_ok = has_qjl ? (key_bits + 1 == value_bits && value_bits >= 2 && value_bits <= 4)
                                  : (key_bits == value_bits && key_bits >= 1 && key_bits <= 4);
    if (!combo_ok) return TQ_ERR_UNSUPPORTED;
    if (!workspace) return TQ_ERR_WORKSPACE;
    if (!(scale > 0.0f)) scale = 1.0f / sqrtf((float)D);

    int64_t tps;
    const int n_split = choose_split(batch * kv_heads, n_tokens > 0 ? n_tokens : 1, &tps);
    const Ws w = ws_layout(batch, q_heads, n_split);
    if (workspace_bytes < w.total) return TQ_ERR_WORKSPACE;
    char* base = static_cast<char*>(workspace);
    float* qr = reinterpret_cast<float*>(base + w.qr);
    float* qp = reinterpret_cast<float*>(base + w.qp);
    float* po = reinterpret_cast<float*>(base + w.po);
    float* pml = reinterpret_cast<float*>(base + w.pml);
    hipStream_t s = static_cast<hipStream_t>(stream);

    hipLaunchKernelGGL(prepare_kernel, dim3(batch * q_heads), dim3(D), 0, s, q, key_rotation, qjl, has_qjl, qr, qp);
    TQ_CHECK_LAUNCH();
    const dim3 grid(n_split, batch * kv_heads);
    int st;
    if (has_qjl) {
        switch (value_bits) {
            case 2: st = launch_split_g<1, 2, true>(G, grid, s, qr, qp, q_heads, kv_heads, seq_starts, seq_lens, n_tokens, cap, k_codes, k_norms, k_signs, k_rnorms, v_codes, v_norms, key_centers, value_centers, scale, tps, n_split, po, pml); break;
            case 3: st = launch_split_g<2, 3, true>(G, grid, s, qr, qp, q_heads, kv_heads, seq_starts, seq_lens, n_tokens, cap, k_codes, k_norms, k_signs, k_rnorms, v_codes, v_norms, key_centers, value_centers, scale, tps, n_split, po, pml); break;
            default: st = launch_split_g<3, 4, true>(G, grid, s, qr, qp, q_heads, kv_heads, seq_starts, seq_lens, n_tokens, cap, k_codes, k_norms, k_signs, k_rnorms, v_codes, v_norms, key_centers, value_centers, scale, tps, n_split, po, pml); break;
        }
    } else {
        switch (value_bits) {
            case 1: st = launch_split_g<1, 1, false>(G, grid, s, qr, qp, q_heads, kv_heads, seq_starts, seq_lens, n_tokens, cap, k_codes, k_norms, k_signs, k_rnorms, v_codes, v_norms, key_centers, value_centers, scale, tps, n_split, po, pml); break;
            case 2: st = launch_split_g<2, 2, false>(G, grid, s, qr, qp, q_heads, kv_heads, seq_starts, seq_lens, n_tokens, cap, k_codes, k_norms, k_signs, k_rnorms, v_codes, v_norms, key_centers, value_centers, scale, tps, n_split, po, pml); break;
            case 3: st = launch_split_g<3, 3, false>(G, grid, s, qr, qp, q_heads, kv_heads, seq_starts, seq_lens, n_tokens, cap, k_codes, k_norms, k_signs, k_rnorms, v_codes, v_norms, key_centers, value_centers, scale, tps, n_split, po, pml); break;
            default: st = launch_split_g<4, 4, false>(G, grid, s, qr, qp, q_heads, kv_heads, seq_starts, seq_lens, n_tokens, cap, k_codes, k_norms, k_signs, k_rnorms, v_codes, v_norms, key_centers, value_centers, scale, tps, n_split, po, pml); break;
        }
    }
    if (st != TQ_OK) return st;
    TQ_CHECK_LAUNCH();
    hipLaunchKernelGGL(merge_kernel, dim3(batch * q_heads), dim3(D), 0, s, po, pml, n_split, value_rotation, out_f32,
                       out_bf16, lse_out);
    TQ_CHECK_LAUNCH();
    return TQ_OK;
}
