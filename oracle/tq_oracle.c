/*
 * tq_oracle.c -- CPU restatement of the TurboQuant quantizer (TEST INFRASTRUCTURE).
 *
 * This file is the checker, never the product: only tests/, the smoke test and
 * bench.py's cpu_baseline leg may load it.  It restates the reference encoder
 *
 *   _encode_group            runtime/packed_qmse_cache.py:376-402
 *   _pack_indices            runtime/packed_qmse_cache.py:13-43
 *   _encode_keys_qjl_group   runtime/packed_qmse_cache.py:285-310
 *   _decode_group (CPU)      runtime/packed_qmse_cache.py:428-435
 *   _pack_qjl_signs          runtime/packed_qmse_cache.py:148-154
 *
 * with ONE fixed fp32 evaluation order, which the HIP quantizer reproduces
 * instruction for instruction, so GPU output is bit-identical to this file:
 *
 *   norm^2  = fma chain over d = 0..D-1 of x_d * x_d, then IEEE sqrt
 *   u_d     = x_d / n                                (IEEE divide, n==0 -> 1)
 *   z_j     = fma chain over d = 0..D-1 of u_d * R[j][d]       (z = u @ R^T)
 *   code_j  = #{ i : boundary_i < z_j }                (torch.bucketize, right=False)
 *   khat_d  = bf16_rne( (fma chain over j = 0..D-1 of C[code_j] * R[j][d]) * f32(f16(n)) )
 *   r_d     = x_d - khat_d ;  rho = sqrt(fma chain of r_d^2) (0 -> 1) ; rhat_d = r_d / rho
 *   p_i     = fma chain over d of rhat_d * S[i][d]                (p = rhat @ S^T)
 *   sign_i  = (p_i >= 0)                               (torch.sign with 0 -> +1)
 *   norms   = f16_rne(n), f16_rne(rho)
 *
 * Layout (reference runtime/packed_qmse_cache.py:13-43): code d occupies bits
 * [d*b, d*b+b) of the row's little-endian bit stream, rows padded with zero
 * bits to whole bytes.  Compile with -ffp-contract=off (the Makefile does) so
 * that the only fused operations are the explicit fmaf() calls.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define TQ_ORACLE_MAX_D 512

static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t tq_oracle_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

/* IEEE binary16 round-to-nearest-even, with overflow to inf and subnormals. */
uint16_t tq_oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? (0x200u | ((ax >> 13) & 0x3FFu)) : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) {                                  /* normal half */
        uint32_t h = ((((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13));
        uint32_t rem = ax & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t e = ax >> 23;
    int shift = 126 - (int)e; /* >= 14 for values below 2^-14 */
    if (shift > 24) return (uint16_t)sign;
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t h = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float tq_oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t u;
    if (e == 0x1Fu) {
        u = sign | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            u = sign;
        } else { /* subnormal: normalise */
            int k = -1;
            do { m <<= 1; k++; } while (!(m & 0x400u));
            u = sign | ((uint32_t)(112 - k) << 23) | ((m & 0x3FFu) << 13);
        }
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline int bucketize(float z, const float* boundaries, int n_bound) {
    int idx = 0;
    for (int i = 0; i < n_bound; ++i) idx += (boundaries[i] < z) ? 1 : 0;
    return idx;
}

static inline void put_code(uint8_t* row, int d, int bits, uint32_t code) {
    int bit = d * bits;
    for (int j = 0; j < bits; ++j, ++bit)
        if ((code >> j) & 1u) row[bit >> 3] |= (uint8_t)(1u << (bit & 7));
}

static inline uint32_t get_code(const uint8_t* row, int d, int bits) {
    uint32_t c = 0;
    int bit = d * bits;
    for (int j = 0; j < bits; ++j, ++bit) c |= (uint32_t)((row[bit >> 3] >> (bit & 7)) & 1u) << j;
    return c;
}

/* Encode one vector with Q_mse; returns the fp32 (unrounded) safe norm. */
static float encode_mse_one(const uint16_t* x, int D, int bits, const float* R, const float* boundaries,
                            uint8_t* row, uint16_t* norm_out, uint8_t* codes_tmp) {
    float xf[TQ_ORACLE_MAX_D], u[TQ_ORACLE_MAX_D];
    float ss = 0.0f;
    for (int d = 0; d < D; ++d) {
        xf[d] = bf16_to_f32(x[d]);
        ss = fmaf(xf[d], xf[d], ss);
    }
    float n = sqrtf(ss);
    if (!(n > 0.0f)) n = 1.0f;
    for (int d = 0; d < D; ++d) u[d] = xf[d] / n;
    int row_bytes = (D * bits + 7) / 8;
    memset(row, 0, (size_t)row_bytes);
    int n_bound = (1 << bits) - 1;
    for (int j = 0; j < D; ++j) {
        const float* rj = R + (size_t)j * D;
        float z = 0.0f;
        for (int d = 0; d < D; ++d) z = fmaf(u[d], rj[d], z);
        int c = bucketize(z, boundaries, n_bound);
        if (codes_tmp) codes_tmp[j] = (uint8_t)c;
        put_code(row, j, bits, (uint32_t)c);
    }
    *norm_out = tq_oracle_f32_to_f16(n);
    return n;
}

/* Q_mse encoder over n_vec contiguous vectors of D bf16 values. */
void tq_oracle_encode_mse(const uint16_t* x, int64_t n_vec, int D, int bits, const float* R,
                          const float* boundaries, uint8_t* codes, uint16_t* norms) {
    int row_bytes = (D * bits + 7) / 8;
    for (int64_t v = 0; v < n_vec; ++v)
        encode_mse_one(x + v * D, D, bits, R, boundaries, codes + v * row_bytes, norms + v, 0);
}

/* Q_mse decode of one row into bf16 (reference _decode_group CPU path, fixed order). */
static void decode_mse_one(const uint8_t* row, uint16_t norm16, int D, int bits, const float* R,
                           const float* centers, float* out_f32) {
    float acc[TQ_ORACLE_MAX_D];
    for (int d = 0; d < D; ++d) acc[d] = 0.0f;
    for (int j = 0; j < D; ++j) {
        float c = centers[get_code(row, j, bits)];
        const float* rj = R + (size_t)j * D;
        for (int d = 0; d < D; ++d) acc[d] = fmaf(c, rj[d], acc[d]);
    }
    float nf = tq_oracle_f16_to_f32(norm16);
    for (int d = 0; d < D; ++d) out_f32[d] = bf16_to_f32(tq_oracle_f32_to_bf16(acc[d] * nf));
}

void tq_oracle_decode_mse(const uint8_t* codes, const uint16_t* norms, int64_t n_vec, int D, int bits,
                          const float* R, const float* centers, uint16_t* out_bf16) {
    int row_bytes = (D * bits + 7) / 8;
    float tmp[TQ_ORACLE_MAX_D];
    for (int64_t v = 0; v < n_vec; ++v) {
        decode_mse_one(codes + v * row_bytes, norms[v], D, bits, R, centers, tmp);
        for (int d = 0; d < D; ++d) out_bf16[v * D + d] = tq_oracle_f32_to_bf16(tmp[d]);
    }
}

/* Q_prod key decode (reference _decode_keys_qjl_group, runtime/packed_qmse_cache.py:312-330):
 * corr_d = bf16(((fma chain over i of s_i * S[i][d]) * rho) * (float)(sqrt(pi/2)/D)),
 * out_d  = bf16(khat_d + corr_d).                                                          */
void tq_oracle_decode_prod(const uint8_t* codes, const uint16_t* norms, const uint8_t* signs,
                           const uint16_t* rnorms, int64_t n_vec, int D, int mse_bits, const float* R,
                           const float* centers, const float* S, uint16_t* out_bf16) {
    int row_bytes = (D * mse_bits + 7) / 8;
    int sign_bytes = (D + 7) / 8;
    const float qs = (float)(1.2533141373155002512078826 / (double)D);
    float kh[TQ_ORACLE_MAX_D], corr[TQ_ORACLE_MAX_D];
    for (int64_t v = 0; v < n_vec; ++v) {
        decode_mse_one(codes + v * row_bytes, norms[v], D, mse_bits, R, centers, kh);
        for (int d = 0; d < D; ++d) corr[d] = 0.0f;
        const uint8_t* srow = signs + v * sign_bytes;
        for (int i = 0; i < D; ++i) {
            float si = ((srow[i >> 3] >> (i & 7)) & 1u) ? 1.0f : -1.0f;
            for (int d = 0; d < D; ++d) corr[d] = fmaf(si, S[(size_t)i * D + d], corr[d]);
        }
        float rho = tq_oracle_f16_to_f32(rnorms[v]);
        for (int d = 0; d < D; ++d) {
            float c = bf16_to_f32(tq_oracle_f32_to_bf16((corr[d] * rho) * qs));
            out_bf16[v * D + d] = tq_oracle_f32_to_bf16(kh[d] + c);
        }
    }
}

/* Q_prod key encoder: (bits)-bit Q_mse codes + 1-bit QJL sketch of the residual. */
void tq_oracle_encode_prod(const uint16_t* x, int64_t n_vec, int D, int mse_bits, const float* R,
                           const float* centers, const float* boundaries, const float* S, uint8_t* codes,
                           uint16_t* norms, uint8_t* signs, uint16_t* rnorms) {
    int row_bytes = (D * mse_bits + 7) / 8;
    int sign_bytes = (D + 7) / 8;
    float khat[TQ_ORACLE_MAX_D], r[TQ_ORACLE_MAX_D];
    for (int64_t v = 0; v < n_vec; ++v) {
        const uint16_t* xv = x + v * D;
        uint8_t* row = codes + v * row_bytes;
        encode_mse_one(xv, D, mse_bits, R, boundaries, row, norms + v, 0);
        decode_mse_one(row, norms[v], D, mse_bits, R, centers, khat);
        float ss = 0.0f;
        for (int d = 0; d < D; ++d) {
            r[d] = bf16_to_f32(xv[d]) - khat[d];
            ss = fmaf(r[d], r[d], ss);
        }
        float rho = sqrtf(ss);
        if (!(rho > 0.0f)) rho = 1.0f;
        for (int d = 0; d < D; ++d) r[d] = r[d] / rho;
        uint8_t* srow = signs + v * sign_bytes;
        memset(srow, 0, (size_t)sign_bytes);
        for (int i = 0; i < D; ++i) {
            const float* si = S + (size_t)i * D;
            float p = 0.0f;
            for (int d = 0; d < D; ++d) p = fmaf(r[d], si[d], p);
            if (p >= 0.0f) srow[i >> 3] |= (uint8_t)(1u << (i & 7));
        }
        rnorms[v] = tq_oracle_f32_to_f16(rho);
    }
}

/* fp32 pre-images of the codes, for tie analysis: z[v][j] exactly as the encoder computes it. */
void tq_oracle_rotated(const uint16_t* x, int64_t n_vec, int D, const float* R, float* z_out) {
    float xf[TQ_ORACLE_MAX_D], u[TQ_ORACLE_MAX_D];
    for (int64_t v = 0; v < n_vec; ++v) {
        float ss = 0.0f;
        for (int d = 0; d < D; ++d) {
            xf[d] = bf16_to_f32(x[v * D + d]);
            ss = fmaf(xf[d], xf[d], ss);
        }
        float n = sqrtf(ss);
        if (!(n > 0.0f)) n = 1.0f;
        for (int d = 0; d < D; ++d) u[d] = xf[d] / n;
        for (int j = 0; j < D; ++j) {
            float z = 0.0f;
            for (int d = 0; d < D; ++d) z = fmaf(u[d], R[(size_t)j * D + d], z);
            z_out[v * D + j] = z;
        }
    }
}

/* fp16 bits of the stored norm of each vector (the encoder's norm step alone):
 * f16_rne(sqrt(fma chain of x_d^2)), 0 -> 1.  For tests over many vectors. */
void tq_oracle_norms(const uint16_t* x, int64_t n_vec, int D, uint16_t* norms_out) {
    for (int64_t v = 0; v < n_vec; ++v) {
        float ss = 0.0f;
        for (int d = 0; d < D; ++d) {
            float f = bf16_to_f32(x[v * D + d]);
            ss = fmaf(f, f, ss);
        }
        float n = sqrtf(ss);
        if (!(n > 0.0f)) n = 1.0f;
        norms_out[v] = tq_oracle_f32_to_f16(n);
    }
}

/* Bulk conversions (used by tests to pin the rounding helpers against numpy). */
void tq_oracle_f32_to_f16_array(const float* in, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = tq_oracle_f32_to_f16(in[i]);
}

void tq_oracle_f32_to_bf16_array(const float* in, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = tq_oracle_f32_to_bf16(in[i]);
}

int tq_oracle_max_dim(void) { return TQ_ORACLE_MAX_D; }
