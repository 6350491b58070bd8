/*
 * tq.h -- C ABI of libtq, the MI355X (gfx950) TurboQuant hot path.
 *
 * Plain C: device pointers, sizes and a hipStream_t passed as void*.  Every
 * entry point is asynchronous on the given stream, never allocates, never
 * throws, and returns a tq_status.  All pointers are device pointers unless
 * stated otherwise.  All memory is owned by the caller.
 *
 * Data types: "bf16" and "f16" arrays are passed as uint16_t bit patterns;
 * rotations / codebooks / QJL matrices are fp32, row-major.
 *
 * Packed-cache layout (reference runtime/packed_qmse_cache.py:13-43, 58-92,
 * 121-154): for G = batch*kv_heads groups with a capacity of `cap` tokens,
 *   codes   u8  [G][cap][ceil(D*bits/8)]  code d at bits [d*bits, d*bits+bits)
 *                                         of the row's LSB-first bit stream
 *   norms   f16 [G][cap]                  fp16 RNE of the fp32 L2 norm (0 -> 1)
 *   signs   u8  [G][cap][D/8]             QJL bit i = (r_hat . S_i >= 0)
 *   rnorms  f16 [G][cap]                  fp16 RNE of the residual norm (0 -> 1)
 * With cap == N this is exactly the reference's contiguous [B,Hkv,N,row].
 */
#ifndef TQ_H_
#define TQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TQ_ABI_VERSION 1

typedef enum tq_status {
    TQ_OK = 0,
    TQ_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size, bad bit width        */
    TQ_ERR_UNSUPPORTED = 2,      /* valid but not implemented (e.g. D != 128)    */
    TQ_ERR_WORKSPACE = 3,        /* workspace missing or too small               */
    TQ_ERR_HIP = 4               /* a HIP runtime call failed (launch, ...)      */
} tq_status;

/* Version of this ABI (TQ_ABI_VERSION). */
int tq_abi_version(void);

/* Static, NUL-terminated description of a status code. */
const char* tq_status_string(int status);

/*
 * Q_mse encoder (prefill and decode-append).
 * Replaces reference PackedMSELayer._encode_group (runtime/packed_qmse_cache.py:376-402)
 * and the bit packing of _pack_indices (:13-43).
 *
 * x: bf16 [batch][heads][tokens][dim] with element strides (x_sb, x_sh, x_st),
 *    the dim axis contiguous.  For each vector: n = |x|, u = x/n, z = u @ R^T,
 *    code_j = #{i : boundaries[i] < z_j}.  Output vector (b,h,t) is written at
 *    token slot (out_offset + t) of group (b*heads + h), groups `out_cap`
 *    tokens apart.  x, rotation and codes 16-byte aligned (TQ_ERR_UNSUPPORTED
 *    otherwise; so are qjl and signs for tq_quantize_prod).
 */
int tq_quantize_mse(const uint16_t* x, int batch, int heads, int64_t tokens, int dim,
                    int64_t x_sb, int64_t x_sh, int64_t x_st,
                    int bits, const float* rotation, const float* boundaries,
                    uint8_t* codes, uint16_t* norms, int64_t out_cap, int64_t out_offset,
                    void* stream);

/*
 * Q_prod key encoder: (mse_bits)-bit Q_mse codes plus the 1-bit QJL sketch of
 * the residual.  Replaces reference PackedMSELayer._encode_keys_qjl_group
 * (runtime/packed_qmse_cache.py:285-310), the residual decode it calls
 * (_decode_group, :404-435) and _pack_qjl_signs (:148-154).
 */
int tq_quantize_prod(const uint16_t* x, int batch, int heads, int64_t tokens, int dim,
                     int64_t x_sb, int64_t x_sh, int64_t x_st,
                     int mse_bits, const float* rotation,
                     const float* centers, const float* boundaries, const float* qjl,
                     uint8_t* codes, uint16_t* norms, uint8_t* signs, uint16_t* rnorms,
                     int64_t out_cap, int64_t out_offset, void* stream);

/*
 * Bytes of workspace tq_decode_attention needs for this shape.
 */
size_t tq_decode_attention_workspace_bytes(int batch, int q_heads, int kv_heads, int dim, int64_t max_tokens);

/*
 * Fused decode attention over the packed cache, one query token per sequence.
 * Replaces reference fused_attention (runtime/triton_kernels.py:238-368) and
 * its _tile_attention_kernel (:84-198): q-side rotations, bit-unpack,
 * codebook dequant, QJL logit correction, softmax, V accumulation, the
 * cross-split log-sum-exp merge and the final un-rotation by R_v.
 *
 *   q        bf16 [batch][q_heads][dim] (contiguous, 16-byte aligned)
 *   seq_starts int32 [batch] first valid token per sequence (nullable: 0), for
 *            left-padded batches
 *   seq_lens int32 [batch] end of the valid tokens per sequence (nullable: n_tokens)
 *   n_tokens tokens stored per group (<= cap)
 *   k_*, v_* packed cache (see layout above), groups `cap` tokens apart
 *   k_signs / k_rnorms / qjl: nullable when has_qjl == 0
 *   scale    logit scale; <= 0 selects 1/sqrt(dim) (the reference's choice)
 *   out_f32  fp32 [batch][q_heads][dim] (nullable)
 *   out_bf16 bf16 [batch][q_heads][dim] (nullable)
 *   lse_out  fp32 [batch][q_heads] log-sum-exp of the scaled logits (nullable;
 *            -inf for an empty sequence), for merging with other attention parts
 *   workspace device scratch of tq_decode_attention_workspace_bytes(); it is
 *            used only during the call (calls sharing one workspace must be
 *            ordered on one stream)
 * logit_t = scale * (|k_t| <q R_k^T, C_k[kidx_t]> + sqrt(pi/2)/D |r_t| <q S^T, s_t>)
 * out     = (sum_t softmax_t |v_t| C_v[vidx_t]) @ R_v
 * The value sums run on fp16 matrix cores: each value centroid enters as its fp16
 * rounding (nearest even).  Over long, evenly spread softmaxes those rounding errors add
 * up; pass value_centers through tq_value_codebook_f16 (below) once per codebook to keep
 * them from doing so.
 */
int tq_decode_attention(const uint16_t* q, int batch, int q_heads, int kv_heads, int dim,
                        const int32_t* seq_starts, const int32_t* seq_lens, int64_t n_tokens, int64_t cap,
                        const uint8_t* k_codes, const uint16_t* k_norms,
                        const uint8_t* k_signs, const uint16_t* k_rnorms,
                        const uint8_t* v_codes, const uint16_t* v_norms,
                        int key_bits, int value_bits, int has_qjl,
                        const float* key_rotation, const float* key_centers, const float* qjl,
                        const float* value_rotation, const float* value_centers,
                        float scale, float* out_f32, uint16_t* out_bf16, float* lse_out,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * The fp16 form of a value codebook for tq_decode_attention.  Host memory in and out;
 * no GPU.  No counterpart in the reference, whose kernel reads the fp32 centroids
 * (runtime/triton_kernels.py:187): it is for callers
 * of tq_decode_attention, which rounds value_centers to fp16.  Each centroid is given one
 * of its two fp16 neighbours, the combination that minimises |sum_c P_c (out_c - c)|, P_c
 * the probability of code c under the coordinate density the Lloyd-Max codebook is built
 * for, (1 - x^2)^((dim - 3)/2) on [-1, 1], cells split at the centroids' midpoints.  The
 * output values are exactly representable in fp16.
 *   centers  fp32 [2^bits], strictly increasing, |c| < 1 (host)
 *   bits     1..4;  dim >= 3 (the head dimension the codebook was built for)
 *   out      fp32 [2^bits] (host)
 */
int tq_value_codebook_f16(const float* centers, int bits, int dim, float* out);

/*
 * tq_decode_attention without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The per-split partials live in a library-owned device array of
 * TQ_NOALLOC_SCRATCH_BYTES, one per GPU, held until the process ends; the caller still
 * passes q, the packed cache and the outputs.  A call whose partials ((dim + 2) fp32 per
 * query head and split) do not fit is rejected with TQ_ERR_WORKSPACE before anything is
 * launched; every shape with batch * q_heads * ceil(1024 / (batch * kv_heads)) <= 16000
 * fits.  All calls on one GPU share its
 * array: calls that overlap in time on one GPU (on different streams, or from several
 * host threads) race and must be ordered by the caller.  Nothing needs clearing
 * between calls (every partial is written before it is read).  Arguments and results
 * are those of tq_decode_attention.
 */
#define TQ_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int tq_decode_attention_noalloc(const uint16_t* q, int batch, int q_heads, int kv_heads, int dim,
                                const int32_t* seq_starts, const int32_t* seq_lens, int64_t n_tokens, int64_t cap,
                                const uint8_t* k_codes, const uint16_t* k_norms,
                                const uint8_t* k_signs, const uint16_t* k_rnorms,
                                const uint8_t* v_codes, const uint16_t* v_norms,
                                int key_bits, int value_bits, int has_qjl,
                                const float* key_rotation, const float* key_centers, const float* qjl,
                                const float* value_rotation, const float* value_centers,
                                float scale, float* out_f32, uint16_t* out_bf16, float* lse_out, void* stream);

/*
 * Dequantise packed Q_mse rows to bf16 (verification / dense fallback of the
 * caller).  Replaces reference _decode_group (runtime/packed_qmse_cache.py:404-435)
 * and triton_decode_group (runtime/triton_kernels.py:227-236):
 * out = bf16((C[codes] @ R) * f32(norm)).  rows are `cap` apart per group.
 * codes and out must be 16-byte aligned, and groups * tokens below 2^31, else
 * TQ_ERR_UNSUPPORTED.
 */
int tq_dequantize_mse(const uint8_t* codes, const uint16_t* norms, int64_t groups, int64_t tokens,
                      int64_t cap, int dim, int bits, const float* rotation, const float* centers,
                      uint16_t* out, void* stream);

/*
 * Dequantise packed Q_prod keys to bf16: the Q_mse reconstruction plus the QJL
 * correction, rounded as the reference does (runtime/packed_qmse_cache.py:312-330):
 *   corr = bf16(((signs(+-1) @ S) * rnorm) * sqrt(pi/2)/D);  out = bf16(khat + corr)
 * codes, signs and out must be 16-byte aligned, and groups * tokens below 2^31,
 * else TQ_ERR_UNSUPPORTED.
 */
int tq_dequantize_prod(const uint8_t* codes, const uint16_t* norms, const uint8_t* signs,
                       const uint16_t* rnorms, int64_t groups, int64_t tokens, int64_t cap, int dim,
                       int mse_bits, const float* rotation, const float* centers, const float* qjl,
                       uint16_t* out, void* stream);

/*
 * Channel groups (the outlier-channel split).  A group is `sub_dim` channels of the
 * dim-channel head, listed in `channels` (HOST memory, strictly ascending), with its
 * own sub_dim x sub_dim rotation / QJL matrix, codebook and bit width (1..8).  The
 * packed rows of a group are ceil(sub_dim*bits/8) code bytes and ceil(sub_dim/8) sign
 * bytes per token (the layout above with D = sub_dim); they need no alignment.
 *
 * Build the group's matrices in channel space once, on the host:
 *   out[j][channels[i]] = sub[j][i] for i, j < sub_dim;  every other entry 0.
 * sub is row-major [sub_dim][sub_dim], out is row-major [dim][dim]; both host memory.
 * Helper for the group-matrix arguments below; no counterpart in the reference, which
 * gathers tensor[..., channels] instead (runtime/packed_qmse_cache.py:441-442, 484-485).
 */
int tq_group_matrix(const float* sub, int sub_dim, const int32_t* channels, int dim, float* out);

/*
 * Encode one channel group: Q_mse at `bits` when qjl is NULL, else Q_prod keys with
 * `bits` MSE bits plus the QJL sketch (centers, signs and rnorms then required).
 * Results are those of tq_quantize_mse / tq_quantize_prod applied to the gathered
 * sub-vectors x[..., channels] with D = sub_dim.  rotation and qjl are the channel-space
 * [dim][dim] matrices of tq_group_matrix (device memory, 16-byte aligned).
 * Replaces reference _encode_split (runtime/packed_qmse_cache.py:481-496) and
 * _encode_keys_split_qjl (:437-454), one group per call.
 */
int tq_quantize_group(const uint16_t* x, int batch, int heads, int64_t tokens, int dim,
                      int64_t x_sb, int64_t x_sh, int64_t x_st,
                      const int32_t* channels, int sub_dim, int bits,
                      const float* rotation, const float* centers, const float* boundaries, const float* qjl,
                      uint8_t* codes, uint16_t* norms, uint8_t* signs, uint16_t* rnorms,
                      int64_t out_cap, int64_t out_offset, void* stream);

/*
 * Decode one channel group into the bf16 rows out [groups*tokens][dim] (16-byte
 * aligned): the group's channels get tq_dequantize_mse / tq_dequantize_prod of the
 * sub-vector (QJL correction when qjl is non-NULL, scaled by sqrt(pi/2)/sub_dim); the
 * other channels are zeroed, or kept when `merge` is non-zero.  Decoding the normal
 * group, then the outlier group with merge = 1, gives the full row.  Code and sign
 * rows need no alignment; groups * tokens, and the code bytes from `codes` to the last
 * row decoded, must stay below 2^31, else TQ_ERR_UNSUPPORTED.
 * Replaces reference _decode_merge (runtime/packed_qmse_cache.py:498-515) and
 * _decode_keys_merge_qjl (:456-479), one group per call.
 */
int tq_dequantize_group(const uint8_t* codes, const uint16_t* norms, const uint8_t* signs,
                        const uint16_t* rnorms, int64_t groups, int64_t tokens, int64_t cap, int dim,
                        const int32_t* channels, int sub_dim, int bits,
                        const float* rotation, const float* centers, const float* qjl,
                        int merge, uint16_t* out, void* stream);

/*
 * Fused decode attention over a layer quantized in channel groups (the outlier split).
 * The reference's fused kernel refuses such layers (runtime/triton_kernels.py:252-253) and
 * its chunked path (runtime/attention.py:215-304) decodes K and V to bf16 for every step;
 * this entry point replaces that path for them.
 *
 * n_groups (1 or 2) groups partition the dim channels; group g has sub_dims[g] channels,
 * key_bits[g] / value_bits[g] (1..8) and the packed arrays k_codes[g] ... v_norms[g] in the
 * channel-group layout above ([G][cap] rows of ceil(sub_dims[g]*bits/8) bytes; signs and
 * rnorms only when has_qjl).  These six are HOST arrays of n_groups device pointers;
 * sub_dims, key_bits and value_bits are host arrays too.  key_centers[g] /
 * value_centers[g] are the groups' codebooks.
 *
 * Two groups with at most 8 channels in group 1, group 0's bit widths as tq_decode_attention
 * takes them, the code and sign arrays at 4-byte boundaries, and either at most 4 query heads
 * per KV head or group 1 one bit wider than group 0 (not with 3-bit Q_mse group 0) run on
 * tq_decode_attention's matrix-core kernel: group 0 there (its value sums in fp16, so
 * value_centers[0] is best given as tq_value_codebook_f16(..., sub_dims[0], ...)), group 1 in
 * fp32 per lane.  Other layers run on an fp32 kernel.
 *
 * key_matrix, qjl_matrix, value_matrix: [dim][dim] device matrices (16-byte aligned)
 * stacking the groups' channel-space matrices (tq_group_matrix), group 0's sub_dims[0]
 * rows first.  The
 * logits are scale * sum_g (|k_g| <q M_k rows of g, C_k,g[codes]> + sqrt(pi/2)/d_g |r_g|
 * <q M_s rows of g, s_g>), the output (sum_t softmax_t |v_g,t| C_v,g[codes]) @ value_matrix.
 * q, seq_starts, seq_lens, n_tokens, cap, scale, the outputs and the workspace (sized by
 * tq_decode_attention_workspace_bytes) are as for tq_decode_attention.
 */
int tq_decode_attention_groups(const uint16_t* q, int batch, int q_heads, int kv_heads, int dim,
                               const int32_t* seq_starts, const int32_t* seq_lens, int64_t n_tokens, int64_t cap,
                               int n_groups, const int* sub_dims, const int* key_bits, const int* value_bits,
                               int has_qjl, const uint8_t* const* k_codes, const uint16_t* const* k_norms,
                               const uint8_t* const* k_signs, const uint16_t* const* k_rnorms,
                               const uint8_t* const* v_codes, const uint16_t* const* v_norms,
                               const float* key_matrix, const float* const* key_centers, const float* qjl_matrix,
                               const float* value_matrix, const float* const* value_centers, float scale,
                               float* out_f32, uint16_t* out_bf16, float* lse_out,
                               void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TQ_H_ */
