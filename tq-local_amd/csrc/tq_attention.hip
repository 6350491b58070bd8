// tq_attention.hip -- fused decode attention over the packed TurboQuant cache (gfx950).
//
// Two launches per call, on the caller's stream:
//
//   split_kernel  grid (n_split, batch * kv_heads), NW waves per workgroup.  A
//                 workgroup first builds its group's q-side operands (q R_k^T,
//                 q S^T) in LDS, then owns a contiguous token range of one (batch
//                 row, KV head), dealt to its waves in 16-token blocks round-robin.
//                 All G query heads of the GQA group share every K/V byte read
//                 (reference runtime/triton_kernels.py:84-198 re-reads the tile
//                 once per query head).
//   merge_kernel  one workgroup per (batch row, query head): log-sum-exp merge over
//                 splits, normalise, un-rotate by R_v, write fp32 / bf16 / lse
//                 (reference :330-336, 366-368).
//
// Per 16-token block, lane l = (n = l & 15, g = l >> 4):
//
//   key score     up to 4 query heads per KV head: v_mfma_i32_16x16x64_i8, 4 per block.
//                 A (registers, fixed for the call): q_rot = q R_k^T times the logit scale
//                 in fixed point, x = rint(q_rot 2^F) with |x| < 2^22, as three balanced
//                 base-256 digits X0..X2; rows = (query head, s = 0..3), k-slots = (dim, key
//                 limb m), row s holding digit X_(s-m).  B = the dequantised keys, Ck 2^E
//                 (|.| < 2^15) as two int8 limbs L0 + 256 L1, one 4-byte LDS lookup per pair
//                 of codes.  The score is (R0 + 256 R1) + 65536 (R2 + 256 R3) of the head's
//                 four rows: both sums exact in int32, then one fp32 rounding.
//                 5..8 heads: v_mfma_f32_16x16x32_bf16, 8 per block, rows = (head, hi|lo part
//                 of q_rot in bf16), k-slots = (dim, hi|lo part of Ck), one 8-byte lookup per
//                 pair of codes; every cross product of the two-term splits is formed.
//   QJL term      v_mfma_i32_16x16x64_i8 on the sign bits left in place (one v_and per 4
//                 dims: bit i of each byte is worth 2^i, -128 for i = 7) against q_proj =
//                 q S^T in fixed point divided by the same 2^i, split in four int8 limbs
//                 (rows = (head, limb)); exact integer accumulation.
//   softmax       online, base 2 (scores are pre-multiplied by log2 e), with a lazily
//                 raised reference maximum: weights are exp2(score - m_ref) and m_ref
//                 is raised (with a rescale of the partial sums) only when a score
//                 exceeds it by more than 2^8, so blocks pay no cross-lane reduction.  m_ref
//                 also tracks the value norm's f16 exponent, which keeps the fp16 weights of
//                 the value sum in range.
//   value sum     v_mfma_f32_16x16x32_f16, 4 per block, D[(head, dim parity)][column] += A B:
//                 A = the softmax weights p |v| in fp16, transposed through per-wave LDS rows;
//                 B = the value codes dequantised in pairs, one 4-byte LDS lookup per pair
//                 of codes returning (Cv[c0], Cv[c1]) in fp16.
//   lookups       pair tables with 32 lane-private copies of every entry (a 32-lane LDS pass
//                 never conflicts).  A pair of 4-bit codes is a byte of the packed words, a
//                 pair of 3-bit codes a "byte window" (a byte holding the 6-bit field in bits
//                 0..5, table T0, or 2..7, table T2): one v_perm forms each lookup address.
//
// All global reads are buffer loads against per-wave descriptors whose size is the
// wave's token range: a lane offset fixed for the call plus a scalar block offset,
// and reads past the range return zeros (no per-lane clamping or 64-bit address
// arithmetic).  Everything accumulates in fp32 (MFMA f32 / i32); no packed-fp32 VALU.

#include "tq_common.h"

#include <mutex>
#include <type_traits>

namespace {

constexpr int D = TQ_DIM;
// waves per split workgroup (one workgroup per CU), the most each kernel's registers allow
// without spills in its loop: with at most 4 query heads per KV head, 4 per SIMD (<= 128
// VGPRs); with 5..8 heads, 3 per SIMD (<= 168)
#ifndef TQ_ATTN_WAVES_G4
#define TQ_ATTN_WAVES_G4 16
#endif
#ifndef TQ_ATTN_WAVES_G8
#define TQ_ATTN_WAVES_G8 12
#endif
#ifndef TQ_ATTN_NB_G4
#define TQ_ATTN_NB_G4 1
#endif
#ifndef TQ_ATTN_NB_G8
#define TQ_ATTN_NB_G8 1
#endif
#ifndef TQ_ATTN_SETS_G4
#define TQ_ATTN_SETS_G4 2
#endif
#ifndef TQ_ATTN_SETS_G8
#define TQ_ATTN_SETS_G8 2
#endif
// layers quantized in two channel groups (SPL): the outlier group's registers take the
// kernel past 128 VGPRs with up to 4 heads per KV head, past 168 with 5-8
#ifndef TQ_ATTN_WAVES_SPL
#define TQ_ATTN_WAVES_SPL 12
#endif
#ifndef TQ_ATTN_WAVES_SPL8
#define TQ_ATTN_WAVES_SPL8 8
#endif
template <int VB, int GC, bool QJL, bool SPL = false>
struct Cfg {
    static constexpr int NW = SPL ? (GC == 1 ? TQ_ATTN_WAVES_SPL : TQ_ATTN_WAVES_SPL8)
                                  : (GC == 1 ? TQ_ATTN_WAVES_G4 : TQ_ATTN_WAVES_G8);
    static constexpr int NT = NW * 64;
    // per-wave blocks in flight (register sets of packed data)
    static constexpr int NSET = GC == 1 ? TQ_ATTN_SETS_G4 : TQ_ATTN_SETS_G8;
    // blocks a wave takes through every stage together (NSET is a multiple)
    static constexpr int NB = GC == 1 ? TQ_ATTN_NB_G4 : TQ_ATTN_NB_G8;
    // register sets of token blocks loaded before the q-side products (the rest right after
    // them): every load instruction issued ahead of a wave's R_k / S rows delays them, and the
    // younger waves' rows wait behind the older waves' token loads.  With 5-8 heads the products
    // take longer (two tiles on some waves), so one set goes first.
    static constexpr int PRO_SETS = GC == 1 ? 0 : 1;
};
constexpr int BLK = 16;        // tokens per block (MFMA N)
constexpr float NEG_INF = -__builtin_huge_valf();
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float QJL_SCALE = 1.2533141373155003f / D;  // sqrt(pi/2) / D
constexpr float LAZY_MAX = 8.0f;                      // log2 headroom before the reference max is raised
constexpr float WEXP0 = 15.0f;  // f16 exponent bias: a raise puts the largest weight p |v| in [1, 2)
constexpr int BUF_DW3 = 0x00020000;                   // buffer descriptor word 3 (gfx9: 32-bit untyped)
#ifndef TQ_KV_NT
#define TQ_KV_NT 2
#endif
constexpr int KV_NT = TQ_KV_NT;  // buffer-load cache policy for the packed stream (2 = nt: streaming, read once)

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_bf16(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f16(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
}
__device__ __forceinline__ i32x4 mfma_i8(const u32x4& a, const u32x4& b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0,
                                                 0);
}

// bf16 RNE (v_cvt_pk_bf16_f32) of x, and of the remainder x - bf16(x): x = hi + lo to ~2^-17.
__device__ __forceinline__ uint32_t bf16_bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x);
}
__device__ __forceinline__ float bf16_val(uint32_t h) { return __uint_as_float(h << 16); }
// (hi, lo) packed low | high
__device__ __forceinline__ uint32_t pack_hilo(float x) {
    const __bf16 hi = (__bf16)x;
    const __bf16 lo = (__bf16)(x - (float)hi);
    return __builtin_bit_cast(uint32_t, bf16x2{hi, lo});
}
// (v, v) packed
__device__ __forceinline__ uint32_t dup_bf16(float v) {
    const __bf16 h = (__bf16)v;
    return __builtin_bit_cast(uint32_t, bf16x2{h, h});
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

// A lane's 24-bit chunk of 3-bit value codes at bit sh of its dword w (sh in {0, 8, 16, 24}),
// aligned to bit 0: the bits past w come from the next lane of the row of 16 (DPP row_shl:1,
// lane i reads lane i + 1), whose dword is the following one of the code row wherever the chunk
// straddles.  Bits 24..31 of the result are not part of the chunk.
__device__ __forceinline__ uint32_t chunk3(uint32_t w, int sh) {
    const uint32_t next = (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0x101, 0xF, 0xF, true);
    return __builtin_amdgcn_alignbit(next, w, sh);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
    const int n = bytes > 0x7FFFFFFF ? 0x7FFFFFFF : (int)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, BUF_DW3);
}

struct Ws {
    size_t po, pml, total;
};

// Per-group q-side image, built in LDS by every split workgroup of the group: the register
// contents of the key-score and QJL A operands for one wave (lane-major, one 16-byte read per
// lane and slot).
constexpr int IMG_QA = 0;                    // [8 j][64 lanes][4]  key-score A operand
constexpr int IMG_QJ = IMG_QA + 8 * 64 * 4;  // [set][2 jj][64 lanes][4]  QJL A operand (int8 limbs)
constexpr int IMG_DW = IMG_QJ + 2 * 2 * 64 * 4;  // dwords per group (a multiple of 4)

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
// MAX_WGS workgroups.
constexpr int MAX_WGS = 1024;
constexpr int MT = 256;  // threads per head in the merge

// ------------------------------------------------------------------ split kernel
// GC = 1: at most 4 query heads per KV head; row 4h + x of every MFMA belongs to
//         head h, so lane group g (lanes 16g..16g+15) holds head g everywhere.
// GC = 2: 5..8 heads; rows 2h + x, lane group g holds heads 2g and 2g + 1.
template <int GC>
struct Rows {
    static constexpr int HPL = GC;  // heads per lane group
    static constexpr int NQJ = GC;  // QJL MFMA sets (four limbs per head in total)
    static constexpr int NH = 4 * GC;
    // key-score rows: GC = 1 (int8 limbs) 4 h + s, s = limb-product order 0..3; GC = 2 (bf16)
    // 2 h + x, x = hi | lo part of q_rot.  Lane group g holds rows 4 g .. 4 g + 3.
    __host__ __device__ static constexpr int row(int h, int x) { return GC == 1 ? 4 * h + x : 2 * h + x; }
    // value rows (head, dim parity p): GC = 1 4 h + 2 p (rows 4 h + 2 p + 1 stay zero), GC = 2
    // 2 h + p; either way lane group g holds the value rows of the heads whose scores it holds
    __host__ __device__ static constexpr int vrow(int h, int p) { return GC == 1 ? 4 * h + 2 * p : 2 * h + p; }
};

// Lookup tables.  Every entry has TCOPIES lane-private copies, copy c in the bank of lane c of a
// 32-lane LDS pass, so a lookup never conflicts.  Entry e of the pair tables sits at byte 256 e
// (one v_perm forms a byte code's address): copies 0..31 of the value pair (fp16 Cv[c0],
// Cv[c1]) at +4 c, and with int8 keys copies 0..31 of the key pair (int8 limbs L0, L1 of
// Ck[c0], then of Ck[c1]) at +128 + 4 c.  bf16 keys (5..8 heads) keep a table of their own:
// (Ck hi|lo of c0, Ck hi|lo of c1) per pair, 8 bytes, copy c at +8 c.
constexpr int TCOPIES = 32;
constexpr int WROW = 16;  // dwords per row of the weight transpose: 4 lane groups x 4 tokens

template <int KB, int VB>
constexpr int PAIR_ENTRIES = (1 << (2 * KB)) > (1 << (2 * VB)) ? (1 << (2 * KB)) : (1 << (2 * VB));

// LDS scratch of the image builder (QR: q R_k^T kept, for the int8 key image or the outlier
// group of a two-group layer)
template <int GC, bool QR = GC == 1>
struct PrepLds {
    static constexpr int NH = 4 * GC;
    float qp[NH][D];                  // q S^T of the group's heads
    float qr[QR ? NH : 1][D];         // q R_k^T times the logit scale
    float red[16];                    // max |.| per matrix-core tile: R_k tiles 0..7, S tiles 8..15
};

// The outlier group of a two-group layer: OD (4 or 8) dims per lane, in fp32.  Code pairs are
// looked up in pair tables of (C[c0], C[c1]) where the widths allow (keys up to 4 bits, values
// up to 5 bits with OD = 4, 4 with OD = 8), single codes in the codebooks otherwise.
constexpr int OD1 = 8;
template <int OD, int NH>
struct OutLds {
    static constexpr int KP = 256, VP = OD == 4 ? 1024 : 256;  // pair-table entries
    float q1[NH][OD];       // per query head: q_rot of the group's dims (log2 units)
    float ts[NH][1 << OD];  // per query head: sum of q_proj (times the QJL scale) over the dims whose sign bit is set
    float ck[256];          // the group's key and value codebooks (up to 8 bits)
    float cv[256];
    float2 tk[KP];          // key code pairs
    float2 tv[VP];          // value code pairs
};
template <int NH>
struct OutLds<0, NH> {};

template <int KB, int VB, bool QJL, int GC, int OD = 0>
struct Smem {
    static constexpr int NH = 4 * GC;
    static constexpr bool SPL = OD > 0;
    static constexpr int NW = Cfg<VB, GC, QJL, SPL>::NW;
    static constexpr bool KI8 = GC == 1;
    // Byte windows (3-bit codes): the 6-bit field of a code pair is looked up by a byte of the
    // packed words that holds it, one v_perm per lookup.  T0 (the pair tables) is indexed by a
    // byte whose bits 0..5 hold the pair, T2 by a byte whose bits 2..7 hold it; the two spare
    // bits belong to neighbouring codes, so each pair has 4 entries in either table.
    static constexpr bool KWIN = KI8 && KB == 3;
    static constexpr bool VWIN = VB == 3;
    static constexpr bool WIN = KWIN || VWIN;
    static constexpr int PE = WIN ? 256 : (KI8 ? PAIR_ENTRIES<KB, VB> : (1 << (2 * VB)));
    static constexpr int KC = KB <= 3 ? 32 : 16;  // copies of the bf16 key pair table
    // ktab and tab sit below 64 KB, so their bases fold into the LDS instructions' offsets; T2
    // starts exactly 64 KB above T0 (a lookup adds the 64 KB through byte 2 of its address)
    uint2 ktab[KI8 ? 2 : (1 << (2 * KB))][KI8 ? 1 : KC];  // bf16 key pairs (int8 keys: padding)
    uint32_t tab[PE][64];                              // value pairs (and int8 key pairs): T0
    union {
        uint32_t t2[WIN ? 256 : 1][64];                // T2, built over the prologue's area
        struct {
            uint4 img[IMG_DW / 4];      // this group's q-side image
            uint4 qst[NW][NH * 16 > 128 ? NH * 16 : 128];  // per wave: the query rows, then the R_k / S restage
            PrepLds<GC, (GC == 1 || SPL)> ps;  // scratch of the image builder
        } pro;
        struct {
            float o[NW][NH][D];
            float m[NW][NH];
            float s[NW][NH];
        } epi;
    } u;
    uint32_t wt[NW][Cfg<VB, GC, QJL, SPL>::NB][16][WROW];   // per-wave transposes of the softmax weights
    OutLds<OD, NH> ol;
};

// LDS byte offset (from T0's base) of the table entry of the 6-bit field at bit p of the word
// array w, p a compile-time constant after unrolling.  s is the stream w >> 4 (s[i] = bits
// 32 i + 4 .. 32 i + 35 of w), needed for fields at p = 4, 6 mod 8 only.  pl is the lane's copy
// offset (byte 0) with byte 2 = 1: the selector copies byte 0 and, for T2, byte 2 (+64 KB).
__device__ __forceinline__ uint32_t win_off(const uint32_t* w, const uint32_t* s, int p, uint32_t pl) {
    const bool sh = (p & 7) >= 4;
    const int q = sh ? p - 4 : p;             // 0 or 2 mod 8 in w or s
    const bool t2 = (q & 7) == 2;
    const int wb = t2 ? q - 2 : q;            // first bit of the byte window
    const uint32_t sel = (t2 ? 0x0C020000u : 0x0C0C0000u) | ((4u + (uint32_t)((wb & 31) >> 3)) << 8);
    return __builtin_amdgcn_perm(sh ? s[wb >> 5] : w[wb >> 5], pl, sel);
}

// ----------------------------------------------------------------- merge
// One query head bh, MT threads (t = 0..MT-1): merge the split partials (maxima in the log2
// domain), normalise, un-rotate by R_v.  Thread t reads R_v rows k in [16 (t / 32), 16 (t / 32)
// + 16), columns 4 (t % 32) .. + 3, as float4.  Every thread of the workgroup calls it (barriers
// inside).
__device__ __forceinline__ void merge_head(int bh, int t, int n_split, const float* __restrict__ part_o,
                                           const float* __restrict__ part_ml, const float* __restrict__ Rv,
                                           float* __restrict__ out_f32, uint16_t* __restrict__ out_bf16,
                                           float* __restrict__ lse_out, float* so, float4 (*part)[D / 4],
                                           float (*red)[2]) {
    const int lane = t & 63, wv = t >> 6;
    // this thread's slice of R_v, loaded first: its L2 latency overlaps the merge of the splits
    const int c4 = t & 31, kr = t >> 5;
    const float4* rv4 = reinterpret_cast<const float4*>(Rv);
    float4 rvs[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) rvs[i] = rv4[(size_t)(16 * kr + i) * (D / 4) + c4];
    const float* ml = part_ml + (size_t)bh * n_split * 2;
    // normalised rotated output: threads (half, d) split the splits in two.  The partials of
    // this thread's first PF splits are loaded with the maxima, before the maximum is known, so
    // the merge waits for one round of loads instead of two
    const int d = t & (D - 1), hf = t >> 7;
    constexpr int PF = 8;
    float pv[PF], pm[PF], ps[PF];
#pragma unroll
    for (int j = 0; j < PF; ++j) {
        const int k = hf + 2 * j;
        const bool in = k < n_split;
        pv[j] = in ? part_o[((size_t)bh * n_split + k) * D + d] : 0.0f;
        pm[j] = in ? ml[2 * k] : NEG_INF;
        ps[j] = in ? ml[2 * k + 1] : 0.0f;
    }
    float M = NEG_INF;
    for (int k = t; k < n_split; k += MT) M = fmaxf(M, ml[2 * k]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    if (lane == 0) red[wv][0] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0][0], red[1][0]), fmaxf(red[2][0], red[3][0]));
    float o = 0.0f, sacc = 0.0f;
    if (M != NEG_INF) {
        // splits hf, hf + 2, ... in order
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            const float e = pm[j] == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(pm[j] - M);
            o = __builtin_fmaf(e, pv[j], o);
            sacc = __builtin_fmaf(e, ps[j], sacc);
        }
        // the rest, unrolled so that several splits' loads are in flight together
#pragma unroll 4
        for (int k = hf + 2 * PF; k < n_split; k += 2) {
            const float mk = ml[2 * k];
            const float e = mk == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mk - M);
            o = __builtin_fmaf(e, part_o[((size_t)bh * n_split + k) * D + d], o);
            sacc = __builtin_fmaf(e, ml[2 * k + 1], sacc);
        }
    }
    float* po2 = reinterpret_cast<float*>(part);
    po2[t] = o;
    if (d == 0) red[hf][1] = sacc;
    __syncthreads();
    if (t < D) {
        const float sum = red[0][1] + red[1][1];
        so[t] = (M != NEG_INF) ? (po2[t] + po2[t + D]) / fmaxf(sum, 1e-8f) : 0.0f;
        if (lse_out && t == 0) lse_out[bh] = (M != NEG_INF) ? M * LN2 + logf(sum) : NEG_INF;
    }
    __syncthreads();
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 r = rvs[i];
        const float w = so[16 * kr + i];
        acc.x = __builtin_fmaf(w, r.x, acc.x);
        acc.y = __builtin_fmaf(w, r.y, acc.y);
        acc.z = __builtin_fmaf(w, r.z, acc.z);
        acc.w = __builtin_fmaf(w, r.w, acc.w);
    }
    __syncthreads();  // so / po2 reads above are done before part is overwritten
    part[kr][c4] = acc;
    __syncthreads();
    if (t < D) {
        const float* pf = reinterpret_cast<const float*>(part);
        float a = 0.0f;
#pragma unroll
        for (int r = 0; r < MT / 32; ++r) a += pf[r * D + t];
        if (out_f32) out_f32[(size_t)bh * D + t] = a;
        if (out_bf16) out_bf16[(size_t)bh * D + t] = (uint16_t)tq::f32_to_bf16(a);
    }
}

// One workgroup per (batch row, query head).
__global__ __launch_bounds__(MT) void merge_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                                   int n_split, const float* __restrict__ Rv,
                                                   float* __restrict__ out_f32, uint16_t* __restrict__ out_bf16,
                                                   float* __restrict__ lse_out) {
    __shared__ float so[D];
    __shared__ float4 part[MT / 32][D / 4];
    __shared__ float red[MT / 64][2];
    merge_head(blockIdx.x, threadIdx.x, n_split, part_o, part_ml, Rv, out_f32, out_bf16, lse_out, so, part, red);
}

// ------------------------------------------------------------------ q-side image
// Per (batch row, KV head): q_rot = q R_k^T and q_proj = q S^T for the group's query heads
// (reference runtime/triton_kernels.py:289, 305-306), split into the MFMA operand layouts the
// split kernel holds in registers:
//   key score: lane (n, g), MFMA j, VGPR r = q_x[h][32 g + 4 j + r] twice (bf16), row n =
//              R::row(h, x), x = 0: bf16(q_rot), x = 1: bf16(q_rot - bf16(q_rot));
//   QJL:       x_d = rint(q_proj_d 2^(G2 - d % 8)) (negated for d % 8 = 7) in four balanced
//              base-256 digits (int8 limbs), rows (head, limb), byte e of VGPR v of MFMA jj <->
//              dim 32 g + 4 jj + v + 8 e.  The key-score operand carries the logit scale times
//              log2 e; the QJL scale 2^(1 - G2) times the QJL logit scale is applied per token.
//
// The mat-vecs run on the matrix cores, one 16-column tile per wave: tile t < 8 is columns
// [16 t, 16 t + 16) of q R_k^T, tile t >= 8 the same columns of q S^T.  A = q (rows = query
// heads, bf16 as given, exact); B = the matrix rows, each fp32 element split exactly into three
// bf16 terms hi + mid + lo (truncations: hi keeps the top 8 significant bits, mid the next 8,
// and the rest has at most 8), so every product is exact and the sums are fp32 MFMA
// accumulations.  Each load instruction reads whole 128-byte lines: the columns [32 s, 32 s +
// 32) of 8 of the tile's rows, lane l row 8 hf + l / 8, floats 32 s + 4 (l mod 8) .. + 3.  The
// wave restages each k-step's 2 KB through its own LDS slot into the MFMA layout (lane (c, kq):
// row c, floats 32 s + 8 kq .. + 7).  Loads that instead took 64 bytes of each of 16 rows per
// instruction (the MFMA layout directly) arrived about half as fast.

// hi | mid | lo bf16 terms of the 8 floats of one lane's k-step (element e <-> k-slot e)
__device__ __forceinline__ void split3_bf16(const f32x4& a, const f32x4& b, u32x4& hi, u32x4& mid, u32x4& lo) {
    const float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t x0 = __float_as_uint(x[2 * p]), x1 = __float_as_uint(x[2 * p + 1]);
        hi[p] = __builtin_amdgcn_perm(x1, x0, 0x07060302u);
        const float r0 = x[2 * p] - __uint_as_float(x0 & 0xFFFF0000u);
        const float r1 = x[2 * p + 1] - __uint_as_float(x1 & 0xFFFF0000u);
        const uint32_t u0 = __float_as_uint(r0), u1 = __float_as_uint(r1);
        mid[p] = __builtin_amdgcn_perm(u1, u0, 0x07060302u);
        const float l0 = r0 - __uint_as_float(u0 & 0xFFFF0000u);
        const float l1 = r1 - __uint_as_float(u1 & 0xFFFF0000u);
        lo[p] = __builtin_amdgcn_perm(__float_as_uint(l1), __float_as_uint(l0), 0x07060302u);
    }
}

// Phase 1 (no barriers).  R_k tiles write their part of the key-score image; S tiles write
// q_proj to L.qp and their max |q_proj| to L.red.  mid() runs in every wave after this wave's
// operand loads are issued and before they are waited for: global loads complete in issue
// order, so loads that mid() issues stay in flight through the products (and the barriers,
// which wait for LDS only).
template <bool QJL, int GC, int NW, bool KI8, bool QR, typename Mid>
__device__ __forceinline__ void image_products(const uint16_t* __restrict__ q, int G, int bh0,
                                               const float* __restrict__ Rk, const float* __restrict__ S,
                                               float c_mse, PrepLds<GC, QR>& L, uint32_t* img, uint4* qst,
                                               int wave, int lane, int d0, Mid&& mid) {
    using R = Rows<GC>;
    constexpr int NH = R::NH;
    constexpr int NTILE = QJL ? 16 : 8;
    constexpr int TPW = (NTILE + NW - 1) / NW;  // tiles per wave
    const bool active = wave < NTILE;           // wave-uniform
    const int c = lane & 15, kq = lane >> 4;
    // A: lane (row c = query head, kq) holds q[c][32 s + 8 kq + e] for k-step s
    u32x4 qa[4];
    // B as loaded: rr[u][2 s + hf], lane l: row 16 t' + 8 hf + l / 8, floats 32 s + 4 (l mod 8) .. + 3
    f32x4 rr[TPW][8];
    // the group's query rows, 16 bytes per lane (rows >= G read as zero through the descriptor),
    // restaged in the wave's LDS slot below: one load per NH / 4 rows instead of four per lane,
    // most of them repeats of the same rows
    u32x4 qv[NH / 4];
    if (active) {
        const __amdgpu_buffer_rsrc_t rq = rsrc(q + (size_t)bh0 * D, (int64_t)G * D * 2);
#pragma unroll
        for (int i = 0; i < NH / 4; ++i) qv[i] = __builtin_amdgcn_raw_buffer_load_b128(rq, (i * 64 + lane) * 16, 0, 0);
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
            const int t = wave + u * NW;
            if (t < NTILE) {
                const float* row = (t < 8 ? Rk : S) + (size_t)(16 * (t & 7) + (lane >> 3)) * D + 4 * (lane & 7);
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf)
                        rr[u][2 * s + hf] = *reinterpret_cast<const f32x4*>(row + (size_t)(8 * hf) * D + 32 * s);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    mid();
    __builtin_amdgcn_sched_barrier(0);
    if (!active) return;
    // the wave's own LDS slot: its accesses execute in order, no barrier needed
#pragma unroll
    for (int i = 0; i < NH / 4; ++i) qst[i * 64 + lane] = __builtin_bit_cast(uint4, qv[i]);
    {
        const int cr = c < NH ? c : 0;
#pragma unroll
        for (int s = 0; s < 4; ++s) qa[s] = __builtin_bit_cast(u32x4, qst[cr * 16 + 4 * s + kq]);
    }
    if (c >= G) {
#pragma unroll
        for (int s = 0; s < 4; ++s) qa[s] = u32x4{0u, 0u, 0u, 0u};
    }
    // the same slot restages the matrix rows (2 KB per k-step; the qa reads above come first in
    // the wave's LDS order): lane (c, kq) takes row c's floats 32 s + 8 kq .. + 7, which lanes
    // 8 (c mod 8) + 2 kq and + 1 of instruction c / 8 loaded
    f32x4* const rst = reinterpret_cast<f32x4*>(qst);
    const int src = 64 * (c >> 3) + 8 * (c & 7) + 2 * kq;
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
        const int t = wave + u * NW;
        if (t >= NTILE) break;
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            rst[lane] = rr[u][2 * s];
            rst[64 + lane] = rr[u][2 * s + 1];
            const f32x4 b0 = rst[src], b1 = rst[src + 1];
            u32x4 hi, mid, lo;
            split3_bf16(b0, b1, hi, mid, lo);
            acc = mfma_bf16(qa[s], lo, acc);
            acc = mfma_bf16(qa[s], mid, acc);
            acc = mfma_bf16(qa[s], hi, acc);
        }
        // lane (c, kq) holds rows 4 kq + i (query heads) of column j
        const int j = 16 * (t & 7) + c;
        if (!KI8 && t < 8) {
            // bf16 key-score image: dword (jj, lane (n, gq), r) holds dim j = 32 gq + 4 jj + r of row n
            if (4 * kq < NH) {
                const int gq = j >> 5, jj = (j >> 2) & 7, r = j & 3;
                uint32_t* base = img + IMG_QA + (jj * 64 + 16 * gq) * 4 + r;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int h = 4 * kq + i;
                    // scores come out in log2 units; dims >= d0 (a two-group layer's outlier
                    // group) are zero here and kept in L.qr for their own term
                    const float xr = acc[i] * c_mse;
                    const float x = j < d0 ? xr : 0.0f;
                    const float xh = bf16_val(bf16_bits(x));
                    base[R::row(h, 0) * 4] = dup_bf16(xh);
                    base[R::row(h, 1) * 4] = dup_bf16(x - xh);
                    if constexpr (QR) L.qr[h][j] = xr;
                }
            }
        } else {
            // q S^T (and with int8 keys q R_k^T times the logit scale) to LDS, with the tile's
            // max |.| for the fixed-point exponents of phase 2
            float* dst = &L.qp[0][0];
            float sc = 1.0f;
            if constexpr (KI8) {
                if (t < 8) dst = &L.qr[0][0], sc = c_mse;
            }
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = acc[i] * sc;
            if (4 * kq < NH) {
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[(4 * kq + i) * D + j] = x[i];
            }
            float mx = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
            mx = row_max16(mx);  // then the four rows of 16 lanes
            mx = fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 0)),
                             __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 16))),
                       fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 32)),
                             __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 48))));
            if (lane == 0) L.red[t] = mx;
        }
    }
}

// Phase 2 (after a barrier): the QJL fixed-point exponent G2 (max |q_proj| 2^(G2 - 7) < 2^22,
// G2 - 7 capped at 60) and the limb image of dims d < d0 (zero beyond: the outlier group of a
// two-group layer has its own term).  Returns G2 in every thread.
template <int GC, int NT, bool QR>
__device__ __forceinline__ int qjl_image(const PrepLds<GC, QR>& L, uint32_t* img, int tid, int d0) {
    constexpr int NH = 4 * GC;
    float mx = 0.0f;
#pragma unroll
    for (int w = 0; w < 8; ++w) mx = fmaxf(mx, L.red[8 + w]);
    int e = 0;
    if (mx > 0.0f) (void)frexpf(mx, &e);  // mx < 2^e
    int F = 22 - e;
    F = F > 60 ? 60 : F;
    const int G2 = F + 7;
    uint8_t* ib = reinterpret_cast<uint8_t*>(img + IMG_QJ);
    for (int i = tid; i < NH * D; i += NT) {
        const int h = i / D, d = i % D, bit = d & 7;
        int x = d < d0 ? (int)rintf(L.qp[h][d] * ldexpf(1.0f, G2 - bit)) : 0;
        if (bit == 7) x = -x;  // bit 7 of a sign byte is worth -128
        const int gq = d >> 5, jj = bit >> 2, v = bit & 3, e8 = (d >> 3) & 3;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int l = ((x + 128) & 255) - 128;  // balanced base-256 digit k
            const int set = GC == 1 ? 0 : k >> 1;
            const int n = GC == 1 ? 4 * h + k : 2 * h + (k & 1);
            ib[(((set * 2 + jj) * 64 + 16 * gq + n) * 4 + v) * 4 + e8] = (uint8_t)(l & 255);
            x = (x - l) >> 8;
        }
    }
    return G2;
}

// sum_d y_d s_d of the lane's head i from the QJL MFMA accumulators (four limb sums, each
// |.| <= 2^21): pairs exact in int32, then one fp32 rounding
template <int GC>
__device__ __forceinline__ float qjl_combine(const i32x4 (&acc)[GC], int i) {
    int lo, hi;
    if constexpr (GC == 1) {
        lo = acc[0][0] + (acc[0][1] << 8);
        hi = acc[0][2] + (acc[0][3] << 8);
    } else {
        lo = acc[0][2 * i] + (acc[0][2 * i + 1] << 8);
        hi = acc[1][2 * i] + (acc[1][2 * i + 1] << 8);
    }
    return __builtin_fmaf((float)hi, 65536.0f, (float)lo);
}


// Phase 2 (after a barrier), int8 key image (at most 4 query heads): x = rint(q_rot 2^F), the
// q-side score operand (q R_k^T times the logit scale) in fixed point with max |x| < 2^22 (F
// capped at 60), in three balanced base-256 digits X0..X2.  Key MFMA j, lane (row 4 h + s,
// group g), byte 4 i + 2 e + m <-> dim d = 32 g + 8 j + 2 i + e and codebook limb m: the A operand
// is X_{s-m}[h][d] where 0 <= s - m <= 2 and zero otherwise, so row 4 h + s sums the products of
// digit pairs of weight 2^(8 s).  Dims d >= d0 are zero (the outlier group of a two-group
// layer).  Returns F in every thread.
template <int NT>
__device__ __forceinline__ int key_image_i8(const PrepLds<1>& L, uint32_t* img, int tid, int d0) {
    float mx = 0.0f;
#pragma unroll
    for (int w = 0; w < 8; ++w) mx = fmaxf(mx, L.red[w]);
    int e = 0;
    if (mx > 0.0f) (void)frexpf(mx, &e);  // mx < 2^e
    int F = 22 - e;
    F = F > 60 ? 60 : F;
    const float sc = ldexpf(1.0f, F);
    uint8_t* ib = reinterpret_cast<uint8_t*>(img + IMG_QA);
    for (int i = tid; i < 4 * D; i += NT) {
        const int h = i / D, d = i % D;
        int x = d < d0 ? (int)rintf(L.qr[h][d] * sc) : 0;
        int X[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            X[k] = ((x + 128) & 255) - 128;  // balanced base-256 digit k
            x = (x - X[k]) >> 8;
        }
        const int g = d >> 5, j = (d >> 3) & 3, ii = (d >> 1) & 3, par = d & 1;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const int l = s - m;
                const int v = (l >= 0 && l <= 2) ? X[l] : 0;
                ib[(j * 64 + 16 * g + 4 * h + s) * 16 + 4 * ii + 2 * par + m] = (uint8_t)(v & 255);
            }
    }
    return F;
}

// Layers quantized in two channel groups (the outlier split, reference
// runtime/packed_qmse_cache.py:437-515), for the split kernel with OD > 0: group 0 (d0 = D - d1
// channels, rotated dims 0 .. d0 - 1 of the stacked matrices) runs through the MFMA stages,
// its rows of ceil(d0 b / 8) bytes read at any byte alignment (the q-side image is zero on
// dims >= d0, so the bytes there, which belong to the next row, add nothing); group 1 (d1 <= OD
// channels, dims d0 .. D - 1) adds a per-lane fp32 term to the scores and keeps its own value
// sums, which replace dims d0 .. D - 1 of the MFMA sums at the end.
struct Og {
    int d0, d1;         // channels of the two groups
    int r0k, r0s, r0v;  // group 0 row bytes: key codes, sign bits, value codes
    int r1k, r1s, r1v;  // group 1 row bytes
    int b1k, b1v;       // group 1 code widths (1..8)
    const uint8_t *kc1, *ks1, *vc1;
    const uint16_t *kn1, *kr1, *vn1;
    const float *Ck1, *Cv1;
    float cq1;          // the logit scale (log2 units) times sqrt(pi/2) / d1
};

// X1 > 0: group 1's widths are group 0's plus X1 (the reference's default outlier_extra_bits
// is 1), compile-time constants; X1 = 0: the widths come from og at run time.
template <int KB, int VB, bool QJL, int GC, int OD = 0, int X1 = 0>
__global__ __launch_bounds__((Cfg<VB, GC, QJL, (OD > 0)>::NT)) void split_kernel(
    const uint16_t* __restrict__ q, int q_heads, int kv_heads, int G, const int32_t* __restrict__ seq_starts,
    const int32_t* __restrict__ seq_lens, int64_t n_tokens, int64_t cap, const uint8_t* __restrict__ kc,
    const uint16_t* __restrict__ kn, const uint8_t* __restrict__ ks, const uint16_t* __restrict__ kr,
    const uint8_t* __restrict__ vc, const uint16_t* __restrict__ vn, const float* __restrict__ Rk,
    const float* __restrict__ S, float c_mse, float c_qjl,
    const float* __restrict__ Ck, const float* __restrict__ Cv, float scale,
    int64_t tokens_per_split, int n_split, float* __restrict__ part_o, float* __restrict__ part_ml, Og og) {
    constexpr bool SPL = OD > 0;
    static_assert(!SPL || OD <= OD1, "two-group layers: at most OD1 outlier dims per lane");
    using Sm = Smem<KB, VB, QJL, GC, OD>;
    using R = Rows<GC>;
    constexpr bool KI8 = Sm::KI8;
    constexpr int NW = Cfg<VB, GC, QJL, SPL>::NW;
    constexpr int NT = Cfg<VB, GC, QJL, SPL>::NT;
    constexpr int KROW = D * KB / 8;  // bytes per key row
    constexpr int VROW = D * VB / 8;  // bytes per value row
    constexpr int VCH = 8 * VB;       // bits of one lane's 8-dim value chunk
    constexpr int NKM = KI8 ? 4 : 8;  // key-score MFMAs per block
    __shared__ Sm sm;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int n = lane & 15, g = lane >> 4;
    const int split = blockIdx.x, grp = blockIdx.y;
    const int b = grp / kv_heads, kvh = grp - b * kv_heads;
    const int bh0 = b * q_heads + kvh * G;  // first query head of the group

    // ---------------------------------------------------------- token range
    // per-row bounds, made provably wave-uniform so the buffer descriptors below live in SGPRs
    int64_t len = n_tokens;
    if (seq_lens) {
        const int64_t l = __builtin_amdgcn_readfirstlane(seq_lens[b]);
        len = l < n_tokens ? (l < 0 ? 0 : l) : n_tokens;
    }
    int64_t start = 0;
    if (seq_starts) {
        const int64_t st = __builtin_amdgcn_readfirstlane(seq_starts[b]);
        start = st < 0 ? 0 : st;
    }
    int64_t r0 = (int64_t)split * tokens_per_split;
    int64_t r1 = r0 + tokens_per_split;
    r0 = r0 > start ? r0 : start;
    r1 = r1 < len ? r1 : len;
    // The workgroup streams [t0, t1) in 16-token blocks dealt round-robin to its waves (block
    // i to wave i mod NW), so at any moment the waves read neighbouring blocks of every array:
    // DRAM pages are shared instead of NW separate streams per array (~14% more bandwidth).
    const int64_t t0 = r0;
    const int64_t t1 = r1 > r0 ? r1 : r0;
    const int64_t ntok = t1 - t0;
    // token offsets within the range are 32-bit: the host keeps the range below 2^24 tokens
    const int nt = (int)ntok;
    constexpr int STEP = NW * BLK;
    const size_t row0 = (size_t)grp * cap + (size_t)(t0 < n_tokens ? t0 : 0);

    // row bytes: the full-width rows, or group 0's of a two-group layer
    const int krow = SPL ? og.r0k : KROW, srow = SPL ? og.r0s : D / 8, vrow = SPL ? og.r0v : VROW;
    // workgroup buffer descriptors over [t0, t1): reads beyond the range return 0.  A row array
    // of a two-group layer starts at any byte: its descriptor starts at the dword holding the
    // range's first byte (*A = that byte's offset in it) and ends at a dword boundary.  The
    // bytes past the range that the last dword holds lie in the page of the range's last byte
    // (an aligned dword never crosses a page), and no valid token's code comes from them.
    const auto rs_row = [&](const void* arr, int r, int* A) {
        const size_t b0 = row0 * (size_t)r;
        *A = SPL ? (int)(b0 & 3) : 0;
        return rsrc(static_cast<const uint8_t*>(arr) + (b0 - (size_t)*A), ((int64_t)*A + ntok * r + 3) & ~(int64_t)3);
    };
    int Ak = 0, As = 0, Av = 0;
    const __amdgpu_buffer_rsrc_t rk = rs_row(kc, krow, &Ak);
    const __amdgpu_buffer_rsrc_t rv = rs_row(vc, vrow, &Av);
    const __amdgpu_buffer_rsrc_t rkn = rsrc(kn + row0, ntok * 2);
    const __amdgpu_buffer_rsrc_t rvn = rsrc(vn + row0, ntok * 2);
    __amdgpu_buffer_rsrc_t rs = rkn, rkr = rkn;
    if constexpr (QJL) {
        rs = rs_row(ks, srow, &As);
        rkr = rsrc(kr + row0, ntok * 2);
    }

    // lane offsets (bytes) into the per-wave buffers.  Rows at any byte alignment (two-group
    // layers) are read from the dword holding the lane's first byte and realigned by a bit
    // shift fixed for the call (block offsets are multiples of 16 rows, so of 4 bytes)
    const int kraw = Ak + n * krow + 4 * KB * g;  // key codes of token n, dims [32 g, 32 g + 32)
    const int ko = kraw & ~3, kalign = 8 * (kraw & 3);
    const int sraw = As + n * srow + 4 * g;       // sign bits of token n, same dims
    const int so = sraw & ~3, salign = 8 * (sraw & 3);
    const int no = 2 * n;                         // f16 norms of token n
    int vo, vsh;
    if constexpr (SPL) {
        // lane n's chunk (dims [8 n, 8 n + 8), VB bytes) in the row of token g; + 4 r vrow for
        // token 4 r + g.  Two dwords per row, realigned by vsh
        const int vraw = Av + g * vrow + VB * n;
        vo = vraw & ~3;
        vsh = 8 * (vraw & 3);
    } else {
        // the dword holding the chunk's first bit, and the chunk's offset in it.  A 3-bit chunk
        // (24 bits at 24 n) straddles two dwords only for n = 1, 2 mod 4 (offsets 24, 16), and
        // then its second dword is the first dword of lane n + 1's chunk: each lane reads one
        // dword per row and takes the next one from its neighbour (reading both dwords in every
        // lane made the value stream ~16% slower to load)
        const int vbit0 = VCH * n;                // value chunk of lane n: dims [8 n, 8 n + 8)
        const int vdw = vbit0 >> 5;
        vo = 4 * vdw + g * VROW;                  // + 4 r VROW for token 4 r + g (each load: 4 whole rows)
        vsh = vbit0 - 32 * vdw;                   // in [0, 32)
    }
    // group 1 of a two-group layer: token n's rows (at most 8 bytes each) from the dword
    // holding their first byte, and its three norms
    __amdgpu_buffer_rsrc_t rk1 = rkn, rs1 = rkn, rv1 = rkn, rkn1 = rkn, rkr1 = rkn, rvn1 = rkn;
    int o1k = 0, o1ksh = 0, o1s = 0, o1ssh = 0, o1v = 0, o1vsh = 0, o1n = 0;
    if constexpr (SPL) {
        int A1k = 0, A1s = 0, A1v = 0;
        rk1 = rs_row(og.kc1, og.r1k, &A1k);
        rv1 = rs_row(og.vc1, og.r1v, &A1v);
        rkn1 = rsrc(og.kn1 + row0, ntok * 2);
        rvn1 = rsrc(og.vn1 + row0, ntok * 2);
        if constexpr (QJL) {
            rs1 = rs_row(og.ks1, og.r1s, &A1s);
            rkr1 = rsrc(og.kr1 + row0, ntok * 2);
        }
        const int k1 = A1k + n * og.r1k, s1 = A1s + n * og.r1s, v1 = A1v + n * og.r1v;
        // lanes 32..63 read the round's second block, STEP tokens on (a multiple of 16 rows,
        // so the same byte shifts)
        const int hb = g >= 2 ? NW * BLK : 0;
        o1k = (k1 & ~3) + hb * og.r1k, o1ksh = 8 * (k1 & 3);
        o1s = (s1 & ~3) + hb * og.r1s, o1ssh = 8 * (s1 & 3);
        o1v = (v1 & ~3) + hb * og.r1v, o1vsh = 8 * (v1 & 3);
        o1n = no + 2 * hb;
    }

    // Per-block data of a wave, in the part the score stage reads (key codes, sign bits and
    // the three norms of token n) and the part the value stage reads (value codes of tokens
    // 4 r + g).
    // Rows at any byte alignment (SPL) carry one dword more, realigned when processed.
    struct Kd {
        uint32_t kw[SPL ? KB + 1 : KB];  // key codes of token n, dims [32 g, 32 g + 32)
        uint32_t sw[SPL ? 2 : 1];        // sign bits of token n, same dims
        uint32_t kn, kr, vn;             // norms (f16 bits) of token n
    };
    struct Vd {
        uint32_t vw[SPL ? 8 : 4];  // value codes of tokens 4 r + g, the dword holding lane n's chunk start
    };
    // group 1 of a two-group layer, for the two blocks of a round (NSET = 2 blocks STEP tokens
    // apart; lanes 0..31 hold the first, lanes 32..63 the second, each block's half reaching all
    // lanes through v_permlane32_swap): token n's key code, sign and value code rows (from the
    // dwords holding their first bytes) and norms.  One load instruction per array serves two
    // blocks (six per block measured ~18 us per call slower at the C2 split shape).
    struct Od {
        uint32_t k[3], s, v[3];
        uint32_t kn, kr, vn;
    };
    struct OdNone {};
    using OdT = std::conditional_t<SPL, Od, OdNone>;
    auto load_o = [&](OdT& O, int rel_) {
        if constexpr (SPL) {
            const int rel = __builtin_amdgcn_readfirstlane(rel_);
            const u32x3 k = __builtin_amdgcn_raw_buffer_load_b96(rk1, o1k, rel * og.r1k, KV_NT);
            O.k[0] = k.x, O.k[1] = k.y, O.k[2] = k.z;
            O.s = QJL ? __builtin_amdgcn_raw_buffer_load_b32(rs1, o1s, rel * og.r1s, KV_NT) : 0u;
            const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(rv1, o1v, rel * og.r1v, KV_NT);
            O.v[0] = v.x, O.v[1] = v.y, O.v[2] = v.z;
            O.kn = __builtin_amdgcn_raw_buffer_load_b16(rkn1, o1n, rel * 2, KV_NT);
            O.kr = QJL ? __builtin_amdgcn_raw_buffer_load_b16(rkr1, o1n, rel * 2, KV_NT) : 0u;
            O.vn = __builtin_amdgcn_raw_buffer_load_b16(rvn1, o1n, rel * 2, KV_NT);
        }
    };
    auto load_k = [&](Kd& B, int rel_) {
        const int rel = __builtin_amdgcn_readfirstlane(rel_);  // scalar block offset
        if constexpr (SPL) {
            // KB + 1 dwords from the one holding the lane's first byte
            if constexpr (KB == 1) {
                const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rk, ko, rel * krow, KV_NT);
                B.kw[0] = x.x, B.kw[1] = x.y;
            } else if constexpr (KB == 2) {
                const u32x3 x = __builtin_amdgcn_raw_buffer_load_b96(rk, ko, rel * krow, KV_NT);
                B.kw[0] = x.x, B.kw[1] = x.y, B.kw[2] = x.z;
            } else {
                const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rk, ko, rel * krow, KV_NT);
                B.kw[0] = x.x, B.kw[1] = x.y, B.kw[2] = x.z, B.kw[3] = x.w;
                if constexpr (KB == 4) B.kw[4] = __builtin_amdgcn_raw_buffer_load_b32(rk, ko + 16, rel * krow, KV_NT);
            }
        } else if constexpr (KB == 1) {
            B.kw[0] = __builtin_amdgcn_raw_buffer_load_b32(rk, ko, rel * KROW, KV_NT);
        } else if constexpr (KB == 2) {
            const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rk, ko, rel * KROW, KV_NT);
            B.kw[0] = w.x, B.kw[1] = w.y;
        } else if constexpr (KB == 3) {
            const u32x3 w = __builtin_amdgcn_raw_buffer_load_b96(rk, ko, rel * KROW, KV_NT);
            B.kw[0] = w.x, B.kw[1] = w.y, B.kw[2] = w.z;
        } else {
            const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rk, ko, rel * KROW, KV_NT);
            B.kw[0] = w.x, B.kw[1] = w.y, B.kw[2] = w.z, B.kw[3] = w.w;
        }
        if constexpr (QJL) {
            if constexpr (SPL) {
                const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rs, so, rel * srow, KV_NT);
                B.sw[0] = x.x, B.sw[1] = x.y;
            } else {
                B.sw[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, so, rel * (D / 8), KV_NT);
            }
            B.kr = __builtin_amdgcn_raw_buffer_load_b16(rkr, no, rel * 2, KV_NT);
        } else {
#pragma unroll
            for (int i = 0; i < (SPL ? 2 : 1); ++i) B.sw[i] = 0u;
            B.kr = 0u;
        }
        B.kn = __builtin_amdgcn_raw_buffer_load_b16(rkn, no, rel * 2, KV_NT);
        B.vn = __builtin_amdgcn_raw_buffer_load_b16(rvn, no, rel * 2, KV_NT);
    };
    auto load_v = [&](Vd& B, int rel_) {
        const int rel = __builtin_amdgcn_readfirstlane(rel_);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if constexpr (SPL) {
                const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rv, vo + 4 * r * vrow, rel * vrow, KV_NT);
                B.vw[2 * r] = x.x, B.vw[2 * r + 1] = x.y;
            } else {
                B.vw[r] = __builtin_amdgcn_raw_buffer_load_b32(rv, vo + 4 * r * VROW, rel * VROW, KV_NT);
            }
        }
    };

    // blocks of this wave: wave, wave + NW, ... (scalar count)
    const int first = wave * BLK;
    const int nb = first < nt ? (nt - first + STEP - 1) / STEP : 0;
    // NSET of this wave's blocks in flight: block i is processed from register set i mod NSET,
    // which is then refilled with block i + NSET, so the sets rotate without copies and a load
    // has NSET - 1 blocks of processing to arrive in.  The refills are unconditional (past the
    // range the buffer loads return zeros and read no memory): with a load count that depends
    // on the path, the compiler's counter waits assume the fewest loads outstanding and block
    // i's first wait would also wait for block i + 1.  For the same reason the load order is
    // pinned with scheduling barriers here as in the loop: the waits at the loop head hold for
    // both ways in, and first loads issued in another order would force a wait for all of them.
    constexpr int NSET = Cfg<VB, GC, QJL, SPL>::NSET;
    constexpr int NB = Cfg<VB, GC, QJL, SPL>::NB;
    static_assert(NSET % NB == 0, "register sets come in whole steps");
    Kd kset[NSET];
    Vd vset[NSET];
    static_assert(!SPL || (NSET == 2 && NB == 1), "two-group layers: group 1's loads serve the two blocks of a round");
    OdT oset[2];  // two-group layers: rounds of even / odd parity

    // ------------------------------------------------------------ prologue
    // phase 1: codebooks and the group's q-side products (every split workgroup of the group
    // computes them: the mat-vecs on the matrix cores from L2-resident R_k and S, cheaper than
    // a separate launch ahead of the split pass)
    uint32_t* img = reinterpret_cast<uint32_t*>(sm.u.pro.img);
    // the products' operands are loaded first, then the codebook entries (unconditionally, in
    // range; only the tables below use them) and the first blocks of the token loop
    // (PRO_SETS register sets before the products, the rest after them), whose HBM latency the
    // rest of the prologue covers
    float ck_e, cv_e;
    float c1k_e = 0.0f, c1v_e = 0.0f;  // group 1's codebooks (two-group layers), entry tid
    // int8 keys: the key codebook in fixed point, |Ck| 2^E < 2^15 (wave-uniform scalar loads)
    int E = 0;
    if constexpr (KI8) {
        float cmax = 0.0f;
#pragma unroll
        for (int c = 0; c < (1 << KB); ++c) cmax = fmaxf(cmax, fabsf(Ck[c]));
        int e = 0;
        if (cmax > 0.0f) (void)frexpf(cmax, &e);  // cmax < 2^e
        E = 15 - e;
    }
    constexpr int PRO_SETS = Cfg<VB, GC, QJL, SPL>::PRO_SETS;
    image_products<QJL, GC, NW, KI8, (GC == 1 || SPL)>(q, G, bh0, Rk, S, c_mse, sm.u.pro.ps, img, sm.u.pro.qst[wave], wave,
                                                       lane, SPL ? og.d0 : D, [&] {
        ck_e = Ck[tid & ((1 << KB) - 1)];
        cv_e = Cv[tid & ((1 << VB) - 1)];
        if constexpr (SPL) {
            if (tid < (1 << og.b1k)) c1k_e = og.Ck1[tid];
            if (tid < (1 << og.b1v)) c1v_e = og.Cv1[tid];
        }
#pragma unroll
        for (int s = 0; s < PRO_SETS; ++s) {
            load_k(kset[s], first + s * STEP), load_v(vset[s], first + s * STEP);
            if (s == 0) load_o(oset[0], first);
            __builtin_amdgcn_sched_barrier(0);
        }
    });
#pragma unroll
    for (int s = PRO_SETS; s < NSET; ++s) {
        load_k(kset[s], first + s * STEP), load_v(vset[s], first + s * STEP);
        if (s == 0) load_o(oset[0], first);  // rounds 0 and 1 (two blocks each)
        __builtin_amdgcn_sched_barrier(0);
    }
    load_o(oset[1], first + NSET * STEP);
    __builtin_amdgcn_sched_barrier(0);
    // pair tables from the codebook entries in the lanes (lane l holds Ck[l mod 2^KB] and
    // Cv[l mod 2^VB]; ds_bpermute), four copies of an entry per 16-byte write, by the older half
    // of the waves: they finish their products first and wait at the barrier below for the
    // younger ones anyway.  Every loop runs whole waves (strides and bounds are multiples of
    // 64), so every lane takes part in each permute.
    if (wave < NW / 2) {
        const auto from_lane = [](uint32_t v, int l) {
            return (uint32_t)__builtin_amdgcn_ds_bpermute(l << 2, (int)v);
        };
        constexpr int QPE = TCOPIES / 4;  // 16-byte writes per entry and table
        uint4* tab4 = reinterpret_cast<uint4*>(&sm.tab[0][0]);
        const uint32_t cvh = tq::f32_to_f16(cv_e);
        // entry e holds pair e mod 2^(2 VB) (byte windows: the byte's two spare bits ignored)
        constexpr int NV = (Sm::VWIN ? 256 : (1 << (2 * VB))) * QPE;
        for (int i = tid; i < (NV + 63) / 64 * 64; i += NT / 2) {
            const int e = i / QPE, qd = i % QPE;
            const int pr = e & ((1 << (2 * VB)) - 1);
            const uint32_t v = from_lane(cvh, pr & ((1 << VB) - 1)) | (from_lane(cvh, pr >> VB) << 16);
            if (i < NV) tab4[e * 16 + qd] = make_uint4(v, v, v, v);
        }
        if constexpr (KI8) {
            // (L0, L1) of Ck in one dword's low half: Ck 2^E = L0 + 256 L1, balanced digits
            const int ci = (int)rintf(ck_e * ldexpf(1.0f, E));
            const int l0 = ((ci + 128) & 255) - 128;
            const uint32_t limbs = (uint32_t)(l0 & 255) | ((uint32_t)(((ci - l0) >> 8) & 255) << 8);
            constexpr int NK = (Sm::KWIN ? 256 : (1 << (2 * KB))) * QPE;
            for (int i = tid; i < (NK + 63) / 64 * 64; i += NT / 2) {
                const int e = i / QPE, qd = i % QPE;
                const int pr = e & ((1 << (2 * KB)) - 1);
                const uint32_t v = from_lane(limbs, pr & ((1 << KB) - 1)) | (from_lane(limbs, pr >> KB) << 16);
                if (i < NK) tab4[e * 16 + 8 + qd] = make_uint4(v, v, v, v);
            }
        } else {
            const uint32_t ckp = pack_hilo(ck_e);
            constexpr int NK = (1 << (2 * KB)) * Sm::KC / 2;  // two copies of an entry per write
            for (int i = tid; i < (NK + 63) / 64 * 64; i += NT / 2) {
                const int e = i / (Sm::KC / 2);
                const uint32_t lo = from_lane(ckp, e & ((1 << KB) - 1)), hi = from_lane(ckp, e >> KB);
                if (i < NK) reinterpret_cast<uint4*>(&sm.ktab[0][0])[i] = make_uint4(lo, hi, lo, hi);
            }
        }
    }
    // the weight transpose starts zeroed: the loop writes only the halves and rows that hold
    // weights, the rest of the value MFMAs' A operand stays zero
    for (int i = tid; i < (int)(sizeof(sm.wt) / 4); i += NT) (&sm.wt[0][0][0][0])[i] = 0u;
    if constexpr (SPL) {
        if (tid < 256) sm.ol.ck[tid] = c1k_e, sm.ol.cv[tid] = c1v_e;
    }
    __syncthreads();
    // phase 2 (LDS only): the QJL limb image and the int8 key image (group 0's dims only), and
    // group 1's q-side values of a two-group layer
    const int d0 = SPL ? og.d0 : D;
    int G2 = 0, F = 0;
    if constexpr (QJL) G2 = qjl_image<GC, NT>(sm.u.pro.ps, img, tid, d0);
    if constexpr (KI8) F = key_image_i8<NT>(sm.u.pro.ps, img, tid, d0);
    // group 1 of a two-group layer: its code widths (constants with X1 > 0) and the widths whose
    // code pairs have tables
    const int b1k = X1 > 0 ? KB + X1 : og.b1k, b1v = X1 > 0 ? VB + X1 : og.b1v;
    const bool kpair = SPL && b1k <= 4, vpair = SPL && b1v <= (OD == 4 ? 5 : 4);
    if constexpr (SPL) {
        // q_rot of group 1's dims per head (zero past d1), the QJL sign-sum table (ts[h][s] =
        // sum of q_proj times the QJL scale over the dims whose bit is set in s, in ascending
        // order) and the code-pair tables (pair index = c0 + c1 2^b, as the two codes lie in
        // the row)
        constexpr int NH = R::NH;
        if (tid < NH * OD) {
            const int h = tid / OD, j = tid % OD;
            sm.ol.q1[h][j] = j < og.d1 ? sm.u.pro.ps.qr[h][d0 + j] : 0.0f;
        }
        for (int i = tid; i < (NH << OD); i += NT) {
            const int h = i >> OD, sg = i & ((1 << OD) - 1);
            float t = 0.0f;
            for (int j = 0; j < og.d1; ++j)
                if ((sg >> j) & 1) t += sm.u.pro.ps.qp[h][d0 + j] * og.cq1;
            sm.ol.ts[h][sg] = t;
        }
        if (kpair)
            for (int i = tid; i < (1 << (2 * b1k)); i += NT)
                sm.ol.tk[i] = make_float2(sm.ol.ck[i & ((1 << b1k) - 1)], sm.ol.ck[i >> b1k]);
        if (vpair)
            for (int i = tid; i < (1 << (2 * b1v)); i += NT)
                sm.ol.tv[i] = make_float2(sm.ol.cv[i & ((1 << b1v) - 1)], sm.ol.cv[i >> b1v]);
    }
    if constexpr (QJL || KI8 || SPL) __syncthreads();
    // phase 3: operands into registers.  A operands of the key-score MFMAs: int8 keys, lane
    // (row 4 h + s, g), MFMA j: digits of dims 32 g + 8 j .. + 7 (16 VGPRs); bf16 keys, lane
    // (n, g), MFMA j, VGPR r holds q_x[h][32 g + 4 j + r] twice (32 VGPRs).
    u32x4 qa[NKM];
#pragma unroll
    for (int j = 0; j < NKM; ++j) qa[j] = *reinterpret_cast<const u32x4*>(img + IMG_QA + (j * 64 + lane) * 4);
    // scores come out of the key MFMAs in units of kscale (int8: 2^-(F + E)) and are taken to
    // log2 units by an fma that is already there; the QJL term is scaled to the same units
    const float kscale = KI8 ? ldexpf(1.0f, -(F + E)) : 1.0f;
    // group 1 of a two-group layer, for lane group g's head: q_rot (log2 units) of dims d0 ..
    // d0 + OD - 1, zero past d1, so the codes read there add nothing; the sum of its q_proj
    // (times the QJL scale); the group's value sums o1, rescaled with the MFMA sums
    constexpr int OD_ = SPL ? OD : 1;
    float q1r[R::HPL][OD_], o1[R::HPL][OD_], sq1[R::HPL];
    const float ikscale = 1.0f / kscale;  // a power of two
#pragma unroll
    for (int i = 0; i < R::HPL; ++i) {
        sq1[i] = 0.0f;
        if constexpr (SPL) {
            const int h = R::HPL * g + i;
#pragma unroll
            for (int j = 0; j < OD; ++j) {
                q1r[i][j] = sm.ol.q1[h][j];
                o1[i][j] = 0.0f;
            }
            sq1[i] = sm.ol.ts[h][(1 << OD) - 1];
        }
    }
    // A operands of the QJL MFMAs: rows = (head, limb); MFMA jj, VGPR v, byte e <-> dim
    // 32 g + 4 jj + v + 8 e.
    u32x4 qj[R::NQJ][2];
    float sq[R::HPL];
    float qfix = 0.0f;  // QJL logit (in score units) per unit of sum_{s_d = 1} y_d
#pragma unroll
    for (int i = 0; i < R::HPL; ++i) sq[i] = 0.0f;
    if constexpr (QJL) {
#pragma unroll
        for (int set = 0; set < R::NQJ; ++set)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
                qj[set][jj] = *reinterpret_cast<const u32x4*>(img + IMG_QJ + ((set * 2 + jj) * 64 + lane) * 4);
        // sum_d q_proj s_d = 2 sum_{s_d = 1} q_proj - sum_d q_proj; sum_d y_d is the QJL MFMA
        // against a token whose sign bits are all set (the same arithmetic as every token's sum)
        qfix = ldexpf(c_qjl, 1 - G2 + (KI8 ? F + E : 0));
        u32x4 ones[2];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int v = 0; v < 4; ++v) ones[jj][v] = 0x01010101u << (4 * jj + v);
        i32x4 acc_all[R::NQJ];
#pragma unroll
        for (int set = 0; set < R::NQJ; ++set) {
            acc_all[set] = mfma_i8(qj[set][0], ones[0], i32x4{0, 0, 0, 0});
            acc_all[set] = mfma_i8(qj[set][1], ones[1], acc_all[set]);
        }
#pragma unroll
        for (int i = 0; i < R::HPL; ++i) sq[i] = qjl_combine<GC>(acc_all, i) * (0.5f * qfix);
    }
    // T2 over the prologue's area, once every wave holds its operands: entry e = T0 entry e / 4
    // (the pair in bits 2..7 of the byte)
    if constexpr (Sm::WIN) {
        __syncthreads();
        const uint4* tab4 = reinterpret_cast<const uint4*>(&sm.tab[0][0]);
        uint4* t24 = reinterpret_cast<uint4*>(&sm.u.t2[0][0]);
        for (int i = tid; i < 256 * 16; i += NT) {
            const int e = i >> 4, part = i & 15;  // parts 0..7 value copies, 8..15 int8 key copies
            if (part < 8 ? Sm::VWIN : Sm::KWIN) t24[i] = tab4[(e >> 2) * 16 + part];
        }
        __syncthreads();
    }

    // per-lane softmax state (heads of this lane group) and value accumulators.  The reference
    // maximum m_ref tracks max(score + e_v) - WEXP0, e_v = the biased f16 exponent of the value
    // norm, so that the largest weight p |v| entering the fp16 value MFMAs is ~1 after a raise and
    // at most 2^(LAZY_MAX + 1) before the next: the fp16 weights neither overflow nor lose their
    // leading bits, whatever the value norms.
    float m_ref[R::HPL], s_lane[R::HPL], m_thr[R::HPL];
#pragma unroll
    for (int i = 0; i < R::HPL; ++i) m_ref[i] = NEG_INF, s_lane[i] = 0.0f, m_thr[i] = NEG_INF;
    // one set of value accumulators per block of a step (independent MFMA chains)
    f32x4 acc_v[NB][4];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int m = 0; m < 4; ++m) acc_v[b][m] = f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t plane = 4u * (uint32_t)(lane & (TCOPIES - 1));        // value copy: +4 c
    const uint32_t kplane = KI8 ? 128u + plane : 8u * (uint32_t)(lane & (Sm::KC - 1));  // key copy
    constexpr int KSHIFT = KI8 ? 8 : (Sm::KC == 32 ? 8 : 7);  // log2 bytes per key-table entry row
    // byte-window lookups: the copy offsets with byte 2 = 1 (T2 lies 64 KB above T0)
    const uint32_t kwin = kplane | 0x10000u, vwin = plane | 0x10000u;
    static_assert(!Sm::WIN || offsetof(Sm, u) == offsetof(Sm, tab) + 65536, "T2 = T0 + 64 KB");
    const char* const tb0 = reinterpret_cast<const char*>(&sm) + offsetof(Sm, tab);
    // the weight of token n = 4 i + k lands in dword i of lane group k's slots
    const int wslot = 4 * (n & 3) + (n >> 2);

    // One step: NB blocks of this wave (register sets s0 .. s0 + NB - 1, blocks rel0, rel0 + STEP,
    // ...) through every stage together, so each stage has NB independent chains of lookups and
    // MFMAs to interleave.  Blocks past the range have all their tokens masked.
    //   scores   key-score and QJL MFMAs, then the scores (in units of kscale) of token n for this
    //            lane's heads, -inf past the range;
    //   raise    (rare, wave-uniform) the lazy reference maximum raised, partial sums and value
    //            accumulators rescaled;
    //   weights  p |v| of token n in fp16 into the value MFMAs' A operand, transposed through
    //            this wave's LDS rows (one wave's LDS accesses execute in order and the compiler
    //            keeps the may-alias writes and reads of wt in program order, so no fence is
    //            needed): row vrow(h, p), dword i of lane group k holds token 4 i + k's weight in
    //            half p;
    //   values   4 fp16 MFMAs per block, MFMA u over the dim pairs (8 c + 2 u, 8 c + 2 u + 1) of
    //            column c; lane (c, k) supplies tokens 4 i + k, each one pair-table lookup
    //            returning the (even, odd) values in k-slot order.
    // The MFMA stages run at raised wave priority: a wave that reaches its matrix work issues
    // ahead of waves in their VALU/LDS phases, so the SIMD's MFMA and VALU work of different
    // waves overlap more.
    auto process = [&](int s0, int rel0, int op) {
        float lg[NB][R::HPL];
        float ev[NB];
        i32x4 acc_i[NB];
        f32x4 acc_k[NB], acc_k1[NB];
        i32x4 acc_q[NB][R::NQJ];
        // key code and sign words of token n (rows at any byte alignment realigned)
        uint32_t kwa[NB][KB], swa[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const Kd& B = kset[s0 + b];
            if constexpr (SPL) {
#pragma unroll
                for (int i = 0; i < KB; ++i) kwa[b][i] = __builtin_amdgcn_alignbit(B.kw[i + 1], B.kw[i], kalign);
                swa[b] = __builtin_amdgcn_alignbit(B.sw[1], B.sw[0], salign);
            } else {
#pragma unroll
                for (int i = 0; i < KB; ++i) kwa[b][i] = B.kw[i];
                swa[b] = B.sw[0];
            }
        }
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            acc_i[b] = i32x4{0, 0, 0, 0};
            acc_k[b] = f32x4{0.f, 0.f, 0.f, 0.f};
            acc_k1[b] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        if constexpr (KI8) {
            // 4 int8 MFMAs per block, dims 32 g + 8 j + 2 i + e: one 4-byte lookup per pair of codes
            // returns both codes' limbs in k-slot order.  3-bit codes: pair 4 j + i at bit 6 (4 j +
            // i) of the lane's 96 bits, a byte window of kw (bit 0 or 2 mod 8) or of kw >> 4 (4, 6)
            uint32_t ksh[NB][3];
            if constexpr (Sm::KWIN) {
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    ksh[b][0] = __builtin_amdgcn_alignbit(kwa[b][1], kwa[b][0], 4);
                    ksh[b][1] = __builtin_amdgcn_alignbit(kwa[b][2], kwa[b][1], 4);
                    ksh[b][2] = kwa[b][2] >> 4;
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    u32x4 bk;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        uint32_t off;
                        if constexpr (KB == 4) {
                            // code byte i of dword j: LDS byte offset 256 * byte + kplane in one v_perm
                            off = __builtin_amdgcn_perm(kwa[b][j], kplane, 0x0C0C0000u | ((4u + (uint32_t)i) << 8));
                        } else if constexpr (Sm::KWIN) {
                            off = win_off(kwa[b], ksh[b], KB * (8 * j + 2 * i), kwin);
                        } else {
                            off = field_x<2 * KB, 8>(kwa[b], KB * (8 * j + 2 * i)) | kplane;
                        }
                        bk[i] = *reinterpret_cast<const uint32_t*>(tb0 + off);
                    }
                    acc_i[b] = mfma_i8(qa[j], bk, acc_i[b]);
                }
            }
        } else {
            // 8 bf16 MFMAs per block over dims 32 g + 4 j + r; two chains per block
#pragma unroll
            for (int j = 0; j < 8; ++j) {
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    u32x4 bk;
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        const uint32_t off = field_x<2 * KB, KSHIFT>(kwa[b], (4 * j + 2 * p) * KB) | kplane;
                        const uint2 e = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(sm.ktab) + off);
                        bk[2 * p] = e.x;
                        bk[2 * p + 1] = e.y;
                    }
                    if (j & 1)
                        acc_k1[b] = mfma_bf16(qa[j], bk, acc_k1[b]);
                    else
                        acc_k[b] = mfma_bf16(qa[j], bk, acc_k[b]);
                }
            }
        }
        if constexpr (QJL) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                u32x4 bq[2];
#pragma unroll
                for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                    for (int v = 0; v < 4; ++v) bq[jj][v] = swa[b] & (0x01010101u << (4 * jj + v));
#pragma unroll
                for (int set = 0; set < R::NQJ; ++set) {
                    acc_q[b][set] = mfma_i8(qj[set][0], bq[0], i32x4{0, 0, 0, 0});
                    acc_q[b][set] = mfma_i8(qj[set][1], bq[1], acc_q[b][set]);
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
        // ---- group 1's score terms of a two-group layer (log2 units), token n, head g:
        // |k1| sum_j q_rot[j] Ck1[code_j] + |r1| (2 sum_{s_j = 1} q_proj[j] - sum_j q_proj[j])
        // group 1's data of token n of this block (NB = 1): the round's block s0 sits in lane
        // half s0 of oset[op]; rows realigned before the swap (both blocks share the shifts)
        uint32_t g1k[2] = {0u, 0u}, g1s = 0u, g1v[2] = {0u, 0u}, g1n = 0u, g1vn = 0u;
        if constexpr (SPL) {
            const Od& O = oset[op];
            const auto half = [&](uint32_t v) {
                const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
                return s0 == 0 ? (uint32_t)r[0] : (uint32_t)r[1];
            };
            g1k[0] = half(__builtin_amdgcn_alignbit(O.k[1], O.k[0], o1ksh));
            g1k[1] = half(__builtin_amdgcn_alignbit(O.k[2], O.k[1], o1ksh));
            g1s = half(O.s >> o1ssh);
            g1v[0] = half(__builtin_amdgcn_alignbit(O.v[1], O.v[0], o1vsh));
            g1v[1] = half(__builtin_amdgcn_alignbit(O.v[2], O.v[1], o1vsh));
            g1n = half(__builtin_amdgcn_perm(O.kr, O.kn, 0x05040100u));  // |k1| | |r1| << 16
            g1vn = half(O.vn);
        }
        float l1[NB][R::HPL];
        if constexpr (SPL) {
            const uint64_t m1k = (1ull << b1k) - 1u;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const uint64_t kb = ((uint64_t)g1k[1] << 32) | g1k[0];
                float a[R::HPL];
#pragma unroll
                for (int i = 0; i < R::HPL; ++i) a[i] = 0.0f;
                if (kpair) {
                    const uint64_t mp = (1ull << (2 * b1k)) - 1u;
#pragma unroll
                    for (int p = 0; p < OD / 2; ++p) {
                        const float2 e = sm.ol.tk[(uint32_t)((kb >> (2 * p * b1k)) & mp)];
#pragma unroll
                        for (int i = 0; i < R::HPL; ++i) {
                            a[i] = __builtin_fmaf(q1r[i][2 * p], e.x, a[i]);
                            a[i] = __builtin_fmaf(q1r[i][2 * p + 1], e.y, a[i]);
                        }
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < OD; ++j) {
                        const float c = sm.ol.ck[(uint32_t)((kb >> (j * b1k)) & m1k)];
#pragma unroll
                        for (int i = 0; i < R::HPL; ++i) a[i] = __builtin_fmaf(q1r[i][j], c, a[i]);
                    }
                }
                const float kn1 = tq::f16_to_f32(g1n & 0xFFFFu), kr1 = tq::f16_to_f32(g1n >> 16);
#pragma unroll
                for (int i = 0; i < R::HPL; ++i) {
                    const float qs = QJL ? sm.ol.ts[R::HPL * g + i][g1s & ((1u << OD) - 1u)] : 0.0f;
                    const float v = kn1 * a[i];
                    l1[b][i] = QJL ? __builtin_fmaf(kr1, __builtin_fmaf(2.0f, qs, -sq1[i]), v) : v;
                }
            }
        }
        // ---- scores
        bool over = false;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const Kd& B = kset[s0 + b];
            const int rel = rel0 + b * STEP;
            // valid tokens of the block: a scalar count, one compare per lane
            const int nvalid = __builtin_amdgcn_readfirstlane(nt - rel < BLK ? nt - rel : BLK);
            const bool valid = n < nvalid;
            // the f16 norms enter v_fma_mix_f32 as they are (no separate conversions)
            const float knf = tq::f16_to_f32(B.kn);
            const float krf = QJL ? tq::f16_to_f32(B.kr) : 0.0f;
            ev[b] = (float)__builtin_amdgcn_ubfe(B.vn, 10, 5);  // biased exponent of the value norm
#pragma unroll
            for (int i = 0; i < R::HPL; ++i) {
                float ksum;
                if constexpr (KI8) {
                    // sum_s 2^(8 s) row_s: pairs exact in int32 (|row_s| <= 2^22), then one fp32 rounding
                    const int lo = acc_i[b][0] + (acc_i[b][1] << 8), hi = acc_i[b][2] + (acc_i[b][3] << 8);
                    ksum = __builtin_fmaf((float)hi, 65536.0f, (float)lo);
                } else {
                    ksum = (acc_k[b][2 * i] + acc_k1[b][2 * i]) + (acc_k[b][2 * i + 1] + acc_k1[b][2 * i + 1]);
                }
                float v;
                if constexpr (QJL) {
                    const float qi = qjl_combine<GC>(acc_q[b], i);  // sum_d y_d s_d
                    v = __builtin_fmaf(knf, ksum, __builtin_fmaf(krf, __builtin_fmaf(qi, qfix, -sq[i]), 0.0f));
                } else {
                    v = knf * ksum;
                }
                if constexpr (SPL) v = __builtin_fmaf(l1[b][i], ikscale, v);
                lg[b][i] = valid ? v : NEG_INF;
                over |= __builtin_fmaf(lg[b][i], kscale, ev[b]) > m_thr[i];
            }
        }
        // ---- the lazy reference maximum raised (rare)
        if (__builtin_amdgcn_ballot_w64(over) != 0) {
#pragma unroll
            for (int i = 0; i < R::HPL; ++i) {
                float t = __builtin_fmaf(lg[0][i], kscale, ev[0]);
#pragma unroll
                for (int b = 1; b < NB; ++b) t = fmaxf(t, __builtin_fmaf(lg[b][i], kscale, ev[b]));
                const float mn = fmaxf(m_ref[i], row_max16(t) - WEXP0);
                const float a = m_ref[i] == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(m_ref[i] - mn);  // 1 if unchanged
                s_lane[i] *= a;
#pragma unroll
                for (int b = 0; b < NB; ++b) {
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        if constexpr (GC == 1) {
                            acc_v[b][m] *= a;  // the lane's four rows are its head's (two of them zero)
                        } else {
                            acc_v[b][m][2 * i] *= a;
                            acc_v[b][m][2 * i + 1] *= a;
                        }
                    }
                }
                if constexpr (SPL) {
#pragma unroll
                    for (int j = 0; j < OD; ++j) o1[i][j] *= a;
                }
                m_ref[i] = mn;
                m_thr[i] = mn + (WEXP0 + LAZY_MAX);
            }
        }
        // ---- weights
        u32x4 av[NB];
        float pv1[NB][R::HPL];  // group 1: p |v1| of token n, the lane's heads
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            uint32_t(*wt)[WROW] = sm.wt[wave][b];
            const float vnf = tq::f16_to_f32(kset[s0 + b].vn);  // invalid tokens have p = 0
#pragma unroll
            for (int i = 0; i < R::HPL; ++i) {
                const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(lg[b][i], kscale, -m_ref[i]));
                if constexpr (SPL) pv1[b][i] = p * tq::f16_to_f32(g1vn);
                s_lane[i] += p;
                const uint16_t w = (uint16_t)tq::f32_to_f16(__builtin_fmaf(vnf, p, 0.0f));
                const int h = R::HPL * g + i;
                reinterpret_cast<uint16_t*>(&wt[R::vrow(h, 0)][wslot])[0] = w;
                reinterpret_cast<uint16_t*>(&wt[R::vrow(h, 1)][wslot])[1] = w;
            }
            av[b] = *reinterpret_cast<const u32x4*>(&wt[n][4 * g]);
        }
        // ---- values
        __builtin_amdgcn_s_setprio(1);
        uint32_t ch[NB][4];  // the lane's chunk of each token, aligned to bit 0 (VB < 4)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t w = vset[s0 + b].vw[SPL ? 2 * i : i];
                if constexpr (SPL)
                    ch[b][i] = __builtin_amdgcn_alignbit(vset[s0 + b].vw[2 * i + 1], w, vsh);
                else if constexpr (VB == 3)
                    ch[b][i] = chunk3(w, vsh);
                else if constexpr (VB < 3)
                    ch[b][i] = w >> vsh;
                else
                    ch[b][i] = w;
            }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                u32x4 bv;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t off;
                    if constexpr (VB == 4) {
                        // code byte u: LDS byte offset 256 * byte + plane in one v_perm
                        off = __builtin_amdgcn_perm(ch[b][i], plane, 0x0C0C0000u | ((4u + (uint32_t)u) << 8));
                    } else if constexpr (Sm::VWIN) {
                        // pair u at bit 6 u of the chunk: byte windows of the chunk (u = 0, 3) or
                        // of chunk >> 4 (u = 1, 2)
                        const uint32_t chs = ch[b][i] >> 4;
                        off = win_off(&ch[b][i], &chs, 6 * u, vwin);
                    } else {
                        off = field_x<2 * VB, 8>(&ch[b][i], 2 * VB * u) | plane;
                    }
                    bv[i] = *reinterpret_cast<const uint32_t*>(tb0 + off);
                }
                acc_v[b][u] = mfma_f16(av[b], bv, acc_v[b][u]);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        // ---- group 1's value sums of a two-group layer: o1[j] += p |v1| Cv1[code_j]
        if constexpr (SPL) {
            const uint64_t m1v = (1ull << b1v) - 1u;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const uint64_t vb = ((uint64_t)g1v[1] << 32) | g1v[0];
                if (vpair) {
                    const uint64_t mp = (1ull << (2 * b1v)) - 1u;
#pragma unroll
                    for (int p = 0; p < OD / 2; ++p) {
                        const float2 e = sm.ol.tv[(uint32_t)((vb >> (2 * p * b1v)) & mp)];
#pragma unroll
                        for (int i = 0; i < R::HPL; ++i) {
                            o1[i][2 * p] = __builtin_fmaf(pv1[b][i], e.x, o1[i][2 * p]);
                            o1[i][2 * p + 1] = __builtin_fmaf(pv1[b][i], e.y, o1[i][2 * p + 1]);
                        }
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < OD; ++j) {
                        const float c = sm.ol.cv[(uint32_t)((vb >> (j * b1v)) & m1v)];
#pragma unroll
                        for (int i = 0; i < R::HPL; ++i) o1[i][j] = __builtin_fmaf(pv1[b][i], c, o1[i][j]);
                    }
                }
            }
        }
    };

    // (the first NSET blocks were issued in the prologue)
    if (nb > 0) {
        // whole rounds of NSET blocks, NB per step: up to NSET - 1 blocks past the range end the
        // wave's last round, and a wave-uniform branch skips a step whose first block is past it
        // (not the refill loads, which stay unconditional).  Skipping matters where a workgroup's
        // blocks do not divide evenly among its waves (C4: 128 blocks over 12 waves, -0.8 us per
        // call; C5 shape -1.4)
        // Two-group layers: two rounds per iteration, so that each round's group-1 register set
        // (refilled with the round two ahead once both its blocks are processed) has a fixed index.
        constexpr int RPI = SPL ? 2 : 1;  // rounds per iteration
        for (int i = 0; i < nb; i += RPI * NSET) {
#pragma unroll
            for (int rp = 0; rp < RPI; ++rp) {
#pragma unroll
                for (int s = 0; s < NSET; s += NB) {
                    const int rel = first + (i + rp * NSET + s) * STEP;
                    if (rel < nt) process(s, rel, rp);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        load_k(kset[s + b], rel + (NSET + b) * STEP), load_v(vset[s + b], rel + (NSET + b) * STEP);
                    __builtin_amdgcn_sched_barrier(0);
                }
                load_o(oset[rp], first + (i + rp * NSET + 2 * NSET) * STEP);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    // ------------------------------------------------------------ epilogue
    __syncthreads();  // the prologue area (read by every wave's phase 3) is reused below
    float s_row[R::HPL];
#pragma unroll
    for (int i = 0; i < R::HPL; ++i) s_row[i] = row_sum16(s_lane[i]);
    // lane (n, g) holds dims 8 n + 2 u + p of heads R::HPL g + i: accumulator u, register 2 p
    // (GC = 1; registers 1 and 3 are the zero rows) or 2 i + p (GC = 2)
#pragma unroll
    for (int i = 0; i < R::HPL; ++i) {
        const int h = R::HPL * g + i;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int r = GC == 1 ? 2 * p : 2 * i + p;
                float o = acc_v[0][u][r];
#pragma unroll
                for (int b = 1; b < NB; ++b) o += acc_v[b][u][r];
                sm.u.epi.o[wave][h][8 * n + 2 * u + p] = o;
            }
        }
        if constexpr (SPL) {
            // group 1's dims d0 .. D - 1 replace the MFMA sums there (which summed the codes
            // read past group 0's rows); the wave's LDS writes execute in program order
#pragma unroll
            for (int j = 0; j < OD; ++j) {
                const float t = row_sum16(o1[i][j]);
                if (n == 0 && j < og.d1) sm.u.epi.o[wave][h][og.d0 + j] = t;
            }
        }
        if (n == 0) {
            sm.u.epi.m[wave][h] = m_ref[i];
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
    const float *Rk, *S;
    float c_mse, c_qjl;
    const float *Ck, *Cv;
    float scale;
    int64_t tps;
    int n_split;
    float *po, *pml;
    Og og;  // two-group layers only
};

int cu_count() {
    static std::atomic<int64_t> cached[tq::MAX_DEVICES];
    return (int)tq::once_per_device(cached, 256, [](int dev) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
        return (int64_t)cus;
    });
}

template <int KB, int VB, bool QJL, int GC, int OD = 0, int X1 = 0>
int wgs_per_cu() {
    static std::atomic<int64_t> cached[tq::MAX_DEVICES];
    return (int)tq::once_per_device(cached, 1, [](int) {
        int o = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, split_kernel<KB, VB, QJL, GC, OD, X1>,
                                                         Cfg<VB, GC, QJL, (OD > 0)>::NT, 0) != hipSuccess ||
            o < 1)
            o = 1;
        return (int64_t)o;
    });
}

int choose_split(int groups, int64_t n_tokens, int target_wgs, int nw, int64_t* tokens_per_split) {
    const int64_t min_per_split = (int64_t)nw * BLK * 2;  // >= two blocks per wave
    const int64_t max_split = (n_tokens + min_per_split - 1) / min_per_split;
    int64_t want = (target_wgs + groups - 1) / groups;
    const int64_t cap_split = (MAX_WGS + groups - 1) / groups;
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

template <int KB, int VB, bool QJL, int GC, int OD = 0, int X1 = 0>
int launch_split(const SplitArgs& a, int groups, hipStream_t s, int* n_split_out, int64_t* tps_out) {
    constexpr bool SPL = OD > 0;
    const int target = wgs_per_cu<KB, VB, QJL, GC, OD, X1>() * cu_count();
    int64_t tps;
    const int ns = choose_split(groups, a.n_tokens > 0 ? a.n_tokens : 1, target, Cfg<VB, GC, QJL, SPL>::NW, &tps);
    *n_split_out = ns;
    *tps_out = tps;
    // a workgroup's range stays below 2^24 tokens: its byte ranges fit the 31-bit buffer
    // descriptors and its token offsets fit 32-bit scalars
    if (tps >= ((int64_t)1 << 24)) return TQ_ERR_UNSUPPORTED;
    if (a.po == nullptr) return TQ_OK;  // sizing query only
    hipLaunchKernelGGL((split_kernel<KB, VB, QJL, GC, OD, X1>), dim3(ns, groups), dim3(Cfg<VB, GC, QJL, SPL>::NT), 0, s,
                       a.q, a.q_heads, a.kv_heads, a.G, a.seq_starts, a.seq_lens, a.n_tokens, a.cap, a.kc, a.kn, a.ks,
                       a.kr, a.vc, a.vn, a.Rk, a.S, a.c_mse, a.c_qjl, a.Ck, a.Cv, a.scale, tps, ns, a.po, a.pml, a.og);
    return TQ_OK;
}

// Two-group layers on the split kernel (group 1 at most OD1 channels): group 0's bit widths as
// for a one-group layer, OD = 4 or 8 per-lane dims, group 1's widths one bit wider (the
// reference's default) as constants, or with up to 4 heads per KV head any widths at run time
// (the host sends 5-8 heads with other widths to the fp32 kernel).
constexpr bool og_wide_ok(int kb, int vb, bool qjl) { return !(kb == 3 && vb == 3 && !qjl); }

template <int KB, int VB, bool QJL>
int launch_split_og(int G, const SplitArgs& a, int groups, hipStream_t s, int* ns, int64_t* tps) {
    const bool x1 = a.og.b1k == KB + 1 && a.og.b1v == VB + 1;
    const bool od4 = a.og.d1 <= 4;
    if (G > 4) {
        // 3-bit Q_mse at 5-8 heads: the byte-window tables leave no LDS for the outlier group
        if constexpr (og_wide_ok(KB, VB, QJL)) {
            if (!x1) return TQ_ERR_UNSUPPORTED;
            return od4 ? launch_split<KB, VB, QJL, 2, 4, 1>(a, groups, s, ns, tps)
                       : launch_split<KB, VB, QJL, 2, OD1, 1>(a, groups, s, ns, tps);
        } else {
            return TQ_ERR_UNSUPPORTED;
        }
    }
    if (od4)
        return x1 ? launch_split<KB, VB, QJL, 1, 4, 1>(a, groups, s, ns, tps)
                  : launch_split<KB, VB, QJL, 1, 4, 0>(a, groups, s, ns, tps);
    return x1 ? launch_split<KB, VB, QJL, 1, OD1, 1>(a, groups, s, ns, tps)
              : launch_split<KB, VB, QJL, 1, OD1, 0>(a, groups, s, ns, tps);
}

int dispatch_og(int value_bits, int has_qjl, int G, const SplitArgs& a, int groups, hipStream_t s, int* ns,
                int64_t* tps) {
    if (has_qjl) {
        switch (value_bits) {
            case 2: return launch_split_og<1, 2, true>(G, a, groups, s, ns, tps);
            case 3: return launch_split_og<2, 3, true>(G, a, groups, s, ns, tps);
            default: return launch_split_og<3, 4, true>(G, a, groups, s, ns, tps);
        }
    }
    switch (value_bits) {
        case 1: return launch_split_og<1, 1, false>(G, a, groups, s, ns, tps);
        case 2: return launch_split_og<2, 2, false>(G, a, groups, s, ns, tps);
        case 3: return launch_split_og<3, 3, false>(G, a, groups, s, ns, tps);
        default: return launch_split_og<4, 4, false>(G, a, groups, s, ns, tps);
    }
}

template <int KB, int VB, bool QJL>
int launch_split_g(int G, const SplitArgs& a, int groups, hipStream_t s, int* ns, int64_t* tps) {
    if (G <= 4) return launch_split<KB, VB, QJL, 1>(a, groups, s, ns, tps);
    if (G <= 8) return launch_split<KB, VB, QJL, 2>(a, groups, s, ns, tps);
    return TQ_ERR_UNSUPPORTED;
}

int dispatch(int value_bits, int has_qjl, int G, const SplitArgs& a, int groups, hipStream_t s, int* ns,
             int64_t* tps) {
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
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------------ channel-group layers
// Decode attention over a layer whose channels are quantized in groups (the outlier split:
// reference runtime/packed_qmse_cache.py:437-515; its fused kernel refuses such layers,
// runtime/triton_kernels.py:252-253).  Group g has d_g channels, its own codebooks, bit
// widths (1..8), norms and QJL sketch, in rows of ceil(d_g b / 8) bytes.  Stacking the
// groups' channel-space matrices gives one D x D matrix per role whose row J < d_0 belongs to
// group 0 and row J >= d_0 to group 1, so q R^T, q S^T and the final un-rotation are single
// mat-vecs over one D-dimensional rotated space, and the partials (o[D], m, s) have the
// split kernel's format: merge_kernel finishes the call with the stacked value matrix.
//
// group_attn_kernel: grid (n_split, batch * kv_heads), GT threads; per tile of GT tokens
//   stage     the tile's key code and sign rows (then its value rows) into LDS with dword
//             buffer loads: rows are not dword aligned, so codes are read from LDS at any
//             bit offset (two dwords and an alignbit);
//   scores    thread = token: sum over the group's codes of q_rot[J] C_g[code] times the
//             token's group norm, plus the QJL term rho_g (2 sum_{s=1} q_proj - sum q_proj),
//             for all heads of the GQA group at once (q_rot / q_proj broadcast from LDS);
//   softmax   base 2, running maximum per head over the tiles;
//   values    thread = (rotated dim J, token parity): o[J] += p |v_g| Cv_g[code_J].
// Everything is fp32 VALU.

constexpr int GT = 256;  // tokens per tile = threads per workgroup
constexpr int NGRP = 2;  // channel groups per layer (at most)
constexpr int GMAXC = 256;

struct GroupAttnArgs {
    const uint16_t* q;
    int q_heads, kv_heads, G, n_groups;
    const int32_t *seq_starts, *seq_lens;
    int64_t n_tokens, cap;
    const uint8_t* kc[NGRP];
    const uint16_t* kn[NGRP];
    const uint8_t* ks[NGRP];
    const uint16_t* kr[NGRP];
    const uint8_t* vc[NGRP];
    const uint16_t* vn[NGRP];
    int d[NGRP], j0[NGRP], kb[NGRP], vb[NGRP];
    int rk[NGRP], rs[NGRP], rv[NGRP];  // row bytes: key codes, signs, value codes
    const float* Ck[NGRP];
    const float* Cv[NGRP];
    float cq[NGRP];  // sqrt(pi/2)/d_g * scale * log2 e
    float cs;        // scale * log2 e
    const float *Mk, *Ms;  // stacked channel-space key / QJL matrices [D][D]
    int kst[NGRP], sst[NGRP], vst[NGRP];  // LDS dword offsets of each staged row array
    int64_t tps;
    int n_split;
    float *po, *pml;
};

// Staged dwords for one tile of rows of r bytes (the tile's first row may start mid-dword).
__host__ __device__ inline int stage_dwords(int r) { return (GT * r + 3) / 4 + 2; }

// Bits [bit, bit + n) (n <= 8) of the LDS dword array w.
__device__ __forceinline__ uint32_t lds_bits(const uint32_t* w, uint32_t bit, uint32_t n) {
    const uint32_t i = bit >> 5;
    return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(w[i + 1], w[i], bit & 31), 0, n);
}

// Copies bytes [t0 r, (t0 + GT) r) of one (batch row, KV head)'s row array into LDS dwords
// dst[0..], starting with the dword that holds byte t0 r; returns that byte's offset in dst.
// `limit` = the array's bytes (cap r): dwords inside it are single loads, the last partial
// dword is assembled from byte loads and nothing past it is read.
__device__ __forceinline__ uint32_t stage_rows(uint32_t* dst, const uint8_t* base, uint32_t limit, uint32_t t0, int r,
                                               int tid) {
    const __amdgpu_buffer_rsrc_t rs = rsrc(base, limit);
    const uint32_t b0 = t0 * (uint32_t)r;
    const uint32_t a0 = b0 & ~3u;
    const uint32_t n = (b0 + GT * (uint32_t)r - a0 + 3) >> 2;
    const uint32_t whole = (limit - a0) >> 2;  // dwords wholly inside the array (a0 <= b0 < limit)
    const uint32_t nf = n < whole ? n : whole;
    // independent loads, several in flight per thread
#pragma unroll 8
    for (uint32_t i = tid; i < nf; i += GT) dst[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, a0 + 4 * i, 0, 0);
    for (uint32_t i = nf + tid; i < n; i += GT) {  // the array's last partial dword, then zeros
        const uint32_t off = a0 + 4 * i;
        uint32_t v = 0;
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k)
            if (off + k < limit) v |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, off + k, 0, 0) << (8 * k);
        dst[i] = v;
    }
    return b0 - a0;
}

template <int GH, bool QJL>
__global__ __launch_bounds__(GT) void group_attn_kernel(GroupAttnArgs a) {
    extern __shared__ uint32_t stage[];
    __shared__ float qr[D][GH];       // q R_k^T (stacked), times scale log2 e
    __shared__ float qp[D][GH];       // q S^T (stacked), times the QJL scale of J's group
    __shared__ float sqp[NGRP][GH];   // sum of qp over each group
    __shared__ float ck[NGRP][GMAXC];
    __shared__ float cv[NGRP][GMAXC];
    __shared__ float wp[GT][GH];      // softmax weights per (token, head): one broadcast read per token
    __shared__ float vns[NGRP][GT];   // value norms of the tile's tokens (0 when invalid)
    __shared__ float red[GT / 64][GH];
    __shared__ float ored[GH][D];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, grp = blockIdx.y;
    const int b = grp / a.kv_heads, hk = grp % a.kv_heads;
    const int G = a.G, ng = a.n_groups;

    // ---- codebooks and the q-side mat-vecs
    for (int g = 0; g < ng; ++g) {
        for (int i = tid; i < (1 << a.kb[g]); i += GT) ck[g][i] = a.Ck[g][i];
        for (int i = tid; i < (1 << a.vb[g]); i += GT) cv[g][i] = a.Cv[g][i];
    }
    // the group's queries in fp32, channel-major (in wp, which the tiles overwrite later)
    float(*qsh)[GH] = reinterpret_cast<float(*)[GH]>(&wp[0][0]);
    for (int i = tid; i < GH * D; i += GT) {
        const int h = i / D, c = i % D;
        qsh[c][h] = h < G ? tq::bf16_to_f32(a.q[((size_t)b * a.q_heads + (size_t)hk * G + h) * D + c]) : 0.0f;
    }
    __syncthreads();
    // thread (matrix, rotated dim J): row J of M_k (or M_s) against every head, 16-byte row reads
    if (tid < (QJL ? 2 : 1) * D) {
        const int which = tid / D, J = tid % D;
        const float4* m4 = reinterpret_cast<const float4*>((which ? a.Ms : a.Mk) + (size_t)J * D);
        float acc[GH];
#pragma unroll
        for (int h = 0; h < GH; ++h) acc[h] = 0.0f;
#pragma unroll 2
        for (int c4 = 0; c4 < D / 4; ++c4) {
            const float4 m = m4[c4];
            const float mv[4] = {m.x, m.y, m.z, m.w};
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int h = 0; h < GH; ++h) acc[h] = __builtin_fmaf(qsh[4 * c4 + k][h], mv[k], acc[h]);
        }
        const int g = (ng > 1 && J >= a.j0[1]) ? 1 : 0;
#pragma unroll
        for (int h = 0; h < GH; ++h) {
            if (which) qp[J][h] = acc[h] * a.cq[g];
            else qr[J][h] = acc[h] * a.cs;
        }
    }
    __syncthreads();
    if (QJL && tid < NGRP * GH) {
        const int g = tid / GH, h = tid % GH;
        float s = 0.0f;
        if (g < ng)
            for (int J = a.j0[g]; J < a.j0[g] + a.d[g]; ++J) s += qp[J][h];
        sqp[g][h] = s;
    }

    // ---- this workgroup's valid token range
    const int64_t t_begin = (int64_t)split * a.tps;
    const int64_t t_end = t_begin + a.tps < a.n_tokens ? t_begin + a.tps : a.n_tokens;
    const int64_t r_lo = a.seq_starts ? (int64_t)a.seq_starts[b] : 0;
    const int64_t r_hi = a.seq_lens ? (int64_t)a.seq_lens[b] : a.n_tokens;
    const int64_t lo = t_begin > r_lo ? t_begin : r_lo;
    const int64_t hi = t_end < r_hi ? t_end : r_hi;

    float M[GH], s_acc[GH], o_acc[GH];
#pragma unroll
    for (int h = 0; h < GH; ++h) {
        M[h] = NEG_INF;
        s_acc[h] = 0.0f;
        o_acc[h] = 0.0f;
    }
    const int vJ = tid & (D - 1), vpar = tid >> 7;
    const int vg = (ng > 1 && vJ >= a.j0[1]) ? 1 : 0;
    const int vj = vJ - a.j0[vg];
    const int64_t gbase = (int64_t)grp * a.cap;

    for (int64_t t0 = lo; t0 < hi; t0 += GT) {
        const int nv = (int)(hi - t0 < GT ? hi - t0 : GT);
        const bool valid = tid < nv;
        const int64_t tok = t0 + tid;
        // ---- stage key codes and signs
        uint32_t koff[NGRP], soff[NGRP];
        for (int g = 0; g < ng; ++g) {
            koff[g] = stage_rows(stage + a.kst[g], a.kc[g] + gbase * a.rk[g], (uint32_t)(a.cap * a.rk[g]), (uint32_t)t0,
                                 a.rk[g], tid);
            if (QJL)
                soff[g] = stage_rows(stage + a.sst[g], a.ks[g] + gbase * a.rs[g], (uint32_t)(a.cap * a.rs[g]),
                                     (uint32_t)t0, a.rs[g], tid);
        }
        __syncthreads();
        // ---- scores, thread = token
        float l[GH];
#pragma unroll
        for (int h = 0; h < GH; ++h) l[h] = valid ? 0.0f : NEG_INF;
        if (valid) {
            for (int g = 0; g < ng; ++g) {
                const uint32_t* ks = stage + a.kst[g];
                const uint32_t bit0 = (koff[g] + (uint32_t)tid * a.rk[g]) * 8;
                const uint32_t kb = a.kb[g];
                float acc[GH];
#pragma unroll
                for (int h = 0; h < GH; ++h) acc[h] = 0.0f;
#pragma unroll 4
                for (int j = 0; j < a.d[g]; ++j) {
                    const float c = ck[g][lds_bits(ks, bit0 + j * kb, kb)];
                    const int J = a.j0[g] + j;
#pragma unroll
                    for (int h = 0; h < GH; ++h) acc[h] = __builtin_fmaf(qr[J][h], c, acc[h]);
                }
                const float nk = tq::f16_to_f32(a.kn[g][gbase + tok]);
#pragma unroll
                for (int h = 0; h < GH; ++h) l[h] = __builtin_fmaf(nk, acc[h], l[h]);
                if (QJL) {
                    const uint32_t* ss = stage + a.sst[g];
                    const uint32_t sb0 = (soff[g] + (uint32_t)tid * a.rs[g]) * 8;
#pragma unroll
                    for (int h = 0; h < GH; ++h) acc[h] = 0.0f;
                    for (int j0 = 0; j0 < a.d[g]; j0 += 32) {
                        const uint32_t i = (sb0 + j0) >> 5;
                        uint32_t w = __builtin_amdgcn_alignbit(ss[i + 1], ss[i], (sb0 + j0) & 31);
                        const int n = a.d[g] - j0 < 32 ? a.d[g] - j0 : 32;
#pragma unroll 4
                        for (int jj = 0; jj < n; ++jj, w >>= 1) {
                            const float f = (float)(w & 1u);
                            const int J = a.j0[g] + j0 + jj;
#pragma unroll
                            for (int h = 0; h < GH; ++h) acc[h] = __builtin_fmaf(f, qp[J][h], acc[h]);
                        }
                    }
                    const float rn = tq::f16_to_f32(a.kr[g][gbase + tok]);
#pragma unroll
                    for (int h = 0; h < GH; ++h) l[h] = __builtin_fmaf(rn, 2.0f * acc[h] - sqp[g][h], l[h]);
                }
            }
        }
        // ---- tile maximum per head
#pragma unroll
        for (int h = 0; h < GH; ++h) {
            float m = l[h];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
            if (lane == 0) red[wave][h] = m;
        }
        __syncthreads();  // key stage consumed, tile maxima visible
        // ---- stage value codes; weights and value norms of the thread's token
        uint32_t voff[NGRP];
        for (int g = 0; g < ng; ++g)
            voff[g] = stage_rows(stage + a.vst[g], a.vc[g] + gbase * a.rv[g], (uint32_t)(a.cap * a.rv[g]),
                                 (uint32_t)t0, a.rv[g], tid);
        float alpha[GH];
#pragma unroll
        for (int h = 0; h < GH; ++h) {
            float m = red[0][h];
#pragma unroll
            for (int w = 1; w < GT / 64; ++w) m = fmaxf(m, red[w][h]);
            const float nm = fmaxf(M[h], m);
            alpha[h] = nm == NEG_INF ? 1.0f : __builtin_amdgcn_exp2f(M[h] - nm);
            M[h] = nm;
            const float p = valid ? __builtin_amdgcn_exp2f(l[h] - nm) : 0.0f;
            s_acc[h] = __builtin_fmaf(s_acc[h], alpha[h], p);
            wp[tid][h] = p;
        }
        for (int g = 0; g < ng; ++g) vns[g][tid] = valid ? tq::f16_to_f32(a.vn[g][gbase + tok]) : 0.0f;
        __syncthreads();
        // ---- values, thread = (rotated dim, token parity)
        {
            const uint32_t* vs = stage + a.vst[vg];
            const uint32_t vb = a.vb[vg], rv = a.rv[vg];
            const uint32_t bitj = voff[vg] * 8 + (uint32_t)vj * vb;
#pragma unroll
            for (int h = 0; h < GH; ++h) o_acc[h] *= alpha[h];
#pragma unroll 4
            for (int tt = vpar; tt < nv; tt += 2) {
                const float v = vns[vg][tt] * cv[vg][lds_bits(vs, bitj + (uint32_t)tt * rv * 8, vb)];
#pragma unroll
                for (int h = 0; h < GH; ++h) o_acc[h] = __builtin_fmaf(wp[tt][h], v, o_acc[h]);
            }
        }
        __syncthreads();  // stage, wp and vns are rewritten by the next tile
    }

    // ---- partials (o[D], m, s) per query head
#pragma unroll
    for (int h = 0; h < GH; ++h) {
        float s = s_acc[h];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
        if (lane == 0) red[wave][h] = s;
    }
    if (vpar) {
#pragma unroll
        for (int h = 0; h < GH; ++h) ored[h][vJ] = o_acc[h];
    }
    __syncthreads();
    if (!vpar) {
        for (int h = 0; h < G; ++h) {
            const size_t pidx = ((size_t)b * a.q_heads + (size_t)hk * G + h) * a.n_split + split;
            a.po[pidx * D + vJ] = o_acc[h] + ored[h][vJ];
            if (vJ == 0) {
                float s = 0.0f;
#pragma unroll
                for (int w = 0; w < GT / 64; ++w) s += red[w][h];
                a.pml[pidx * 2 + 0] = M[h];
                a.pml[pidx * 2 + 1] = s;
            }
        }
    }
}

int group_split(int groups, int64_t n_tokens, int64_t* tps) {
    const int64_t max_split = (n_tokens + GT - 1) / GT;
    int64_t ns = (MAX_WGS + groups - 1) / groups;
    if (ns > max_split) ns = max_split;
    if (ns < 1) ns = 1;
    int64_t per = (n_tokens + ns - 1) / ns;
    per = (per + GT - 1) / GT * GT;
    if (per < GT) per = GT;
    *tps = per;
    const int64_t got = (n_tokens + per - 1) / per;
    return (int)(got > 0 ? got : 1);
}

}  // namespace

extern "C" size_t tq_decode_attention_workspace_bytes(int batch, int q_heads, int kv_heads, int dim,
                                                      int64_t max_tokens) {
    if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || dim != D || max_tokens < 0) return 0;
    // any n_tokens yields at most ceil(MAX_WGS / groups) splits
    const int64_t groups = (int64_t)batch * kv_heads;
    const int bound = (int)((MAX_WGS + groups - 1) / groups);
    return ws_layout(batch, q_heads, bound).total;
}

namespace {
// The body of tq_decode_attention and tq_decode_attention_noalloc: validation, split sizing,
// the split pass and the merge, with the partials at `workspace`.
int decode_attention_impl(const uint16_t* q, int batch, int q_heads, int kv_heads, int dim,
                          const int32_t* seq_starts, const int32_t* seq_lens, int64_t n_tokens, int64_t cap,
                          const uint8_t* k_codes, const uint16_t* k_norms, const uint8_t* k_signs,
                          const uint16_t* k_rnorms, const uint8_t* v_codes, const uint16_t* v_norms, int key_bits,
                          int value_bits, int has_qjl, const float* key_rotation, const float* key_centers,
                          const float* qjl, const float* value_rotation, const float* value_centers, float scale,
                          float* out_f32, uint16_t* out_bf16, float* lse_out, void* workspace,
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
    if (!aligned16(q) || (k_codes && !aligned16(k_codes)) || (k_signs && !aligned16(k_signs)) ||
        (v_codes && !aligned16(v_codes)) || !aligned16(key_rotation) || !aligned16(value_rotation) ||
        (qjl && !aligned16(qjl)))
        return TQ_ERR_UNSUPPORTED;
    const bool combo_ok = has_qjl ? (key_bits + 1 == value_bits && value_bits >= 2 && value_bits <= 4)
                                  : (key_bits == value_bits && key_bits >= 1 && key_bits <= 4);
    if (!combo_ok) return TQ_ERR_UNSUPPORTED;
    if (!workspace) return TQ_ERR_WORKSPACE;
    if (!(scale > 0.0f)) scale = 1.0f / sqrtf((float)D);

    hipStream_t s = static_cast<hipStream_t>(stream);
    const int groups = batch * kv_heads;
    SplitArgs a{q,        q_heads,  kv_heads, G,           seq_starts,    seq_lens,
                n_tokens, cap,      k_codes,  k_norms,     k_signs,       k_rnorms,
                v_codes,  v_norms,  key_rotation, qjl,     scale * LOG2E, scale * LOG2E * QJL_SCALE,
                key_centers, value_centers, scale, 0,      0,             nullptr,
                nullptr};
    int n_split = 0;
    int64_t tps = 0;
    int st = dispatch(value_bits, has_qjl, G, a, groups, s, &n_split, &tps);  // sizing
    if (st != TQ_OK) return st;
    const Ws w = ws_layout(batch, q_heads, n_split);
    if (workspace_bytes < w.total) return TQ_ERR_WORKSPACE;
    char* base = static_cast<char*>(workspace);
    a.po = reinterpret_cast<float*>(base + w.po);
    a.pml = reinterpret_cast<float*>(base + w.pml);
    // every split workgroup builds its group's q-side operands, then the merge
    st = dispatch(value_bits, has_qjl, G, a, groups, s, &n_split, &tps);
    if (st != TQ_OK) return st;
    TQ_CHECK_LAUNCH();
    hipLaunchKernelGGL(merge_kernel, dim3(batch * q_heads), dim3(MT), 0, s, a.po, a.pml, n_split, value_rotation,
                       out_f32, out_bf16, lse_out);
    TQ_CHECK_LAUNCH();
    return TQ_OK;
}
}  // namespace

extern "C" int tq_decode_attention(const uint16_t* q, int batch, int q_heads, int kv_heads, int dim,
                                   const int32_t* seq_starts, const int32_t* seq_lens, int64_t n_tokens, int64_t cap,
                                   const uint8_t* k_codes, const uint16_t* k_norms, const uint8_t* k_signs,
                                   const uint16_t* k_rnorms, const uint8_t* v_codes, const uint16_t* v_norms,
                                   int key_bits, int value_bits, int has_qjl, const float* key_rotation,
                                   const float* key_centers, const float* qjl, const float* value_rotation,
                                   const float* value_centers, float scale, float* out_f32, uint16_t* out_bf16,
                                   float* lse_out, void* workspace, size_t workspace_bytes, void* stream) {
    return decode_attention_impl(q, batch, q_heads, kv_heads, dim, seq_starts, seq_lens, n_tokens, cap, k_codes,
                                 k_norms, k_signs, k_rnorms, v_codes, v_norms, key_bits, value_bits, has_qjl,
                                 key_rotation, key_centers, qjl, value_rotation, value_centers, scale, out_f32,
                                 out_bf16, lse_out, workspace, workspace_bytes, stream);
}

// ------------------------------------------------------------------ no-allocation entry point
// The partials of tq_decode_attention_noalloc: one copy per GPU, held until the process ends.
// In host code `scratch` names a host-side stand-in, not device memory: the device address
// of each GPU's copy comes from hipGetSymbolAddress, made once per device (with that device
// current) on the first call there, and only that address is ever passed to a kernel.
static __device__ __align__(256) unsigned char scratch[TQ_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex scratch_mutex;
void* scratch_ptr[MAX_DEVICES];  // device address of `scratch` on each device, once resolved

int device_scratch(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return TQ_ERR_HIP;
    if (dev < 0 || dev >= MAX_DEVICES) return TQ_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return TQ_ERR_HIP;
        scratch_ptr[dev] = p;
    }
    *out = scratch_ptr[dev];
    return TQ_OK;
}
}  // namespace

extern "C" int tq_decode_attention_noalloc(const uint16_t* q, int batch, int q_heads, int kv_heads, int dim,
                                           const int32_t* seq_starts, const int32_t* seq_lens, int64_t n_tokens,
                                           int64_t cap, const uint8_t* k_codes, const uint16_t* k_norms,
                                           const uint8_t* k_signs, const uint16_t* k_rnorms, const uint8_t* v_codes,
                                           const uint16_t* v_norms, int key_bits, int value_bits, int has_qjl,
                                           const float* key_rotation, const float* key_centers, const float* qjl,
                                           const float* value_rotation, const float* value_centers, float scale,
                                           float* out_f32, uint16_t* out_bf16, float* lse_out, void* stream) {
    void* ws = nullptr;
    const int st = device_scratch(&ws);
    if (st != TQ_OK) return st;
    // the shared body sizes the partials for this call and returns TQ_ERR_WORKSPACE, before
    // any launch, when they exceed the array
    return decode_attention_impl(q, batch, q_heads, kv_heads, dim, seq_starts, seq_lens, n_tokens, cap, k_codes,
                                 k_norms, k_signs, k_rnorms, v_codes, v_norms, key_bits, value_bits, has_qjl,
                                 key_rotation, key_centers, qjl, value_rotation, value_centers, scale, out_f32,
                                 out_bf16, lse_out, ws, TQ_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int tq_decode_attention_groups(const uint16_t* q, int batch, int q_heads, int kv_heads, int dim,
                                          const int32_t* seq_starts, const int32_t* seq_lens, int64_t n_tokens,
                                          int64_t cap, int n_groups, const int* sub_dims, const int* key_bits,
                                          const int* value_bits, int has_qjl, const uint8_t* const* k_codes,
                                          const uint16_t* const* k_norms, const uint8_t* const* k_signs,
                                          const uint16_t* const* k_rnorms, const uint8_t* const* v_codes,
                                          const uint16_t* const* v_norms, const float* key_matrix,
                                          const float* const* key_centers, const float* qjl_matrix,
                                          const float* value_matrix, const float* const* value_centers, float scale,
                                          float* out_f32, uint16_t* out_bf16, float* lse_out, void* workspace,
                                          size_t workspace_bytes, void* stream) {
    if (!q || batch <= 0 || q_heads <= 0 || kv_heads <= 0 || n_tokens < 0 || cap < n_tokens)
        return TQ_ERR_INVALID_ARGUMENT;
    if (dim != D) return TQ_ERR_UNSUPPORTED;
    if (q_heads % kv_heads) return TQ_ERR_INVALID_ARGUMENT;
    const int G = q_heads / kv_heads;
    if (G > TQ_MAX_GROUP) return TQ_ERR_UNSUPPORTED;
    if (n_groups < 1 || n_groups > NGRP || !sub_dims || !key_bits || !value_bits || !k_codes || !k_norms ||
        !v_codes || !v_norms || !key_centers || !value_centers)
        return TQ_ERR_INVALID_ARGUMENT;
    if (!key_matrix || !value_matrix || (has_qjl && (!qjl_matrix || !k_signs || !k_rnorms)))
        return TQ_ERR_INVALID_ARGUMENT;
    if (!aligned16(key_matrix) || !aligned16(value_matrix) || (has_qjl && !aligned16(qjl_matrix)))
        return TQ_ERR_UNSUPPORTED;  // rows are read as float4
    if (!out_f32 && !out_bf16 && !lse_out) return TQ_ERR_INVALID_ARGUMENT;
    if (!workspace) return TQ_ERR_WORKSPACE;
    if (!(scale > 0.0f)) scale = 1.0f / sqrtf((float)D);
    GroupAttnArgs a{};
    a.q = q;
    a.q_heads = q_heads;
    a.kv_heads = kv_heads;
    a.G = G;
    a.n_groups = n_groups;
    a.seq_starts = seq_starts;
    a.seq_lens = seq_lens;
    a.n_tokens = n_tokens;
    a.cap = cap;
    a.cs = scale * LOG2E;
    a.Mk = key_matrix;
    a.Ms = qjl_matrix;
    int dsum = 0, kst = 0, vst = 0;
    for (int g = 0; g < n_groups; ++g) {
        const int d = sub_dims[g], kb = key_bits[g], vb = value_bits[g];
        if (d < 1 || kb < 1 || kb > 8 || vb < 1 || vb > 8) return TQ_ERR_INVALID_ARGUMENT;
        if (!k_codes[g] || !k_norms[g] || !v_codes[g] || !v_norms[g] || !key_centers[g] || !value_centers[g])
            return TQ_ERR_INVALID_ARGUMENT;
        if (has_qjl && (!k_signs[g] || !k_rnorms[g])) return TQ_ERR_INVALID_ARGUMENT;
        a.kc[g] = k_codes[g];
        a.kn[g] = k_norms[g];
        a.ks[g] = has_qjl ? k_signs[g] : nullptr;
        a.kr[g] = has_qjl ? k_rnorms[g] : nullptr;
        a.vc[g] = v_codes[g];
        a.vn[g] = v_norms[g];
        a.d[g] = d;
        a.j0[g] = dsum;
        a.kb[g] = kb;
        a.vb[g] = vb;
        a.rk[g] = (d * kb + 7) / 8;
        a.rs[g] = (d + 7) / 8;
        a.rv[g] = (d * vb + 7) / 8;
        a.Ck[g] = key_centers[g];
        a.Cv[g] = value_centers[g];
        a.cq[g] = scale * LOG2E * (float)(sqrt(M_PI / 2.0) / (double)d);
        // every byte offset of the group's rows, including one tile past the capacity, fits
        // the 31-bit buffer range and 32-bit offsets
        const int64_t rmax = a.rk[g] > a.rv[g] ? a.rk[g] : a.rv[g];
        if ((cap + GT) * rmax >= ((int64_t)1 << 31)) return TQ_ERR_UNSUPPORTED;
        a.kst[g] = kst;
        kst += stage_dwords(a.rk[g]);
        a.sst[g] = kst;
        if (has_qjl) kst += stage_dwords(a.rs[g]);
        a.vst[g] = vst;
        vst += stage_dwords(a.rv[g]);
        dsum += d;
    }
    if (dsum != D) return TQ_ERR_INVALID_ARGUMENT;  // the groups partition the head's channels
    const int groups = batch * kv_heads;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // Two groups with at most OD1 outlier channels: the split kernel's matrix-core stages for
    // group 0 and a per-lane term for group 1, when group 0's bit widths are a one-group
    // layer's, group 1 is one bit wider or there are at most 4 query heads per KV head, and the
    // row arrays start at 4-byte boundaries
    const auto a4 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; };
    const bool og_bits = has_qjl ? (key_bits[0] + 1 == value_bits[0] && value_bits[0] >= 2 && value_bits[0] <= 4)
                                 : (key_bits[0] == value_bits[0] && key_bits[0] >= 1 && key_bits[0] <= 4);
    const bool og_x1 = n_groups == 2 && key_bits[1] == key_bits[0] + 1 && value_bits[1] == value_bits[0] + 1;
    bool og_ok = n_groups == 2 && (G <= 4 || (og_x1 && og_wide_ok(key_bits[0], value_bits[0], has_qjl))) &&
                 sub_dims[1] <= OD1 && og_bits && aligned16(q);
    for (int g = 0; og_ok && g < 2; ++g)
        og_ok = a4(k_codes[g]) && a4(v_codes[g]) && (!has_qjl || a4(k_signs[g]));
    if (og_ok) {
        const int d0 = sub_dims[0], d1 = sub_dims[1];
        const double qs = sqrt(M_PI / 2.0);
        SplitArgs sa{q,        q_heads,   kv_heads,  G,          seq_starts,
                     seq_lens, n_tokens,  cap,       k_codes[0], k_norms[0],
                     has_qjl ? k_signs[0] : nullptr, has_qjl ? k_rnorms[0] : nullptr, v_codes[0], v_norms[0],
                     key_matrix, qjl_matrix, scale * LOG2E, (float)(scale * LOG2E * (qs / d0)), key_centers[0],
                     value_centers[0], scale, 0, 0, nullptr, nullptr};
        Og& o = sa.og;
        o.d0 = d0, o.d1 = d1;
        o.r0k = a.rk[0], o.r0s = a.rs[0], o.r0v = a.rv[0];
        o.r1k = a.rk[1], o.r1s = a.rs[1], o.r1v = a.rv[1];
        o.b1k = key_bits[1], o.b1v = value_bits[1];
        o.kc1 = k_codes[1], o.ks1 = has_qjl ? k_signs[1] : nullptr, o.vc1 = v_codes[1];
        o.kn1 = k_norms[1], o.kr1 = has_qjl ? k_rnorms[1] : nullptr, o.vn1 = v_norms[1];
        o.Ck1 = key_centers[1], o.Cv1 = value_centers[1];
        o.cq1 = (float)(scale * LOG2E * (qs / d1));
        int n_split = 0;
        int64_t tps = 0;
        int st = dispatch_og(value_bits[0], has_qjl, G, sa, groups, s, &n_split, &tps);  // sizing
        if (st != TQ_OK) return st;
        const Ws w = ws_layout(batch, q_heads, n_split);
        if (workspace_bytes < w.total) return TQ_ERR_WORKSPACE;
        char* base = static_cast<char*>(workspace);
        sa.po = reinterpret_cast<float*>(base + w.po);
        sa.pml = reinterpret_cast<float*>(base + w.pml);
        st = dispatch_og(value_bits[0], has_qjl, G, sa, groups, s, &n_split, &tps);
        if (st != TQ_OK) return st;
        TQ_CHECK_LAUNCH();
        hipLaunchKernelGGL(merge_kernel, dim3(batch * q_heads), dim3(MT), 0, s, sa.po, sa.pml, n_split, value_matrix,
                           out_f32, out_bf16, lse_out);
        TQ_CHECK_LAUNCH();
        return TQ_OK;
    }
    int64_t tps = 0;
    const int n_split = group_split(groups, n_tokens > 0 ? n_tokens : 1, &tps);
    const Ws w = ws_layout(batch, q_heads, n_split);
    if (workspace_bytes < w.total) return TQ_ERR_WORKSPACE;
    char* base = static_cast<char*>(workspace);
    a.po = reinterpret_cast<float*>(base + w.po);
    a.pml = reinterpret_cast<float*>(base + w.pml);
    a.tps = tps;
    a.n_split = n_split;
    const size_t lds = (size_t)(kst > vst ? kst : vst) * sizeof(uint32_t);
    const dim3 grid(n_split, groups);
    if (G <= 4) {
        if (has_qjl) hipLaunchKernelGGL((group_attn_kernel<4, true>), grid, dim3(GT), lds, s, a);
        else hipLaunchKernelGGL((group_attn_kernel<4, false>), grid, dim3(GT), lds, s, a);
    } else {
        if (has_qjl) hipLaunchKernelGGL((group_attn_kernel<8, true>), grid, dim3(GT), lds, s, a);
        else hipLaunchKernelGGL((group_attn_kernel<8, false>), grid, dim3(GT), lds, s, a);
    }
    TQ_CHECK_LAUNCH();
    hipLaunchKernelGGL(merge_kernel, dim3(batch * q_heads), dim3(MT), 0, s, a.po, a.pml, n_split, value_matrix,
                       out_f32, out_bf16, lse_out);
    TQ_CHECK_LAUNCH();
    return TQ_OK;
}
