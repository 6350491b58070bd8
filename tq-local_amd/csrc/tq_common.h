// tq_common.h -- device helpers shared by the libtq HIP kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/tq.h"

#define TQ_DIM 128          // head_dim supported by the kernels
#define TQ_MAX_GROUP 8      // max query heads per KV head (GQA group)

namespace tq {

// bf16 bit pattern -> fp32 (exact).
__device__ __forceinline__ float bf16_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

// fp32 -> bf16 bit pattern, round to nearest even (NaN kept quiet).  A select rather than a
// branch: unrolled over a vector, branches would keep every element's value live at once.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t rounded = (x + 0x7FFFu + ((x >> 16) & 1u)) >> 16;
    return ((x & 0x7FFFFFFFu) > 0x7F800000u) ? ((x >> 16) | 0x40u) : rounded;
}

// fp32 -> IEEE binary16 bit pattern, round to nearest even (v_cvt_f16_f32).
__device__ __forceinline__ uint32_t f32_to_f16(float f) {
    _Float16 h = (_Float16)f;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// IEEE-exact fp32 division and square root (the quantizer is bit-exact against
// a CPU restatement that uses C's '/' and sqrtf).  '/' lowers to the full IEEE division
// sequence; __builtin_sqrtf to v_sqrt_f32 plus a +-1 ulp fma-residual correction, which
// rounds correctly.  (__fsqrt_rn is the bare v_sqrt_f32 unless the header's rounded-
// operation switch is set, and is off by one ulp for some inputs.)
__device__ __forceinline__ float div_rn(float a, float b) { return a / b; }
__device__ __forceinline__ float sqrt_rn(float a) { return __builtin_sqrtf(a); }

// Bits [pos, pos+n) of a little-endian word array held in registers, pos and
// n compile-time constants after unrolling: one v_bfe_u32, plus a v_alignbit_b32
// when the field straddles two words.
template <int N>
__device__ __forceinline__ uint32_t extract_bits(const uint32_t* w, int pos) {
    const int wi = pos >> 5, sh = pos & 31;
    if (sh + N > 32) return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh), 0, N);
    return __builtin_amdgcn_ubfe(w[wi], sh, N);
}

// Host: a per-device figure (CU count, occupancy) computed on the first call for the current
// device and kept.  Host threads racing on a first call compute the same value and publish it
// with an atomic store, so there is no data race; `slots` is a zero-initialised static array.
constexpr int MAX_DEVICES = 64;
template <typename F>
inline int64_t once_per_device(std::atomic<int64_t>* slots, int64_t fallback, F&& compute) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return fallback;
    int64_t v = slots[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        v = compute(dev);
        slots[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

}  // namespace tq

#define TQ_CHECK_LAUNCH()                                 \
    do {                                                  \
        if (hipGetLastError() != hipSuccess) return TQ_ERR_HIP; \
    } while (0)
