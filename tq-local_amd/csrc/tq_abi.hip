// tq_abi.hip -- version and status helpers of the libtq C ABI, and the fp16 value codebook of
// the decode attention (a host computation).
#include "tq_common.h"

extern "C" int tq_abi_version(void) { return TQ_ABI_VERSION; }

extern "C" const char* tq_status_string(int status) {
    switch (status) {
        case TQ_OK: return "ok";
        case TQ_ERR_INVALID_ARGUMENT: return "invalid argument";
        case TQ_ERR_UNSUPPORTED: return "unsupported shape, alignment or bit width";
        case TQ_ERR_WORKSPACE: return "workspace missing or too small";
        case TQ_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

// ------------------------------------------------------------------ value codebook in fp16
// tq_decode_attention sums the values on fp16 matrix cores, so every value centroid enters as
// one fp16 number.  Its rounding error is the same for every token that carries the code: over
// a long, evenly spread softmax the output is a near-cancelling average while these errors add
// up (as sqrt(tokens) relative to the output).  Each centroid is therefore given the fp16
// neighbour (below or above it) that makes sum_c P_c (h_c - c) smallest, P_c the probability of
// code c under the coordinate density the Lloyd-Max codebook is built for, f(x) ~ (1 - x^2)^((d -
// 3) / 2) on [-1, 1] (one coordinate of a uniform point on S^(d-1)), cells split at the
// midpoints of the centroids.
#include <cmath>
#include <cstring>

namespace {

// IEEE binary16 bits of f, round to nearest even
uint16_t f16_bits_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int e = (int)((x >> 23) & 0xFF);
    uint32_t m = x & 0x7FFFFFu;
    if (e == 0xFF) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u : 0u));
    const int he = e - 127 + 15;
    if (he >= 31) return (uint16_t)(sign | 0x7C00u);
    if (he <= 0) {                       // binary16 subnormal (or zero): units of 2^-24
        if (he < -10) return (uint16_t)sign;
        m |= 0x800000u;
        const int sh = 14 - he;          // 14 .. 24
        uint32_t q = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);     // a carry into bit 10 is the smallest normal
    }
    uint32_t h = sign | ((uint32_t)he << 10) | (m >> 13);
    const uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // a carry rounds up the exponent
    return (uint16_t)h;
}

float f16_bits_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const int e = (h >> 10) & 0x1F;
    const uint32_t m = h & 0x3FFu;
    float v;
    if (e == 0) v = std::ldexp((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = std::ldexp((float)(m | 0x400u), e - 25);
    uint32_t x;
    std::memcpy(&x, &v, 4);
    x |= sign;
    std::memcpy(&v, &x, 4);
    return v;
}

// the next binary16 value above (up) or below h, for finite h
uint16_t f16_step(uint16_t h, bool up) {
    const bool neg = (h & 0x8000u) != 0;
    if ((h & 0x7FFFu) == 0) return up ? (uint16_t)0x0001u : (uint16_t)0x8001u;
    return (uint16_t)((up != neg) ? h + 1 : h - 1);
}

}  // namespace

extern "C" int tq_value_codebook_f16(const float* centers, int bits, int dim, float* out) {
    if (!centers || !out || bits < 1 || bits > 4 || dim < 3) return TQ_ERR_INVALID_ARGUMENT;
    const int n = 1 << bits;
    for (int c = 0; c < n; ++c) {
        if (!(std::fabs(centers[c]) < 1.0f)) return TQ_ERR_INVALID_ARGUMENT;  // NaN too
        if (c > 0 && !(centers[c] > centers[c - 1])) return TQ_ERR_INVALID_ARGUMENT;
    }
    // cell probabilities (composite Simpson, 4096 intervals per cell; the density is bounded
    // for d >= 3)
    const double ex = (dim - 3) / 2.0;
    double P[16], total = 0.0;
    for (int c = 0; c < n; ++c) {
        const double a = c == 0 ? -1.0 : 0.5 * ((double)centers[c - 1] + centers[c]);
        const double b = c == n - 1 ? 1.0 : 0.5 * ((double)centers[c] + centers[c + 1]);
        constexpr int M = 4096;
        const double hstep = (b - a) / M;
        double s = 0.0;
        for (int i = 0; i <= M; ++i) {
            const double x = a + hstep * i;
            const double f = std::pow(std::fmax(0.0, 1.0 - x * x), ex);
            s += f * (i == 0 || i == M ? 1.0 : (i & 1 ? 4.0 : 2.0));
        }
        P[c] = s * hstep / 3.0;
        total += P[c];
    }
    if (!(total > 0.0)) return TQ_ERR_INVALID_ARGUMENT;
    // the two fp16 neighbours of each centroid (equal when it is exactly representable)
    double lo[16], hi[16];
    for (int c = 0; c < n; ++c) {
        P[c] /= total;
        const uint16_t h = f16_bits_rne(centers[c]);
        const double v = f16_bits_to_float(h);
        if (v == (double)centers[c]) {
            lo[c] = hi[c] = v;
        } else if (v > (double)centers[c]) {
            hi[c] = v, lo[c] = f16_bits_to_float(f16_step(h, false));
        } else {
            lo[c] = v, hi[c] = f16_bits_to_float(f16_step(h, true));
        }
    }
    // every combination of neighbours (2^16 at most); ties keep the first
    uint32_t best = 0;
    double best_abs = INFINITY;
    for (uint32_t mask = 0; mask < (1u << n); ++mask) {
        double s = 0.0;
        for (int c = 0; c < n; ++c) s += P[c] * (((mask >> c) & 1u ? hi[c] : lo[c]) - (double)centers[c]);
        if (std::fabs(s) < best_abs) best_abs = std::fabs(s), best = mask;
    }
    for (int c = 0; c < n; ++c) out[c] = (float)(((best >> c) & 1u) ? hi[c] : lo[c]);
    return TQ_OK;
}
