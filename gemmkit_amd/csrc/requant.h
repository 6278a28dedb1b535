// requant.h -- the requantization map of gemmkit's KRequantize::apply
// (src/kernel/epilogue.rs:810-830) in integer arithmetic:
//
//   q = clamp((rne(f64(acc wrapping+ bias) * f64(scale)) as i64) sat+ zp, lo, hi)
//
// The product of an i32 and an f32 significand is an exact integer P of at
// most 55 bits times a power of two, P * 2^e.  The f64 multiply rounds P to 53
// significant bits (round half to even); rne then rounds P * 2^e to an
// integer, also half to even.  Both roundings are done here on 64-bit
// integers, so the result equals the f64 formula bit for bit without f64
// arithmetic (which runs at a fraction of the integer rate on CDNA4).
// Non-finite scales follow the formula too: NaN gives rne = NaN, `as i64`
// = 0; an infinite scale saturates by the sign of the product (0 * inf = NaN).
//
// Plain C++ so the same functions run in the device kernels and in the
// host-side test that checks them against the oracle (the pragma below makes
// them host+device functions under the HIP compiler; g++ ignores it).
#pragma once

#include <stdint.h>

#pragma clang force_cuda_host_device begin

namespace gk {

// Round |p| * 2^-s to an integer, half to even (s >= 1).
inline uint64_t rne_shift(uint64_t p, int s) {
    if (s >= 64) return 0;  // p < 2^56, so the value is below 1/2
    const uint64_t q = p >> s, rem = p & ((1ull << s) - 1), half = 1ull << (s - 1);
    return (rem > half || (rem == half && (q & 1))) ? q + 1 : q;
}

inline int32_t requant_bits(int32_t acc, int32_t bias, uint32_t scale_bits, int32_t zp,
                               int32_t lo, int32_t hi) {
    const int32_t v = (int32_t)((uint32_t)acc + (uint32_t)bias);
    const uint32_t ex = (scale_bits >> 23) & 0xFFu, frac = scale_bits & 0x7FFFFFu;
    const bool neg = ((scale_bits >> 31) != 0) != (v < 0);
    // Magnitude of the rounded product, saturated at kBig (any |q| >= 2^40
    // lands on a band edge after adding zp).
    const int64_t kBig = 1ll << 40;
    int64_t mag = 0;
    if (ex == 0xFFu) {
        mag = (frac != 0 || v == 0) ? 0 : kBig;  // NaN or 0*inf: 0; inf: saturate
    } else {
        const uint64_t m = ex ? (frac | 0x800000u) : frac;  // scale = m * 2^e
        const int e = ex ? (int)ex - 150 : -149;
        const uint64_t av = v < 0 ? (uint64_t)(-(int64_t)v) : (uint64_t)v;
        uint64_t p = av * m;  // < 2^55, exact
        // f64 product: round to 53 significant bits.
        if (p >= (1ull << 54)) p = rne_shift(p, 2) << 2;
        else if (p >= (1ull << 53)) p = rne_shift(p, 1) << 1;
        if (p == 0) {
            mag = 0;
        } else if (e >= 0) {
            mag = (e >= 16 || p >= (1ull << 40)) ? kBig : (int64_t)(p << e);
            if (mag > kBig) mag = kBig;
        } else {
            mag = (int64_t)rne_shift(p, -e);
        }
    }
    int64_t q = (neg ? -mag : mag) + zp;
    if (q < lo) q = lo;
    if (q > hi) q = hi;
    return (int32_t)q;
}

// The same map, evaluated mostly in f32: when |acc + bias| < 2^24 (every
// accumulator of a 4096-deep i8 dot product of random data, for instance)
// the operand is exact in f32, the product has at most 48 bits and is exact
// in f64, so the reference rounds the exact product.  Its two-float split
// hi + lo (hi = fl32(v*s), lo = fma(v, s, -hi), exact) rounds like the exact
// product: rint(hi) is right unless hi sits exactly on a half, where the sign
// of lo breaks the tie (lo = 0: a true tie, rint's even choice).  Other
// operands take requant_bits.
inline int32_t requant_fast(int32_t acc, int32_t bias, float scale, int32_t zp, int32_t lo,
                               int32_t hi) {
    // Every rounding below is one IEEE f32 operation: no multiply may be
    // fused into a later add (the device compiler fuses across statements
    // unless told not to).
#pragma clang fp contract(off)
    const int32_t v = (int32_t)((uint32_t)acc + (uint32_t)bias);
    const uint32_t sbits = __builtin_bit_cast(uint32_t, scale);
    if (v >= (1 << 24) || v <= -(1 << 24) || ((sbits >> 23) & 0xFFu) == 0xFFu)
        return requant_bits(acc, bias, sbits, zp, lo, hi);
    const float vf = (float)v;
    const float ph = vf * scale;
    const float pl = __builtin_fmaf(vf, scale, -ph);
    float t = __builtin_rintf(ph);
    const float d = ph - t;
    if ((d == 0.5f || d == -0.5f) && pl != 0.0f) t = ph + (pl > 0.0f ? 0.5f : -0.5f);
    // Anything beyond 2^24 (or an f32 overflow to +-inf) saturates the band;
    // clamp before converting.
    t = __builtin_fminf(__builtin_fmaxf(t, -16777216.0f), 16777216.0f);
    int32_t q = (int32_t)t + zp;
    q = q < lo ? lo : q;
    q = q > hi ? hi : q;
    return q;
}

// The device epilogue's form of requant_fast, in three tiers so the common
// case costs about a dozen VALU instructions per value:
//   requant_f32      rint of the f32 product, clamp, zero point, band.  Exact
//                    unless the f32 product sits on a half (`tie`: the sign
//                    of the product's low part may then decide) or the lane
//                    needs the integer path (`slow`: |acc + bias| >= 2^24,
//                    where the f32 operand is no longer exact, or a
//                    non-finite product -- a NaN or infinite scale, or an f32
//                    overflow);
//   requant_f32_tie  the same with the two-float tie correction (exact for
//                    every lane that is not slow);
//   requant_bits     exact for every input.
// Callers evaluate requant_f32 and take a later tier for the whole wave only
// when some lane flags it, so the exceptional paths cost nothing when no lane
// needs them.
struct RequantF32 {
    int32_t q;
    bool slow;
    bool tie;
};

inline int32_t requant_band(float t, int32_t zp, int32_t lo, int32_t hi) {
    // Zero point and band in f32: t is an integer (or infinite), |zp| <= 255
    // and the band lies within [-128, 255], so t + zp is exact wherever the
    // result can land inside the band, and anything larger clamps to an edge
    // either way.  Three instructions (add, clamp, convert).
#pragma clang fp contract(off)
    const float v = t + (float)zp;
    return (int32_t)__builtin_fminf(__builtin_fmaxf(v, (float)lo), (float)hi);
}

inline RequantF32 requant_f32(int32_t acc, int32_t bias, float scale, int32_t zp, int32_t lo,
                                 int32_t hi) {
#pragma clang fp contract(off)
    const int32_t v = (int32_t)((uint32_t)acc + (uint32_t)bias);
    const float vf = (float)v;
    const float ph = vf * scale;
    const float t = __builtin_rintf(ph);
    RequantF32 r;
    r.tie = __builtin_fabsf(ph - t) == 0.5f;
    r.slow = !(__builtin_fabsf(vf) < 16777216.0f) || !(__builtin_fabsf(ph) < __builtin_inff());
    r.q = requant_band(t, zp, lo, hi);
    return r;
}

inline int32_t requant_f32_tie(int32_t acc, int32_t bias, float scale, int32_t zp, int32_t lo,
                                  int32_t hi) {
#pragma clang fp contract(off)
    const int32_t v = (int32_t)((uint32_t)acc + (uint32_t)bias);
    const float vf = (float)v;
    const float ph = vf * scale;
    const float pl = __builtin_fmaf(vf, scale, -ph);  // ph + pl = the exact product
    float t = __builtin_rintf(ph);
    const float d = ph - t;
    // On a half, rint chose the even neighbour; the exact product lies past
    // the half (away from t) when pl has the sign of d.  (Signs compared,
    // not multiplied: d * pl can underflow to zero.)
    const bool away = d > 0.0f ? pl > 0.0f : pl < 0.0f;
    if (__builtin_fabsf(d) == 0.5f && away) t += d + d;
    return requant_band(t, zp, lo, hi);
}

}  // namespace gk

#pragma clang force_cuda_host_device end
