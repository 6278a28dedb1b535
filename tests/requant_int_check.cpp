// Host-side check of the device requantization map (gemmkit_amd/csrc/requant.h)
// against the oracle's or_requant_one (the f64 formula of KRequantize::apply,
// src/kernel/epilogue.rs:810-830).  Built and run by test_requant_int.py.
//
// Cases: the requant_store sweep values of src/simd.rs:771-826 crossed with
// scales, zero points and bands; power-of-two scales landing exactly on
// halves; constructed products of 54-55 significant bits within 3 units of a
// half, where the f64 multiply's rounding decides rne; random i32 x random
// f32 (all exponents, subnormals, infinities, NaN).  Prints "mismatches N cases M" and up to 10
// mismatches.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <initializer_list>

#include "requant.h"

extern "C" int32_t or_requant_one(int32_t acc, int32_t bias, float scale, int32_t zp, int32_t lo,
                                  int32_t hi);

static uint64_t g_state = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {  // xorshift64*
    g_state ^= g_state >> 12;
    g_state ^= g_state << 25;
    g_state ^= g_state >> 27;
    return g_state * 0x2545F4914F6CDD1Dull;
}

static long g_cases = 0, g_bad = 0;

static void check(int32_t acc, int32_t bias, float scale, int32_t zp, int32_t lo, int32_t hi) {
    uint32_t bits;
    memcpy(&bits, &scale, 4);
    const int32_t got = gk::requant_bits(acc, bias, bits, zp, lo, hi);
    const int32_t fast = gk::requant_fast(acc, bias, scale, zp, lo, hi);
    // the device epilogue: requant_f32, requant_f32_tie when it flags a tie,
    // requant_bits when it flags the lane slow; a wave applies the tie tier
    // to every lane when any lane needs it, so that tier must be exact on
    // every lane that is not slow
    const gk::RequantF32 f = gk::requant_f32(acc, bias, scale, zp, lo, hi);
    const int32_t tq = gk::requant_f32_tie(acc, bias, scale, zp, lo, hi);
    const int32_t dev = f.slow ? got : (f.tie ? tq : f.q);
    const int32_t want = or_requant_one(acc, bias, scale, zp, lo, hi);
    ++g_cases;
    if (got != want || fast != want || dev != want || (!f.slow && tq != want)) {
        if (g_bad < 10)
            printf("MISMATCH acc=%d bias=%d scale=%a (0x%08x) zp=%d band=[%d,%d] bits=%d fast=%d "
                   "dev=%d tie=%d want=%d\n", acc, bias, (double)scale, bits, zp, lo, hi, got, fast,
                   dev, tq, want);
        ++g_bad;
    }
}

static float from_bits(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}

int main() {
    const int32_t bands[][2] = {{-128, 127}, {0, 255}, {0, 127}, {3, 255}, {-3, 127}};
    const int32_t zps[] = {0, -128, 127, 3, 255, -3};
    // requant_store sweep accumulators (src/simd.rs:771-826)
    int32_t accs[8 + 96] = {INT32_MIN, INT32_MIN + 1, -1, 0, 1, 1 << 30, INT32_MAX - 1, INT32_MAX};
    uint64_t lcg = 0x123456789abcdef0ull;
    for (int i = 0; i < 96; ++i) {
        lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
        accs[8 + i] = (int32_t)(uint32_t)(lcg >> 32);
    }
    const float scales[] = {1.0f, 0.1f, 1e30f, 1e-30f, 0.0078125f, 0.5f, 1e-9f, 3e-4f, 0.003f,
                            7.25f, 1e-40f, 1.4e-45f, 3e38f, 2.0f, 1.0f / 3.0f, 0.0f, -0.0f,
                            from_bits(0x7F800000u), from_bits(0xFF800000u), from_bits(0x7FC00000u),
                            from_bits(0x00800000u), from_bits(0x7F7FFFFFu)};
    const int32_t biases[] = {0, 1, -1, 65536, -65536, INT32_MAX, INT32_MIN};
    for (int32_t a : accs)
        for (int32_t b : biases)
            for (float s : scales)
                for (int32_t zp : zps)
                    for (auto &bd : bands) check(a, b, s, zp, bd[0], bd[1]);

    // Exact halves: acc * 2^-k with odd numerators at the half.
    for (int k = 1; k < 40; ++k)
        for (int j = -300; j <= 300; ++j) {
            const int64_t a = (2 * (int64_t)j + 1) << (k - 1);
            if (a > INT32_MAX || a < INT32_MIN) continue;
            const float s = from_bits((uint32_t)(127 - k) << 23);
            for (int32_t zp : {0, 3}) check((int32_t)a, 0, s, zp, -128, 127);
        }

    // Near-ties the f64 multiply can move: products v*m of 54-55 bits that sit
    // within 3 units of a half, (k + 1/2) * 2^s + d, for scale = m * 2^-s.  For
    // odd m, v = (2^(s-1) + d) * m^-1 mod 2^s; the pairs with v < 2^31 are kept.
    long near = 0;
    for (int it = 0; it < (1 << 21); ++it) {
        const uint64_t m = (next_u64() % (1ull << 23)) | (1ull << 23) | 1ull;  // odd, 24 bits
        uint64_t inv = m;  // m^-1 mod 2^64 by Newton's iteration
        for (int r = 0; r < 5; ++r) inv *= 2 - m * inv;
        for (int s = 46; s <= 54; ++s) {
            for (int d = -3; d <= 3; d += 2) {
                const uint64_t mask = (1ull << s) - 1;
                const uint64_t v = (((1ull << (s - 1)) + (uint64_t)(int64_t)d) * inv) & mask;
                if (v == 0 || v >= (1ull << 31)) continue;
                const float sc = from_bits(((uint32_t)(150 - s) << 23) | ((uint32_t)m & 0x7FFFFFu));
                for (int sign = 0; sign < 2; ++sign) {
                    const int32_t vv = sign ? (int32_t)(-(int64_t)v) : (int32_t)v;
                    check(vv, 0, sc, 0, -128, 127);
                    check(vv, 0, sc, 1, 0, 255);
                }
                ++near;
            }
        }
    }
    printf("near-tie products %ld\n", near);

    // Random: any i32 pair, any finite or special f32.
    for (int it = 0; it < 6000000; ++it) {
        const uint64_t r = next_u64();
        const int32_t a = (int32_t)(uint32_t)r, b = (int32_t)(uint32_t)(r >> 32);
        const uint64_t r2 = next_u64();
        float s = from_bits((uint32_t)r2);
        if ((r2 >> 40) % 4 == 0) s = from_bits(((uint32_t)(100 + (r2 >> 48) % 40) << 23) | ((uint32_t)r2 & 0x7FFFFFu));
        const int32_t zp = (int32_t)((r2 >> 32) % 256) - 128;
        check(a, b & 0x1FFFF, s, zp, -128, 127);
        check(a, b, s, zp + 128, 0, 255);
    }
    // Operands below 2^24 (the f32 fast path): random, and exact halves of
    // the two-float split (power-of-two scales times odd values, plus scales
    // whose product has low bits beyond f32's 24).
    for (int it = 0; it < 4000000; ++it) {
        const uint64_t r = next_u64();
        const int32_t a = (int32_t)(r % (1u << 25)) - (1 << 24);
        const uint64_t r2 = next_u64();
        const uint32_t ex = 100 + (uint32_t)((r2 >> 32) % 40);
        const float s = from_bits((ex << 23) | ((uint32_t)r2 & 0x7FFFFFu));
        check(a, 0, s, 0, -128, 127);
        check(a, (int32_t)(r >> 40) % 1000, s, 7, 0, 255);
    }
    for (int k = 1; k < 24; ++k)
        for (int j = 0; j < 20000; ++j) {
            const int32_t a = (int32_t)((next_u64() % (1u << 24)) | 1u);
            const float s = from_bits(((uint32_t)(127 - k) << 23) | ((uint32_t)next_u64() & 0x7Fu));
            check(a, 0, s, 0, -128, 127);
            check(-a, 0, s, 0, -128, 127);
        }
    // f32 products that round exactly onto a half while the exact product is
    // off it: scale = fl32((q + 1/2) / v) for random v < 2^24.
    long on_half = 0;
    for (int it = 0; it < 2000000; ++it) {
        const int32_t v = (int32_t)(next_u64() % ((1u << 24) - 1)) + 1;
        const int32_t q = (int32_t)(next_u64() % 250) - 125;
        const float sc = (float)(((double)q + 0.5) / (double)v);
        if (!(sc > 0.0f)) continue;
        const float ph = (float)v * sc;
        if (ph == (float)q + 0.5f) ++on_half;
        check(v, 0, sc, 0, -128, 127);
        check(-v, 0, sc, 3, -128, 127);
    }
    printf("f32 products on a half %ld\n", on_half);
    printf("mismatches %ld cases %ld\n", g_bad, g_cases);
    return g_bad != 0;
}
