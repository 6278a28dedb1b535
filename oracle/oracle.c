/*
 * oracle.c -- CPU closed-form restatement of gemmkit's GEMM semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the parity tests compare
 * the HIP kernels against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library (gemmkit_amd) never links,
 * loads or calls anything under oracle/.
 *
 * Every function cites the gemmkit source it restates (paths relative to the
 * gemmkit crate root, i.e. gemmkit/src/... and gemmkit/tests/...).
 *
 * Parity status (each function is pinned by the checks named; see
 * tests/test_oracle.py):
 *   or_gemm_i8          pinned: exact numpy int64 product, hand-computed wrap KAT,
 *                       brute-force Python loops on tiny shapes, the ABFT checksum
 *   or_requant_one      pinned: reference KATs (ties, vector ties, k==0 fill,
 *                       extremes) and an independent Python model (round() is
 *                       ties-to-even, ints are unbounded) over the LCG sweep
 *   or_gemm_i8_requant  pinned: composition of the two above, against fixtures
 *   or_bf16_from_f32    pinned: torch's RNE conversion on random/edge floats,
 *                       hand-checked NaN/inf/ties cases
 *   or_gemm_f64         pinned: README 2x2 KAT, numpy float64 matmul
 *   or_gemv_f64         pinned: numpy float64 matvec
 *   or_fused_map_f32    pinned: the reference's fused known answers (NaN -> +0
 *                       under ReLU and LeakyReLU, LeakyReLU(0) with a negative
 *                       slope -> +0, the degenerate ReLU(0.5*C0 + bias)), and
 *                       numpy float32 closed forms per activation branch
 *   or_fused_map_bf16   pinned: or_fused_map_f32 composed with or_bf16_from_f32,
 *                       plus the bias-widening identity on bf16 inputs
 */
#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <math.h>

#define OR_API __attribute__((visibility("default")))

/* ---------------------------------------------------------------- generators */

/* xorshift* generator of tests/epilogue/common.rs:16-34 (Rng).  The state is
 * seed|1; each step xorshifts (12, 25, 27) then multiplies by an odd constant. */
OR_API uint64_t or_rng_next(uint64_t *state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return x * 0x2545F4914F6CDD1DULL;
}

/* make_i8 of tests/epilogue/requant.rs:25-30: values in [-127, 127]. */
OR_API void or_fill_i8_sym127(uint64_t seed, size_t n, int8_t *out) {
    uint64_t s = seed | 1ULL;
    for (size_t i = 0; i < n; ++i) out[i] = (int8_t)((int64_t)(or_rng_next(&s) % 255) - 127);
}

/* Full i8 range [-128, 127] from the same Rng: next_u64() % 256 - 128. */
OR_API void or_fill_i8_full(uint64_t seed, size_t n, int8_t *out) {
    uint64_t s = seed | 1ULL;
    for (size_t i = 0; i < n; ++i) out[i] = (int8_t)((int64_t)(or_rng_next(&s) % 256) - 128);
}

/* rand_i8 of tests/correctness/common.rs:137-147: xorshift64 (13, 7, 17) seeded
 * with seed + golden-ratio constant, values in [-100, 100]. */
OR_API void or_rand_i8_100(uint64_t seed, size_t n, int8_t *out) {
    uint64_t s = seed + 0x9E3779B97F4A7C15ULL;
    for (size_t i = 0; i < n; ++i) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        out[i] = (int8_t)((int64_t)(s >> 24) % 201 - 100);
    }
}

/* rand_vec of tests/oracle_common/mod.rs:121-132: uniform [-1, 1) as f64, the
 * caller rounds to its element type. */
OR_API void or_rand_vec_f64(uint64_t seed, size_t n, double *out) {
    uint64_t s = seed + 0x9E3779B97F4A7C15ULL;
    for (size_t i = 0; i < n; ++i) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        double u = (double)(s >> 11) / 9007199254740992.0; /* 2^53 */
        out[i] = 2.0 * u - 1.0;
    }
}

/* Rng::unit of tests/epilogue/common.rs:30-33: (next >> 11) / 2^53 * 2 - 1. */
OR_API void or_rng_unit_f64(uint64_t seed, size_t n, double *out) {
    uint64_t s = seed | 1ULL;
    for (size_t i = 0; i < n; ++i)
        out[i] = (double)(or_rng_next(&s) >> 11) / 9007199254740992.0 * 2.0 - 1.0;
}

/* Standard normals by Box-Muller over Rng::unit-style uniforms in (0, 1]. */
OR_API void or_rng_normal_f64(uint64_t seed, size_t n, double *out) {
    uint64_t s = seed | 1ULL;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = ((double)(or_rng_next(&s) >> 11) + 1.0) / 9007199254740992.0;
        double u2 = (double)(or_rng_next(&s) >> 11) / 9007199254740992.0;
        double r = sqrt(-2.0 * log(u1));
        out[i] = r * cos(two_pi * u2);
        if (i + 1 < n) out[i + 1] = r * sin(two_pi * u2);
    }
}

/* --------------------------------------------------------------- i8 -> i32 */

/* C <- alpha*A*B + beta*C over strided views, all arithmetic wrapping i32.
 *
 * Restates gemmkit's integer contract: execute_int (src/dispatch/int.rs:131-148)
 * returns on m|n == 0; k == 0 or alpha == 0 runs scale_c_int (:150-163: beta == 0
 * writes 0, beta == 1 leaves C unwritten, else beta*C wrapping); otherwise
 * int32_epilogue (src/kernel/int.rs:36-120) computes alpha*acc then C, C+acc or
 * beta*C+acc, all wrapping.  Wrapping i32 addition is associative, so the
 * accumulation order of the blocked driver does not matter (src/kernel/int.rs:381-384,
 * tests/correctness/int8.rs:234-237): accumulating in uint32 here is exact mod 2^32.
 * Strides are element strides and may be negative, as on the unchecked tier. */
OR_API void or_gemm_i8(size_t m, size_t k, size_t n, int32_t alpha,
                       const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa,
                       const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb,
                       int32_t beta, int32_t *c, ptrdiff_t rsc, ptrdiff_t csc) {
    if (m == 0 || n == 0) return;
    if (k == 0 || alpha == 0) {
        for (size_t j = 0; j < n; ++j)
            for (size_t i = 0; i < m; ++i) {
                int32_t *p = c + (ptrdiff_t)i * rsc + (ptrdiff_t)j * csc;
                if (beta == 0) *p = 0;
                else if (beta != 1) *p = (int32_t)((uint32_t)beta * (uint32_t)*p);
            }
        return;
    }
    #pragma omp parallel for schedule(static) if (m * n * k > (1u << 22))
    for (ptrdiff_t i = 0; i < (ptrdiff_t)m; ++i) {
        for (size_t j = 0; j < n; ++j) {
            uint32_t acc = 0;
            const int8_t *ap = a + i * rsa;
            const int8_t *bp = b + (ptrdiff_t)j * csb;
            for (size_t p = 0; p < k; ++p)
                acc += (uint32_t)((int32_t)ap[(ptrdiff_t)p * csa] * (int32_t)bp[(ptrdiff_t)p * rsb]);
            uint32_t v = (uint32_t)alpha * acc;
            int32_t *cp = c + i * rsc + (ptrdiff_t)j * csc;
            if (beta == 0) *cp = (int32_t)v;
            else if (beta == 1) *cp = (int32_t)((uint32_t)*cp + v);
            else *cp = (int32_t)((uint32_t)beta * (uint32_t)*cp + v);
        }
    }
}

/* ------------------------------------------------------------------ requant */

/* round_ne_f64 of src/kernel/epilogue.rs:886-897: the 2^52 add/subtract trick
 * under the default round-to-nearest-even mode; |x| >= 2^52 and NaN pass through. */
OR_API double or_round_ne_f64(double x) {
    const double C = 4503599627370496.0; /* 2^52 */
    volatile double t; /* keep the compiler from folding (x + C) - C */
    if (x != x || x >= C || x <= -C) return x;
    if (x >= 0.0) { t = x + C; return t - C; }
    t = x - C;
    return t + C;
}

/* Rust's saturating `f64 as i64` (NaN -> 0), used by KRequantize::apply. */
static int64_t sat_f64_to_i64(double x) {
    if (x != x) return 0;
    if (x >= 9223372036854775808.0) return INT64_MAX;
    if (x < -9223372036854775808.0) return INT64_MIN;
    return (int64_t)x;
}

static int64_t sat_add_i64(int64_t a, int64_t b) {
    int64_t r;
    if (__builtin_add_overflow(a, b, &r)) return b > 0 ? INT64_MAX : INT64_MIN;
    return r;
}

/* KRequantize::apply of src/kernel/epilogue.rs:810-830:
 *   q = clamp((rne(f64(acc wrapping+ bias) * f64(scale)) as i64) sat+ zp, LO, HI)
 * and the caller stores the low byte (QuantOut::from_clamped, :748-765).
 * `lo`/`hi` are [-128, 127] for i8 and [0, 255] for u8.  The ReLU extension of
 * this build raises the lower bound to max(lo, zp) (rne is monotone with
 * rne(0) = 0, so max(0, real value) quantizes to max(zp, q)); the caller
 * passes the raised bound. */
OR_API int32_t or_requant_one(int32_t acc, int32_t bias, float scale, int32_t zp,
                              int32_t lo, int32_t hi) {
    int32_t v = (int32_t)((uint32_t)acc + (uint32_t)bias);
    double scaled = or_round_ne_f64((double)v * (double)scale);
    int64_t q = sat_add_i64(sat_f64_to_i64(scaled), (int64_t)zp);
    if (q < lo) q = lo;
    if (q > hi) q = hi;
    return (int32_t)q;
}

/* The requantizing GEMM: exact i32 accumulator (alpha = 1, beta = 0, as
 * run_typed_int_requant fixes them, src/dispatch/int.rs:794-797) mapped through
 * or_requant_one per element.  k == 0 fills apply(0) (requant_degenerate,
 * src/dispatch/int.rs:735-752).
 *   axis:      0 = scale/bias per row of C (length m, the reference's only
 *              choice), 1 = per column (length n, the per-output-channel
 *              extension of this build).
 *   scales:    NULL for the per-tensor `scale`.
 *   bias:      NULL for no bias.
 *   out_bytes: low byte of each clamped value, written at c + i*rsc + j*csc. */
OR_API void or_gemm_i8_requant(size_t m, size_t k, size_t n,
                               const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa,
                               const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb,
                               float scale, const float *scales, int32_t zp,
                               const int32_t *bias, int axis, int32_t lo, int32_t hi,
                               uint8_t *c, ptrdiff_t rsc, ptrdiff_t csc) {
    if (m == 0 || n == 0) return;
    #pragma omp parallel for schedule(static) if (m * n * k > (1u << 22))
    for (ptrdiff_t i = 0; i < (ptrdiff_t)m; ++i) {
        for (size_t j = 0; j < n; ++j) {
            uint32_t acc = 0;
            for (size_t p = 0; p < k; ++p)
                acc += (uint32_t)((int32_t)a[i * rsa + (ptrdiff_t)p * csa] *
                                  (int32_t)b[(ptrdiff_t)p * rsb + (ptrdiff_t)j * csb]);
            size_t ch = axis ? j : (size_t)i;
            float s = scales ? scales[ch] : scale;
            int32_t bb = bias ? bias[ch] : 0;
            int32_t q = or_requant_one((int32_t)acc, bb, s, zp, lo, hi);
            c[i * rsc + (ptrdiff_t)j * csc] = (uint8_t)(q & 0xFF);
        }
    }
}

/* The requant map applied to an existing i32 accumulator matrix (acc given
 * at strides ra/ca, bytes written at rc/cc): the same per-element map as
 * or_gemm_i8_requant, for checking a requantizing GEMM against a separately
 * checked i32 GEMM of the same operands. */
OR_API void or_requant_map(size_t m, size_t n, const int32_t *acc, ptrdiff_t ra, ptrdiff_t ca,
                           float scale, const float *scales, int32_t zp, const int32_t *bias,
                           int axis, int32_t lo, int32_t hi, uint8_t *c, ptrdiff_t rc,
                           ptrdiff_t cc) {
    #pragma omp parallel for schedule(static) if (m * n > (1u << 20))
    for (ptrdiff_t i = 0; i < (ptrdiff_t)m; ++i)
        for (size_t j = 0; j < n; ++j) {
            size_t ch = axis ? j : (size_t)i;
            float s = scales ? scales[ch] : scale;
            int32_t bb = bias ? bias[ch] : 0;
            int32_t q = or_requant_one(acc[i * ra + (ptrdiff_t)j * ca], bb, s, zp, lo, hi);
            c[i * rc + (ptrdiff_t)j * cc] = (uint8_t)(q & 0xFF);
        }
}

/* --------------------------------------------------------------------- bf16 */

/* f32 -> bf16 bits, round-to-nearest-even; NaN becomes (bits >> 16) | 0x0040.
 * Restates the narrowing of half::bf16::from_f32 (half 2.7.1) as the
 * reference's own vector twin spells it out (src/simd/avx512.rs:194-212). */
OR_API uint16_t or_bf16_from_f32(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    if ((bits & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t lsb = (bits >> 16) & 1u;
    return (uint16_t)((bits + 0x7FFFu + lsb) >> 16);
}

OR_API float or_f32_from_bf16(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

OR_API void or_bf16_from_f32_n(const float *x, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; ++i) out[i] = or_bf16_from_f32(x[i]);
}

/* ------------------------------------------------------------ f64 reference */

/* f64 closed form of tests/oracle_common/mod.rs:158-176 (`reference`):
 * out[i*n + j] = alpha * sum_p A[i,p] B[p,j] + (beta == 0 ? 0 : beta * C0[i,j]),
 * inputs widened to f64 exactly.  A/B/C0 are f32 views; bf16 inputs are widened
 * to f32 by the caller (exact).  `out` is dense row-major m x n. */
OR_API void or_gemm_f64(size_t m, size_t k, size_t n, double alpha,
                        const float *a, ptrdiff_t rsa, ptrdiff_t csa,
                        const float *b, ptrdiff_t rsb, ptrdiff_t csb,
                        double beta, const float *c0, ptrdiff_t rsc, ptrdiff_t csc,
                        double *out) {
    #pragma omp parallel for schedule(static) if (m * n * k > (1u << 22))
    for (ptrdiff_t i = 0; i < (ptrdiff_t)m; ++i) {
        for (size_t j = 0; j < n; ++j) {
            double acc = 0.0;
            for (size_t p = 0; p < k; ++p)
                acc += (double)a[i * rsa + (ptrdiff_t)p * csa] *
                       (double)b[(ptrdiff_t)p * rsb + (ptrdiff_t)j * csb];
            double base = (beta == 0.0 || c0 == NULL)
                              ? 0.0 : beta * (double)c0[i * rsc + (ptrdiff_t)j * csc];
            out[(size_t)i * n + j] = base + alpha * acc;
        }
    }
}

/* GEMV closed form, y[i] = alpha * <A[i,:], x> + beta * y0[i], f64 throughout
 * (the quantity gemv::dot_rows, src/special/gemv.rs:523-600, approximates). */
OR_API void or_gemv_f64(size_t rows, size_t k, double alpha,
                        const float *a, ptrdiff_t rs, ptrdiff_t cs,
                        const float *x, ptrdiff_t xs, double beta, const float *y0,
                        ptrdiff_t ys, double *out) {
    #pragma omp parallel for schedule(static) if (rows * k > (1u << 22))
    for (ptrdiff_t i = 0; i < (ptrdiff_t)rows; ++i) {
        double acc = 0.0;
        for (size_t p = 0; p < k; ++p)
            acc += (double)a[i * rs + (ptrdiff_t)p * cs] * (double)x[(ptrdiff_t)p * xs];
        double base = (beta == 0.0 || y0 == NULL) ? 0.0 : beta * (double)y0[i * ys];
        out[i] = base + alpha * acc;
    }
}

/* ABFT checksum of an i32 GEMM output, exact in i64: column sums of C and the
 * row vector (column sums of A) times B.  With alpha = 1, beta = 0 and no i32
 * wrap, sum_i C[i,j] == sum_p (sum_i A[i,p]) * B[p,j] for every j. */
OR_API void or_colsum_i32(size_t m, size_t n, const int32_t *c, ptrdiff_t rsc,
                          ptrdiff_t csc, int64_t *out) {
    for (size_t j = 0; j < n; ++j) out[j] = 0;
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) out[j] += c[(ptrdiff_t)i * rsc + (ptrdiff_t)j * csc];
}

OR_API void or_abft_i8(size_t m, size_t k, size_t n,
                       const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa,
                       const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb, int64_t *out) {
    for (size_t j = 0; j < n; ++j) out[j] = 0;
    for (size_t p = 0; p < k; ++p) {
        int64_t s = 0;
        for (size_t i = 0; i < m; ++i) s += a[(ptrdiff_t)i * rsa + (ptrdiff_t)p * csa];
        for (size_t j = 0; j < n; ++j) out[j] += s * b[(ptrdiff_t)p * rsb + (ptrdiff_t)j * csb];
    }
}

/* ----------------------------------------------------------- fused epilogue */

/* FusedEpi::apply for f32 (src/kernel/epilogue.rs:309-330; the tests' scalar
 * model ref_apply, tests/epilogue/common.rs:74-94) over an m x n matrix of
 * values v: out[i,j] = act(v[i,j] + bias[ch]) in f32, ch = i (dim 0, PerRow)
 * or j (dim 1, PerCol), bias == NULL for none; act 0 none, 1 ReLU (v > 0 ? v :
 * 0), 2 LeakyReLU (hi + slope*lo, hi = v > 0 ? v : 0, lo = v < 0 ? v : 0).
 * Built with -ffp-contract=off: every operation rounds on its own. */
static float fused_one_f32(float v, const float *bias, size_t ch, int act, float slope) {
    if (bias) v = v + bias[ch];
    if (act == 1) return v > 0.0f ? v : 0.0f;
    if (act == 2) {
        float hi = v > 0.0f ? v : 0.0f;
        float lo = v < 0.0f ? v : 0.0f;
        return hi + slope * lo;
    }
    return v;
}

OR_API void or_fused_map_f32(size_t m, size_t n, const float *v, ptrdiff_t rv, ptrdiff_t cv,
                             const float *bias, int dim, int act, float slope, float *out,
                             ptrdiff_t ro, ptrdiff_t co) {
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j)
            out[(ptrdiff_t)i * ro + (ptrdiff_t)j * co] =
                fused_one_f32(v[(ptrdiff_t)i * rv + (ptrdiff_t)j * cv], bias, dim ? j : i, act,
                              slope);
}

/* The narrow twin (src/kernel/epilogue.rs:569-596): the bf16 bias and slope
 * widen exactly to f32, the map runs in f32 on the f32 value v, and the result
 * narrows once with or_bf16_from_f32. */
OR_API void or_fused_map_bf16(size_t m, size_t n, const float *v, ptrdiff_t rv, ptrdiff_t cv,
                              const uint16_t *bias, int dim, int act, uint16_t slope,
                              uint16_t *out, ptrdiff_t ro, ptrdiff_t co) {
    const float s = or_f32_from_bf16(slope);
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) {
            float b = bias ? or_f32_from_bf16(bias[dim ? j : i]) : 0.0f;
            float x = v[(ptrdiff_t)i * rv + (ptrdiff_t)j * cv];
            out[(ptrdiff_t)i * ro + (ptrdiff_t)j * co] =
                or_bf16_from_f32(fused_one_f32(x, bias ? &b : NULL, 0, act, s));
        }
}
