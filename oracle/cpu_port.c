/*
 * cpu_port.c -- C restatement of gemmkit's CPU GEMM paths, used only as the
 * timed CPU baseline beside the GPU numbers (and checked against the closed
 * forms in oracle.c by tests/test_oracle.py: bit-exact for the integer paths,
 * within the float bars for the float ones).
 *
 * TEST INFRASTRUCTURE ONLY: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library never does.
 *
 * What it restates:
 *   - orientation swap when C is row-major-ish (src/dispatch.rs:395-417), the
 *     requantization channel axis flipping with it (src/dispatch/int.rs:779-786)
 *   - the BLIS 5-loop: jc (nc) -> pc (kc) -> pack B -> pack A -> (ic, jr) jobs
 *     (src/driver.rs:402-944), with the prepacked-RHS form that skips the B
 *     pack (src/driver.rs run_packed_rhs; src/api/packed.rs:372-656)
 *   - the 32 x 12 microtiles of the AVX-512 families:
 *       IntGemmVnni (src/kernel/int.rs:386-490): A packed k-quad interleaved
 *         with +128, B k-quad interleaved signed, vpdpbusd with the
 *         -128*colsum(B) correction (src/simd/avx512.rs:483-545);
 *       IntGemmVnniQ (src/kernel/int.rs:596-688): the same loop over the whole
 *         depth (kc = k) with the requantize map applied to the drained tile
 *         (src/kernel/epilogue.rs:810-830, src/simd/avx512.rs:274-321);
 *       FloatGemm<f32> on Avx512F (src/kernel/float.rs:150-281,
 *         src/dispatch/float.rs:305-308): MR = 2 x 16 rows, NR = 12, ascending-k
 *         FMA chains;
 *       Bf16DotGemm (src/kernel/mixed.rs:342-400, src/simd/avx512.rs:604-631):
 *         k-pair interleaved packs, vdpbf16ps, kc = k so the whole contraction
 *         accumulates in f32;
 *   - int32_epilogue (src/kernel/int.rs:36-120): alpha fold, beta 0/1/other, all
 *     wrapping, beta -> 1 after the first depth slice (src/driver.rs:725-730)
 *   - the row-partitioned GEMV dot_rows (src/special/gemv.rs:511-600): four
 *     rows at a time, 16-lane FMA accumulators, lane reduction, scalar tail,
 *     y = alpha*dot + beta*y
 *   - the analytical blocking of src/cache.rs:412-470 with this host's caches
 * Threads: OpenMP stands in for rayon's fork-join (src/parallel.rs:602-700);
 * a batch runs one element per worker (src/parallel.rs:348-420).
 * Hosts without AVX-512 VNNI / BF16 take the widen kernels (IntGemm,
 * src/kernel/int.rs:138-190; MixedGemm, src/kernel/mixed.rs:31-200), as the
 * reference's ISA selection does.
 */
#include <math.h>
#include <stdint.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include <immintrin.h>
#include <omp.h>

#define PORT_API __attribute__((visibility("default")))

enum { MR = 32, NR = 12 };

static size_t round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }

static size_t cache_bytes(int name, size_t fallback) {
    long v = sysconf(name);
    return v > 0 ? (size_t)v : fallback;
}

static int have_vnni(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw");
}

static int have_avx512f(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f");
}

static int have_bf16(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512bf16") && __builtin_cpu_supports("avx512bw");
}

/* ------------------------------------------------------------------ families */

/* Where a microtile's results go: the tile origin in C, its valid extent, its
 * global coordinates (kernel frame, for per-channel epilogues) and whether
 * this is the first depth slice (the user's beta) or a later one (beta 1). */
typedef struct {
    void *c;
    ptrdiff_t rsc, csc;
    size_t mr, nr;
    size_t row0, col0;
    int first;
    const void *epi;
} tile_out;

typedef struct {
    int q;    /* depth steps per packed group (4 i8, 2 bf16, 1 f32) */
    int esz;  /* bytes per element, source and packed */
    void (*pack_a)(void *dst, const void *a, ptrdiff_t rsa, ptrdiff_t csa, size_t mc, size_t kc);
    void (*pack_b)(void *dst, const void *b, ptrdiff_t rsb, ptrdiff_t csb, size_t kc, size_t nr_eff);
    void (*ukr)(size_t kc, const void *ap, const void *bp, const tile_out *o);
} family_t;

/* Generic k-group panel packs: per MR-row (NR-col) panel, per group of Q depth
 * steps, the panel's rows (cols) x Q contiguous elements; padding packs as 0
 * (through XFORM for the LHS: +128 for the VNNI family). */
#define DEFINE_PACKS(NAME, T, Q, XFORM)                                                      \
    static void pack_a_##NAME(void *dst_, const void *a_, ptrdiff_t rsa, ptrdiff_t csa,        \
                              size_t mc, size_t kc) {                                           \
        T *dst = (T *)dst_;                                                                     \
        const T *a = (const T *)a_;                                                             \
        size_t kq = round_up(kc, Q);                                                            \
        for (size_t ip = 0; ip < mc; ip += MR) {                                                \
            T *panel = dst + ip * kq;                                                           \
            for (size_t p = 0; p < kq; p += Q)                                                  \
                for (size_t r = 0; r < MR; ++r)                                                 \
                    for (size_t t = 0; t < Q; ++t) {                                            \
                        size_t i = ip + r, pp = p + t;                                          \
                        T v = (i < mc && pp < kc) ? a[(ptrdiff_t)i * rsa + (ptrdiff_t)pp * csa] \
                                                  : (T)0;                                       \
                        panel[p * MR + r * Q + t] = XFORM(v);                                   \
                    }                                                                           \
        }                                                                                       \
    }                                                                                           \
    static void pack_b_##NAME(void *dst_, const void *b_, ptrdiff_t rsb, ptrdiff_t csb,        \
                              size_t kc, size_t nr_eff) {                                       \
        T *dst = (T *)dst_;                                                                     \
        const T *b = (const T *)b_;                                                             \
        size_t kq = round_up(kc, Q);                                                            \
        for (size_t p = 0; p < kq; p += Q)                                                      \
            for (size_t j = 0; j < NR; ++j)                                                     \
                for (size_t t = 0; t < Q; ++t) {                                                \
                    size_t pp = p + t;                                                          \
                    dst[p * NR + j * Q + t] =                                                   \
                        (j < nr_eff && pp < kc) ? b[(ptrdiff_t)pp * rsb + (ptrdiff_t)j * csb]   \
                                                : (T)0;                                         \
                }                                                                               \
    }

#define XF_ID(v) (v)
#define XF_VNNI(v) ((int8_t)((uint8_t)((int)(v) + 128)))
DEFINE_PACKS(i8, int8_t, 4, XF_VNNI)
DEFINE_PACKS(bf16, uint16_t, 2, XF_ID)
DEFINE_PACKS(f32, float, 1, XF_ID)

/* ------------------------------------------------------------------ epilogues */

typedef struct { int32_t alpha, beta; } epi_i32;
typedef struct { float alpha, beta; } epi_f32;
typedef struct {
    float scale;
    const float *scales;   /* per-channel scales or NULL */
    const int32_t *bias;   /* per-channel bias or NULL */
    int axis;              /* 0: channel = kernel row, 1: channel = kernel column */
    int32_t zp, lo, hi;
} epi_q8;

/* KRequantize::apply (src/kernel/epilogue.rs:810-830): rne(f64(acc wrapping+
 * bias) * f64(scale)) saturated to i64, saturating + zp, clamped to [lo, hi]. */
static inline int32_t requant(int32_t acc, int32_t bias, float scale, int32_t zp, int32_t lo,
                              int32_t hi) {
    int32_t v = (int32_t)((uint32_t)acc + (uint32_t)bias);
    double x = nearbyint((double)v * (double)scale);  /* round-half-even (default mode) */
    int64_t q;
    if (x != x) q = 0;
    else if (x >= 9223372036854775808.0) q = INT64_MAX;
    else if (x < -9223372036854775808.0) q = INT64_MIN;
    else q = (int64_t)x;
    int64_t r;
    if (__builtin_add_overflow(q, (int64_t)zp, &r)) r = zp > 0 ? INT64_MAX : INT64_MIN;
    if (r < lo) r = lo;
    if (r > hi) r = hi;
    return (int32_t)r;
}

/* acc: NR x MR, column j at acc + j*MR. */
static void store_i32(const int32_t *acc, const tile_out *o) {
    const epi_i32 *e = (const epi_i32 *)o->epi;
    int32_t beta = o->first ? e->beta : 1;
    int32_t *c = (int32_t *)o->c;
    for (size_t j = 0; j < o->nr; ++j)
        for (size_t i = 0; i < o->mr; ++i) {
            uint32_t v = (uint32_t)e->alpha * (uint32_t)acc[j * MR + i];
            int32_t *cp = c + (ptrdiff_t)i * o->rsc + (ptrdiff_t)j * o->csc;
            if (beta == 0) *cp = (int32_t)v;
            else if (beta == 1) *cp = (int32_t)((uint32_t)*cp + v);
            else *cp = (int32_t)((uint32_t)beta * (uint32_t)*cp + v);
        }
}

static void store_q8(const int32_t *acc, const tile_out *o) {
    const epi_q8 *e = (const epi_q8 *)o->epi;
    uint8_t *c = (uint8_t *)o->c;
    for (size_t j = 0; j < o->nr; ++j)
        for (size_t i = 0; i < o->mr; ++i) {
            size_t ch = e->axis ? o->col0 + j : o->row0 + i;
            float s = e->scales ? e->scales[ch] : e->scale;
            int32_t b = e->bias ? e->bias[ch] : 0;
            int32_t q = requant(acc[j * MR + i], b, s, e->zp, e->lo, e->hi);
            c[(ptrdiff_t)i * o->rsc + (ptrdiff_t)j * o->csc] = (uint8_t)(q & 0xFF);
        }
}

/* f32 output: C = alpha*acc (+ beta*C); later depth slices add. */
static void store_f32(const float *acc, const tile_out *o) {
    const epi_f32 *e = (const epi_f32 *)o->epi;
    float *c = (float *)o->c;
    for (size_t j = 0; j < o->nr; ++j)
        for (size_t i = 0; i < o->mr; ++i) {
            float v = e->alpha * acc[j * MR + i];
            float *cp = c + (ptrdiff_t)i * o->rsc + (ptrdiff_t)j * o->csc;
            if (!o->first) *cp = *cp + v;
            else if (e->beta == 0.0f) *cp = v;
            else *cp = fmaf(e->beta, *cp, v);
        }
}

/* --------------------------------------------------------------- microkernels */

__attribute__((target("avx512f,avx512bw,avx512vnni")))
static void vnni_tile(size_t kc, const int8_t *ap, const int8_t *bp, int32_t *tmp) {
    __m512i acc[NR][2];
    for (int j = 0; j < NR; ++j) acc[j][0] = acc[j][1] = _mm512_setzero_si512();
    size_t nq = round_up(kc, 4) / 4;
    int32_t colsum[NR] = {0};
    for (size_t q = 0; q < nq; ++q)
        for (int j = 0; j < NR; ++j) {
            const int8_t *s = bp + q * NR * 4 + j * 4;
            colsum[j] += s[0] + s[1] + s[2] + s[3];
        }
    for (size_t q = 0; q < nq; ++q) {
        __m512i a0 = _mm512_loadu_si512((const void *)(ap + q * MR * 4));
        __m512i a1 = _mm512_loadu_si512((const void *)(ap + q * MR * 4 + 64));
        const int8_t *bq = bp + q * NR * 4;
        for (int j = 0; j < NR; ++j) {
            int32_t bw;
            memcpy(&bw, bq + j * 4, 4);
            __m512i bj = _mm512_set1_epi32(bw);
            acc[j][0] = _mm512_dpbusd_epi32(acc[j][0], a0, bj);
            acc[j][1] = _mm512_dpbusd_epi32(acc[j][1], a1, bj);
        }
    }
    for (int j = 0; j < NR; ++j) {
        __m512i corr = _mm512_set1_epi32((int32_t)(128u * (uint32_t)colsum[j]));
        _mm512_storeu_si512((void *)(tmp + j * MR), _mm512_sub_epi32(acc[j][0], corr));
        _mm512_storeu_si512((void *)(tmp + j * MR + 16), _mm512_sub_epi32(acc[j][1], corr));
    }
}

/* Widen kernel (IntGemm): sign-extended products, ascending k, wrapping.  The
 * packed A carries +128, removed on read. */
static void widen_tile(size_t kc, const int8_t *ap, const int8_t *bp, int32_t *tmp) {
    uint32_t acc[NR * MR];
    memset(acc, 0, sizeof acc);
    size_t nq = round_up(kc, 4) / 4;
    for (size_t q = 0; q < nq; ++q)
        for (int t = 0; t < 4; ++t)
            for (int j = 0; j < NR; ++j) {
                int32_t bv = bp[q * NR * 4 + j * 4 + t];
                for (int i = 0; i < MR; ++i)
                    acc[j * MR + i] +=
                        (uint32_t)(((int32_t)(uint8_t)ap[q * MR * 4 + i * 4 + t] - 128) * bv);
            }
    memcpy(tmp, acc, sizeof acc);
}

static int g_vnni = -1, g_avx512 = -1, g_bf16 = -1;

static void ukr_i8(size_t kc, const void *ap, const void *bp, const tile_out *o) {
    int32_t tmp[NR * MR];
    if (g_vnni) vnni_tile(kc, (const int8_t *)ap, (const int8_t *)bp, tmp);
    else widen_tile(kc, (const int8_t *)ap, (const int8_t *)bp, tmp);
    store_i32(tmp, o);
}

static void ukr_q8(size_t kc, const void *ap, const void *bp, const tile_out *o) {
    int32_t tmp[NR * MR];
    if (g_vnni) vnni_tile(kc, (const int8_t *)ap, (const int8_t *)bp, tmp);
    else widen_tile(kc, (const int8_t *)ap, (const int8_t *)bp, tmp);
    store_q8(tmp, o);
}

__attribute__((target("avx512f")))
static void f32_tile_avx512(size_t kc, const float *ap, const float *bp, float *tmp) {
    __m512 acc[NR][2];
    for (int j = 0; j < NR; ++j) acc[j][0] = acc[j][1] = _mm512_setzero_ps();
    for (size_t p = 0; p < kc; ++p) {
        __m512 a0 = _mm512_loadu_ps(ap + p * MR), a1 = _mm512_loadu_ps(ap + p * MR + 16);
        const float *bq = bp + p * NR;
        for (int j = 0; j < NR; ++j) {
            __m512 bj = _mm512_set1_ps(bq[j]);
            acc[j][0] = _mm512_fmadd_ps(a0, bj, acc[j][0]);
            acc[j][1] = _mm512_fmadd_ps(a1, bj, acc[j][1]);
        }
    }
    for (int j = 0; j < NR; ++j) {
        _mm512_storeu_ps(tmp + j * MR, acc[j][0]);
        _mm512_storeu_ps(tmp + j * MR + 16, acc[j][1]);
    }
}

static void f32_tile_scalar(size_t kc, const float *ap, const float *bp, float *tmp) {
    float acc[NR * MR];
    memset(acc, 0, sizeof acc);
    for (size_t p = 0; p < kc; ++p)
        for (int j = 0; j < NR; ++j)
            for (int i = 0; i < MR; ++i)
                acc[j * MR + i] = fmaf(ap[p * MR + i], bp[p * NR + j], acc[j * MR + i]);
    memcpy(tmp, acc, sizeof acc);
}

static void ukr_f32(size_t kc, const void *ap, const void *bp, const tile_out *o) {
    float tmp[NR * MR];
    if (g_avx512) f32_tile_avx512(kc, (const float *)ap, (const float *)bp, tmp);
    else f32_tile_scalar(kc, (const float *)ap, (const float *)bp, tmp);
    store_f32(tmp, o);
}

__attribute__((target("avx512f,avx512bw,avx512bf16")))
static void bf16_tile_dot(size_t kc, const uint16_t *ap, const uint16_t *bp, float *tmp) {
    __m512 acc[NR][2];
    for (int j = 0; j < NR; ++j) acc[j][0] = acc[j][1] = _mm512_setzero_ps();
    size_t npairs = (kc + 1) / 2;
    for (size_t p2 = 0; p2 < npairs; ++p2) {
        __m512bh a0 = (__m512bh)_mm512_loadu_si512((const void *)(ap + p2 * MR * 2));
        __m512bh a1 = (__m512bh)_mm512_loadu_si512((const void *)(ap + p2 * MR * 2 + 32));
        const uint16_t *bq = bp + p2 * NR * 2;
        for (int j = 0; j < NR; ++j) {
            int32_t bw;
            memcpy(&bw, bq + j * 2, 4);
            __m512bh bj = (__m512bh)_mm512_set1_epi32(bw);
            acc[j][0] = _mm512_dpbf16_ps(acc[j][0], a0, bj);
            acc[j][1] = _mm512_dpbf16_ps(acc[j][1], a1, bj);
        }
    }
    for (int j = 0; j < NR; ++j) {
        _mm512_storeu_ps(tmp + j * MR, acc[j][0]);
        _mm512_storeu_ps(tmp + j * MR + 16, acc[j][1]);
    }
}

static inline float bf16_widen(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* MixedGemm<bf16> widen path: exact f32 widening, ascending-k FMA chains. */
static void bf16_tile_widen(size_t kc, const uint16_t *ap, const uint16_t *bp, float *tmp) {
    float acc[NR * MR];
    memset(acc, 0, sizeof acc);
    size_t npairs = (kc + 1) / 2;
    for (size_t p2 = 0; p2 < npairs; ++p2)
        for (int t = 0; t < 2; ++t)
            for (int j = 0; j < NR; ++j) {
                float bv = bf16_widen(bp[p2 * NR * 2 + j * 2 + t]);
                for (int i = 0; i < MR; ++i)
                    acc[j * MR + i] =
                        fmaf(bf16_widen(ap[p2 * MR * 2 + i * 2 + t]), bv, acc[j * MR + i]);
            }
    memcpy(tmp, acc, sizeof acc);
}

static void ukr_bf16(size_t kc, const void *ap, const void *bp, const tile_out *o) {
    float tmp[NR * MR];
    if (g_bf16) bf16_tile_dot(kc, (const uint16_t *)ap, (const uint16_t *)bp, tmp);
    else bf16_tile_widen(kc, (const uint16_t *)ap, (const uint16_t *)bp, tmp);
    store_f32(tmp, o);
}

static const family_t FAM_I8 = {4, 1, pack_a_i8, pack_b_i8, ukr_i8};
static const family_t FAM_Q8 = {4, 1, pack_a_i8, pack_b_i8, ukr_q8};
static const family_t FAM_F32 = {1, 4, pack_a_f32, pack_b_f32, ukr_f32};
static const family_t FAM_BF16 = {2, 2, pack_a_bf16, pack_b_bf16, ukr_bf16};

static void isa_init(void) {
    if (g_vnni < 0) g_vnni = have_vnni();
    if (g_avx512 < 0) g_avx512 = have_avx512f();
    if (g_bf16 < 0) g_bf16 = have_bf16();
}

/* ------------------------------------------------------------------- driver */

/* Blocking in the spirit of src/cache.rs:412-470: kc keeps the A and B
 * micropanels in L1, mc fits the A macro-panel in L2, nc the B macro-panel in
 * L3.  `whole_k` fixes kc = k (the requantizing and bf16-dot families). */
static void blocking(const family_t *f, size_t m, size_t n, size_t k, int whole_k, size_t *mc,
                     size_t *kc, size_t *nc) {
    size_t l1 = cache_bytes(_SC_LEVEL1_DCACHE_SIZE, 48 * 1024);
    size_t l2 = cache_bytes(_SC_LEVEL2_CACHE_SIZE, 2 * 1024 * 1024);
    size_t l3 = cache_bytes(_SC_LEVEL3_CACHE_SIZE, 32 * 1024 * 1024);
    size_t q = (size_t)f->q, esz = (size_t)f->esz;
    size_t kk;
    if (whole_k) {
        kk = round_up(k, q);
    } else {
        kk = l1 / 2 / ((MR + NR) * esz);
        kk = kk < 256 ? 256 : kk;
        kk = round_up(kk, q);
        if (kk > k) kk = round_up(k, q);
        size_t kiter = (k + kk - 1) / kk;
        kk = round_up((k + kiter - 1) / kiter, q);
    }
    size_t mm = (l2 / 2) / (kk * esz) / MR * MR;
    if (mm < MR) mm = MR;
    if (mm > round_up(m, MR)) mm = round_up(m, MR);
    size_t nn = (l3 / 4) / (kk * esz) / NR * NR;
    if (nn < NR) nn = NR;
    if (nn > round_up(n, NR)) nn = round_up(n, NR);
    *mc = mm; *kc = kk; *nc = nn;
}

/* The 5-loop over a kernel-frame product (C row index = A row).  `bpacked`:
 * the whole B already packed with kc = k (NR-column panels, each kq x NR),
 * then whole_k must be set.  `nt` threads. */
static void run_blis(const family_t *f, size_t m, size_t k, size_t n, const void *a,
                     ptrdiff_t rsa, ptrdiff_t csa, const void *b, ptrdiff_t rsb, ptrdiff_t csb,
                     void *c, ptrdiff_t rsc, ptrdiff_t csc, size_t osz, const void *epi,
                     int whole_k, const void *bpacked, int nt) {
    size_t mc, kc, nc;
    blocking(f, m, n, k, whole_k || bpacked, &mc, &kc, &nc);
    if (bpacked) nc = round_up(n, NR);
    const size_t esz = (size_t)f->esz, q = (size_t)f->q;
    const size_t kq = round_up(kc, q);
    const size_t n_mc = (m + mc - 1) / mc;
    uint8_t *apack = (uint8_t *)aligned_alloc(64, round_up(n_mc * mc * kq * esz, 64));
    uint8_t *bpack = bpacked ? NULL
                             : (uint8_t *)aligned_alloc(64, round_up(round_up(nc, NR) * kq * esz, 64));
    for (size_t jc = 0; jc < n; jc += nc) {
        size_t nc_eff = n - jc < nc ? n - jc : nc;
        size_t n_nt = (nc_eff + NR - 1) / NR;
        for (size_t pc = 0; pc < k; pc += kc) {
            size_t kc_eff = k - pc < kc ? k - pc : kc;
            size_t kq_eff = round_up(kc_eff, q);
            const uint8_t *bbase = bpacked ? (const uint8_t *)bpacked + (jc / NR) * kq_eff * NR * esz
                                           : bpack;
            #pragma omp parallel num_threads(nt)
            {
                if (!bpacked) {
                    #pragma omp for schedule(static)
                    for (ptrdiff_t jt = 0; jt < (ptrdiff_t)n_nt; ++jt) {
                        size_t col = jc + jt * NR;
                        size_t nr_eff = nc_eff - jt * NR < NR ? nc_eff - jt * NR : NR;
                        f->pack_b(bpack + jt * kq_eff * NR * esz,
                                  (const uint8_t *)b + ((ptrdiff_t)pc * rsb + (ptrdiff_t)col * csb) *
                                                           (ptrdiff_t)esz,
                                  rsb, csb, kc_eff, nr_eff);
                    }
                }
                #pragma omp for schedule(static)
                for (ptrdiff_t ic = 0; ic < (ptrdiff_t)n_mc; ++ic) {
                    size_t mc_eff = m - ic * mc < mc ? m - ic * mc : mc;
                    f->pack_a(apack + ic * mc * kq_eff * esz,
                              (const uint8_t *)a + ((ptrdiff_t)(ic * mc) * rsa + (ptrdiff_t)pc * csa) *
                                                       (ptrdiff_t)esz,
                              rsa, csa, mc_eff, kc_eff);
                }
                size_t n_mt_per = mc / MR;
                size_t jobs = n_mc * n_mt_per * n_nt;
                #pragma omp for schedule(dynamic, 4)
                for (ptrdiff_t job = 0; job < (ptrdiff_t)jobs; ++job) {
                    size_t jt = job % n_nt;
                    size_t it = job / n_nt;
                    size_t row = it * MR;
                    if (row >= m) continue;
                    size_t ic = row / mc;
                    size_t col = jc + jt * NR;
                    tile_out o;
                    o.c = (uint8_t *)c + ((ptrdiff_t)row * rsc + (ptrdiff_t)col * csc) * (ptrdiff_t)osz;
                    o.rsc = rsc;
                    o.csc = csc;
                    o.mr = m - row < MR ? m - row : MR;
                    o.nr = nc_eff - jt * NR < NR ? nc_eff - jt * NR : NR;
                    o.row0 = row;
                    o.col0 = col;
                    o.first = pc == 0;
                    o.epi = epi;
                    const uint8_t *ap = apack + (ic * mc * kq_eff + (row - ic * mc) * kq_eff) * esz;
                    const uint8_t *bp = bbase + jt * kq_eff * NR * esz;
                    f->ukr(kc_eff, ap, bp, &o);
                }
            }
        }
    }
    free(apack);
    free(bpack);
}

static int threads_of(int threads) { return threads > 0 ? threads : omp_get_max_threads(); }

/* orient_swap: a row-major-ish C computes C^T = B^T A^T. */
static int swap_wanted(ptrdiff_t rsc, ptrdiff_t csc) {
    return (csc < 0 ? -csc : csc) < (rsc < 0 ? -rsc : rsc);
}

/* ------------------------------------------------------------------ entries */

/* gemm_i8_unchecked (src/api/int8.rs:86-178).  `threads` 0 = all (Rayon(0)),
 * 1 = Serial, n = Rayon(n).  Returns the number of OpenMP threads used. */
PORT_API int port_gemm_i8(size_t m, size_t k, size_t n, int32_t alpha,
                          const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa,
                          const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb,
                          int32_t beta, int32_t *c, ptrdiff_t rsc, ptrdiff_t csc,
                          int threads) {
    int nt = threads_of(threads);
    isa_init();
    if (m == 0 || n == 0) return nt;
    if (k == 0 || alpha == 0) {
        for (size_t j = 0; j < n; ++j)
            for (size_t i = 0; i < m; ++i) {
                int32_t *p = c + (ptrdiff_t)i * rsc + (ptrdiff_t)j * csc;
                if (beta == 0) *p = 0;
                else if (beta != 1) *p = (int32_t)((uint32_t)beta * (uint32_t)*p);
            }
        return nt;
    }
    if (swap_wanted(rsc, csc)) {
        size_t t = m; m = n; n = t;
        const int8_t *tp = a; a = b; b = tp;
        ptrdiff_t o_rsa = rsa, o_csa = csa;
        rsa = csb; csa = rsb; rsb = o_csa; csb = o_rsa;
        ptrdiff_t ts = rsc; rsc = csc; csc = ts;
    }
    epi_i32 e = {alpha, beta};
    run_blis(&FAM_I8, m, k, n, a, rsa, csa, b, rsb, csb, c, rsc, csc, 4, &e, 0, NULL, nt);
    return nt;
}

/* A B operand packed once for the requantizing kernel (kc = k): the reference's
 * prepack_rhs_i8 (src/api/packed.rs:372-470) in the VNNI panel layout. */
typedef struct {
    size_t k, n;
    int8_t *buf;
} port_packed_b;

PORT_API void *port_prepack_b_i8(size_t k, size_t n, const int8_t *b, ptrdiff_t rsb,
                                 ptrdiff_t csb, int threads) {
    int nt = threads_of(threads);
    port_packed_b *p = (port_packed_b *)calloc(1, sizeof *p);
    size_t kq = round_up(k > 0 ? k : 1, 4), npan = (n + NR - 1) / NR;
    p->k = k;
    p->n = n;
    p->buf = (int8_t *)aligned_alloc(64, round_up(npan * kq * NR, 64));
    #pragma omp parallel for num_threads(nt) schedule(static)
    for (ptrdiff_t jt = 0; jt < (ptrdiff_t)npan; ++jt) {
        size_t col = jt * NR, nr_eff = n - col < NR ? n - col : NR;
        pack_b_i8(p->buf + jt * kq * NR, b + (ptrdiff_t)col * csb, rsb, csb, k, nr_eff);
    }
    return p;
}

PORT_API void port_packed_b_free(void *h) {
    port_packed_b *p = (port_packed_b *)h;
    if (!p) return;
    free(p->buf);
    free(p);
}

/* The requantizing GEMM (gemm_i8_requant(_u8)_unchecked, src/api/int8.rs:347-457,
 * :562-672, composed as execute_int_requant, src/dispatch/int.rs:672-799):
 * alpha 1, beta 0, kc = k, the map applied to each drained tile.  axis: 0 =
 * channel per row of C (length m), 1 = per column (length n).  lo/hi: the
 * clamp band, ReLU already folded into lo.  `packed` (from port_prepack_b_i8)
 * replaces b when non-NULL; the packed operand fixes the roles, so no
 * orientation swap happens then and C is written through its strides as
 * given. */
PORT_API int port_gemm_i8_requant(size_t m, size_t k, size_t n, const int8_t *a, ptrdiff_t rsa,
                                  ptrdiff_t csa, const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb,
                                  const void *packed, float scale, const float *scales,
                                  int32_t zp, const int32_t *bias, int axis, int32_t lo,
                                  int32_t hi, uint8_t *c, ptrdiff_t rsc, ptrdiff_t csc,
                                  int threads) {
    int nt = threads_of(threads);
    isa_init();
    if (m == 0 || n == 0) return nt;
    epi_q8 e = {scale, scales, bias, axis, zp, lo, hi};
    if (k == 0) {
        for (size_t i = 0; i < m; ++i)
            for (size_t j = 0; j < n; ++j) {
                size_t ch = axis ? j : i;
                int32_t q = requant(0, bias ? bias[ch] : 0, scales ? scales[ch] : scale, zp, lo, hi);
                c[(ptrdiff_t)i * rsc + (ptrdiff_t)j * csc] = (uint8_t)(q & 0xFF);
            }
        return nt;
    }
    if (!packed && swap_wanted(rsc, csc)) {
        size_t t = m; m = n; n = t;
        const int8_t *tp = a; a = b; b = tp;
        ptrdiff_t o_rsa = rsa, o_csa = csa;
        rsa = csb; csa = rsb; rsb = o_csa; csb = o_rsa;
        ptrdiff_t ts = rsc; rsc = csc; csc = ts;
        e.axis ^= 1;
    }
    const port_packed_b *pb = (const port_packed_b *)packed;
    run_blis(&FAM_Q8, m, k, n, a, rsa, csa, b, rsb, csb, c, rsc, csc, 1, &e, 1,
             pb ? pb->buf : NULL, nt);
    return nt;
}

/* gemm_unchecked for f32 (src/api.rs:469-580) on FloatGemm<f32>. */
PORT_API int port_gemm_f32(size_t m, size_t k, size_t n, float alpha, const float *a,
                           ptrdiff_t rsa, ptrdiff_t csa, const float *b, ptrdiff_t rsb,
                           ptrdiff_t csb, float beta, float *c, ptrdiff_t rsc, ptrdiff_t csc,
                           int threads) {
    int nt = threads_of(threads);
    isa_init();
    if (m == 0 || n == 0) return nt;
    if (k == 0 || alpha == 0.0f) {
        for (size_t j = 0; j < n; ++j)
            for (size_t i = 0; i < m; ++i) {
                float *p = c + (ptrdiff_t)i * rsc + (ptrdiff_t)j * csc;
                *p = beta == 0.0f ? 0.0f : (beta == 1.0f ? *p : beta * *p);
            }
        return nt;
    }
    if (swap_wanted(rsc, csc)) {
        size_t t = m; m = n; n = t;
        const float *tp = a; a = b; b = tp;
        ptrdiff_t o_rsa = rsa, o_csa = csa;
        rsa = csb; csa = rsb; rsb = o_csa; csb = o_rsa;
        ptrdiff_t ts = rsc; rsc = csc; csc = ts;
    }
    epi_f32 e = {alpha, beta};
    run_blis(&FAM_F32, m, k, n, a, rsa, csa, b, rsb, csb, c, rsc, csc, 4, &e, 0, NULL, nt);
    return nt;
}

/* One bf16 product with f32 output (the attention-score form: f32
 * accumulation, alpha*acc + beta*C with no narrowing). */
static void bf16_f32out_one(size_t m, size_t k, size_t n, float alpha, const uint16_t *a,
                            ptrdiff_t rsa, ptrdiff_t csa, const uint16_t *b, ptrdiff_t rsb,
                            ptrdiff_t csb, float beta, float *c, ptrdiff_t rsc, ptrdiff_t csc,
                            int nt) {
    if (m == 0 || n == 0) return;
    if (k == 0 || alpha == 0.0f) {
        for (size_t j = 0; j < n; ++j)
            for (size_t i = 0; i < m; ++i) {
                float *p = c + (ptrdiff_t)i * rsc + (ptrdiff_t)j * csc;
                *p = beta == 0.0f ? 0.0f : (beta == 1.0f ? *p : beta * *p);
            }
        return;
    }
    if (swap_wanted(rsc, csc)) {
        size_t t = m; m = n; n = t;
        const uint16_t *tp = a; a = b; b = tp;
        ptrdiff_t o_rsa = rsa, o_csa = csa;
        rsa = csb; csa = rsb; rsb = o_csa; csb = o_rsa;
        ptrdiff_t ts = rsc; rsc = csc; csc = ts;
    }
    epi_f32 e = {alpha, beta};
    run_blis(&FAM_BF16, m, k, n, a, rsa, csa, b, rsb, csb, c, rsc, csc, 4, &e, 1, NULL, nt);
}

/* gemm_batched over bf16 with f32 output (src/api/batched.rs:188-283,
 * src/special/batched.rs:49-141): a batch of at least as many elements as
 * threads runs one element per worker, each serially; a shorter batch runs
 * its elements one after another with every thread. */
PORT_API int port_gemm_batched_bf16_f32out(size_t batch, size_t m, size_t k, size_t n,
                                           float alpha, const uint16_t *a, ptrdiff_t rsa,
                                           ptrdiff_t csa, ptrdiff_t a_bs, const uint16_t *b,
                                           ptrdiff_t rsb, ptrdiff_t csb, ptrdiff_t b_bs,
                                           float beta, float *c, ptrdiff_t rsc, ptrdiff_t csc,
                                           ptrdiff_t c_bs, int threads) {
    int nt = threads_of(threads);
    isa_init();
    if (batch >= (size_t)nt && nt > 1) {
        #pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
        for (ptrdiff_t z = 0; z < (ptrdiff_t)batch; ++z)
            bf16_f32out_one(m, k, n, alpha, a + z * a_bs, rsa, csa, b + z * b_bs, rsb, csb, beta,
                            c + z * c_bs, rsc, csc, 1);
    } else {
        for (size_t z = 0; z < batch; ++z)
            bf16_f32out_one(m, k, n, alpha, a + (ptrdiff_t)z * a_bs, rsa, csa,
                            b + (ptrdiff_t)z * b_bs, rsb, csb, beta, c + (ptrdiff_t)z * c_bs, rsc,
                            csc, nt);
    }
    return nt;
}

__attribute__((target("avx512f")))
static void dot_rows4_avx512(size_t k, const float *const rows[4], const float *x, float out[4]) {
    __m512 acc[4] = {_mm512_setzero_ps(), _mm512_setzero_ps(), _mm512_setzero_ps(),
                     _mm512_setzero_ps()};
    size_t p = 0;
    for (; p + 16 <= k; p += 16) {
        __m512 xv = _mm512_loadu_ps(x + p);
        for (int r = 0; r < 4; ++r) acc[r] = _mm512_fmadd_ps(_mm512_loadu_ps(rows[r] + p), xv, acc[r]);
    }
    for (int r = 0; r < 4; ++r) {
        float s = _mm512_reduce_add_ps(acc[r]);
        for (size_t t = p; t < k; ++t) s = fmaf(rows[r][t], x[t], s);
        out[r] = s;
    }
}

static void dot_rows4_scalar(size_t k, const float *const rows[4], const float *x, float out[4]) {
    for (int r = 0; r < 4; ++r) {
        float s = 0.0f;
        for (size_t t = 0; t < k; ++t) s = fmaf(rows[r][t], x[t], s);
        out[r] = s;
    }
}

/* The f32 GEMV y = alpha*A*x + beta*y for a row-major A (gemv::core_epi /
 * dot_rows, src/special/gemv.rs:101-258, :511-600): rows split across
 * threads, four at a time; unit-stride x. */
PORT_API int port_gemv_f32(size_t rows, size_t k, float alpha, const float *a, ptrdiff_t lda,
                           const float *x, float beta, float *y, ptrdiff_t ys, int threads) {
    int nt = threads_of(threads);
    isa_init();
    size_t nblk = (rows + 3) / 4;
    #pragma omp parallel for num_threads(nt) schedule(static)
    for (ptrdiff_t bi = 0; bi < (ptrdiff_t)nblk; ++bi) {
        size_t r0 = (size_t)bi * 4;
        const float *rp[4];
        for (int r = 0; r < 4; ++r) {
            size_t row = r0 + r < rows ? r0 + r : rows - 1;
            rp[r] = a + (ptrdiff_t)row * lda;
        }
        float d[4];
        if (g_avx512) dot_rows4_avx512(k, rp, x, d);
        else dot_rows4_scalar(k, rp, x, d);
        for (int r = 0; r < 4 && r0 + r < rows; ++r) {
            float *yp = y + (ptrdiff_t)(r0 + r) * ys;
            float v = alpha * d[r];
            *yp = beta == 0.0f ? v : beta * *yp + v;
        }
    }
    return nt;
}

PORT_API int port_has_vnni(void) { return have_vnni(); }
PORT_API int port_has_avx512f(void) { return have_avx512f(); }
PORT_API int port_has_bf16(void) { return have_bf16(); }
PORT_API int port_max_threads(void) { return omp_get_max_threads(); }
