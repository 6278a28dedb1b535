/*
 * cpu_port.c -- C restatement of gemmkit's CPU i8 -> i32 GEMM path, used only as
 * the timed CPU baseline beside the GPU numbers (and checked bit-exact against
 * the closed form in oracle.c by tests/test_oracle.py).
 *
 * TEST INFRASTRUCTURE ONLY: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library never does.
 *
 * What it restates:
 *   - orientation swap when C is row-major-ish (src/dispatch.rs:395-417)
 *   - the BLIS 5-loop: jc (nc) -> pc (kc) -> pack B -> pack A -> (ic, jr) jobs
 *     (src/driver.rs:402-944)
 *   - the IntGemmVnni family (src/kernel/int.rs:386-490): A packed k-quad
 *     interleaved with +128 (vnni_a_xform), B packed k-quad interleaved signed,
 *     32x12 microtile of vpdpbusd with the -128*colsum(B) correction
 *     (src/simd/avx512.rs:483-545)
 *   - int32_epilogue (src/kernel/int.rs:36-120): alpha fold, beta 0/1/other, all
 *     wrapping, beta -> 1 after the first depth slice (src/driver.rs:725-730)
 *   - the analytical blocking of src/cache.rs:412-470 with this host's caches
 * Threads: OpenMP stands in for rayon's fork-join (src/parallel.rs:602-700).
 * When the host lacks AVX-512 VNNI the widen kernel (IntGemm,
 * src/kernel/int.rs:138-190) runs instead, as the reference's select_i8 does.
 */
#include <stdint.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include <immintrin.h>
#include <omp.h>

#define PORT_API __attribute__((visibility("default")))

enum { MR = 32, NR = 12, Q = 4 };

static size_t round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }

static size_t cache_bytes(int name, size_t fallback) {
    long v = sysconf(name);
    return v > 0 ? (size_t)v : fallback;
}

/* Blocking in the spirit of src/cache.rs:412-470: kc keeps the A and B
 * micropanels in L1, mc fits the A macro-panel in L2, nc the B macro-panel in L3;
 * i8 results do not depend on these choices. */
static void blocking(size_t m, size_t n, size_t k, size_t *mc, size_t *kc, size_t *nc) {
    size_t l1 = cache_bytes(_SC_LEVEL1_DCACHE_SIZE, 48 * 1024);
    size_t l2 = cache_bytes(_SC_LEVEL2_CACHE_SIZE, 2 * 1024 * 1024);
    size_t l3 = cache_bytes(_SC_LEVEL3_CACHE_SIZE, 32 * 1024 * 1024);
    size_t kk = l1 / 2 / (MR + NR);
    kk = kk < 256 ? 256 : kk;
    kk = round_up(kk, Q);
    if (kk > k) kk = round_up(k, Q);
    size_t kiter = (k + kk - 1) / kk;
    kk = round_up((k + kiter - 1) / kiter, Q);
    size_t mm = (l2 / 2) / kk / MR * MR;
    if (mm < MR) mm = MR;
    if (mm > round_up(m, MR)) mm = round_up(m, MR);
    size_t nn = (l3 / 4) / kk / NR * NR;
    if (nn < NR) nn = NR;
    if (nn > round_up(n, NR)) nn = round_up(n, NR);
    *mc = mm; *kc = kk; *nc = nn;
}

/* Pack an mc x kc block of A: per MR-row panel, per k quad, MR rows x 4 bytes,
 * each byte offset by +128 (so vpdpbusd sees it unsigned).  Padding packs as
 * 0 + 128, which the colsum correction cancels (pad B is 0). */
static void pack_a(uint8_t *dst, const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa,
                   size_t mc, size_t kc) {
    size_t kq = round_up(kc, Q);
    for (size_t ip = 0; ip < mc; ip += MR) {
        uint8_t *panel = dst + ip * kq;
        for (size_t p = 0; p < kq; p += Q)
            for (size_t r = 0; r < MR; ++r)
                for (size_t t = 0; t < Q; ++t) {
                    size_t i = ip + r, pp = p + t;
                    int v = (i < mc && pp < kc) ? a[(ptrdiff_t)i * rsa + (ptrdiff_t)pp * csa] : 0;
                    panel[p * MR + r * Q + t] = (uint8_t)(v + 128);
                }
    }
}

/* Pack a kc x nc block of B: per NR-column panel, per k quad, NR cols x 4 bytes. */
static void pack_b_panel(int8_t *dst, const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb,
                         size_t kc, size_t nr_eff) {
    size_t kq = round_up(kc, Q);
    for (size_t p = 0; p < kq; p += Q)
        for (size_t j = 0; j < NR; ++j)
            for (size_t t = 0; t < Q; ++t) {
                size_t pp = p + t;
                dst[p * NR + j * Q + t] =
                    (j < nr_eff && pp < kc) ? b[(ptrdiff_t)pp * rsb + (ptrdiff_t)j * csb] : 0;
            }
}

typedef struct { int32_t alpha, beta; } epi_t;

static inline void store_tile(const int32_t *acc /* NR x MR, column-major */, int32_t *c,
                              ptrdiff_t rsc, ptrdiff_t csc, size_t mr_eff, size_t nr_eff,
                              int32_t alpha, int32_t beta) {
    for (size_t j = 0; j < nr_eff; ++j)
        for (size_t i = 0; i < mr_eff; ++i) {
            uint32_t v = (uint32_t)alpha * (uint32_t)acc[j * MR + i];
            int32_t *cp = c + (ptrdiff_t)i * rsc + (ptrdiff_t)j * csc;
            if (beta == 0) *cp = (int32_t)v;
            else if (beta == 1) *cp = (int32_t)((uint32_t)*cp + v);
            else *cp = (int32_t)((uint32_t)beta * (uint32_t)*cp + v);
        }
}

__attribute__((target("avx512f,avx512bw,avx512vnni")))
static void ukernel_vnni(size_t kc, const uint8_t *ap, const int8_t *bp, int32_t *c,
                         ptrdiff_t rsc, ptrdiff_t csc, size_t mr_eff, size_t nr_eff,
                         int32_t alpha, int32_t beta) {
    __m512i acc[NR][2];
    for (int j = 0; j < NR; ++j) acc[j][0] = acc[j][1] = _mm512_setzero_si512();
    size_t nq = round_up(kc, Q) / Q;
    int32_t colsum[NR] = {0};
    for (size_t q = 0; q < nq; ++q)
        for (int j = 0; j < NR; ++j) {
            const int8_t *s = bp + q * NR * Q + j * Q;
            colsum[j] += s[0] + s[1] + s[2] + s[3];
        }
    for (size_t q = 0; q < nq; ++q) {
        __m512i a0 = _mm512_loadu_si512((const void *)(ap + q * MR * Q));
        __m512i a1 = _mm512_loadu_si512((const void *)(ap + q * MR * Q + 64));
        const int8_t *bq = bp + q * NR * Q;
        for (int j = 0; j < NR; ++j) {
            int32_t bw;
            memcpy(&bw, bq + j * Q, 4);
            __m512i bj = _mm512_set1_epi32(bw);
            acc[j][0] = _mm512_dpbusd_epi32(acc[j][0], a0, bj);
            acc[j][1] = _mm512_dpbusd_epi32(acc[j][1], a1, bj);
        }
    }
    for (int j = 0; j < NR; ++j) {
        __m512i corr = _mm512_set1_epi32((int32_t)(128u * (uint32_t)colsum[j]));
        acc[j][0] = _mm512_sub_epi32(acc[j][0], corr);
        acc[j][1] = _mm512_sub_epi32(acc[j][1], corr);
    }
    if (mr_eff == MR && nr_eff == NR && rsc == 1 && beta == 0 && alpha == 1) {
        for (int j = 0; j < NR; ++j) {
            _mm512_storeu_si512((void *)(c + (ptrdiff_t)j * csc), acc[j][0]);
            _mm512_storeu_si512((void *)(c + (ptrdiff_t)j * csc + 16), acc[j][1]);
        }
        return;
    }
    int32_t tmp[NR * MR];
    for (int j = 0; j < NR; ++j) {
        _mm512_storeu_si512((void *)(tmp + j * MR), acc[j][0]);
        _mm512_storeu_si512((void *)(tmp + j * MR + 16), acc[j][1]);
    }
    store_tile(tmp, c, rsc, csc, mr_eff, nr_eff, alpha, beta);
}

/* Widen kernel (IntGemm): sign-extended i8 products, ascending k, wrapping. The
 * packed A still carries +128, removed on read. */
static void ukernel_widen(size_t kc, const uint8_t *ap, const int8_t *bp, int32_t *c,
                          ptrdiff_t rsc, ptrdiff_t csc, size_t mr_eff, size_t nr_eff,
                          int32_t alpha, int32_t beta) {
    uint32_t acc[NR * MR];
    memset(acc, 0, sizeof acc);
    size_t nq = round_up(kc, Q) / Q;
    for (size_t q = 0; q < nq; ++q)
        for (int t = 0; t < Q; ++t)
            for (int j = 0; j < NR; ++j) {
                int32_t bv = bp[q * NR * Q + j * Q + t];
                for (int i = 0; i < MR; ++i)
                    acc[j * MR + i] += (uint32_t)(((int32_t)ap[q * MR * Q + i * Q + t] - 128) * bv);
            }
    store_tile((const int32_t *)acc, c, rsc, csc, mr_eff, nr_eff, alpha, beta);
}

static int have_vnni(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw");
}

/* Returns the number of OpenMP threads used. `threads` 0 = all (Rayon(0)),
 * 1 = Serial, n = Rayon(n).  The contract is gemm_i8_unchecked's
 * (src/api/int8.rs:86-178). */
PORT_API int port_gemm_i8(size_t m, size_t k, size_t n, int32_t alpha,
                          const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa,
                          const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb,
                          int32_t beta, int32_t *c, ptrdiff_t rsc, ptrdiff_t csc,
                          int threads) {
    int nt = threads > 0 ? threads : omp_get_max_threads();
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
    /* orient_swap: row-major-ish C computes C^T = B^T A^T */
    if ((csc < 0 ? -csc : csc) < (rsc < 0 ? -rsc : rsc)) {
        size_t t = m; m = n; n = t;
        const int8_t *tp = a; a = b; b = tp;
        ptrdiff_t o_rsa = rsa, o_csa = csa;
        rsa = csb; csa = rsb; rsb = o_csa; csb = o_rsa;
        ptrdiff_t ts = rsc; rsc = csc; csc = ts;
    }
    size_t mc, kc, nc;
    blocking(m, n, k, &mc, &kc, &nc);
    int vnni = have_vnni();
    size_t kq = round_up(kc, Q);
    size_t n_mc = (m + mc - 1) / mc;
    uint8_t *apack = (uint8_t *)aligned_alloc(64, round_up(n_mc * mc * kq, 64));
    int8_t *bpack = (int8_t *)aligned_alloc(64, round_up(round_up(nc, NR) * kq, 64));
    for (size_t jc = 0; jc < n; jc += nc) {
        size_t nc_eff = n - jc < nc ? n - jc : nc;
        size_t n_nt = (nc_eff + NR - 1) / NR;
        for (size_t pc = 0; pc < k; pc += kc) {
            size_t kc_eff = k - pc < kc ? k - pc : kc;
            size_t kq_eff = round_up(kc_eff, Q);
            int32_t beta_eff = pc == 0 ? beta : 1;
            #pragma omp parallel num_threads(nt)
            {
                #pragma omp for schedule(static)
                for (ptrdiff_t jt = 0; jt < (ptrdiff_t)n_nt; ++jt) {
                    size_t col = jc + jt * NR;
                    size_t nr_eff = nc_eff - jt * NR < NR ? nc_eff - jt * NR : NR;
                    pack_b_panel(bpack + jt * kq_eff * NR,
                                 b + (ptrdiff_t)pc * rsb + (ptrdiff_t)col * csb,
                                 rsb, csb, kc_eff, nr_eff);
                }
                #pragma omp for schedule(static)
                for (ptrdiff_t ic = 0; ic < (ptrdiff_t)n_mc; ++ic) {
                    size_t mc_eff = m - ic * mc < mc ? m - ic * mc : mc;
                    pack_a(apack + ic * mc * kq_eff,
                           a + (ptrdiff_t)(ic * mc) * rsa + (ptrdiff_t)pc * csa,
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
                    size_t mr_eff = m - row < MR ? m - row : MR;
                    size_t col = jc + jt * NR;
                    size_t nr_eff = nc_eff - jt * NR < NR ? nc_eff - jt * NR : NR;
                    const uint8_t *ap = apack + ic * mc * kq_eff + (row - ic * mc) * kq_eff;
                    const int8_t *bp = bpack + jt * kq_eff * NR;
                    int32_t *cp = c + (ptrdiff_t)row * rsc + (ptrdiff_t)col * csc;
                    if (vnni)
                        ukernel_vnni(kc_eff, ap, bp, cp, rsc, csc, mr_eff, nr_eff,
                                     alpha, beta_eff);
                    else
                        ukernel_widen(kc_eff, ap, bp, cp, rsc, csc, mr_eff, nr_eff,
                                      alpha, beta_eff);
                }
            }
        }
    }
    free(apack);
    free(bpack);
    return nt;
}

PORT_API int port_has_vnni(void) { return have_vnni(); }
PORT_API int port_max_threads(void) { return omp_get_max_threads(); }
