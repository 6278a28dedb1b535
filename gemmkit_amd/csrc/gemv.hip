// gemv.hip -- HBM-bandwidth GEMV for skinny products (1..8 vectors).
//
// Replaces gemmkit's gemv route (src/special/gemv.rs:101-600, taken at
// m == 1 || n == 1 by src/dispatch/float.rs:81) and serves the i8 skinny shapes
// too (the reference has no i8 gemv: src/dispatch/int.rs:165-168; i8 results do
// not depend on the route because wrapping i32 addition is associative).
//
// out[j, r] = epi( sum_p mat[r, p] * vec[j, p] ),  r < R rows, j < nvec <= 8.
//
// The matrix streams from HBM exactly once, as 16-byte nontemporal loads; it is
// the only large operand, so the kernels are built around keeping enough of it
// in flight.  A row is split into 16-byte chunks; lane l of a wave owns chunks
// l, l+64, l+128, ... of every row it visits, so the vector chunks a lane
// multiplies are the same for every row.  Waves are persistent (a grid of a
// few workgroups per CU) and walk row groups with a grid stride:
//   * gemv_reg: rows of at most 64*CPL chunks.  Each lane loads its vector
//     chunks once into registers; the next row group's matrix loads are issued
//     before the current group is multiplied, so one group is always in flight
//     behind the arithmetic.
//   * gemv_wgrow: longer rows, one or two vectors.  The vectors are staged
//     once per workgroup in LDS and the whole workgroup reads one row at a
//     time, 32 KiB per batch, the next batch in flight behind the current.
//   * gemv_lds: longer rows, more vectors.  The vectors are staged in LDS and
//     each lane keeps UNROLL chunks per row in flight.
// Per-lane partial sums of the RPW x NV outputs of a row group are combined by
// a butterfly over the 64 lanes that halves the number of values each lane
// carries at every step (V values cost V-1 + log2(64/V) shuffles instead of
// 6*V), leaving output v on lanes [v*64/V, (v+1)*64/V).
#include <stdio.h>
#include <stdlib.h>

#include "epilogue.h"

namespace gk {

typedef int v4i_g __attribute__((ext_vector_type(4)));
typedef float v4f_g __attribute__((ext_vector_type(4)));

template <InType T>
struct Dot16;

template <>
struct Dot16<InType::I8> {
    using acc_t = int32_t;
    __device__ __forceinline__ static acc_t dot(v4i_g m, v4i_g x, acc_t acc) {
        acc = __builtin_amdgcn_sdot4(m[0], x[0], acc, false);
        acc = __builtin_amdgcn_sdot4(m[1], x[1], acc, false);
        acc = __builtin_amdgcn_sdot4(m[2], x[2], acc, false);
        acc = __builtin_amdgcn_sdot4(m[3], x[3], acc, false);
        return acc;
    }
};

template <>
struct Dot16<InType::F32> {
    using acc_t = float;
    __device__ __forceinline__ static acc_t dot(v4i_g m, v4i_g x, acc_t acc) {
        v4f_g a = __builtin_bit_cast(v4f_g, m), b = __builtin_bit_cast(v4f_g, x);
        acc = __builtin_fmaf(a[0], b[0], acc);
        acc = __builtin_fmaf(a[1], b[1], acc);
        acc = __builtin_fmaf(a[2], b[2], acc);
        acc = __builtin_fmaf(a[3], b[3], acc);
        return acc;
    }
};

template <>
struct Dot16<InType::BF16> {
    using acc_t = float;
    __device__ __forceinline__ static acc_t dot(v4i_g m, v4i_g x, acc_t acc) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t mu = (uint32_t)m[w], xu = (uint32_t)x[w];
            acc = __builtin_fmaf(__uint_as_float(mu << 16), __uint_as_float(xu << 16), acc);
            acc = __builtin_fmaf(__uint_as_float(mu & 0xFFFF0000u), __uint_as_float(xu & 0xFFFF0000u), acc);
        }
        return acc;
    }
};

// Butterfly over the wave: on entry v[0..V) are this lane's partial sums of V
// outputs; on exit v[0] holds the wave total of output (lane >> (6 - log2 V)).
template <int V, typename A>
__device__ __forceinline__ void wave_reduce(A (&v)[V]) {
    static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V must be a power of two <= 64");
    const int lane = threadIdx.x & 63;
    int n = V;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        if (n > 1) {
            const bool hi = (lane & off) != 0;
            const int h = n / 2;
#pragma unroll
            for (int i = 0; i < V / 2; ++i) {
                if (i < h) {
                    A send = hi ? v[i] : v[i + h];
                    A keep = hi ? v[i + h] : v[i];
                    v[i] = keep + __shfl_xor(send, off, 64);
                }
            }
            n = h;
        } else {
            v[0] += __shfl_xor(v[0], off, 64);
        }
    }
}

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / 64;

template <int V>
constexpr int log2c() {
    return V <= 1 ? 0 : 1 + log2c<V / 2>();
}

// Stores the reduced outputs of row group [r0, r0 + RPW): output index
// v = r*NV + j lives on lanes [v*64/V, ...); its first lane stores it.
template <InType T, EpiKind E, int NV, int RPW, typename A>
__device__ __forceinline__ void store_group(const GemvArgs &g, const EpiParams &ep, int64_t r0,
                                            const A (&v)[RPW * NV]) {
    constexpr int V = RPW * NV;
    constexpr int SH = 6 - log2c<V>();
    const int lane = threadIdx.x & 63;
    if ((lane & ((1 << SH) - 1)) == 0) {
        const int idx = lane >> SH;
        const int r = idx / NV, j = idx % NV;
        if (j < g.nvec && r0 + r < g.R) Store<E>::apply(ep, blockIdx.y, j, (int)(r0 + r), v[0]);
    }
}

template <InType T, EpiKind E, int NV, int CPL, int RPW>
__global__ __launch_bounds__(kGemvThreads) void gemv_reg(const GemvArgs g, const EpiParams ep) {
    using D = Dot16<T>;
    using acc_t = typename D::acc_t;
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    // A K*esz that is not a multiple of 16 only reaches this kernel through
    // the pack, which zero-fills both operands' rows up to the next 16 bytes.
    const int nch = (int)(((int64_t)g.K * esz + 15) / 16);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t zb = blockIdx.y;  // batch element
    const uint8_t *mat = (const uint8_t *)g.mat + zb * g.bsm * esz;
    const uint8_t *vec = (const uint8_t *)g.vec + zb * g.bsv * esz;
    const int64_t ld_b = g.ld * esz, vld_b = g.vld * esz;

    v4i_g x[NV][CPL];
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            const int c = lane + 64 * u;
            x[j][u] = (j < g.nvec && c < nch) ? *(const v4i_g *)(vec + j * vld_b + (int64_t)c * 16)
                                              : v4i_g{0, 0, 0, 0};
        }

    const int64_t groups = ((int64_t)g.R + RPW - 1) / RPW;
    const int64_t stride = (int64_t)gridDim.x * kGemvWaves;
    auto load = [&](int64_t grp, v4i_g (&m)[RPW][CPL]) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            int64_t row = grp * RPW + r;
            row = row < g.R ? row : g.R - 1;
            const uint8_t *p = mat + row * ld_b;
#pragma unroll
            for (int u = 0; u < CPL; ++u) {
                const int c = lane + 64 * u;
                m[r][u] = c < nch ? __builtin_nontemporal_load((const v4i_g *)(p + (int64_t)c * 16))
                                  : v4i_g{0, 0, 0, 0};
            }
        }
    };

    int64_t grp = (int64_t)blockIdx.x * kGemvWaves + wave;
    if (grp >= groups) return;
    v4i_g cur[RPW][CPL], nxt[RPW][CPL];
    load(grp, nxt);
    for (; grp < groups; grp += stride) {
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int u = 0; u < CPL; ++u) cur[r][u] = nxt[r][u];
        if (grp + stride < groups) load(grp + stride, nxt);
        acc_t v[RPW * NV];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                acc_t a = acc_t(0);
#pragma unroll
                for (int u = 0; u < CPL; ++u) a = D::dot(cur[r][u], x[j][u], a);
                v[r * NV + j] = a;
            }
        wave_reduce(v);
        store_group<T, E, NV, RPW>(g, ep, grp * RPW, v);
    }
}

// Largest staged vector block (bytes) a workgroup keeps in LDS.
constexpr int kGemvLdsMax = 64 * 1024;
constexpr int kLdsUnroll = 8;

template <InType T, EpiKind E, int NV, int RPW>
__global__ __launch_bounds__(kGemvThreads) void gemv_lds(const GemvArgs g, const EpiParams ep) {
    using D = Dot16<T>;
    using acc_t = typename D::acc_t;
    extern __shared__ __attribute__((aligned(16))) uint8_t sv[];
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    const int64_t nch = ((int64_t)g.K * esz + 15) / 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t zb = blockIdx.y;  // batch element
    const uint8_t *vec = (const uint8_t *)g.vec + zb * g.bsv * esz;
    const int64_t vld_b = g.vld * esz;
    // Vectors beyond nvec (up to NV) read as zeros; when the block does not
    // fit in LDS the vectors are read from global memory (L2-resident).
    const bool staged = (int64_t)NV * nch * 16 <= kGemvLdsMax;
    if (staged) {
        for (int64_t c = tid; c < NV * nch; c += kGemvThreads) {
            const int64_t j = c / nch, ch = c % nch;
            *(v4i_g *)(sv + c * 16) = j < g.nvec ? *(const v4i_g *)(vec + j * vld_b + ch * 16)
                                                 : v4i_g{0, 0, 0, 0};
        }
        __syncthreads();
    }
    auto xchunk = [&](int j, int64_t ch) -> v4i_g {
        if (staged) return *(const v4i_g *)(sv + (j * nch + ch) * 16);
        return j < g.nvec ? *(const v4i_g *)(vec + j * vld_b + ch * 16) : v4i_g{0, 0, 0, 0};
    };
    const uint8_t *mat = (const uint8_t *)g.mat + zb * g.bsm * esz;
    const int64_t ld_b = g.ld * esz;
    const int64_t groups = ((int64_t)g.R + RPW - 1) / RPW;
    const int64_t stride = (int64_t)gridDim.x * kGemvWaves;
    for (int64_t grp = (int64_t)blockIdx.x * kGemvWaves + wave; grp < groups; grp += stride) {
        const int64_t r0 = grp * RPW;
        const uint8_t *rowp[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) rowp[r] = mat + (r0 + r < g.R ? r0 + r : g.R - 1) * ld_b;
        acc_t acc[RPW][NV];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int j = 0; j < NV; ++j) acc[r][j] = acc_t(0);
        int64_t ch = lane;
        for (; ch + 64 * (kLdsUnroll - 1) < nch; ch += 64 * kLdsUnroll) {
            v4i_g m[kLdsUnroll][RPW];
#pragma unroll
            for (int u = 0; u < kLdsUnroll; ++u)
#pragma unroll
                for (int r = 0; r < RPW; ++r)
                    m[u][r] = __builtin_nontemporal_load((const v4i_g *)(rowp[r] + (ch + 64 * u) * 16));
#pragma unroll
            for (int u = 0; u < kLdsUnroll; ++u)
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    const v4i_g xv = xchunk(j, ch + 64 * u);
#pragma unroll
                    for (int r = 0; r < RPW; ++r) acc[r][j] = D::dot(m[u][r], xv, acc[r][j]);
                }
        }
        for (; ch < nch; ch += 64) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const v4i_g xv = xchunk(j, ch);
#pragma unroll
                for (int r = 0; r < RPW; ++r)
                    acc[r][j] = D::dot(*(const v4i_g *)(rowp[r] + ch * 16), xv, acc[r][j]);
            }
        }
        acc_t v[RPW * NV];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int j = 0; j < NV; ++j) v[r * NV + j] = acc[r][j];
        wave_reduce(v);
        store_group<T, E, NV, RPW>(g, ep, r0, v);
    }
}

// Long rows with one or two vectors: the workgroup takes one row at a time
// (rows blockIdx.x, + gridDim.x, ...), its 256 lanes reading 256*U
// consecutive 16-byte chunks per batch (thread t: chunks t + 256u), so each
// workgroup streams one contiguous 32..64 KiB window instead of four waves
// streaming four rows 8 KiB at a time (on a 16384^2 f32 matrix: 0.86 of HBM
// peak for this access pattern against 0.82 for a row per wave and 0.77 for
// two rows per wave, plain reads measured alone).  Batches run as one flat
// sequence over the workgroup's rows with the next batch's loads issued
// before the current one is multiplied; the last batch of a row is masked
// past the row's end.  At a row's end each wave reduces its lanes'
// partial sums, the four wave totals meet in LDS (two slots alternating by
// row, so one barrier per row suffices) and wave 0 adds them in wave order
// and stores.
template <InType T, EpiKind E, int NV, int U>
__global__ __launch_bounds__(kGemvThreads) void gemv_wgrow(const GemvArgs g, const EpiParams ep) {
    using D = Dot16<T>;
    using acc_t = typename D::acc_t;
    extern __shared__ __attribute__((aligned(16))) uint8_t sv[];
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    const int64_t nch = ((int64_t)g.K * esz + 15) / 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t zb = blockIdx.y;  // batch element
    const uint8_t *vec = (const uint8_t *)g.vec + zb * g.bsv * esz;
    const int64_t vld_b = g.vld * esz;
    // The vectors are staged in LDS when they fit (else read from global
    // memory, L2-resident); the wave-total exchange follows them.
    const bool staged = (int64_t)NV * nch * 16 <= kGemvLdsMax;
    acc_t *comb = (acc_t *)(sv + (staged ? NV * nch * 16 : 0));
    if (staged) {
        for (int64_t c = tid; c < NV * nch; c += kGemvThreads) {
            const int64_t j = c / nch, ch = c % nch;
            *(v4i_g *)(sv + c * 16) = j < g.nvec ? *(const v4i_g *)(vec + j * vld_b + ch * 16)
                                                 : v4i_g{0, 0, 0, 0};
        }
    }
    __syncthreads();
    auto xchunk = [&](int j, int64_t ch) -> v4i_g {
        if (staged) return *(const v4i_g *)(sv + (j * nch + ch) * 16);
        return j < g.nvec ? *(const v4i_g *)(vec + j * vld_b + ch * 16) : v4i_g{0, 0, 0, 0};
    };
    const uint8_t *mat = (const uint8_t *)g.mat + zb * g.bsm * esz;
    const int64_t ld_b = g.ld * esz;
    constexpr int64_t kBatch = (int64_t)kGemvThreads * U;  // chunks per batch
    const int64_t nbr = (nch + kBatch - 1) / kBatch;       // batches per row
    int64_t irow = blockIdx.x, ib = 0;  // next batch to issue
    int64_t rrow = blockIdx.x, rb = 0;  // next batch to multiply
    int slot = 0;
    acc_t acc[NV];
    auto issue = [&](v4i_g (&m)[U]) {
        const uint8_t *rp = mat + irow * ld_b;
        const int64_t c0 = ib * kBatch + tid;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c = c0 + (int64_t)kGemvThreads * u;
            m[u] = c < nch ? __builtin_nontemporal_load((const v4i_g *)(rp + c * 16))
                           : v4i_g{0, 0, 0, 0};
        }
        if (++ib == nbr) {
            ib = 0;
            irow += gridDim.x;
        }
    };
    auto run = [&](const v4i_g (&m)[U]) {
        if (rb == 0) {
#pragma unroll
            for (int j = 0; j < NV; ++j) acc[j] = acc_t(0);
        }
        const int64_t c0 = rb * kBatch + tid;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c = c0 + (int64_t)kGemvThreads * u;
            if (c < nch) {
#pragma unroll
                for (int j = 0; j < NV; ++j) acc[j] = D::dot(m[u], xchunk(j, c), acc[j]);
            }
        }
        if (++rb < nbr) return;
        acc_t v[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) v[j] = acc[j];
        wave_reduce(v);
        constexpr int SH = 6 - log2c<NV>();
        if ((lane & ((1 << SH) - 1)) == 0)
            comb[(slot * kGemvWaves + wave) * NV + (lane >> SH)] = v[0];
        __syncthreads();
        if (wave == 0 && lane < NV) {
            acc_t s = comb[slot * kGemvWaves * NV + lane];
#pragma unroll
            for (int w = 1; w < kGemvWaves; ++w) s += comb[(slot * kGemvWaves + w) * NV + lane];
            if (lane < g.nvec) Store<E>::apply(ep, blockIdx.y, lane, (int)rrow, s);
        }
        slot ^= 1;
        rb = 0;
        rrow += gridDim.x;
    };
    v4i_g m0[U], m1[U];
    if (irow < g.R) issue(m0);
    while (rrow < g.R) {
        if (irow < g.R) issue(m1);
        run(m0);
        if (rrow >= g.R) break;
        if (irow < g.R) issue(m0);
        run(m1);
    }
}

// Persistent grid: enough workgroups to cover the row groups, at most
// `per_cu` per CU over all batch elements (grid y); every element gets at
// least one workgroup.
static dim3 gemv_grid(int64_t groups, int cus, int per_cu, int batch) {
    int64_t blocks = (groups + kGemvWaves - 1) / kGemvWaves;
    const int64_t nb = batch > 1 ? batch : 1;
    const int64_t cap = ((int64_t)(cus > 0 ? cus : 256) * per_cu + nb - 1) / nb;
    if (blocks > cap) blocks = cap;
    return dim3((unsigned)(blocks < 1 ? 1 : blocks), (unsigned)nb);
}

// Rows per wave iteration and workgroups per CU, from a graph-timed sweep over
// 1 KB..8 KB rows (i8, f32 and bf16, 4096..65536 rows, five rotating matrix
// copies so the Infinity Cache cannot serve them).  Rows of 4 KB or more want
// about 8 KB per wave iteration (2 rows of 4 KB, 1 of 8 KB) and 3 workgroups
// per CU: on a 58.7 MB i8 matrix that is 10.2 us against 11.4 us for 4 rows
// and up to 8 workgroups per CU, which keeps more bytes in flight but spends
// longer in each wave's reduction and store before its next loads.  Shorter
// rows keep 4 rows per iteration and up to 8 workgroups per CU.
template <int CPL>
constexpr int rows_per_wave() {
    return CPL >= 8 ? 1 : (CPL >= 4 ? 2 : 4);
}

template <int CPL>
constexpr int reg_per_cu() {
    return CPL >= 4 ? 3 : 8;
}

// GEMMKIT_HIP_GEMV_SHAPE="rows,wgs" overrides the register GEMV's launch shape:
// rows per wave iteration (1, 2 or 4; one vector only) and workgroups per CU.
// A tuning switch for the launch-shape sweep: i8 results do not change; float
// sums may round differently with the rows per iteration (the butterfly's
// tree depends on the number of values it reduces).
struct GemvShape {
    int rpw = 0, per_cu = 0;
};
static GemvShape gemv_shape_env() {
    GemvShape sh;
    const char *e = getenv("GEMMKIT_HIP_GEMV_SHAPE");
    if (e && sscanf(e, "%d,%d", &sh.rpw, &sh.per_cu) != 2) sh = GemvShape{};
    return sh;
}

template <InType T, EpiKind E, int NV, int CPL, int RPW>
static hipError_t go_reg_rpw(const GemvArgs &g, const EpiParams &ep, int per_cu,
                             hipStream_t stream) {
    const int64_t groups = ((int64_t)g.R + RPW - 1) / RPW;
    hipLaunchKernelGGL((gemv_reg<T, E, NV, CPL, RPW>), gemv_grid(groups, g.cus, per_cu, g.batch),
                       dim3(kGemvThreads), 0, stream, g, ep);
    return hipGetLastError();
}

template <InType T, EpiKind E, int NV, int CPL>
static hipError_t go_reg(const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    const GemvShape sh = gemv_shape_env();
    const int per_cu = sh.per_cu > 0 ? sh.per_cu : reg_per_cu<CPL>();
    if constexpr (NV == 1) {
        if (sh.rpw == 1) return go_reg_rpw<T, E, NV, CPL, 1>(g, ep, per_cu, stream);
        if (sh.rpw == 2) return go_reg_rpw<T, E, NV, CPL, 2>(g, ep, per_cu, stream);
        if (sh.rpw == 4) return go_reg_rpw<T, E, NV, CPL, 4>(g, ep, per_cu, stream);
    }
    return go_reg_rpw<T, E, NV, CPL, rows_per_wave<CPL>()>(g, ep, per_cu, stream);
}

// Workgroup-per-row launch: as many workgroups per CU as LDS holds, at most
// 3 (2 and 3 measure alike; 4 or more contend in HBM), or the switch's count.
template <InType T, EpiKind E, int NV, int U>
static hipError_t go_wgrow(const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    const int64_t vbytes = (int64_t)NV * (((int64_t)g.K * esz + 15) / 16) * 16;
    const size_t shm = (vbytes <= kGemvLdsMax ? (size_t)vbytes : 0) + 2 * kGemvWaves * NV * 4;
    const int fit = (int)(160 * 1024 / shm);
    int per_cu = fit < 3 ? (fit > 1 ? fit : 1) : 3;
    const GemvShape sh = gemv_shape_env();
    if (sh.per_cu > 0) per_cu = sh.per_cu < fit ? sh.per_cu : (fit > 1 ? fit : 1);
    const int64_t nb = g.batch > 1 ? g.batch : 1;
    int64_t blocks = ((int64_t)(g.cus > 0 ? g.cus : 256) * per_cu + nb - 1) / nb;
    if (blocks > g.R) blocks = g.R;
    hipLaunchKernelGGL((gemv_wgrow<T, E, NV, U>), dim3((unsigned)blocks, (unsigned)nb),
                       dim3(kGemvThreads), shm, stream, g, ep);
    return hipGetLastError();
}

template <InType T, EpiKind E, int NV>
static hipError_t go_lds(const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    // one or two vectors (bf16: one, for registers): a workgroup per row
    if constexpr (T == InType::BF16 ? NV == 1 : NV <= 2) return go_wgrow<T, E, NV, 8>(g, ep, stream);
    constexpr int RPW = 1;
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    const int64_t vbytes = (int64_t)NV * (((int64_t)g.K * esz + 15) / 16) * 16;
    const size_t shm = vbytes <= kGemvLdsMax ? (size_t)vbytes : 0;
    const int64_t groups = ((int64_t)g.R + RPW - 1) / RPW;
    hipLaunchKernelGGL((gemv_lds<T, E, NV, RPW>), gemv_grid(groups, g.cus, 2, g.batch),
                       dim3(kGemvThreads), shm, stream, g, ep);
    return hipGetLastError();
}

// Register-resident vectors while NV x CPL chunks per lane stay within the
// register budget (bf16 needs extra registers to widen its operands).
template <InType T, int NV, int CPL>
constexpr bool reg_fits() {
    return NV * CPL <= (T == InType::BF16 ? 16 : 32);
}

template <InType T, EpiKind E, int NV>
static hipError_t go_nv(const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    const int64_t nch = ((int64_t)g.K * esz + 15) / 16;
    if (nch <= 64) return go_reg<T, E, NV, 1>(g, ep, stream);
    if (nch <= 128) return go_reg<T, E, NV, 2>(g, ep, stream);
    if constexpr (reg_fits<T, NV, 4>())
        if (nch <= 256) return go_reg<T, E, NV, 4>(g, ep, stream);
    if constexpr (reg_fits<T, NV, 8>())
        if (nch <= 512) return go_reg<T, E, NV, 8>(g, ep, stream);
    return go_lds<T, E, NV>(g, ep, stream);
}

template <InType T, EpiKind E>
static hipError_t gemv_nv(const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    if (g.nvec <= 1) return go_nv<T, E, 1>(g, ep, stream);
    if (g.nvec <= 2) return go_nv<T, E, 2>(g, ep, stream);
    if (g.nvec <= 4) return go_nv<T, E, 4>(g, ep, stream);
    return go_nv<T, E, 8>(g, ep, stream);
}

hipError_t launch_gemv(InType in, const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    // Row addresses are formed in 64 bits (any non-negative row stride); the
    // host packs a matrix with a negative one.
    if (g.nvec < 1 || g.nvec > 8 || g.R < 1 || g.ld < 0 || g.batch < 1 || g.batch > kMaxGridZ)
        return hipErrorInvalidValue;
    switch (in) {
    case InType::I8:
        if (ep.kind == EpiKind::I32) return gemv_nv<InType::I8, EpiKind::I32>(g, ep, stream);
        if (ep.kind == EpiKind::Q8) return gemv_nv<InType::I8, EpiKind::Q8>(g, ep, stream);
        break;
    case InType::F32:
        if (ep.kind == EpiKind::F32) return gemv_nv<InType::F32, EpiKind::F32>(g, ep, stream);
        break;
    case InType::BF16:
        if (ep.kind == EpiKind::F32) return gemv_nv<InType::BF16, EpiKind::F32>(g, ep, stream);
        if (ep.kind == EpiKind::BF16) return gemv_nv<InType::BF16, EpiKind::BF16>(g, ep, stream);
        break;
    }
    return hipErrorInvalidValue;
}

}  // namespace gk
