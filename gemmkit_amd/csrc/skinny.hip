// skinny.hip -- matrix-core kernel for skinny products: 1..16 short-side rows
// (decode-shaped GEMV / small-batch linear layers), bound by streaming the
// long operand from HBM once.
//
// Serves the same route as gemv.hip (gemmkit's gemv, src/special/gemv.rs:101-600,
// and the i8 skinny shapes, src/dispatch/int.rs:165-168), for short sides up to
// 16: out[j, r] = epi( sum_p mat[r, p] * vec[j, p] ), r < R, j < nvec.
//
// Layout on the matrix cores: v_mfma_*_16x16x(64 i8 | 32 bf16 | 4x4 f32) with
// the (zero-padded) vectors as the instruction's 16 columns.  A load
// instruction reads 8 matrix rows x 128 contiguous bytes (a 128-byte k step):
// lane l (i = l%16, g = l/16) takes row i/2 of the 8, chunk c = 2g + i%2.  As
// MFMA operand, lane l is instruction row i with k group g, so row i pairs
// chunk 2g + i%2 of its matrix row with whatever chunk the vector operand
// holds for group g.  Two MFMAs per load, one with vector chunks 2g (h = 0)
// and one with 2g + 1 (h = 1), make the products of the even rows exact in
// the first and of the odd rows in the second; the other halves are ignored.
// Result (16x16 accumulator: register q of lane l is instruction row
// 4*(l/16) + q, vector l%16): matrix row 2*(l/16) + e of the block is
// acc_h0[2e] + acc_h1[2e+1], a per-lane add.  The vectors are staged once per
// workgroup in LDS (row stride padded so the 16 lanes of an LDS cycle hit
// distinct banks); the matrix goes global -> VGPRs through a buffer resource
// (rows past R and bytes past K read as zeros).
//
// Work item: BLK 8-row blocks (32 rows, or 8 when there are too few rows to
// give every CU an item) x all of K.  The 4 waves of a workgroup split K into
// 4 contiguous ranges; each keeps 4 k steps x BLK blocks of loads in flight
// behind its MFMAs, and the four partial sums are added through LDS, in wave
// order, before the epilogue.
// The vectors may have any strides: k-contiguous, 16-byte aligned rows are
// staged as 16-byte chunks, anything else element by element (so a strided
// activation needs no separate pack launch).
#include <stdio.h>
#include <stdlib.h>

#include <type_traits>

#include "epilogue.h"

namespace gk {

typedef int v4i_s __attribute__((ext_vector_type(4)));
typedef float v4f_s __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf_s __attribute__((ext_vector_type(8)));

template <InType T>
struct Mma16;

template <>
struct Mma16<InType::I8> {
    using acc_t = v4i_s;
    using val_t = int32_t;
    __device__ __forceinline__ static acc_t step(v4i_s a, v4i_s b, acc_t c) {
        return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mma16<InType::BF16> {
    using acc_t = v4f_s;
    using val_t = float;
    __device__ __forceinline__ static acc_t step(v4i_s a, v4i_s b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf_s, a),
                                                       __builtin_bit_cast(v8bf_s, b), c, 0, 0, 0);
    }
};

template <>
struct Mma16<InType::F32> {
    using acc_t = v4f_s;
    using val_t = float;
    __device__ __forceinline__ static acc_t step(v4i_s a, v4i_s b, acc_t c) {
        v4f_s af = __builtin_bit_cast(v4f_s, a), bf = __builtin_bit_cast(v4f_s, b);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[0], bf[0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[1], bf[1], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[2], bf[2], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[3], bf[3], c, 0, 0, 0);
        return c;
    }
};

constexpr int kSkThreads = 256;
constexpr int kSkWaves = 4;
constexpr int kSkBlocks = 4;               // 8-row blocks per work item (at most)
constexpr int kSkStep = 128;               // k bytes per step (one load per block)
constexpr int kSkPF = 4;                   // k steps per load batch
constexpr int kSkCombine = kSkWaves * kSkBlocks * 2 * 64 * 4;  // partial-sum exchange bytes
constexpr uint32_t kSkOut = 0x80000000u;   // out-of-range buffer offset (reads zeros)
constexpr int kSkRsrcWord3 = 0x00020000;   // raw buffer, 32-bit data format

// LDS row stride of a staged vector: K bytes rounded up to 256, plus 16, so
// the 16 vectors read in one LDS cycle start in distinct 16-byte bank groups.
__host__ __device__ constexpr int64_t skinny_xstride(int64_t kbytes) {
    return (kbytes + 255) / 256 * 256 + 16;
}

// A vector chunk: the default cache policy (every workgroup reads the vectors).
__device__ __forceinline__ v4i_s load16v(const uint8_t *base, uint32_t num, uint32_t off) {
    __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)num, kSkRsrcWord3);
    return __builtin_bit_cast(v4i_s, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ v4i_s load16(const uint8_t *base, uint32_t num, uint32_t off) {
    __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)num, kSkRsrcWord3);
    // Cache policy 2 = nontemporal: the matrix is read once (12.6 against
    // 13.0 us with the default policy on the 14336x4096 i8 weight, 8 vectors).
    return __builtin_bit_cast(v4i_s, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}

template <InType T, EpiKind E, int BLK>
__global__ __launch_bounds__(kSkThreads) void skinny_mfma(const GemvArgs g, const EpiParams ep) {
    constexpr int kSkRows = 8 * BLK;  // matrix rows per work item
    using Mm = Mma16<T>;
    using acc_t = typename Mm::acc_t;
    using val_t = typename Mm::val_t;
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    extern __shared__ __attribute__((aligned(16))) uint8_t sh[];

    // Row bytes rounded up to whole 16-byte chunks: a K*esz that is not a
    // multiple of 16 only arrives through the pack, which zero-fills both
    // operands' rows up to the next 16 bytes.
    const int64_t kb = ((int64_t)g.K * esz + 15) / 16 * 16;
    const int nk = (int)((kb + kSkStep - 1) / kSkStep);
    const int64_t xs = skinny_xstride(kb);
    const int nvec = g.nvec;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const int li = lane & 15, lg = lane >> 4;
    const int chunk = 2 * lg + (li & 1);      // this lane's 16-byte chunk of a k step
    const bool lvec = li < nvec;
    const int64_t xaddr = (int64_t)(lvec ? li : 0) * xs + 32 * lg;  // + 16*h for MFMA h
    const int kseg = (nk + kSkWaves - 1) / kSkWaves;
    const int ks0 = wave * kseg, ks1 = ks0 + kseg < nk ? ks0 + kseg : nk;

    // This wave's load batches, in order: for each of the workgroup's items
    // (blockIdx.x, + gridDim.x, ...), nbw batches of kSkPF k steps of its K
    // range (at least one, all out of range when the range is empty, so every
    // wave takes part in every item's exchange).  Two register buffers
    // alternate: batch t+1 is in flight while batch t is multiplied, across
    // item boundaries too.  (Issuing batch 1 before the vector staging as
    // well measured slower: 14.3 against 12.6 us on the 14336x4096 i8
    // weight with 8 vectors.)
    const int64_t zb = blockIdx.y;  // batch element
    const uint8_t *mat = (const uint8_t *)g.mat + zb * g.bsm * esz;
    const int64_t ld_b = g.ld * esz;
    // (64-bit: R may be up to 2^31 - 1; every item's first row is below R)
    const int items = (int)(((int64_t)g.R + kSkRows - 1) / kSkRows);
    const int my_items = (int)blockIdx.x < items ? (items - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
    const int nbw = ks1 > ks0 ? (ks1 - ks0 + kSkPF - 1) / kSkPF : 1;
    const int total = my_items * nbw;
    uint32_t off[BLK];
#pragma unroll
    for (int b = 0; b < BLK; ++b) off[b] = (uint32_t)((8 * b + (li >> 1)) * ld_b + 16 * chunk);
    auto issue = [&](int t, v4i_s (&m)[kSkPF][BLK]) {
        const int r0 = ((int)blockIdx.x + (t / nbw) * (int)gridDim.x) * kSkRows;
        const int s0 = ks0 + (t % nbw) * kSkPF;
        const uint8_t *base = mat + (int64_t)r0 * ld_b;
        // Extent of the item's valid rows (rows may overlap: ld_b < kb is a
        // legal view); rows past R read zeros when they start past it and
        // otherwise produce outputs that are never stored.
        const bool live = t < total;  // batch 0 is issued even for a workgroup without items
        const int nrows = g.R - r0 < kSkRows ? g.R - r0 : kSkRows;
        const uint32_t num = live ? (uint32_t)((nrows - 1) * ld_b + kb) : 0u;
#pragma unroll
        for (int p = 0; p < kSkPF; ++p) {
            const int s = s0 + p;
            const bool in = live && s < ks1 && (int64_t)s * kSkStep + 16 * chunk < kb;
            // Out-of-range lanes get bit 31 set, past any resource size here
            // (an item spans at most 32 rows of at most 8 MiB, both for the
            // matrix's row stride and its row, so num and every in-range
            // offset stay below 2^31), without a select: every load is
            // issued on every path, so the wait counts after a batch are
            // exact.
            const uint32_t oor = (uint32_t)!in << 31;
#pragma unroll
            for (int b = 0; b < BLK; ++b)
                m[p][b] = load16(base, num, (off[b] + (uint32_t)s * kSkStep) | oor);
        }
    };
    v4i_s buf0[kSkPF][BLK], buf1[kSkPF][BLK];

    // Stage the vectors: nvec rows of kb bytes (zeros past K), 8 chunks or
    // elements per thread in flight at a time (one L2 round trip for up to
    // 32 KiB).
    const uint8_t *vec = (const uint8_t *)g.vec + zb * g.bsv * esz;
    const int64_t vld_b = g.vld * esz;
    if (g.vks == 1 && g.K * esz % 16 == 0 && vld_b % 16 == 0 && (uintptr_t)vec % 16 == 0) {
        // Chunk p of every vector (no index division), 8 loads in flight.
        // The first pass (chunk tid of vectors 0-7) is issued before the
        // matrix's batch 0 in straight-line code, so its LDS writes wait for
        // the vector loads only, not for batch 0 from HBM (8 vectors on the
        // 14336x4096 i8 weight: 11.95-11.98 against 12.54-12.59 us with
        // batch 0 first and a 64-bit index division per chunk).
        const int64_t cpr = kb / 16;
        // (A negative vector stride, legal on the unchecked tier, takes the
        // 64-bit pointer path: the buffer offsets below are unsigned.)
        if (vld_b >= 0 && (int64_t)(nvec - 1) * vld_b + kb <= 0x7FFFFFF0ll) {
            const uint32_t vnum = (uint32_t)((int64_t)(nvec - 1) * vld_b + kb);
            v4i_s tmp[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                tmp[u] = load16v(vec, vnum, (tid < cpr && u < nvec)
                                                ? (uint32_t)(u * vld_b + (int64_t)tid * 16)
                                                : kSkOut);
            issue(0, buf0);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (tid < cpr && u < nvec) *(v4i_s *)(sh + (int64_t)u * xs + (int64_t)tid * 16) = tmp[u];
        } else {
            issue(0, buf0);
            for (int j = 0; j < 8 && j < nvec; ++j)
                if (tid < cpr)
                    *(v4i_s *)(sh + (int64_t)j * xs + (int64_t)tid * 16) =
                        *(const v4i_s *)(vec + (int64_t)j * vld_b + (int64_t)tid * 16);
        }
        for (int64_t p = tid; p < cpr; p += kSkThreads) {
            for (int j0 = p == tid ? 8 : 0; j0 < nvec; j0 += 8) {
                v4i_s tmp[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    tmp[u] = j0 + u < nvec ? *(const v4i_s *)(vec + (int64_t)(j0 + u) * vld_b + p * 16)
                                           : v4i_s{0, 0, 0, 0};
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (j0 + u < nvec) *(v4i_s *)(sh + (int64_t)(j0 + u) * xs + p * 16) = tmp[u];
            }
        }
    } else if (g.vld == 1 && g.vks >= nvec && (uintptr_t)vec % 4 == 0 &&
               (int64_t)(g.K - 1) * g.vks + nvec <= 0xFFFFFFFFll) {
        issue(0, buf0);
        // Column-major vectors (element (j, p) at p*vks + j): the span they
        // cover is read as aligned 4-byte words, 8 per thread in flight, and
        // each element is scattered to its vector's row.  A word never
        // straddles a page, so the bytes a last partial word reads past the
        // span are mapped; they are discarded.
        using elem_t = typename std::conditional<esz == 1, uint8_t,
                         typename std::conditional<esz == 2, uint16_t, uint32_t>::type>::type;
        constexpr int EPW = 4 / esz;  // elements per word
        const uint32_t vks = (uint32_t)g.vks;
        // idx / vks as a multiply-high (Granlund-Montgomery, exact for every
        // 32-bit idx): l = ceil(log2 vks), magic = 2^32 (2^l - vks) / vks + 1.
        const int dl = 32 - __builtin_clz(vks - 1);
        const uint32_t magic = (uint32_t)(((1ull << 32) * ((1ull << dl) - vks)) / vks + 1);
        const int64_t span = ((int64_t)(g.K - 1) * vks + nvec) * esz;
        const int64_t nw = (span + 3) / 4;
        const uint32_t *vw = (const uint32_t *)vec;
        for (int64_t w0 = tid; w0 < nw; w0 += kSkThreads * 8) {
            uint32_t tmp[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t w = w0 + (int64_t)u * kSkThreads;
                tmp[u] = w < nw ? vw[w] : 0u;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t w = w0 + (int64_t)u * kSkThreads;
#pragma unroll
                for (int e = 0; e < EPW; ++e) {
                    const uint32_t idx = (uint32_t)(w * EPW + e);
                    const uint32_t hi = __umulhi(magic, idx);
                    const uint32_t p = (hi + ((idx - hi) >> 1)) >> (dl - 1), j = idx - p * vks;
                    if (w < nw && j < (uint32_t)nvec && p < (uint32_t)g.K)
                        *(elem_t *)(sh + j * xs + (int64_t)p * esz) =
                            (elem_t)(tmp[u] >> (8 * esz * e));
                }
            }
        }
        // Zero each vector's bytes from K up to the 16-byte padded length.
        const int64_t pad = kb - (int64_t)g.K * esz;
        if (tid < nvec * 16 && (tid & 15) < pad)
            sh[(tid >> 4) * xs + (int64_t)g.K * esz + (tid & 15)] = 0;
    } else {
        issue(0, buf0);
        using elem_t = typename std::conditional<esz == 1, uint8_t,
                         typename std::conditional<esz == 2, uint16_t, uint32_t>::type>::type;
        const elem_t *ve = (const elem_t *)vec;
        const int64_t epr = kb / esz, nel = nvec * epr;
        for (int64_t c0 = tid; c0 < nel; c0 += kSkThreads * 8) {
            elem_t tmp[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t c = c0 + (int64_t)u * kSkThreads;
                const int64_t j = c / epr, p = c % epr;
                tmp[u] = (c < nel && p < g.K) ? ve[j * g.vld + p * g.vks] : (elem_t)0;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t c = c0 + (int64_t)u * kSkThreads;
                if (c < nel) *(elem_t *)(sh + (c / epr) * xs + (c % epr) * esz) = tmp[u];
            }
        }
    }
    val_t *comb = (val_t *)(sh + nvec * xs);
    __syncthreads();

    acc_t acc[2][BLK];
    // Multiplies batch t; after an item's last batch, forms each matrix row's
    // result from the two MFMAs, sums the four K ranges (wave order) through
    // LDS and applies the epilogue.
    auto run = [&](int t, const v4i_s (&m)[kSkPF][BLK]) {
        const int q = t % nbw;
        if (q == 0) {
#pragma unroll
            for (int b = 0; b < BLK; ++b) acc[0][b] = acc[1][b] = acc_t{};
        }
        const int s0 = ks0 + q * kSkPF;
#pragma unroll
        for (int p = 0; p < kSkPF; ++p) {
            const int s = s0 + p;
            if (s < ks1) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    v4i_s xv = *(const v4i_s *)(sh + xaddr + (int64_t)s * kSkStep + 16 * h);
                    if (!lvec || (int64_t)s * kSkStep + 16 * (2 * lg + h) >= kb) xv = v4i_s{0, 0, 0, 0};
#pragma unroll
                    for (int b = 0; b < BLK; ++b) acc[h][b] = Mm::step(m[p][b], xv, acc[h][b]);
                }
            }
        }
        if (q != nbw - 1) return;
        const int r0 = ((int)blockIdx.x + (t / nbw) * (int)gridDim.x) * kSkRows;
#pragma unroll
        for (int b = 0; b < BLK; ++b)
#pragma unroll
            for (int e = 0; e < 2; ++e)
                comb[((wave * BLK + b) * 2 + e) * 64 + lane] =
                    (val_t)acc[0][b][2 * e] + (val_t)acc[1][b][2 * e + 1];
        __syncthreads();
#pragma unroll
        for (int x = tid; x < BLK * 2 * 64; x += kSkThreads) {
            const int b = x / 128, e = (x / 64) % 2, ln = x % 64;
            val_t sum = comb[x];
#pragma unroll
            for (int w = 1; w < kSkWaves; ++w) sum += comb[w * BLK * 2 * 64 + x];
            const int64_t row = (int64_t)r0 + 8 * b + 2 * (ln >> 4) + e;
            const int j = ln & 15;
            if (j < nvec && row < g.R) Store<E>::apply(ep, zb, j, (int)row, sum);
        }
        __syncthreads();
    };
    for (int t = 0; t < total; t += 2) {
        if (t + 1 < total) issue(t + 1, buf1);
        run(t, buf0);
        if (t + 1 < total) {
            if (t + 2 < total) issue(t + 2, buf0);
            run(t + 1, buf1);
        }
    }
}

// Bytes of LDS the kernel needs (vectors + partial-sum exchange).
int64_t skinny_lds_bytes(InType in, int64_t K, int nvec) {
    const int64_t esz = in == InType::I8 ? 1 : (in == InType::BF16 ? 2 : 4);
    return nvec * skinny_xstride((K * esz + 15) / 16 * 16) + kSkCombine;
}

template <InType T, EpiKind E>
static hipError_t skinny_go(const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    const int64_t shm = skinny_lds_bytes(T, g.K, g.nvec);
    const int cus = g.cus > 0 ? g.cus : 256;
    // 32-row items when there are enough of them for every CU, else 8-row
    // items (4x as many workgroups streaming the same bytes).
    const int64_t R = g.R;
    int rows = (R + 31) / 32 >= cus ? 32 : 8;
    // GEMMKIT_HIP_SKINNY_SHAPE="rows,wgs": rows per work item (8, 16 or 32)
    // and workgroups per CU, a tuning switch for the launch-shape sweep
    // (results do not change: each row's K ranges and their order are fixed
    // by K).
    int rows_env = 0, wgs_env = 0;
    if (const char *e = getenv("GEMMKIT_HIP_SKINNY_SHAPE"))
        if (sscanf(e, "%d,%d", &rows_env, &wgs_env) == 2 &&
            (rows_env == 8 || rows_env == 16 || rows_env == 32))
            rows = rows_env;
    const int64_t items = (R + rows - 1) / rows;
    // As many resident workgroups per CU as its 160 KiB of LDS holds (<= 4).
    const int fit = (int)(160 * 1024 / shm);
    int per_cu = fit < 4 ? (fit > 1 ? fit : 1) : 4;
    if (wgs_env > 0) per_cu = wgs_env < fit ? wgs_env : (fit > 1 ? fit : 1);
    // Batch elements share the persistent grid (grid y), each at least one
    // workgroup.
    const int64_t nb = g.batch > 1 ? g.batch : 1;
    int64_t blocks = ((int64_t)cus * per_cu + nb - 1) / nb;
    if (blocks > items) blocks = items;
    const dim3 grid((unsigned)blocks, (unsigned)nb);
    if (rows == 32)
        hipLaunchKernelGGL((skinny_mfma<T, E, 4>), grid, dim3(kSkThreads), (size_t)shm, stream, g,
                           ep);
    else if (rows == 16)
        hipLaunchKernelGGL((skinny_mfma<T, E, 2>), grid, dim3(kSkThreads), (size_t)shm, stream, g,
                           ep);
    else
        hipLaunchKernelGGL((skinny_mfma<T, E, 1>), grid, dim3(kSkThreads), (size_t)shm, stream, g,
                           ep);
    return hipGetLastError();
}

hipError_t launch_skinny(InType in, const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    // The matrix rows are addressed as unsigned 32-bit offsets from an item's
    // first row, so its row stride must be non-negative (the vectors may
    // have any strides).
    if (g.nvec < 1 || g.nvec > 16 || g.R < 1 || g.ld < 0 || g.batch < 1 || g.batch > kMaxGridZ ||
        skinny_lds_bytes(in, g.K, g.nvec) > kSkinnyLdsMax)
        return hipErrorInvalidValue;
    switch (in) {
    case InType::I8:
        if (ep.kind == EpiKind::I32) return skinny_go<InType::I8, EpiKind::I32>(g, ep, stream);
        if (ep.kind == EpiKind::Q8) return skinny_go<InType::I8, EpiKind::Q8>(g, ep, stream);
        break;
    case InType::F32:
        if (ep.kind == EpiKind::F32) return skinny_go<InType::F32, EpiKind::F32>(g, ep, stream);
        break;
    case InType::BF16:
        if (ep.kind == EpiKind::F32) return skinny_go<InType::BF16, EpiKind::F32>(g, ep, stream);
        if (ep.kind == EpiKind::BF16) return skinny_go<InType::BF16, EpiKind::BF16>(g, ep, stream);
        break;
    }
    return hipErrorInvalidValue;
}

}  // namespace gk
