// skinny.hip -- matrix-core kernel for skinny products: 1..16 short-side rows
// (decode-shaped GEMV / small-batch linear layers), bound by streaming the
// long operand from HBM once.
//
// Serves the same route as gemv.hip (gemmkit's gemv, src/special/gemv.rs:101-600,
// and the i8 skinny shapes, src/dispatch/int.rs:165-168), for short sides up to
// 16: out[j, r] = epi( sum_p mat[r, p] * vec[j, p] ), r < R, j < nvec.
//
// Layout on the matrix cores: v_mfma_*_16x16x(64 i8 | 32 bf16 | 4x4 f32) with
// the matrix rows as the instruction's 16 rows and the (zero-padded) vectors
// as its 16 columns.  Lane l supplies row l%16 and vector l%16 with the 16
// bytes at k offset 16*(l/16) of each 64-byte k step, so every load
// instruction reads 16 rows x 64 contiguous bytes of the matrix.  The vectors
// are staged once per workgroup in LDS (row stride padded so the 16 lanes of
// an LDS cycle hit distinct banks); the matrix goes global -> VGPRs through a
// buffer resource (rows past R and bytes past K read as zeros).
//
// Work item: 32 matrix rows (two 16-row blocks) x all of K.  The 4 waves of a
// workgroup split K into 4 contiguous ranges; each keeps 8 k steps x 2 blocks
// (16 KiB) of loads in flight behind its MFMAs, and the four partial 16x16
// blocks are summed through LDS, in wave order, before the epilogue.
// Accumulator layout (16x16 block): register r of lane l holds matrix row
// 4*(l/16) + r, vector l%16.
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
constexpr int kSkRB = 2;                   // 16-row blocks per work item
constexpr int kSkRows = 16 * kSkRB;        // matrix rows per work item
constexpr int kSkPF = 8;                   // k steps per load batch
constexpr int kSkCombine = kSkWaves * kSkRB * 4 * 64 * 4;  // partial-sum exchange bytes
constexpr uint32_t kSkOut = 0x80000000u;   // out-of-range buffer offset (reads zeros)
constexpr int kSkRsrcWord3 = 0x00020000;   // raw buffer, 32-bit data format

// LDS row stride of a staged vector: K bytes rounded up to 256, plus 16, so
// the 16 vectors read in one LDS cycle start in distinct 16-byte bank groups.
__host__ __device__ constexpr int64_t skinny_xstride(int64_t kbytes) {
    return (kbytes + 255) / 256 * 256 + 16;
}

__device__ __forceinline__ v4i_s load16(const uint8_t *base, uint32_t num, uint32_t off) {
    __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)num, kSkRsrcWord3);
    return __builtin_bit_cast(v4i_s, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

template <InType T, EpiKind E>
__global__ __launch_bounds__(kSkThreads) void skinny_mfma(const GemvArgs g, const EpiParams ep) {
    using Mm = Mma16<T>;
    using acc_t = typename Mm::acc_t;
    using val_t = typename Mm::val_t;
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    extern __shared__ __attribute__((aligned(16))) uint8_t sh[];

    // Row bytes rounded up to whole 16-byte chunks: a K*esz that is not a
    // multiple of 16 only arrives through the pack, which zero-fills both
    // operands' rows up to the next 16 bytes.
    const int64_t kb = ((int64_t)g.K * esz + 15) / 16 * 16;
    const int nk = (int)((kb + 63) / 64);
    const int64_t xs = skinny_xstride(kb);
    const int nvec = g.nvec;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // Stage the vectors: nvec rows of kb bytes.
    const uint8_t *vec = (const uint8_t *)g.vec;
    const int64_t vld_b = g.vld * esz, cpr = kb / 16;
    for (int64_t c = tid; c < nvec * cpr; c += kSkThreads) {
        const int64_t j = c / cpr, q = c % cpr;
        *(v4i_s *)(sh + j * xs + q * 16) = *(const v4i_s *)(vec + j * vld_b + q * 16);
    }
    val_t *comb = (val_t *)(sh + nvec * xs);
    __syncthreads();

    const int lrow = lane & 15, lgrp = lane >> 4;
    const bool lvec = lrow < nvec;
    const int64_t xaddr = (int64_t)(lvec ? lrow : 0) * xs + lgrp * 16;
    const int kseg = (nk + kSkWaves - 1) / kSkWaves;
    const int ks0 = wave * kseg, ks1 = ks0 + kseg < nk ? ks0 + kseg : nk;

    const uint8_t *mat = (const uint8_t *)g.mat;
    const int64_t ld_b = g.ld * esz;
    const int items = (g.R + kSkRows - 1) / kSkRows;
    for (int item = blockIdx.x; item < items; item += gridDim.x) {
        const int r0 = item * kSkRows;
        const uint8_t *base = mat + (int64_t)r0 * ld_b;
        // Extent of the item's valid rows (rows may overlap: ld_b < kb is a
        // legal view); rows past R read zeros when they start past it and
        // otherwise produce outputs that are never stored.
        const int nrows = g.R - r0 < kSkRows ? g.R - r0 : kSkRows;
        const uint32_t num = (uint32_t)((nrows - 1) * ld_b + kb);
        uint32_t off[kSkRB];
#pragma unroll
        for (int b = 0; b < kSkRB; ++b) off[b] = (uint32_t)((b * 16 + lrow) * ld_b + lgrp * 16);

        auto load_batch = [&](int s0, v4i_s (&m)[kSkPF][kSkRB]) {
#pragma unroll
            for (int p = 0; p < kSkPF; ++p) {
                const int s = s0 + p;
                const bool in = s < ks1 && (int64_t)s * 64 + lgrp * 16 < kb;
#pragma unroll
                for (int b = 0; b < kSkRB; ++b)
                    m[p][b] = load16(base, num, in ? off[b] + (uint32_t)s * 64 : kSkOut);
            }
        };

        acc_t acc[kSkRB];
#pragma unroll
        for (int b = 0; b < kSkRB; ++b) acc[b] = acc_t{};
        v4i_s cur[kSkPF][kSkRB], nxt[kSkPF][kSkRB];
        if (ks0 < ks1) load_batch(ks0, nxt);
        for (int s0 = ks0; s0 < ks1; s0 += kSkPF) {
#pragma unroll
            for (int p = 0; p < kSkPF; ++p)
#pragma unroll
                for (int b = 0; b < kSkRB; ++b) cur[p][b] = nxt[p][b];
            if (s0 + kSkPF < ks1) load_batch(s0 + kSkPF, nxt);
#pragma unroll
            for (int p = 0; p < kSkPF; ++p) {
                const int s = s0 + p;
                if (s < ks1) {
                    v4i_s xv = *(const v4i_s *)(sh + xaddr + (int64_t)s * 64);
                    if (!lvec || (int64_t)s * 64 + lgrp * 16 >= kb) xv = v4i_s{0, 0, 0, 0};
#pragma unroll
                    for (int b = 0; b < kSkRB; ++b) acc[b] = Mm::step(cur[p][b], xv, acc[b]);
                }
            }
        }

        // Sum the four K ranges (wave order) and apply the epilogue.
#pragma unroll
        for (int b = 0; b < kSkRB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) comb[((wave * kSkRB + b) * 4 + r) * 64 + lane] = (val_t)acc[b][r];
        __syncthreads();
#pragma unroll
        for (int t = 0; t < kSkRB * 4 / kSkWaves; ++t) {
            const int e = (wave * (kSkRB * 4 / kSkWaves) + t) * 64 + lane;  // over kSkRB*4*64
            const int b = e / 256, r = (e / 64) % 4, ln = e % 64;
            val_t sum = comb[e];
#pragma unroll
            for (int w = 1; w < kSkWaves; ++w) sum += comb[w * kSkRB * 4 * 64 + e];
            const int row = r0 + b * 16 + 4 * (ln / 16) + r, j = ln % 16;
            if (j < nvec && row < g.R) Store<E>::apply(ep, 0, j, row, sum);
        }
        __syncthreads();
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
    const int64_t items = (g.R + kSkRows - 1) / kSkRows;
    const int per_cu = (int)(kSkinnyLdsMax / shm) < 4 ? (int)(kSkinnyLdsMax / shm) : 4;
    int64_t blocks = (int64_t)(g.cus > 0 ? g.cus : 256) * (per_cu > 1 ? per_cu : 1);
    if (blocks > items) blocks = items;
    hipLaunchKernelGGL((skinny_mfma<T, E>), dim3((unsigned)blocks), dim3(kSkThreads), (size_t)shm,
                       stream, g, ep);
    return hipGetLastError();
}

hipError_t launch_skinny(InType in, const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    if (g.nvec < 1 || g.nvec > 16 || g.R < 1 || skinny_lds_bytes(in, g.K, g.nvec) > kSkinnyLdsMax)
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
