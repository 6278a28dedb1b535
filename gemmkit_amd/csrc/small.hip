// small.hip -- f32 GEMM for products too small to fill the CUs with the tile
// kernels (gemmkit's f32 gemm at M = N = K = 512, src/api.rs:469-580, is the
// shape it is built for): one launch, operands read in place with any
// strides, no pack and no separate reduction.
//
// A workgroup owns a 32 x 32 block of C and its sixteen waves split K into
// sixteen contiguous ranges: at these sizes the time is the memory latency of
// each wave's chain of loads, so more, shorter chains win (f32 512^3: 10.6 us
// per call with 4 waves, 8.8 with 8, 7.4 with 16; the split-K route took 17.3
// with its pack and reduction launches).  Each wave runs
// v_mfma_f32_32x32x2_f32 over its range,
// reading its operands straight from global memory (L2-resident at these
// sizes): per group of 8 k, lane l (row or column l%32, half h = l/32) loads
// A[m][k0 + 4h + t] and B^T[n][k0 + 4h + t] for t = 0..3 and issues four
// MFMAs, instruction t pairing k0 + t (half 0) with k0 + 4 + t (half 1) -- the
// k order the tile kernels use within a 16-byte chunk.  Groups of 32 k are
// double-buffered in registers: the next group's loads are in flight while
// the current one is multiplied.  At the end the partial blocks meet in LDS
// and are added in wave order, then the call's epilogue (alpha, beta,
// fused bias/activation) stores them: every output's arithmetic depends only
// on K, so batched elements equal standalone calls bit for bit.
//
// The accumulator layout of the 32x32 MFMA: register r of lane l holds C row
// 8*(r/4) + 4*(l/32) + r%4, column l%32 of the block.
#include "epilogue.h"

namespace gk {

constexpr int kSmWaves = 16;            // waves per block, splitting K
constexpr int kSmThreads = 64 * kSmWaves;
constexpr int kSmGroup = 32;  // k per register buffer (four 8-k groups)

typedef float v16f_s __attribute__((ext_vector_type(16)));

typedef float v4f_sm __attribute__((ext_vector_type(4)));

// AV / BV: the operand is k-contiguous with 16-byte aligned rows, so a lane's
// four k of a group come as one 16-byte load (a k-strided operand takes four
// 4-byte loads, which coalesce across the lanes instead).
template <bool AV, bool BV>
__global__ __launch_bounds__(kSmThreads) void small_f32_kernel(const SmallArgs g,
                                                               const EpiParams ep) {
    __shared__ float part[kSmWaves][16][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, li = lane & 31;
    const int tiles_n = (g.N + 31) / 32;
    const int m0 = (int)(blockIdx.x / tiles_n) * 32, n0 = (int)(blockIdx.x % tiles_n) * 32;
    const int64_t zb = blockIdx.y;
    const float *A = (const float *)g.a + zb * g.bsa;
    const float *B = (const float *)g.b + zb * g.bsb;  // B^T: element (n, k) at n*rsb + k*ksb
    const int m = m0 + li, n = n0 + li;
    const bool m_in = m < g.M, n_in = n < g.N;
    const float *arow = A + (int64_t)(m_in ? m : 0) * g.rsa;
    const float *brow = B + (int64_t)(n_in ? n : 0) * g.rsb;
    // This wave's K range: whole 8-k groups.
    const int64_t kq = ((g.K + kSmWaves - 1) / kSmWaves + 7) / 8 * 8;
    const int64_t k_lo = wave * kq < g.K ? wave * kq : g.K;
    const int64_t k_hi = k_lo + kq < g.K ? k_lo + kq : g.K;

    auto load = [&](int64_t kb, float (&av)[16], float (&bv)[16]) {
        if (kb + kSmGroup <= k_hi) {
            // a whole group: no k checks
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t k0 = kb + 8 * q + 4 * h;
                if constexpr (AV) {
                    const v4f_sm v = m_in ? *(const v4f_sm *)(arow + k0) : v4f_sm{0, 0, 0, 0};
#pragma unroll
                    for (int t = 0; t < 4; ++t) av[4 * q + t] = v[t];
                } else {
#pragma unroll
                    for (int t = 0; t < 4; ++t) av[4 * q + t] = m_in ? arow[(k0 + t) * g.ksa] : 0.0f;
                }
                if constexpr (BV) {
                    const v4f_sm v = n_in ? *(const v4f_sm *)(brow + k0) : v4f_sm{0, 0, 0, 0};
#pragma unroll
                    for (int t = 0; t < 4; ++t) bv[4 * q + t] = v[t];
                } else {
#pragma unroll
                    for (int t = 0; t < 4; ++t) bv[4 * q + t] = n_in ? brow[(k0 + t) * g.ksb] : 0.0f;
                }
            }
            return;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int64_t k = kb + 8 * q + 4 * h + t;
                const bool in = k < k_hi;
                av[4 * q + t] = (in && m_in) ? arow[k * g.ksa] : 0.0f;
                bv[4 * q + t] = (in && n_in) ? brow[k * g.ksb] : 0.0f;
            }
    };
    v16f_s acc = {};
    float a0[16], b0[16], a1[16], b1[16];
    auto mul = [&](const float (&av)[16], const float (&bv)[16]) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[i], acc, 0, 0, 0);
    };
    int64_t kb = k_lo;
    if (kb < k_hi) load(kb, a0, b0);
    while (kb < k_hi) {
        const int64_t k1 = kb + kSmGroup;
        if (k1 < k_hi) load(k1, a1, b1);
        mul(a0, b0);
        if (k1 >= k_hi) break;
        const int64_t k2 = k1 + kSmGroup;
        if (k2 < k_hi) load(k2, a0, b0);
        mul(a1, b1);
        kb = k2;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) part[wave][r][lane] = acc[r];
    __syncthreads();
    for (int o = tid; o < 16 * 64; o += kSmThreads) {  // (register, lane) of the block
        const int r = o >> 6, l = o & 63;
        float v = part[0][r][l];
#pragma unroll
        for (int w = 1; w < kSmWaves; ++w) v += part[w][r][l];
        const int row = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3), col = n0 + (l & 31);
        if (row < g.M && col < g.N) Store<EpiKind::F32>::apply(ep, zb, row, col, v);
    }
}

hipError_t launch_small_f32(const SmallArgs &g, const EpiParams &ep, hipStream_t stream) {
    if (g.M < 1 || g.N < 1 || g.K < 1 || g.batch < 1 || g.batch > kMaxGridZ ||
        ep.kind != EpiKind::F32)
        return hipErrorInvalidValue;
    const int64_t tiles = ((int64_t)(g.M + 31) / 32) * ((g.N + 31) / 32);
    if (tiles > INT32_MAX) return hipErrorInvalidValue;
    auto vec_ok = [](const void *p, int64_t rs, int64_t ks, int64_t bs, int32_t batch) {
        return ks == 1 && rs % 4 == 0 && (batch == 1 || bs % 4 == 0) && (uintptr_t)p % 16 == 0;
    };
    const bool av = vec_ok(g.a, g.rsa, g.ksa, g.bsa, g.batch);
    const bool bv = vec_ok(g.b, g.rsb, g.ksb, g.bsb, g.batch);
    const dim3 grid((unsigned)tiles, (unsigned)g.batch);
    if (av && bv)
        hipLaunchKernelGGL((small_f32_kernel<true, true>), grid, dim3(kSmThreads), 0, stream, g, ep);
    else if (av)
        hipLaunchKernelGGL((small_f32_kernel<true, false>), grid, dim3(kSmThreads), 0, stream, g, ep);
    else if (bv)
        hipLaunchKernelGGL((small_f32_kernel<false, true>), grid, dim3(kSmThreads), 0, stream, g, ep);
    else
        hipLaunchKernelGGL((small_f32_kernel<false, false>), grid, dim3(kSmThreads), 0, stream, g, ep);
    return hipGetLastError();
}

}  // namespace gk
