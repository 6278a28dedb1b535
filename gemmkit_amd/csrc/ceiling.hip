// ceiling.hip -- the matrix cores' practical ceiling on this chip: every CU
// issuing nothing but back-to-back MFMAs on random register operands (no
// loads, no LDS), as the GEMM kernels' instructions would with perfect
// overlap.  MI355X is power-limited under such a load: the clock the chip
// holds sets the best rate any GEMM kernel can reach, below the published
// peak (which assumes 2.4 GHz).  Exposed as gk_debug_mfma_ceiling, beside
// gk_debug_read_stream and gk_debug_write_stream (plain HBM reads and
// writes, the ceilings of the HBM-bound kernels); diagnostics with no
// counterpart in the reference.
#include "mma_kernel.h"

#include "../../include/gemmkit_hip.h"

namespace gk {

// Each wave keeps 16 independent 32x32 accumulator blocks (256 registers, as
// the 4-wave GEMM tile does) and runs `iters` rounds of 16 MFMAs over
// operands drawn from a per-lane xorshift, refreshed every round so the
// multipliers see changing data.  Wave 0 of workgroup 0 reads the shader
// clock counter (s_memtime) and the 100 MHz real-time counter at start and
// end; every lane folds its accumulators into one word so nothing is dead.
template <InType T>
__global__ __launch_bounds__(256) void mfma_ceiling_kernel(int64_t iters, uint32_t *sink,
                                                           uint64_t *clocks) {
    using M = Mma<T>;
    using acc_t = typename M::acc_t;
    uint32_t s = 0x9E3779B9u ^ (blockIdx.x * 256u + threadIdx.x) * 0x85EBCA6Bu;
    auto rnd = [&]() {
        s ^= s << 13;
        s ^= s >> 17;
        s ^= s << 5;
        return (int)s;
    };
    v4i a0 = {rnd(), rnd(), rnd(), rnd()}, a1 = {rnd(), rnd(), rnd(), rnd()};
    v4i b0 = {rnd(), rnd(), rnd(), rnd()}, b1 = {rnd(), rnd(), rnd(), rnd()};
    if constexpr (T == InType::BF16) {
        // keep bf16 operands finite: clear the top exponent bit of each half
        const int m = (int)0xBFFFBFFFu;
        a0 &= m; a1 &= m; b0 &= m; b1 &= m;
    }
    // Distinct starting values: blocks that share operands must not be
    // recognisable as the same computation (the compiler would merge them).
    acc_t acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        acc[i] = acc_t{};
        acc[i][0] = (typename M::scalar_t)(i + 1);
    }
    uint64_t t0 = 0, r0 = 0;
    const bool timer = blockIdx.x == 0 && threadIdx.x == 0;
    if (timer) {
        t0 = __builtin_amdgcn_s_memtime();
        r0 = __builtin_amdgcn_s_memrealtime();
    }
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            acc[i] = M::step((i & 1) ? b1 : b0, (i & 2) ? a1 : a0, acc[i]);
        // new operands for the next round (VALU work beside the matrix pipe)
        a0 = a0 ^ (b1 << 1);
        b0 = b0 ^ (a1 >> 1);
        if constexpr (T == InType::BF16) {
            const int m = (int)0xBFFFBFFFu;
            a0 &= m; b0 &= m;
        }
    }
    uint32_t fold = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) fold = fold * 31u + __builtin_bit_cast(uint32_t, acc[i][e]);
    sink[blockIdx.x * 256 + threadIdx.x] = fold;
    if (timer) {
        clocks[0] = __builtin_amdgcn_s_memtime() - t0;
        clocks[1] = __builtin_amdgcn_s_memrealtime() - r0;
    }
}

// A pure HBM read at the GEMV's own sizes: the workgroups stride through
// `n16` 16-byte words with four nontemporal loads in flight per lane (the
// GEMV's own cache policy for its once-read matrix) and fold them into one
// word, which is stored only if it equals a value random data hits once in
// 2^32 (so the loads are live and the kernel writes next to nothing).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void read_stream_kernel(const u32x4_t *__restrict__ p,
                                                          int64_t n16, uint32_t *sink) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        u32x4_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc += (v[u].x ^ v[u].y) + (v[u].z ^ v[u].w) * (u + 1);
    }
    for (; i < n16; i += stride) {
        const u32x4_t v = __builtin_nontemporal_load(p + i);
        acc += v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

// A pure HBM write: the workgroups stride through `n16` 16-byte words, four
// stores per lane per round, nontemporal (NT) or through the cache.  The
// stored words depend on the address so nothing is constant-folded.
template <bool NT>
__global__ __launch_bounds__(256) void write_stream_kernel(u32x4_t *__restrict__ p, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t w = (uint32_t)(i + u * stride);
            const u32x4_t v = {w, w ^ 1u, w ^ 2u, w ^ 3u};
            if constexpr (NT) __builtin_nontemporal_store(v, p + i + u * stride);
            else p[i + u * stride] = v;
        }
    }
    for (; i < n16; i += stride) {
        const uint32_t w = (uint32_t)i;
        const u32x4_t v = {w, w ^ 1u, w ^ 2u, w ^ 3u};
        if constexpr (NT) __builtin_nontemporal_store(v, p + i);
        else p[i] = v;
    }
}

}  // namespace gk

using namespace gk;

extern "C" int gk_debug_write_stream(void *buf, int64_t bytes, int32_t wgs_per_cu,
                                     int32_t nontemporal, void *stream) {
    if (!buf || bytes < 16 || (bytes & 15) || wgs_per_cu < 1 || wgs_per_cu > 32 ||
        ((uintptr_t)buf & 15))
        return GK_ERR_ARG;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return GK_ERR_DEVICE;
    const int64_t n16 = bytes / 16;
    int64_t blocks = (int64_t)(cus > 0 ? cus : 256) * wgs_per_cu;
    if (blocks > (n16 + 255) / 256) blocks = (n16 + 255) / 256;
    if (nontemporal)
        hipLaunchKernelGGL(write_stream_kernel<true>, dim3((unsigned)blocks), dim3(256), 0,
                           (hipStream_t)stream, (u32x4_t *)buf, n16);
    else
        hipLaunchKernelGGL(write_stream_kernel<false>, dim3((unsigned)blocks), dim3(256), 0,
                           (hipStream_t)stream, (u32x4_t *)buf, n16);
    return hipGetLastError() == hipSuccess ? GK_OK : GK_ERR_DEVICE;
}

extern "C" int gk_debug_read_stream(const void *buf, int64_t bytes, int32_t wgs_per_cu,
                                    void *sink, void *stream) {
    if (!buf || !sink || bytes < 16 || (bytes & 15) || wgs_per_cu < 1 || wgs_per_cu > 32 ||
        ((uintptr_t)buf & 15))
        return GK_ERR_ARG;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return GK_ERR_DEVICE;
    const int64_t n16 = bytes / 16;
    int64_t blocks = (int64_t)(cus > 0 ? cus : 256) * wgs_per_cu;
    if (blocks > (n16 + 255) / 256) blocks = (n16 + 255) / 256;
    hipLaunchKernelGGL(read_stream_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, (const u32x4_t *)buf, n16, (uint32_t *)sink);
    return hipGetLastError() == hipSuccess ? GK_OK : GK_ERR_DEVICE;
}

extern "C" int gk_debug_mfma_ceiling(int32_t in_type, int64_t iters, int32_t wgs_per_cu,
                                     int32_t launches, double *ops_per_s, double *clock_ghz) {
    if (!ops_per_s || !clock_ghz || iters < 1 || wgs_per_cu != 1 ||
        launches < 1 || in_type < 0 || in_type > 3)
        return GK_ERR_ARG;
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess)
        return GK_ERR_DEVICE;
    const int cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    const int blocks = cus * wgs_per_cu;
    uint32_t *sink = nullptr;
    uint64_t *clocks = nullptr;
    if (hipMalloc(&sink, (size_t)blocks * 256 * 4) != hipSuccess) return GK_ERR_NOMEM;
    if (hipMalloc(&clocks, 16) != hipSuccess) {
        (void)hipFree(sink);
        return GK_ERR_NOMEM;
    }
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    int rc = GK_OK;
    float ms = 0.0f;
    for (int l = 0; l < launches && rc == GK_OK; ++l) {
        // the last launch is the measured one; the ones before bring the
        // clocks to their steady state under load
        (void)hipEventRecord(e0, nullptr);
        if (in_type == 0)
            hipLaunchKernelGGL(mfma_ceiling_kernel<InType::I8>, dim3(blocks), dim3(256), 0,
                               nullptr, iters, sink, clocks);
        else if (in_type == 1)
            hipLaunchKernelGGL(mfma_ceiling_kernel<InType::BF16>, dim3(blocks), dim3(256), 0,
                               nullptr, iters, sink, clocks);
        else
            (void)launch_mfma16_ceiling(in_type == 2 ? InType::I8 : InType::BF16, blocks, iters,
                                        sink, clocks);
        (void)hipEventRecord(e1, nullptr);
        if (hipGetLastError() != hipSuccess || hipEventSynchronize(e1) != hipSuccess)
            rc = GK_ERR_DEVICE;
    }
    uint64_t c[2] = {0, 0};
    if (rc == GK_OK && (hipEventElapsedTime(&ms, e0, e1) != hipSuccess ||
                        hipMemcpy(c, clocks, 16, hipMemcpyDeviceToHost) != hipSuccess))
        rc = GK_ERR_DEVICE;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipFree(sink);
    (void)hipFree(clocks);
    if (rc != GK_OK) return rc;
    // per round: 16 MFMAs of 2*32*32*32 (i8) or 2*32*32*16 (bf16) operations,
    // or 32 of 2*16*16*64 (i8) or 2*16*16*32 (bf16)
    const double per_round = in_type == 0 ? 16 * 65536.0 : in_type == 1 ? 16 * 32768.0
                           : in_type == 2 ? 32 * 32768.0 : 32 * 16384.0;
    const double ops = (double)blocks * 4 * per_round * (double)iters;
    *ops_per_s = ops / (ms * 1e-3);
    *clock_ghz = c[1] ? (double)c[0] / (double)c[1] * 0.1 : 0.0;
    return GK_OK;
}
