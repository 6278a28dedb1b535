// pack.hip -- layout and degenerate-case kernels.
//
//   pack_kernel      copies a strided operand into the kernels' k-contiguous
//                    layout (gemmkit's pack_panels role, src/pack.rs:28-117, but
//                    one plain row-per-row layout instead of micropanels).  A
//                    64 x 64 tile goes through LDS so both the strided read and
//                    the k-contiguous write are coalesced.
//   scale_c_kernel   C <- beta*C when the A*B term vanishes (scale_c_int,
//                    src/dispatch/int.rs:150-163; scale_c_float,
//                    src/dispatch.rs:484-497; the narrow twin for bf16).
//   requant_fill     the k == 0 requant fill (requant_degenerate,
//                    src/dispatch/int.rs:735-752).
//   fused_fill       C <- act(beta*C + bias) when the A*B term of a fused
//                    call vanishes (src/dispatch/float.rs:661-680).
#include "epilogue.h"

namespace gk {

template <typename T>
__global__ __launch_bounds__(256) void pack_kernel(const T *__restrict__ src, int64_t rs,
                                                   int64_t cs, int64_t rows, int64_t K,
                                                   T *__restrict__ dst, int64_t ld) {
    __shared__ T tile[64][65];
    const int64_t r0 = (int64_t)blockIdx.y * 64;
    const int64_t p0 = (int64_t)blockIdx.x * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
    // Read: let consecutive threads walk the operand's faster-moving index.
    const bool k_fast = (cs < 0 ? -cs : cs) <= (rs < 0 ? -rs : rs);
    for (int y = ty; y < 64; y += 4) {
        int64_t r, p;
        if (k_fast) { r = r0 + y; p = p0 + tx; } else { r = r0 + tx; p = p0 + y; }
        T v = T(0);
        if (r < rows && p < K) v = src[r * rs + p * cs];
        if (k_fast) tile[y][tx] = v; else tile[tx][y] = v;
    }
    __syncthreads();
    // Write: consecutive threads write consecutive k; columns [K, ld) get zeros.
    for (int y = ty; y < 64; y += 4) {
        int64_t r = r0 + y, p = p0 + tx;
        if (r < rows && p < ld) dst[r * ld + p] = (p < K) ? tile[y][tx] : T(0);
    }
}

hipError_t launch_pack(InType in, const void *src, int64_t rs, int64_t cs, int64_t rows,
                       int64_t K, void *dst, int64_t ld, hipStream_t stream) {
    dim3 grid((unsigned)((ld + 63) / 64), (unsigned)((rows + 63) / 64));
    switch (in_size(in)) {
    case 1:
        hipLaunchKernelGGL(pack_kernel<int8_t>, grid, dim3(256), 0, stream, (const int8_t *)src,
                           rs, cs, rows, K, (int8_t *)dst, ld);
        break;
    case 2:
        hipLaunchKernelGGL(pack_kernel<uint16_t>, grid, dim3(256), 0, stream,
                           (const uint16_t *)src, rs, cs, rows, K, (uint16_t *)dst, ld);
        break;
    default:
        hipLaunchKernelGGL(pack_kernel<uint32_t>, grid, dim3(256), 0, stream,
                           (const uint32_t *)src, rs, cs, rows, K, (uint32_t *)dst, ld);
        break;
    }
    return hipGetLastError();
}

// One thread per element of a (batch x) m x n view; beta == 1 never launches.
__global__ __launch_bounds__(256) void scale_c_kernel(int kind, void *c, int64_t m, int64_t n,
                                                      int64_t rsc, int64_t csc, int64_t bsc,
                                                      int32_t beta_i, float beta_f) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t z = blockIdx.y;
    if (idx >= m * n) return;
    const int64_t i = idx / n, j = idx % n;
    const int64_t off = z * bsc + i * rsc + j * csc;
    if (kind == (int)EpiKind::I32) {
        int32_t *p = (int32_t *)c + off;
        *p = beta_i == 0 ? 0 : (int32_t)((uint32_t)beta_i * (uint32_t)*p);
    } else if (kind == (int)EpiKind::F32) {
        float *p = (float *)c + off;
        *p = beta_f == 0.0f ? 0.0f : beta_f * *p;
    } else {
        uint16_t *p = (uint16_t *)c + off;
        *p = beta_f == 0.0f ? (uint16_t)0 : bf16_rne(beta_f * bf16_widen(*p));
    }
}

hipError_t launch_scale_c(EpiKind kind, void *c, int64_t m, int64_t n, int64_t rsc,
                          int64_t csc, int64_t batch, int64_t bsc, int32_t beta_i,
                          float beta_f, hipStream_t stream) {
    if (m == 0 || n == 0 || batch == 0) return hipSuccess;
    dim3 grid((unsigned)((m * n + 255) / 256), (unsigned)batch);
    hipLaunchKernelGGL(scale_c_kernel, grid, dim3(256), 0, stream, (int)kind, c, m, n, rsc, csc,
                       bsc, beta_i, beta_f);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void requant_fill_kernel(const EpiParams ep, int64_t m,
                                                           int64_t n) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= m * n) return;
    Store<EpiKind::Q8>::apply(ep, 0, (int)(idx / n), (int)(idx % n), 0);
}

hipError_t launch_requant_fill(const EpiParams &ep, int64_t m, int64_t n, hipStream_t stream) {
    if (m == 0 || n == 0) return hipSuccess;
    dim3 grid((unsigned)((m * n + 255) / 256));
    hipLaunchKernelGGL(requant_fill_kernel, grid, dim3(256), 0, stream, ep, m, n);
    return hipGetLastError();
}

// Fused degenerate map: one thread per element of a (batch x) m x n view in the
// user frame.  beta*C stays a separate rounding before the bias add, as in the
// reference's scalar loop.
__global__ __launch_bounds__(256) void fused_fill_kernel(const EpiParams ep, int64_t m,
                                                         int64_t n) {
#pragma clang fp contract(off)
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t z = blockIdx.y;
    if (idx >= m * n) return;
    const int i = (int)(idx / n), j = (int)(idx % n);
    const int64_t off = z * ep.bsc + (int64_t)i * ep.rsc + (int64_t)j * ep.csc;
    if (ep.kind == EpiKind::F32) {
        float *p = (float *)ep.c + off;
        const float base = ep.beta_f == 0.0f ? 0.0f : (ep.beta_f == 1.0f ? *p : ep.beta_f * *p);
        *p = fused_map<false>(ep, base, i, j);
    } else {
        uint16_t *p = (uint16_t *)ep.c + off;
        const float base = ep.beta_f == 0.0f
                               ? 0.0f
                               : (ep.beta_f == 1.0f ? bf16_widen(*p) : ep.beta_f * bf16_widen(*p));
        *p = bf16_rne(fused_map<true>(ep, base, i, j));
    }
}

hipError_t launch_fused_fill(const EpiParams &ep, int64_t m, int64_t n, int64_t batch,
                             hipStream_t stream) {
    if (m == 0 || n == 0 || batch == 0) return hipSuccess;
    dim3 grid((unsigned)((m * n + 255) / 256), (unsigned)batch);
    hipLaunchKernelGGL(fused_fill_kernel, grid, dim3(256), 0, stream, ep, m, n);
    return hipGetLastError();
}

}  // namespace gk
