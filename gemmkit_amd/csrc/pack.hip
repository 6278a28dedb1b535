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
//   split_reduce     sums the partial products of a split-K matrix-core launch
//                    and applies the call's epilogue.
#include <type_traits>

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
    // All 16 loads of a thread are issued before any is used (one memory
    // round trip per tile, not sixteen).
    const bool k_fast = (cs < 0 ? -cs : cs) <= (rs < 0 ? -rs : rs);
    T v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int y = ty + 4 * i;
        int64_t r, p;
        if (k_fast) { r = r0 + y; p = p0 + tx; } else { r = r0 + tx; p = p0 + y; }
        v[i] = (r < rows && p < K) ? src[r * rs + p * cs] : T(0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int y = ty + 4 * i;
        if (k_fast) tile[y][tx] = v[i]; else tile[tx][y] = v[i];
    }
    __syncthreads();
    // Write: consecutive threads write consecutive k; columns [K, ld) get zeros.
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int y = ty + 4 * i;
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

// Split-K reduction: one thread per 4 consecutive output elements of one
// batch element (blockIdx.y) when N % 4 == 0 (16-byte partial loads), else
// one per element.  The partial slabs are summed in K-range order (wrapping
// for i32), eight slabs' loads in flight at a time, then stored through the
// call's epilogue.
template <EpiKind E, typename A, int W>
__global__ __launch_bounds__(256) void split_reduce_kernel(const A *__restrict__ part, int splits,
                                                           int64_t M, int64_t N,
                                                           const EpiParams ep) {
    typedef A vec_t __attribute__((ext_vector_type(W)));
    const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * W;
    const int64_t z = blockIdx.y;
    const int64_t slab = M * N;
    if (idx >= slab) return;
    const A *p = part + z * splits * slab + idx;
    vec_t acc = *(const vec_t *)p;
    for (int r0 = 1; r0 < splits; r0 += 8) {
        vec_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (r0 + u < splits) v[u] = *(const vec_t *)(p + (r0 + u) * slab);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (r0 + u < splits) {
                if constexpr (std::is_integral<A>::value) {
#pragma unroll
                    for (int e = 0; e < W; ++e) acc[e] = (A)((uint32_t)acc[e] + (uint32_t)v[u][e]);
                } else {
                    acc = acc + v[u];
                }
            }
        }
    }
    const int row = (int)(idx / N), col = (int)(idx % N);
#pragma unroll
    for (int e = 0; e < W; ++e) Store<E>::apply(ep, z, row, col + e, acc[e]);
}

template <EpiKind E, typename A>
static void split_reduce_go(const A *p, int splits, int64_t M, int64_t N, int64_t batch,
                            const EpiParams &ep, hipStream_t stream) {
    if (N % 4 == 0) {
        dim3 grid((unsigned)((M * N / 4 + 255) / 256), (unsigned)batch);
        hipLaunchKernelGGL((split_reduce_kernel<E, A, 4>), grid, dim3(256), 0, stream, p, splits,
                           M, N, ep);
    } else {
        dim3 grid((unsigned)((M * N + 255) / 256), (unsigned)batch);
        hipLaunchKernelGGL((split_reduce_kernel<E, A, 1>), grid, dim3(256), 0, stream, p, splits,
                           M, N, ep);
    }
}

hipError_t launch_split_reduce(InType in, const void *part, int splits, int64_t M, int64_t N,
                               int64_t batch, const EpiParams &ep, hipStream_t stream) {
    if (M == 0 || N == 0 || batch == 0) return hipSuccess;
    if (in == InType::I8) {
        const int32_t *p = (const int32_t *)part;
        if (ep.kind == EpiKind::I32)
            split_reduce_go<EpiKind::I32>(p, splits, M, N, batch, ep, stream);
        else if (ep.kind == EpiKind::Q8)
            split_reduce_go<EpiKind::Q8>(p, splits, M, N, batch, ep, stream);
        else
            return hipErrorInvalidValue;
    } else {
        const float *p = (const float *)part;
        if (ep.kind == EpiKind::F32)
            split_reduce_go<EpiKind::F32>(p, splits, M, N, batch, ep, stream);
        else if (ep.kind == EpiKind::BF16)
            split_reduce_go<EpiKind::BF16>(p, splits, M, N, batch, ep, stream);
        else
            return hipErrorInvalidValue;
    }
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
