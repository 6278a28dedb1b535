// gemv.hip -- HBM-bandwidth GEMV for skinny products (1..8 vectors).
//
// Replaces gemmkit's gemv route (src/special/gemv.rs:101-600, taken at
// m == 1 || n == 1 by src/dispatch/float.rs:81) and serves the i8 skinny shapes
// too (the reference has no i8 gemv: src/dispatch/int.rs:165-168; i8 results do
// not depend on the route because wrapping i32 addition is associative).
//
// out[j, r] = epi( sum_p mat[r, p] * vec[j, p] ),  r < R rows, j < nvec <= 8.
// The matrix streams from HBM exactly once with 16-byte loads; the nvec
// vectors are staged once per workgroup in LDS.  Each wave owns RPW rows at a
// time and keeps RPW x UNROLL loads in flight per lane; partial sums are
// reduced across the wave with cross-lane shuffles.
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
    __device__ __forceinline__ static acc_t reduce(acc_t v) {
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        return v;
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
    __device__ __forceinline__ static acc_t reduce(acc_t v) {
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        return v;
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
    __device__ __forceinline__ static acc_t reduce(acc_t v) {
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        return v;
    }
};

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / 64;
constexpr int kUnroll = 4;

// Largest staged vector block (bytes) a workgroup keeps in LDS.
constexpr int kGemvLdsMax = 64 * 1024;

template <InType T, EpiKind E, int NV, int RPW>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(const GemvArgs g, const EpiParams ep) {
    using D = Dot16<T>;
    using acc_t = typename D::acc_t;
    extern __shared__ __attribute__((aligned(16))) uint8_t sv[];
    const int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    // 16-byte chunks per row.  A K*esz that is not a multiple of 16 only reaches
    // this kernel through the pack, which zero-fills both operands' rows up to
    // the next 16 bytes, so the padded tail adds nothing.
    const int64_t nch = ((int64_t)g.K * esz + 15) / 16;
    const int nvec = g.nvec;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint8_t *vec = (const uint8_t *)g.vec;
    const int64_t vld_b = g.vld * esz;
    const bool staged = (int64_t)nvec * nch * 16 <= kGemvLdsMax;
    if (staged) {
        for (int64_t c = tid; c < nvec * nch; c += kGemvThreads) {
            int64_t j = c / nch, ch = c % nch;
            *(v4i_g *)(sv + c * 16) = *(const v4i_g *)(vec + j * vld_b + ch * 16);
        }
        __syncthreads();
    }
    const uint8_t *mat = (const uint8_t *)g.mat;
    const int64_t ld_b = g.ld * esz;
    const int64_t total_waves = (int64_t)gridDim.x * kGemvWaves;
    for (int64_t r0 = ((int64_t)blockIdx.x * kGemvWaves + wave) * RPW; r0 < g.R;
         r0 += total_waves * RPW) {
        acc_t acc[RPW][NV];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int j = 0; j < NV; ++j) acc[r][j] = acc_t(0);
        const uint8_t *rowp[RPW];
        bool rok[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            rok[r] = r0 + r < g.R;
            rowp[r] = mat + (rok[r] ? r0 + r : r0) * ld_b;
        }
        int64_t ch = lane;
        for (; ch + 64 * (kUnroll - 1) < nch; ch += 64 * kUnroll) {
            v4i_g m[kUnroll][RPW];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
#pragma unroll
                for (int r = 0; r < RPW; ++r)
                    m[u][r] = __builtin_nontemporal_load((const v4i_g *)(rowp[r] + (ch + 64 * u) * 16));
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    if (j < nvec) {
                        const int64_t xc = j * nch + ch + 64 * u;
                        v4i_g x = staged ? *(const v4i_g *)(sv + xc * 16)
                                         : *(const v4i_g *)(vec + j * vld_b + (ch + 64 * u) * 16);
#pragma unroll
                        for (int r = 0; r < RPW; ++r) acc[r][j] = D::dot(m[u][r], x, acc[r][j]);
                    }
                }
            }
        }
        for (; ch < nch; ch += 64) {
            v4i_g m[RPW];
#pragma unroll
            for (int r = 0; r < RPW; ++r) m[r] = *(const v4i_g *)(rowp[r] + ch * 16);
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                if (j < nvec) {
                    v4i_g x = staged ? *(const v4i_g *)(sv + (j * nch + ch) * 16)
                                     : *(const v4i_g *)(vec + j * vld_b + ch * 16);
#pragma unroll
                    for (int r = 0; r < RPW; ++r) acc[r][j] = D::dot(m[r], x, acc[r][j]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                if (j < nvec) {
                    acc_t v = D::reduce(acc[r][j]);
                    if (lane == j && rok[r]) Store<E>::apply(ep, 0, j, (int)(r0 + r), v);
                }
            }
        }
    }
}

template <InType T, EpiKind E, int NV>
static hipError_t gemv_go(const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    constexpr int RPW = (NV <= 2) ? 4 : 2;
    const int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    int64_t vbytes = (int64_t)g.nvec * (((int64_t)g.K * esz + 15) / 16) * 16;
    size_t shm = vbytes <= kGemvLdsMax ? (size_t)vbytes : 0;
    int64_t waves_needed = (g.R + RPW - 1) / RPW;
    int64_t blocks = (waves_needed + kGemvWaves - 1) / kGemvWaves;
    // Cap the grid so staging the vectors stays a small fraction of the traffic.
    const int64_t cap = 256 * 8;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL((gemv_kernel<T, E, NV, RPW>), dim3((unsigned)blocks), dim3(kGemvThreads),
                       shm, stream, g, ep);
    return hipGetLastError();
}

template <InType T, EpiKind E>
static hipError_t gemv_nv(const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    if (g.nvec <= 1) return gemv_go<T, E, 1>(g, ep, stream);
    if (g.nvec <= 2) return gemv_go<T, E, 2>(g, ep, stream);
    if (g.nvec <= 4) return gemv_go<T, E, 4>(g, ep, stream);
    return gemv_go<T, E, 8>(g, ep, stream);
}

hipError_t launch_gemv(InType in, const GemvArgs &g, const EpiParams &ep, hipStream_t stream) {
    if (g.nvec < 1 || g.nvec > 8) return hipErrorInvalidValue;
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
