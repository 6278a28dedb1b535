// mfma_gemm.hip -- LDS-tiled CDNA4 matrix-core GEMM for i8 -> i32, bf16 -> f32 and
// f32 -> f32, with the epilogue applied to the accumulator registers.
//
// Replaces gemmkit's packing + BLIS 5-loop + microkernel layers
// (src/driver.rs:402-944, src/kernel/int.rs:138-490, src/kernel/mixed.rs:31-400,
// src/kernel/float.rs:150-281) with one workgroup per BM x BN output tile.
//
// Data path (one workgroup = 4 waves of 64 lanes, 2 x 2 over the tile):
//   * K advances in stages of 128 bytes per row (128 i8, 64 bf16, 32 f32).
//   * Each thread loads whole 16-byte chunks of the A and B stage (8 chunks per
//     row, consecutive threads cover consecutive chunks of a row: coalesced),
//     and writes them to a double-buffered LDS tile.  Row r of a stage stores
//     chunk c at slot c ^ (r & 7), so the MFMA operand reads below -- 8 lanes
//     reading the same chunk of 8 consecutive rows -- hit 8 distinct 16-byte
//     bank groups (no LDS bank conflicts).
//   * Every MFMA operand is 16 bytes per lane: lane l reads row l%32 of a
//     32-row block, chunk 2*s + l/32 of sub-step s.  That is one
//     v_mfma_i32_32x32x32_i8 (16 i8), one v_mfma_f32_32x32x16_bf16 (8 bf16) or
//     four v_mfma_f32_32x32x2_f32 (1 f32 each) per 32x32 block.  A and B use
//     the same lane -> k mapping, so each instruction pairs A[i,k] with B[k,j]
//     whatever order the hardware sums its k values in.
//   * The next stage's global loads are issued before the current stage's
//     MFMAs, so their latency hides behind the matrix work.
// The 32x32 accumulator block lives in 16 registers per lane: register r of
// lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include "epilogue.h"

namespace gk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

template <InType T>
struct Mma;

template <>
struct Mma<InType::I8> {
    using acc_t = v16i;
    using scalar_t = int32_t;
    static constexpr EpiKind native = EpiKind::I32;
    __device__ __forceinline__ static acc_t step(v4i a, v4i b, acc_t c) {
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mma<InType::BF16> {
    using acc_t = v16f;
    using scalar_t = float;
    static constexpr EpiKind native = EpiKind::F32;
    __device__ __forceinline__ static acc_t step(v4i a, v4i b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a),
                                                       __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
    }
};

template <>
struct Mma<InType::F32> {
    using acc_t = v16f;
    using scalar_t = float;
    static constexpr EpiKind native = EpiKind::F32;
    __device__ __forceinline__ static acc_t step(v4i a, v4i b, acc_t c) {
        v4f af = __builtin_bit_cast(v4f, a);
        v4f bf = __builtin_bit_cast(v4f, b);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(af[0], bf[0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(af[1], bf[1], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(af[2], bf[2], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(af[3], bf[3], c, 0, 0, 0);
        return c;
    }
};

constexpr int kThreads = 256;
constexpr int kStageBytes = 128;  // K bytes per row per stage

// Workgroup id -> (tile_m, tile_n).  The hardware hands consecutive workgroup
// ids to the 8 XCDs round-robin; the first remap gives every XCD one
// contiguous range of logical ids, and the grouped order below makes each
// range a compact block of tiles, so the A rows and B columns it needs stay in
// that XCD's L2.
__device__ __forceinline__ void tile_coords(int bid, int nblocks, int tiles_m, int tiles_n,
                                            int &tm, int &tn) {
    const int X = 8;
    int per = nblocks / X, rem = nblocks % X;
    int xcd = bid % X, idx = bid / X;
    int pid = xcd * per + (xcd < rem ? xcd : rem) + idx;
    const int G = 8;
    int in_group = G * tiles_n;
    int group = pid / in_group;
    int first_m = group * G;
    int gsize = tiles_m - first_m < G ? tiles_m - first_m : G;
    int r = pid % in_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

template <InType T, EpiKind E, int BM, int BN>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
void mma_kernel(const MmaArgs args, const EpiParams ep) {
    constexpr int WM = 2, WN = 2;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int A_CH = BM * 8 / kThreads;  // 16-byte chunks per thread per stage
    constexpr int B_CH = BN * 8 / kThreads;
    constexpr int A_BYTES = BM * kStageBytes;
    constexpr int STAGE = (BM + BN) * kStageBytes;
    static_assert(A_CH >= 1 && B_CH >= 1 && TM >= 1 && TN >= 1, "tile too small");
    using M = Mma<T>;
    using acc_t = typename M::acc_t;

    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    const int tiles_m = (args.M + BM - 1) / BM;
    const int tiles_n = (args.N + BN - 1) / BN;
    int tmi, tni;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tmi, tni);
    const int m0 = tmi * BM, n0 = tni * BN;
    const int64_t z = blockIdx.z;

    const int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    const int64_t kbytes = (int64_t)args.K * esz;
    const int64_t lda_b = args.lda * esz, ldb_b = args.ldb * esz;
    const uint8_t *A = (const uint8_t *)args.a + z * args.bsa * esz;
    const uint8_t *B = (const uint8_t *)args.b + z * args.bsb * esz;

    // Per-thread global chunk coordinates (fixed across stages).
    const uint8_t *a_src[A_CH];
    bool a_ok[A_CH];
    int a_lds[A_CH];
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
        int q = tid + i * kThreads;
        int row = q >> 3, ch = q & 7;
        int grow = m0 + row;
        a_ok[i] = grow < args.M;
        a_src[i] = A + (int64_t)(a_ok[i] ? grow : 0) * lda_b + ch * 16;
        a_lds[i] = row * kStageBytes + ((ch ^ (row & 7)) << 4);
    }
    const uint8_t *b_src[B_CH];
    bool b_ok[B_CH];
    int b_lds[B_CH];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
        int q = tid + i * kThreads;
        int row = q >> 3, ch = q & 7;
        int gcol = n0 + row;
        b_ok[i] = gcol < args.N;
        b_src[i] = B + (int64_t)(b_ok[i] ? gcol : 0) * ldb_b + ch * 16;
        b_lds[i] = A_BYTES + row * kStageBytes + ((ch ^ (row & 7)) << 4);
    }

    v4i ra[A_CH], rb[B_CH];
    auto load_stage = [&](int kt) {
        const int64_t kb = (int64_t)kt * kStageBytes;
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            int ch = (tid + i * kThreads) & 7;
            bool ok = a_ok[i] && (kb + ch * 16 < kbytes);
            ra[i] = ok ? *(const v4i *)(a_src[i] + kb) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            int ch = (tid + i * kThreads) & 7;
            bool ok = b_ok[i] && (kb + ch * 16 < kbytes);
            rb[i] = ok ? *(const v4i *)(b_src[i] + kb) : v4i{0, 0, 0, 0};
        }
    };
    auto store_stage = [&](int buf) {
        uint8_t *s = smem + buf * STAGE;
#pragma unroll
        for (int i = 0; i < A_CH; ++i) *(v4i *)(s + a_lds[i]) = ra[i];
#pragma unroll
        for (int i = 0; i < B_CH; ++i) *(v4i *)(s + b_lds[i]) = rb[i];
    };

    acc_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = acc_t{};

    // Operand read offsets within a stage for this lane.
    const int lrow = lane & 31, lhalf = lane >> 5;
    int a_row_off[TM], b_row_off[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) a_row_off[i] = (wm * WTM + i * 32 + lrow) * kStageBytes;
#pragma unroll
    for (int j = 0; j < TN; ++j) b_row_off[j] = A_BYTES + (wn * WTN + j * 32 + lrow) * kStageBytes;
    const int swz = lrow & 7;  // (row & 7) == (lrow & 7): block bases are multiples of 32

    const int KT = (int)((kbytes + kStageBytes - 1) / kStageBytes);
    load_stage(0);
    store_stage(0);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) load_stage(kt + 1);
        const uint8_t *s = smem + cur * STAGE;
#pragma unroll
        for (int ss = 0; ss < 4; ++ss) {
            const int slot = ((2 * ss + lhalf) ^ swz) << 4;
            v4i af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = *(const v4i *)(s + a_row_off[i] + slot);
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = *(const v4i *)(s + b_row_off[j] + slot);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = M::step(af[i], bf[j], acc[i][j]);
        }
        if (kt + 1 < KT) store_stage(cur ^ 1);
        __syncthreads();
    }

    // Epilogue on the accumulator registers.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WTN + j * 32 + lrow;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WTM + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
                if (row < args.M && col < args.N)
                    Store<E>::apply(ep, z, row, col, acc[i][j][r]);
            }
        }
    }
}

template <InType T, EpiKind E, int BM, int BN>
static hipError_t launch_one(const MmaArgs &args, const EpiParams &ep, hipStream_t stream) {
    int tiles = ((args.M + BM - 1) / BM) * ((args.N + BN - 1) / BN);
    dim3 grid(tiles, 1, args.batch);
    hipLaunchKernelGGL((mma_kernel<T, E, BM, BN>), grid, dim3(kThreads), 0, stream, args, ep);
    return hipGetLastError();
}

template <InType T, EpiKind E>
static hipError_t launch_tile(Tile tile, const MmaArgs &args, const EpiParams &ep,
                              hipStream_t stream) {
    switch (tile) {
    case Tile::T256x256: return launch_one<T, E, 256, 256>(args, ep, stream);
    case Tile::T256x128: return launch_one<T, E, 256, 128>(args, ep, stream);
    case Tile::T128x128: return launch_one<T, E, 128, 128>(args, ep, stream);
    case Tile::T64x64: return launch_one<T, E, 64, 64>(args, ep, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_mma(InType in, Tile tile, const MmaArgs &args, const EpiParams &ep,
                      hipStream_t stream) {
    switch (in) {
    case InType::I8:
        if (ep.kind == EpiKind::I32) return launch_tile<InType::I8, EpiKind::I32>(tile, args, ep, stream);
        if (ep.kind == EpiKind::Q8) return launch_tile<InType::I8, EpiKind::Q8>(tile, args, ep, stream);
        break;
    case InType::BF16:
        if (ep.kind == EpiKind::F32) return launch_tile<InType::BF16, EpiKind::F32>(tile, args, ep, stream);
        if (ep.kind == EpiKind::BF16) return launch_tile<InType::BF16, EpiKind::BF16>(tile, args, ep, stream);
        break;
    case InType::F32:
        if (ep.kind == EpiKind::F32) return launch_tile<InType::F32, EpiKind::F32>(tile, args, ep, stream);
        break;
    }
    return hipErrorInvalidValue;
}

}  // namespace gk
