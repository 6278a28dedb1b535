// internal.h -- shared declarations of the gfx950 GEMM engine (not installed).
//
// Kernel frame.  Every MFMA launch computes C[M,N] = epi(sum_k A[m,k] * B[n,k])
// where A (M x K) and B (N x K) are "k-contiguous": element (r, p) of an operand
// lives at base + r*ld + p, rows 16-byte aligned, K*sizeof(T) a multiple of 16.
// That is the layout gemmkit's packers produce for its microkernels
// (src/pack.rs:28-117): the contraction index is the fast one.  The host
// dispatcher (capi.cpp) brings every call into this frame with the
// reference's orientation swap (src/dispatch.rs:395-417) -- free here because
// both operands are k-contiguous -- and packs an operand into the workspace
// only when its own strides are not k-contiguous.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace gk {

enum class InType : int { I8 = 0, BF16 = 1, F32 = 2 };
enum class EpiKind : int { I32 = 0, F32 = 1, BF16 = 2, Q8 = 3 };

inline size_t in_size(InType t) { return t == InType::I8 ? 1 : (t == InType::BF16 ? 2 : 4); }

// Epilogue parameters, a POD passed by value to the kernels.
struct EpiParams {
    EpiKind kind;
    void *c;               // output base (kernel frame)
    int64_t rsc, csc;      // output element strides (kernel frame)
    int64_t bsc;           // batch stride of C in elements
    int32_t alpha_i, beta_i;
    float alpha_f, beta_f;
    // requantization (EpiKind::Q8)
    float scale;
    const float *scales;   // per-channel scales or nullptr
    const int32_t *bias;   // per-channel bias or nullptr
    int32_t axis;          // 0: channel = kernel row, 1: channel = kernel column
    int32_t zp, lo, hi;    // zero point and clamp band (ReLU already folded into lo)
    int32_t vec4;          // C is unit-stride along columns and 4-element aligned
    // fused bias and activation (EpiKind::F32 / BF16, FusedEpi in
    // src/kernel/epilogue.rs:269-330): v <- act(v + fbias[channel]) on the f32
    // value the plain store would write, channel along `axis`; fbias holds f32
    // for F32 output and bf16 for BF16 output.
    int32_t fused;         // fbias != nullptr || act != kActNone
    int32_t act;           // FusedAct
    float slope;           // LeakyReLU slope (widened to f32)
    const void *fbias;     // bias vector or nullptr
};

enum FusedAct : int32_t { kActNone = 0, kActRelu = 1, kActLeakyRelu = 2 };

// Largest operand row stride and row length (bytes) the matrix-core kernels
// address: 256 row strides plus a row stay below 2^31 bytes of 32-bit buffer
// offsets.
constexpr int64_t kMaxTileRowBytes = 0x7FFFFFF0 / 256;
// Buffer-resource sizes of the matrix-core kernels stay at or below
// kMaxRecords; a lane meant to read zeros uses the offset kOutOfRange.  Every
// row a tile addresses (all BM rows of A and BN rows of B^T, past the matrix
// edge and the column pitch included) plus its K bytes must stay within
// kMaxRecords, so 32-bit offsets never wrap and kOutOfRange is always out of
// range.
constexpr uint32_t kMaxRecords = 0x7FFFFFF0u;
constexpr uint32_t kOutOfRange = 0x80000000u;
static_assert(kOutOfRange > kMaxRecords, "out-of-range offset must exceed every resource size");
inline bool panels_fit(int64_t bm, int64_t bn, int64_t lda_bytes, int64_t ldb_bytes, int64_t kbytes) {
    const int64_t kb16 = (kbytes + 15) / 16 * 16;
    return (bm - 1) * lda_bytes + kb16 <= (int64_t)kMaxRecords &&
           (bn - 1) * ldb_bytes + kb16 <= (int64_t)kMaxRecords;
}

struct MmaArgs {
    const void *a;         // M x K, k-contiguous
    const void *b;         // N x K, k-contiguous
    int64_t lda, ldb;      // row strides in elements
    int64_t bsa, bsb;      // batch strides in elements
    int32_t M, N, K;       // K in elements
    int32_t batch;
    // Split K (1 = off): K range r = [r*kchunk, min(K, (r+1)*kchunk)) of batch
    // element b (grid y = r, z = b) writes its partial sums to output slab
    // b*splits + r; kchunk is a multiple of 64 bytes of K.
    int32_t splits, kchunk;
    // Column pitch of the tiles (0 = the tile's width): tile j computes and
    // stores columns [j*pn, min(N, (j+1)*pn)), its last BN - pn B rows read
    // as zeros, so a product's columns can be cut into exactly as many tiles
    // as there are CUs for it.
    int32_t pn;
};

// Tile shapes instantiated in mfma_{i8,bf16,f32}.hip.
enum class Tile : int {
    T256x256 = 0,
    T256x128 = 1,
    T128x128 = 2,
    T64x64 = 3,
    T256x256w8 = 4,
    T256x128o2 = 5,  // 3-stage ring: two workgroups per CU
    T256x256k128 = 6,  // 128-byte stages, 2-stage ring
    T256x256w8k128 = 7,  // 8 waves, 128-byte stages, 2-stage ring
    T128x192k128 = 8,  // 128-byte stages, 3-stage ring; the pitched rest of a tail split
    T128x96k128o2 = 9,  // 4 x 1 waves, 128-byte stages, 2-stage ring, two per CU: requantizing rests
    T256x384w8k128 = 10,  // 2 x 4 waves, 128-byte stages, 2-stage ring; one round at a column pitch
    T256x352w8k128 = 11,  // likewise, 2 x 4 waves over 256 x 256 plus a 96-column strip
    T256x256w8m16 = 12,  // 8 waves, 128-byte stages, 2-stage ring, 16x16 MFMAs (mma16.hip)
    T256x352w8m16 = 13,  // 8 waves (4 x 2), 16x16 MFMAs, ping-pong, one round at a column pitch (mma16w.hip)
};

hipError_t launch_mma_i8(Tile tile, const MmaArgs &args, const EpiParams &ep, hipStream_t stream);
hipError_t launch_mma_bf16(Tile tile, const MmaArgs &args, const EpiParams &ep, hipStream_t stream);
hipError_t launch_mma(InType in, Tile tile, const MmaArgs &args, const EpiParams &ep,
                      hipStream_t stream);
// The 256 x 256 tile on 16x16 matrix-core instructions (mma16.hip): int8
// (i32, requantized) and bf16 (f32, bf16) output, unsplit, unpitched.
hipError_t launch_mma16(InType in, const MmaArgs &args, const EpiParams &ep, hipStream_t stream);
// The 256 x 352 tile on 16x16 matrix-core instructions (mma16w.hip): int8
// (i32, requantized) output, unsplit, at a column pitch of at most 352.
hipError_t launch_mma16w(InType in, const MmaArgs &args, const EpiParams &ep, hipStream_t stream);

// Short-contraction route (kstream.hip): K*esz <= kstream_max_kbytes(), the
// same kernel frame and bit-identical results as launch_mma, 128-row panels
// streaming 128-column tiles with the output write overlapping the next
// tile's loads.  Output kinds I32 (i8), F32 and BF16; no split K.
int64_t kstream_max_kbytes();
hipError_t launch_kstream(InType in, const MmaArgs &args, const EpiParams &ep, int cus,
                          hipStream_t stream);

// GEMV route (gemv.hip).  Dot form: out[r] = epi(sum_p mat[r,p] * vec_j[p]) for
// nvec vectors (nvec <= 8); mat rows are k-contiguous.
struct GemvArgs {
    const void *mat;       // R x K, k-contiguous rows, ld elements apart
    int64_t ld;
    const void *vec;       // nvec x K: element (j, p) at vec + j*vld + p*vks
    int64_t vld, vks;      // vks == 1 (k-contiguous) except on the skinny route
    int32_t R, K, nvec;
    int32_t cus;           // compute units of the device (persistent grid size)
    int32_t batch;         // batch elements (grid y), at most kMaxGridZ
    int64_t bsm, bsv;      // batch strides of mat and vec in elements
    // Output element (vector j, matrix row r) of batch element z is stored as
    // the epilogue's (row j, column r) of element z: at c + z*bsc + j*rsc +
    // r*csc of the EpiParams.  Each element's arithmetic does not depend on
    // the batch count or the grid size.
};

// Small f32 products (small.hip): one workgroup per 32 x 32 block of C, K
// split over its sixteen waves, operands read in place.  A is M x K with element
// (m, k) at a + m*rsa + k*ksa; B^T is N x K with element (n, k) at
// b + n*rsb + k*ksb; batch element z at + z*bsa / z*bsb (grid y).
struct SmallArgs {
    const void *a, *b;
    int64_t rsa, ksa, rsb, ksb, bsa, bsb;
    int32_t M, N, K, batch;
};
hipError_t launch_small_f32(const SmallArgs &g, const EpiParams &ep, hipStream_t stream);

// Batch elements one launch covers (grid z of the tiles, grid y of the
// skinny and GEMV kernels).
constexpr int64_t kMaxGridZ = 65535;
hipError_t launch_gemv(InType in, const GemvArgs &g, const EpiParams &ep, hipStream_t stream);

// Matrix-core skinny route (1..16 vectors): the vectors are staged in LDS,
// which must hold skinny_lds_bytes() <= kSkinnyLdsMax (a CU has 160 KiB).
constexpr int64_t kSkinnyLdsMax = 128 * 1024;
int64_t skinny_lds_bytes(InType in, int64_t K, int nvec);
hipError_t launch_skinny(InType in, const GemvArgs &g, const EpiParams &ep, hipStream_t stream);

// Pack a strided rows x K operand into a k-contiguous buffer with row stride
// ld (>= K, ld*esize a multiple of 16); columns [K, ld) are zero-filled.
hipError_t launch_pack(InType in, const void *src, int64_t rs, int64_t cs, int64_t rows,
                       int64_t K, void *dst, int64_t ld, hipStream_t stream);

// C <- beta*C for the degenerate k == 0 / alpha == 0 cases (scale_c_int,
// src/dispatch/int.rs:150-163, and its float twin src/dispatch.rs:484-497).
hipError_t launch_scale_c(EpiKind kind, void *c, int64_t m, int64_t n, int64_t rsc,
                          int64_t csc, int64_t batch, int64_t bsc, int32_t beta_i,
                          float beta_f, hipStream_t stream);

// k == 0 requant fill (requant_degenerate, src/dispatch/int.rs:735-752).
hipError_t launch_requant_fill(const EpiParams &ep, int64_t m, int64_t n, hipStream_t stream);

// Split-K reduction: C = epi(sum over r of partial slab b*splits + r), the
// slabs (M x N, row-major, i32 for i8 inputs, f32 otherwise) summed in r
// order; `ep` in the kernel frame, batch element b at ep.bsc.
hipError_t launch_split_reduce(InType in, const void *part, int splits, int64_t M, int64_t N,
                               int64_t batch, const EpiParams &ep, hipStream_t stream);

// Fused degenerate map C <- act(beta*C + bias) when the A*B term vanishes
// (fused_degenerate_float, src/dispatch/float.rs:739-758; fused_degenerate_mixed,
// src/dispatch/mixed.rs:490-512).  `ep` in the user frame, batch elements bsc apart.
hipError_t launch_fused_fill(const EpiParams &ep, int64_t m, int64_t n, int64_t batch,
                             hipStream_t stream);

}  // namespace gk
