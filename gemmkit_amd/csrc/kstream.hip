// kstream.hip -- matrix-core GEMM for a short contraction (K at most 256 bytes
// per row: K <= 128 bf16, 64 f32, 256 i8), where the output write, not the
// arithmetic, bounds the product: batched attention scores (64 x 512 x 512 x
// 128 bf16 with f32 output write 67 MB and read 17 MB).
//
// Same kernel frame and arithmetic as mma_kernel (mma_kernel.h): C[M,N] =
// epi(sum_k A[m,k] B[n,k]) with k-contiguous operands, the same MFMA
// instructions fed the same 16-byte k chunks in the same order, so every
// output is bit-identical to the tile kernels'.  What differs is the data
// flow.  A workgroup owns a 128-row panel of one batch element and streams a
// run of 128-column tiles across it:
//   * one producer wave loads (direct-to-LDS) the panel's A rows once and
//     the B rows of each tile into a ring of S slots (3 for 256-byte rows, 4
//     for shorter ones), up to S tiles ahead (after the first tile has
//     landed): a tile's loads take a memory round trip, longer than the
//     consumers spend on a tile;
//   * eight consumer waves (4 x 2, 32 x 64 each) run the MFMAs of tile t
//     from LDS, then write tile t through a per-wave LDS staging area (16 rows
//     of a 32 x 32 block at a time, as whole 128-byte row segments) while later
//     tiles load.  Eight storing waves keep more of the write stream in flight
//     than four (attention scores 16.0 against 16.9 us in a same-process A/B).
// The consumer waves issue no loads, so their stores never hold up a wait
// (loads and stores share one completion counter), and each workgroup writes
// its tiles back to back instead of all 256 CUs writing at once at the end.
// The whole contraction sits in LDS: rows are KB = 64, 128 or 256 bytes
// (K*esz rounded up to a power of two; bytes past K load as zeros).
#include <stdlib.h>
#include <string.h>

#include "mma_kernel.h"

namespace gk {

constexpr int kKsTile = 128;                       // tile rows and columns
constexpr int kKsConsumers = 8;                    // 4 x 2 waves of 32 x 64
constexpr int kKsThreads = (kKsConsumers + 1) * 64;
constexpr int kKsEpiLd = 32 + 4;                   // staging row stride (words)

// B slots of the ring: as many as fit beside the panel and the staging.
template <int KB>
constexpr int ks_slots() {
    return KB >= 256 ? 3 : 4;
}

// Slot of 16-byte chunk c of row r in a KB-byte LDS row: 16 consecutive rows
// reading one chunk hit 16 distinct 16-byte bank groups.
template <int KB>
__device__ __forceinline__ int ks_slot(int r, int c) {
    constexpr int NCH = KB / 16;
    return c ^ ((r / (16 / NCH)) & (NCH - 1));
}

// FUSED: the call has a fused bias or activation.  Instantiated apart so
// that the plain kernel loads nothing in the consumers: a bias load would
// make the compiler wait for the wave's outstanding stores (loads and stores
// share one counter) at every block, even where the call has no bias
// (attention scores 16.95-17.5 against 17.5-17.95 us on one box).
template <InType T, EpiKind E, int KB, bool FUSED>
__global__ __launch_bounds__(kKsThreads) void kstream_kernel(const MmaArgs args, const EpiParams ep,
                                                             int tiles_m, int tiles_n, int chunk,
                                                             int nchunks) {
    using M = Mma<T>;
    using acc_t = typename M::acc_t;
    using val_t = typename M::scalar_t;
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    constexpr int TILE = kKsTile * KB;              // bytes of one 128-row operand tile
    constexpr int NLD = TILE / 1024;                // 1 KiB loads per tile
    constexpr int RPL = 1024 / KB;                  // rows one load fills
    constexpr int CPR = KB / 16;                    // chunks per row
    constexpr int SUB = KB / 32;                    // MFMA sub-steps
    constexpr int STG = 16 * kKsEpiLd * 4;          // staging bytes per consumer wave (16 rows)
    constexpr int S = ks_slots<KB>();
    __shared__ __attribute__((aligned(1024))) uint8_t smem[(1 + S) * TILE + kKsConsumers * STG];
    static_assert(sizeof(smem) <= 160 * 1024, "LDS");
    uint8_t *const a_lds = smem;
    uint8_t *const b_lds = smem + TILE;             // S slots of TILE bytes

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // Unit -> (batch element, row panel, column chunk), XCD-contiguous so the
    // panels of one element share an XCD's L2.
    const int64_t unit = xcd_logical(blockIdx.x, gridDim.x);
    const int64_t per_elem = (int64_t)tiles_m * nchunks;
    const int64_t zb = unit / per_elem;
    const int pm = (int)((unit % per_elem) / nchunks);
    const int ch0 = (int)(unit % nchunks) * chunk;
    const int ntile = tiles_n - ch0 < chunk ? tiles_n - ch0 : chunk;
    const int m0 = pm * kKsTile;

    const int64_t kbytes = (int64_t)args.K * esz;
    // A row's bytes rounded up to whole chunks: a K*esz that is not a
    // multiple of 16 only arrives through the pack, which zero-fills the rest
    // of the chunk.
    const int64_t kb16 = (kbytes + 15) / 16 * 16;
    const int64_t lda_b = args.lda * esz, ldb_b = args.ldb * esz;
    const uint8_t *A = (const uint8_t *)args.a + zb * args.bsa * esz + (int64_t)m0 * lda_b;
    const uint8_t *B = (const uint8_t *)args.b + zb * args.bsb * esz;

    if (wave == kKsConsumers) {
        // ---------------------------------------------------------- producer
        // Load q of a tile fills LDS bytes [q*1024, +1024): rows q*RPL + l/CPR,
        // slot l%CPR holding chunk slot ^ swz(row); chunks at or past K read
        // zeros (offset past the resource), as do rows past the matrix edge.
        const int rl = lane / CPR, sl = lane % CPR;
        auto load_tile = [&](const uint8_t *base, int64_t ld_b, int rows_valid, uint8_t *dst) {
            const uint32_t num = rows_valid > 0 ? (uint32_t)((rows_valid - 1) * ld_b + kb16) : 0;
#pragma unroll
            for (int q = 0; q < NLD; ++q) {
                const int row = q * RPL + rl;
                const int c = ks_slot<KB>(row, sl);  // the swizzle is its own inverse
                const bool in = (int64_t)c * 16 < kbytes && row < rows_valid;
                const uint32_t off = in ? (uint32_t)(row * ld_b + c * 16) : kOutOfRange;
                dma16(base, num, off, dst + q * 1024);
            }
        };
        auto load_b = [&](int t) {
            const int n0 = (ch0 + t) * kKsTile;
            const int rows_b = args.N - n0 < kKsTile ? args.N - n0 : kKsTile;
            load_tile(B + (int64_t)n0 * ldb_b, ldb_b, rows_b, b_lds + (t % S) * TILE);
        };
        const int rows_a = args.M - m0 < kKsTile ? args.M - m0 : kKsTile;
        // The panel and the first tile alone at first: every workgroup of the
        // launch needs them before any output exists, so the other tiles'
        // loads wait until they have landed (all of Q and the first K tiles,
        // 10 MB on the attention scores, instead of 15 MB with the ring
        // filled at once).
        load_tile(A, lda_b, rows_a, a_lds);
        load_b(0);
        // Tile t is waited for with the loads issued after it still in flight
        // (loads complete in order; the counter holds at most 63, and waiting
        // for that many or fewer is only stronger).  Barrier t publishes it;
        // every consumer has then finished tile t-1, so its slot takes tile
        // t-1+S (after barrier 0, the ring's other slots are filled).
        int hi = 0;  // last tile issued
        for (int t = 0; t < ntile; ++t) {
            const int after = hi - t;
            if (after >= 2) wait_vmcnt<(2 * NLD < 63 ? 2 * NLD : 63)>();
            else if (after == 1) wait_vmcnt<NLD>();
            else wait_vmcnt<0>();
            stage_barrier();
            if (t == 0) {
                for (int u = 1; u < S && u < ntile; ++u) load_b(u);
                hi = (S < ntile ? S : ntile) - 1;
            } else if (t - 1 + S < ntile) {
                load_b(t - 1 + S);
                hi = t - 1 + S;
            }
        }
        stage_barrier();      // the consumers' last tile
        return;
    }

    // ------------------------------------------------------------- consumers
    const int wm = wave >> 1, wn = wave & 1;
    const int lrow = lane & 31, lhalf = lane >> 5;
    constexpr int TI = 1;  // 32-row blocks per wave
    int a_off[TI], b_off[2];
#pragma unroll
    for (int i = 0; i < TI; ++i) a_off[i] = (wm * 32 * TI + i * 32 + lrow) * KB;
#pragma unroll
    for (int j = 0; j < 2; ++j) b_off[j] = (wn * 64 + j * 32 + lrow) * KB;
    val_t *const stg = (val_t *)(smem + (1 + S) * TILE + wave * STG);
    constexpr int CPRE = 8;               // 4-column chunks per staged row (32 columns)
    constexpr int RPIT = 64 / CPRE;       // rows per read iteration
    constexpr bool FB = (E == EpiKind::F32 || E == EpiKind::BF16) && FUSED;

    for (int t = 0; t < ntile; ++t) {
        stage_barrier();  // tile t's B landed (and, for t > 0, the previous tile is done)
        const uint8_t *bs = b_lds + (t % S) * TILE;
        acc_t acc[TI][2];
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = acc_t{};
#pragma unroll
        for (int s = 0; s < SUB; ++s) {
            // (block bases are multiples of 32 rows, so the swizzle of row
            // base + lrow is that of lrow)
            const int slot = ks_slot<KB>(lrow, 2 * s + lhalf) << 4;
            v4i af[TI], bf[2];
#pragma unroll
            for (int i = 0; i < TI; ++i) af[i] = *(const v4i *)(a_lds + a_off[i] + slot);
#pragma unroll
            for (int j = 0; j < 2; ++j) bf[j] = *(const v4i *)(bs + b_off[j] + slot);
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = M::step(bf[j], af[i], acc[i][j]);
        }
        // Epilogue, one 32 x 32 block at a time, 16 rows per pass through this
        // wave's staging rows: register 4g+e of lane l is C row l%32, column
        // 8g + 4*(l/32) + e of the block; rows come back as 128-byte segments
        // (8 lanes a row).
        const int n0 = (ch0 + t) * kKsTile;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int gcol0 = n0 + wn * 64 + j * 32;
            const int c4 = (lane % CPRE) * 4;
            float col_f[4] = {0, 0, 0, 0};
            if constexpr (FB) {
                if (ep.fused && ep.axis) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        col_f[e] = gcol0 + c4 + e < args.N
                                       ? fused_bias<E == EpiKind::BF16>(ep, gcol0 + c4 + e)
                                       : 0.0f;
                }
            }
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                typedef val_t v4_t __attribute__((ext_vector_type(4)));
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    // rows 16h .. 16h+15 of the block: lanes holding them stage
                    if ((lrow >> 4) == h) {
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const v4_t w = {(val_t)acc[i][j][4 * g], (val_t)acc[i][j][4 * g + 1],
                                            (val_t)acc[i][j][4 * g + 2], (val_t)acc[i][j][4 * g + 3]};
                            *(v4_t *)(stg + (lrow & 15) * kKsEpiLd + 8 * g + 4 * lhalf) = w;
                        }
                    }
                    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): staging writes done
                    __builtin_amdgcn_wave_barrier();
                    const int grow0 = m0 + wm * 32 * TI + i * 32 + 16 * h;
#pragma unroll
                    for (int it = 0; it < 16 / RPIT; ++it) {
                        const int row = it * RPIT + lane / CPRE;
                        const v4_t v4 = *(const v4_t *)(stg + row * kKsEpiLd + c4);
                        const val_t v[4] = {v4[0], v4[1], v4[2], v4[3]};
                        const int grow = grow0 + row;
                        float f4[4] = {col_f[0], col_f[1], col_f[2], col_f[3]};
                        if constexpr (FB) {
                            if (ep.fused && !ep.axis) {
                                const float f =
                                    grow < args.M ? fused_bias<E == EpiKind::BF16>(ep, grow) : 0.0f;
#pragma unroll
                                for (int e = 0; e < 4; ++e) f4[e] = f;
                            }
                        }
                        if (grow < args.M && gcol0 + c4 < args.N)
                            store4<E, val_t>(ep, zb, grow, gcol0 + c4, args.N, v, nullptr, nullptr, f4);
                    }
                    __builtin_amdgcn_s_waitcnt(0xC07F);  // staging reads done before the next half
                    __builtin_amdgcn_wave_barrier();
                }
            }
        }
    }
    stage_barrier();  // pairs with the producer's last barrier
}

// Column tiles per workgroup: all of a panel's when the panels alone give
// every CU one, else the fewest that do.
static int ks_chunk(int64_t panels, int tiles_n, int cus) {
    if (panels >= cus) return tiles_n;
    const int64_t split = (cus + panels - 1) / panels;
    const int64_t s = split < tiles_n ? split : tiles_n;
    return (int)((tiles_n + s - 1) / s);
}

template <InType T, EpiKind E, int KB>
static hipError_t ks_go(const MmaArgs &args, const EpiParams &ep, int cus, hipStream_t stream) {
    const int tiles_m = (args.M + kKsTile - 1) / kKsTile;
    const int tiles_n = (args.N + kKsTile - 1) / kKsTile;
    const int64_t panels = (int64_t)tiles_m * args.batch;
    const int chunk = ks_chunk(panels, tiles_n, cus);
    const int nchunks = (tiles_n + chunk - 1) / chunk;
    const int64_t units = panels * nchunks;
    if (units > INT32_MAX) return hipErrorInvalidValue;
    constexpr bool FLOAT_OUT = E == EpiKind::F32 || E == EpiKind::BF16;
    if (FLOAT_OUT && ep.fused)
        hipLaunchKernelGGL((kstream_kernel<T, E, KB, FLOAT_OUT>), dim3((unsigned)units),
                           dim3(kKsThreads), 0, stream, args, ep, tiles_m, tiles_n, chunk, nchunks);
    else
        hipLaunchKernelGGL((kstream_kernel<T, E, KB, false>), dim3((unsigned)units),
                           dim3(kKsThreads), 0, stream, args, ep, tiles_m, tiles_n, chunk, nchunks);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// kband_kernel -- whole output rows for the widest short contractions: rows of
// 129..256 bytes of K (KB = 256) and at most 512 columns, with enough
// 128-row panels (batch elements x row panels) to give every CU one; the
// attention scores are 256 such panels.
//
// Where kstream_kernel writes 128 x 128 tiles (512-byte row pieces), this
// kernel writes 32-row bands of whole C rows, one store instruction per 1 KiB
// run of a row, and keeps the write stream free of loads:
//   * each of the 8 waves owns 64 columns of C and holds those columns' B
//     rows (all of K) in registers for the workgroup's life (64 VGPRs): it
//     loads them once, direct-to-LDS into a region of its own (whole 256-byte
//     rows per 16 lanes, so every load is a full-line read), and reads its
//     fragments from there (no barrier: no other wave touches the region);
//     the regions then hold the output staging;
//   * the workgroup's 128-row A panel goes to LDS by direct-to-LDS loads at
//     the start, band 0's rows first;
//   * per 32-row band: each wave's two 32 x 32 blocks (the same instructions,
//     operand order and k order as the other routes, so every output is
//     bit-identical), staged in LDS as whole rows, then each wave stores 4
//     rows as 1 KiB runs (nontemporal, written through the L2: StPol::NTWT).
// Every load is issued before the first store, so no wait for a load waits
// on a store (loads and stores share one completion counter): the stores of
// all four bands go out back to back behind one startup.
constexpr int kKbBand = 32;          // rows per band
constexpr int kKbKB = 256;           // K bytes per row (the rest read as zeros)

template <InType T, EpiKind E>
__global__ __launch_bounds__(512) void kband_kernel(const MmaArgs args, const EpiParams ep,
                                                    int tiles_m) {
    using M = Mma<T>;
    using acc_t = typename M::acc_t;
    using val_t = typename M::scalar_t;
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    constexpr int NW = 8;                         // waves, 64 columns each
    constexpr int KB = kKbKB;
    constexpr int SUB = KB / 32;                  // MFMA sub-steps per 32 x 32 block
    constexpr int PANEL = 128;                    // rows per workgroup
    constexpr int NBAND = PANEL / kKbBand;        // 4
    constexpr int COLS = NW * 64;                 // columns: whole rows of up to 512
    constexpr int LD = COLS + 4;                  // staging row stride (words)
    constexpr int CPR = KB / 16;                  // chunks per row
    constexpr int RPL = 1024 / KB;                // rows one 1 KiB load fills
    constexpr int A_BYTES = PANEL * KB;
    constexpr int LPB = kKbBand * KB / 1024 / NW; // A loads per wave per band
    constexpr int BW_BYTES = 64 * KB;             // one wave's B rows: 16 KiB
    constexpr int NLB = BW_BYTES / 1024;          // 1 KiB loads of them
    constexpr int RUNS = COLS / 256;              // store instructions per row (1 KiB for f32 / i32)
    constexpr int RPW = kKbBand / NW;             // band rows each wave stores
    static_assert(kKbBand * LD * 4 <= NW * BW_BYTES, "staging fits the B regions");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[A_BYTES + NW * BW_BYTES];
    static_assert(sizeof(smem) <= 160 * 1024, "LDS");
    uint8_t *const a_lds = smem;
    val_t *const stg = (val_t *)(smem + A_BYTES);  // after the B fragments are in registers

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, lhalf = lane >> 5;

    // Unit -> (batch element, row panel), XCD-contiguous: an element's four
    // panels share its B rows in one XCD's L2.
    const int64_t unit = xcd_logical(blockIdx.x, gridDim.x);
    const int64_t zb = unit / tiles_m;
    const int m0 = (int)(unit % tiles_m) * PANEL;

    const int64_t kbytes = (int64_t)args.K * esz;
    const int64_t kb16 = (kbytes + 15) / 16 * 16;
    const int64_t lda_b = args.lda * esz, ldb_b = args.ldb * esz;
    const uint8_t *A = (const uint8_t *)args.a + zb * args.bsa * esz + (int64_t)m0 * lda_b;

    // A panel: load q = (band*NW + wave)*LPB + u fills LDS bytes
    // [q*1024, +1024), rows q*RPL + l/CPR, slot l%CPR holding chunk
    // ks_slot(row, slot); chunks at or past K and rows past M read zeros.
    const int rows_a = args.M - m0 < PANEL ? args.M - m0 : PANEL;
    const uint32_t a_num = (uint32_t)((rows_a - 1) * lda_b + kb16);
    auto load_a = [&](int band) {
#pragma unroll
        for (int u = 0; u < LPB; ++u) {
            const int q = (band * NW + wave) * LPB + u;
            const int row = q * RPL + lane / CPR;
            const int c = ks_slot<KB>(row, lane % CPR);
            const bool in = (int64_t)c * 16 < kbytes && row < rows_a;
            dma16(A, a_num, in ? (uint32_t)(row * lda_b + c * 16) : kOutOfRange, a_lds + q * 1024);
        }
    };

    // This wave's B rows (C columns n0 .. n0+63) into its LDS region, laid
    // out as the A panel; columns at or past N read zeros (and are not
    // stored).
    const int n0 = wave * 64;
    const int rows_b = args.N - n0 < 64 ? args.N - n0 : 64;
    const uint8_t *Bw = (const uint8_t *)args.b + zb * args.bsb * esz;
    const uint32_t b_num = rows_b > 0 ? (uint32_t)((rows_b - 1) * ldb_b + kb16) : 0u;
    if (rows_b > 0) Bw += (int64_t)n0 * ldb_b;
    uint8_t *const b_lds = smem + A_BYTES + wave * BW_BYTES;

    load_a(0);
#pragma unroll
    for (int q = 0; q < NLB; ++q) {
        const int row = q * RPL + lane / CPR;
        const int c = ks_slot<KB>(row, lane % CPR);
        const bool in = (int64_t)c * 16 < kbytes && row < rows_b;
        dma16(Bw, b_num, in ? (uint32_t)(row * ldb_b + c * 16) : kOutOfRange, b_lds + q * 1024);
    }
#pragma unroll
    for (int b = 1; b < NBAND; ++b) load_a(b);
    wait_vmcnt<(NBAND - 1) * LPB>();  // band 0's A rows and this wave's B rows landed
    // Fragment (s, j) of lane l: row j*32 + l%32, chunk 2s + l/32, as the
    // other routes' LDS fragment reads lay it out (block bases are multiples
    // of 32 rows, so the swizzle of row base + lrow is that of lrow).
    v4i bfr[SUB][2];
#pragma unroll
    for (int s = 0; s < SUB; ++s)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            bfr[s][j] = *(const v4i *)(b_lds + (j * 32 + lrow) * KB + (ks_slot<KB>(lrow, 2 * s + lhalf) << 4));
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): B fragments read before the regions hold staging
    stage_barrier();                     // (and every wave's band 0 A rows landed)

    typedef val_t v4_t __attribute__((ext_vector_type(4)));
#pragma unroll 1
    for (int b = 0; b < NBAND; ++b) {
        acc_t acc[2] = {acc_t{}, acc_t{}};
        const int arow = b * kKbBand + lrow;
#pragma unroll
        for (int s = 0; s < SUB; ++s) {
            const v4i af = *(const v4i *)(a_lds + arow * KB + (ks_slot<KB>(arow, 2 * s + lhalf) << 4));
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[j] = M::step(bfr[s][j], af, acc[j]);
        }
        if (b == 0) wait_vmcnt<0>();  // the other bands' A rows, before any store
        // Stage: register 4g+e of block j is C row l%32, column
        // 32j + 8g + 4*(l/32) + e of this wave's 64.
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const v4_t w = {(val_t)acc[j][4 * g], (val_t)acc[j][4 * g + 1],
                                (val_t)acc[j][4 * g + 2], (val_t)acc[j][4 * g + 3]};
                *(v4_t *)(stg + lrow * LD + wave * 64 + 32 * j + 8 * g + 4 * lhalf) = w;
            }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): staging writes done
        stage_barrier();                     // (and, at band 0, every wave's A rows landed)
        // Wave w stores band rows RPW*w .. RPW*w + RPW-1, each as RUNS 1 KiB runs.
        const int64_t grow0 = (int64_t)m0 + b * kKbBand + RPW * wave;
#pragma unroll
        for (int i = 0; i < RPW * RUNS; ++i) {
            const int r = RPW * wave + i / RUNS, col = (i % RUNS) * 256 + 4 * lane;
            const v4_t v4 = *(const v4_t *)(stg + r * LD + col);
            const val_t v[4] = {v4[0], v4[1], v4[2], v4[3]};
            const int64_t grow = grow0 + i / RUNS;
            if (grow < args.M && col < args.N) store4<E, val_t, StPol::NTWT>(ep, zb, (int)grow, col, args.N, v);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // staging reads done before the next band's writes
        stage_barrier();
    }
}

// GEMMKIT_HIP_KBAND=0 keeps the widest short contractions on kstream_kernel.
static bool kband_enabled() {
    const char *s = getenv("GEMMKIT_HIP_KBAND");
    return !(s && !strcmp(s, "0"));
}

// The band kernel takes unfused calls with 129..256 K bytes per row, 257..512
// columns, rows addressable by 32-bit offsets and at least one 128-row panel
// per CU (otherwise too few workgroups).  Its arithmetic is the other routes',
// so which route runs never changes a result.
template <InType T, EpiKind E>
static bool kband_takes(const MmaArgs &args, const EpiParams &ep, int cus) {
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    const int64_t kb = (int64_t)args.K * esz;
    const int64_t kb16 = (kb + 15) / 16 * 16;
    const int64_t panels = (int64_t)((args.M + 127) / 128) * args.batch;
    return kband_enabled() && !ep.fused && kb > 128 && kb <= kKbKB && args.N > 256 && args.N <= 512 &&
           panels >= (cus > 0 ? cus : 256) && panels <= INT32_MAX &&
           panels_fit(128, 64, args.lda * esz, args.ldb * esz, kb16);
}

template <InType T, EpiKind E>
static hipError_t kb_go(const MmaArgs &args, const EpiParams &ep, hipStream_t stream) {
    const int tiles_m = (args.M + 127) / 128;
    const int64_t units = (int64_t)tiles_m * args.batch;
    hipLaunchKernelGGL((kband_kernel<T, E>), dim3((unsigned)units), dim3(512), 0, stream, args, ep,
                       tiles_m);
    return hipGetLastError();
}

template <InType T, EpiKind E>
static hipError_t ks_kb(const MmaArgs &args, const EpiParams &ep, int cus, hipStream_t stream) {
    constexpr int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    const int64_t kb = (int64_t)args.K * esz;
    if (kb <= 64) return ks_go<T, E, 64>(args, ep, cus, stream);
    if (kb <= 128) return ks_go<T, E, 128>(args, ep, cus, stream);
    if (kband_takes<T, E>(args, ep, cus)) return kb_go<T, E>(args, ep, stream);
    return ks_go<T, E, 256>(args, ep, cus, stream);
}

int64_t kstream_max_kbytes() { return 256; }

hipError_t launch_kstream(InType in, const MmaArgs &args, const EpiParams &ep, int cus,
                          hipStream_t stream) {
    // Tile rows are addressed as unsigned 32-bit offsets from the tile's
    // first row: row strides must be non-negative and short enough.
    if (args.lda < 0 || args.ldb < 0 || args.splits > 1 || args.batch < 1 ||
        args.batch > kMaxGridZ || (int64_t)args.K * in_size(in) > kstream_max_kbytes())
        return hipErrorInvalidValue;
    switch (in) {
    case InType::I8:
        if (ep.kind == EpiKind::I32) return ks_kb<InType::I8, EpiKind::I32>(args, ep, cus, stream);
        break;
    case InType::BF16:
        if (ep.kind == EpiKind::F32) return ks_kb<InType::BF16, EpiKind::F32>(args, ep, cus, stream);
        if (ep.kind == EpiKind::BF16) return ks_kb<InType::BF16, EpiKind::BF16>(args, ep, cus, stream);
        break;
    case InType::F32:
        if (ep.kind == EpiKind::F32) return ks_kb<InType::F32, EpiKind::F32>(args, ep, cus, stream);
        break;
    }
    return hipErrorInvalidValue;
}

}  // namespace gk
