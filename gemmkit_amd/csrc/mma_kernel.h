#pragma once
// mma_kernel.h -- LDS-tiled CDNA4 matrix-core GEMM for i8 -> i32, bf16 -> f32 and
// f32 -> f32, with the epilogue applied to the accumulator registers.  The
// template is instantiated per input type in mfma_{i8,bf16,f32}.hip.
//
// Replaces gemmkit's packing + BLIS 5-loop + microkernel layers
// (src/driver.rs:402-944, src/kernel/int.rs:138-490, src/kernel/mixed.rs:31-400,
// src/kernel/float.rs:150-281) with one workgroup per BM x BN output tile.
//
// Data path (one workgroup = 4 or 8 waves of 64 lanes over one tile):
//   * K advances in stages of 64 bytes per row (64 i8, 32 bf16, 16 f32).  The
//     stage's A and B rows go global -> LDS with direct-to-LDS buffer loads
//     (buffer_load_dwordx4 ... lds: lane l of an instruction fills LDS bytes
//     base + 16*l), into a ring of NS stages, so no VGPRs stage the operands.
//     A 32-bit offset per lane (not a 64-bit address) halves the address
//     traffic of each load, and the resource's range check supplies the zero
//     padding of edge tiles and of the K tail.
//     Row r of a stage stores its chunk c (16 bytes) in slot c ^ swz(r), which
//     keeps the operand reads below free of LDS bank conflicts.
//   * Every MFMA operand is 16 bytes per lane: lane l reads row l%32 of a
//     32-row block, chunk 2*s + l/32 of sub-step s.  That is one
//     v_mfma_i32_32x32x32_i8 (16 i8), one v_mfma_f32_32x32x16_bf16 (8 bf16) or
//     four v_mfma_f32_32x32x2_f32 (1 f32 each) per 32x32 block.  A and B use
//     the same lane -> k mapping, so each instruction pairs A[i,k] with B[k,j]
//     whatever order the hardware sums its k values in.
//   * The main loop (see mma_kernel) keeps the matrix pipe fed: fragment
//     reads, the next stages' loads and the stage barrier are interleaved with
//     the MFMAs, and the next stage's first fragments are read while the
//     current stage's second half of MFMAs run.
// The 32x32 accumulator block lives in 16 registers per lane: register r of
// lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include <type_traits>

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

// The hardware hands consecutive workgroups (in x, then y, then z order) to
// the 8 XCDs round-robin.  This gives every XCD one contiguous range of
// logical ids instead: workgroup `bid` of `nblocks` -> logical id.
__device__ __forceinline__ int64_t xcd_logical(int64_t bid, int64_t nblocks) {
    const int64_t X = 8;
    const int64_t per = nblocks / X, rem = nblocks % X;
    const int64_t xcd = bid % X, idx = bid / X;
    return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

// Logical tile id -> (tile_m, tile_n).  The grouped order makes each XCD's
// contiguous range a compact block of tiles, so the A rows and B columns it
// needs stay in that XCD's L2.
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int G = 8;
    int in_group = G * tiles_n;
    int group = pid / in_group;
    int first_m = group * G;
    int gsize = tiles_m - first_m < G ? tiles_m - first_m : G;
    int r = pid % in_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;
constexpr int kSchedVmem = 0x010;

// Operand loads go through buffer resources (base + 32-bit per-lane offset,
// range-checked by the address unit): a lane whose offset is at or past the
// resource's size reads zeros and touches no memory.  That zero-fills the rows
// past the matrix edge and the K tail of the last stage, and lets the loop
// issue its loads past the end of K without traffic.  Offsets stay below
// kMaxRecords (internal.h), which the host guarantees for every row a tile
// addresses.
constexpr int kRsrcWord3 = 0x00020000;  // raw (unswizzled) buffer, 32-bit data format

// One direct-to-LDS load of 16 bytes per lane: lane l reads base[voff] into
// LDS bytes lds + 16*l (zeros when voff >= num).
__device__ __forceinline__ void dma16(const uint8_t *base, uint32_t num, uint32_t voff,
                                      uint8_t *lds) {
    __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)num, kRsrcWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                             voff, 0, 0, 0);
}

// The same with a wave-uniform byte offset `soff` added in the scalar operand:
// no per-lane address arithmetic.  The range check may leave `soff` out, so
// the caller guarantees that every lane with voff < num stays inside the
// resource with soff added, and that lanes meant to read zeros have
// voff >= num.
__device__ __forceinline__ void dma16s(const uint8_t *base, uint32_t num, uint32_t voff,
                                       uint32_t soff, uint8_t *lds) {
    __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)num, kRsrcWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                             voff, (int)soff, 0, 0);
}

// A sub-step's memory operations in program order: NR fragment reads with NL
// direct-to-LDS loads spread among them (a load after read r when
// (r+1)*NL/NR > r*NL/NR).  The compiler cannot tell a load's LDS destination
// from the reads' sources, so it keeps the two in program order; writing them
// interleaved is what lets the schedule below interleave them.
template <int NR, int NL>
__device__ constexpr bool op_is_load(int o) {
    int pos = 0;
    for (int r = 0; r < NR; ++r) {
        if (pos++ == o) return false;
        if ((r + 1) * NL / NR != r * NL / NR && pos++ == o) return true;
    }
    return false;
}

// Schedule of one sub-step: NM MFMAs with the NR + NL operations above spread
// over the first SPAN of them (the reads feed the next sub-step, so they go
// out early).
template <int NM, int NR, int NL, int SPAN>
__device__ __forceinline__ void sched_ops() {
    constexpr int NOPS = NR + NL;
#pragma unroll
    for (int i = 0; i < NM; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
#pragma unroll
        for (int o = 0; o < NOPS; ++o) {
            if (o * SPAN / NOPS == i) {
                if (op_is_load<NR, NL>(o))
                    __builtin_amdgcn_sched_group_barrier(kSchedVmem, 1, 0);
                else
                    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
            }
        }
    }
}

// A stage holds BK bytes of K for every A and B row of the tile: row r at
// r*BK, chunk c (16 bytes) in slot c ^ swz(r).  An operand read is 16 lanes
// per LDS cycle (64 banks of 4 bytes) reading the same chunk of 16 consecutive
// rows; the swizzle spreads them over 16 distinct 16-byte bank groups.  For
// BK = 64 (4 chunks per row) rows r and r+4 share bank groups unless their
// slots differ, hence swz = (r >> 2) & 3; for BK = 128, swz = (r >> 1) & 7.
template <int BK>
__device__ __forceinline__ int swz_of(int row) {
    return BK == 64 ? ((row >> 2) & 3) : ((row >> 1) & 7);
}

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding: vmcnt low bits [3:0] and high
// bits [15:14], expcnt [6:4] left at 7, lgkmcnt [11:8] = 0).  lgkmcnt(0) also
// retires this wave's LDS reads of the slot the next loads will overwrite.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x70);
}

// Workgroup barrier for the stage ring.  The caller has already waited for
// this wave's loads of the stage and for its LDS reads (wait_vmcnt), so every
// wave passing the barrier means the stage is complete in LDS.  A fence here
// (even an LDS-only one) would make the compiler drain every direct-to-LDS
// load in flight, i.e. the later stages too; the memory clobber alone keeps
// the compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void stage_barrier() {
    asm volatile("s_barrier" ::: "memory");
}

// Kernel: one workgroup of 4 waves (2 x 2) per BM x BN tile of C.
//   BK  K bytes per stage (64), NS stages in the LDS ring.
// Main loop per stage kt:
//   wait for this wave's loads of stage kt, barrier (every wave's landed);
//   issue the direct-to-LDS loads of stage kt+NS-1 into the slot stage kt-1
//   used (every wave finished reading it before the barrier);
//   MFMAs over stage kt, reading each sub-step's fragments while the previous
//   sub-step's MFMAs run.
// Epilogue: each wave stages 32 accumulator rows at a time through LDS and
// writes them back as row-contiguous 4-element chunks (16-byte stores for
// i32/f32 output).
// Register budget: the waves of as many workgroups as the 160 KiB of LDS
// holds (at most two), spread over the CU's 4 SIMDs.
template <int BM, int BN, int WM, int WN, int BK, int NS>
constexpr int waves_per_simd() {
    constexpr int smem = NS * (BM + BN) * BK;
    constexpr int wgs = smem * 2 <= 160 * 1024 ? 2 : 1;
    return wgs * WM * WN / 4 > 1 ? wgs * WM * WN / 4 : 1;
}

template <InType T, EpiKind E, int BM, int BN, int WM, int WN, int BK, int NS, bool SPLIT>
__global__ __launch_bounds__(WM * WN * 64)
__attribute__((amdgpu_waves_per_eu(waves_per_simd<BM, BN, WM, WN, BK, NS>(),
                                   waves_per_simd<BM, BN, WM, WN, BK, NS>())))
void mma_kernel(const MmaArgs args, const EpiParams ep) {
    constexpr int NWAVES = WM * WN;
    // Strip tiles (STRIP: 256 x 352 on 2 x 4 waves): the wave grid covers the
    // first BNM columns, BN/WN rounded down to whole 32-column blocks, and
    // the SW columns past them form a strip of TS blocks per 32-row block.
    // Wave (wm, wn) also computes the strip's row block wm*WTM + wn*32, one
    // of its own, so every wave runs TM*TN + TS MFMAs per sub-step (11:
    // balanced where the 11 column blocks of 352 columns cannot be split
    // over 4 wave columns) and reads no extra A rows.
    constexpr int SW = BN % (WN * 32);
    constexpr bool STRIP = SW > 0;
    constexpr int BNM = BN - SW;
    constexpr int WTM = BM / WM, WTN = BNM / WN;
    constexpr int TM = WTM / 32, TN = WTN / 32, TS = SW / 32;
    static_assert(!STRIP || (SW % 32 == 0 && TM == WN && WM * WN * 32 == BM), "strip layout");
    constexpr int STAGE = (BM + BN) * BK;
    constexpr int A_BYTES = BM * BK;
    constexpr int NI = STAGE / 1024;      // direct-to-LDS instructions per stage
    // ... per wave; when NI is not a multiple of the waves (RAGGED: the strip
    // tile's 76), only the first NLAST waves have a real last instruction and
    // the others issue it with every lane out of range into a spare 1 KiB.
    constexpr int NIW = (NI + NWAVES - 1) / NWAVES;
    constexpr int NLAST = NI - (NIW - 1) * NWAVES;
    constexpr bool RAGGED = NLAST != NWAVES;
    constexpr int RPI = 1024 / BK;        // stage rows one instruction fills
    constexpr int CPR = BK / 16;          // 16-byte chunks per stage row
    constexpr int SUB = BK / 32;          // MFMA sub-steps per stage
    constexpr int EPI_W = WTN > SW ? WTN : SW;  // widest staged row (columns)
    constexpr int EPI_LD = EPI_W + 4;     // staged-epilogue row stride (4-byte words)
    constexpr int SMEM = NS * STAGE;
    static_assert((NI % NWAVES == 0 || STRIP) && TM >= 1 && TN >= 1, "tile too small");
    static_assert(NWAVES * 32 * EPI_LD * 4 <= SMEM, "epilogue staging does not fit");
    using M = Mma<T>;
    using acc_t = typename M::acc_t;
    using val_t = typename M::scalar_t;

    // One LDS object for everything (the stage ring, then the requantization
    // channels): with a second __shared__ array the compiler can no longer
    // tell the operand reads from the direct-to-LDS loads in flight and
    // drains every load (vmcnt(0)) before each stage's fragment reads.
    // When the ring fills the CU's 160 KiB (256 x 384 tiles: two 80 KiB
    // stages), the channels are staged after the main loop instead, at the
    // ring's end, past the epilogue's staging rows (Q_LATE).
    constexpr int QCH = (E == EpiKind::Q8) ? (BM > BN ? BM : BN) : 1;
    constexpr int QBYTES = (E == EpiKind::Q8) ? QCH * 8 : 0;
    constexpr bool Q_LATE = SMEM + QBYTES > 160 * 1024;
    static_assert(!Q_LATE || NWAVES * 32 * EPI_LD * 4 + QBYTES <= SMEM,
                  "late channel staging overlaps the epilogue's rows");
    constexpr int SPARE = Q_LATE ? SMEM : SMEM + QBYTES;  // RAGGED: the dummy loads' target
    __shared__ __attribute__((aligned(1024))) uint8_t smem[SPARE + (RAGGED ? 1024 : 0)];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps load setup scalar
    const int wm = wave / WN, wn = wave % WN;

    const int tiles_m = (args.M + BM - 1) / BM;
    const int PN = args.pn > 0 ? args.pn : BN;  // column pitch (<= BN)
    const int tiles_n = (args.N + PN - 1) / PN;
    // Batch element zb, output slab z.  A batched launch remaps (tile, element)
    // pairs as one range, so the few tiles of an element share an XCD (and its
    // L2 copy of the element's operands).  SPLIT: K range blockIdx.y, and each
    // range's partial sums go to a slab of their own, z = zb * splits + range
    // (the epilogue's batch stride), to be reduced in range order afterwards.
    // The unsplit kernels are separate instantiations, so their code is
    // untouched by this.  Which workgroup computes a tile does not change its
    // arithmetic.
    int64_t zb = blockIdx.z;
    int tid_logical;
    if (!SPLIT && gridDim.z > 1) {
        const int64_t pid = xcd_logical((int64_t)blockIdx.z * gridDim.x + blockIdx.x,
                                        (int64_t)gridDim.x * gridDim.z);
        zb = pid / gridDim.x;
        tid_logical = (int)(pid % gridDim.x);
    } else {
        tid_logical = (int)xcd_logical(blockIdx.x, gridDim.x);
    }
    int tmi, tni;
    tile_coords(tid_logical, tiles_m, tiles_n, tmi, tni);
    const int m0 = tmi * BM, n0 = tni * PN;
    const int n_end = args.N - n0 < PN ? args.N : n0 + PN;  // columns this tile stores
    int64_t z = zb, k0 = 0, kel = args.K;
    if constexpr (SPLIT) {
        z = zb * args.splits + blockIdx.y;
        k0 = (int64_t)blockIdx.y * args.kchunk;
        kel = args.K - k0 < args.kchunk ? args.K - k0 : args.kchunk;
    }

    const int esz = (T == InType::I8) ? 1 : (T == InType::BF16 ? 2 : 4);
    const int64_t kbytes = kel * esz;
    const int64_t lda_b = args.lda * esz, ldb_b = args.ldb * esz;
    const uint8_t *A = (const uint8_t *)args.a + (zb * args.bsa + k0) * esz;
    const uint8_t *B = (const uint8_t *)args.b + (zb * args.bsb + k0) * esz;
    const int KT = (int)((kbytes + BK - 1) / BK);
    const bool k_whole = (kbytes % BK) == 0;

    // The tile's A rows [m0, m0+BM) and B rows [n0, n0+PN) as two buffer
    // resources spanning the valid rows' bytes (rows may overlap: a stride
    // below the row length is a legal view).  Rows past the matrix edge (and
    // B rows past the column pitch, whose outputs the next tile stores) start
    // outside them and read zeros, or, with overlapping rows, feed outputs
    // that are never stored.
    const int64_t kb16 = (kbytes + 15) / 16 * 16;
    const uint8_t *a_pan = A + (int64_t)m0 * lda_b;
    const uint8_t *b_pan = B + (int64_t)n0 * ldb_b;
    const uint32_t a_num = (uint32_t)(((args.M - m0 < BM ? args.M - m0 : BM) - 1) * lda_b + kb16);
    const uint32_t b_num = (uint32_t)(((args.N - n0 < PN ? args.N - n0 : PN) - 1) * ldb_b + kb16);

    // This lane's source chunk for each of the wave's NIW load instructions:
    // instruction q fills stage bytes [q*1024, q*1024 + 1024), lane l the 16
    // bytes at +16*l, i.e. stage row q*RPI + l/CPR, slot l%CPR, which holds
    // chunk (l%CPR) ^ swz(row).  Each instruction covers RPI whole rows, all
    // of A or all of B (BM is a multiple of RPI), so from_a is wave-uniform.
    // When all of a wave's rows come from one operand (WAVE_OP: every tile
    // here but 256x128), instruction i's rows lie RPI*i rows below
    // instruction 0's and its chunk differs only through the swizzle, which
    // repeats every NPAT instructions; the offsets are then formed per load
    // from NPAT bases (fewer live registers), else kept per instruction.
    // Otherwise, for 128-byte stages whose A rows fill whole rounds of the
    // waves (STRIDED: the 128 x 96, 128 x 192 and 256 x 384 tiles), the
    // wave's instruction i is instruction q = i*NWAVES + wave: instructions
    // [0, IA) take A rows, the rest B rows, each NWAVES*RPI rows (a multiple
    // of 32, so the same swizzle pattern) below the one before, and two base
    // offsets serve them all.
    constexpr bool WAVE_OP = (BM % (NIW * RPI)) == 0;
    constexpr bool STRIDED = !WAVE_OP && BK == 128 && BM % (NWAVES * RPI) == 0;
    constexpr int IA = BM / (NWAVES * RPI);
    static_assert(!STRIDED || (NWAVES * RPI) % 32 == 0, "strided rows must keep the swizzle");
    constexpr int NPAT = BK == 128 ? 2 : 1;
    constexpr int NOFF = WAVE_OP ? NPAT : (STRIDED ? 2 : NIW);
    auto q_of = [&](int i) { return STRIDED ? i * NWAVES + wave : wave * NIW + i; };
    uint32_t voff[NOFF];
    int kch[NOFF];
    bool from_a[NOFF];
#pragma unroll
    for (int i = 0; i < NOFF; ++i) {
        const int q = q_of(STRIDED ? i * IA : i);
        const int row = q * RPI + lane / CPR;
        const int ch = (lane % CPR) ^ swz_of<BK>(row);
        kch[i] = ch * 16;
        from_a[i] = q * RPI < BM;
        voff[i] = from_a[i] ? (uint32_t)(row * lda_b + ch * 16)
                            : (uint32_t)((row - BM) * ldb_b + ch * 16);
    }
    const uint32_t rstep = (uint32_t)(RPI * (from_a[0] ? lda_b : ldb_b));
    const uint32_t sstep_a = (uint32_t)(NWAVES * RPI * lda_b);
    const uint32_t sstep_b = (uint32_t)(NWAVES * RPI * ldb_b);
    // RAGGED: this wave's last instruction is a dummy (every lane out of
    // range, into the spare 1 KiB), so all waves issue NIW loads per stage
    // and wait for the same counts.
    const bool dummy_last = RAGGED && wave >= NLAST;
    auto is_dummy = [&](int i) { return RAGGED && i == NIW - 1 && dummy_last; };
    auto lane_off = [&](int i) -> uint32_t {
        if (is_dummy(i)) return kOutOfRange;
        if constexpr (WAVE_OP)
            return voff[i % NPAT] + (uint32_t)(i - i % NPAT) * rstep;
        else if constexpr (STRIDED)
            return i < IA ? voff[0] + (uint32_t)i * sstep_a : voff[1] + (uint32_t)(i - IA) * sstep_b;
        else
            return voff[i];
    };
    auto lane_kch = [&](int i) { return kch[WAVE_OP ? i % NPAT : (STRIDED ? (i < IA ? 0 : 1) : i)]; };
    auto lane_from_a = [&](int i) {
        return WAVE_OP ? from_a[0] : (STRIDED ? i < IA : from_a[i]);
    };
    // LDS destination of the wave's instruction i in ring slot `slot`.
    auto dst_of = [&](int slot, int i) {
        return is_dummy(i) ? smem + SPARE : smem + slot * STAGE + q_of(i) * 1024;
    };
    // Loads of stage kt into ring slot `slot`.  Stages past the end of K load
    // nothing but zeros (every lane out of range), as do the chunks past K of
    // a partial last stage.
    auto issue_stage = [&](int kt, int slot, int first, int count) {
        const uint32_t kb = (uint32_t)kt * BK;
        const bool dead = kt >= KT;
        const bool tail = !k_whole && kt == KT - 1;
#pragma unroll
        for (int i = first; i < first + count; ++i) {
            uint32_t off = lane_off(i) + kb;
            if (dead || (tail && (int64_t)kb + lane_kch(i) >= kbytes) || is_dummy(i))
                off = kOutOfRange;
            dma16(lane_from_a(i) ? a_pan : b_pan, lane_from_a(i) ? a_num : b_num, off,
                  dst_of(slot, i));
        }
    };
    // Loads of a stage wholly inside K: the stage offset goes in the scalar
    // operand.  Allowed when rows do not overlap (row stride >= the row's
    // 16-byte-rounded length), so rows past the matrix edge start at or past
    // their resource's end and read zeros whatever the offset, and the valid
    // rows' bytes of a whole stage lie inside the resource.  When every wave's
    // rows come from one operand (the tiles here but 256x128), the wave keeps
    // one resource.
    const bool w_from_a = wave * NIW * RPI < BM;
    const uint8_t *const w_pan = w_from_a ? a_pan : b_pan;
    const uint32_t w_num = w_from_a ? a_num : b_num;
    const bool soff_ok = lda_b >= kb16 && ldb_b >= kb16;
    auto issue_whole = [&](int kt, int slot, int first, int count) {
        const uint32_t kb = (uint32_t)kt * BK;
#pragma unroll
        for (int i = first; i < first + count; ++i) {
            if constexpr (WAVE_OP)
                dma16s(w_pan, w_num, lane_off(i), kb, dst_of(slot, i));
            else
                dma16s(lane_from_a(i) ? a_pan : b_pan, lane_from_a(i) ? a_num : b_num,
                       lane_off(i), kb, dst_of(slot, i));
        }
    };

    constexpr int TSA = STRIP ? TS : 1;
    acc_t acc[TM][TN], accs[TSA];  // accs: the strip's blocks (STRIP)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = acc_t{};
#pragma unroll
    for (int t = 0; t < TSA; ++t) accs[t] = acc_t{};

    // The wave's row block i is block rb(i) of its WTM rows: i itself, or,
    // for strip tiles, rotated by wn, so that block 0 is the wave's strip
    // row block.
    auto rb = [&](int i) { return STRIP ? (i + wn) % TM : i; };
    const int lrow = lane & 31, lhalf = lane >> 5;
    int a_row_off[TM], b_row_off[TN], s_row_off[TSA];
#pragma unroll
    for (int i = 0; i < TM; ++i) a_row_off[i] = (wm * WTM + rb(i) * 32 + lrow) * BK;
#pragma unroll
    for (int j = 0; j < TN; ++j) b_row_off[j] = A_BYTES + (wn * WTN + j * 32 + lrow) * BK;
#pragma unroll
    for (int t = 0; t < TSA; ++t) s_row_off[t] = A_BYTES + (BNM + t * 32 + lrow) * BK;
    const int swz = swz_of<BK>(lrow);  // operand block bases are multiples of 32 rows

    // ASINGLE: see the 128-byte two-stage loop.
    constexpr bool ASINGLE = BK == 128 && NS == 2 && NWAVES == 8 && (TM * TN >= 12 || STRIP);
    static_assert(!STRIP || ASINGLE, "strip tiles run the single-A loop");
    v4i af[SUB][TM], bf[SUB][TN], sf[TSA];  // sf: the strip's B fragments, single set
    auto read_frags = [&](const uint8_t *s, int ss, int set) {
        const int slot = ((2 * ss + lhalf) ^ swz) << 4;
#pragma unroll
        for (int i = 0; i < TM; ++i) af[set][i] = *(const v4i *)(s + a_row_off[i] + slot);
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[set][j] = *(const v4i *)(s + b_row_off[j] + slot);
        if constexpr (STRIP) {
#pragma unroll
            for (int t = 0; t < TS; ++t) sf[t] = *(const v4i *)(s + s_row_off[t] + slot);
        }
    };
    auto mfmas = [&](int set) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = M::step(bf[set][j], af[set][i], acc[i][j]);
    };

    // Every iteration issues exactly one stage of loads: past the end of K they
    // are out-of-range loads (zeros into a slot nothing reads again, no memory
    // traffic), which keeps the loop body straight-line code and makes the
    // wait count a constant.  The full barrier before the epilogue drains them.
    //
    // Lookahead: stage kt+1 is certified complete (wait + barrier) half way
    // through stage kt, so its first fragments are read under stage kt's
    // second half of MFMAs and no LDS latency is exposed at a stage boundary.
    //   phase A: stage kt sub-step 0 MFMAs (fragments F0), with sub-step 1's
    //            fragment reads (F1) and half of the loads of stage kt+NS-1 --
    //            into the slot of stage kt-1, finished by every wave before the
    //            previous barrier -- spread between them;
    //   barrier: this wave's loads of stage kt+1 landed and its LDS reads
    //            retired, then s_barrier;
    //   phase C: sub-step 1 MFMAs (F1), with stage kt+1's sub-step 0 reads
    //            (into F0) and the other half of the loads spread between them.
    // Splitting the loads over both phases keeps the CU's address unit (one
    // 1 KiB load takes it ~16 cycles, and four waves share it) from backing up
    // into the waves' instruction issue.
    // The empty asm statements pin F0 and F1 around the barrier so the compiler
    // keeps each phase's MFMAs on its side.
    constexpr int H0 = NIW / 2, H1 = NIW - H0;  // loads issued in phase A / C
    // 128-byte stages: a stage's loads in three parts, after the barrier that
    // frees its slot (P0) and under the next two sub-steps (P1, P2).  (Four
    // parts, one per sub-step, measured slower: the last part then has too
    // little time to land.)
    constexpr int P0 = (NIW + 2) / 3, P1 = (NIW - P0 + 1) / 2, P2 = NIW - P0 - P1;

    // Requantization: the tile's channels (rows for a per-row map, columns
    // for a per-column one) get their scale and bias staged in LDS, so the
    // epilogue reads them without global loads.  They are loaded here, stay
    // in flight behind the prologue's stage loads (loads complete in order),
    // and reach LDS after the prologue wait; the main loop's barriers publish
    // them.
    constexpr int QPT = (QCH + NWAVES * 64 - 1) / (NWAVES * 64);  // channels per thread
    float *const q_scale = (float *)(smem + (Q_LATE ? SMEM - QBYTES : SMEM));
    int32_t *const q_bias = (int32_t *)(smem + (Q_LATE ? SMEM - QBYTES : SMEM) + QCH * 4);
    int q_ch0 = 0, q_n = 0;
    float q_s[QPT] = {};
    int32_t q_b[QPT] = {};
    if constexpr (E == EpiKind::Q8) {
        q_n = ep.axis ? BN : BM;
        q_ch0 = ep.axis ? n0 : m0;
        const int lim = ep.axis ? args.N : args.M;
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
            const int c = tid + u * NWAVES * 64, ch = q_ch0 + c;
            if (c < q_n) {
                q_s[u] = ep.scales ? (ch < lim ? ep.scales[ch] : 1.0f) : ep.scale;
                q_b[u] = (ep.bias && ch < lim) ? ep.bias[ch] : 0;
            }
        }
    }

    if constexpr (SUB == 2) {
#pragma unroll
        for (int s0 = 0; s0 < NS - 1; ++s0) issue_stage(s0, s0, 0, NIW);
        wait_vmcnt<(NS - 2) * NIW>();
    } else if constexpr (NS == 2) {
        // Stage 0 whole, and the first part of stage 1 (the main loop issues
        // the rest of each stage, and the first part of the one after it).
        issue_stage(0, 0, 0, NIW);
        issue_stage(1, 1, 0, P0);
        wait_vmcnt<P0>();
    } else {
        // Three-stage ring: stages 0 and 1 whole, the first part of stage 2.
        issue_stage(0, 0, 0, NIW);
        issue_stage(1, 1, 0, NIW);
        issue_stage(2, 2, 0, P0);
        wait_vmcnt<NIW + P0>();
    }
    auto stage_channels = [&]() {
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
            const int c = tid + u * NWAVES * 64;
            if (c < q_n) {
                q_scale[c] = q_s[u];
                q_bias[c] = q_b[u];
            }
        }
    };
    if constexpr (E == EpiKind::Q8 && !Q_LATE) stage_channels();
    stage_barrier();
    read_frags(smem, 0, 0);

    // Fragment reads of sub-step ss into `set`, with loads [first, first + NL)
    // of stage st into `slot` among them in program order (op_is_load); whole
    // stages take the scalar-offset loads.
    constexpr int NM = TM * TN, NR = TM + TN;
    constexpr int SPAN = NM * 7 / 8;
    auto ops = [&](auto whole, const uint8_t *src, int ss, int set, auto nl, int st, int slot,
                   int first) {
        constexpr bool WHOLE = decltype(whole)::value;
        constexpr int NL = decltype(nl)::value;
        const int sl = ((2 * ss + lhalf) ^ swz) << 4;
        int l = first;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            if (r < TM)
                af[set][r] = *(const v4i *)(src + a_row_off[r] + sl);
            else
                bf[set][r - TM] = *(const v4i *)(src + b_row_off[r - TM] + sl);
            if ((r + 1) * NL / NR != r * NL / NR) {
                if constexpr (WHOLE)
                    issue_whole(st, slot, l, 1);
                else
                    issue_stage(st, slot, l, 1);
                ++l;
            }
        }
    };
    const int ktw = (int)(kbytes / BK);  // whole stages

    if constexpr (SUB == 2) {
        using LA = std::integral_constant<int, H0>;
        using LC = std::integral_constant<int, H1>;
        auto kstep = [&](int kt, auto whole) {
            const uint8_t *s = smem + (kt % NS) * STAGE;
            const int nslot = (kt + NS - 1) % NS;
            mfmas(0);
            ops(whole, s, 1, 1, LA{}, kt + NS - 1, nslot, 0);
            sched_ops<NM, NR, H0, SPAN>();
#pragma unroll
            for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[0][i]));
#pragma unroll
            for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bf[0][j]));
            // Stage kt+1's loads were issued at iteration kt+2-NS; issued after
            // them: NS-3 whole iterations plus this phase A.
            wait_vmcnt<(NS - 3) * NIW + H0>();
            stage_barrier();
#pragma unroll
            for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[1][i]));
#pragma unroll
            for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bf[1][j]));
            mfmas(1);
            ops(whole, smem + ((kt + 1) % NS) * STAGE, 0, 0, LC{}, kt + NS - 1, nslot, H0);
            sched_ops<NM, NR, H1, SPAN>();
        };
        // Iteration kt issues stage kt+NS-1.
        const int lim = ktw - NS + 1;
        const int kt_whole = soff_ok ? (lim < KT ? (lim > 0 ? lim : 0) : KT) : 0;
        int kt = 0;
        for (; kt < kt_whole; ++kt) kstep(kt, std::true_type{});
        for (; kt < KT; ++kt) kstep(kt, std::false_type{});
    } else {
        // 128-byte stages in a two-stage ring: each row of a stage is one
        // whole 128-byte line of K (half the cache-line requests of two
        // 64-byte stages) and one barrier covers four sub-steps.  Stage kt+2's
        // loads go into stage kt's slot from the barrier at the end of stage
        // kt on (every wave has finished reading the slot): a third under
        // stage kt's last sub-step, the rest under stage kt+1's first two, so
        // the CU's address unit (one 1 KiB load takes it ~16 cycles) is never
        // asked for more than three quarters of a sub-step and each load has
        // at least a sub-step to land.  Stage kt+1's first fragments are read
        // under stage kt's last MFMAs.  Each sub-step's fragment reads and
        // loads are written interleaved (op_is_load) and scheduled one per
        // MFMA (sched_ops).  Iterations whose loads all fall on whole stages
        // take the stage offset in the loads' scalar operand and skip the
        // per-lane tail checks.
        static_assert(SUB == 4 && (NS == 2 || NS == 3), "four sub-steps run with a 2- or 3-stage ring");
        if constexpr (NS == 3) {
            // Three-stage ring (the tiles small enough for three 128-byte
            // stages in LDS): the same per-sub-step spread of the loads, but
            // for the stage after next, into the slot of the stage before
            // this one (free from the barrier that ended it), so every load
            // has a whole stage more to land: iteration kt issues the rest
            // of stage kt+2 and the first part of stage kt+3, and waits for
            // stage kt+1 with stage kt+2's loads still in flight.
            auto kstep3 = [&](int kt, auto whole) {
                using L0 = std::integral_constant<int, P0>;
                using L1 = std::integral_constant<int, P1>;
                using L2 = std::integral_constant<int, P2>;
                using LN = std::integral_constant<int, 0>;
                const uint8_t *s = smem + (kt % 3) * STAGE;
                const int lslot = (kt + 2) % 3;
                mfmas(0);
                ops(whole, s, 1, 1, L1{}, kt + 2, lslot, P0);
                sched_ops<NM, NR, P1, SPAN>();
                mfmas(1);
                ops(whole, s, 2, 0, L2{}, kt + 2, lslot, P0 + P1);
                sched_ops<NM, NR, P2, SPAN>();
                mfmas(0);
                ops(whole, s, 3, 1, LN{}, kt + 2, lslot, NIW);
                sched_ops<NM, NR, 0, SPAN>();
#pragma unroll
                for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[0][i]));
#pragma unroll
                for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bf[0][j]));
                wait_vmcnt<NIW>();
                stage_barrier();
#pragma unroll
                for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[1][i]));
#pragma unroll
                for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bf[1][j]));
                mfmas(1);
                ops(whole, smem + ((kt + 1) % 3) * STAGE, 0, 0, L0{}, kt + 3, kt % 3, 0);
                sched_ops<NM, NR, P0, SPAN>();
            };
            // Iteration kt issues stages kt+2 and kt+3.
            const int kt_whole = soff_ok ? (ktw - 3 < KT ? (ktw - 3 > 0 ? ktw - 3 : 0) : KT) : 0;
            int kt = 0;
            for (; kt < kt_whole; ++kt) kstep3(kt, std::true_type{});
            for (; kt < KT; ++kt) kstep3(kt, std::false_type{});
        } else if constexpr (ASINGLE) {
        // Register-tight tiles (256 x 384 on eight waves: 192 accumulator
        // registers of the 256 a wave has at two waves per SIMD): one set of
        // A fragments.  Each sub-step reads the next sub-step's B fragments
        // under its first row of MFMAs and each next A fragment right after
        // the last MFMA of its row, into the registers that row used, so only
        // the B fragments are double-buffered.  The loads spread over the
        // remaining MFMAs.
        // Strip tiles: row 0's MFMAs also run the strip's blocks (row 0 is the
        // wave's strip row block), each strip B fragment re-read right after
        // its MFMA (single set), all before row 0's A fragment is replaced.
        auto substep = [&](int set, auto whole, const uint8_t *src, int ss, int nset, auto nl,
                           int st, int slot, int first) {
            constexpr bool WHOLE = decltype(whole)::value;
            constexpr int NL = decltype(nl)::value;
            constexpr int NFIRST = TN + (STRIP ? TS : 0);  // row 0's MFMAs
            constexpr int NREST = NM - TN;                 // the loads spread over these
            const int sl = ((2 * ss + lhalf) ^ swz) << 4;
            int l = first;
            auto load_after = [&](int m) {  // m: MFMA index past row 0
                if (m >= 0 && (m + 1) * NL / NREST != m * NL / NREST) {
                    if constexpr (WHOLE)
                        issue_whole(st, slot, l, 1);
                    else
                        issue_stage(st, slot, l, 1);
                    ++l;
                }
            };
#pragma unroll
            for (int i = 0; i < TM; ++i) {
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    acc[i][j] = M::step(bf[set][j], af[0][i], acc[i][j]);
                    if (i == 0) bf[nset][j] = *(const v4i *)(src + b_row_off[j] + sl);
                    load_after(i * TN + j - TN);
                }
                if constexpr (STRIP) {
                    if (i == 0) {
#pragma unroll
                        for (int t = 0; t < TS; ++t) {
                            accs[t] = M::step(sf[t], af[0][0], accs[t]);
                            sf[t] = *(const v4i *)(src + s_row_off[t] + sl);
                        }
                    }
                }
                af[0][i] = *(const v4i *)(src + a_row_off[i] + sl);
            }
            (void)NFIRST;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
                    if (i == 0) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
                    const int m = i * TN + j - TN;
                    if (m >= 0 && (m + 1) * NL / NREST != m * NL / NREST)
                        __builtin_amdgcn_sched_group_barrier(kSchedVmem, 1, 0);
                }
                if (STRIP && i == 0) {
#pragma unroll
                    for (int t = 0; t < TS; ++t) {
                        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
                    }
                }
                __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
            }
        };
        auto kstep = [&](int kt, auto whole) {
            using L0 = std::integral_constant<int, P0>;
            using L1 = std::integral_constant<int, P1>;
            using L2 = std::integral_constant<int, P2>;
            using LN = std::integral_constant<int, 0>;
            const uint8_t *s = smem + (kt & 1) * STAGE;
            const int nslot = (kt + 1) & 1;
            substep(0, whole, s, 1, 1, L1{}, kt + 1, nslot, P0);
            substep(1, whole, s, 2, 0, L2{}, kt + 1, nslot, P0 + P1);
            substep(0, whole, s, 3, 1, LN{}, kt + 1, nslot, NIW);
#pragma unroll
            for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bf[0][j]));
            wait_vmcnt<0>();
            stage_barrier();
#pragma unroll
            for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[0][i]));
#pragma unroll
            for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bf[1][j]));
            if constexpr (STRIP) {
#pragma unroll
                for (int t = 0; t < TS; ++t) asm volatile("" : "+v"(sf[t]));
            }
            substep(1, whole, smem + nslot * STAGE, 0, 0, L0{}, kt + 2, kt & 1, 0);
        };
        const int kt_whole = soff_ok ? (ktw - 2 < KT ? (ktw - 2 > 0 ? ktw - 2 : 0) : KT) : 0;
        int kt = 0;
        for (; kt < kt_whole; ++kt) kstep(kt, std::true_type{});
        for (; kt < KT; ++kt) kstep(kt, std::false_type{});
        } else {
        auto kstep = [&](int kt, auto whole) {
            using L0 = std::integral_constant<int, P0>;
            using L1 = std::integral_constant<int, P1>;
            using L2 = std::integral_constant<int, P2>;
            using LN = std::integral_constant<int, 0>;
            const uint8_t *s = smem + (kt & 1) * STAGE;
            const int nslot = (kt + 1) & 1;
            mfmas(0);
            ops(whole, s, 1, 1, L1{}, kt + 1, nslot, P0);
            sched_ops<NM, NR, P1, SPAN>();
            mfmas(1);
            ops(whole, s, 2, 0, L2{}, kt + 1, nslot, P0 + P1);
            sched_ops<NM, NR, P2, SPAN>();
            mfmas(0);
            ops(whole, s, 3, 1, LN{}, kt + 1, nslot, NIW);
            sched_ops<NM, NR, 0, SPAN>();
#pragma unroll
            for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[0][i]));
#pragma unroll
            for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bf[0][j]));
            wait_vmcnt<0>();
            stage_barrier();
#pragma unroll
            for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[1][i]));
#pragma unroll
            for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bf[1][j]));
            mfmas(1);
            ops(whole, smem + nslot * STAGE, 0, 0, L0{}, kt + 2, kt & 1, 0);
            sched_ops<NM, NR, P0, SPAN>();
        };
        // Iteration kt issues stages kt+1 and kt+2.
        const int kt_whole = soff_ok ? (ktw - 2 < KT ? (ktw - 2 > 0 ? ktw - 2 : 0) : KT) : 0;
        int kt = 0;
        for (; kt < kt_whole; ++kt) kstep(kt, std::true_type{});
        for (; kt < KT; ++kt) kstep(kt, std::false_type{});
        }
    }

    // Staged epilogue.  The MFMAs take B^T's fragment as their first operand,
    // so a 32x32 accumulator block holds C^T: register 4g+e of lane l is C row
    // l%32, column 8g + 4*(l/32) + e, i.e. four consecutive columns per lane
    // and group.  Each 32-row block goes to LDS as 16-byte writes (the ring is
    // free now; 32 rows x EPI_LD words per wave, EPI_LD = 4 mod 64 words so the
    // writes and the row reads below are conflict-free) and comes back as rows:
    // one row per CPRE lanes, whole 16-byte chunks, so the global stores write
    // full contiguous rows (storing the registers directly would write 32-byte
    // pieces of 32 rows per instruction, which the memory system handles at a
    // fraction of the rate).  The barrier also retires the zero-fill loads past
    // the end of K.
    __syncthreads();
    if constexpr (E == EpiKind::Q8 && Q_LATE) {
        stage_channels();
        __syncthreads();
    }
    val_t *stg = (val_t *)smem + wave * 32 * EPI_LD;
    typedef val_t v4_t __attribute__((ext_vector_type(4)));
    constexpr bool FB = E == EpiKind::F32 || E == EpiKind::BF16;
    // Channels of this lane's 4 columns in a row of NB blocks starting at
    // tile column lc0 (fixed for the whole row loop when they are columns):
    // requantization scale and bias, and the fused per-column bias.
    auto channels = [&](auto nb_c, int lc0, float (&cs)[4], int32_t (&cb)[4], float (&cf)[4]) {
        constexpr int CPRE = decltype(nb_c)::value * 8;  // 4-column chunks per staged row
        if constexpr (E == EpiKind::Q8) {
            if (ep.axis) {
                const int ci = lc0 + (lane % CPRE) * 4;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    cs[e] = q_scale[ci + e];
                    cb[e] = q_bias[ci + e];
                }
            }
        }
        if constexpr (FB) {
            if (ep.fused && ep.axis) {
                const int c = n0 + lc0 + (lane % CPRE) * 4;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    cf[e] = c + e < args.N ? fused_bias<E == EpiKind::BF16>(ep, c + e) : 0.0f;
            }
        }
    };
    // One 32-row block of NB accumulator blocks (rows grow0.., tile columns
    // lc0..): staged, then stored as rows, CPRE lanes per row.
    auto store_rows = [&](auto nb_c, const auto &blk, int grow0, int lc0, const float (&cs)[4],
                          const int32_t (&cb)[4], const float (&cf)[4]) {
        constexpr int NB = decltype(nb_c)::value;
        constexpr int CPRE = NB * 8;           // 4-column chunks per staged row
        constexpr int RPIT = 64 / CPRE;        // rows per read iteration
        static_assert(CPRE <= 64 && NB * 32 <= EPI_W, "staged row too wide");
        // The requantizing and the bf16 (narrowing, fused) stores are long;
        // unrolling their row loop fully would make the block loop too large
        // to unroll, and the accumulator array would then be indexed at run
        // time (scratch memory).
        constexpr int IT_UNROLL =
            (E == EpiKind::Q8 || E == EpiKind::BF16) && 32 / RPIT > 4 ? 4 : 32 / RPIT;
        // Lanes past RPIT*CPRE idle in the row loop (96-column rows: 48 of 64).
        const bool lane_on = lane < RPIT * CPRE;
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const v4_t w = {(val_t)blk[j][4 * g], (val_t)blk[j][4 * g + 1],
                                (val_t)blk[j][4 * g + 2], (val_t)blk[j][4 * g + 3]};
                *(v4_t *)(stg + lrow * EPI_LD + j * 32 + 8 * g + 4 * lhalf) = w;
            }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes done
        __builtin_amdgcn_wave_barrier();
        const int gcol0 = n0 + lc0;
#pragma unroll IT_UNROLL
        for (int it = 0; it < 32 / RPIT; ++it) {
            const int row = it * RPIT + (lane_on ? lane / CPRE : 0);
            const int c4 = (lane % CPRE) * 4;
            v4_t v4 = *(const v4_t *)(stg + row * EPI_LD + c4);
            val_t v[4] = {v4[0], v4[1], v4[2], v4[3]};
            const int grow = grow0 + row;
            float s4[4] = {cs[0], cs[1], cs[2], cs[3]};
            int32_t b4[4] = {cb[0], cb[1], cb[2], cb[3]};
            if constexpr (E == EpiKind::Q8) {
                if (!ep.axis) {
                    const int ri = grow - q_ch0 < BM ? grow - q_ch0 : BM - 1;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        s4[e] = q_scale[ri];
                        b4[e] = q_bias[ri];
                    }
                }
            }
            float f4[4] = {cf[0], cf[1], cf[2], cf[3]};
            if constexpr (FB) {
                if (ep.fused && !ep.axis) {
                    const float f = grow < args.M ? fused_bias<E == EpiKind::BF16>(ep, grow) : 0.0f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) f4[e] = f;
                }
            }
            if (lane_on && grow < args.M && gcol0 + c4 < n_end)
                store4<E, val_t, StPol::Plain>(ep, z, grow, gcol0 + c4, n_end, v, s4, b4, f4);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    };
    float col_s[4] = {0, 0, 0, 0}, col_f[4] = {0, 0, 0, 0};
    int32_t col_b[4] = {0, 0, 0, 0};
    channels(std::integral_constant<int, TN>{}, wn * WTN, col_s, col_b, col_f);
#pragma unroll
    for (int i = 0; i < TM; ++i)
        store_rows(std::integral_constant<int, TN>{}, acc[i], m0 + wm * WTM + rb(i) * 32, wn * WTN,
                   col_s, col_b, col_f);
    if constexpr (STRIP) {
        float st_s[4] = {0, 0, 0, 0}, st_f[4] = {0, 0, 0, 0};
        int32_t st_b[4] = {0, 0, 0, 0};
        channels(std::integral_constant<int, TS>{}, BNM, st_s, st_b, st_f);
        store_rows(std::integral_constant<int, TS>{}, accs, m0 + wm * WTM + wn * 32, BNM, st_s,
                   st_b, st_f);
    }
}

template <InType T, EpiKind E, int BM, int BN, int WM, int WN, int NS, bool SPLIT = false,
          int BK = 64>
static hipError_t launch_one(const MmaArgs &args, const EpiParams &ep, hipStream_t stream) {
    const int pn = args.pn > 0 ? args.pn : BN;
    if (pn > BN || pn % 4 != 0) return hipErrorInvalidValue;
    const int esz = T == InType::I8 ? 1 : (T == InType::BF16 ? 2 : 4);
    if (!panels_fit(BM, BN, args.lda * esz, args.ldb * esz,
                    (int64_t)(SPLIT ? args.kchunk : args.K) * esz))
        return hipErrorInvalidValue;
    int tiles = ((args.M + BM - 1) / BM) * ((args.N + pn - 1) / pn);
    dim3 grid(tiles, SPLIT ? args.splits : 1, args.batch);
    hipLaunchKernelGGL((mma_kernel<T, E, BM, BN, WM, WN, BK, NS, SPLIT>), grid,
                       dim3(WM * WN * 64), 0, stream, args, ep);
    return hipGetLastError();
}

// A split K runs on the 64 x 64 tile only (the host's choice); the partial
// products are always the native accumulator type.
template <InType T, EpiKind E>
static hipError_t launch_tile(Tile tile, const MmaArgs &args, const EpiParams &ep,
                              hipStream_t stream) {
    if (args.splits > 1) {
        if constexpr (E == Mma<T>::native) {
            if (tile == Tile::T64x64) return launch_one<T, E, 64, 64, 2, 2, 4, true>(args, ep, stream);
        }
        return hipErrorInvalidValue;
    }
    switch (tile) {
    case Tile::T256x256: return launch_one<T, E, 256, 256, 2, 2, 4>(args, ep, stream);
    case Tile::T256x256w8: return launch_one<T, E, 256, 256, 2, 4, 4>(args, ep, stream);
    case Tile::T256x128: return launch_one<T, E, 256, 128, 2, 2, 4>(args, ep, stream);
    case Tile::T256x128o2: return launch_one<T, E, 256, 128, 2, 2, 3>(args, ep, stream);
    case Tile::T128x128: return launch_one<T, E, 128, 128, 2, 2, 4>(args, ep, stream);
    case Tile::T64x64: return launch_one<T, E, 64, 64, 2, 2, 4>(args, ep, stream);
    case Tile::T256x256k128: return launch_one<T, E, 256, 256, 2, 2, 2, false, 128>(args, ep, stream);
    case Tile::T256x256w8k128: return launch_one<T, E, 256, 256, 2, 4, 2, false, 128>(args, ep, stream);
    case Tile::T128x192k128: return launch_one<T, E, 128, 192, 2, 2, 3, false, 128>(args, ep, stream);
    case Tile::T128x96k128o2: return launch_one<T, E, 128, 96, 4, 1, 2, false, 128>(args, ep, stream);
    case Tile::T256x384w8k128: return launch_one<T, E, 256, 384, 2, 4, 2, false, 128>(args, ep, stream);
    case Tile::T256x352w8k128: return launch_one<T, E, 256, 352, 2, 4, 2, false, 128>(args, ep, stream);
    case Tile::T256x256w8m16: break;  // mma16.hip (launch_mma dispatches it first)
    case Tile::T256x352w8m16: break;  // mma16w.hip (likewise)
    }
    return hipErrorInvalidValue;
}

}  // namespace gk
