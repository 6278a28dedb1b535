// mma16.hip -- the 256 x 256 eight-wave tile on 16x16 matrix-core
// instructions (v_mfma_i32_16x16x64_i8, v_mfma_f32_16x16x32_bf16).
//
// Same data path as mma_kernel.h (direct-to-LDS loads of 128-byte stages into
// a swizzled ring -- here three A slots and two B slots, so a stage's A loads
// go out a stage earlier than its B loads --, fragment reads interleaved with
// the MFMAs, one barrier per stage, the staged epilogue), with 16x16 blocks: on this chip
// the 16x16 instructions draw less power per operation than the 32x32 ones,
// so under the same power limit the clock stays higher (int8 16x16x64:
// 4.29 POP/s sustained on back-to-back MFMAs at 2.14 GHz, against 3.5 POP/s
// at 1.74 GHz for 32x32x32).  This file is built with the accumulators in
// VGPRs (-mllvm -amdgpu-mfma-vgpr-form): with them in AGPRs the compiler
// moves every 16x16 accumulator between register files around each MFMA.
//
// Wave (wm, wn) of the 2 x 4 grid owns 128 rows x 64 columns: 8 x 4 blocks of
// 16 x 16, 128 accumulator registers.  A 64-byte sub-step feeds one MFMA per
// block: lane l reads row l%16 of a 16-row block, 16-byte chunk 4*s + l/16
// of sub-step s, for A and B alike, so each instruction pairs A[i,k] with
// B[k,j].  A 128-byte stage is two sub-steps, run as four phases of 16 MFMAs
// (rows 0-3, then 4-7 of the wave's blocks), which carry the same load and
// barrier schedule as the 32x32 tile's four sub-steps.  Accumulator block
// layout (B^T's fragment is the first operand): register r of lane l holds C
// row l%16, column 4*(l/16) + r of the block.
#include "mma_kernel.h"

namespace gk {

template <InType T>
struct Mma16x;

template <>
struct Mma16x<InType::I8> {
    using acc_t = v4i;
    using scalar_t = int32_t;
    __device__ __forceinline__ static acc_t step(v4i a, v4i b, acc_t c) {
        return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mma16x<InType::BF16> {
    using acc_t = v4f;
    using scalar_t = float;
    __device__ __forceinline__ static acc_t step(v4i a, v4i b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a),
                                                       __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
    }
};

template <InType T, EpiKind E>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mma16_kernel(const MmaArgs args, const EpiParams ep) {
    constexpr int BM = 256, BN = 256, WN = 4, BK = 128;
    constexpr int NWAVES = 8;
    constexpr int WTM = 128, WTN = 64;
    constexpr int TM = WTM / 16, TN = WTN / 16;  // 8 x 4 blocks of 16 x 16
    constexpr int ASTAGE = BM * BK, BSTAGE = BN * BK;  // 32 KiB each
    constexpr int NSA = 3, NSB = 2;              // A and B ring slots
    constexpr int B_BASE = NSA * ASTAGE;
    constexpr int LPW = ASTAGE / 1024 / NWAVES;  // loads per wave per operand per stage (4)
    constexpr int RPI = 1024 / BK;               // stage rows one instruction fills
    constexpr int CPR = BK / 16;                 // 16-byte chunks per stage row
    constexpr int EPI_LD = WTN + 4;              // staged-epilogue row stride (words)
    constexpr int SMEM = B_BASE + NSB * BSTAGE;  // 160 KiB, all of the CU's LDS
    constexpr int EPI_BYTES = NWAVES * 16 * EPI_LD * 4;
    static_assert(SMEM <= 160 * 1024, "LDS");
    using M = Mma16x<T>;
    using acc_t = typename M::acc_t;
    using val_t = typename M::scalar_t;
    constexpr int QCH = (E == EpiKind::Q8) ? BM : 1;
    static_assert(EPI_BYTES + QCH * 8 <= SMEM, "epilogue staging and channel table do not fit");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;

    const int tiles_m = (args.M + BM - 1) / BM;
    const int tiles_n = (args.N + BN - 1) / BN;
    int64_t zb = blockIdx.z;
    int tid_logical;
    if (gridDim.z > 1) {
        const int64_t pid = xcd_logical((int64_t)blockIdx.z * gridDim.x + blockIdx.x,
                                        (int64_t)gridDim.x * gridDim.z);
        zb = pid / gridDim.x;
        tid_logical = (int)(pid % gridDim.x);
    } else {
        tid_logical = (int)xcd_logical(blockIdx.x, gridDim.x);
    }
    int tmi, tni;
    tile_coords(tid_logical, tiles_m, tiles_n, tmi, tni);
    const int m0 = tmi * BM, n0 = tni * BN;
    const int n_end = args.N - n0 < BN ? args.N : n0 + BN;
    const int64_t z = zb;

    const int esz = (T == InType::I8) ? 1 : 2;
    const int64_t kbytes = (int64_t)args.K * esz;
    const int64_t lda_b = args.lda * esz, ldb_b = args.ldb * esz;
    const uint8_t *A = (const uint8_t *)args.a + zb * args.bsa * esz;
    const uint8_t *B = (const uint8_t *)args.b + zb * args.bsb * esz;
    const int KT = (int)((kbytes + BK - 1) / BK);

    // Operand panels as buffer resources (rows past the matrix edge read
    // zeros), as in mma_kernel.
    const int64_t kb16 = (kbytes + 15) / 16 * 16;
    const uint8_t *a_pan = A + (int64_t)m0 * lda_b;
    const uint8_t *b_pan = B + (int64_t)n0 * ldb_b;
    const uint32_t a_num = (uint32_t)(((args.M - m0 < BM ? args.M - m0 : BM) - 1) * lda_b + kb16);
    const uint32_t b_num = (uint32_t)(((args.N - n0 < BN ? args.N - n0 : BN) - 1) * ldb_b + kb16);

    // Loads: wave w fills rows [w*LPW*RPI, +LPW*RPI) of an A stage and of a B
    // stage; instruction i's rows lie RPI*i below instruction 0's and its
    // chunk repeats every two instructions (the swizzle).
    uint32_t voa[2], vob[2];
    int kch[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = (wave * LPW + i) * RPI + lane / CPR;
        const int ch = (lane % CPR) ^ swz_of<BK>(row);
        kch[i] = ch * 16;
        voa[i] = (uint32_t)(row * lda_b + ch * 16);
        vob[i] = (uint32_t)(row * ldb_b + ch * 16);
    }
    const uint32_t rsa = (uint32_t)(RPI * lda_b), rsb = (uint32_t)(RPI * ldb_b);
    const bool soff_ok = lda_b >= kb16 && ldb_b >= kb16;
    // Load i of operand X (0: A, 1: B) of stage kt into its slot; stages wholly
    // inside K take the stage offset in the scalar operand.
    auto load1 = [&](auto whole, int X, int kt, int slot, int i) {
        const uint32_t kb = (uint32_t)kt * BK;
        const uint32_t lo = X == 0 ? voa[i % 2] + (uint32_t)(i - i % 2) * rsa
                                   : vob[i % 2] + (uint32_t)(i - i % 2) * rsb;
        const uint8_t *pan = X == 0 ? a_pan : b_pan;
        const uint32_t num = X == 0 ? a_num : b_num;
        uint8_t *dst = smem + (X == 0 ? slot * ASTAGE : B_BASE + slot * BSTAGE) +
                       (wave * LPW + i) * 1024;
        if constexpr (decltype(whole)::value) {
            dma16s(pan, num, lo, kb, dst);
        } else {
            uint32_t off = lo + kb;
            if (kt >= KT || (int64_t)kb + kch[i % 2] >= kbytes) off = kOutOfRange;
            dma16(pan, num, off, dst);
        }
    };

    acc_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = acc_t{};

    const int l16 = lane & 15, lq = lane >> 4;
    const int a_off0 = (wm * WTM + l16) * BK;             // + i*16*BK for block i
    const int b_off0 = (wn * WTN + l16) * BK;             // + j*16*BK for block j
    const int swz = swz_of<BK>(l16);  // block bases are multiples of 16 rows
    auto slot_of = [&](int ss) { return ((4 * ss + lq) ^ swz) << 4; };

    v4i af[2][TM], bf[2][TN];
    auto mfma_rows = [&](int set, int r0) {
#pragma unroll
        for (int i = r0; i < r0 + TM / 2; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = M::step(bf[set][j], af[set][i], acc[i][j]);
    };
    // Program-order memory operations of a phase: A reads of blocks
    // [alo, alo+NA) from stage sa and (WB) the B reads from stage sb, with NL
    // loads (ld(l), l = 0..NL-1) spread among them (op_is_load).
    auto ops = [&](const uint8_t *sa, const uint8_t *sb, int ss, int set, int alo, auto na, auto wb,
                   auto nl, auto ld) {
        constexpr int NA = decltype(na)::value;
        constexpr int NB = decltype(wb)::value ? TN : 0;
        constexpr int NR = NA + NB;
        constexpr int NL = decltype(nl)::value;
        const int sl = slot_of(ss);
        int l = 0;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            // Order: A[alo], the B fragments, then A[alo+1 ..]: the next
            // phase's first MFMAs pair A[alo] with every B fragment (measured
            // on int8 4096^3: 58.4-58.9 against 58.6-60.7 us with the A
            // fragments first).
            const int ra = r == 0 ? 0 : (r <= NB ? -1 : r - NB);
            const int rbi = r - (NA > 0 ? 1 : 0);
            if (NA > 0 && ra >= 0)
                af[set][alo + ra] = *(const v4i *)(sa + a_off0 + (alo + ra) * 16 * BK + sl);
            else
                bf[set][rbi] = *(const v4i *)(sb + b_off0 + rbi * 16 * BK + sl);
            if ((r + 1) * NL / NR != r * NL / NR) {
                ld(l);
                ++l;
            }
        }
    };

    // Requantization channels: loaded now, staged in LDS beside the epilogue
    // staging once the ring is free (see mma_kernel).
    constexpr int QPT = (QCH + NWAVES * 64 - 1) / (NWAVES * 64);
    float *const q_scale = (float *)(smem + EPI_BYTES);
    int32_t *const q_bias = (int32_t *)(smem + EPI_BYTES + QCH * 4);
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

    // Load schedule: stage kt+2's A loads go out under stage kt's first phase
    // (A slot (kt+2)%3 last held stage kt-1, whose reads ended before stage
    // kt-1's barrier), its B loads under stage kt's last phase, after the
    // barrier that ends stage kt's B reads; both are waited for at stage
    // kt+1's barrier, with the four A loads per wave of stage kt+3 still in
    // flight.  The A loads thus have two stages to land and the B loads,
    // issued before them in the address unit's queue, one: with all of a
    // stage's loads after the barrier in a two-slot ring they landed late
    // (int8 4096^3 main loop 78.5k against 73.9k shader cycles per
    // workgroup; bf16 157.8k against 146.0k).
    using ZL = std::integral_constant<int, 0>;
    using LW = std::integral_constant<int, LPW>;
    auto noload = [](int) {};
#pragma unroll
    for (int i = 0; i < LPW; ++i) load1(std::false_type{}, 0, 0, 0, i);
#pragma unroll
    for (int i = 0; i < LPW; ++i) load1(std::false_type{}, 1, 0, 0, i);
#pragma unroll
    for (int i = 0; i < LPW; ++i) load1(std::false_type{}, 0, 1, 1, i);
#pragma unroll
    for (int i = 0; i < LPW; ++i) load1(std::false_type{}, 1, 1, 1, i);
    wait_vmcnt<2 * LPW>();  // stage 0 landed
    stage_barrier();
    {
        using NA = std::integral_constant<int, TM>;
        ops(smem, smem + B_BASE, 0, 0, 0, NA{}, std::true_type{}, ZL{}, noload);
    }

    constexpr int NM = (TM / 2) * TN;  // MFMAs per phase (16)
    constexpr int SPAN = NM * 7 / 8;
    const int ktw = (int)(kbytes / BK);
    // sa: stage kt's A slot (kt % 3).
    auto kstep = [&](int kt, int sa, auto whole) {
        using H = std::integral_constant<int, TM / 2>;
        using FA = std::integral_constant<int, TM>;
        const int sa1 = sa == NSA - 1 ? 0 : sa + 1, sa2 = sa1 == NSA - 1 ? 0 : sa1 + 1;
        const uint8_t *s_a = smem + sa * ASTAGE, *s_b = smem + B_BASE + (kt & 1) * BSTAGE;
        const uint8_t *n_a = smem + sa1 * ASTAGE, *n_b = smem + B_BASE + ((kt + 1) & 1) * BSTAGE;
        auto ld_a = [&](int i) { load1(whole, 0, kt + 2, sa2, i); };
        auto ld_b = [&](int i) { load1(whole, 1, kt + 2, kt & 1, i); };
        // phase 0: sub-step 0, blocks 0-3; read sub-step 1's A 0-3 and B;
        // stage kt+2's A loads
        mfma_rows(0, 0);
        ops(s_a, s_b, 1, 1, 0, H{}, std::true_type{}, LW{}, ld_a);
        sched_ops<NM, TM / 2 + TN, LPW, SPAN>();
        // phase 1: sub-step 0, blocks 4-7; read sub-step 1's A 4-7
        mfma_rows(0, TM / 2);
        ops(s_a, s_b, 1, 1, TM / 2, H{}, std::false_type{}, ZL{}, noload);
        sched_ops<NM, TM / 2, 0, SPAN>();
        // phase 2: sub-step 1, blocks 0-3; stage kt+1 landed (the A loads of
        // stage kt+2 may fly), then the barrier
        mfma_rows(1, 0);
#pragma unroll
        for (int m = 0; m < NM; ++m) __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
#pragma unroll
        for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[0][i]));
#pragma unroll
        for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bf[0][j]));
        wait_vmcnt<LPW>();
        stage_barrier();
#pragma unroll
        for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[1][i]));
#pragma unroll
        for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bf[1][j]));
        // phase 3: sub-step 1, blocks 4-7; read stage kt+1's sub-step 0;
        // stage kt+2's B loads
        mfma_rows(1, TM / 2);
        ops(n_a, n_b, 0, 0, 0, FA{}, std::true_type{}, LW{}, ld_b);
        sched_ops<NM, TM + TN, LPW, SPAN>();
    };
    // Stages whose loads (of stage kt+2) lie wholly inside K take the
    // scalar-offset loads.
    const int kt_whole = soff_ok ? (ktw - 2 > 0 ? ktw - 2 : 0) : 0;
    int kt = 0, sa = 0;
    for (; kt < kt_whole; ++kt) {
        kstep(kt, sa, std::true_type{});
        sa = sa == NSA - 1 ? 0 : sa + 1;
    }
    for (; kt < KT; ++kt) {
        kstep(kt, sa, std::false_type{});
        sa = sa == NSA - 1 ? 0 : sa + 1;
    }

    // Staged epilogue, 16 rows per block: each 16 x 64 row band of the wave
    // goes to LDS as 16-byte writes (EPI_LD = 4 mod 64 words: conflict-free)
    // and comes back as rows, 16 lanes per row, whole 16-byte chunks.  The
    // loads issued past the end of K (zeros into ring slots) land first.
    wait_vmcnt<0>();
    __syncthreads();
    if constexpr (E == EpiKind::Q8) {
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
            const int c = tid + u * NWAVES * 64;
            if (c < q_n) {
                q_scale[c] = q_s[u];
                q_bias[c] = q_b[u];
            }
        }
        __syncthreads();
    }
    val_t *stg = (val_t *)smem + wave * 16 * EPI_LD;
    typedef val_t v4_t __attribute__((ext_vector_type(4)));
    constexpr bool FB = E == EpiKind::F32 || E == EpiKind::BF16;
    constexpr int CPRE = WTN / 4;   // 16 chunks per staged row
    constexpr int RPIT = 64 / CPRE; // 4 rows per read iteration
    float col_s[4] = {0, 0, 0, 0}, col_f[4] = {0, 0, 0, 0};
    int32_t col_b[4] = {0, 0, 0, 0};
    if constexpr (E == EpiKind::Q8) {
        if (ep.axis) {
            const int ci = wn * WTN + (lane % CPRE) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                col_s[e] = q_scale[ci + e];
                col_b[e] = q_bias[ci + e];
            }
        }
    }
    if constexpr (FB) {
        if (ep.fused && ep.axis) {
            const int c = n0 + wn * WTN + (lane % CPRE) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                col_f[e] = c + e < args.N ? fused_bias<E == EpiKind::BF16>(ep, c + e) : 0.0f;
        }
    }
    const int gcol0 = n0 + wn * WTN;
    // A lane's column is fixed and its row advances by RPIT per pass, so its
    // output address is a per-band base plus a stepped offset (no 64-bit
    // multiplies per chunk; used by the requantizing store).
    constexpr int ESZ = E == EpiKind::Q8 ? 1 : (E == EpiKind::BF16 ? 2 : 4);
    const int64_t row_step = ep.rsc * ESZ;
    const int64_t out_off = (int64_t)(lane / CPRE) * row_step + (lane % CPRE) * 4 * ESZ;
    // Whether every channel scale this wave uses is finite and below 2^100
    // (requant_pack4's fast tier needs no overflow check then).
    bool tame = true;
    if constexpr (E == EpiKind::Q8) {
        static_assert(WTN == 64 && WTM == 128, "one channel per lane (columns) or two (rows)");
        bool bad;
        if (ep.axis) {
            bad = !(__builtin_fabsf(q_scale[wn * WTN + lane]) < 0x1p100f);
        } else {
            bad = !(__builtin_fabsf(q_scale[wm * WTM + lane]) < 0x1p100f) ||
                  !(__builtin_fabsf(q_scale[wm * WTM + 64 + lane]) < 0x1p100f);
        }
        tame = __builtin_amdgcn_ballot_w64(bad) == 0;
    }
    // The requantizing and bf16 stores are long: their row loop stays rolled
    // (unrolled under the unrolled block loop, 32 copies of it thrash the
    // instruction cache: requantized 4096^3 88 against 67 us).
    constexpr int IT_UNROLL = (E == EpiKind::Q8 || E == EpiKind::BF16) ? 1 : 16 / RPIT;
    // i32 outputs are written through the L2 (StPol::WT; whole 16-byte
    // chunks, 256 bytes per row segment, so whole lines go out).
    constexpr StPol kPol = E == EpiKind::I32 ? StPol::WT : StPol::Plain;
    if constexpr (E == EpiKind::F32) {
        if (!ep.fused) {
            // Unfused f32: whole tile rows.  The four waves of a row half
            // stage their 16 x 64 blocks side by side (two buffers alternating
            // by block, so one barrier per block), then each wave stores four
            // of the 16 rows, one 1 KiB row per instruction, written through
            // the L2 (bf16 4096^3 with f32 out: 99.19 against 99.79 and
            // 100.58 against 101.10 us in same-process A/Bs).
            constexpr int LDW = BN + 4;  // 4 mod 64 words: conflict-free 16-byte writes
            static_assert(4 * 16 * LDW * 4 <= SMEM, "row staging");
            val_t *const rows = (val_t *)smem;
            const int col = n0 + lane * 4;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                val_t *const sb = rows + (wm * 2 + (i & 1)) * 16 * LDW;
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const v4_t w = {(val_t)acc[i][j][0], (val_t)acc[i][j][1], (val_t)acc[i][j][2],
                                    (val_t)acc[i][j][3]};
                    *(v4_t *)(sb + l16 * LDW + wn * WTN + j * 16 + 4 * lq) = w;
                }
                // After this barrier every wave's block i is staged.  (The
                // buffer was rewritten only after block i-1's barrier, which
                // each wave reaches once its reads of block i-2 are done.)
                __builtin_amdgcn_s_waitcnt(0xC07F);
                stage_barrier();
                const int grow0 = m0 + wm * WTM + i * 16 + wn * 4;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const v4_t v4 = *(const v4_t *)(sb + (wn * 4 + r) * LDW + lane * 4);
                    const val_t v[4] = {v4[0], v4[1], v4[2], v4[3]};
                    if (grow0 + r < args.M && col < n_end)
                        store4<E, val_t, StPol::WT>(ep, z, grow0 + r, col, n_end, v, col_s, col_b,
                                                    col_f);
                }
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const v4_t w = {(val_t)acc[i][j][0], (val_t)acc[i][j][1], (val_t)acc[i][j][2],
                            (val_t)acc[i][j][3]};
            *(v4_t *)(stg + l16 * EPI_LD + j * 16 + 4 * lq) = w;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
        const int grow0 = m0 + wm * WTM + i * 16;
        uint8_t *const cb =
            (uint8_t *)ep.c + (z * ep.bsc + (int64_t)grow0 * ep.rsc + gcol0) * ESZ + out_off;
#pragma unroll IT_UNROLL
        for (int it = 0; it < 16 / RPIT; ++it) {
            const int row = it * RPIT + lane / CPRE;
            const int c4 = (lane % CPRE) * 4;
            v4_t v4 = *(const v4_t *)(stg + row * EPI_LD + c4);
            val_t v[4] = {v4[0], v4[1], v4[2], v4[3]};
            const int grow = grow0 + row;
            float s4[4] = {col_s[0], col_s[1], col_s[2], col_s[3]};
            int32_t b4[4] = {col_b[0], col_b[1], col_b[2], col_b[3]};
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
            float f4[4] = {col_f[0], col_f[1], col_f[2], col_f[3]};
            if constexpr (FB) {
                if (ep.fused && !ep.axis) {
                    const float f = grow < args.M ? fused_bias<E == EpiKind::BF16>(ep, grow) : 0.0f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) f4[e] = f;
                }
            }
            if (grow < args.M && gcol0 + c4 < n_end) {
                // The requantizing store is VALU-bound: whole chunks take the
                // stepped address and requant_pack4 (requantized 4096^3: 57.8
                // against 59.7 us).  The i32/f32/bf16 stores are bound by the
                // write stream; there the per-chunk address costs nothing
                // measurable and they keep store4.
                if (E == EpiKind::Q8 && ep.vec4 && gcol0 + c4 + 4 <= n_end)
                    store4_at<E, val_t, kPol>(ep, cb + (int64_t)it * RPIT * row_step, v, s4, b4,
                                               f4, tame);
                else
                    store4<E, val_t, kPol>(ep, z, grow, gcol0 + c4, n_end, v, s4, b4, f4);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }
}

template <InType T, EpiKind E>
static hipError_t launch16(const MmaArgs &args, const EpiParams &ep, hipStream_t stream) {
    if ((args.pn != 0 && args.pn != 256) || args.splits > 1) return hipErrorInvalidValue;
    const int esz = T == InType::I8 ? 1 : 2;
    if (!panels_fit(256, 256, args.lda * esz, args.ldb * esz, (int64_t)args.K * esz))
        return hipErrorInvalidValue;
    const int tiles = ((args.M + 255) / 256) * ((args.N + 255) / 256);
    hipLaunchKernelGGL((mma16_kernel<T, E>), dim3(tiles, 1, args.batch), dim3(512), 0, stream,
                       args, ep);
    return hipGetLastError();
}

hipError_t launch_mma16(InType in, const MmaArgs &args, const EpiParams &ep, hipStream_t stream) {
    if (in == InType::I8) {
        if (ep.kind == EpiKind::I32) return launch16<InType::I8, EpiKind::I32>(args, ep, stream);
        if (ep.kind == EpiKind::Q8) return launch16<InType::I8, EpiKind::Q8>(args, ep, stream);
    } else if (in == InType::BF16) {
        if (ep.kind == EpiKind::F32) return launch16<InType::BF16, EpiKind::F32>(args, ep, stream);
        if (ep.kind == EpiKind::BF16) return launch16<InType::BF16, EpiKind::BF16>(args, ep, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace gk
