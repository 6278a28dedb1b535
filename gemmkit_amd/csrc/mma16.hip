// mma16.hip -- the 256 x 256 eight-wave tile on 16x16 matrix-core
// instructions (v_mfma_i32_16x16x64_i8, v_mfma_f32_16x16x32_bf16).
//
// Same data path as mma_kernel.h (direct-to-LDS loads of 128-byte stages into
// a two-stage swizzled ring, fragment reads interleaved with the MFMAs, one
// barrier per stage, the staged epilogue), with 16x16 blocks: on this chip
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
    constexpr int STAGE = (BM + BN) * BK;        // 64 KiB
    constexpr int A_BYTES = BM * BK;
    constexpr int NI = STAGE / 1024;             // direct-to-LDS instructions per stage
    constexpr int NIW = NI / NWAVES;             // ... per wave (8)
    constexpr int RPI = 1024 / BK;               // stage rows one instruction fills
    constexpr int CPR = BK / 16;                 // 16-byte chunks per stage row
    constexpr int EPI_LD = WTN + 4;              // staged-epilogue row stride (words)
    constexpr int SMEM = 2 * STAGE;
    static_assert(BM % (NIW * RPI) == 0, "each wave's loads come from one operand");
    static_assert(NWAVES * 16 * EPI_LD * 4 <= SMEM, "epilogue staging does not fit");
    using M = Mma16x<T>;
    using acc_t = typename M::acc_t;
    using val_t = typename M::scalar_t;
    constexpr int QCH = (E == EpiKind::Q8) ? BM : 1;
    constexpr int QBYTES = (E == EpiKind::Q8) ? QCH * 8 : 0;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM + QBYTES];

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
    const bool k_whole = (kbytes % BK) == 0;

    // Operand panels as buffer resources (rows past the matrix edge read
    // zeros), as in mma_kernel.
    const int64_t kb16 = (kbytes + 15) / 16 * 16;
    const uint8_t *a_pan = A + (int64_t)m0 * lda_b;
    const uint8_t *b_pan = B + (int64_t)n0 * ldb_b;
    const uint32_t a_num = (uint32_t)(((args.M - m0 < BM ? args.M - m0 : BM) - 1) * lda_b + kb16);
    const uint32_t b_num = (uint32_t)(((args.N - n0 < BN ? args.N - n0 : BN) - 1) * ldb_b + kb16);

    // Loads: wave w fills stage bytes [w*NIW*1024, (w+1)*NIW*1024), all from
    // one operand; instruction i's rows lie RPI*i below instruction 0's and
    // its chunk repeats every two instructions (the swizzle).
    uint32_t voff[2];
    int kch[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = wave * NIW + i;
        const int row = q * RPI + lane / CPR;
        const int ch = (lane % CPR) ^ swz_of<BK>(row);
        kch[i] = ch * 16;
        voff[i] = q * RPI < BM ? (uint32_t)(row * lda_b + ch * 16)
                               : (uint32_t)((row - BM) * ldb_b + ch * 16);
    }
    const bool w_from_a = wave * NIW * RPI < BM;
    const uint8_t *const w_pan = w_from_a ? a_pan : b_pan;
    const uint32_t w_num = w_from_a ? a_num : b_num;
    const uint32_t rstep = (uint32_t)(RPI * (w_from_a ? lda_b : ldb_b));
    auto lane_off = [&](int i) -> uint32_t { return voff[i % 2] + (uint32_t)(i - i % 2) * rstep; };
    auto issue_stage = [&](int kt, int slot, int first, int count) {
        const uint32_t kb = (uint32_t)kt * BK;
        uint8_t *dst = smem + slot * STAGE + wave * NIW * 1024;
        const bool dead = kt >= KT;
        const bool tail = !k_whole && kt == KT - 1;
#pragma unroll
        for (int i = first; i < first + count; ++i) {
            uint32_t off = lane_off(i) + kb;
            if (dead || (tail && (int64_t)kb + kch[i % 2] >= kbytes)) off = kOutOfRange;
            dma16(w_pan, w_num, off, dst + i * 1024);
        }
    };
    const bool soff_ok = lda_b >= kb16 && ldb_b >= kb16;
    auto issue_whole = [&](int kt, int slot, int first, int count) {
        const uint32_t kb = (uint32_t)kt * BK;
        uint8_t *dst = smem + slot * STAGE + wave * NIW * 1024;
#pragma unroll
        for (int i = first; i < first + count; ++i) dma16s(w_pan, w_num, lane_off(i), kb, dst + i * 1024);
    };

    acc_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = acc_t{};

    const int l16 = lane & 15, lq = lane >> 4;
    const int a_off0 = (wm * WTM + l16) * BK;             // + i*16*BK for block i
    const int b_off0 = A_BYTES + (wn * WTN + l16) * BK;   // + j*16*BK for block j
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
    // [alo, alo+NA) and (WB) the B reads, with NL loads of stage st into
    // `slot` spread among them (op_is_load); whole stages take scalar-offset
    // loads.
    auto ops = [&](auto whole, const uint8_t *src, int ss, int set, int alo, auto na, auto wb,
                   auto nl, int st, int slot, int first) {
        constexpr bool WHOLE = decltype(whole)::value;
        constexpr int NA = decltype(na)::value;
        constexpr int NB = decltype(wb)::value ? TN : 0;
        constexpr int NR = NA + NB;
        constexpr int NL = decltype(nl)::value;
        const int sl = slot_of(ss);
        int l = first;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            // Order: A[alo], the B fragments, then A[alo+1 ..]: the next
            // phase's first MFMAs pair A[alo] with every B fragment (measured
            // on int8 4096^3: 58.4-58.9 against 58.6-60.7 us with the A
            // fragments first).
            const int ra = r == 0 ? 0 : (r <= NB ? -1 : r - NB);
            const int rbi = r - (NA > 0 ? 1 : 0);
            if (NA > 0 && ra >= 0)
                af[set][alo + ra] = *(const v4i *)(src + a_off0 + (alo + ra) * 16 * BK + sl);
            else
                bf[set][rbi] = *(const v4i *)(src + b_off0 + rbi * 16 * BK + sl);
            if ((r + 1) * NL / NR != r * NL / NR) {
                if constexpr (WHOLE)
                    issue_whole(st, slot, l, 1);
                else
                    issue_stage(st, slot, l, 1);
                ++l;
            }
        }
    };

    // Requantization channels staged in LDS (see mma_kernel).
    constexpr int QPT = (QCH + NWAVES * 64 - 1) / (NWAVES * 64);
    float *const q_scale = (float *)(smem + SMEM);
    int32_t *const q_bias = (int32_t *)(smem + SMEM + QCH * 4);
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

    // Load schedule: stage kt+2's loads go into stage kt's slot as soon as the
    // barrier that ends the reads of stage kt allows, all of them under stage
    // kt's last phase (P0), so each has three phases to land.  (At this
    // kernel's higher clock the 32x32 tile's split -- a third there, the rest
    // under stage kt+1's first two phases -- leaves the last loads too little
    // time: 63.5-65.6 against 59.4-61.5 us on int8 4096^3.  Giving the A
    // panel a third 32 KiB slot instead, its loads two stages ahead, measured
    // 63.2-63.8 us.)
    constexpr int P0 = NIW, P1 = 0, P2 = 0;
    issue_stage(0, 0, 0, NIW);
    issue_stage(1, 1, 0, P0);
    wait_vmcnt<P0>();
    if constexpr (E == EpiKind::Q8) {
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
            const int c = tid + u * NWAVES * 64;
            if (c < q_n) {
                q_scale[c] = q_s[u];
                q_bias[c] = q_b[u];
            }
        }
    }
    stage_barrier();
    {
        using Z = std::integral_constant<int, 0>;
        using NA = std::integral_constant<int, TM>;
        ops(std::false_type{}, smem, 0, 0, 0, NA{}, std::true_type{}, Z{}, 0, 0, 0);
    }

    constexpr int NM = (TM / 2) * TN;  // MFMAs per phase (16)
    constexpr int SPAN = NM * 7 / 8;
    const int ktw = (int)(kbytes / BK);
    auto kstep = [&](int kt, auto whole) {
        using L0 = std::integral_constant<int, P0>;
        using L1 = std::integral_constant<int, P1>;
        using L2 = std::integral_constant<int, P2>;
        using LN = std::integral_constant<int, 0>;
        using H = std::integral_constant<int, TM / 2>;
        using FA = std::integral_constant<int, TM>;
        using A0 = std::integral_constant<int, 0>;
        const uint8_t *s = smem + (kt & 1) * STAGE;
        const int nslot = (kt + 1) & 1;
        // phase 0: sub-step 0, blocks 0-3; read sub-step 1's A 0-3 and B
        mfma_rows(0, 0);
        ops(whole, s, 1, 1, 0, H{}, std::true_type{}, L1{}, kt + 1, nslot, P0);
        sched_ops<NM, TM / 2 + TN, P1, SPAN>();
        // phase 1: sub-step 0, blocks 4-7; read sub-step 1's A 4-7
        mfma_rows(0, TM / 2);
        ops(whole, s, 1, 1, TM / 2, H{}, std::false_type{}, L2{}, kt + 1, nslot, P0 + P1);
        sched_ops<NM, TM / 2, P2, SPAN>();
        // phase 2: sub-step 1, blocks 0-3
        mfma_rows(1, 0);
#pragma unroll
        for (int m = 0; m < NM; ++m) __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
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
        // phase 3: sub-step 1, blocks 4-7; read stage kt+1's sub-step 0
        mfma_rows(1, TM / 2);
        ops(whole, smem + nslot * STAGE, 0, 0, 0, FA{}, std::true_type{}, L0{}, kt + 2, kt & 1, 0);
        sched_ops<NM, TM + TN, P0, SPAN>();
        (void)LN{};
        (void)A0{};
    };
    const int kt_whole = soff_ok ? (ktw - 2 < KT ? (ktw - 2 > 0 ? ktw - 2 : 0) : KT) : 0;
    int kt = 0;
    for (; kt < kt_whole; ++kt) kstep(kt, std::true_type{});
    for (; kt < KT; ++kt) kstep(kt, std::false_type{});

    // Staged epilogue, 16 rows per block: each 16 x 64 row band of the wave
    // goes to LDS as 16-byte writes (EPI_LD = 4 mod 64 words: conflict-free)
    // and comes back as rows, 16 lanes per row, whole 16-byte chunks.
    __syncthreads();
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
                    store4_at<E, val_t, false>(ep, cb + (int64_t)it * RPIT * row_step, v, s4, b4,
                                               f4, tame);
                else
                    store4<E, val_t, false>(ep, z, grow, gcol0 + c4, n_end, v, s4, b4, f4);
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
