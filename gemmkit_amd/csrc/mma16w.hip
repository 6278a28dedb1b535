// mma16w.hip -- the 256 x 352 eight-wave tile on 16x16 matrix-core
// instructions (int8: v_mfma_i32_16x16x64_i8), for products whose 256-wide
// tiles would need a second, short round of the CUs: one round of these tiles
// at a column pitch of at most 352 (the host's choice, plan_mma) covers them
// instead (2048 x 11008 x 4096: 8 x 32 tiles at a pitch of 344 columns).
//
// Data path as in mma16.hip: 128-byte K stages loaded global -> LDS with
// direct-to-LDS buffer loads into a two-stage swizzled ring (2 x 76 KiB),
// operand fragments read from LDS, i32 accumulators in VGPRs.  Layout: the
// eight waves form 4 x 2, each 64 rows x 176 columns = 4 x 11 blocks of 16 x
// 16 (176 accumulator registers); a 64-byte sub-step is 15 fragment reads
// (4 A, 11 B) for 44 MFMAs.  Lane l reads row l%16 of a 16-row block, chunk
// 4*s + l/16 of sub-step s, for A and B alike; register r of lane l holds C
// row l%16, column 4*(l/16) + r of a block.
//
// Schedule (ping-pong): the two wave groups (waves 0-3: rows 0-127, waves
// 4-7: rows 128-255; each SIMD holds one wave of each) take turns a barrier
// apart.  Both run the same body per sub-step -- its 44 MFMAs, a barrier, the
// fragment reads of the next sub-step (after a stage's second sub-step, with
// the loads of the stage two ahead), a barrier -- with the second group one
// slot behind (an extra barrier before its first body), so one group's LDS
// reads and their latency hide under the other group's matrix work.  A wave
// never reads fragments while its own MFMAs run, so one fragment set (60
// registers) serves it, which is what lets the 176 accumulators fit.
// Barriers per stage, absolute slots 4kt .. 4kt+3:
//   4kt   group 0 MFMAs sub-step 0 | group 1 reads sub-step 0
//   4kt+1 group 0 reads sub-step 1 | group 1 MFMAs sub-step 0
//   4kt+2 group 0 MFMAs sub-step 1 | group 1 reads sub-step 1
//   --- stage kt+1 landed (each wave waited for its loads), stage kt read ---
//   4kt+3 group 0 reads stage kt+1's sub-step 0, loads stage kt+2 |
//         group 1 MFMAs sub-step 1
// (group 1 issues its loads of stage kt+2 in its next read slot, 4kt+4).
#include "mma_kernel.h"

namespace gk {

template <EpiKind E>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mma16w_kernel(const MmaArgs args, const EpiParams ep) {
    constexpr int BM = 256, BN = 352, BK = 128;
    constexpr int NWAVES = 8, WN = 2;
    constexpr int WTM = 64, WTN = 176;
    constexpr int TM = WTM / 16, TN = WTN / 16;  // 4 x 11 blocks
    constexpr int STAGE = (BM + BN) * BK;        // 76 KiB
    constexpr int A_BYTES = BM * BK;
    constexpr int NI = STAGE / 1024;             // 76 direct-to-LDS instructions per stage
    constexpr int NIW = (NI + NWAVES - 1) / NWAVES;  // 10 per wave (the last one of waves 4-7 a dummy)
    constexpr int IA = BM / (NWAVES * 8);        // instructions 0..3 of each wave load A rows
    constexpr int SMEM = 2 * STAGE;
    constexpr int QCH = (E == EpiKind::Q8) ? BN : 1;
    constexpr int QBYTES = (E == EpiKind::Q8) ? QCH * 8 : 0;
    constexpr int SPARE = SMEM + QBYTES;         // the dummy loads' target (1 KiB)
    constexpr int EPI_LD = WTN + 4;              // staged-epilogue row stride (words)
    static_assert(NWAVES * 16 * EPI_LD * 4 <= SMEM, "epilogue staging does not fit");
    static_assert(SPARE + 1024 <= 160 * 1024, "LDS");
    static_assert(NI > (NIW - 1) * NWAVES && NI <= NIW * NWAVES, "ragged loads");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[SPARE + 1024];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int grp = wave >> 2;  // 0: waves 0-3 (rows 0-127), 1: waves 4-7

    const int PN = args.pn > 0 ? args.pn : BN;  // column pitch (<= BN)
    const int tiles_m = (args.M + BM - 1) / BM;
    const int tiles_n = (args.N + PN - 1) / PN;
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
    const int m0 = tmi * BM, n0 = tni * PN;
    const int n_end = args.N - n0 < PN ? args.N : n0 + PN;  // columns this tile stores
    const int64_t z = zb;

    const int64_t kbytes = (int64_t)args.K;  // int8: one byte per element
    const int64_t lda_b = args.lda, ldb_b = args.ldb;
    const uint8_t *A = (const uint8_t *)args.a + zb * args.bsa;
    const uint8_t *B = (const uint8_t *)args.b + zb * args.bsb;
    const int KT = (int)((kbytes + BK - 1) / BK);
    const bool k_whole = (kbytes % BK) == 0;

    // Operand panels: A rows [m0, m0+BM) and B rows [n0, n0+PN) as buffer
    // resources over the valid rows' bytes; rows past the matrix edge or the
    // pitch start outside them and read zeros (or, when rows overlap, feed
    // outputs that are never stored).
    const int64_t kb16 = (kbytes + 15) / 16 * 16;
    const uint8_t *a_pan = A + (int64_t)m0 * lda_b;
    const uint8_t *b_pan = B + (int64_t)n0 * ldb_b;
    const uint32_t a_num = (uint32_t)(((args.M - m0 < BM ? args.M - m0 : BM) - 1) * lda_b + kb16);
    const uint32_t b_num = (uint32_t)(((args.N - n0 < PN ? args.N - n0 : PN) - 1) * ldb_b + kb16);

    // Loads: the wave's instruction i is stage instruction q = i*8 + wave,
    // filling stage bytes [q*1024, q*1024 + 1024) = stage rows 8q .. 8q+7
    // (lane l: row 8q + l/8, slot l%8, which holds chunk (l%8) ^ swz(row)).
    // Instructions 0..3 take A rows (64 rows apart: same swizzle), 4..9 B
    // rows; q >= 76 (waves 4-7's last) is a dummy into the spare 1 KiB.
    const int lrow = wave * 8 + lane / 8;
    const int lch = (lane % 8) ^ swz_of<BK>(lrow);
    const uint32_t voff_a = (uint32_t)(lrow * lda_b + lch * 16);
    const uint32_t voff_b = (uint32_t)(lrow * ldb_b + lch * 16);
    const uint32_t step_a = (uint32_t)(64 * lda_b), step_b = (uint32_t)(64 * ldb_b);
    auto lane_off = [&](int i) -> uint32_t {
        return i < IA ? voff_a + (uint32_t)i * step_a : voff_b + (uint32_t)(i - IA) * step_b;
    };
    auto is_dummy = [&](int i) { return i == NIW - 1 && (i * NWAVES + wave) >= NI; };
    auto dst_of = [&](int slot, int i) {
        return is_dummy(i) ? smem + SPARE : smem + slot * STAGE + (i * NWAVES + wave) * 1024;
    };
    auto issue_stage = [&](int kt, int slot, int first, int count) {
        const uint32_t kb = (uint32_t)kt * BK;
        const bool dead = kt >= KT;
        const bool tail = !k_whole && kt == KT - 1;
#pragma unroll
        for (int i = first; i < first + count; ++i) {
            uint32_t off = lane_off(i) + kb;
            if (dead || is_dummy(i) || (tail && (int64_t)kb + lch * 16 >= kbytes)) off = kOutOfRange;
            dma16(i < IA ? a_pan : b_pan, i < IA ? a_num : b_num, off, dst_of(slot, i));
        }
    };
    // Stages wholly inside K with rows that do not overlap: the stage offset
    // in the scalar operand (a lane out of range stays out of range).
    const bool soff_ok = lda_b >= kb16 && ldb_b >= kb16;
    auto issue_whole = [&](int kt, int slot, int first, int count) {
        const uint32_t kb = (uint32_t)kt * BK;
#pragma unroll
        for (int i = first; i < first + count; ++i)
            dma16s(i < IA ? a_pan : b_pan, i < IA ? a_num : b_num,
                   is_dummy(i) ? kOutOfRange : lane_off(i), kb, dst_of(slot, i));
    };

    v4i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    const int l16 = lane & 15, lq = lane >> 4;
    const int a_off0 = (wm * WTM + l16) * BK;            // + i*16*BK for block i
    const int b_off0 = A_BYTES + (wn * WTN + l16) * BK;  // + j*16*BK for block j
    const int swz = swz_of<BK>(l16);                     // block bases are multiples of 16 rows
    auto slot_of = [&](int ss) { return ((4 * ss + lq) ^ swz) << 4; };

    v4i af[TM], bf[TN];
    // The fragment reads of sub-step ss of the stage at `src` (A[0], the B
    // fragments, then A[1..]: the order the MFMAs use them), with NL loads of
    // stage st into `slot` spread among them.
    auto reads = [&](auto whole, const uint8_t *src, int ss, auto nl, int st, int slot) {
        constexpr int NL = decltype(nl)::value;
        constexpr int NR = TM + TN;
        const int sl = slot_of(ss);
        int l = 0;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            if (r == 0)
                af[0] = *(const v4i *)(src + a_off0 + sl);
            else if (r <= TN)
                bf[r - 1] = *(const v4i *)(src + b_off0 + (r - 1) * 16 * BK + sl);
            else
                af[r - TN] = *(const v4i *)(src + a_off0 + (r - TN) * 16 * BK + sl);
            if ((r + 1) * NL / NR != r * NL / NR) {
                if constexpr (decltype(whole)::value)
                    issue_whole(st, slot, l, 1);
                else
                    issue_stage(st, slot, l, 1);
                ++l;
            }
        }
    };
    auto mfmas = [&]() {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
    };
    auto barrier = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };

    // Requantization channels staged in LDS past the ring.
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

    using Z = std::integral_constant<int, 0>;
    using LW = std::integral_constant<int, NIW>;
    issue_stage(0, 0, 0, NIW);
    issue_stage(1, 1, 0, NIW);
    wait_vmcnt<NIW>();
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
    reads(std::false_type{}, smem, 0, Z{}, 0, 0);

    auto stage = [&](int kt, auto whole) {
        const uint8_t *s = smem + (kt & 1) * STAGE;
        const uint8_t *ns = smem + ((kt + 1) & 1) * STAGE;
        // sub-step 0 of stage kt, then the reads of its sub-step 1
        mfmas();
        barrier();
        reads(whole, s, 1, Z{}, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (grp == 1) wait_vmcnt<0>();  // group 1: stage kt+1 landed, stage kt read
        barrier();
        // sub-step 1, then the reads of stage kt+1's sub-step 0 with the
        // loads of stage kt+2 into stage kt's slot
        mfmas();
        __builtin_amdgcn_sched_barrier(0);
        if (grp == 0) wait_vmcnt<0>();  // group 0: likewise, one slot earlier in its body
        barrier();
        reads(whole, ns, 0, LW{}, kt + 2, kt & 1);
        barrier();
    };
    const int ktw = (int)(kbytes / BK);
    const int kt_whole = soff_ok ? (ktw - 2 < KT ? (ktw - 2 > 0 ? ktw - 2 : 0) : KT) : 0;
    if (grp == 1) barrier();
    int kt = 0;
    for (; kt < kt_whole; ++kt) stage(kt, std::true_type{});
    for (; kt < KT; ++kt) stage(kt, std::false_type{});
    if (grp == 0) barrier();

    // Staged epilogue: each wave's 16 x 176 row bands go to LDS as 16-byte
    // writes and come back as rows, 4 consecutive columns per lane, 44 lanes
    // per row (11 passes over the 704 chunks of a band).  A lane's row and
    // chunk advance by 1 row + 20 chunks per pass, so its LDS and output
    // addresses are stepped, not recomputed: the 64-bit multiplies of a
    // per-chunk address cost more VALU time than the requantization itself.
    // Per-column channel scales and biases come as one 16-byte LDS read each
    // per chunk.
    __syncthreads();
    int32_t *stg = (int32_t *)smem + wave * 16 * EPI_LD;
    typedef int32_t v4_t __attribute__((ext_vector_type(4)));
    typedef float v4f_t __attribute__((ext_vector_type(4)));
    constexpr int CPRE = WTN / 4;    // 44 chunks per staged row
    constexpr int STEP = 64 - CPRE;  // chunks a lane moves per pass past one row
    constexpr int ESZ = E == EpiKind::Q8 ? 1 : 4;
    static_assert(WTM == 64 && STEP > 0 && STEP < CPRE, "pass stepping assumes 44-chunk rows");
    const int gcol0 = n0 + wn * WTN;
    // Whether every channel scale this wave uses is finite and below 2^100
    // (requant_pack4's fast tier needs no overflow check then).
    bool tame = true;
    if constexpr (E == EpiKind::Q8) {
        bool bad = false;
        if (ep.axis) {
            for (int c = lane; c < WTN; c += 64)
                bad = bad || !(__builtin_fabsf(q_scale[wn * WTN + c]) < 0x1p100f);
        } else {
            bad = !(__builtin_fabsf(q_scale[wm * WTM + lane]) < 0x1p100f);
        }
        tame = __builtin_amdgcn_ballot_w64(bad) == 0;
    }
    const int64_t row_step = ep.rsc * ESZ;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
            *(v4_t *)(stg + l16 * EPI_LD + j * 16 + 4 * lq) = acc[i][j];
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
        const int grow0 = m0 + wm * WTM + i * 16;
        // element (grow0, gcol0) of C; the lane's chunk is at cb + off
        uint8_t *const cb =
            (uint8_t *)ep.c + (z * ep.bsc + (int64_t)grow0 * ep.rsc + gcol0) * ESZ;
        int row = lane / CPRE, cc = lane % CPRE;
        int64_t off = row * row_step + 4 * cc * ESZ;
        int sidx = row * EPI_LD + 4 * cc;  // the chunk's word in the staging rows
#pragma unroll 1
        for (int it = 0; it < 16 * CPRE / 64; ++it) {
            const int c4 = 4 * cc;
            const v4_t w = *(const v4_t *)(stg + sidx);
            const int32_t v[4] = {w[0], w[1], w[2], w[3]};
            const int grow = grow0 + row, gcol = gcol0 + c4;
            float s4[4] = {0, 0, 0, 0};
            int32_t b4[4] = {0, 0, 0, 0};
            if constexpr (E == EpiKind::Q8) {
                if (ep.axis) {
                    const v4f_t sv = *(const v4f_t *)(q_scale + wn * WTN + c4);
                    const v4_t bv = *(const v4_t *)(q_bias + wn * WTN + c4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        s4[e] = sv[e];
                        b4[e] = bv[e];
                    }
                } else {
                    const int ri = grow - q_ch0 < BM ? grow - q_ch0 : BM - 1;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        s4[e] = q_scale[ri];
                        b4[e] = q_bias[ri];
                    }
                }
            }
            if (grow < args.M && gcol < n_end) {
                if (ep.vec4 && gcol + 4 <= n_end)
                    store4_at<E, int32_t, StPol::Plain>(ep, cb + off, v, s4, b4, nullptr, tame);
                else
                    store4<E, int32_t, StPol::Plain>(ep, z, grow, gcol, n_end, v, s4, b4, nullptr);
            }
            cc += STEP;
            row += 1;
            off += row_step + 4 * STEP * ESZ;
            sidx += EPI_LD + 4 * STEP;
            if (cc >= CPRE) {
                cc -= CPRE;
                row += 1;
                off += row_step - 4 * CPRE * ESZ;
                sidx += EPI_LD - 4 * CPRE;
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }
}

template <EpiKind E>
static hipError_t launch16w(const MmaArgs &args, const EpiParams &ep, hipStream_t stream) {
    const int pn = args.pn > 0 ? args.pn : 352;
    if (pn > 352 || pn % 4 != 0 || args.splits > 1) return hipErrorInvalidValue;
    if (!panels_fit(256, 352, args.lda, args.ldb, (int64_t)args.K)) return hipErrorInvalidValue;
    const int tiles = ((args.M + 255) / 256) * ((args.N + pn - 1) / pn);
    hipLaunchKernelGGL((mma16w_kernel<E>), dim3(tiles, 1, args.batch), dim3(512), 0, stream, args,
                       ep);
    return hipGetLastError();
}

hipError_t launch_mma16w(InType in, const MmaArgs &args, const EpiParams &ep, hipStream_t stream) {
    if (in != InType::I8) return hipErrorInvalidValue;
    if (ep.kind == EpiKind::I32) return launch16w<EpiKind::I32>(args, ep, stream);
    if (ep.kind == EpiKind::Q8) return launch16w<EpiKind::Q8>(args, ep, stream);
    return hipErrorInvalidValue;
}

}  // namespace gk
