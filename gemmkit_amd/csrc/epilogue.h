// epilogue.h -- per-element output maps applied to accumulator registers.
//
// Each map restates one of gemmkit's epilogues on a single accumulator value,
// so the MFMA and GEMV kernels store through the same code:
//   I32  int32_epilogue  (src/kernel/int.rs:36-120): alpha*acc, then C / C+acc /
//        beta*C+acc, all wrapping i32;
//   F32  the float epilogue (src/kernel/float.rs:150-281): alpha*acc, then
//        beta*C + acc in f32 (beta == 0 never reads C);
//   BF16 mixed_epilogue (src/kernel/mixed.rs:96-200): the f32 value of F32, then
//        one round-to-nearest-even narrowing to bf16 with the NaN rule of
//        src/simd/avx512.rs:194-212;
//   Q8   KRequantize::apply (src/kernel/epilogue.rs:810-830): wrapping bias add,
//        one f64 multiply by the widened f32 scale, round half to even, zero
//        point, clamp to [lo, hi], store the low byte -- computed exactly
//        without f64 arithmetic (requant.h).
// F32 and BF16 also carry gemmkit's fused bias/activation (FusedEpi,
// src/kernel/epilogue.rs:269-330 and :556-596) on the f32 value before the store.
#pragma once

#include "internal.h"
#include "requant.h"

namespace gk {

// f32 -> bf16 as gemmkit's narrowing (half::bf16::from_f32): round to nearest
// even, NaN kept quiet with its sign and top payload bits ((bits >> 16) |
// 0x40).  gfx950's v_cvt_pk_bf16_f32 gives exactly that for every f32 input
// (denormals preserved, the kernels' default float mode) and converts two
// values per instruction.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t bf16x2_rne(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint16_t bf16_rne(float f) {
    return (uint16_t)bf16x2_rne(f, 0.0f);
}

__device__ __forceinline__ float bf16_widen(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}

// The requant map on one i32 accumulator (requant.h): f32 arithmetic with an
// exact tie correction for operands below 2^24, 64-bit integer arithmetic
// otherwise; bit-identical to the f64 formula either way, without CDNA4's
// slow f64 VALU ops.
__device__ __forceinline__ int32_t requant_value(int32_t acc, int32_t bias, float scale,
                                                 int32_t zp, int32_t lo, int32_t hi) {
    return requant_fast(acc, bias, scale, zp, lo, hi);
}

// FusedEpi::apply (src/kernel/epilogue.rs:309-330, :569-596) on the f32 value
// the plain store would write, with the bias value b already loaded (0 when
// there is no bias: v + 0 differs from v only for v = -0, which every
// activation maps to +0, and the map is off when there is neither).  ReLU is
// v > 0 ? v : 0, so NaN and -0 give +0; LeakyReLU is hi + slope*lo with
// hi = v > 0 ? v : 0 and lo = v < 0 ? v : 0.  Nothing here may contract into
// an FMA, which keeps f32 results bit-identical to the plain GEMM followed by
// the same scalar map.
__device__ __forceinline__ float fused_apply(const EpiParams &ep, float v, float b) {
#pragma clang fp contract(off)
    v = v + b;
    const float hi = v > 0.0f ? v : 0.0f;
    const float lo = v < 0.0f ? v : 0.0f;
    const float leaky = hi + ep.slope * lo;
    return ep.act == kActRelu ? hi : (ep.act == kActLeakyRelu ? leaky : v);
}

// The bias value of channel ch: f32, or bf16 widened exactly when BF16_BIAS.
template <bool BF16_BIAS>
__device__ __forceinline__ float fused_bias(const EpiParams &ep, int ch) {
    if (!ep.fbias) return 0.0f;
    return BF16_BIAS ? bf16_widen(((const uint16_t *)ep.fbias)[ch]) : ((const float *)ep.fbias)[ch];
}

template <bool BF16_BIAS>
__device__ __forceinline__ float fused_map(const EpiParams &ep, float v, int row, int col) {
    return fused_apply(ep, v, fused_bias<BF16_BIAS>(ep, ep.axis ? col : row));
}

// Stores one accumulator at output coordinate (row, col) of batch element z.
template <EpiKind K>
struct Store;

template <>
struct Store<EpiKind::I32> {
    __device__ __forceinline__ static void apply(const EpiParams &ep, int64_t z, int row, int col,
                                                 int32_t acc) {
        int32_t *c = (int32_t *)ep.c + z * ep.bsc + (int64_t)row * ep.rsc + (int64_t)col * ep.csc;
        uint32_t v = (uint32_t)ep.alpha_i * (uint32_t)acc;
        if (ep.beta_i == 0) {
            *c = (int32_t)v;
        } else if (ep.beta_i == 1) {
            *c = (int32_t)((uint32_t)*c + v);
        } else {
            *c = (int32_t)((uint32_t)ep.beta_i * (uint32_t)*c + v);
        }
    }
};

template <>
struct Store<EpiKind::F32> {
    __device__ __forceinline__ static void apply(const EpiParams &ep, int64_t z, int row, int col,
                                                 float acc) {
        float *c = (float *)ep.c + z * ep.bsc + (int64_t)row * ep.rsc + (int64_t)col * ep.csc;
        float v = ep.alpha_f * acc;
        if (ep.beta_f == 1.0f) {
            v = *c + v;
        } else if (ep.beta_f != 0.0f) {
            v = __builtin_fmaf(ep.beta_f, *c, v);
        }
        if (ep.fused) v = fused_map<false>(ep, v, row, col);
        *c = v;
    }
};

template <>
struct Store<EpiKind::BF16> {
    __device__ __forceinline__ static void apply(const EpiParams &ep, int64_t z, int row, int col,
                                                 float acc) {
        uint16_t *c = (uint16_t *)ep.c + z * ep.bsc + (int64_t)row * ep.rsc + (int64_t)col * ep.csc;
        float v = ep.alpha_f * acc;
        if (ep.beta_f == 1.0f) {
            v = bf16_widen(*c) + v;
        } else if (ep.beta_f != 0.0f) {
            v = __builtin_fmaf(ep.beta_f, bf16_widen(*c), v);
        }
        if (ep.fused) v = fused_map<true>(ep, v, row, col);
        *c = bf16_rne(v);
    }
};

template <>
struct Store<EpiKind::Q8> {
    __device__ __forceinline__ static void apply(const EpiParams &ep, int64_t z, int row, int col,
                                                 int32_t acc) {
        int ch = ep.axis ? col : row;
        float s = ep.scales ? ep.scales[ch] : ep.scale;
        int32_t b = ep.bias ? ep.bias[ch] : 0;
        int32_t q = requant_value(acc, b, s, ep.zp, ep.lo, ep.hi);
        uint8_t *c = (uint8_t *)ep.c + z * ep.bsc + (int64_t)row * ep.rsc + (int64_t)col * ep.csc;
        *c = (uint8_t)(q & 0xFF);
    }
};


// Cache policy of an output store.
//   Plain  write-back: the line stays dirty in the XCD's L2 and reaches the
//          256 MB Infinity Cache when evicted or at the kernel's end;
//   NT     nontemporal (streamed towards HBM): outputs written once while other
//          data streams, such as the short-contraction kernel's rotating batches
//          (the big tiles measured 1.7 us slower with it on 4096^3 i32 and 2 us on
//          bf16 4096^3 with f32 out; the batched attention scores 4 us faster);
//   WT     write-back with the sc1 (device scope) bit, which writes the data
//          through the L2 as it is stored, in pieces per store instruction:
//          right only where every instruction covers whole 128-byte lines.
//          The big tile's i32 rows (256-byte segments) take it: int8 4096^3
//          56.2 / 58.8 / 58.3 against 57.7 / 58.4 / 58.1 us in same-process
//          A/Bs on three boxes, WRITE_SIZE unchanged.  The requantizing layer
//          measured 2 us faster with it (78.7 / 79.7 / 79.6 against 80.7 /
//          81.8 / 81.7) but its 176-byte row pieces then leave the L2 as
//          partial lines, 27.0 MB written for the 22.5 MB output (1.2x), so it
//          stays Plain.  f32 rows take it where the tile stores whole 1 KiB
//          rows (0.5-0.6 us on bf16 4096^3 with f32 out); with the per-wave
//          256-byte pieces f32 measured no change, bf16 output keeps NT;
//   NTWT   nontemporal with sc1: the band kernel's attention scores
//          15.2-15.4 against 15.5-15.7 us with NT alone (four A/Bs).
// Every policy stores the same bytes; only where the line is kept differs.
enum class StPol { Plain, NT, WT, NTWT };

// Requantized words follow a WT request and are stored Plain otherwise
// (no kernel requests WT for them; see above).
constexpr StPol q8_pol(StPol p) { return p == StPol::WT ? StPol::WT : StPol::Plain; }

template <StPol P, typename V>
__device__ __forceinline__ void st_out(V *p, V v) {
    static_assert(sizeof(V) == 16 || sizeof(V) == 4, "16-byte chunks or 4-byte words");
    if constexpr (P == StPol::Plain) {
        *p = v;
    } else if constexpr (P == StPol::NT) {
        __builtin_nontemporal_store(v, p);
    } else if constexpr (sizeof(V) == 16) {
        if constexpr (P == StPol::WT)
            asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
        else
            asm volatile("global_store_dwordx4 %0, %1, off nt sc1" : : "v"(p), "v"(v) : "memory");
    } else {
        if constexpr (P == StPol::WT)
            asm volatile("global_store_dword %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
        else
            asm volatile("global_store_dword %0, %1, off nt sc1" : : "v"(p), "v"(v) : "memory");
    }
}

// Four consecutive output columns (col .. col+3) of one row, from the
// LDS-staged accumulators.  `vec` (uniform) says C is unit-stride along columns
// and 4-element aligned, so whole chunks take one vector access; otherwise, and
// for chunks that straddle the matrix edge, each element is stored alone.
// Requantization uses the caller's per-element channel scale and bias (qs,
// qb): the f32 path for all four, its tie correction for every lane of the
// wave when any lane's product sits on a half, and the exact integer path for
// every lane of the wave when any lane needs it.
// For F32/BF16 with a fused epilogue, fb holds the four elements' bias values.
// P is the cache policy of the i32, f32 and requantized stores (StPol); bf16
// chunks are always stored nontemporally.
template <EpiKind K, typename A, StPol P = StPol::NT>
__device__ __forceinline__ void store4(const EpiParams &ep, int64_t z, int row, int col, int ncols,
                                       const A v[4], const float *qs = nullptr,
                                       const int32_t *qb = nullptr, const float *fb = nullptr) {
    const int nvalid = ncols - col < 4 ? ncols - col : 4;
    int32_t q[4] = {0, 0, 0, 0};
    if constexpr (K == EpiKind::Q8) {
        bool slow = false, tie = false;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const RequantF32 r = requant_f32((int32_t)v[e], qb[e], qs[e], ep.zp, ep.lo, ep.hi);
            q[e] = r.q;
            slow = slow || r.slow;
            tie = tie || r.tie;
        }
        if (__builtin_amdgcn_ballot_w64(tie) != 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                q[e] = requant_f32_tie((int32_t)v[e], qb[e], qs[e], ep.zp, ep.lo, ep.hi);
        }
        if (__builtin_amdgcn_ballot_w64(slow) != 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                q[e] = requant_bits((int32_t)v[e], qb[e], __float_as_uint(qs[e]), ep.zp, ep.lo,
                                    ep.hi);
        }
    }
    if (!ep.vec4 || nvalid < 4) {
        // (a static loop: a runtime bound would index v[] dynamically and
        // send it through scratch memory)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (e >= nvalid) break;
            if constexpr (K == EpiKind::Q8) {
                uint8_t *c = (uint8_t *)ep.c + z * ep.bsc + (int64_t)row * ep.rsc +
                             (int64_t)(col + e) * ep.csc;
                *c = (uint8_t)(q[e] & 0xFF);
            } else {
                Store<K>::apply(ep, z, row, col + e, v[e]);
            }
        }
        return;
    }
    const int64_t off = z * ep.bsc + (int64_t)row * ep.rsc + col;
    if constexpr (K == EpiKind::I32) {
        typedef int v4i_e __attribute__((ext_vector_type(4)));
        v4i_e *c = (v4i_e *)((int32_t *)ep.c + off);
        v4i_e o;
        for (int e = 0; e < 4; ++e) o[e] = (int32_t)((uint32_t)ep.alpha_i * (uint32_t)v[e]);
        if (ep.beta_i != 0) {
            v4i_e old = *c;
            for (int e = 0; e < 4; ++e)
                o[e] = (int32_t)((ep.beta_i == 1 ? (uint32_t)old[e]
                                                 : (uint32_t)ep.beta_i * (uint32_t)old[e]) +
                                 (uint32_t)o[e]);
        }
        st_out<P>(c, o);
    } else if constexpr (K == EpiKind::F32) {
        typedef float v4f_e __attribute__((ext_vector_type(4)));
        v4f_e *c = (v4f_e *)((float *)ep.c + off);
        v4f_e o;
        for (int e = 0; e < 4; ++e) o[e] = ep.alpha_f * v[e];
        if (ep.beta_f != 0.0f) {
            v4f_e old = *c;
            for (int e = 0; e < 4; ++e)
                o[e] = ep.beta_f == 1.0f ? old[e] + o[e] : __builtin_fmaf(ep.beta_f, old[e], o[e]);
        }
        if (ep.fused) {
            for (int e = 0; e < 4; ++e) o[e] = fused_apply(ep, o[e], fb[e]);
        }
        st_out<P>(c, o);
    } else if constexpr (K == EpiKind::BF16) {
        typedef uint32_t v2u_e __attribute__((ext_vector_type(2)));
        v2u_e *c = (v2u_e *)((uint16_t *)ep.c + off);
        float f[4];
        for (int e = 0; e < 4; ++e) f[e] = ep.alpha_f * v[e];
        if (ep.beta_f != 0.0f) {
            v2u_e old = *c;
            for (int e = 0; e < 4; ++e) {
                float w = bf16_widen((uint16_t)(old[e >> 1] >> (16 * (e & 1))));
                f[e] = ep.beta_f == 1.0f ? w + f[e] : __builtin_fmaf(ep.beta_f, w, f[e]);
            }
        }
        if (ep.fused) {
            for (int e = 0; e < 4; ++e) f[e] = fused_apply(ep, f[e], fb[e]);
        }
        v2u_e o;
        o[0] = bf16x2_rne(f[0], f[1]);
        o[1] = bf16x2_rne(f[2], f[3]);
        __builtin_nontemporal_store(o, c);
    } else {
        const uint32_t word = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) |
                              ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)q[3] << 24);
        st_out<q8_pol(P)>((uint32_t *)((uint8_t *)ep.c + off), word);
    }
}

// The requant map on four accumulators of one row (channel scales s, biases
// b), returned as the four output bytes (element e in byte e).  The same three
// tiers as store4, fewer instructions in the common one:
//   * the wave takes requant_bits when some lane's operand reaches 2^24, or
//     when `tame` is false (the caller has seen a channel scale that is not
//     finite or reaches 2^100 -- below that, an operand under 2^24 keeps the
//     f32 product finite, so no per-element overflow check is needed);
//   * otherwise t = rint of the f32 product, with requant_f32_tie's correction
//     for the wave when some lane's product sits on a half;
//   * the zero point and band are applied in f32 with an offset of 128 when
//     the band reaches below zero (i8 output: the band lies in [-128, 127]),
//     which puts every in-band value in [0, 255]: one v_med3_f32 clamps it and
//     one v_cvt_pk_u8_f32 converts and packs it (exact on those integers), and
//     XOR 0x80 per byte removes the offset, leaving q & 0xFF.  t + zp is exact
//     wherever the result can land in the band (requant_band).
__device__ __forceinline__ uint32_t requant_pack4(const EpiParams &ep, const int32_t a[4],
                                                  const float s[4], const int32_t b[4],
                                                  bool tame) {
#pragma clang fp contract(off)
    float vf[4], ph[4], t[4], d[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        vf[e] = (float)(int32_t)((uint32_t)a[e] + (uint32_t)b[e]);
        ph[e] = vf[e] * s[e];
        t[e] = __builtin_rintf(ph[e]);
        d[e] = ph[e] - t[e];
    }
    // |ph - rint(ph)| <= 1/2, so some product sits on a half exactly when the
    // largest distance is 1/2; likewise one maximum bounds the four operands.
    const float vmax = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(vf[0]), __builtin_fabsf(vf[1])),
                                       __builtin_fmaxf(__builtin_fabsf(vf[2]), __builtin_fabsf(vf[3])));
    const float dmax = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(d[0]), __builtin_fabsf(d[1])),
                                       __builtin_fmaxf(__builtin_fabsf(d[2]), __builtin_fabsf(d[3])));
    const bool slow = !tame || !(vmax < 16777216.0f);
    const bool tie = dmax == 0.5f;
    if (__builtin_amdgcn_ballot_w64(slow) != 0) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w |= ((uint32_t)requant_bits(a[e], b[e], __float_as_uint(s[e]), ep.zp, ep.lo, ep.hi) &
                  0xFFu) << (8 * e);
        return w;
    }
    if (__builtin_amdgcn_ballot_w64(tie) != 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float pl = __builtin_fmaf(vf[e], s[e], -ph[e]);
            const bool away = d[e] > 0.0f ? pl > 0.0f : pl < 0.0f;
            if (__builtin_fabsf(d[e]) == 0.5f && away) t[e] += d[e] + d[e];
        }
    }
    const int32_t off = ep.lo < 0 ? 128 : 0;
    const float zo = (float)(ep.zp + off), lo = (float)(ep.lo + off), hi = (float)(ep.hi + off);
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        w = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_fmed3f(t[e] + zo, lo, hi), e, w);
    return off ? w ^ 0x80808080u : w;
}

// store4 for a chunk wholly inside the matrix with C unit-stride along
// columns and 4-element aligned (ep.vec4), at the address p of its first
// element, which the caller steps from chunk to chunk instead of forming it
// from (row, col) with 64-bit multiplies.  alpha = 1 skips the i32 multiplies;
// requantized chunks take requant_pack4 (`tame` as there).  Results equal
// store4's.
template <EpiKind K, typename A, StPol P = StPol::NT>
__device__ __forceinline__ void store4_at(const EpiParams &ep, void *p, const A v[4],
                                          const float *qs = nullptr, const int32_t *qb = nullptr,
                                          const float *fb = nullptr, bool tame = true) {
    if constexpr (K == EpiKind::Q8) {
        const int32_t a[4] = {(int32_t)v[0], (int32_t)v[1], (int32_t)v[2], (int32_t)v[3]};
        st_out<q8_pol(P)>((uint32_t *)p, requant_pack4(ep, a, qs, qb, tame));
    } else if constexpr (K == EpiKind::I32) {
        typedef int v4i_e __attribute__((ext_vector_type(4)));
        v4i_e *c = (v4i_e *)p;
        v4i_e o = {(int32_t)v[0], (int32_t)v[1], (int32_t)v[2], (int32_t)v[3]};
        if (ep.alpha_i != 1)
            for (int e = 0; e < 4; ++e) o[e] = (int32_t)((uint32_t)ep.alpha_i * (uint32_t)o[e]);
        if (ep.beta_i != 0) {
            v4i_e old = *c;
            for (int e = 0; e < 4; ++e)
                o[e] = (int32_t)((ep.beta_i == 1 ? (uint32_t)old[e]
                                                 : (uint32_t)ep.beta_i * (uint32_t)old[e]) +
                                 (uint32_t)o[e]);
        }
        st_out<P>(c, o);
    } else if constexpr (K == EpiKind::F32) {
        typedef float v4f_e __attribute__((ext_vector_type(4)));
        v4f_e *c = (v4f_e *)p;
        v4f_e o;
        for (int e = 0; e < 4; ++e) o[e] = ep.alpha_f * v[e];
        if (ep.beta_f != 0.0f) {
            v4f_e old = *c;
            for (int e = 0; e < 4; ++e)
                o[e] = ep.beta_f == 1.0f ? old[e] + o[e] : __builtin_fmaf(ep.beta_f, old[e], o[e]);
        }
        if (ep.fused) {
            for (int e = 0; e < 4; ++e) o[e] = fused_apply(ep, o[e], fb[e]);
        }
        st_out<P>(c, o);
    } else {
        typedef uint32_t v2u_e __attribute__((ext_vector_type(2)));
        v2u_e *c = (v2u_e *)p;
        float f[4];
        for (int e = 0; e < 4; ++e) f[e] = ep.alpha_f * v[e];
        if (ep.beta_f != 0.0f) {
            v2u_e old = *c;
            for (int e = 0; e < 4; ++e) {
                float w = bf16_widen((uint16_t)(old[e >> 1] >> (16 * (e & 1))));
                f[e] = ep.beta_f == 1.0f ? w + f[e] : __builtin_fmaf(ep.beta_f, w, f[e]);
            }
        }
        if (ep.fused) {
            for (int e = 0; e < 4; ++e) f[e] = fused_apply(ep, f[e], fb[e]);
        }
        v2u_e o;
        o[0] = bf16x2_rne(f[0], f[1]);
        o[1] = bf16x2_rne(f[2], f[3]);
        __builtin_nontemporal_store(o, c);
    }
}

}  // namespace gk
