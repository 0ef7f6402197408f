// Device building blocks shared by the paged-attention kernels (decode and
// prefill): KV tile loads in the [NB, Hkv, D, 16] layout and the per-block
// MFMA attention step with an online softmax.
#pragma once

#include "common.hpp"

namespace swiftllm {
namespace attn {

constexpr float kLog2e = 1.4426950408889634f;
// Probabilities are produced as 2^kPExp * exp2(s - m) (<= 2^15 < 65504).
constexpr float kPExp = 15.0f;
// Lazy rescaling: as 2^kPExpLazy * exp2(s - m) with m allowed to lag the true
// running max by up to kLazyMargin, so they stay <= 2^(7 + 8) = 2^15.
constexpr float kPExpLazy = 7.0f;
constexpr float kLazyMargin = 8.0f;

__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __fp16 h2 __attribute__((ext_vector_type(2)));

// gfx950's full-rate 16 x 16 x 32 form: lane (m, q) holds k = 8q .. 8q + 7.
__device__ __forceinline__ f4 mfma16x32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h8 cat8(h4 lo, h4 hi) {
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Reductions over the lane pairs l, l ^ 16 and l, l ^ 32 on gfx950's
// permlane swaps (VALU, no trip through the LDS crossbar that __shfl_xor
// takes). With both operands equal, permlane16_swap returns each lane's own
// value and its l ^ 16 partner's (in row order), permlane32_swap the same for
// l ^ 32 (checked on the GPU with an in-bounds probe); both lanes of a pair
// combine the two values in the same order.
__device__ __forceinline__ void swap16(float v, float& lo, float& hi) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    lo = __builtin_bit_cast(float, static_cast<unsigned>(r[0]));
    hi = __builtin_bit_cast(float, static_cast<unsigned>(r[1]));
}
__device__ __forceinline__ void swap32(float v, float& lo, float& hi) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    lo = __builtin_bit_cast(float, static_cast<unsigned>(r[0]));
    hi = __builtin_bit_cast(float, static_cast<unsigned>(r[1]));
}
// max(a, b) / max(a, b, c) as the bare instructions. For the values here
// (finite scores and -inf) they equal fmaxf; fmaxf itself costs an extra
// v_max x, x per operand that the compiler cannot prove canonical (results
// of lane swaps and selects), to quiet signalling NaNs.
__device__ __forceinline__ float max2(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float max3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
// max / sum over lanes l, l ^ 16, l ^ 32, l ^ 48.
__device__ __forceinline__ float max_over_kg(float v) {
    float a, b;
    swap16(v, a, b);
    v = max2(a, b);
    swap32(v, a, b);
    return max2(a, b);
}
__device__ __forceinline__ float sum_over_kg(float v) {
    float a, b;
    swap16(v, a, b);
    v = a + b;
    swap32(v, a, b);
    return a + b;
}

__device__ __forceinline__ h4 mask_h4(h4 v, unsigned long long m) {
    return __builtin_bit_cast(h4, __builtin_bit_cast(unsigned long long, v) & m);
}

// p - h[0] and p - h[1] for packed fp16 h, each one v_fma_mix_f32 reading
// the fp16 half directly (p + (-h) * 1.0, rounded once: the same value as
// converting h to fp32 and subtracting).
__device__ __forceinline__ float sub_h2_lo(float p, h2 h) {
    float r;
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(p));
    return r;
}
__device__ __forceinline__ float sub_h2_hi(float p, h2 h) {
    float r;
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(p));
    return r;
}

// fp32 values that are exact fp16 numbers (the identity-MFMA transpose of a
// K slice: one product with 1.0 plus exact zeros) back to fp16, two per
// instruction. Any rounding mode is exact for them; the packed conversion
// rounds toward zero.
__device__ __forceinline__ h4 to_h4(f4 v) {
    const h2 lo = __builtin_amdgcn_cvt_pkrtz(v[0], v[1]);
    const h2 hi = __builtin_amdgcn_cvt_pkrtz(v[2], v[3]);
    return __builtin_bit_cast(h4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3));
}

// A block id names a block of the pool: never negative, and below the pool
// size when that is known (num_blocks > 0).
__device__ __forceinline__ bool block_ok(int b, int num_blocks) {
    return b >= 0 && (num_blocks <= 0 || b < num_blocks);
}

// Decode reads each KV tile once per call, so it loads them nontemporally
// (streamed past the caches instead of evicting Q, block tables and the
// other waves' prefetched tiles; config 2: 113.0 us -> 104.9 us per call).
// Prefill reads each tile once per query group and keeps them cached (NT =
// false).
template <bool NT>
__device__ __forceinline__ h4 load_kv(const f16* p) {
    if (NT) return __builtin_nontemporal_load(reinterpret_cast<const h4*>(p));
    return *reinterpret_cast<const h4*>(p);
}

template <int D, bool NT = true>
__device__ __forceinline__ void load_tile(const f16* kc, const f16* vc, int Hkv, int num_blocks,
                                          int b, int kvh, int loff, h4 (&k)[D / 16],
                                          h4 (&v)[D / 16]) {
    constexpr int NJ = D / 16;
    // An id outside the pool reads block 0 instead (in bounds); the caller
    // skips such a block.
    const int bsafe = block_ok(b, num_blocks) ? b : 0;
    const size_t base = kv_tile_offset(bsafe, kvh, Hkv, D) + loff;
    const f16* kp = kc + base;
    const f16* vp = vc + base;
#pragma unroll
    for (int J = 0; J < NJ; ++J) {
        k[J] = load_kv<NT>(kp + kv_elem_offset(16 * J, 0));
    }
#pragma unroll
    for (int J = 0; J < NJ; ++J) {
        v[J] = load_kv<NT>(vp + kv_elem_offset(16 * J, 0));
    }
}

// Q^T operand of step 2: lane (r, kg) holds q[h0 + r][16J + 4kg .. +3].
template <int D>
struct QOperand {
    h4 v[D / 16];
    __device__ __forceinline__ h4 get(int J) const { return v[J]; }
};

// Running softmax state of one wave: max (log2 domain), sum of
// 2^15 * exp2(s - max) over this lane's token rows, and O^T accumulators.
template <int D>
struct WaveState {
    float m;
    float l;
    f4 acc[D / 16];
};

// One 16-token block for the wave's 16 query rows (MFMA N side), all on
// v_mfma_f32_16x16x16_f16:
//   1. the K tile rows arrive tokens-contiguous ([d][t]); an MFMA against a
//      0/1 identity operand returns them in the transposed ([t][d]) register
//      layout, exactly (one product per output);
//   2. S^T[t][g] = sum_d K^T[t][d] Q^T[d][g];
//   3. online softmax in fp32 in the log2 domain; the 4 token rows of query
//      row g live in lanes g, g^16, g^32, g^48 (two xor shuffles);
//   4. O^T[d][g] += V[d][t] P^T[t][g] with V in its stored layout and P fed
//      as fp16 hi + lo parts (~20 bits), P = 2^15 * exp2(s - m).
// The first nv tokens of the tile exist (the rest is zeroed so stale values
// cannot reach a sum; nv == 0: the block contributes nothing), and query row
// g = lane % 16 of this lane sees tokens t < lim (lim <= nv).
// Zeroes the K/V of tokens nv.. of the tile (tail block) so no stale value
// (possibly NaN) reaches a sum through a 0 weight.
template <int D>
__device__ __forceinline__ void mask_tail(int nv, int kg, h4 (&kA)[D / 16], h4 (&vA)[D / 16]) {
    constexpr int NJ = D / 16;
    // nv is the same in every lane: a scalar branch, which the compiler would
    // otherwise turn into an all-ones mask ANDed into every tile register.
    if (__builtin_amdgcn_readfirstlane(nv) < kBlockTokens) [[unlikely]] {
        const int c = min(max(nv - 4 * kg, 0), 4);
        const unsigned long long m = (c >= 4) ? ~0ull : ((1ull << (16 * c)) - 1ull);
#pragma unroll
        for (int J = 0; J < NJ; ++J) {
            kA[J] = mask_h4(kA[J], m);
            vA[J] = mask_h4(vA[J], m);
        }
    }
}

// Steps 3 + 4 for one group of 16 query rows, from the S^T accumulator sc.
// Lane (r, kg) holds S^T[t = 4kg + i][g = r].
// PV32 runs PV on the 16x16x32 form: k = 8q + i is token 4q + i of the hi
// half of P for i < 4 and of the lo half otherwise, so the A operand is the
// lane's V piece twice and the B operand its hi and lo pieces side by side.
// FOLD (scale_log2 > 0 only): the max is taken on the unscaled scores and
// scaled once per row (a positive factor keeps the max in place, exactly),
// and each score's scale goes into the fused multiply-add before exp2.
// LAZY: the accumulators are rescaled only when some row's max grows by more
// than kLazyMargin (log2 units); otherwise m stays behind and the weights
// carry the difference, at most 2^kLazyMargin. Weights are 2^kPExpLazy *
// exp2(s - m). Below 2^-3 the fp16 lo half of a weight is subnormal: its
// error, at most 2^-24, is under 2^-31 of the row sum (>= 2^7).
template <int D, bool PV32 = false, bool FOLD = false, bool LAZY = false>
__device__ __forceinline__ void softmax_pv(WaveState<D>& st, f4 sc, int lim, int kg,
                                           const h4 (&vA)[D / 16], float scale_log2) {
    constexpr int NJ = D / 16;
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = FOLD ? sc[i] : sc[i] * scale_log2;
    // Masks only where some row sees part of the block (tail blocks, the
    // causal diagonal): interior blocks skip the compares.
    if (__any(lim < kBlockTokens)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (4 * kg + i >= lim) sv[i] = -INFINITY;
        }
    }
    float bm = max2(max3(sv[0], sv[1], sv[2]), sv[3]);
    bm = max_over_kg(bm);
    if constexpr (FOLD) bm *= scale_log2;
    if (__any(bm > (LAZY ? st.m + kLazyMargin : st.m))) {
        const float m_new = fmaxf(st.m, bm);
        const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
#pragma unroll
        for (int J = 0; J < NJ; ++J) st.acc[J] *= alpha;
        st.l *= alpha;
        st.m = m_new;
    }
    // While no valid token has been seen (an out-of-pool block, nv == 0) the
    // max is still -inf and every sv is -inf: use 0 so the weights are 0.
    const float m_use = (st.m == -INFINITY) ? 0.0f : st.m;
    const float c = m_use - (LAZY ? kPExpLazy : kPExp);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        p[i] = __builtin_amdgcn_exp2f(FOLD ? __builtin_fmaf(sv[i], scale_log2, -c) : sv[i] - c);
    }
    st.l += (p[0] + p[1]) + (p[2] + p[3]);
    // hi = p rounded toward zero to fp16, lo = the remainder (exact in fp32)
    // rounded toward zero again: hi + lo keeps ~20 bits of p. The packed
    // conversions make two halves per instruction.
    const h2 h01 = __builtin_amdgcn_cvt_pkrtz(p[0], p[1]);
    const h2 h23 = __builtin_amdgcn_cvt_pkrtz(p[2], p[3]);
    const h2 l01 = __builtin_amdgcn_cvt_pkrtz(sub_h2_lo(p[0], h01), sub_h2_hi(p[1], h01));
    const h2 l23 = __builtin_amdgcn_cvt_pkrtz(sub_h2_lo(p[2], h23), sub_h2_hi(p[3], h23));
    const h4 ph = __builtin_bit_cast(h4, __builtin_shufflevector(h01, h23, 0, 1, 2, 3));
    const h4 pl = __builtin_bit_cast(h4, __builtin_shufflevector(l01, l23, 0, 1, 2, 3));
    // Step 4. Lane (r, kg) accumulates O^T[d = 16J + 4kg + i][g = r].
    if constexpr (PV32) {
        const h8 p8 = cat8(ph, pl);
#pragma unroll
        for (int J = 0; J < NJ; ++J) st.acc[J] = mfma16x32(cat8(vA[J], vA[J]), p8, st.acc[J]);
    } else {
#pragma unroll
        for (int J = 0; J < NJ; ++J) {
            st.acc[J] = mfma16(vA[J], ph, st.acc[J]);
            st.acc[J] = mfma16(vA[J], pl, st.acc[J]);
        }
    }
}

template <int D>
__device__ __forceinline__ void attend_block(WaveState<D>& st, int nv, int lim, int kg,
                                             h4 (&kA)[D / 16], h4 (&vA)[D / 16],
                                             const QOperand<D>& qB, h4 ident,
                                             float scale_log2) {
    constexpr int NJ = D / 16;
    mask_tail<D>(nv, kg, kA, vA);
    // Steps 1 + 2.
    f4 s0 = f4{0, 0, 0, 0}, s1 = f4{0, 0, 0, 0};
#pragma unroll
    for (int J = 0; J < NJ; ++J) {
        const f4 t = mfma16(kA[J], ident, f4{0, 0, 0, 0});
        const h4 kT = to_h4(t);
        if (J & 1) {
            s1 = mfma16(kT, qB.get(J), s1);
        } else {
            s0 = mfma16(kT, qB.get(J), s0);
        }
    }
    softmax_pv<D>(st, s0 + s1, lim, kg, vA, scale_log2);
}

// The same block for two groups of 16 query rows that share the kv head:
// the K tile is transposed once and feeds both QK^T products. QK^T runs on
// the 16x16x32 form over pairs of 16-row slices (J0 = 2J', J1 = 2J' + 1):
// with k = 8q + i read as d = 16 J0 + 4q + i for i < 4 and 16 J1 + 4q + i - 4
// otherwise, the A operand is the lane's two transposed slices side by side
// and the B operand its two Q pieces side by side.
template <int D, bool FOLD = false>
__device__ __forceinline__ void attend_block_pair(WaveState<D>& sa, WaveState<D>& sb, int nv,
                                                  int lim_a, int lim_b, int kg,
                                                  h4 (&kA)[D / 16], h4 (&vA)[D / 16],
                                                  const QOperand<D>& qa, const QOperand<D>& qb,
                                                  h4 ident, float scale_log2) {
    constexpr int NJ = D / 16;
    mask_tail<D>(nv, kg, kA, vA);
    // One accumulator per group: the two groups' MFMAs interleave, so
    // neither chain waits on its own previous result.
    f4 sa_ = f4{0, 0, 0, 0}, sb_ = f4{0, 0, 0, 0};
#pragma unroll
    for (int J = 0; J < NJ; J += 2) {
        const h8 kT = cat8(to_h4(mfma16(kA[J], ident, f4{0, 0, 0, 0})),
                           to_h4(mfma16(kA[J + 1], ident, f4{0, 0, 0, 0})));
        sa_ = mfma16x32(kT, cat8(qa.get(J), qa.get(J + 1)), sa_);
        sb_ = mfma16x32(kT, cat8(qb.get(J), qb.get(J + 1)), sb_);
    }
    softmax_pv<D, true, FOLD, true>(sa, sa_, lim_a, kg, vA, scale_log2);
    softmax_pv<D, true, FOLD, true>(sb, sb_, lim_b, kg, vA, scale_log2);
}

// Every query row sees the same nv tokens (decode).
template <int D>
__device__ __forceinline__ void attend_block(WaveState<D>& st, int nv, int kg,
                                             h4 (&kA)[D / 16], h4 (&vA)[D / 16],
                                             const QOperand<D>& qB, h4 ident,
                                             float scale_log2) {
    attend_block<D>(st, nv, nv, kg, kA, vA, qB, ident, scale_log2);
}

}  // namespace attn
}  // namespace swiftllm
