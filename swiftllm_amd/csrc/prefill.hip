// Paged prefill attention for gfx950.
//
// Contract (crates/swiftllm-cuda/src/bindings.rs:33-54 declares the launch;
// crates/swiftllm-core/src/memory/paged_attention.rs:154-189 lists the steps:
// scores Q K^T / sqrt(d), causal mask, softmax, times V, with K and V stored
// into the cache by slot_mapping). The reference computes none of it. Here:
//   the query tokens of the batch are packed: sequence s owns tokens
//   [start_s, start_s + L_s), start_s = sum of context_lens before s, and
//   token p of s sits in the cache at slot_mapping[start_s + p] (the caller
//   writes K/V there first, e.g. with reshape_and_cache);
//   out[start_s + i, h] = sum_{j <= i} softmax_j(scale q[start_s + i, h] .
//                         K(slot[start_s + j], kvh)) V(slot[start_s + j], kvh)
//   with kvh = h / (H / Hkv). fp16 in and out, fp32 accumulation.
// The slots of a sequence must follow its block table from position 0
// (slot of p = table[p / 16] * 16 + p % 16, what get_slot_mapping produces):
// the kernel reads the block of 16 positions from the slot of the first.
//
// Work decomposition. A wave owns two groups of 16 MFMA query rows; a group
// is tpw = 16 / gw consecutive query tokens times gw = min(G, 16) query heads
// of one kv head, and the second group takes the next tpw tokens. Every K/V
// tile the wave loads serves both groups, and the K tile is transposed once
// for both. The wave walks the key blocks up to its last token; each lane's
// query row carries its own causal limit. K tiles are copied unchanged into
// the wave's LDS by direct loads and read back already transposed
// (ds_read_b64_tr_b16), and the walk goes by pairs of blocks: one softmax
// step per 32 keys, whose PV products take the two blocks' V side by side.
// Key caches that are 8- but not 16-byte aligned take the per-block MFMA
// step shared with decode (attention_core.hpp: an identity-MFMA
// transposition of K in registers). A wave's rows are complete when
// its walk ends, so it writes its outputs directly: no combine, no barriers.
// Four waves per workgroup take consecutive token groups. Each XCD runs the
// (sequence, kv head) units of its residue mod 8 one after the other, each
// unit's workgroups latest tokens first (the longest walks start first), so
// the workgroups resident on an XCD share one unit's K/V in its L2. K/V tiles are loaded
// with ordinary (cached) loads: every query group of a sequence re-reads them.

#include <type_traits>
#include "attention_core.hpp"

namespace swiftllm {
namespace {

using namespace attn;

constexpr int kPrefillWaves = 4;

struct PrefillArgs {
    f16* out;            // [T][H][D]
    const f16* q;        // [T][H][D]
    const f16* kc;
    const f16* vc;
    const int* slots;    // [T]
    const int* ctx;      // [S] query tokens per sequence
    float scale_log2;
    int S;
    int H;
    int Hkv;
    int G;               // query heads per kv head
    int nhc;             // head chunks of 16 per kv head
    int gw;              // query heads per row group: min(G, 16)
    int tpw;             // query tokens per row group: 16 / gw (a wave has two groups)
    int groups;          // workgroups per (sequence, kv head chunk) in the grid
    long long units;     // (sequence, kv head chunk) pairs: S * Hkv * nhc
    int num_blocks;      // bound on block ids; <= 0: unbounded
};

// FOLD: scale_log2 > 0 (the usual 1/sqrt(D)), whose scale then goes into the
// softmax's exp2 argument.
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4 lds_s4;

// The K^T operand of one 16-row slice J from a K tile copied unchanged into
// LDS ([d][16 tokens], 2 KiB per 64 rows). With lane l reading the 8 bytes at
// element 256 J + 4 l, ds_read_b64_tr_b16 hands lane l the elements
// K[16 J + 4 (l / 16) + i][l % 16], i = 0..3: within each 16-lane group, lane
// i receives element i % 4 of lanes i / 4, + 4, + 8, + 12 (checked on the
// GPU with an in-bounds probe). That is the transposed slice in the MFMA's
// A-operand layout, the same values the identity-MFMA transposition makes.
__device__ __forceinline__ h4 read_kT(const f16* tile, int J, int lane) {
    const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s4*)(const_cast<f16*>(tile) + 256 * J + 4 * lane));
    return __builtin_bit_cast(h4, v);
}

// Zeroes the V columns of the tokens past nv0 in the low halves (the pair's
// first block) and past nv1 in the high halves (its second block); nv0 and
// nv1 are the same in every lane, so this is a scalar branch.
template <int D>
__device__ __forceinline__ void mask_v_pair(int nv0, int nv1, int kg, h8 (&vp)[D / 16]) {
    if (__builtin_amdgcn_readfirstlane(min(nv0, nv1)) < kBlockTokens) [[unlikely]] {
        const int c0 = min(max(nv0 - 4 * kg, 0), 4);
        const int c1 = min(max(nv1 - 4 * kg, 0), 4);
        const unsigned long long m0 = (c0 >= 4) ? ~0ull : ((1ull << (16 * c0)) - 1ull);
        const unsigned long long m1 = (c1 >= 4) ? ~0ull : ((1ull << (16 * c1)) - 1ull);
#pragma unroll
        for (int J = 0; J < D / 16; ++J) {
            const h4 lo = __builtin_shufflevector(vp[J], vp[J], 0, 1, 2, 3);
            const h4 hi = __builtin_shufflevector(vp[J], vp[J], 4, 5, 6, 7);
            vp[J] = cat8(mask_h4(lo, m0), mask_h4(hi, m1));
        }
    }
}

// Steps 3 + 4 for one group of 16 query rows over a pair of key blocks (32
// keys), from the S^T accumulators s0 (first block) and s1 (second): lane
// (r, kg) holds S^T[t = 4kg + i][g = r] of each. The same online softmax as
// the per-block step (lazy rescaling, weights 2^kPExpLazy * exp2(s - m) as
// fp16 hi + lo parts, FOLD as there), with one row max per 32 keys. PV runs
// on the 16x16x32 form with k = 8q + i the token 4q + i of the first block
// for i < 4 and of the second otherwise: the A operand is the lane's V
// pieces of the two blocks side by side (vp), the B operand the two blocks'
// hi parts, then their lo parts.
template <int D, bool FOLD>
__device__ __forceinline__ void softmax_pv_pair(WaveState<D>& st, f4 s0, f4 s1, bool masked,
                                                int lim0, int lim1, int kg,
                                                const h8 (&vp)[D / 16], float scale_log2) {
    constexpr int NJ = D / 16;
    float sv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sv[i] = FOLD ? s0[i] : s0[i] * scale_log2;
        sv[4 + i] = FOLD ? s1[i] : s1[i] * scale_log2;
    }
    if (masked) [[unlikely]] {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (4 * kg + i >= lim0) sv[i] = -INFINITY;
            if (4 * kg + i >= lim1) sv[4 + i] = -INFINITY;
        }
    }
    float bm = max3(max3(sv[0], sv[1], sv[2]), max3(sv[3], sv[4], sv[5]), max2(sv[6], sv[7]));
    bm = max_over_kg(bm);
    if constexpr (FOLD) bm *= scale_log2;
    if (__any(bm > st.m + kLazyMargin)) {
        const float m_new = fmaxf(st.m, bm);
        const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
#pragma unroll
        for (int J = 0; J < NJ; ++J) st.acc[J] *= alpha;
        st.l *= alpha;
        st.m = m_new;
    }
    // No valid token seen yet: m is -inf and so is every sv; 0 keeps the
    // weights 0.
    const float m_use = (st.m == -INFINITY) ? 0.0f : st.m;
    const float c = m_use - kPExpLazy;
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        p[i] = __builtin_amdgcn_exp2f(FOLD ? __builtin_fmaf(sv[i], scale_log2, -c) : sv[i] - c);
    }
    st.l += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    h2 hh[4], ll[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        hh[i] = __builtin_amdgcn_cvt_pkrtz(p[2 * i], p[2 * i + 1]);
        ll[i] = __builtin_amdgcn_cvt_pkrtz(sub_h2_lo(p[2 * i], hh[i]),
                                           sub_h2_hi(p[2 * i + 1], hh[i]));
    }
    const h8 ph = __builtin_bit_cast(
        h8, __builtin_shufflevector(__builtin_shufflevector(hh[0], hh[1], 0, 1, 2, 3),
                                    __builtin_shufflevector(hh[2], hh[3], 0, 1, 2, 3), 0, 1, 2,
                                    3, 4, 5, 6, 7));
    const h8 pl = __builtin_bit_cast(
        h8, __builtin_shufflevector(__builtin_shufflevector(ll[0], ll[1], 0, 1, 2, 3),
                                    __builtin_shufflevector(ll[2], ll[3], 0, 1, 2, 3), 0, 1, 2,
                                    3, 4, 5, 6, 7));
#pragma unroll
    for (int J = 0; J < NJ; ++J) st.acc[J] = mfma16x32(vp[J], ph, st.acc[J]);
#pragma unroll
    for (int J = 0; J < NJ; ++J) st.acc[J] = mfma16x32(vp[J], pl, st.acc[J]);
}

// Steps 1 + 2 of a pair of key blocks for both row groups: S^T of the first
// block (s[0] group a, s[1] group b) and of the second (s[2], s[3]), K^T read
// from the pair's two K tiles in LDS (ktiles, the second D * 16 halves after
// the first). Four independent accumulator chains.
template <int D>
__device__ __forceinline__ void qk_pair_lds(f4 (&s)[4], int lane, const f16* ktiles,
                                            const QOperand<D>& qa, const QOperand<D>& qb) {
    constexpr int NJ = D / 16;
    constexpr int kTileHalfs = D * kBlockTokens;
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = f4{0, 0, 0, 0};
#pragma unroll
    for (int J = 0; J < NJ; J += 2) {
        const h8 k0 = cat8(read_kT(ktiles, J, lane), read_kT(ktiles, J + 1, lane));
        const h8 k1 = cat8(read_kT(ktiles + kTileHalfs, J, lane),
                           read_kT(ktiles + kTileHalfs, J + 1, lane));
        const h8 qA = cat8(qa.get(J), qa.get(J + 1));
        const h8 qB = cat8(qb.get(J), qb.get(J + 1));
        s[0] = mfma16x32(k0, qA, s[0]);
        s[1] = mfma16x32(k0, qB, s[1]);
        s[2] = mfma16x32(k1, qA, s[2]);
        s[3] = mfma16x32(k1, qB, s[3]);
    }
}

// LDSK: K tiles go straight from memory into LDS (global_load_lds, 16 bytes
// a lane; the key cache is 16-byte aligned) and come back transposed by
// ds_read_b64_tr_b16; otherwise through registers and an identity-MFMA
// transposition.
template <int D, bool FOLD, bool LDSK>
__global__ __launch_bounds__(64 * kPrefillWaves) __attribute__((amdgpu_waves_per_eu(2)))
void paged_prefill_kernel(const PrefillArgs a) {
    constexpr int NJ = D / 16;
    __shared__ int s_part[kPrefillWaves];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;
    const int kg = lane >> 4;
    // Workgroups are dealt to the 8 XCDs round-robin in launch order (x
    // fastest), so blockIdx.x % 8 names the XCD. XCD x takes the units
    // (sequence, kv head chunk) x, x + 8, x + 16, ... one after the other,
    // each unit's groups latest tokens first: the workgroups an XCD runs at
    // one time share one unit's K/V in that XCD's L2, and every XCD gets
    // the same kv heads of every sequence (equal work for any lengths when
    // the kv heads divide over the XCDs).
    const long long round =
        static_cast<long long>(blockIdx.y) + static_cast<long long>(gridDim.y) * blockIdx.z;
    const long long unit = static_cast<long long>(blockIdx.x & 7) + 8 * round;
    if (unit >= a.units) return;  // the whole workgroup: no barrier is skipped
    const int per_seq = a.Hkv * a.nhc;
    const int s = static_cast<int>(unit / per_seq);
    const int yy = static_cast<int>(unit - static_cast<long long>(s) * per_seq);
    const int kvh = yy / a.nhc;
    const int hc = yy - kvh * a.nhc;
    const int gi = a.groups - 1 - static_cast<int>(blockIdx.x >> 3);  // latest tokens first

    // start_s = sum of the lengths before s (all threads share the sum).
    int part = 0;
    for (int i = threadIdx.x; i < s; i += 64 * kPrefillWaves) part += max(a.ctx[i], 0);
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) part += __shfl_xor(part, d);
    if (lane == 0) s_part[w] = part;
    __syncthreads();
    int start = 0;
#pragma unroll
    for (int i = 0; i < kPrefillWaves; ++i) start += s_part[i];
    const int L = max(a.ctx[s], 0);

    // The wave's two groups of 16 query rows: tokens tq0 .. tq0 + tpw - 1
    // (group a) and the next tpw (group b).
    const int tq0 = (gi * kPrefillWaves + w) * 2 * a.tpw;
    if (tq0 >= L) return;
    const int tq_last = min(tq0 + 2 * a.tpw, L) - 1;

    // Query row r of group k: token tq0 + k * tpw + r / gw, head h0 + r % gw.
    const int rt = r / a.gw;
    const int rh = r - rt * a.gw;
    const int g = hc * 16 + rh;
    const int h = kvh * a.G + min(g, a.G - 1);
    const int tqa = tq0 + rt;
    const int tqb = tq0 + a.tpw + rt;
    const bool ok_a = (rt < a.tpw) && (tqa < L) && (g < a.G);
    const bool ok_b = (rt < a.tpw) && (tqb < L) && (g < a.G);
    const size_t qrow_a = (static_cast<size_t>(start) + min(tqa, L - 1)) * a.H + h;
    const size_t qrow_b = (static_cast<size_t>(start) + min(tqb, L - 1)) * a.H + h;

    QOperand<D> qa, qb;
    {
        const f16* pa_ = a.q + qrow_a * D + 4 * kg;
        const f16* pb_ = a.q + qrow_b * D + 4 * kg;
#pragma unroll
        for (int J = 0; J < NJ; ++J) {
            const h4 va = *reinterpret_cast<const h4*>(pa_ + 16 * J);
            const h4 vb = *reinterpret_cast<const h4*>(pb_ + 16 * J);
            qa.v[J] = ok_a ? va : h4{0, 0, 0, 0};
            qb.v[J] = ok_b ? vb : h4{0, 0, 0, 0};
        }
    }
    h4 ident;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ident[i] = (4 * kg + i == r) ? static_cast<f16>(1.0f) : static_cast<f16>(0.0f);
    }
    const int loff = kv_elem_offset(r, 4 * kg);
    const const_int* srow = as_const(a.slots) + start;

    WaveState<D> sa, sb;
    sa.m = sb.m = -INFINITY;
    sa.l = sb.l = 0.0f;
#pragma unroll
    for (int J = 0; J < NJ; ++J) sa.acc[J] = sb.acc[J] = f4{0, 0, 0, 0};

    // Key blocks 0 .. nkb-1, double-buffered like the decode walk: the
    // steady loop runs while at least three blocks are left (both loads of
    // an iteration are real blocks, no load depends on a condition), and the
    // last one or two are peeled off.
    const int nkb = tq_last / kBlockTokens + 1;
    auto block_at = [&](int jb) {
        return __builtin_amdgcn_readfirstlane(srow[jb * kBlockTokens]) >> kBlockShift;
    };
    auto attend = [&](int jb, int b, h4 (&k)[NJ], h4 (&v)[NJ]) {
        const int base = jb * kBlockTokens;
        const int nv = block_ok(b, a.num_blocks) ? min(kBlockTokens, L - base) : 0;
        const int lim_a = ok_a ? min(max(tqa + 1 - base, 0), nv) : 0;
        const int lim_b = ok_b ? min(max(tqb + 1 - base, 0), nv) : 0;
        attend_block_pair<D, FOLD>(sa, sb, nv, lim_a, lim_b, kg, k, v, qa, qb, ident, a.scale_log2);
    };
    if constexpr (LDSK) {
        // The walk goes by pairs of key blocks (steps of 32 keys): step t
        // covers blocks 2t and 2t + 1 (the second past nkb when nkb is odd:
        // it then contributes nothing). Per step, both K tiles go into the
        // wave's LDS and both V tiles into registers, double-buffered.
        constexpr int kTileHalfs = D * kBlockTokens;
        constexpr int kDma = kTileHalfs * 2 / (64 * 16);  // 16-byte loads per lane per tile
        // Two arrays, so the compiler can tell one step's reads from the
        // other step's loads in flight (one array made it wait for those too).
        __shared__ __align__(16) f16 s_k0[kPrefillWaves * 2 * kTileHalfs];
        __shared__ __align__(16) f16 s_k1[kPrefillWaves * 2 * kTileHalfs];
        f16* const kt0 = s_k0 + w * 2 * kTileHalfs;
        f16* const kt1 = s_k1 + w * 2 * kTileHalfs;
        const int nsteps = (nkb + 1) / 2;
        // Every LDS read of a buffer has been used by an MFMA (so it has
        // returned) before the buffer is loaded again.
        auto issue = [&](int b0, int b1, f16* dst, h8 (&vp)[NJ]) {
            const int bs0 = block_ok(b0, a.num_blocks) ? b0 : 0;
            const int bs1 = block_ok(b1, a.num_blocks) ? b1 : 0;
            const f16* k0 = a.kc + kv_tile_offset(bs0, kvh, a.Hkv, D) + 8 * lane;
            const f16* k1 = a.kc + kv_tile_offset(bs1, kvh, a.Hkv, D) + 8 * lane;
#pragma unroll
            for (int j = 0; j < kDma; ++j) {
                __builtin_amdgcn_global_load_lds(k0 + 512 * j, dst + 512 * j, 16, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < kDma; ++j) {
                __builtin_amdgcn_global_load_lds(k1 + 512 * j, dst + kTileHalfs + 512 * j, 16,
                                                 0, 0);
            }
            const f16* v0 = a.vc + kv_tile_offset(bs0, kvh, a.Hkv, D) + loff;
            const f16* v1 = a.vc + kv_tile_offset(bs1, kvh, a.Hkv, D) + loff;
#pragma unroll
            for (int J = 0; J < NJ; ++J) {
                vp[J] = cat8(load_kv<false>(v0 + kv_elem_offset(16 * J, 0)),
                             load_kv<false>(v1 + kv_elem_offset(16 * J, 0)));
            }
        };
        // Steps 3 + 4 of step t for both groups. Masks apply only where a
        // key of the step lies past the wave's first query token (the causal
        // diagonal; a partial last block and the missing second block of an
        // odd walk always do) or a block id is out of the pool: a scalar
        // test. Stale K columns (tokens >= nv) only reach the score rows of
        // those tokens, which the masks (lim <= nv) replace by -inf.
        // vw: loads issued after the pair's V loads (std::integral_constant);
        // the wait for V before PV is explicit, since the compiler's count of
        // loads into LDS mixed with loads into registers cannot be relied on.
        auto finish = [&](auto vw, int t, int b0, int b1, f4 (&sc)[4], h8 (&vp)[NJ]) {
            const int base0 = 2 * t * kBlockTokens;
            const int base1 = base0 + kBlockTokens;
            const bool ok0 = block_ok(b0, a.num_blocks);
            const bool ok1 = (2 * t + 1 < nkb) && block_ok(b1, a.num_blocks);
            const bool masked = (base0 + 2 * kBlockTokens - 1 > tq0) || !ok0 || !ok1;
            const int nv0 = ok0 ? min(kBlockTokens, L - base0) : 0;
            const int nv1 = ok1 ? min(kBlockTokens, L - base1) : 0;
            const int la0 = ok_a ? min(max(tqa + 1 - base0, 0), nv0) : 0;
            const int la1 = ok_a ? min(max(tqa + 1 - base1, 0), nv1) : 0;
            const int lb0 = ok_b ? min(max(tqb + 1 - base0, 0), nv0) : 0;
            const int lb1 = ok_b ? min(max(tqb + 1 - base1, 0), nv1) : 0;
            wait_vm<decltype(vw)::value>();
            mask_v_pair<D>(nv0, nv1, kg, vp);
            softmax_pv_pair<D, FOLD>(sa, sc[0], sc[2], masked, la0, la1, kg, vp, a.scale_log2);
            softmax_pv_pair<D, FOLD>(sb, sc[1], sc[3], masked, lb0, lb1, kg, vp, a.scale_log2);
        };
        // Block ids without scalar loads in the walk (those share their wait
        // counter with the LDS reads, and every K^T read would wait for
        // them): chunks of 64 ids (the first slots of blocks 64 c .. 64 c +
        // 63 of the walk, clamped to block nkb - 1) go into the wave's LDS by
        // direct loads, chunk c + 1 while the walk is in chunk c, and a step
        // reads the ids of its two blocks with one LDS read. A chunk is
        // loaded 64 blocks before its first read; the waits of the steps in
        // between (each at most 2 * (2 kDma + 2 NJ) loads behind) retire it.
        __shared__ __align__(16) int s_ids[kPrefillWaves][2][64];
        auto load_chunk = [&](int c) {
            const int j = min(64 * c + lane, nkb - 1);
            __builtin_amdgcn_global_load_lds(srow + j * kBlockTokens, &s_ids[w][c & 1][0], 4, 0,
                                             0);
        };
        load_chunk(0);
        load_chunk(1);
        __builtin_amdgcn_s_waitcnt(0);
        int chunk = 0;
        // Ids of step t's two blocks (steps asked for in increasing order).
        auto ids_of = [&](int t, int& b0, int& b1) {
            const int j = min(2 * t, (nkb - 1) & ~1);
            if ((j >> 6) != chunk) {
                chunk = j >> 6;
                load_chunk(chunk + 1);
            }
            const int2 v = *reinterpret_cast<const int2*>(&s_ids[w][chunk & 1][j & 63]);
            b0 = __builtin_amdgcn_readfirstlane(v.x) >> kBlockShift;
            b1 = __builtin_amdgcn_readfirstlane(v.y) >> kBlockShift;
        };
        // Loads in flight behind a step's K tiles: its V tiles, then the next
        // step's K and V tiles (when there is a next step); behind its V
        // tiles, the next step's or nothing.
        constexpr int kBehindNext = 2 * NJ + 2 * kDma + 2 * NJ;
        constexpr int kBehindLast = 2 * NJ;
        const std::integral_constant<int, 2 * kDma + 2 * NJ> v_next;
        const std::integral_constant<int, 0> v_last;
        h8 vA[NJ], vB[NJ];
        f4 sc[4];
        auto qk_then_ids = [&](const f16* kt, int t_ids, int& n0, int& n1) {
            ids_of(t_ids, n0, n1);
            qk_pair_lds<D>(sc, lane, kt, qa, qb);
        };
        int tA = 0;
        int bA0, bA1, bN0, bN1;  // step tA, step tA + 1 (clamped)
        ids_of(0, bA0, bA1);
        ids_of(1, bN0, bN1);
        issue(bA0, bA1, kt0, vA);
        int left = nsteps;
        for (; left > 2; left -= 2) {
            const int tB = tA + 1;
            const int bB0 = bN0, bB1 = bN1;
            issue(bB0, bB1, kt1, vB);
            wait_vm<kBehindNext>();
            qk_then_ids(kt0, tB + 1, bN0, bN1);
            finish(v_next, tA, bA0, bA1, sc, vA);
            tA = tB + 1;
            bA0 = bN0;
            bA1 = bN1;
            issue(bA0, bA1, kt0, vA);
            wait_vm<kBehindNext>();
            qk_then_ids(kt1, tA + 1, bN0, bN1);
            finish(v_next, tB, bB0, bB1, sc, vB);
        }
        if (left == 2) {
            const int tB = tA + 1;
            issue(bN0, bN1, kt1, vB);
            wait_vm<kBehindNext>();
            qk_pair_lds<D>(sc, lane, kt0, qa, qb);
            finish(v_next, tA, bA0, bA1, sc, vA);
            wait_vm<kBehindLast>();
            qk_pair_lds<D>(sc, lane, kt1, qa, qb);
            finish(v_last, tB, bN0, bN1, sc, vB);
        } else {
            wait_vm<kBehindLast>();
            qk_pair_lds<D>(sc, lane, kt0, qa, qb);
            finish(v_last, tA, bA0, bA1, sc, vA);
        }
        // No load may still be writing this wave's LDS when it exits.
        __builtin_amdgcn_s_waitcnt(0);
    } else {
        // The next block's id (a scalar load of its first slot) is fetched
        // one block ahead, so no load waits on it; ids past the prompt's
        // last block are clamped to it.
        h4 kA[NJ], vA[NJ], kB[NJ], vB[NJ];
        int jA = 0;
        int bA = block_at(0);
        int bNext = block_at(min(1, nkb - 1));  // block jA + 1
        load_tile<D, false>(a.kc, a.vc, a.Hkv, a.num_blocks, bA, kvh, loff, kA, vA);
        int left = nkb;
        for (; left > 2; left -= 2) {
            const int jB = jA + 1;
            const int bB = bNext;
            load_tile<D, false>(a.kc, a.vc, a.Hkv, a.num_blocks, bB, kvh, loff, kB, vB);
            bNext = block_at(jB + 1);
            attend(jA, bA, kA, vA);
            jA = jB + 1;
            bA = bNext;
            load_tile<D, false>(a.kc, a.vc, a.Hkv, a.num_blocks, bA, kvh, loff, kA, vA);
            bNext = block_at(min(jA + 1, nkb - 1));
            attend(jB, bB, kB, vB);
        }
        if (left == 2) {
            const int jB = jA + 1;
            const int bB = bNext;
            load_tile<D, false>(a.kc, a.vc, a.Hkv, a.num_blocks, bB, kvh, loff, kB, vB);
            attend(jA, bA, kA, vA);
            attend(jB, bB, kB, vB);
        } else {
            attend(jA, bA, kA, vA);
        }
    }

    auto store = [&](const WaveState<D>& st, bool ok, size_t qrow) {
        float l_run = st.l;
        l_run = sum_over_kg(l_run);
        if (!ok) return;
        const float inv = (l_run > 0.0f) ? 1.0f / l_run : 0.0f;
        f16* op = a.out + qrow * D + 4 * kg;
#pragma unroll
        for (int J = 0; J < NJ; ++J) {
            h4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = static_cast<f16>(st.acc[J][i] * inv);
            *reinterpret_cast<h4*>(op + 16 * J) = o;
        }
    };
    store(sa, ok_a, qrow_a);
    store(sb, ok_b, qrow_b);
}

int prefill(const char* who, void* out, const void* q, const void* kc, const void* vc,
            const int* slots, const int* ctx, float scale, long long S, long long H, long long Hkv,
            long long D, long long BS, long long max_len, int num_blocks, hipStream_t stream) {
    if (S < 0 || H <= 0 || Hkv <= 0 || D <= 0 || BS <= 0 || max_len < 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                    "%s: num_seqs=%lld num_heads=%lld num_kv_heads=%lld head_dim=%lld "
                    "block_size=%lld max_context_len=%lld", who, S, H, Hkv, D, BS, max_len);
    }
    if (H % Hkv != 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: num_heads %lld not a multiple of num_kv_heads %lld",
                    who, H, Hkv);
    }
    if ((D != 64 && D != 128) || BS != kBlockTokens) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: head_dim=%lld block_size=%lld (supported: 64/128, 16)",
                    who, D, BS);
    }
    if (S > 65535 || H > 65535 || max_len > (1LL << 30)) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: num_seqs=%lld num_heads=%lld max_context_len=%lld",
                    who, S, H, max_len);
    }
    if (S > 0 && max_len > 0 && (!out || !q || !kc || !vc || !slots || !ctx)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    if (!aligned(out, 8) || !aligned(q, 8) || !aligned(kc, 8) || !aligned(vc, 8) ||
        !aligned(slots, 4) || !aligned(ctx, 4)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: misaligned pointer", who);
    }
    // Workgroups per (sequence, kv head chunk): x = 8 of them per XCD round
    // times 64 * kPrefillWaves threads must stay below 2^32 threads.
    const long long G = H / Hkv;
    const long long tpw = 16 / (G < 16 ? G : 16);
    const long long per_wg = static_cast<long long>(kPrefillWaves) * 2 * tpw;
    const long long groups = (max_len + per_wg - 1) / per_wg;
    if (groups >= (1LL << 21)) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED,
                    "%s: max_context_len=%lld needs %lld workgroups per sequence (limit 2^21)", who,
                    max_len, groups);
    }
    int rc = require_device();
    if (rc != SWIFTLLM_OK) return rc;
    if (S == 0 || max_len == 0) return ok();
    PrefillArgs a{};
    a.out = static_cast<f16*>(out);
    a.q = static_cast<const f16*>(q);
    a.kc = static_cast<const f16*>(kc);
    a.vc = static_cast<const f16*>(vc);
    a.slots = slots;
    a.ctx = ctx;
    a.scale_log2 = static_cast<float>(static_cast<double>(scale) * static_cast<double>(kLog2e));
    a.S = static_cast<int>(S);
    a.H = static_cast<int>(H);
    a.Hkv = static_cast<int>(Hkv);
    a.G = a.H / a.Hkv;
    a.nhc = (a.G + 15) / 16;
    a.gw = a.G < 16 ? a.G : 16;
    a.tpw = 16 / a.gw;
    a.groups = static_cast<int>(groups);
    a.units = S * static_cast<long long>(a.Hkv) * a.nhc;
    a.num_blocks = num_blocks;
    const long long rounds = (a.units + 7) / 8;
    const long long gy = rounds < 65535 ? rounds : 65535;
    const dim3 grid(static_cast<unsigned>(8 * a.groups), static_cast<unsigned>(gy),
                    static_cast<unsigned>((rounds + gy - 1) / gy));
    const dim3 block(64 * kPrefillWaves);
    const bool fold = a.scale_log2 > 0.0f;
    const bool ldsk = aligned(kc, 16);
    using K = void (*)(PrefillArgs);
    static const K kernels[2][2][2] = {
        {{paged_prefill_kernel<64, false, false>, paged_prefill_kernel<64, false, true>},
         {paged_prefill_kernel<64, true, false>, paged_prefill_kernel<64, true, true>}},
        {{paged_prefill_kernel<128, false, false>, paged_prefill_kernel<128, false, true>},
         {paged_prefill_kernel<128, true, false>, paged_prefill_kernel<128, true, true>}}};
    const hipError_t err =
        launch(kernels[D == 128][fold][ldsk], grid, block, 0, stream, a);
    return launched(err, who);
}

}  // namespace
}  // namespace swiftllm

using namespace swiftllm;

extern "C" {

int swiftllm_hip_paged_attention_prefill(void* output, const void* query, const void* key_cache,
                                         const void* value_cache, const int32_t* slot_mapping,
                                         const int32_t* context_lens,
                                         const swiftllm_paged_attention_params* p,
                                         hipStream_t stream) {
    const char* who = "swiftllm_hip_paged_attention_prefill";
    if (p == nullptr) return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null params", who);
    const size_t lim = 0x7fffffff;
    if (p->num_seqs > lim || p->num_heads > lim || p->num_kv_heads > lim || p->head_dim > lim ||
        p->block_size > lim || p->max_context_len > lim) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: parameter out of range", who);
    }
    return prefill(who, output, query, key_cache, value_cache, slot_mapping, context_lens, p->scale,
                   static_cast<long long>(p->num_seqs), static_cast<long long>(p->num_heads),
                   static_cast<long long>(p->num_kv_heads), static_cast<long long>(p->head_dim),
                   static_cast<long long>(p->block_size), static_cast<long long>(p->max_context_len),
                   0, stream);
}

int swiftllm_hip_launch_paged_prefill(void* output, const void* query, const void* key_cache,
                                      const void* value_cache, const int32_t* slot_mapping,
                                      const int32_t* context_lens, float scale, int num_seqs,
                                      int num_heads, int num_kv_heads, int head_dim, int block_size,
                                      int max_context_len, int num_blocks, hipStream_t stream) {
    return prefill("swiftllm_hip_launch_paged_prefill", output, query, key_cache, value_cache,
                   slot_mapping, context_lens, scale, num_seqs, num_heads, num_kv_heads, head_dim,
                   block_size, max_context_len, num_blocks, stream);
}

}  // extern "C"
