// Paged-attention decode for gfx950 (CDNA4).
//
// Contract (paged_attention.cu:35-137 is the reference's text; its output
// stage is a stub, so the behaviour below is the textbook attention its
// comments and indexing describe):
//   for sequence s, query head h, kv head kvh = h / (H / Hkv)   (cu:52)
//   L = context_lens[s]; token j lives in block bt[s, j / 16] at offset j % 16
//   logit_j = scale * sum_d q[s,h,d] * K(b, kvh, d, j % 16)     (cu:92-96)
//   out[s,h,:] = sum_j softmax(logit)_j * V(b, kvh, :, j % 16)  (cu:113-135)
// fp16 in and out, fp32 accumulation; L <= 0 writes zeros.
//
// Work decomposition. One workgroup serves every query head of one kv head
// (up to 16 per workgroup), so each K/V tile is read from HBM once. The
// reference grid (S, H) (cu:248) re-reads it H/Hkv times. The waves of a
// workgroup take the blocks of its token range round-robin; the range is the
// whole context (single pass) or one partition of it (split-K). Each wave
// keeps a running max, sum and output for its blocks; the waves merge through
// LDS. Split-K partitions leave (max, sum, output) in a workspace and a
// second kernel does the rescaled reduce (the kernel boundary makes the
// partials visible; an in-kernel last-arriver reduce would need device-scope
// fences, which write back and invalidate the whole L2 on this GPU).
//
// Per 16-token block, each wave runs the whole computation on the matrix
// cores with v_mfma_f32_16x16x16_f16 (the group of query heads is the N = 16
// side, zero-padded):
//   1. K tile rows 16J..16J+15 arrive with tokens contiguous ([d][t]); an
//      MFMA against a 0/1 identity operand returns the same values in the
//      transposed ([t][d]) register layout, exactly (one product per output).
//   2. S^T[t][g] = sum_d K^T[t][d] Q^T[d][g]          (D/16 MFMAs)
//   3. Online softmax in fp32 on the S^T accumulator; the 4 token rows of a
//      head live in lanes l, l^16, l^32, l^48, so the block max is two xor
//      shuffles.
//   4. O^T[d][g] += V[d][t] P^T[t][g] with V in its stored layout. P is fed as
//      an fp16 hi part plus an fp16 lo part (two MFMAs), which keeps ~22 bits
//      of each probability; P is computed as 2^15 * exp2(s - m) so both parts
//      stay in fp16's normal range.

#include <algorithm>
#include <cmath>
#include <mutex>

#include "attention_core.hpp"

namespace swiftllm {
namespace {

using namespace attn;

struct DecodeArgs {
    f16* out;
    const f16* q;
    const f16* kc;
    const f16* vc;
    const int* bt;
    const int* ctx;
    float* ws_max;       // [S][H][MP]         log2-domain max logit
    float* ws_sum;       // [S][H][MP]         sum of 2^15 * exp2(s - max)
    float* ws_out;       // [S][H][MP][D]      normalised partial output
    float scale_log2;    // scale * log2(e)
    int H;
    int Hkv;
    int G;            // query heads per kv head
    int nhc;          // head chunks of 16 per kv head
    int MB;           // max_num_blocks_per_seq (row stride of bt)
    int num_blocks;   // bound on block ids; <= 0: unbounded
    int part_blocks;  // blocks per partition; 0: single pass
    int MP;           // partitions per sequence in the workspace
    int S;            // sequences
    int snake;        // > 0: single-pass item order in snake rounds of this many
    // Partition streams (paged_partition_stream_kernel) only:
    float* frag;      // [W][kFragHead + gstride * D]: the piece a wave's range starts with
    int* meta;        // [0] blocks per team q, [1] teams, [2 .. S + 2] block prefix
    int W;            // waves in the grid
    int stage_off;    // ints of dynamic LDS before the waves' partial slots
};

// Attends `count` blocks of one sequence: logical blocks first,
// first + stride, ... Blocks are double-buffered in registers, so the next
// block's loads are in flight while one is attended. The steady-state loop
// runs while at least three blocks are left: both of its loads are real
// blocks, no load depends on a condition, and the compiler's wait counts stay
// exact. The last one or two blocks are peeled off, so no tile is read twice.
template <int D>
__device__ __forceinline__ void attend_blocks(WaveState<D>& st, const const_int* btrow, int first,
                                              int stride, int count, int L, const f16* kc,
                                              const f16* vc, int Hkv, int num_blocks, int kvh,
                                              int loff, int kg, const QOperand<D>& qB, h4 ident,
                                              float scale_log2) {
    constexpr int NJ = D / 16;
    if (count <= 0) return;
    auto block_at = [&](int j) { return __builtin_amdgcn_readfirstlane(btrow[j]); };
    auto valid_of = [&](int j, int b) {
        return block_ok(b, num_blocks) ? min(kBlockTokens, L - j * kBlockTokens) : 0;
    };
    h4 kA[NJ], vA[NJ], kB[NJ], vB[NJ];
    int jA = first;
    int bA = block_at(jA);
    load_tile<D>(kc, vc, Hkv, num_blocks, bA, kvh, loff, kA, vA);
    int left = count;
    for (; left > 2; left -= 2) {
        const int jB = jA + stride;
        const int bB = block_at(jB);
        load_tile<D>(kc, vc, Hkv, num_blocks, bB, kvh, loff, kB, vB);
        attend_block<D>(st, valid_of(jA, bA), kg, kA, vA, qB, ident, scale_log2);
        jA = jB + stride;
        bA = block_at(jA);
        load_tile<D>(kc, vc, Hkv, num_blocks, bA, kvh, loff, kA, vA);
        attend_block<D>(st, valid_of(jB, bB), kg, kB, vB, qB, ident, scale_log2);
    }
    if (left == 2) {
        const int jB = jA + stride;
        const int bB = block_at(jB);
        load_tile<D>(kc, vc, Hkv, num_blocks, bB, kvh, loff, kB, vB);
        attend_block<D>(st, valid_of(jA, bA), kg, kA, vA, qB, ident, scale_log2);
        attend_block<D>(st, valid_of(jB, bB), kg, kB, vB, qB, ident, scale_log2);
    } else {
        attend_block<D>(st, valid_of(jA, bA), kg, kA, vA, qB, ident, scale_log2);
    }
}

// The sequence with the r-th longest context (ties by index), found by every
// workgroup of a single-pass grid that is resident all at once (the snake
// order below). Each thread ranks S / 256 sequences against all S, so the
// cost grows as S^2: measured on MI355X with the ranking in every grid,
// 1024 sequences of 32-128 tokens took 1324 us against 67 us in plain order,
// and 256 of them 39.7 against 18.8 us. So only batches of up to
// kLptMaxSeqs sequences are ranked (at most 128 compares a thread), and larger
// grids run in sequence order, which the dispatcher balances as workgroups
// finish.
constexpr int kLptMaxSeqs = 128;

__device__ __forceinline__ int sequence_for_block(const int* ctx, int S, int r) {
    if (S > kLptMaxSeqs) return r;
    __shared__ int s_ctx[kLptMaxSeqs > 0 ? kLptMaxSeqs : 1];
    __shared__ int s_seq;
    for (int c = threadIdx.x; c < S; c += blockDim.x) s_ctx[c] = ctx[c];
    if (threadIdx.x == 0) s_seq = r;
    __syncthreads();
    for (int c = threadIdx.x; c < S; c += blockDim.x) {
        const int lc = s_ctx[c];
        int rank = 0;
        for (int o = 0; o < S; ++o) {
            const int lo = s_ctx[o];
            rank += (lo > lc) || (lo == lc && o < c);
        }
        if (rank == r) s_seq = c;
    }
    __syncthreads();
    return s_seq;
}

// Dynamic LDS of decode_item's wave merge, in floats: per wave 16 maxima,
// 16 sums and gstride = min(G, 16) rows of D partial outputs.
template <int D, int NW>
__host__ __device__ constexpr int merge_lds_floats(int G) {
    return NW * 32 + NW * (G < 16 ? G : 16) * D;
}

// Bytes of the partition kernel's item list for S sequences (int prefix of
// S + 1 entries, 16-bit sequence list of S), rounded to 16.
__host__ __device__ constexpr size_t part_list_lds_bytes(int S) {
    return ((static_cast<size_t>(S) + 1) * 4 + static_cast<size_t>(S) * 2 + 15) / 16 * 16;
}

// One (sequence, kv head, head chunk, partition) item. The NW waves of the
// workgroup take the item's blocks round-robin and merge through LDS; the
// result is the output (single pass, or a sequence with one partition) or a
// split-K partial. Every thread of the workgroup calls it with the same item.
template <int D, int NW>
__device__ __forceinline__ void decode_item(const DecodeArgs& a, int s, int kvh, int hc,
                                            int part) {
    constexpr int NJ = D / 16;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;   // MFMA column / row-in-slice index
    const int kg = lane >> 4;  // MFMA k-group: 4 consecutive k per lane

    const int g0 = hc * 16;
    const int gn = min(16, a.G - g0);  // query heads served here
    const int gstride = min(16, a.G);  // LDS rows per wave
    const int h0 = kvh * a.G + g0;

    int L = a.ctx[s];
    L = max(L, 0);
    const int nblk = min((L + kBlockTokens - 1) / kBlockTokens, a.MB);
    L = min(L, nblk * kBlockTokens);
    int nparts, jb0, jb1;
    if (a.part_blocks > 0) {
        nparts = (nblk + a.part_blocks - 1) / a.part_blocks;
        jb0 = part * a.part_blocks;
        jb1 = min(nblk, jb0 + a.part_blocks);
    } else {
        nparts = 1;
        jb0 = 0;
        jb1 = nblk;
    }
    if (nblk == 0) {
        if (part == 0) {
            for (int i = threadIdx.x; i < gn * D; i += NW * 64) {
                a.out[(static_cast<size_t>(s) * a.H + h0) * D + i] = static_cast<f16>(0.0f);
            }
        }
        return;
    }
    if (part >= nparts) return;

    QOperand<D> qB;
    {
        const f16* qp = a.q + (static_cast<size_t>(s) * a.H + h0 + min(r, gn - 1)) * D + 4 * kg;
#pragma unroll
        for (int J = 0; J < NJ; ++J) {
            const h4 v = *reinterpret_cast<const h4*>(qp + 16 * J);
            qB.v[J] = (r < gn) ? v : h4{0, 0, 0, 0};
        }
    }
    // Identity operand of step 1: B[k = 4kg + i][n = r] = (k == n).
    h4 ident;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ident[i] = (4 * kg + i == r) ? static_cast<f16>(1.0f) : static_cast<f16>(0.0f);
    }
    // Lane (r, kg) loads tile row 16J + r, tokens 4kg .. 4kg + 3.
    const int loff = kv_elem_offset(r, 4 * kg);
    const const_int* btrow = as_const(a.bt) + static_cast<size_t>(s) * a.MB;

    WaveState<D> st;
    st.m = -INFINITY;
    st.l = 0.0f;
#pragma unroll
    for (int J = 0; J < NJ; ++J) st.acc[J] = f4{0, 0, 0, 0};

    // Blocks jb0 + w, jb0 + w + NW, ... of this wave.
    const int first = jb0 + w;
    const int nbw = (jb1 > first) ? (jb1 - first + NW - 1) / NW : 0;
    attend_blocks<D>(st, btrow, first, NW, nbw, L, a.kc, a.vc, a.Hkv, a.num_blocks, kvh, loff, kg,
                     qB, ident, a.scale_log2);
    float m_run = st.m;
    float l_run = st.l;
    f4 (&acc)[NJ] = st.acc;
    // Per-lane partial sums cover tokens 4kg..4kg+3 of every block.
    l_run = sum_over_kg(l_run);

    // Merge the waves of this workgroup.
    extern __shared__ __align__(16) float smem[];
    float* sm_m = smem;            // [NW][16]
    float* sm_l = smem + NW * 16;  // [NW][16]
    float* sm_o = smem + NW * 32;  // [NW][gstride][D]
    if (kg == 0) {
        sm_m[w * 16 + r] = m_run;
        sm_l[w * 16 + r] = l_run;
    }
    if (r < gn) {
#pragma unroll
        for (int J = 0; J < NJ; ++J) {
            *reinterpret_cast<f4*>(sm_o + static_cast<size_t>(w * gstride + r) * D + 16 * J + 4 * kg) = acc[J];
        }
    }
    __syncthreads();

    const bool direct = (nparts == 1);
    for (int idx = threadIdx.x; idx < gn * D; idx += NW * 64) {
        const int g = idx / D;
        const int d = idx - g * D;
        float M = -INFINITY;
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) M = fmaxf(M, sm_m[w2 * 16 + g]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) {
            const float mw = sm_m[w2 * 16 + g];
            const float f = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
            num += f * sm_o[static_cast<size_t>(w2 * gstride + g) * D + d];
            den += f * sm_l[w2 * 16 + g];
        }
        const int h = h0 + g;
        const float o = (den > 0.0f) ? num / den : 0.0f;
        if (direct) {
            a.out[(static_cast<size_t>(s) * a.H + h) * D + d] = static_cast<f16>(o);
        } else {
            const size_t pi = (static_cast<size_t>(s) * a.H + h) * a.MP + part;
            a.ws_out[pi * D + d] = o;
            if (d == 0) {
                a.ws_max[pi] = M;
                a.ws_sum[pi] = den;
            }
        }
    }
}


// At least two waves per SIMD: caps the registers (at 157 VGPRs for D=128 the
// kernel fits three waves per SIMD), so several workgroups share a CU.
template <int D, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
void paged_decode_kernel(const DecodeArgs a) {
    int kvh, hc, s;
    if (a.snake > 0) {
        // Single pass, whole grid resident: workgroup i takes item
        // snake(i) of the longest-first list of (sequence, kv head, head
        // chunk) items, where the list is cut into rounds of `snake`
        // items and every other round runs backwards. Workgroups i and
        // i + snake, which the dispatcher puts on the same CU, then pair a
        // long sequence with a short one.
        const int HC = gridDim.y;
        const int i = blockIdx.z * HC + blockIdx.y;
        const int k = i / a.snake;
        const int pos = i - k * a.snake;
        const int rlen = min(a.snake, static_cast<int>(gridDim.z) * HC - k * a.snake);
        const int item = k * a.snake + ((k & 1) ? (rlen - 1 - pos) : pos);
        const int sub = item % HC;
        kvh = sub / a.nhc;
        hc = sub - kvh * a.nhc;
        s = sequence_for_block(a.ctx, gridDim.z, item / HC);
    } else {
        kvh = blockIdx.y / a.nhc;
        hc = blockIdx.y - kvh * a.nhc;
        s = blockIdx.z;
    }
    decode_item<D, NW>(a, s, kvh, hc, 0);
}

// Split-K partitions. The items are the real (sequence, partition) pairs
// times the kv-head chunks, longest first: every workgroup lists them in LDS
// and walks items blockIdx.x, + gridDim.x, ... The grid is sized to the
// resident workgroups, not to the worst case of every sequence, so a ragged
// batch launches no empty workgroups (a grid over max_num_blocks_per_seq
// would be mostly empty). Workgroups start in blockIdx order, so the order of
// the list is the order the items start in: first every full partition
// (part_blocks blocks), then the last, partial partition of each sequence in
// kLptClasses length classes, longest first (an empty sequence's item, which
// writes zeros, is a partial of length 0). Measured with the gather kernel
// of libswiftllm_ceilings on config 4's items at 1024-token partitions:
// 151 us longest first against 166 us in sequence order.
//
// The item of one list position is run by several workgroups (one per kv-head
// chunk), each with its own copy of the list, so the list must come out the
// same in every workgroup: within a class the partials keep sequence order,
// placed by prefix sums, never by the order atomics happen to land in.
// Batches of more than kPartMaxSeqs sequences take one item per workgroup
// over the full grid.
constexpr int kPartMaxSeqs = 4096;
constexpr int kLptClasses = 16;  // counted in 16-bit fields, two per int

template <int D, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(3)))
void paged_partition_kernel(const DecodeArgs a) {
    const int HC = a.Hkv * a.nhc;
    if (a.S > kPartMaxSeqs) {
        const int it = blockIdx.x;
        const int part = it % a.MP;
        const int sub = (it / a.MP) % HC;
        const int s = it / (a.MP * HC);
        if (s < a.S) decode_item<D, NW>(a, s, sub / a.nhc, sub % a.nhc, part);
        return;
    }
    constexpr int kPacked = kLptClasses / 2;
    // The item list sits in dynamic LDS after decode_item's merge area,
    // sized by the host for this batch (part_list_lds_bytes): s_pre[S + 1]
    // exclusive prefix of full partitions, s_part[S] sequences with a
    // partial partition, longest first.
    extern __shared__ __align__(16) float smem[];
    int* s_pre = reinterpret_cast<int*>(smem + merge_lds_floats<D, NW>(a.G));
    unsigned short* s_part = reinterpret_cast<unsigned short*>(s_pre + a.S + 1);
    __shared__ int s_wpk[NW][kPacked];               // per-wave class counts of a chunk
    __shared__ int s_cls[kLptClasses];               // next list position of each class
    __shared__ int s_wave[NW];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int pb = a.part_blocks;
    auto nblk_of = [&](int sq) {
        const int L = max(a.ctx[sq], 0);
        return min((L + kBlockTokens - 1) / kBlockTokens, a.MB);
    };
    // Class of a sequence's partial partition (0 = longest), or -1 when its
    // last partition is full.
    auto class_of = [&](int nblk) {
        const int rem = nblk - (nblk / pb) * pb;
        if (rem == 0 && nblk > 0) return -1;
        return kLptClasses - 1 - static_cast<int>((static_cast<long long>(rem) * kLptClasses) / pb);
    };
    // Inclusive scan over the wave of 8 packed ints (two 16-bit class counts
    // each; a workgroup chunk holds at most 256 of any class).
    auto wave_scan8 = [&](int (&x)[kPacked]) {
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
#pragma unroll
            for (int i = 0; i < kPacked; ++i) {
                const int y = __shfl_up(x[i], d);
                if (lane >= d) x[i] += y;
            }
        }
    };
    auto field = [](const int (&x)[kPacked], int c) { return (x[c >> 1] >> (16 * (c & 1))) & 0xffff; };
    // Pass 1: full partitions per sequence (exclusive prefix, in chunks of
    // the workgroup) and partials per class.
    int carry = 0;
    int cls_total[kPacked] = {};
    for (int c0 = 0; c0 < a.S; c0 += NW * 64) {
        const int sq = c0 + static_cast<int>(threadIdx.x);
        int v = 0;
        int pk[kPacked] = {};
        if (sq < a.S) {
            const int nblk = nblk_of(sq);
            v = nblk / pb;
            const int c = class_of(nblk);
            if (c >= 0) pk[c >> 1] = 1 << (16 * (c & 1));
        }
        int x = v;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int y = __shfl_up(x, d);
            if (lane >= d) x += y;
        }
        wave_scan8(pk);
        if (lane == 63) {
            s_wave[w] = x;
#pragma unroll
            for (int i = 0; i < kPacked; ++i) s_wpk[w][i] = pk[i];
        }
        __syncthreads();
        int before = carry, chunk = 0;
        for (int i = 0; i < NW; ++i) {
            before += (i < w) ? s_wave[i] : 0;
            chunk += s_wave[i];
#pragma unroll
            for (int j = 0; j < kPacked; ++j) cls_total[j] += s_wpk[i][j];
        }
        if (sq < a.S) s_pre[sq] = before + x - v;
        carry += chunk;
        __syncthreads();
    }
    // First list position of each class (every thread holds the totals).
    if (threadIdx.x == 0) {
        int pos = 0;
        for (int c = 0; c < kLptClasses; ++c) {
            s_cls[c] = pos;
            pos += field(cls_total, c);
        }
        s_pre[a.S] = carry;
    }
    int npartial = 0;
#pragma unroll
    for (int c = 0; c < kLptClasses; ++c) npartial += field(cls_total, c);
    __syncthreads();
    // Pass 2: each partial at its class's next position, in sequence order:
    // the position is the class cursor plus the number of lower-numbered
    // sequences of the same class in this chunk.
    for (int c0 = 0; c0 < a.S; c0 += NW * 64) {
        const int sq = c0 + static_cast<int>(threadIdx.x);
        int c = -1;
        int pk[kPacked] = {};
        if (sq < a.S) {
            c = class_of(nblk_of(sq));
            if (c >= 0) pk[c >> 1] = 1 << (16 * (c & 1));
        }
        int incl[kPacked];
#pragma unroll
        for (int i = 0; i < kPacked; ++i) incl[i] = pk[i];
        wave_scan8(incl);
        if (lane == 63) {
#pragma unroll
            for (int i = 0; i < kPacked; ++i) s_wpk[w][i] = incl[i];
        }
        __syncthreads();
        if (c >= 0) {
            int rank = field(incl, c) - 1;
            for (int i = 0; i < w; ++i) rank += (s_wpk[i][c >> 1] >> (16 * (c & 1))) & 0xffff;
            s_part[s_cls[c] + rank] = static_cast<unsigned short>(sq);
        }
        __syncthreads();
        if (threadIdx.x < kLptClasses) {
            int n = 0;
            for (int i = 0; i < NW; ++i) n += (s_wpk[i][threadIdx.x >> 1] >> (16 * (threadIdx.x & 1))) & 0xffff;
            s_cls[threadIdx.x] += n;
        }
        __syncthreads();
    }
    const int nfull = carry;
    const int total = (nfull + npartial) * HC;
    for (int it = blockIdx.x; it < total; it += gridDim.x) {
        const int pidx = it / HC;
        const int sub = it - pidx * HC;
        int sq, part;
        if (pidx < nfull) {
            int lo = 0, hi = a.S;  // s_pre[lo] <= pidx < s_pre[hi]
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (s_pre[mid] <= pidx) lo = mid; else hi = mid;
            }
            sq = lo;
            part = pidx - s_pre[lo];
        } else {
            sq = s_part[pidx - nfull];
            part = s_pre[sq + 1] - s_pre[sq];  // after the full ones
        }
        decode_item<D, NW>(a, sq, sub / a.nhc, sub % a.nhc, part);
        __syncthreads();  // the item's LDS is free again
    }
}

// Rescaled combine of P fragments of one query head: fragment p holds a max
// m_p (log2 domain), a sum l_p and a normalised partial output o_p[D], and
// out[d] = sum_p w_p o_p[d] / sum_p w_p with w_p = exp2(m_p - M) l_p,
// M = max_p m_p. Accessors: fm(p), fl(p) and fo(p) (pointer to o_p, 8-byte
// aligned); out(d, v) stores one output.
// One wave combines a head: no barriers, lane l owns outputs
// [l * D / 64, (l + 1) * D / 64), so every fragment row is one coalesced load.
// The rows of the first CH fragments are loaded before the headers (max and
// sum) of the first 64, all in flight together, so the combine pays one
// memory latency per CH fragments; rows past the last fragment re-read it
// and get weight 0. The weights live one per lane and are broadcast with
// readlane; the rows are added in fragment order.
template <int D>
__device__ __forceinline__ void load_row(const float* p, float (&v)[D / 64]) {
    if constexpr (D == 128) {
        const float2 x = *reinterpret_cast<const float2*>(p);
        v[0] = x.x;
        v[1] = x.y;
    } else {
        v[0] = *p;
    }
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

template <int D, int CH, typename FM, typename FL, typename FO, typename OUT>
__device__ __forceinline__ void combine_head_wave(int P, FM fm, FL fl, FO fo, OUT out) {
    static_assert(CH == 16 || CH == 64, "rows per load batch");
    constexpr int DL = D / 64;
    const int lane = threadIdx.x & 63;
    if (P <= 0) {
#pragma unroll
        for (int j = 0; j < DL; ++j) out(lane * DL + j, 0.0f);
        return;
    }
    float v[CH][DL];
#pragma unroll
    for (int i = 0; i < CH; ++i) load_row<D>(fo(min(i, P - 1)) + lane * DL, v[i]);
    const float m0 = lane < P ? fm(lane) : -INFINITY;
    const float l0 = lane < P ? fl(lane) : 0.0f;
    float M = m0;
    for (int p = 64 + lane; p < P; p += 64) M = fmaxf(M, fm(p));
    M = wave_max(M);
    float acc[DL];
#pragma unroll
    for (int j = 0; j < DL; ++j) acc[j] = 0.0f;
    float den = 0.0f;
    float w = 0.0f;
    for (int c0 = 0; c0 < P; c0 += CH) {
        if ((c0 & 63) == 0) {
            // Weights of fragments c0 .. c0 + 63, fragment c0 + l on lane l.
            if (c0 == 0) {
                w = (m0 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m0 - M) * l0;
            } else {
                const int p = c0 + lane;
                const float mp = p < P ? fm(p) : -INFINITY;
                w = (mp == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mp - M) * fl(p);
            }
            den += w;
        }
        if (c0 > 0) {
#pragma unroll
            for (int i = 0; i < CH; ++i) load_row<D>(fo(min(c0 + i, P - 1)) + lane * DL, v[i]);
        }
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const float wi = readlane_f(w, (c0 & 63) + i);
#pragma unroll
            for (int j = 0; j < DL; ++j) acc[j] += wi * v[i][j];
        }
    }
    den = wave_sum(den);
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
#pragma unroll
    for (int j = 0; j < DL; ++j) out(lane * DL + j, acc[j] * inv);
}

// Fragment rows per load batch of a head's combine: 16 for up to 16
// fragments, else 64 (128 registers of rows at D = 128).
constexpr int kReduceSmall = 16;

// The same combine by the NW waves of a workgroup, for heads with many
// fragments: wave w takes the 16-fragment chunks w, w + NW, ..., keeping a
// running max, sum and rescaled partial over its chunks (one memory latency
// per chunk, its 16 rows loaded before the headers), and wave 0 merges the
// NW partials through LDS. A head then costs ceil(P / (16 NW)) latencies
// instead of ceil(P / 64), with NW times the waves in flight.
template <int D, int NW, typename FM, typename FL, typename FO, typename OUT>
__device__ __forceinline__ void combine_head_split(int P, FM fm, FL fl, FO fo, OUT out) {
    constexpr int DL = D / 64;
    constexpr int CH = 16;
    __shared__ float s_acc[NW][D];
    __shared__ float s_md[NW][2];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    if (P <= 0) {
        if (wv == 0) {
#pragma unroll
            for (int j = 0; j < DL; ++j) out(lane * DL + j, 0.0f);
        }
        return;
    }
    float M = -INFINITY;
    float den = 0.0f;
    float acc[DL];
#pragma unroll
    for (int j = 0; j < DL; ++j) acc[j] = 0.0f;
    for (int c0 = wv * CH; c0 < P; c0 += NW * CH) {
        float v[CH][DL];
#pragma unroll
        for (int i = 0; i < CH; ++i) load_row<D>(fo(min(c0 + i, P - 1)) + lane * DL, v[i]);
        const int p = c0 + lane;
        const bool mine = lane < CH && p < P;
        const float mp = mine ? fm(p) : -INFINITY;
        const float lp = mine ? fl(p) : 0.0f;
        const float Mn = fmaxf(M, wave_max(mp));
        if (Mn == -INFINITY) continue;  // every fragment so far empty (wave-uniform)
        const float sc = (M == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
        const float w = (mp == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mp - Mn) * lp;
        den = den * sc + wave_sum(w);
#pragma unroll
        for (int j = 0; j < DL; ++j) acc[j] *= sc;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const float wi = readlane_f(w, i);
#pragma unroll
            for (int j = 0; j < DL; ++j) acc[j] += wi * v[i][j];
        }
        M = Mn;
    }
#pragma unroll
    for (int j = 0; j < DL; ++j) s_acc[wv][lane * DL + j] = acc[j];
    if (lane == 0) {
        s_md[wv][0] = M;
        s_md[wv][1] = den;
    }
    __syncthreads();
    if (wv != 0) return;
    float Mall = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) Mall = fmaxf(Mall, s_md[w][0]);
    float tot[DL];
#pragma unroll
    for (int j = 0; j < DL; ++j) tot[j] = 0.0f;
    float dall = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const float Mw = s_md[w][0];
        const float f = (Mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(Mw - Mall);
        dall += f * s_md[w][1];
#pragma unroll
        for (int j = 0; j < DL; ++j) tot[j] += f * s_acc[w][lane * DL + j];
    }
    const float inv = dall > 0.0f ? 1.0f / dall : 0.0f;
#pragma unroll
    for (int j = 0; j < DL; ++j) out(lane * DL + j, tot[j] * inv);
}

// Split-K reduce of the partition kernel: one wave per (query head,
// sequence); sequences with a single partition were written directly by the
// partition kernel.
struct ReduceArgs {
    f16* out;
    const int* ctx;
    const float* ws_max;
    const float* ws_sum;
    const float* ws_out;
    int H;
    int MB;
    int part_blocks;
    int MP;
};

// Combine of head h of sequence s; CH: fragment rows per load batch of the
// one-wave combine, 0: the four waves of the workgroup (combine_head_split).
template <int D, int CH>
__device__ __forceinline__ void reduce_head(const ReduceArgs& a, int s, int h) {
    const int L = max(a.ctx[s], 0);
    const int nblk = min((L + kBlockTokens - 1) / kBlockTokens, a.MB);
    const int nparts = (nblk + a.part_blocks - 1) / a.part_blocks;
    if (nparts <= 1) return;
    const size_t row = static_cast<size_t>(s) * a.H + h;
    const float* pm = a.ws_max + row * a.MP;
    const float* pl = a.ws_sum + row * a.MP;
    const float* po = a.ws_out + row * a.MP * D;
    f16* o = a.out + row * D;
    auto fm = [&](int p) { return pm[p]; };
    auto fl = [&](int p) { return pl[p]; };
    auto fo = [&](int p) { return po + static_cast<size_t>(p) * D; };
    auto out = [&](int d, float v) { o[d] = static_cast<f16>(v); };
    if constexpr (CH == 0) {
        combine_head_split<D, 4>(nparts, fm, fl, fo, out);
    } else {
        combine_head_wave<D, CH>(nparts, fm, fl, fo, out);
    }
}

// One wave per (query head, sequence), four heads per workgroup; CH fragment
// rows per load batch.
template <int D, int CH>
__global__ __launch_bounds__(256) void paged_reduce_wave_kernel(const ReduceArgs a) {
    const int h = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (h >= a.H) return;
    reduce_head<D, CH>(a, blockIdx.y, h);
}

// One (query head, sequence) per workgroup of four waves, for more than 16
// partitions per sequence.
template <int D>
__global__ __launch_bounds__(256) void paged_reduce_split_kernel(const ReduceArgs a) {
    reduce_head<D, 0>(a, blockIdx.y, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Balanced ("stream-K") decode. The blocks of all sequences form one list,
// sequence by sequence. A team of TS = Hkv * nhc consecutive waves (one per
// kv head and head chunk) takes blocks [t*q, (t+1)*q) of that list, with
// q = ceil(blocks / teams): every team gets the same number of blocks
// whatever the context lengths, the grid runs in one round, and the waves of
// a team read the kv-head tiles of the same blocks at the same time (one
// block's tiles are contiguous in HBM). A wave walks its range as up to a few
// segments (one per sequence it touches): a segment that covers the whole
// sequence writes the final output; otherwise it leaves a fragment (max, sum,
// partial output) in slot 2w (the wave's first segment) or 2w+1 (its last),
// and paged_streamk_reduce_kernel combines the fragments of each split item.
// ---------------------------------------------------------------------------
constexpr int kStreamMaxSeqs = 4096;  // LDS prefix table bound
constexpr int kFragHead = 32;         // floats before a fragment's partial output (16-byte aligned)
constexpr int kStreamWaves = 4;       // waves per workgroup
// Waves per SIMD the kernel's registers must allow: the grid is sized so
// every wave is resident at once (4 SIMDs per CU).
constexpr int kStreamWavesPerSimd = 3;

struct StreamArgs {
    f16* out;
    const f16* q;
    const f16* kc;
    const f16* vc;
    const int* bt;
    const int* ctx;
    float* frag;  // [2W][kFragHead + gstride * D]: max[16], sum[16], out[gstride][D]
    // [W][4] + 1: first block of the sequence, sequence, blocks of the
    // sequence (first segment of each wave, -1 if whole), then blocks per
    // team. 64-bit on purpose: no store of the kernel has the block table's
    // type.
    long long* meta;
    float scale_log2;
    int S, H, Hkv, G, nhc, MB, num_blocks;
    int W;  // waves in the grid
};

// Blocks per sequence -> exclusive prefix in s_pre[0..S] (s_pre[S] = total),
// clamped context lengths in s_len. All threads of the workgroup take part.
// A: any argument struct with S, ctx and MB.
template <typename A>
__device__ __forceinline__ void stream_prefix(const A& a, int* s_pre, int* s_len, int* s_tot) {
    const int chunk = (a.S + blockDim.x - 1) / blockDim.x;
    const int c0 = threadIdx.x * chunk;
    int run = 0;
    for (int c = c0; c < min(a.S, c0 + chunk); ++c) {
        const int L0 = max(a.ctx[c], 0);
        const int nb = min((L0 + kBlockTokens - 1) / kBlockTokens, a.MB);
        s_len[c] = min(L0, nb * kBlockTokens);
        s_pre[c] = run;  // local exclusive prefix, offset added below
        run += nb;
    }
    s_tot[threadIdx.x] = run;
    __syncthreads();
    if (threadIdx.x < 64) {
        // exclusive scan of the (<= 256) chunk totals by wave 0
        const int n = blockDim.x;
        int v[4];
        int sum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = threadIdx.x * 4 + i;
            v[i] = idx < n ? s_tot[idx] : 0;
            sum += v[i];
        }
        int incl = sum;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(incl, off);
            if (static_cast<int>(threadIdx.x) >= off) incl += t;
        }
        int ex = incl - sum;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = threadIdx.x * 4 + i;
            if (idx < n) s_tot[idx] = ex;
            ex += v[i];
        }
        if (threadIdx.x == 63) s_pre[a.S] = incl;
    }
    __syncthreads();
    const int off = s_tot[threadIdx.x];
    for (int c = c0; c < min(a.S, c0 + chunk); ++c) s_pre[c] += off;
    __syncthreads();
}

template <int D>
__global__ __launch_bounds__(64 * kStreamWaves) __attribute__((amdgpu_waves_per_eu(kStreamWavesPerSimd)))
void paged_decode_streamk_kernel(const StreamArgs a) {
    constexpr int NJ = D / 16;
    extern __shared__ int s_dyn[];
    int* s_pre = s_dyn;              // [S + 1]
    int* s_len = s_dyn + a.S + 1;    // [S]
    __shared__ int s_tot[64 * kStreamWaves];
    stream_prefix(a, s_pre, s_len, s_tot);

    // Sequences without blocks are not in the list: zero their outputs here.
    for (int sz = blockIdx.x; sz < a.S; sz += gridDim.x) {
        if (s_pre[sz + 1] == s_pre[sz]) {
            for (int i = threadIdx.x; i < a.H * D; i += blockDim.x) {
                a.out[static_cast<size_t>(sz) * a.H * D + i] = static_cast<f16>(0.0f);
            }
        }
    }

    const int lane = threadIdx.x & 63;
    const int w = blockIdx.x * kStreamWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;
    const int kg = lane >> 4;
    const int gstride = min(16, a.G);
    const int TS = a.Hkv * a.nhc;  // waves per team
    const int teams = a.W / TS;
    const int team = w / TS;
    const int member = w - team * TS;
    const int kvh = member / a.nhc;
    const int hc = member - kvh * a.nhc;
    const int g0 = hc * 16;
    const int gn = min(16, a.G - g0);
    const int h0 = kvh * a.G + g0;
    const int U = __builtin_amdgcn_readfirstlane(s_pre[a.S]);
    const int q = (U + teams - 1) / teams;
    const int u0 = team < teams ? min(U, team * q) : U;
    const int u1 = team < teams ? min(U, u0 + q) : U;
    long long* meta = a.meta + 4 * w;
    if (lane == 0) meta[0] = -1;  // no split first segment (overwritten below if there is one)
    if (w == 0 && lane == 0) a.meta[4 * a.W] = q;  // blocks per team, for the reduce

    h4 ident;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ident[i] = (4 * kg + i == r) ? static_cast<f16>(1.0f) : static_cast<f16>(0.0f);
    }
    const int loff = kv_elem_offset(r, 4 * kg);

    bool first_seg = true;
    int u = u0;
    while (u < u1) {
        // sequence of block u: largest s with s_pre[s] <= u
        int lo = 0, hi = a.S;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (s_pre[mid] <= u) lo = mid; else hi = mid;
        }
        // Everything below is wave-uniform; readfirstlane keeps it in scalar
        // registers so the block-table reads stay scalar loads.
        const int s = __builtin_amdgcn_readfirstlane(lo);
        const int L = __builtin_amdgcn_readfirstlane(s_len[s]);
        const int pre = __builtin_amdgcn_readfirstlane(s_pre[s]);
        const int nb = __builtin_amdgcn_readfirstlane(s_pre[s + 1]) - pre;
        const int j0 = u - pre;
        const int seg = min(nb - j0, u1 - u);

        QOperand<D> qB;
        {
            const f16* qp = a.q + (static_cast<size_t>(s) * a.H + h0 + min(r, gn - 1)) * D + 4 * kg;
#pragma unroll
            for (int J = 0; J < NJ; ++J) {
                const h4 v = *reinterpret_cast<const h4*>(qp + 16 * J);
                qB.v[J] = (r < gn) ? v : h4{0, 0, 0, 0};
            }
        }
        const const_int* btrow = as_const(a.bt) + static_cast<size_t>(s) * a.MB;
        WaveState<D> st;
        st.m = -INFINITY;
        st.l = 0.0f;
#pragma unroll
        for (int J = 0; J < NJ; ++J) st.acc[J] = f4{0, 0, 0, 0};
        attend_blocks<D>(st, btrow, j0, 1, seg, L, a.kc, a.vc, a.Hkv, a.num_blocks, kvh, loff, kg,
                         qB, ident, a.scale_log2);
        float l_run = st.l;
        l_run = sum_over_kg(l_run);
        const float inv = (l_run > 0.0f) ? 1.0f / l_run : 0.0f;
        if (j0 == 0 && seg == nb) {
            if (r < gn) {
                f16* op = a.out + (static_cast<size_t>(s) * a.H + h0 + r) * D + 4 * kg;
#pragma unroll
                for (int J = 0; J < NJ; ++J) {
                    h4 o;
#pragma unroll
                    for (int i = 0; i < 4; ++i) o[i] = static_cast<f16>(st.acc[J][i] * inv);
                    *reinterpret_cast<h4*>(op + 16 * J) = o;
                }
            }
        } else {
            const int slot = 2 * w + (first_seg ? 0 : 1);
            float* f = a.frag + static_cast<size_t>(slot) * (kFragHead + gstride * D);
            if (r < gn) {
                if (kg == 0) {
                    f[r] = st.m;
                    f[16 + r] = l_run;
                }
                float* fo = f + kFragHead + static_cast<size_t>(r) * D + 4 * kg;
#pragma unroll
                for (int J = 0; J < NJ; ++J) *reinterpret_cast<f4*>(fo + 16 * J) = st.acc[J] * inv;
            }
            if (first_seg && lane == 0) {
                meta[0] = pre;  // first block of the sequence in the list
                meta[1] = s;
                meta[2] = nb;
            }
        }
        first_seg = false;
        u += seg;
    }
}

// Combines the fragments of every split item: one wave per (w, g) reduces
// query head g of the item whose fragments wave w owns (four heads per
// workgroup). Wave w owns the item of its
// first segment when that segment is split, starts inside the sequence, and
// w's team is the first team to start inside it (every other workgroup exits
// at once). Fragments of the item come from the waves with the same team
// member index in teams ta..tb.
struct StreamReduceArgs {
    f16* out;
    const float* frag;
    const long long* meta;
    int H, Hkv, G, nhc, W;
    int gstride;
};

template <int D>
__global__ __launch_bounds__(256) void paged_streamk_reduce_kernel(const StreamReduceArgs a) {
    const int w = blockIdx.x;
    const int g = blockIdx.y * 4 + (threadIdx.x >> 6);
    const long long* m = a.meta + 4 * w;
    if (m[0] < 0) return;
    const int TS = a.Hkv * a.nhc;
    const int q = static_cast<int>(a.meta[4 * a.W]);
    const int ustart = static_cast<int>(m[0]);
    const int team = w / TS;
    const int ta = ustart / q;
    if (team != ta + 1 || ustart == team * q) return;  // not the owner
    const int member = w - team * TS;
    const int kvh = member / a.nhc;
    const int hc = member - kvh * a.nhc;
    const int g0 = hc * 16;
    const int gn = min(16, a.G - g0);
    if (g >= gn) return;
    const int s = static_cast<int>(m[1]);
    const int nb = static_cast<int>(m[2]);
    const int P = (ustart + nb - 1) / q - ta + 1;
    const size_t fs = kFragHead + static_cast<size_t>(a.gstride) * D;
    // fragment i of the item comes from team ta + i
    auto frag_of = [&](int i) {
        const int t = ta + i;
        const int v = t * TS + member;
        const int slot = (t == ta && ta * q < ustart) ? 2 * v + 1 : 2 * v;
        return a.frag + slot * fs;
    };
    f16* o = a.out + (static_cast<size_t>(s) * a.H + kvh * a.G + g0 + g) * D;
    combine_head_wave<D, kReduceSmall>(
        P, [&](int i) { return frag_of(i)[g]; }, [&](int i) { return frag_of(i)[16 + g]; },
        [&](int i) { return frag_of(i) + kFragHead + static_cast<size_t>(g) * D; },
        [&](int d, float v) { o[d] = static_cast<f16>(v); });
}

// ---------------------------------------------------------------------------
// Split-K in partition streams. The blocks of all sequences form one list,
// sequence by sequence, as in the balanced mode; a team of TS = Hkv * nhc
// consecutive waves takes blocks [t*q, (t+1)*q) of it, each wave one kv head
// and head chunk, so every wave gets the same number of blocks whatever the
// context lengths. A wave walks its range with one continuous load pipeline
// (the next block's tiles are in flight while a block is attended) and
// leaves a partial (max, sum, normalised output) each time it reaches the
// end of a partition: no LDS merge, no barrier and no pipeline drain per
// partition, which is what the per-item walk pays over short partitions.
// A range boundary t*q that falls strictly inside a partition splits it into
// pieces. Only a wave's first piece can start at such a boundary; every
// other piece starts at a partition start. A piece from a partition's start
// goes to the partition's slot of the regular workspace, a piece from a
// boundary to the boundary slot of wave (t, member) in `frag`. A sequence
// with one partition and no boundary inside writes its output directly.
// The partial of a piece that ends before the wave's range does is held in
// the wave's LDS slot (one per wave) and written with the wave's last one,
// so a wave's HBM writes come after its reads instead of among them (writes
// landing in the read stream cost far more than their bytes).
// paged_reduce_pstream_wave_kernel (up to 16 fragments per head, a wave per
// head) and paged_reduce_pstream_split_kernel (more, four waves per head)
// combine, per head, the partition slots and the boundary slots that fall
// inside the sequence.
// ---------------------------------------------------------------------------

// A wave-uniform pointer held in SGPRs at this point of the program: the
// empty asm hides its value from the optimiser, so address arithmetic on it
// is done where it is used instead of being hoisted into a loop-invariant
// 64-bit vector register pair.
__device__ __forceinline__ char* pinned_sgpr(char* p) {
    asm volatile("" : "+s"(p));
    return p;
}

// Attends blocks j0 .. j1 - 1 of one sequence in order, double-buffered like
// attend_blocks, and calls done(j) after block j; the next block's loads are
// in flight while done(j) runs.
template <int D, typename Done>
__device__ __forceinline__ void attend_run(WaveState<D>& st, const const_int* btrow, int j0, int j1,
                                           int L, const f16* kc, const f16* vc, int Hkv,
                                           int num_blocks, int kvh, int loff, int kg,
                                           const QOperand<D>& qB, h4 ident, float scale_log2,
                                           Done done) {
    constexpr int NJ = D / 16;
    const int count = j1 - j0;
    if (count <= 0) return;
    auto block_at = [&](int j) { return __builtin_amdgcn_readfirstlane(btrow[j]); };
    auto valid_of = [&](int j, int b) {
        return block_ok(b, num_blocks) ? min(kBlockTokens, L - j * kBlockTokens) : 0;
    };
    h4 kA[NJ], vA[NJ], kB[NJ], vB[NJ];
    int jA = j0;
    int bA = block_at(jA);
    load_tile<D>(kc, vc, Hkv, num_blocks, bA, kvh, loff, kA, vA);
    int left = count;
    for (; left > 2; left -= 2) {
        const int jB = jA + 1;
        const int bB = block_at(jB);
        load_tile<D>(kc, vc, Hkv, num_blocks, bB, kvh, loff, kB, vB);
        attend_block<D>(st, valid_of(jA, bA), kg, kA, vA, qB, ident, scale_log2);
        done(jA);
        jA = jB + 1;
        bA = block_at(jA);
        load_tile<D>(kc, vc, Hkv, num_blocks, bA, kvh, loff, kA, vA);
        attend_block<D>(st, valid_of(jB, bB), kg, kB, vB, qB, ident, scale_log2);
        done(jB);
    }
    if (left == 2) {
        const int jB = jA + 1;
        const int bB = block_at(jB);
        load_tile<D>(kc, vc, Hkv, num_blocks, bB, kvh, loff, kB, vB);
        attend_block<D>(st, valid_of(jA, bA), kg, kA, vA, qB, ident, scale_log2);
        done(jA);
        attend_block<D>(st, valid_of(jB, bB), kg, kB, vB, qB, ident, scale_log2);
        done(jB);
    } else {
        attend_block<D>(st, valid_of(jA, bA), kg, kA, vA, qB, ident, scale_log2);
        done(jA);
    }
}

// Partition streams serve partitions of up to kPStreamMaxPartBlocks blocks,
// in batches whose block prefix fits in LDS, with a grid of
// kPStreamWavesPerSimd waves per SIMD (the kernel's register cap).
#ifndef SWIFTLLM_PSTREAM_MAX_PART_BLOCKS
#define SWIFTLLM_PSTREAM_MAX_PART_BLOCKS 64
#endif
#ifndef SWIFTLLM_PSTREAM_WAVES_PER_SIMD
#define SWIFTLLM_PSTREAM_WAVES_PER_SIMD 2
#endif
constexpr int kPStreamMaxPartBlocks = SWIFTLLM_PSTREAM_MAX_PART_BLOCKS;
constexpr int kPStreamWavesPerSimd = SWIFTLLM_PSTREAM_WAVES_PER_SIMD;

// Teams of a partition-stream grid of W waves, TS waves per team.
__host__ __device__ __forceinline__ int pstream_teams(int W, int TS) { return max(1, W / TS); }

// Where a piece's partial goes: rows (lane row r at rows + r * rstride, 16
// bytes per lane group and 16-row slice), max and sum (row r at m / l +
// r * mstride). Wave-uniform.
struct PieceDst {
    char* rows;
    char* m;
    char* l;
    unsigned rstride;
    unsigned mstride;
};

// Floats a lane keeps in its LDS slot: its NJ output vectors, max and sum
// (padded to 16 bytes).
template <int D>
constexpr int kStageFloats = 4 * (D / 16) + 4;

// Writes a piece's partial: lane (r, kg) its four outputs of each 16-row
// slice of row r, lanes with kg = 0 the row's max and sum; rows r >= gn
// (padding) are skipped. The lane offsets are computed here from the lane
// index (behind an empty asm), so none stays live in a register.
template <int D>
__device__ __forceinline__ void write_piece(const PieceDst& d, int lane, bool row_ok, const f4 (&v)[D / 16],
                                            float m, float l) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const unsigned rr = static_cast<unsigned>(ln & 15);
    const unsigned kk = static_cast<unsigned>(ln >> 4);
    char* rows = pinned_sgpr(d.rows);
    if (row_ok) {
        const unsigned lo = rr * d.rstride + 16u * kk;
#pragma unroll
        for (int J = 0; J < D / 16; ++J) __builtin_nontemporal_store(v[J], reinterpret_cast<f4*>(rows + lo + 64u * J));
        if (kk == 0) {
            *reinterpret_cast<float*>(pinned_sgpr(d.m) + rr * d.mstride) = m;
            *reinterpret_cast<float*>(pinned_sgpr(d.l) + rr * d.mstride) = l;
        }
    }
}

template <int D>
__global__ __launch_bounds__(64 * kStreamWaves) __attribute__((amdgpu_waves_per_eu(kPStreamWavesPerSimd)))
void paged_partition_stream_kernel(const DecodeArgs a) {
    constexpr int NJ = D / 16;
    extern __shared__ int s_dyn[];
    int* s_pre = s_dyn;              // [S + 1]
    int* s_len = s_dyn + a.S + 1;    // [S]
    __shared__ int s_tot[64 * kStreamWaves];
    stream_prefix(a, s_pre, s_len, s_tot);

    const int U = __builtin_amdgcn_readfirstlane(s_pre[a.S]);
    const int P = a.part_blocks;
    const int TS = a.Hkv * a.nhc;
    const int teams = pstream_teams(a.W, TS);
    const int q = (U + teams - 1) / teams;
    if (blockIdx.x == 0) {
        // For the reduce: blocks per team, teams, and the block prefix.
        for (int i = threadIdx.x; i <= a.S; i += blockDim.x) a.meta[2 + i] = s_pre[i];
        if (threadIdx.x == 0) {
            a.meta[0] = q;
            a.meta[1] = teams;
        }
    }
    // Sequences without blocks are not in the list: zero their outputs here.
    for (int sz = blockIdx.x; sz < a.S; sz += gridDim.x) {
        if (s_pre[sz + 1] == s_pre[sz]) {
            for (int i = threadIdx.x; i < a.H * D; i += blockDim.x) {
                a.out[static_cast<size_t>(sz) * a.H * D + i] = static_cast<f16>(0.0f);
            }
        }
    }

    const int lane = threadIdx.x & 63;
    const int w = blockIdx.x * kStreamWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int team = w / TS;
    if (team >= teams || U == 0) return;
    const int member = w - team * TS;
    const int r = lane & 15;
    const int kg = lane >> 4;
    const int gstride = min(16, a.G);
    const int kvh = member / a.nhc;
    const int hc = member - kvh * a.nhc;
    const int g0 = hc * 16;
    const int gn = min(16, a.G - g0);
    const int h0 = kvh * a.G + g0;
    const int u0 = min(U, team * q);
    const int u1 = min(U, u0 + q);

    h4 ident;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ident[i] = (4 * kg + i == r) ? static_cast<f16>(1.0f) : static_cast<f16>(0.0f);
    }
    const int loff = kv_elem_offset(r, 4 * kg);

    // One partial per wave can wait in LDS (this wave's 64-lane slot) for the
    // end of the wave's range.
    float* slot = reinterpret_cast<float*>(s_dyn + a.stage_off) +
                  (static_cast<size_t>(threadIdx.x >> 6) * 64 + lane) * kStageFloats<D>;
    bool staged = false;
    PieceDst held{};

    int u = u0;
    while (u < u1) {
        // Sequence of block u: the largest s with s_pre[s] <= u. Wave-uniform
        // values go through readfirstlane so the block-table reads stay
        // scalar loads.
        int lo = 0, hi = a.S;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (s_pre[mid] <= u) lo = mid; else hi = mid;
        }
        const int s = __builtin_amdgcn_readfirstlane(lo);
        const int L = __builtin_amdgcn_readfirstlane(s_len[s]);
        const int pre = __builtin_amdgcn_readfirstlane(s_pre[s]);
        const int nb = __builtin_amdgcn_readfirstlane(s_pre[s + 1]) - pre;
        const int j0 = u - pre;
        const int j1 = min(nb, u1 - pre);
        const int nparts = (nb + P - 1) / P;

        QOperand<D> qB;
        {
            const f16* qp = a.q + (static_cast<size_t>(s) * a.H + h0 + min(r, gn - 1)) * D + 4 * kg;
#pragma unroll
            for (int J = 0; J < NJ; ++J) {
                const h4 v = *reinterpret_cast<const h4*>(qp + 16 * J);
                qB.v[J] = (r < gn) ? v : h4{0, 0, 0, 0};
            }
        }
        const const_int* btrow = as_const(a.bt) + static_cast<size_t>(s) * a.MB;
        WaveState<D> st;
        st.m = -INFINITY;
        st.l = 0.0f;
#pragma unroll
        for (int J = 0; J < NJ; ++J) st.acc[J] = f4{0, 0, 0, 0};
        int seg0 = j0;                            // first block of the open piece
        int cut = min(j1, (j0 / P + 1) * P);      // block after the open piece
        attend_run<D>(st, btrow, j0, j1, L, a.kc, a.vc, a.Hkv, a.num_blocks, kvh, loff, kg, qB,
                      ident, a.scale_log2, [&](int j) {
            if (j + 1 != cut) return;
            const int part = seg0 / P;
            const float l_run = sum_over_kg(st.l);
            const float inv = (l_run > 0.0f) ? 1.0f / l_run : 0.0f;
            const bool whole = (seg0 == part * P) && (cut == min(nb, (part + 1) * P));
            const size_t row0 = static_cast<size_t>(s) * a.H + h0;
            if (whole && nparts == 1) {
                // Lane offsets computed here from the lane index, so no lane
                // address stays live across the block loop (the kernel runs
                // at its 168-register cap).
                int ln = lane;
                asm volatile("" : "+v"(ln));
                const int rr = ln & 15;
                const int kk = ln >> 4;
                char* ob = pinned_sgpr(reinterpret_cast<char*>(a.out + row0 * D));
                const unsigned lo = static_cast<unsigned>(rr * D + 4 * kk) * sizeof(f16);
                if (r < gn) {
#pragma unroll
                    for (int J = 0; J < NJ; ++J) {
                        h4 o;
#pragma unroll
                        for (int i = 0; i < 4; ++i) o[i] = static_cast<f16>(st.acc[J][i] * inv);
                        *reinterpret_cast<h4*>(ob + lo + 32u * J) = o;
                    }
                }
                // The compiler treats the wave's memory counter as out of
                // order while stores and loads are both in flight, and then
                // waits for every load before each block: a full wait here
                // keeps the waits in the block loop exact.
                wait_vm<0>();
            } else {
                // A partition slot (the piece starts at its partition's
                // start) or the wave's boundary slot.
                PieceDst dst;
                if (seg0 == part * P) {
                    const size_t p0 = row0 * a.MP + part;
                    dst.rows = reinterpret_cast<char*>(a.ws_out + p0 * D);
                    dst.rstride = static_cast<unsigned>(a.MP) * D * sizeof(float);
                    dst.m = reinterpret_cast<char*>(a.ws_max + p0);
                    dst.l = reinterpret_cast<char*>(a.ws_sum + p0);
                    dst.mstride = static_cast<unsigned>(a.MP) * sizeof(float);
                } else {
                    char* f = reinterpret_cast<char*>(a.frag + static_cast<size_t>(w) * (kFragHead + gstride * D));
                    dst.rows = f + kFragHead * sizeof(float);
                    dst.rstride = D * sizeof(float);
                    dst.m = f;
                    dst.l = f + 16 * sizeof(float);
                    dst.mstride = sizeof(float);
                }
                if (!staged && pre + cut != u1) {
                    // Held in LDS until the wave's range ends, so that its
                    // HBM writes do not land among the wave's reads.
#pragma unroll
                    for (int J = 0; J < NJ; ++J) *reinterpret_cast<f4*>(slot + 4 * J) = st.acc[J] * inv;
                    slot[4 * NJ] = st.m;
                    slot[4 * NJ + 1] = l_run;
                    held = dst;
                    staged = true;
                } else {
                    f4 v[NJ];
#pragma unroll
                    for (int J = 0; J < NJ; ++J) v[J] = st.acc[J] * inv;
                    write_piece<D>(dst, lane, r < gn, v, st.m, l_run);
                    wait_vm<0>();
                }
            }
            st.m = -INFINITY;
            st.l = 0.0f;
#pragma unroll
            for (int J = 0; J < NJ; ++J) st.acc[J] = f4{0, 0, 0, 0};
            seg0 = cut;
            cut = min(j1, cut + P);
        });
        u = pre + j1;
    }
    if (staged) {
        f4 v[NJ];
#pragma unroll
        for (int J = 0; J < NJ; ++J) v[J] = *reinterpret_cast<const f4*>(slot + 4 * J);
        write_piece<D>(held, lane, r < gn, v, slot[4 * NJ], slot[4 * NJ + 1]);
    }
}

// Reduce of the partition streams: one (query head, sequence) combines its
// nparts partition slots and the boundary slots of teams ta .. tb whose
// boundary falls strictly inside the sequence's blocks. A boundary at a
// partition start splits nothing; its fragment is given weight 0 (and the
// partition slot 0 row, which is finite, as its row).
struct PStreamReduceArgs {
    f16* out;
    const float* ws_max;
    const float* ws_sum;
    const float* ws_out;
    const float* frag;
    const int* meta;
    int H, G, nhc, MP, part_blocks, gstride, TS;
};

// CH: fragment rows per batch of the one-wave combine; 0: the head is
// combined by the four waves of the workgroup (combine_head_split).
template <int D, int CH>
__device__ __forceinline__ void pstream_reduce_head(const PStreamReduceArgs& a, int s, int h) {
    const int q = a.meta[0];
    const int pre = a.meta[2 + s];
    const int nb = a.meta[3 + s] - pre;
    const int P = a.part_blocks;
    const int nparts = (nb + P - 1) / P;
    // Boundaries t*q strictly inside (pre, pre + nb). When q and pre are
    // multiples of P every boundary falls on a partition start and splits
    // nothing, so none is combined.
    const int ta = pre / q + 1;
    const int tb = nb > 0 ? (pre + nb - 1) / q : ta - 1;
    const bool on_starts = (q % P == 0) && (pre % P == 0);
    const int nbound = on_starts ? 0 : max(0, tb - ta + 1);
    if (nb == 0 || (nparts == 1 && nbound == 0)) return;  // zeros or written directly
    const int kvh = h / a.G;
    const int gk = h - kvh * a.G;
    const int hc = gk / 16;
    const int g = gk - hc * 16;
    const int member = kvh * a.nhc + hc;
    const size_t row = static_cast<size_t>(s) * a.H + h;
    const float* pm = a.ws_max + row * a.MP;
    const float* pl = a.ws_sum + row * a.MP;
    const float* po = a.ws_out + row * a.MP * D;
    const size_t fs = kFragHead + static_cast<size_t>(a.gstride) * D;
    auto split = [&](int i) {  // boundary fragment i: a piece of its own?
        const int t = ta + i;
        return (t * q - pre) % P != 0;
    };
    auto frag_of = [&](int i) { return a.frag + static_cast<size_t>((ta + i) * a.TS + member) * fs; };
    auto fm = [&](int p) {
        if (p < nparts) return pm[p];
        const int i = p - nparts;
        return split(i) ? frag_of(i)[g] : -INFINITY;
    };
    auto fl = [&](int p) {
        if (p < nparts) return pl[p];
        const int i = p - nparts;
        return split(i) ? frag_of(i)[16 + g] : 0.0f;
    };
    auto fo = [&](int p) {
        if (p < nparts) return po + static_cast<size_t>(p) * D;
        const int i = p - nparts;
        return split(i) ? frag_of(i) + kFragHead + static_cast<size_t>(g) * D : po;
    };
    f16* o = a.out + row * D;
    auto out = [&](int d, float v) { o[d] = static_cast<f16>(v); };
    if constexpr (CH == 0) {
        combine_head_split<D, 4>(nparts + nbound, fm, fl, fo, out);
    } else {
        combine_head_wave<D, CH>(nparts + nbound, fm, fl, fo, out);
    }
}

template <int D, int CH>
__global__ __launch_bounds__(256) void paged_reduce_pstream_wave_kernel(const PStreamReduceArgs a) {
    const int h = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (h >= a.H) return;
    pstream_reduce_head<D, CH>(a, blockIdx.y, h);
}

// One (query head, sequence) per workgroup of four waves.
template <int D>
__global__ __launch_bounds__(256) void paged_reduce_pstream_split_kernel(const PStreamReduceArgs a) {
    pstream_reduce_head<D, 0>(a, blockIdx.y, blockIdx.x);
}

// Bit-exact materialisation of one (sequence, kv head) through the tile
// addressing above.
struct GatherArgs {
    const uint16_t* kc;
    const uint16_t* vc;
    const int* bt;
    const int* ctx;
    uint16_t* ko;
    uint16_t* vo;
    int s, kvh, Hkv, D, MB, max_len;
};

__global__ __launch_bounds__(256) void gather_kv_kernel(const GatherArgs a) {
    int L = max(a.ctx[a.s], 0);
    L = min(L, min(a.MB * kBlockTokens, a.max_len));
    const int* btrow = a.bt + static_cast<size_t>(a.s) * a.MB;
    const size_t n = static_cast<size_t>(a.max_len) * a.D;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const int t = static_cast<int>(i / a.D);
        const int d = static_cast<int>(i - static_cast<size_t>(t) * a.D);
        uint16_t kv = 0, vv = 0;
        if (t < L) {
            const int b = btrow[t / kBlockTokens];
            const size_t off = kv_tile_offset(b, a.kvh, a.Hkv, a.D) + kv_elem_offset(d, t % kBlockTokens);
            kv = a.kc[off];
            vv = a.vc[off];
        }
        a.ko[i] = kv;
        a.vo[i] = vv;
    }
}

struct ClearArgs {
    uint32_t* p;
    size_t words;
};

__global__ __launch_bounds__(256) void clear_kernel(const ClearArgs a) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < a.words;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        a.p[i] = 0u;
    }
}


// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
constexpr size_t kAlign = 256;

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

struct Shape {
    int S, H, Hkv, D, BS, MB;
};

int validate_decode(const char* who, const void* out, const void* q, const void* kc,
                    const void* vc, const int* bt, const int* ctx, const Shape& sh) {
    if (sh.S < 0 || sh.H <= 0 || sh.Hkv <= 0 || sh.MB < 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                    "%s: num_seqs=%d num_heads=%d num_kv_heads=%d max_num_blocks_per_seq=%d",
                    who, sh.S, sh.H, sh.Hkv, sh.MB);
    }
    if (sh.H % sh.Hkv != 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                    "%s: num_heads %d is not a multiple of num_kv_heads %d", who, sh.H, sh.Hkv);
    }
    if (sh.D != 64 && sh.D != 128) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: head_dim %d (supported: 64, 128)", who, sh.D);
    }
    if (sh.BS != kBlockTokens) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: block_size %d (supported: 16)", who, sh.BS);
    }
    if (sh.S > 65535) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: num_seqs %d > 65535", who, sh.S);
    }
    const long long nhc = (sh.H / sh.Hkv + 15) / 16;
    if (static_cast<long long>(sh.Hkv) * nhc > 65535) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: too many kv heads", who);
    }
    if (sh.S == 0) return SWIFTLLM_OK;
    if (!out || !q || !kc || !vc || !bt || !ctx) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    if (!aligned(out, 2) || !aligned(q, 8) || !aligned(kc, 8) || !aligned(vc, 8) ||
        !aligned(bt, 4) || !aligned(ctx, 4)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                    "%s: misaligned pointer (query and caches need 8-byte alignment)", who);
    }
    return SWIFTLLM_OK;
}

// Waves per workgroup of the single-pass kernel: the whole context of a
// (sequence, kv head) is one workgroup, so it gets the most waves.
#ifndef SWIFTLLM_WAVES_V1
#define SWIFTLLM_WAVES_V1 4
#endif
constexpr int kWavesV1 = SWIFTLLM_WAVES_V1;
// Waves per workgroup of a split-K partition.
#ifndef SWIFTLLM_WAVES_V2
#define SWIFTLLM_WAVES_V2 4
#endif
constexpr int kWavesV2 = SWIFTLLM_WAVES_V2;

template <int D, int NW>
hipError_t launch_decode_t(const DecodeArgs& a, int S, int mp_grid, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(merge_lds_floats<D, NW>(a.G)) * sizeof(float);
    dim3 grid(mp_grid, a.Hkv * a.nhc, S);
    return launch(paged_decode_kernel<D, NW>, grid, dim3(NW * 64), lds, stream, a);
}

template <int NW>
hipError_t launch_decode(const DecodeArgs& a, int D, int S, int mp_grid, hipStream_t stream) {
    return D == 128 ? launch_decode_t<128, NW>(a, S, mp_grid, stream)
                    : launch_decode_t<64, NW>(a, S, mp_grid, stream);
}

template <int D, int NW>
hipError_t launch_partition_t(const DecodeArgs& a, unsigned grid, hipStream_t stream) {
    size_t lds = static_cast<size_t>(merge_lds_floats<D, NW>(a.G)) * sizeof(float);
    if (a.S <= kPartMaxSeqs) lds += part_list_lds_bytes(a.S);
    return launch(paged_partition_kernel<D, NW>, dim3(grid), dim3(NW * 64), lds, stream, a);
}

int device_cus();

// Split-K partition kernel: a grid of resident workgroups (three 4-wave
// workgroups per CU, four rounds) walking the compacted item list, or one
// workgroup per possible item for batches too large to compact in LDS.
template <int NW>
hipError_t launch_partition(const DecodeArgs& a, int D, hipStream_t stream, bool* too_large) {
    const long long possible = static_cast<long long>(a.MP) * a.Hkv * a.nhc * a.S;
    long long grid = possible;
    if (a.S <= kPartMaxSeqs) grid = std::min(possible, 12LL * device_cus());
    *too_large = grid > 0x7fffffffLL;
    if (*too_large || grid <= 0) return hipSuccess;
    const unsigned g = static_cast<unsigned>(grid);
    return D == 128 ? launch_partition_t<128, NW>(a, g, stream)
                    : launch_partition_t<64, NW>(a, g, stream);
}

DecodeArgs make_args(void* out, const void* q, const void* kc, const void* vc, const int* bt,
                     const int* ctx, float scale, const Shape& sh, int num_blocks) {
    DecodeArgs a{};
    a.out = static_cast<f16*>(out);
    a.q = static_cast<const f16*>(q);
    a.kc = static_cast<const f16*>(kc);
    a.vc = static_cast<const f16*>(vc);
    a.bt = bt;
    a.ctx = ctx;
    a.scale_log2 = static_cast<float>(static_cast<double>(scale) * static_cast<double>(kLog2e));
    a.H = sh.H;
    a.Hkv = sh.Hkv;
    a.G = sh.H / sh.Hkv;
    a.nhc = (a.G + 15) / 16;
    a.MB = sh.MB;
    a.S = sh.S;
    a.num_blocks = num_blocks;
    return a;
}


int decode_v1(void* out, const void* q, const void* kc, const void* vc, const int* bt,
              const int* ctx, float scale, const Shape& sh, int num_blocks, hipStream_t stream,
              const char* who) {
    int rc = validate_decode(who, out, q, kc, vc, bt, ctx, sh);
    if (rc != SWIFTLLM_OK) return rc;
    if ((rc = require_device()) != SWIFTLLM_OK) return rc;
    if (sh.S == 0) return ok();
    DecodeArgs a = make_args(out, q, kc, vc, bt, ctx, scale, sh, num_blocks);
    a.part_blocks = 0;
    a.MP = 1;
    // Snake order over the ranked sequences when the whole grid is resident
    // at once (three 4-wave workgroups per CU at the kernel's register count)
    // and small enough to rank; otherwise sequence order, balanced by the
    // dispatcher as workgroups finish.
    const long long items = static_cast<long long>(sh.S) * a.Hkv * a.nhc;
    a.snake = (kWavesV1 == 4 && sh.S <= kLptMaxSeqs && items <= 3LL * device_cus()) ? device_cus() : 0;
    return launched(launch_decode<kWavesV1>(a, sh.D, sh.S, 1, stream), who);
}

constexpr int kPStreamWavesPerCU = 4 * kPStreamWavesPerSimd;

// Split-K workspace: max logits and exp sums [S][H][MP] and partial outputs
// [S][H][MP][D], all fp32; with partition streams also the boundary pieces
// [W][kFragHead + gstride * D] and the team metadata (q, teams, block
// prefix [S + 1]). Plain scratch: every value a call reads was written
// earlier in the same call, so it needs no initialisation.
struct V2Need {
    int MP;          // partitions per sequence
    size_t stat;     // bytes of one [S][H][MP] float array
    bool pstream;    // partition streams
    int W;           // waves of the partition-stream grid
    size_t frag;     // offset of the boundary pieces
    size_t meta;     // offset of the team metadata
    size_t total;    // bytes of the whole workspace
};

V2Need v2_need(const Shape& sh, int partition_size, int cus) {
    V2Need n{};
    const int part_blocks = partition_size / kBlockTokens;
    n.MP = sh.MB == 0 ? 1 : (sh.MB + part_blocks - 1) / part_blocks;
    n.stat = align_up(sizeof(float) * static_cast<size_t>(sh.S) * sh.H * n.MP);
    n.total = 2 * n.stat + align_up(sizeof(float) * static_cast<size_t>(sh.S) * sh.H * n.MP * sh.D);
    const int G = sh.H / sh.Hkv;
    const long long TS = static_cast<long long>(sh.Hkv) * ((G + 15) / 16);
    n.W = cus * kPStreamWavesPerCU;
    // Partition streams when partitions are short and the batch has at most
    // a quarter as many sequences as the grid has teams (a wave then starts
    // few new sequences, each a pipeline restart), and the lane offsets of
    // a wave's partial rows fit in 31 bits.
    const long long teams = TS > 0 ? n.W / TS : 0;
    n.pstream = sh.S <= kStreamMaxSeqs && part_blocks <= kPStreamMaxPartBlocks && TS > 0 && TS <= n.W &&
                4LL * sh.S <= teams && 64LL * n.MP * sh.D < (1LL << 31);
    if (n.pstream) {
        const size_t gstride = static_cast<size_t>(std::min(16, G));
        n.frag = n.total;
        n.meta = n.frag + align_up(sizeof(float) * static_cast<size_t>(n.W) * (kFragHead + gstride * sh.D));
        n.total = n.meta + align_up(sizeof(int) * (static_cast<size_t>(sh.S) + 3));
    }
    return n;
}

// A wave combines a head in one batch of kReduceSmall rows for up to that
// many partitions per sequence; beyond, the four waves of a workgroup do.
template <int D>
hipError_t launch_reduce_t(const ReduceArgs& r, int S, hipStream_t stream) {
    if (r.MP <= kReduceSmall) {
        return launch(paged_reduce_wave_kernel<D, kReduceSmall>, dim3((r.H + 3) / 4, S), dim3(256), 0, stream, r);
    }
    return launch(paged_reduce_split_kernel<D>, dim3(r.H, S), dim3(256), 0, stream, r);
}

int validate_partition(const char* who, int partition_size) {
    if (partition_size < 0 || partition_size % kBlockTokens != 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                    "%s: partition_size %d must be 0 (balanced) or a positive multiple of 16", who,
                    partition_size);
    }
    return SWIFTLLM_OK;
}

// Balanced mode: waves resident per CU (3 per SIMD at the kernel's register
// count) times the device's CUs, so the whole grid runs in one round.
constexpr int kStreamWavesPerCU = 4 * kStreamWavesPerSimd;
constexpr int kDefaultCUs = 304;  // used to size workspaces when no device is visible

int device_cus() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kDefaultCUs;
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            return kDefaultCUs;
        }
        cache[dev] = n;
    }
    return cache[dev];
}

struct StreamNeed {
    int W;
    size_t frag, total;
};

StreamNeed stream_need(const Shape& sh, int cus) {
    StreamNeed n{};
    n.W = cus * kStreamWavesPerCU;
    const size_t gstride = static_cast<size_t>(std::min(16, sh.H / sh.Hkv));
    n.frag = align_up(sizeof(float) * 2 * static_cast<size_t>(n.W) * (kFragHead + gstride * sh.D));
    n.total = n.frag + align_up(sizeof(long long) * (4 * static_cast<size_t>(n.W) + 1));
    return n;
}

int decode_balanced(void* out, void* ws, size_t ws_bytes, const void* q, const void* kc,
                    const void* vc, const int* bt, const int* ctx, float scale, const Shape& sh,
                    int num_blocks, hipStream_t stream, const char* who) {
    const StreamNeed need = stream_need(sh, device_cus());
    if (ws_bytes < need.total) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: workspace of %zu bytes, %zu needed", who,
                    ws_bytes, need.total);
    }
    DecodeArgs d = make_args(out, q, kc, vc, bt, ctx, scale, sh, num_blocks);
    StreamArgs a{};
    a.out = d.out;
    a.q = d.q;
    a.kc = d.kc;
    a.vc = d.vc;
    a.bt = bt;
    a.ctx = ctx;
    a.frag = reinterpret_cast<float*>(ws);
    a.meta = reinterpret_cast<long long*>(static_cast<char*>(ws) + need.frag);
    a.scale_log2 = d.scale_log2;
    a.S = sh.S;
    a.H = sh.H;
    a.Hkv = sh.Hkv;
    a.G = d.G;
    a.nhc = d.nhc;
    a.MB = sh.MB;
    a.num_blocks = num_blocks;
    a.W = need.W;
    const size_t lds = sizeof(int) * (2 * static_cast<size_t>(sh.S) + 1);
    const dim3 grid(need.W / kStreamWaves);
    hipError_t err = sh.D == 128
        ? launch(paged_decode_streamk_kernel<128>, grid, dim3(64 * kStreamWaves), lds, stream, a)
        : launch(paged_decode_streamk_kernel<64>, grid, dim3(64 * kStreamWaves), lds, stream, a);
    if (err != hipSuccess) return launched(err, who);
    StreamReduceArgs r{};
    r.out = a.out;
    r.frag = a.frag;
    r.meta = a.meta;
    r.H = a.H;
    r.Hkv = a.Hkv;
    r.G = a.G;
    r.nhc = a.nhc;
    r.W = a.W;
    r.gstride = std::min(16, a.G);
    const dim3 rgrid(need.W, (r.gstride + 3) / 4);
    err = sh.D == 128 ? launch(paged_streamk_reduce_kernel<128>, rgrid, dim3(256), 0, stream, r)
                      : launch(paged_streamk_reduce_kernel<64>, rgrid, dim3(256), 0, stream, r);
    return launched(err, who);
}

// The partition size a v2 call runs with: balanced mode (0) needs its
// prefix table in LDS and at least 4 teams of Hkv * nhc waves; otherwise it
// falls back to partitions of 512 tokens.
int effective_partition(const Shape& sh, int partition_size, int cus) {
    if (partition_size == 0 &&
        (sh.S > kStreamMaxSeqs ||
         static_cast<long long>(sh.Hkv) * ((sh.H / sh.Hkv + 15) / 16) * 4 > cus * kStreamWavesPerCU)) {
        return 512;
    }
    return partition_size;
}

// Workspace bytes a v2 call with this (effective) partition size uses.
size_t v2_bytes(const Shape& sh, int partition_size, int cus) {
    return partition_size == 0 ? stream_need(sh, cus).total : v2_need(sh, partition_size, cus).total;
}

// Partition streams, then their reduce (which also combines a partition
// split by a range boundary when the sequence has one partition).
int decode_pstream(DecodeArgs& a, char* base, const V2Need& need, const Shape& sh,
                   hipStream_t stream, const char* who) {
    a.frag = reinterpret_cast<float*>(base + need.frag);
    a.meta = reinterpret_cast<int*>(base + need.meta);
    a.W = need.W;
    // Dynamic LDS: the block prefix and lengths (2S + 1 ints), then every
    // wave's slot for one held partial (16-byte aligned).
    a.stage_off = static_cast<int>((2 * static_cast<size_t>(sh.S) + 1 + 3) & ~static_cast<size_t>(3));
    const size_t stage = static_cast<size_t>(kStreamWaves) * 64 * sizeof(float) *
                         (sh.D == 128 ? kStageFloats<128> : kStageFloats<64>);
    const size_t lds = sizeof(int) * static_cast<size_t>(a.stage_off) + stage;
    const dim3 grid(need.W / kStreamWaves);
    hipError_t err = sh.D == 128
        ? launch(paged_partition_stream_kernel<128>, grid, dim3(64 * kStreamWaves), lds, stream, a)
        : launch(paged_partition_stream_kernel<64>, grid, dim3(64 * kStreamWaves), lds, stream, a);
    if (err != hipSuccess) return launched(err, who);
    PStreamReduceArgs r{};
    r.out = a.out;
    r.ws_max = a.ws_max;
    r.ws_sum = a.ws_sum;
    r.ws_out = a.ws_out;
    r.frag = a.frag;
    r.meta = a.meta;
    r.H = a.H;
    r.G = a.G;
    r.nhc = a.nhc;
    r.MP = a.MP;
    r.part_blocks = a.part_blocks;
    r.gstride = std::min(16, a.G);
    r.TS = a.Hkv * a.nhc;
    // Partition slots and boundary slots: at most MP + (MP - 1) fragments
    // per head when every partition holds a boundary.
    const dim3 rgrid((a.H + 3) / 4, sh.S);
    if (2 * a.MP - 1 <= kReduceSmall) {
        err = sh.D == 128 ? launch(paged_reduce_pstream_wave_kernel<128, kReduceSmall>, rgrid, dim3(256), 0, stream, r)
                          : launch(paged_reduce_pstream_wave_kernel<64, kReduceSmall>, rgrid, dim3(256), 0, stream, r);
    } else {
        const dim3 sgrid(a.H, sh.S);
        err = sh.D == 128 ? launch(paged_reduce_pstream_split_kernel<128>, sgrid, dim3(256), 0, stream, r)
                          : launch(paged_reduce_pstream_split_kernel<64>, sgrid, dim3(256), 0, stream, r);
    }
    return launched(err, who);
}

int decode_v2(void* out, void* ws, size_t ws_bytes, const void* q, const void* kc, const void* vc,
              const int* bt, const int* ctx, float scale, const Shape& sh, int partition_size,
              int num_blocks, hipStream_t stream, const char* who) {
    int rc = validate_decode(who, out, q, kc, vc, bt, ctx, sh);
    if (rc != SWIFTLLM_OK) return rc;
    if ((rc = validate_partition(who, partition_size)) != SWIFTLLM_OK) return rc;
    partition_size = effective_partition(sh, partition_size, device_cus());
    if (partition_size == 0) {
        if (sh.S > 0 && (ws == nullptr || !aligned(ws, 256))) {
            return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: workspace null or not 256-byte aligned", who);
        }
        if ((rc = require_device()) != SWIFTLLM_OK) return rc;
        if (sh.S == 0) return ok();
        return decode_balanced(out, ws, ws_bytes, q, kc, vc, bt, ctx, scale, sh, num_blocks, stream, who);
    }
    const V2Need need = v2_need(sh, partition_size, device_cus());
    if (sh.S > 0) {
        if (ws == nullptr || !aligned(ws, 256)) {
            return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: workspace null or not 256-byte aligned", who);
        }
        if (ws_bytes < need.total) {
            return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: workspace of %zu bytes, %zu needed", who,
                        ws_bytes, need.total);
        }
    }
    if ((rc = require_device()) != SWIFTLLM_OK) return rc;
    if (sh.S == 0) return ok();
    DecodeArgs a = make_args(out, q, kc, vc, bt, ctx, scale, sh, num_blocks);
    char* base = static_cast<char*>(ws);
    a.ws_max = reinterpret_cast<float*>(base);
    a.ws_sum = reinterpret_cast<float*>(base + need.stat);
    a.ws_out = reinterpret_cast<float*>(base + 2 * need.stat);
    a.part_blocks = partition_size / kBlockTokens;
    a.MP = need.MP;
    if (need.pstream) return decode_pstream(a, base, need, sh, stream, who);
    bool too_large = false;
    hipError_t err = launch_partition<kWavesV2>(a, sh.D, stream, &too_large);
    if (too_large) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: %d sequences x %d partitions is too many",
                    who, sh.S, need.MP);
    }
    if (err != hipSuccess || need.MP <= 1) return launched(err, who);
    ReduceArgs r{};
    r.out = a.out;
    r.ctx = ctx;
    r.ws_max = a.ws_max;
    r.ws_sum = a.ws_sum;
    r.ws_out = a.ws_out;
    r.H = a.H;
    r.MB = a.MB;
    r.part_blocks = a.part_blocks;
    r.MP = a.MP;
    err = sh.D == 128 ? launch_reduce_t<128>(r, sh.S, stream)
                      : launch_reduce_t<64>(r, sh.S, stream);
    return launched(err, who);
}

}  // namespace
}  // namespace swiftllm

// ---------------------------------------------------------------------------
// Split-K decode with no allocation. Some callers cannot allocate (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc),
// so swiftllm_hip_launch_paged_attention_v2_noalloc takes its workspace from
// this static device array instead of an argument. Each device that loads the
// library holds its own copy until the process ends. All calls on a device
// share that copy: calls that overlap on one device (several streams or host
// threads) race on it and must be ordered on one stream. The split-K
// workspace is plain scratch (a call reads only what it wrote first), so
// nothing is cleared between calls.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[SWIFTLLM_HIP_NOALLOC_SCRATCH_BYTES];

namespace swiftllm {
namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device, looked up on the first
// call on that device. In host code the array's name is only a host-side
// stand-in; this address is what kernels receive.
int static_scratch(void** ptr, const char* who) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        return fail(SWIFTLLM_ERR_DEVICE_NOT_FOUND, "%s: no current HIP device", who);
    }
    if (dev < 0 || dev >= kMaxScratchDevices) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: device %d beyond the %d the library tracks", who,
                    dev, kMaxScratchDevices);
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || p == nullptr) {
            return fail(SWIFTLLM_ERR_INIT, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev,
                        hipGetErrorString(err));
        }
        g_scratch[dev] = p;
    }
    *ptr = g_scratch[dev];
    return SWIFTLLM_OK;
}

int decode_v2_noalloc(void* out, const void* q, const void* kc, const void* vc, const int* bt,
                      const int* ctx, float scale, const Shape& sh, int partition_size,
                      int num_blocks, hipStream_t stream, const char* who) {
    int rc = validate_decode(who, out, q, kc, vc, bt, ctx, sh);
    if (rc != SWIFTLLM_OK) return rc;
    if ((rc = validate_partition(who, partition_size)) != SWIFTLLM_OK) return rc;
    const int cus = device_cus();
    const size_t need = v2_bytes(sh, effective_partition(sh, partition_size, cus), cus);
    if (need > SWIFTLLM_HIP_NOALLOC_SCRATCH_BYTES) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                    "%s: these sizes need %zu bytes of split-K scratch, more than the %zu bytes of "
                    "its static scratch; use swiftllm_hip_launch_paged_attention_v2 with a workspace",
                    who, need, static_cast<size_t>(SWIFTLLM_HIP_NOALLOC_SCRATCH_BYTES));
    }
    if ((rc = require_device()) != SWIFTLLM_OK) return rc;
    if (sh.S == 0) return ok();
    void* ws = nullptr;
    if ((rc = static_scratch(&ws, who)) != SWIFTLLM_OK) return rc;
    return decode_v2(out, ws, SWIFTLLM_HIP_NOALLOC_SCRATCH_BYTES, q, kc, vc, bt, ctx, scale, sh,
                     partition_size, num_blocks, stream, who);
}

}  // namespace
}  // namespace swiftllm

using namespace swiftllm;

extern "C" {

void launch_paged_attention_v1(void* output, void* query, void* key_cache, void* value_cache,
                               int* block_tables, int* context_lens, float scale, int num_seqs,
                               int num_heads, int num_kv_heads, int head_dim, int block_size,
                               int max_num_blocks_per_seq, hipStream_t stream) {
    const Shape sh{num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_num_blocks_per_seq};
    decode_v1(output, query, key_cache, value_cache, block_tables, context_lens, scale, sh, 0,
              stream, "launch_paged_attention_v1");
}

int swiftllm_hip_launch_paged_attention_v1(void* output, const void* query, const void* key_cache,
                                           const void* value_cache, const int* block_tables,
                                           const int* context_lens, float scale, int num_seqs,
                                           int num_heads, int num_kv_heads, int head_dim,
                                           int block_size, int max_num_blocks_per_seq,
                                           int num_blocks, hipStream_t stream) {
    const Shape sh{num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_num_blocks_per_seq};
    return decode_v1(output, query, key_cache, value_cache, block_tables, context_lens, scale, sh,
                     num_blocks, stream, "swiftllm_hip_launch_paged_attention_v1");
}

void launch_paged_attention_v2(void* output, void* workspace, size_t workspace_bytes, void* query,
                               void* key_cache, void* value_cache, int* block_tables,
                               int* context_lens, float scale, int num_seqs, int num_heads,
                               int num_kv_heads, int head_dim, int block_size,
                               int max_num_blocks_per_seq, int partition_size, hipStream_t stream) {
    const Shape sh{num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_num_blocks_per_seq};
    decode_v2(output, workspace, workspace_bytes, query, key_cache, value_cache, block_tables,
              context_lens, scale, sh, partition_size, 0, stream, "launch_paged_attention_v2");
}

int swiftllm_hip_launch_paged_attention_v2(void* output, void* workspace, size_t workspace_bytes,
                                           const void* query, const void* key_cache,
                                           const void* value_cache, const int* block_tables,
                                           const int* context_lens, float scale, int num_seqs,
                                           int num_heads, int num_kv_heads, int head_dim,
                                           int block_size, int max_num_blocks_per_seq,
                                           int partition_size, int num_blocks, hipStream_t stream) {
    const Shape sh{num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_num_blocks_per_seq};
    return decode_v2(output, workspace, workspace_bytes, query, key_cache, value_cache, block_tables,
                     context_lens, scale, sh, partition_size, num_blocks, stream,
                     "swiftllm_hip_launch_paged_attention_v2");
}

int swiftllm_hip_launch_paged_attention_v2_noalloc(void* output, const void* query,
                                                   const void* key_cache, const void* value_cache,
                                                   const int* block_tables, const int* context_lens,
                                                   float scale, int num_seqs, int num_heads,
                                                   int num_kv_heads, int head_dim, int block_size,
                                                   int max_num_blocks_per_seq, int partition_size,
                                                   int num_blocks, hipStream_t stream) {
    const Shape sh{num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_num_blocks_per_seq};
    return decode_v2_noalloc(output, query, key_cache, value_cache, block_tables, context_lens,
                             scale, sh, partition_size, num_blocks, stream,
                             "swiftllm_hip_launch_paged_attention_v2_noalloc");
}

size_t swiftllm_hip_paged_attention_v2_workspace_size(int num_seqs, int num_heads, int num_kv_heads,
                                                      int head_dim, int block_size,
                                                      int max_num_blocks_per_seq,
                                                      int partition_size) {
    if (num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
        head_dim <= 0 || block_size != kBlockTokens || max_num_blocks_per_seq < 0 ||
        partition_size < 0 || partition_size % kBlockTokens != 0) {
        fail(SWIFTLLM_ERR_INVALID_PARAMETER, "swiftllm_hip_paged_attention_v2_workspace_size: bad shape");
        return 0;
    }
    const Shape sh{num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_num_blocks_per_seq};
    ok();
    if (partition_size == 0) {
        int n = 0;
        const int cus = (hipGetDeviceCount(&n) == hipSuccess && n > 0) ? device_cus() : kDefaultCUs;
        // the balanced workspace also covers its partitioned fallback
        return std::max(stream_need(sh, cus).total, v2_need(sh, 512, cus).total);
    }
    int n = 0;
    const int cus = (hipGetDeviceCount(&n) == hipSuccess && n > 0) ? device_cus() : kDefaultCUs;
    return v2_need(sh, partition_size, cus).total;
}

int swiftllm_hip_workspace_clear(void* workspace, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return ok();
    if (workspace == nullptr || !aligned(workspace, 4) || bytes % 4 != 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                    "swiftllm_hip_workspace_clear: null or misaligned workspace / size");
    }
    int rc = require_device();
    if (rc != SWIFTLLM_OK) return rc;
    ClearArgs a{static_cast<uint32_t*>(workspace), bytes / 4};
    const size_t blocks = (a.words + 255) / 256;
    const unsigned grid = static_cast<unsigned>(blocks < 4096 ? blocks : 4096);
    return launched(launch(clear_kernel, dim3(grid), dim3(256), 0, stream, a),
                    "swiftllm_hip_workspace_clear");
}

int swiftllm_hip_paged_attention_decode(void* output, const void* query, const void* key_cache,
                                        const void* value_cache, const int32_t* block_tables,
                                        const int32_t* context_lens,
                                        const swiftllm_paged_attention_params* p,
                                        hipStream_t stream) {
    const char* who = "swiftllm_hip_paged_attention_decode";
    if (p == nullptr) return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null params", who);
    const size_t lim = 0x7fffffff;
    if (p->num_seqs > lim || p->num_heads > lim || p->num_kv_heads > lim || p->head_dim > lim ||
        p->block_size > lim || p->max_context_len > lim || p->block_size == 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: parameter out of range", who);
    }
    const size_t mb = (p->max_context_len + p->block_size - 1) / p->block_size;
    const Shape sh{static_cast<int>(p->num_seqs), static_cast<int>(p->num_heads),
                   static_cast<int>(p->num_kv_heads), static_cast<int>(p->head_dim),
                   static_cast<int>(p->block_size), static_cast<int>(mb)};
    return decode_v1(output, query, key_cache, value_cache, block_tables, context_lens, p->scale,
                     sh, 0, stream, who);
}

int swiftllm_hip_gather_kv(const void* key_cache, const void* value_cache, const int* block_tables,
                           const int* context_lens, int seq, int kv_head, int num_kv_heads,
                           int head_dim, int block_size, int max_num_blocks_per_seq,
                           int max_context_len, void* k_out, void* v_out, hipStream_t stream) {
    const char* who = "swiftllm_hip_gather_kv";
    if (seq < 0 || num_kv_heads <= 0 || kv_head < 0 || kv_head >= num_kv_heads || head_dim <= 0 ||
        max_num_blocks_per_seq < 0 || max_context_len < 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: bad shape", who);
    }
    if (block_size != kBlockTokens) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: block_size %d (supported: 16)", who, block_size);
    }
    if (max_context_len > 0 &&
        (!key_cache || !value_cache || !block_tables || !context_lens || !k_out || !v_out)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    int rc = require_device();
    if (rc != SWIFTLLM_OK) return rc;
    if (max_context_len == 0) return ok();
    GatherArgs a{static_cast<const uint16_t*>(key_cache), static_cast<const uint16_t*>(value_cache),
                 block_tables, context_lens, static_cast<uint16_t*>(k_out),
                 static_cast<uint16_t*>(v_out), seq, kv_head, num_kv_heads, head_dim,
                 max_num_blocks_per_seq, max_context_len};
    const size_t n = static_cast<size_t>(max_context_len) * head_dim;
    const size_t blocks = (n + 255) / 256;
    const unsigned grid = static_cast<unsigned>(blocks < 65535 ? blocks : 65535);
    return launched(launch(gather_kv_kernel, dim3(grid), dim3(256), 0, stream, a), who);
}

}  // extern "C"
