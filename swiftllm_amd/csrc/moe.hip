// MoE top-k routing and expert-contiguous dispatch for gfx950.
//
// The reference names the steps in MoeMlp::forward
// (crates/swiftllm-models/src/layers/mlp.rs:240-246: router logits, top-k,
// route, combine) and returns zeros (:247-251). Conventions come from the
// reference's sampling code: softmax subtracts the max
// (crates/swiftllm-core/src/sampling/mod.rs:380-385) and ranking is a stable
// descending sort, so equal logits keep the lower index first (:367-377).
//
// route:    one thread per token; K argmax passes over the E logits (value
//           descending, ties to the lower index), then weights
//           w_k = exp(x_k - x_max) / sum_k' exp(x_k' - x_max), which equals the
//           softmax probabilities renormalised over the selected experts, in
//           fp32. Rows of up to 8 or 16 logits are loaded into registers at
//           once.
// dispatch: two kernels, with no grid-wide synchronisation inside either.
//           (1) rank: one wave per 64-token chunk ranks the chunk's entries
//               among equal experts with ballots (stable (t, k) order; for up
//               to 16 experts one unrolled pass of ballots and mbcnt per
//               expert) and stores per-(chunk, expert) counts. The fused entry point routes
//               the chunk's tokens first, in the same wave.
//           (2) permute: each workgroup scans the chunk counts (up to 4096
//               of them) in LDS into per-(chunk, expert) prefixes and expert
//               offsets, while the first loads of its rows are in flight.
//               Then one wave per token computes the K destination rows,
//               writes the inverse index and sorted token ids, and copies the
//               token's row once from HBM into its K destinations, every load
//               of a batch issued before its stores. Rows are read with
//               nontemporal loads and written with nontemporal stores (both
//               measured faster than plain ones for this one-read, K-write
//               pattern).
//           Larger count matrices get a scan kernel between the two: one
//           workgroup per expert turns its column into exclusive prefixes
//           and the expert's total.
//           Kernel boundaries order the phases, so the workspace needs no
//           initialisation and no device-scope fences are issued.

#include <climits>
#include <cmath>

#include "common.hpp"

namespace swiftllm {
namespace {

constexpr int kMaxTopK = 8;
constexpr int kMaxExperts = 256;
constexpr int kChunkTokens = 64;  // tokens per ranking wave

struct RouteArgs {
    const float* logits;
    int* ids;
    float* w;
    int T;
    int E;
};

// Rows of up to R experts (8 or 16) are held in registers: the route and rank
// kernels are instantiated for both, and wider rows take the loop over memory.

// One argmax pass of the top-K selection: the largest logit among experts
// not yet taken; the strict '>' keeps the lowest index among equal logits.
template <int K>
__device__ __forceinline__ void consider(int e, float x, int k, const int (&bi)[K], float& best,
                                         int& besti) {
    bool taken = false;
#pragma unroll
    for (int j = 0; j < K; ++j) taken = taken || (j < k && bi[j] == e);
    if (!taken && (besti < 0 || x > best)) {
        best = x;
        besti = e;
    }
}

// Writes ids and weights w_k = exp(x_k - x_0) / sum_k' exp(x_k' - x_0) of token t,
// in fp32: every exponent is <= 0 and the sum lies in [1, K], so the weights
// are within a few fp32 ulps (under 1e-6) of the fp64 values.
template <int K>
__device__ __forceinline__ void write_route(const RouteArgs& a, int t, const float (&bv)[K],
                                            const int (&bi)[K]) {
    float ex[K];
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        ex[k] = expf(bv[k] - bv[0]);
        sum += ex[k];
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        a.ids[static_cast<size_t>(t) * K + k] = bi[k];
        a.w[static_cast<size_t>(t) * K + k] = ex[k] / sum;
    }
}

// Top-K of one row of logits into bv (values) and bi (expert ids).
template <int K, int R>
__device__ __forceinline__ void select_topk(const float* row, int E, float (&bv)[K], int (&bi)[K]) {
    static_assert(R == 8 || R == 16, "register row width");
#pragma unroll
    for (int k = 0; k < K; ++k) bi[k] = -1;
    if (E <= R) {
        // All loads issued together (16-byte loads when the row allows); the K
        // passes then run on registers.
        float v[R];
        if ((E & 3) == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0) {
            typedef float f4v __attribute__((ext_vector_type(4)));
            // Every load is issued, the ones past the row re-reading its
            // first 16 bytes, so no branch separates them and one wait
            // covers all.
            f4v x[R / 4];
#pragma unroll
            for (int q = 0; q < R / 4; ++q) x[q] = reinterpret_cast<const f4v*>(row)[4 * q < E ? q : 0];
#pragma unroll
            for (int q = 0; q < R / 4; ++q) {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[4 * q + i] = (4 * q < E) ? x[q][i] : 0.0f;
            }
        } else {
#pragma unroll
            for (int e = 0; e < R; ++e) v[e] = (e < E) ? row[e] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            float best = 0.0f;
            int besti = -1;
#pragma unroll
            for (int e = 0; e < R; ++e) {
                if (e < E) consider<K>(e, v[e], k, bi, best, besti);
            }
            bv[k] = best;
            bi[k] = besti;
        }
    } else {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            float best = 0.0f;
            int besti = -1;
            for (int e = 0; e < E; ++e) consider<K>(e, row[e], k, bi, best, besti);
            bv[k] = best;
            bi[k] = besti;
        }
    }
}

template <int K, int R>
__global__ __launch_bounds__(256) void moe_route_kernel(const RouteArgs a) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= a.T) return;
    float bv[K];
    int bi[K];
    select_topk<K, R>(a.logits + static_cast<size_t>(t) * a.E, a.E, bv, bi);
    write_route<K>(a, t, bv, bi);
}

// Ranks the entries of one 64-token chunk among equal experts, stable in
// (t, k) order: rk[k] = number of earlier entries of the chunk with the same
// expert, or -1 for an id outside [0, E). Lane 0 stores the count of every
// expert present in the chunk to cnt[e]; entries of absent experts are left
// as they are. One round per distinct expert: the lowest pending entry of
// the wave names the expert, and ballots over the K slots give each entry
// the number of equal entries below it.
template <int K>
__device__ __forceinline__ void rank_chunk(const int (&id)[K], int (&rk)[K], int E, int lane,
                                           int* cnt) {
    bool pend[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        pend[k] = id[k] >= 0 && id[k] < E;
        rk[k] = -1;
    }
    const unsigned long long below_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    while (true) {
        int cand = -1;
#pragma unroll
        for (int k = K - 1; k >= 0; --k) {
            if (pend[k]) cand = id[k];
        }
        const unsigned long long any = __ballot(cand >= 0);
        if (any == 0ull) break;
        const int e = __builtin_amdgcn_readlane(cand, __ffsll(static_cast<long long>(any)) - 1);
        int below = 0, total = 0;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const unsigned long long m = __ballot(pend[k] && id[k] == e);
            below += __popcll(m & below_mask);
            total += __popcll(m);
        }
        int own = 0;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            if (pend[k] && id[k] == e) {
                rk[k] = below + own;
                ++own;
                pend[k] = false;
            }
        }
        if (lane == 0) cnt[e] = total;
    }
}

// rank_chunk for E <= kRankUnrolled, with no loop-carried branch: for each
// expert e, K ballots give the chunk's entries of e per top-k slot, and
// mbcnt counts those below the lane. An entry (t, k) of expert e ranks after
// every entry of e at a lower token (any slot) and after the token's own
// slots k' < k holding e. Lane e < E returns expert e's count in `cnt`.
constexpr int kRankUnrolled = 16;

template <int K>
__device__ __forceinline__ void rank_chunk_unrolled(const int (&id)[K], int (&rk)[K], int E, int lane,
                                                    int& cnt) {
    bool ok[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        ok[k] = id[k] >= 0 && id[k] < E;
        rk[k] = -1;
    }
    cnt = 0;
#pragma unroll
    for (int e = 0; e < kRankUnrolled; ++e) {
        if (e < E) {  // wave-uniform
            int below = 0, total = 0;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const unsigned long long m = __ballot(ok[k] && id[k] == e);
                below += __builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(m >> 32),
                                                   __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(m), 0u));
                total += __popcll(m);
            }
            int own = 0;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                if (ok[k] && id[k] == e) {
                    rk[k] = below + own;
                    ++own;
                }
            }
            if (lane == e) cnt = total;
        }
    }
}

// ---------------------------------------------------------------------------
// (1) Rank, optionally after routing.
// ---------------------------------------------------------------------------
struct RankArgs {
    const float* logits;  // non-null: route the chunk first (ids and w are outputs)
    int* ids;             // [T*K]
    float* w;             // [T*K], with logits
    int* rank;            // [T*K] rank among equal experts inside the 64-token chunk
    int* cnt;             // [nchunks][E] counts
    int T;
    int E;
    int nchunks;
};

constexpr int kRankWaves = 4;

template <int K, int R>
__global__ __launch_bounds__(64 * kRankWaves) void moe_rank_kernel(const RankArgs a) {
    __shared__ int s_cnt[kRankWaves][kMaxExperts];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int c = blockIdx.x * kRankWaves + wv;  // chunk of this wave
    if (c >= a.nchunks) return;                   // whole waves only; no barriers below
    if (a.E > kRankUnrolled) {
        for (int e = lane; e < a.E; e += 64) s_cnt[wv][e] = 0;
    }

    const int t = c * kChunkTokens + lane;
    const bool live = t < a.T;
    int id[K], rk[K];
    if (a.logits != nullptr) {
        float bv[K];
        if (live) {
            select_topk<K, R>(a.logits + static_cast<size_t>(t) * a.E, a.E, bv, id);
            RouteArgs ra{a.logits, a.ids, a.w, a.T, a.E};
            write_route<K>(ra, t, bv, id);
        } else {
#pragma unroll
            for (int k = 0; k < K; ++k) id[k] = -1;
        }
    } else {
#pragma unroll
        for (int k = 0; k < K; ++k) id[k] = live ? a.ids[static_cast<size_t>(t) * K + k] : -1;
    }
    if (a.E <= kRankUnrolled) {
        int cnt;
        rank_chunk_unrolled<K>(id, rk, a.E, lane, cnt);
        if (live) {
#pragma unroll
            for (int k = 0; k < K; ++k) a.rank[static_cast<size_t>(t) * K + k] = rk[k];
        }
        if (lane < a.E) a.cnt[static_cast<size_t>(c) * a.E + lane] = cnt;
        return;
    }
    rank_chunk<K>(id, rk, a.E, lane, s_cnt[wv]);
    if (live) {
#pragma unroll
        for (int k = 0; k < K; ++k) a.rank[static_cast<size_t>(t) * K + k] = rk[k];
    }
    // LDS operations of one wave complete in order: lane 0's counts are seen.
    for (int e = lane; e < a.E; e += 64) a.cnt[static_cast<size_t>(c) * a.E + e] = s_cnt[wv][e];
}

// ---------------------------------------------------------------------------
// (2) Scan: workgroup e turns column e of the chunk counts into exclusive
// prefixes and writes the expert's total.
// ---------------------------------------------------------------------------
constexpr int kScanThreads = 256;

struct ScanArgs {
    const int* cnt;  // [nchunks][E]
    int* base;       // [nchunks][E] entries of the expert in earlier chunks
    int* tot;        // [E]
    int nchunks;
    int E;
};

__global__ __launch_bounds__(kScanThreads) void moe_scan_kernel(const ScanArgs a) {
    __shared__ int s_wave[kScanThreads / 64];
    const int e = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    // Thread i owns chunks [i * per, (i + 1) * per).
    const int per = (a.nchunks + kScanThreads - 1) / kScanThreads;
    const int c0 = threadIdx.x * per;
    const int c1 = min(c0 + per, a.nchunks);
    int sum = 0;
    for (int c = c0; c < c1; ++c) sum += a.cnt[static_cast<size_t>(c) * a.E + e];
    const int x = wave_inclusive_scan(sum, lane);
    if (lane == 63) s_wave[wv] = x;
    __syncthreads();
    int run = x - sum;
    int total = 0;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; ++w) {
        run += (w < wv) ? s_wave[w] : 0;
        total += s_wave[w];
    }
    for (int c = c0; c < c1; ++c) {
        const size_t i = static_cast<size_t>(c) * a.E + e;
        const int v = a.cnt[i];
        a.base[i] = run;
        run += v;
    }
    if (threadIdx.x == 0) a.tot[e] = total;
}

// ---------------------------------------------------------------------------
// (3) Permute.
// ---------------------------------------------------------------------------
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kCopyBatch = 8;          // 16-byte loads per lane in flight before the stores
constexpr int kPermuteWaves = 4;       // one token per wave
constexpr int kLdsCounts = 4096;       // count matrices up to this size are scanned in LDS

struct PermuteArgs {
    const int* ids;
    const int* rank;
    const int* cnt;   // [nchunks][E] counts; scanned in LDS when `base` is null
    const int* base;  // [nchunks][E] prefixes from the scan kernel, or null
    const int* tot;   // [E] totals from the scan kernel (with `base`)
    const uint16_t* x;
    uint16_t* xp;     // null: index arrays only
    int* counts;
    int* offsets;
    int* inverse;
    int* sorted;
    int T;
    int E;
    int nchunks;
    int hidden;
    int vec;  // 1: rows move as 16-byte vectors
};

// VEC: rows move as 16-byte vectors (a.xp set and a.vec); otherwise index
// arrays only, or a 2-byte copy of unaligned rows.
template <int K, bool VEC>
__global__ __launch_bounds__(64 * kPermuteWaves) void moe_permute_kernel(const PermuteArgs a) {
    __shared__ int s_base[kLdsCounts];  // [nchunks][E] exclusive prefixes over chunks
    __shared__ int s_off[kMaxExperts];  // expert offsets
    if (a.T == 0) {
        // No tokens (one workgroup): zero counts and offsets. Below, T >= 1,
        // so the clamped indices of the preloads are valid.
        for (int e = threadIdx.x; e < a.E; e += blockDim.x) a.counts[e] = 0;
        for (int e = threadIdx.x; e <= a.E; e += blockDim.x) a.offsets[e] = 0;
        return;
    }
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int t = blockIdx.x * kPermuteWaves + wv;
    const bool live = t < a.T;
    const int nv = a.hidden / 8;
    const u32x4* __restrict__ src =
        reinterpret_cast<const u32x4*>(a.x + static_cast<size_t>(min(t, a.T - 1)) * a.hidden);

    // Loads in the order their values are needed, since the memory counter
    // completes in order: the chunk counts (scanned first), the token's expert
    // ids and ranks, then the first batch of the row, whose latency hides the
    // scans. Every load is issued unconditionally (out-of-range ones re-read a
    // valid element and are discarded), so no branch merge makes the compiler
    // wait for all of them before the first count is used.
    constexpr int kCntPerThread = kLdsCounts / (64 * kPermuteWaves);
    const int n = a.nchunks * a.E;
    int cv[kCntPerThread];
    if (a.base == nullptr) {
#pragma unroll
        for (int j = 0; j < kCntPerThread; ++j) {
            const int i = threadIdx.x + 64 * kPermuteWaves * j;
            cv[j] = a.cnt[min(i, n - 1)];
        }
    }
    const int tc = min(t, a.T - 1);
    int eid[K], erk[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        eid[k] = a.ids[static_cast<size_t>(tc) * K + k];
        erk[k] = a.rank[static_cast<size_t>(tc) * K + k];
    }
    u32x4 v[kCopyBatch];
    if constexpr (VEC) {
#pragma unroll
        for (int u = 0; u < kCopyBatch; ++u) v[u] = __builtin_nontemporal_load(src + min(64 * u + lane, nv - 1));
    }

    // Per-expert totals: from the scan kernel, or scanned here from the counts.
    if (a.base == nullptr) {
#pragma unroll
        for (int j = 0; j < kCntPerThread; ++j) {
            const int i = threadIdx.x + 64 * kPermuteWaves * j;
            if (i < n) s_base[i] = cv[j];
        }
        __syncthreads();
        // One wave per expert column, 64 chunks per step.
        for (int e = wv; e < a.E; e += kPermuteWaves) {
            int run = 0;
            for (int c0 = 0; c0 < a.nchunks; c0 += 64) {
                const int c = c0 + lane;
                const int val = (c < a.nchunks) ? s_base[c * a.E + e] : 0;
                const int x = wave_inclusive_scan(val, lane);
                if (c < a.nchunks) s_base[c * a.E + e] = run + x - val;
                run += __shfl(x, 63);
            }
            if (lane == 0) s_off[e] = run;
        }
    } else {
        for (int e = threadIdx.x; e < a.E; e += 64 * kPermuteWaves) s_off[e] = a.tot[e];
    }
    __syncthreads();
    // Expert offsets: exclusive scan of the totals; workgroup 0 also
    // publishes counts and offsets.
    if (wv == 0) {
        int run = 0;
        for (int e0 = 0; e0 < a.E; e0 += 64) {
            const int e = e0 + lane;
            const int val = (e < a.E) ? s_off[e] : 0;
            const int x = wave_inclusive_scan(val, lane);
            if (e < a.E) {
                s_off[e] = run + x - val;
                if (blockIdx.x == 0) {
                    a.counts[e] = val;
                    a.offsets[e] = run + x - val;
                }
            }
            run += __shfl(x, 63);
        }
        if (blockIdx.x == 0 && lane == 0) a.offsets[a.E] = run;
    }
    __syncthreads();
    if (!live) return;

    const int c = t / kChunkTokens;
    long long rows[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int e = eid[k];
        const int rk = erk[k];
        int row = -1;
        if (e >= 0 && e < a.E && rk >= 0) {
            const size_t ce = static_cast<size_t>(c) * a.E + e;
            row = s_off[e] + (a.base != nullptr ? a.base[ce] : s_base[ce]) + rk;
        }
        rows[k] = row;
        if (lane == 0) {
            a.inverse[static_cast<size_t>(t) * K + k] = row;
            if (row >= 0) a.sorted[row] = t;
        }
    }
    if (a.xp == nullptr) return;
    if constexpr (VEC) {
        for (int i0 = 0; i0 < nv; i0 += 64 * kCopyBatch) {
            if (i0 > 0) {
#pragma unroll
                for (int u = 0; u < kCopyBatch; ++u) {
                    const int i = i0 + 64 * u + lane;
                    if (i < nv) v[u] = __builtin_nontemporal_load(src + i);
                }
            }
#pragma unroll
            for (int k = 0; k < K; ++k) {
                if (rows[k] < 0) continue;
                u32x4* __restrict__ dst = reinterpret_cast<u32x4*>(a.xp + rows[k] * a.hidden);
#pragma unroll
                for (int u = 0; u < kCopyBatch; ++u) {
                    const int i = i0 + 64 * u + lane;
                    if (i < nv) __builtin_nontemporal_store(v[u], dst + i);
                }
            }
        }
    } else {
        const uint16_t* s16 = a.x + static_cast<size_t>(t) * a.hidden;
        for (int i = lane; i < a.hidden; i += 64) {
            const uint16_t val = s16[i];
#pragma unroll
            for (int k = 0; k < K; ++k) {
                if (rows[k] >= 0) a.xp[rows[k] * a.hidden + i] = val;
            }
        }
    }
}

template <template <int> class Fn, typename... Args>
hipError_t by_k(int K, Args&&... args) {
    switch (K) {
        case 1: return Fn<1>::run(args...);
        case 2: return Fn<2>::run(args...);
        case 3: return Fn<3>::run(args...);
        case 4: return Fn<4>::run(args...);
        case 5: return Fn<5>::run(args...);
        case 6: return Fn<6>::run(args...);
        case 7: return Fn<7>::run(args...);
        default: return Fn<8>::run(args...);
    }
}

template <int K>
struct RouteLaunch {
    static hipError_t run(const RouteArgs& a, hipStream_t s) {
        if (a.E <= 8) return launch(moe_route_kernel<K, 8>, dim3((a.T + 255) / 256), dim3(256), 0, s, a);
        return launch(moe_route_kernel<K, 16>, dim3((a.T + 255) / 256), dim3(256), 0, s, a);
    }
};

template <int K>
struct RankLaunch {
    static hipError_t run(const RankArgs& a, hipStream_t s) {
        const int grid = (a.nchunks + kRankWaves - 1) / kRankWaves;
        if (a.E <= 8) return launch(moe_rank_kernel<K, 8>, dim3(grid), dim3(64 * kRankWaves), 0, s, a);
        return launch(moe_rank_kernel<K, 16>, dim3(grid), dim3(64 * kRankWaves), 0, s, a);
    }
};

template <int K>
struct PermuteLaunch {
    static hipError_t run(const PermuteArgs& a, hipStream_t s) {
        // One wave per token; at least one workgroup so counts and offsets
        // are written when there are no tokens.
        const int grid = a.T > 0 ? (a.T + kPermuteWaves - 1) / kPermuteWaves : 1;
        if (a.xp != nullptr && a.vec) {
            return launch(moe_permute_kernel<K, true>, dim3(grid), dim3(64 * kPermuteWaves), 0, s, a);
        }
        return launch(moe_permute_kernel<K, false>, dim3(grid), dim3(64 * kPermuteWaves), 0, s, a);
    }
};

struct DispatchLayout {
    int nchunks;
    size_t cnt, base, tot, rank, total;
};

DispatchLayout dispatch_layout(int T, int E, int K) {
    DispatchLayout l{};
    l.nchunks = (T + kChunkTokens - 1) / kChunkTokens;
    auto up = [](size_t x) { return (x + 255) / 256 * 256; };
    const size_t counts = sizeof(int) * static_cast<size_t>(l.nchunks) * E;
    l.cnt = 0;
    l.base = l.cnt + up(counts);
    l.tot = l.base + up(counts);
    l.rank = l.tot + up(sizeof(int) * static_cast<size_t>(E));
    l.total = l.rank + up(sizeof(int) * static_cast<size_t>(T) * K);
    return l;
}

int validate_moe(const char* who, int T, int E, int K) {
    if (T < 0 || E <= 0 || K <= 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: num_tokens=%d num_experts=%d top_k=%d",
                    who, T, E, K);
    }
    if (K > kMaxTopK || E > kMaxExperts || K > E) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED,
                    "%s: top_k=%d num_experts=%d (supported: top_k <= 8, top_k <= num_experts <= 256)",
                    who, K, E);
    }
    return SWIFTLLM_OK;
}

}  // namespace
}  // namespace swiftllm

using namespace swiftllm;

extern "C" {

int swiftllm_hip_moe_route(const float* logits, int num_tokens, int num_experts, int top_k,
                           int32_t* expert_ids, float* weights, hipStream_t stream) {
    const char* who = "swiftllm_hip_moe_route";
    int rc = validate_moe(who, num_tokens, num_experts, top_k);
    if (rc != SWIFTLLM_OK) return rc;
    if (num_tokens > 0 && (!logits || !expert_ids || !weights)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    if ((rc = require_device()) != SWIFTLLM_OK) return rc;
    if (num_tokens == 0) return ok();
    RouteArgs a{logits, expert_ids, weights, num_tokens, num_experts};
    return launched(by_k<RouteLaunch>(top_k, a, stream), who);
}

size_t swiftllm_hip_moe_dispatch_workspace_size(int num_tokens, int num_experts, int top_k) {
    if (validate_moe("swiftllm_hip_moe_dispatch_workspace_size", num_tokens, num_experts, top_k) !=
        SWIFTLLM_OK) {
        return 0;
    }
    ok();
    return dispatch_layout(num_tokens, num_experts, top_k).total;
}

}  // extern "C"

namespace swiftllm {
namespace {

// Shared body of the dispatch entry points. With `logits`, the rank kernel
// routes each chunk first and writes expert_ids and weights.
int dispatch(const char* who, const float* logits, int32_t* expert_ids, float* weights,
             const void* x, int num_tokens, int top_k, int num_experts, int hidden,
             int32_t* expert_counts, int32_t* expert_offsets, void* x_perm, int32_t* inverse,
             int32_t* sorted_token_ids, void* workspace, size_t workspace_bytes,
             hipStream_t stream) {
    int rc = validate_moe(who, num_tokens, num_experts, top_k);
    if (rc != SWIFTLLM_OK) return rc;
    if (hidden < 0 || (x_perm != nullptr && hidden == 0)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: hidden=%d", who, hidden);
    }
    if (!expert_counts || !expert_offsets || !workspace) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    if (num_tokens > 0 && (!expert_ids || !inverse || !sorted_token_ids || (x_perm && !x) ||
                           (logits && !weights))) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    const DispatchLayout l = dispatch_layout(num_tokens, num_experts, top_k);
    if (!aligned(workspace, 256) || workspace_bytes < l.total) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                    "%s: workspace of %zu bytes (%zu needed, 256-byte aligned)", who,
                    workspace_bytes, l.total);
    }
    if (x_perm && (!aligned(x, 2) || !aligned(x_perm, 2))) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: misaligned activations", who);
    }
    if ((rc = require_device()) != SWIFTLLM_OK) return rc;
    char* ws = static_cast<char*>(workspace);
    int* cnt = reinterpret_cast<int*>(ws + l.cnt);
    int* base = reinterpret_cast<int*>(ws + l.base);
    int* tot = reinterpret_cast<int*>(ws + l.tot);
    int* rank = reinterpret_cast<int*>(ws + l.rank);
    if (num_tokens > 0) {
        RankArgs ra{logits, expert_ids, weights, rank, cnt, num_tokens, num_experts, l.nchunks};
        hipError_t err = by_k<RankLaunch>(top_k, ra, stream);
        if (err != hipSuccess) return launched(err, who);
    }
    PermuteArgs pa{};
    pa.cnt = cnt;
    if (static_cast<long long>(l.nchunks) * num_experts > kLdsCounts) {
        ScanArgs sa{cnt, base, tot, l.nchunks, num_experts};
        hipError_t err =
            launch(moe_scan_kernel, dim3(num_experts), dim3(kScanThreads), 0, stream, sa);
        if (err != hipSuccess) return launched(err, who);
        pa.base = base;
        pa.tot = tot;
    }
    pa.ids = expert_ids;
    pa.rank = rank;
    pa.x = static_cast<const uint16_t*>(x);
    pa.xp = static_cast<uint16_t*>(x_perm);
    pa.counts = expert_counts;
    pa.offsets = expert_offsets;
    pa.inverse = inverse;
    pa.sorted = sorted_token_ids;
    pa.T = num_tokens;
    pa.E = num_experts;
    pa.nchunks = l.nchunks;
    pa.hidden = hidden;
    pa.vec = (hidden % 8 == 0) && (x_perm == nullptr || (aligned(x, 16) && aligned(x_perm, 16)));
    return launched(by_k<PermuteLaunch>(top_k, pa, stream), who);
}

}  // namespace
}  // namespace swiftllm

extern "C" {

int swiftllm_hip_moe_dispatch(const int32_t* expert_ids, const void* x, int num_tokens, int top_k,
                              int num_experts, int hidden, int32_t* expert_counts,
                              int32_t* expert_offsets, void* x_perm, int32_t* inverse,
                              int32_t* sorted_token_ids, void* workspace, size_t workspace_bytes,
                              hipStream_t stream) {
    return dispatch("swiftllm_hip_moe_dispatch", nullptr, const_cast<int32_t*>(expert_ids),
                    nullptr, x, num_tokens, top_k, num_experts, hidden, expert_counts,
                    expert_offsets, x_perm, inverse, sorted_token_ids, workspace, workspace_bytes,
                    stream);
}

int swiftllm_hip_moe_route_dispatch(const float* logits, const void* x, int num_tokens,
                                    int top_k, int num_experts, int hidden, int32_t* expert_ids,
                                    float* weights, int32_t* expert_counts,
                                    int32_t* expert_offsets, void* x_perm, int32_t* inverse,
                                    int32_t* sorted_token_ids, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
    const char* who = "swiftllm_hip_moe_route_dispatch";
    if (num_tokens > 0 && !logits) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    return dispatch(who, logits, expert_ids, weights, x, num_tokens, top_k, num_experts, hidden,
                    expert_counts, expert_offsets, x_perm, inverse, sorted_token_ids, workspace,
                    workspace_bytes, stream);
}

}  // extern "C"
