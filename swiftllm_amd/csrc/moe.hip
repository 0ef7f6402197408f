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
//           softmax probabilities renormalised over the selected experts. The
//           few exponentials per token run in fp64.
// dispatch: (1) one wave per 64 tokens ranks its entries among equal experts
//           with ballots (stable (t, k) order) and counts them; the last
//           workgroup to finish scans the chunk counts into per-(chunk,
//           expert) row bases. (2) one wave per token writes the inverse index
//           and sorted token ids and copies the token's row once from HBM
//           into its K destination rows with 16-byte accesses.

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

template <int K>
__global__ __launch_bounds__(256) void moe_route_kernel(const RouteArgs a) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= a.T) return;
    const float* row = a.logits + static_cast<size_t>(t) * a.E;
    // K argmax passes over the row, each skipping the experts already taken;
    // the strict '>' keeps the lowest index among equal logits.
    float bv[K];
    int bi[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        float best = 0.0f;
        int besti = -1;
        for (int e = 0; e < a.E; ++e) {
            bool taken = false;
#pragma unroll
            for (int j = 0; j < k; ++j) taken = taken || (bi[j] == e);
            const float x = row[e];
            if (!taken && (besti < 0 || x > best)) {
                best = x;
                besti = e;
            }
        }
        bv[k] = best;
        bi[k] = besti;
    }
    double ex[K];
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        ex[k] = exp(static_cast<double>(bv[k]) - static_cast<double>(bv[0]));
        sum += ex[k];
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        a.ids[static_cast<size_t>(t) * K + k] = bi[k];
        a.w[static_cast<size_t>(t) * K + k] = static_cast<float>(ex[k] / sum);
    }
}

struct RankArgs {
    const int* ids;
    int* rank;       // [T*K] rank among equal experts inside the 64-token chunk
    int* chunk;      // [nchunks][E] counts; rewritten as row bases by the scan
    int* counts;     // [E]
    int* offsets;    // [E + 1]
    unsigned* ticket;
    int T;
    int E;
    int nchunks;
};

template <int K>
__global__ __launch_bounds__(256) void moe_rank_kernel(const RankArgs a) {
    __shared__ int s_cnt[4][kMaxExperts];
    __shared__ int s_tot[kMaxExperts + 1];
    __shared__ int s_last;
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int c = blockIdx.x * 4 + wv;  // chunk of this wave
    for (int e = lane; e < a.E; e += 64) s_cnt[wv][e] = 0;

    const int t = c * kChunkTokens + lane;
    const bool live = (c < a.nchunks) && (t < a.T);
    int id[K];
    bool pend[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        id[k] = live ? a.ids[static_cast<size_t>(t) * K + k] : -1;
        pend[k] = live && id[k] >= 0 && id[k] < a.E;
    }
    const unsigned long long below_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int rk[K];
#pragma unroll
    for (int k = 0; k < K; ++k) rk[k] = -1;
    // Peel one expert at a time: as many rounds as distinct experts in the chunk.
    while (true) {
        int cand = -1;
#pragma unroll
        for (int k = K - 1; k >= 0; --k) {
            if (pend[k]) cand = id[k];
        }
        const unsigned long long any = __ballot(cand >= 0);
        if (any == 0ull) break;
        const int e = __shfl(cand, __ffsll(static_cast<long long>(any)) - 1);
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
        if (lane == 0) s_cnt[wv][e] = total;
    }
    if (live) {
#pragma unroll
        for (int k = 0; k < K; ++k) a.rank[static_cast<size_t>(t) * K + k] = rk[k];
    }
    __syncthreads();
    if (c < a.nchunks) {
        for (int e = lane; e < a.E; e += 64) a.chunk[static_cast<size_t>(c) * a.E + e] = s_cnt[wv][e];
    }

    // The last workgroup to arrive scans the chunk counts.
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = atomicAdd(a.ticket, 1u);
        const int last = (prev == gridDim.x - 1);
        if (last) *a.ticket = 0u;
        s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int e = threadIdx.x; e < a.E; e += blockDim.x) {
        int run = 0;
        for (int cc = 0; cc < a.nchunks; ++cc) run += a.chunk[static_cast<size_t>(cc) * a.E + e];
        s_tot[e] = run;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int e = 0; e < a.E; ++e) {
            const int n = s_tot[e];
            s_tot[e] = run;
            a.offsets[e] = run;
            a.counts[e] = n;
            run += n;
        }
        a.offsets[a.E] = run;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < a.E; e += blockDim.x) {
        int run = s_tot[e];
        for (int cc = 0; cc < a.nchunks; ++cc) {
            int* p = a.chunk + static_cast<size_t>(cc) * a.E + e;
            const int n = *p;
            *p = run;
            run += n;
        }
    }
}

struct PermuteArgs {
    const int* ids;
    const int* rank;
    const int* base;  // [nchunks][E] row bases
    const uint16_t* x;
    uint16_t* xp;
    int* inverse;
    int* sorted;
    int T;
    int E;
    int hidden;
    int vec;  // 1: rows move as 16-byte vectors
};

template <int K>
__global__ __launch_bounds__(256) void moe_permute_kernel(const PermuteArgs a) {
    const int lane = threadIdx.x & 63;
    const int waves = gridDim.x * (blockDim.x >> 6);
    for (int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); t < a.T; t += waves) {
        const int c = t / kChunkTokens;
        long long rows[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int e = a.ids[static_cast<size_t>(t) * K + k];
            const int rk = a.rank[static_cast<size_t>(t) * K + k];
            int row = -1;
            if (e >= 0 && e < a.E && rk >= 0) row = a.base[static_cast<size_t>(c) * a.E + e] + rk;
            rows[k] = row;
            if (lane == 0) {
                a.inverse[static_cast<size_t>(t) * K + k] = row;
                if (row >= 0) a.sorted[row] = t;
            }
        }
        if (a.xp == nullptr) continue;
        if (a.vec) {
            const int nv = a.hidden / 8;
            const uint4* src = reinterpret_cast<const uint4*>(a.x + static_cast<size_t>(t) * a.hidden);
            for (int i = lane; i < nv; i += 64) {
                const uint4 v = src[i];
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    if (rows[k] >= 0) {
                        reinterpret_cast<uint4*>(a.xp + rows[k] * a.hidden)[i] = v;
                    }
                }
            }
        } else {
            const uint16_t* src = a.x + static_cast<size_t>(t) * a.hidden;
            for (int i = lane; i < a.hidden; i += 64) {
                const uint16_t v = src[i];
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    if (rows[k] >= 0) a.xp[rows[k] * a.hidden + i] = v;
                }
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
        return launch(moe_route_kernel<K>, dim3((a.T + 255) / 256), dim3(256), 0, s, a);
    }
};

template <int K>
struct RankLaunch {
    static hipError_t run(const RankArgs& a, hipStream_t s) {
        const int grid = (a.nchunks + 3) / 4 > 0 ? (a.nchunks + 3) / 4 : 1;
        return launch(moe_rank_kernel<K>, dim3(grid), dim3(256), 0, s, a);
    }
};

template <int K>
struct PermuteLaunch {
    static hipError_t run(const PermuteArgs& a, hipStream_t s) {
        const int wg = (a.T + 3) / 4;
        const int grid = wg < 65536 ? (wg > 0 ? wg : 1) : 65536;
        return launch(moe_permute_kernel<K>, dim3(grid), dim3(256), 0, s, a);
    }
};

struct DispatchLayout {
    int nchunks;
    size_t ticket, chunk, rank, total;
};

DispatchLayout dispatch_layout(int T, int E, int K) {
    DispatchLayout l{};
    l.nchunks = (T + kChunkTokens - 1) / kChunkTokens;
    auto up = [](size_t x) { return (x + 255) / 256 * 256; };
    l.ticket = 0;
    l.chunk = 256;
    l.rank = l.chunk + up(sizeof(int) * static_cast<size_t>(l.nchunks) * E);
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

int swiftllm_hip_moe_dispatch(const int32_t* expert_ids, const void* x, int num_tokens, int top_k,
                              int num_experts, int hidden, int32_t* expert_counts,
                              int32_t* expert_offsets, void* x_perm, int32_t* inverse,
                              int32_t* sorted_token_ids, void* workspace, size_t workspace_bytes,
                              hipStream_t stream) {
    const char* who = "swiftllm_hip_moe_dispatch";
    int rc = validate_moe(who, num_tokens, num_experts, top_k);
    if (rc != SWIFTLLM_OK) return rc;
    if (hidden < 0 || (x_perm != nullptr && hidden == 0)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: hidden=%d", who, hidden);
    }
    if (!expert_counts || !expert_offsets || !workspace) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    if (num_tokens > 0 && (!expert_ids || !inverse || !sorted_token_ids || (x_perm && !x))) {
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
    RankArgs ra{};
    ra.ids = expert_ids;
    ra.rank = reinterpret_cast<int*>(ws + l.rank);
    ra.chunk = reinterpret_cast<int*>(ws + l.chunk);
    ra.counts = expert_counts;
    ra.offsets = expert_offsets;
    ra.ticket = reinterpret_cast<unsigned*>(ws + l.ticket);
    ra.T = num_tokens;
    ra.E = num_experts;
    ra.nchunks = l.nchunks;
    hipError_t err = by_k<RankLaunch>(top_k, ra, stream);
    if (err != hipSuccess || num_tokens == 0) return launched(err, who);
    PermuteArgs pa{};
    pa.ids = expert_ids;
    pa.rank = ra.rank;
    pa.base = ra.chunk;
    pa.x = static_cast<const uint16_t*>(x);
    pa.xp = static_cast<uint16_t*>(x_perm);
    pa.inverse = inverse;
    pa.sorted = sorted_token_ids;
    pa.T = num_tokens;
    pa.E = num_experts;
    pa.hidden = hidden;
    pa.vec = (hidden % 8 == 0) && (x_perm == nullptr || (aligned(x, 16) && aligned(x_perm, 16)));
    return launched(by_k<PermuteLaunch>(top_k, pa, stream), who);
}

}  // extern "C"
